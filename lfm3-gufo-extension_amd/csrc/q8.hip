// Q8_0 weights on gfx950: tile repack, the skinny decode GEMV on MFMA, and
// the embedding gather.
//
// The GEMV (B <= 8 FP32 rows) runs on MFMA: a block stages its K slice of x
// once as fp16 hi/lo operands in LDS and its waves stream 16-row weight
// tiles against it (see Q8Gemv).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "common.hpp"
#include "internal.hpp"
#include "norm_image.hpp"

namespace lfm3amd {
namespace {

struct Q8Block {
  std::uint16_t d;
  std::int8_t q[32];
};
static_assert(sizeof(Q8Block) == 34, "Q8_0 block is 34 bytes");

__global__ void PackKernel(const std::uint8_t* __restrict__ src,
                           std::uint32_t rows, std::uint32_t cols,
                           std::uint8_t* __restrict__ codes,
                           Half* __restrict__ scales, std::uint32_t nchunks,
                           std::uint32_t src_tiles, std::uint32_t tile_offset,
                           std::uint32_t tile_stride) {
  // One thread per (source tile, chunk, lane): 16 code bytes, and the two
  // block scales of its row for the lanes of group 0.
  const std::size_t unit = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::size_t total = std::size_t(src_tiles) * nchunks * 64;
  if (unit >= total)
    return;
  const std::uint32_t lane = unit % 64;
  const std::size_t tc = unit / 64;
  const std::uint32_t chunk = tc % nchunks, tile = tc / nchunks;
  const std::uint32_t n = lane % 16, g = lane / 16;
  const std::uint32_t row = tile * kTileRows + n;
  const std::uint32_t blocks = cols / 32;
  const std::size_t dst_tile = std::size_t(tile_offset) + std::size_t(tile) * tile_stride;
  const std::size_t dst = dst_tile * nchunks + chunk;
  unsigned char bytes[16];
  Half d[2] = {0, 0};
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const std::uint32_t b = chunk * 2 + blk;
    const bool live = row < rows && b < blocks;
    const std::uint8_t* block = src + (std::size_t(row) * blocks + b) * 34;
    for (int j = 0; j < 8; ++j)
      bytes[blk * 8 + j] = live ? std::uint8_t(block[2 + 8 * g + j] ^ kCodeBias) : kCodeBias;
    if (live)
      d[blk] = Half(block[0] | (block[1] << 8));
  }
  uint4 packed;
  __builtin_memcpy(&packed, bytes, 16);
  *reinterpret_cast<uint4*>(codes + dst * kTileCodeBytes + lane * 16) = packed;
  if (g == 0) {
    scales[dst * kTileScales + n * 2] = d[0];
    scales[dst * kTileScales + n * 2 + 1] = d[1];
  }
}

// Launch plan of one GEMV: RT row tiles per block (RT / 2 gate/up pairs
// with SwiGLU), W waves per block, each wave owning the chunks c = w mod W
// of every K slice of W * SPW chunks. Each block covers the whole of K, so
// no output needs a merge across blocks: on gfx950 a merge through memory
// costs a device-scope fence, which writes back and invalidates the XCD's
// L2.
struct GemvPlan {
  int row_tiles, nchunks, groups, RT, W, SPW, parts;
};

// Number of K parts a partial-sum launch of this shape takes: enough that
// each part fits one LDS slice (32 chunks), then doubled while the grid
// stays within 256 blocks and parts keep 8 chunks (at 8 rows, 2048 x 2048
// runs fastest in 2 parts and 2048 x 7680 in 4; fewer parts are also
// fewer partial rows for the norm to read).
constexpr int kMaxGemvParts = 8;
int GemvParts(std::uint32_t rows, std::uint32_t cols) {
  const int tiles = int(RowTiles(rows)), nchunks = int(Chunks(cols));
  int parts = std::min((nchunks + 31) / 32, kMaxGemvParts);
  while (parts * 2 <= kMaxGemvParts && tiles * parts * 2 <= 256 &&
         nchunks / (parts * 2) >= 8)
    parts *= 2;
  return parts;
}

GemvPlan PlanGemv(std::uint32_t rows, std::uint32_t cols, bool swiglu,
                  int parts = 1) {
  GemvPlan p{};
  const int unit = swiglu ? 2 : 1;
  p.parts = parts;
  p.row_tiles = int(RowTiles(rows)) * unit;
  p.nchunks = int(Chunks(cols));
  const int nloc = (p.nchunks + parts - 1) / parts;
  p.SPW = 4;
  p.W = nloc <= 4 ? 1 : nloc <= 8 ? 2 : nloc <= 16 ? 4 : 8;
  if (nloc > 32)
    p.SPW = 5;  // slices of 40 chunks (80 KB of LDS operands), prefetched
  // Two 64 KB blocks fit a CU. Past 256 tiles a block takes two tiles: it
  // stages x and reduces across waves once for both (at 8192 x 2048 this is
  // about 10% faster than 512 one-tile blocks). So does a part of 24 chunks
  // or more: each tile then costs fewer staged x chunks (2048 x 7680 in 4
  // parts: 6.8 us against 7.9 us with one tile; 2048 x 2048 in 2 parts,
  // 16 chunks a part, stays fastest with one). A multi-slice block keeps
  // two slices of weights in registers: one tile (or gate/up pair).
  const int units = p.row_tiles / unit;
  int per = (units > 256 || nloc >= 24) && !swiglu ? 2 : 1;
  if (p.SPW == 5)
    per = 1;
  p.RT = per * unit;
  p.groups = (p.row_tiles + p.RT - 1) / p.RT;
  return p;
}

// Kernel tail shared by the GEMVs: total[r] holds this lane's sums for A
// rows 4 (L / 16) + i (tokens hi 0-7 then lo 0-7) of tile r's weight row
// L % 16. hi and lo add, then the W waves' partial sums add in wave order
// through LDS (red: W * RT * 128 + RT * 128 floats): fin[r * 128 + tok * 16
// + n] holds tile r's row n for token tok when the block's barrier returns.
// GemvEpilogue then writes the block's rows (SwiGLU: tile 2j is gate,
// 2j + 1 up, rows j * 16 + n).
template<int W, int RT, bool kLdsOnly = false>
__device__ __forceinline__ void StoreWaveSums(f4 (&total)[RT], float* red);
template<int W, int RT>
__device__ __forceinline__ float SumOverWaves(const float* red, int r, int idx);

template<int W, int RT>
__device__ __forceinline__ float* ReduceWaves(f4 (&total)[RT], float* red) {
  constexpr int T = W * 64;
  float* fin = red + W * RT * 128;
  StoreWaveSums<W, RT>(total, red);
  for (int o = threadIdx.x; o < RT * 128; o += T)
    fin[o] = SumOverWaves<W, RT>(red, o / 128, o % 128);
  __syncthreads();
  return fin;
}

// Each lane's hi + lo sums go to red[(wave * RT + r) * 128 + tok * 16 + n]
// (lanes L and L ^ 32 hold a token's hi and lo parts); after the block
// barrier, SumOverWaves adds one output's W wave sums in wave order.
// A block barrier that orders LDS only: the waves' LDS stores complete,
// then s_barrier; vector memory loads and stores in flight stay in flight
// (__syncthreads would wait for them too).
__device__ __forceinline__ void LdsBarrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
template<int W, int RT, bool kLdsOnly>
__device__ __forceinline__ void StoreWaveSums(f4 (&total)[RT], float* red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok0 = ((lane >> 4) & 1) * 4;
#pragma unroll
  for (int r = 0; r < RT; ++r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float val = SumXor32(total[r][i]);
      if (lane < 32)
        red[(wave * RT + r) * 128 + (tok0 + i) * 16 + (lane & 15)] = val;
    }
  }
  if constexpr (kLdsOnly)
    LdsBarrier();
  else
    __syncthreads();
}
template<int W, int RT>
__device__ __forceinline__ float SumOverWaves(const float* red, int r, int idx) {
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w)
    sum += red[(w * RT + r) * 128 + idx];
  return sum;
}

template<int W, int RT, bool kSwiGLU>
__device__ __forceinline__ void GemvEpilogue(f4 (&total)[RT], float* red, int group,
                                             int B, float* __restrict__ y, int ldy,
                                             int rows_out, float* const* y_rows = nullptr,
                                             unsigned long long* keys = nullptr,
                                             int groups = 0) {
  constexpr int T = W * 64;
  const int tid = threadIdx.x;
  // With T a multiple of 128 a thread stores one token's outputs; its row
  // pointer is loaded before the reductions, so the load's latency hides
  // behind them and it does not wait for the keys store.
  float* yrow = nullptr;
  if constexpr (!kSwiGLU && T % 128 == 0) {
    const int tok = (tid % 128) / 16;
    if (y_rows && tok < B)
      yrow = y_rows[tok];
  }
  StoreWaveSums<W, RT>(total, red);
  if (keys) {
    // Greedy candidates: token t's best ArgKey over the block's rows, one
    // (token, row) per lane, reduced over the token's lanes.
    constexpr int R = RT * kTileRows;  // rows of the block: 16 or 32
    if constexpr (8 * R <= T) {
      const int tok = tid / R, r = (tid % R) / kTileRows, n = tid % kTileRows;
      const int row = (group * RT + r) * kTileRows + n;
      unsigned long long key = 0;
      if (tid < 8 * R && row < rows_out)
        key = ArgKey(SumOverWaves<W, RT>(red, r, tok * 16 + n), unsigned(row));
#pragma unroll
      for (int m = R / 2; m; m >>= 1) {
        const unsigned long long other = __shfl_xor(key, m, 64);
        key = other > key ? other : key;
      }
      if (tid < 8 * R && tid % R == 0 && tok < B)
        keys[std::size_t(tok) * groups + group] = key;
    } else if (tid < B) {  // small blocks: one lane per token
      unsigned long long best = 0;
      for (int i = 0; i < R; ++i) {
        const int row = (group * RT + i / kTileRows) * kTileRows + i % kTileRows;
        const unsigned long long k = ArgKey(
            SumOverWaves<W, RT>(red, i / kTileRows, tid * 16 + i % kTileRows), unsigned(row));
        best = row < rows_out && k > best ? k : best;
      }
      keys[std::size_t(tid) * groups + group] = best;
    }
  }
  if constexpr (kSwiGLU) {
    for (int o = tid; o < (RT / 2) * 128; o += T) {
      const int pr = o / 128, idx = o % 128, tok = idx / 16, n = idx % 16;
      const int row = (group * (RT / 2) + pr) * kTileRows + n;
      const float gv = SumOverWaves<W, RT>(red, 2 * pr, idx);
      const float uv = SumOverWaves<W, RT>(red, 2 * pr + 1, idx);
      if (tok < B && row < rows_out)
        y[std::size_t(tok) * ldy + row] = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
    }
  } else {
    for (int o = tid; o < RT * 128; o += T) {
      const int r = o / 128, idx = o % 128, tok = idx / 16, n = idx % 16;
      const int row = (group * RT + r) * kTileRows + n;
      if (tok < B && row < rows_out)
        (y_rows ? (T % 128 == 0 ? yrow : y_rows[tok]) : y + std::size_t(tok) * ldy)[row] =
            SumOverWaves<W, RT>(red, r, idx);
    }
  }
}

// y[b][r] = sum_k W[r][k] x[b][k] for b < B <= 8. Each wave stages the x
// columns of its own chunks (chunk wave + W j of a K slice) in LDS as the
// MFMA A operand, with no block barrier: per token a power of two 2^e puts
// the maximum over those columns in [2^14, 2^15), hi = fp16(x 2^e) and
// lo = fp16((x 2^e - hi) 2^11), both truncated; A rows 0-7 are the tokens'
// hi parts and rows 8-15 their lo parts, so hi + lo 2^-11 keeps about 21
// bits of each value and every code x half product is exact in FP32. The
// B operand is 16 weight rows of one Q8_0 block decoded exactly to fp16,
// so one MFMA gives 16 rows' block dots and the block scale applies as
// acc = fma(d, dot, acc) in K order (hip/ops.hip:671-856: sums += scale *
// block_dot); 2^-e applies to each wave's sums. Weight loads of the next
// slice are issued before the current slice is staged. Waves sum in wave
// order, so results do not depend on scheduling.
template<int W, int SPW, int RT, bool kSwiGLU>
__launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(RT >= 2 ? 2 : 4)))
__global__ void Q8Gemv(const std::uint8_t* __restrict__ codes,
                       const Half* __restrict__ scales, int row_tiles,
                       int nchunks, int K, const float* __restrict__ x, int ldx,
                       int B, float* __restrict__ y, int ldy, int rows_out,
                       std::size_t part_stride) {
  constexpr int SLICE = W * SPW;
  // SPW 4 plans cover a block's K range in one slice; SPW 5 plans loop over
  // slices and prefetch the next slice's weights.
  constexpr bool kMulti = SPW > 4;
  __shared__ uint4 s_a[W][SPW * 2 * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = blockIdx.x;
  // K part of this block (blockIdx.y of gridDim.y); part p writes its sums
  // to y + p * part_stride.
  const int c_begin = int(blockIdx.y) * nchunks / int(gridDim.y);
  const int nloc = (int(blockIdx.y) + 1) * nchunks / int(gridDim.y) - c_begin;
  y += std::size_t(blockIdx.y) * part_stride;
  const int nslices = (nloc + SLICE - 1) / SLICE;

  // Weight tiles and scales of one slice: chunk wave + W j of the slice.
  // Buffer loads: a tile or chunk past the end reads zeros, without a
  // branch.
  const unsigned tiles_bytes = unsigned(row_tiles) * unsigned(nchunks);
  const BufferResource c_res = MakeBuffer(codes, tiles_bytes * kTileCodeBytes);
  const BufferResource s_res = MakeBuffer(scales, tiles_bytes * kTileScales * 2);
  const BufferResource x_res = MakeBuffer(x, unsigned(((B - 1) * ldx + K) * 4));
  uint4 q[RT][SPW], qn[RT][kMulti ? SPW : 1];
  unsigned sc[RT][SPW], scn[RT][kMulti ? SPW : 1];
  const auto fetch = [&](int slice, auto& qq, auto& ss) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int tile = group * RT + r;
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        const int chunk = slice * SLICE + wave + W * j;
        const bool live = tile < row_tiles && chunk < nloc;
        const unsigned off = unsigned(tile) * unsigned(nchunks) + unsigned(c_begin + chunk);
        qq[r][j] = LoadB128(c_res, live ? off * kTileCodeBytes + lane * 16 : kOutOfRange);
        ss[r][j] = LoadB32(s_res, live ? off * (kTileScales * 2) + (lane & 15) * 4 : kOutOfRange);
      }
    }
  };
  // Staging lane layout: token t = L % 8, eight columns 8 (L / 8) .. + 7 of
  // each of the wave's chunks.
  const int t = lane & 7, g8 = lane >> 3;
  float v[SPW][8];
  const auto load_x = [&](int slice) {
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int local = slice * SLICE + wave + W * j;
      const int k = (c_begin + local) * kChunk + g8 * 8;
      const unsigned off = t < B && local < nloc && k < K ? unsigned(t * ldx + k) * 4 : kOutOfRange;
      const float4 lo4 = LoadF4(x_res, off), hi4 = LoadF4(x_res, off + 16);
      v[j][0] = lo4.x; v[j][1] = lo4.y; v[j][2] = lo4.z; v[j][3] = lo4.w;
      v[j][4] = hi4.x; v[j][5] = hi4.y; v[j][6] = hi4.z; v[j][7] = hi4.w;
    }
  };
  // Memory results return in issue order: x (from L2) goes first so the
  // slice is staged while the weights stream in.
  load_x(0);
  fetch(0, q, sc);

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 total[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    total[r] = zero;
  const int part = lane >> 5, tok0 = ((lane >> 4) & 1) * 4;
  uint4* s_own = s_a[wave];

  for (int slice = 0; slice < nslices; ++slice) {
    if constexpr (kMulti) {
      if (slice > 0)
        load_x(slice);
      fetch(slice + 1, qn, scn);  // past the last slice: zeros, no traffic
    }
    // Token t's maximum over the wave's columns: its 8 lanes (L ^ 8, ^ 16,
    // ^ 32) reduce, then each lane reads the exponents of its A rows.
    float maximum = 0.0f;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        maximum = fmaxf(maximum, fabsf(v[j][i]));
    }
    maximum = MaxXor32(MaxXor16(MaxXor8(maximum)));
    const int e = RowExponent(maximum);
    int ex[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int lo_tok = __builtin_amdgcn_readlane(e, i), hi_tok = __builtin_amdgcn_readlane(e, 4 + i);
      ex[i] = -((tok0 ? hi_tok : lo_tok) + (part ? 11 : 0));
    }
    // A words of chunk j, block b = g8 / 4, lane group g8 % 4: row t (hi)
    // and row 8 + t (lo), after the previous slice's reads.
    if (slice) {
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      unsigned hw[4], lw[4];
#pragma unroll
      for (int i = 0; i < 8; i += 2)
        SplitPair(v[j][i], v[j][i + 1], e, hw[i / 2], lw[i / 2]);
      const int idx = (j * 2 + (g8 >> 2)) * 64 + 16 * (g8 & 3) + t;
      s_own[idx] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      s_own[idx + 8] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
    // The wave reads what its own lanes wrote: LDS keeps a wave's operations
    // in order; the fence keeps the compiler's order too.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // This wave's chunks of the slice: one MFMA per Q8_0 block. Chunk
    // outer, tile inner, so one chunk's A operands are live at a time.
    f4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
      acc[r] = zero;
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (slice * SLICE + wave + W * j >= nloc)
        continue;
      const h8 a0 = __builtin_bit_cast(h8, s_own[(j * 2) * 64 + lane]);
      const h8 a1 = __builtin_bit_cast(h8, s_own[(j * 2 + 1) * 64 + lane]);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (group * RT + r >= row_tiles)
          continue;
        const h8 w0 = EightCodes(q[r][j].x, q[r][j].y);
        const h8 w1 = EightCodes(q[r][j].z, q[r][j].w);
        const f4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, w0, zero, 0, 0, 0);
        const f4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, w1, zero, 0, 0, 0);
        const float d0 = HalfBitsToFloat(sc[r][j] & 0xffffu);
        const float d1 = HalfBitsToFloat(sc[r][j] >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = fmaf(d0, p0[i], acc[r][i]);
          acc[r][i] = fmaf(d1, p1[i], acc[r][i]);
        }
      }
    }
    // D layout: lane L holds A rows 4 (L / 16) + i (tokens hi 0-7, then lo
    // 0-7) of weight row L % 16; undo the slice's powers of two.
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        total[r][i] += ldexpf(acc[r][i], ex[i]);
    if constexpr (kMulti) {
      if (slice + 1 < nslices) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
          for (int j = 0; j < SPW; ++j) {
            q[r][j] = qn[r][j];
            sc[r][j] = scn[r][j];
          }
      }
    }
  }

  // hi + lo, then the waves in wave order through LDS (the operand image
  // is free once every wave has its operands).
  __syncthreads();
  GemvEpilogue<W, RT, kSwiGLU>(total, reinterpret_cast<float*>(s_a), group, B,
                               y, ldy, rows_out);
}

// The operand-image GEMV's main loop: tile r of the block is tile_of(r);
// returns each lane's un-scaled sums (D layout: lane L holds A rows
// 4 (L / 16) + i of weight row L % 16) with the rows' powers of two undone.
// With kAwait (a fused launch) the image is written by this launch's norm
// blocks: each compute wave issues its first round's weight loads, waits
// for its block's watcher wave (AwaitReady: the rows are published), then
// loads the image, so the weights stream in while the norm runs.
template<int W, int RT, int SPW, bool kAwait = false, typename TileOf>
__device__ __forceinline__ void ImageGemvCore(const std::uint8_t* __restrict__ codes,
                                              const Half* __restrict__ scales, int row_tiles,
                                              int nchunks, const uint4* __restrict__ image,
                                              const int* __restrict__ exps, int B, int c_begin,
                                              int nloc, TileOf tile_of, f4 (&total)[RT],
                                              const unsigned* ready = nullptr,
                                              unsigned seq = 0) {
  constexpr int ROUND = W * SPW;  // chunks per wave per round
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool a_live = (lane & 7) < B;
  const int part = lane >> 5, tok0 = ((lane >> 4) & 1) * 4;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    acc[r] = zero;
  const unsigned tiles_bytes = unsigned(row_tiles) * unsigned(nchunks);
  const BufferResource c_res = MakeBuffer(codes, tiles_bytes * kTileCodeBytes);
  const BufferResource s_res = MakeBuffer(scales, tiles_bytes * kTileScales * 2);
  const BufferResource a_res = MakeBuffer(image, unsigned(nchunks) * 2 * 64 * 16);
  if constexpr (kAwait) {
    if (nloc <= 0)
      AwaitReady(ready, seq);  // no round: the exponents still wait
  }
  for (int base = 0; base < nloc; base += ROUND) {
    uint4 q[RT][SPW];
    unsigned sc[RT][SPW];
    uint4 a[SPW][2];
    const auto load_a = [&](int j) {
      const int chunk = base + wave + W * j;
      const bool live = chunk < nloc;
      const unsigned at = (unsigned(c_begin + chunk) * 2 * 64 + lane) * 16;
      a[j][0] = LoadB128(a_res, live && a_live ? at : kOutOfRange);
      a[j][1] = LoadB128(a_res, live && a_live ? at + 64 * 16 : kOutOfRange);
    };
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const int chunk = base + wave + W * j;
      const bool live = chunk < nloc;
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const int tile = tile_of(r);
        const unsigned off = unsigned(tile) * unsigned(nchunks) + unsigned(c_begin + chunk);
        const bool ok = live && tile < row_tiles;
        q[r][j] = LoadB128(c_res, ok ? off * kTileCodeBytes + lane * 16 : kOutOfRange);
        sc[r][j] = LoadB32(s_res, ok ? off * (kTileScales * 2) + (lane & 15) * 4 : kOutOfRange);
      }
      if constexpr (!kAwait)
        load_a(j);
    }
    if constexpr (kAwait) {
      if (base == 0)
        AwaitReady(ready, seq);
#pragma unroll
      for (int j = 0; j < SPW; ++j)
        load_a(j);
    }
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      if (base + wave + W * j >= nloc)
        continue;
      const h8 a0 = __builtin_bit_cast(h8, a[j][0]), a1 = __builtin_bit_cast(h8, a[j][1]);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        if (tile_of(r) >= row_tiles)
          continue;
        const h8 w0 = EightCodes(q[r][j].x, q[r][j].y);
        const h8 w1 = EightCodes(q[r][j].z, q[r][j].w);
        const f4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, w0, zero, 0, 0, 0);
        const f4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, w1, zero, 0, 0, 0);
        const float d0 = HalfBitsToFloat(sc[r][j] & 0xffffu);
        const float d1 = HalfBitsToFloat(sc[r][j] >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = fmaf(d0, p0[i], acc[r][i]);
          acc[r][i] = fmaf(d1, p1[i], acc[r][i]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = tok0 + i;
    const int ex = -((t < B ? exps[t] : 0) + (part ? 11 : 0));
#pragma unroll
    for (int r = 0; r < RT; ++r)
      total[r][i] = ldexpf(acc[r][i], ex);
  }
}

// A fused launch (kNorm) has W + 1 waves a block: its first B blocks run
// the norm rows and publish them (NormImageRow); in every other block wave
// W watches the rows' flags (WatchRows) and hands over through an LDS word
// while waves 0 .. W - 1 have their weight loads in flight, then leaves.
template<int W, int RT, bool kSwiGLU, int SPW, bool kNorm = false>
__launch_bounds__((W + kNorm) * 64)
__attribute__((amdgpu_waves_per_eu(RT >= 4 ? 2 : kNorm ? 5 : 4)))
__global__ void Q8GemvImage(const std::uint8_t* __restrict__ codes,
                            const Half* __restrict__ scales, int row_tiles,
                            int nchunks, const uint4* __restrict__ image,
                            const int* __restrict__ exps, int B,
                            float* __restrict__ y, int ldy, int rows_out,
                            std::size_t part_stride, float* const* __restrict__ y_rows,
                            unsigned long long* __restrict__ keys, const FusedNorm fused) {
  __shared__ float red[W * RT * 128 + RT * 128];
  // A fused launch's first B blocks are the norm of its B rows.
  const int lead = kNorm ? B : 0;
  const int c_begin = int(blockIdx.y) * nchunks / int(gridDim.y);
  const int nloc = (int(blockIdx.y) + 1) * nchunks / int(gridDim.y) - c_begin;
  __shared__ unsigned s_ready;
  if constexpr (kNorm) {
    if (int(blockIdx.x) < B) {
      NormImageRow<(W + 1) * 64, 1, true>(fused.args, blockIdx.x, fused.flags, fused.seq);
      return;
    }
    // s_ready starts cleared for every wave (LDS is not initialized).
    if (threadIdx.x == 0)
      s_ready = 0;
    __syncthreads();
    if ((threadIdx.x >> 6) == W) {
      WatchRows(fused.flags, fused.seq, fused.error, B, &s_ready);
      return;
    }
  }
  const int group = int(blockIdx.x) - lead;
  y += std::size_t(blockIdx.y) * part_stride;
  f4 total[RT];
  ImageGemvCore<W, RT, SPW, kNorm>(codes, scales, row_tiles, nchunks, image, exps, B, c_begin,
                                   nloc, [=](int r) { return group * RT + r; }, total, &s_ready,
                                   fused.seq);
  GemvEpilogue<W, RT, kSwiGLU>(total, red, group, B, y, ldy, rows_out, y_rows, keys,
                               int(gridDim.x) - lead);
}

// The operand-image GEMV over many row groups (the vocabulary head: 4000
// groups of two tiles) as a grid-stride loop over one block a CU: each
// wave stages its image operands in LDS once, and issues the next group's
// weight loads before it computes and writes the current one, so its
// weight stream does not stop at group boundaries (one block a group
// drains its loads before its epilogue, and the next block starts behind
// it: the head 59.7 us against 54.8 with this loop). K is one round of
// chunks (nchunks <= W * SPW); parts = 1. Per group, tile and chunk the
// same loads, products and reductions as Q8GemvImage, so the outputs and
// greedy keys are bit-identical to it. Block barriers in the loop order
// LDS only, so the next group's loads stay in flight across them.
template<int W, int RT, int SPW, bool kNorm>
__launch_bounds__((W + kNorm) * 64)
__global__ void Q8GemvImageLoop(const std::uint8_t* __restrict__ codes,
                                const Half* __restrict__ scales, int row_tiles, int nchunks,
                                int groups, const uint4* __restrict__ image,
                                const int* __restrict__ exps, int B, float* __restrict__ y,
                                int ldy, int rows_out, float* const* __restrict__ y_rows,
                                unsigned long long* __restrict__ keys, const FusedNorm fused) {
  __shared__ float red[W * RT * 128 + RT * 128];
  __shared__ uint4 s_img[W][SPW * 2][64];
  __shared__ unsigned s_ready;
  const int lead = kNorm ? B : 0;
  if constexpr (kNorm) {
    if (int(blockIdx.x) < B) {
      NormImageRow<(W + 1) * 64, 1, true>(fused.args, blockIdx.x, fused.flags, fused.seq);
      return;
    }
    if (threadIdx.x == 0)
      s_ready = 0;
    __syncthreads();
    if ((threadIdx.x >> 6) == W) {
      WatchRows(fused.flags, fused.seq, fused.error, B, &s_ready);
      return;
    }
  }
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool a_live = (lane & 7) < B;
  const int part = lane >> 5, tok0 = ((lane >> 4) & 1) * 4;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const unsigned tiles_bytes = unsigned(row_tiles) * unsigned(nchunks);
  const BufferResource c_res = MakeBuffer(codes, tiles_bytes * kTileCodeBytes);
  const BufferResource s_res = MakeBuffer(scales, tiles_bytes * kTileScales * 2);
  const BufferResource a_res = MakeBuffer(image, unsigned(nchunks) * 2 * 64 * 16);
  // Empty resources: every load through them reads zeros.
  const BufferResource c_none = MakeBuffer(codes, 0), s_none = MakeBuffer(scales, 0);
  // The lanes' VGPR offsets are fixed for the whole loop (a VGPR that an
  // in-flight load still reads is never rewritten, so no wait drains the
  // loads in flight); the group and chunk offsets ride in the SGPR offset.
  unsigned c_off[SPW], s_off[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const bool live = wave + W * j < nchunks;
    c_off[j] = live ? unsigned(wave) * kTileCodeBytes + unsigned(lane) * 16 : kOutOfRange;
    s_off[j] = live ? unsigned(wave) * (kTileScales * 2) + unsigned(lane & 15) * 4 : kOutOfRange;
  }
  const int stride = int(gridDim.x) - lead;
  using Codes = uint4[RT][SPW];
  using Scales = unsigned[RT][SPW];
  const auto fetch = [&](int g, Codes& q, Scales& sc) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      // Block-uniform: a tile past the matrix (or a group past the last)
      // reads through the empty resources.
      const int tile = g * RT + r;
      const bool in = g < groups && tile < row_tiles;
      const BufferResource cr = in ? c_res : c_none, sr = in ? s_res : s_none;
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        const unsigned at = in ? unsigned(tile) * unsigned(nchunks) + unsigned(W * j) : 0u;
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(cr, c_off[j], at * kTileCodeBytes, 0);
        q[r][j] = make_uint4(v.x, v.y, v.z, v.w);
        sc[r][j] = __builtin_amdgcn_raw_buffer_load_b32(sr, s_off[j], at * (kTileScales * 2), 0);
      }
    }
  };
  int group = int(blockIdx.x) - lead;
  Codes q0, q1;
  Scales s0, s1;
  fetch(group, q0, s0);
  if constexpr (kNorm)
    AwaitReady(&s_ready, fused.seq);
  // The wave's image chunks (wave + W j) into its own LDS rows; it reads
  // only what its own lanes wrote, in order.
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int chunk = wave + W * j;
    const unsigned at = (unsigned(chunk) * 2 * 64 + lane) * 16;
    const bool live = chunk < nchunks && a_live;
    s_img[wave][2 * j][lane] = LoadB128(a_res, live ? at : kOutOfRange);
    s_img[wave][2 * j + 1][lane] = LoadB128(a_res, live ? at + 64 * 16 : kOutOfRange);
  }
  int ex[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = tok0 + i;
    ex[i] = -((t < B ? exps[t] : 0) + (part ? 11 : 0));
  }
  // Thread tid stores token (tid % 128) / 16's outputs: its row pointer is
  // loaded once, before any group's weight loads are in flight behind it.
  using GlobalFloat = __attribute__((address_space(1))) float;
  static_assert(W * 64 % 128 == 0, "a thread stores one token's outputs");
  const int my_tok = (tid % 128) / 16;
  GlobalFloat* yrow = nullptr;
  if (my_tok < B)
    yrow = (GlobalFloat*)(y_rows ? y_rows[my_tok] : y + std::size_t(my_tok) * ldy);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const auto step = [&](int g, const Codes& q, const Scales& sc) {
    f4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
      acc[r] = zero;
    // Chunks past nchunks (and groups past the last) loaded zeros: their
    // products add exactly 0, so every MFMA runs unconditionally.
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const h8 a0 = __builtin_bit_cast(h8, s_img[wave][2 * j][lane]);
      const h8 a1 = __builtin_bit_cast(h8, s_img[wave][2 * j + 1][lane]);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const h8 w0 = EightCodes(q[r][j].x, q[r][j].y);
        const h8 w1 = EightCodes(q[r][j].z, q[r][j].w);
        const f4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, w0, zero, 0, 0, 0);
        const f4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, w1, zero, 0, 0, 0);
        const float d0 = HalfBitsToFloat(sc[r][j] & 0xffffu);
        const float d1 = HalfBitsToFloat(sc[r][j] >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = fmaf(d0, p0[i], acc[r][i]);
          acc[r][i] = fmaf(d1, p1[i], acc[r][i]);
        }
      }
    }
    f4 total[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        total[r][i] = ldexpf(acc[r][i], ex[i]);
    // GemvEpilogue's reductions and stores, with the row pointer above.
    StoreWaveSums<W, RT, true>(total, red);
    if (keys) {
      constexpr int R = RT * kTileRows, T = W * 64;
      static_assert(8 * R <= T, "one (token, row) a lane");
      const int tok = tid / R, r = (tid % R) / kTileRows, n = tid % kTileRows;
      const int row = (g * RT + r) * kTileRows + n;
      unsigned long long key = 0;
      if (tid < 8 * R && row < rows_out)
        key = ArgKey(SumOverWaves<W, RT>(red, r, tok * 16 + n), unsigned(row));
#pragma unroll
      for (int m = R / 2; m; m >>= 1) {
        const unsigned long long other = __shfl_xor(key, m, 64);
        key = other > key ? other : key;
      }
      if (tid < 8 * R && tid % R == 0 && tok < B)
        keys[std::size_t(tok) * groups + g] = key;
    }
    for (int o = tid; o < RT * 128; o += W * 64) {
      const int r = o / 128, idx = o % 128, n = idx % 16;
      const int row = (g * RT + r) * kTileRows + n;
      if (my_tok < B && row < rows_out)
        yrow[row] = SumOverWaves<W, RT>(red, r, idx);
    }
    LdsBarrier();  // red is rewritten by the next group
  };
  // Two register sets, alternating, so no copy waits on the loads in flight;
  // the next group's loads issue before the current group's first MFMA.
  while (group < groups) {
    fetch(group + stride, q1, s1);
    __builtin_amdgcn_sched_barrier(0);
    step(group, q0, s0);
    group += stride;
    if (group >= groups)
      break;
    fetch(group + stride, q0, s0);
    __builtin_amdgcn_sched_barrier(0);
    step(group, q1, s1);
    group += stride;
  }
}

// Q8Gemv over many row groups (the vocabulary head on FP32 rows: 4000
// groups of two tiles) as the same grid-stride loop as Q8GemvImageLoop:
// each wave stages its chunks of x once (Q8Gemv's one-slice staging: the
// same exponents and hi/lo operands), then issues the next group's weight
// loads before it computes and writes the current one. Per group the
// loads, products and reductions are Q8Gemv's, so the outputs are
// bit-identical to it. K is one slice (nchunks <= W * SPW); parts = 1.
template<int W, int RT, int SPW>
__launch_bounds__(W * 64)
__global__ void Q8GemvLoop(const std::uint8_t* __restrict__ codes,
                           const Half* __restrict__ scales, int row_tiles, int nchunks,
                           int groups, int K, const float* __restrict__ x, int ldx, int B,
                           float* __restrict__ y, int ldy, int rows_out) {
  __shared__ uint4 s_a[W][SPW * 2 * 64];
  __shared__ float red[W * RT * 128 + RT * 128];
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const unsigned tiles_bytes = unsigned(row_tiles) * unsigned(nchunks);
  const BufferResource c_res = MakeBuffer(codes, tiles_bytes * kTileCodeBytes);
  const BufferResource s_res = MakeBuffer(scales, tiles_bytes * kTileScales * 2);
  const BufferResource c_none = MakeBuffer(codes, 0), s_none = MakeBuffer(scales, 0);
  const BufferResource x_res = MakeBuffer(x, unsigned(((B - 1) * ldx + K) * 4));
  // Fixed lane offsets, group and chunk in the SGPR offset (as in
  // Q8GemvImageLoop).
  unsigned c_off[SPW], s_off[SPW];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const bool live = wave + W * j < nchunks;
    c_off[j] = live ? unsigned(wave) * kTileCodeBytes + unsigned(lane) * 16 : kOutOfRange;
    s_off[j] = live ? unsigned(wave) * (kTileScales * 2) + unsigned(lane & 15) * 4 : kOutOfRange;
  }
  const int stride = int(gridDim.x);
  using Codes = uint4[RT][SPW];
  using Scales = unsigned[RT][SPW];
  const auto fetch = [&](int g, Codes& q, Scales& sc) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int tile = g * RT + r;
      const bool in = g < groups && tile < row_tiles;
      const BufferResource cr = in ? c_res : c_none, sr = in ? s_res : s_none;
#pragma unroll
      for (int j = 0; j < SPW; ++j) {
        const unsigned at = in ? unsigned(tile) * unsigned(nchunks) + unsigned(W * j) : 0u;
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(cr, c_off[j], at * kTileCodeBytes, 0);
        q[r][j] = make_uint4(v.x, v.y, v.z, v.w);
        sc[r][j] = __builtin_amdgcn_raw_buffer_load_b32(sr, s_off[j], at * (kTileScales * 2), 0);
      }
    }
  };
  // Q8Gemv's staging of the wave's chunks (token t = L % 8, columns
  // 8 (L / 8) .. + 7 of each chunk), x first so it returns before the
  // weights.
  const int t = lane & 7, g8 = lane >> 3;
  float v[SPW][8];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int chunk = wave + W * j;
    const int k = chunk * kChunk + g8 * 8;
    const unsigned off = t < B && chunk < nchunks && k < K ? unsigned(t * ldx + k) * 4 : kOutOfRange;
    const float4 lo4 = LoadF4(x_res, off), hi4 = LoadF4(x_res, off + 16);
    v[j][0] = lo4.x; v[j][1] = lo4.y; v[j][2] = lo4.z; v[j][3] = lo4.w;
    v[j][4] = hi4.x; v[j][5] = hi4.y; v[j][6] = hi4.z; v[j][7] = hi4.w;
  }
  int group = int(blockIdx.x);
  Codes q0, q1;
  Scales s0, s1;
  fetch(group, q0, s0);
  __builtin_amdgcn_sched_barrier(0);
  const int part = lane >> 5, tok0 = ((lane >> 4) & 1) * 4;
  float maximum = 0.0f;
#pragma unroll
  for (int j = 0; j < SPW; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      maximum = fmaxf(maximum, fabsf(v[j][i]));
  maximum = MaxXor32(MaxXor16(MaxXor8(maximum)));
  const int e = RowExponent(maximum);
  int ex[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lo_tok = __builtin_amdgcn_readlane(e, i), hi_tok = __builtin_amdgcn_readlane(e, 4 + i);
    ex[i] = -((tok0 ? hi_tok : lo_tok) + (part ? 11 : 0));
  }
  uint4* s_own = s_a[wave];
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    unsigned hw[4], lw[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2)
      SplitPair(v[j][i], v[j][i + 1], e, hw[i / 2], lw[i / 2]);
    const int idx = (j * 2 + (g8 >> 2)) * 64 + 16 * (g8 & 3) + t;
    s_own[idx] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    s_own[idx + 8] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
  }
  // The wave reads what its own lanes wrote: LDS keeps a wave's operations
  // in order; the fence keeps the compiler's order too.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const auto step = [&](int g, const Codes& q, const Scales& sc) {
    f4 acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
      acc[r] = zero;
    // Chunks past nchunks (and groups past the last) loaded zeros: their
    // products add exactly 0, so every MFMA runs unconditionally.
#pragma unroll
    for (int j = 0; j < SPW; ++j) {
      const h8 a0 = __builtin_bit_cast(h8, s_own[(j * 2) * 64 + lane]);
      const h8 a1 = __builtin_bit_cast(h8, s_own[(j * 2 + 1) * 64 + lane]);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const h8 w0 = EightCodes(q[r][j].x, q[r][j].y);
        const h8 w1 = EightCodes(q[r][j].z, q[r][j].w);
        const f4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, w0, zero, 0, 0, 0);
        const f4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, w1, zero, 0, 0, 0);
        const float d0 = HalfBitsToFloat(sc[r][j] & 0xffffu);
        const float d1 = HalfBitsToFloat(sc[r][j] >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[r][i] = fmaf(d0, p0[i], acc[r][i]);
          acc[r][i] = fmaf(d1, p1[i], acc[r][i]);
        }
      }
    }
    f4 total[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        total[r][i] = ldexpf(acc[r][i], ex[i]);
    // GemvEpilogue's reductions and stores (y is a global pointer: no
    // load behind the next group's weights).
    StoreWaveSums<W, RT, true>(total, red);
    for (int o = tid; o < RT * 128; o += W * 64) {
      const int r = o / 128, idx = o % 128, tok = idx / 16, n = idx % 16;
      const int row = (g * RT + r) * kTileRows + n;
      if (tok < B && row < rows_out)
        y[std::size_t(tok) * ldy + row] = SumOverWaves<W, RT>(red, r, idx);
    }
    LdsBarrier();  // red is rewritten by the next group
  };
  while (group < groups) {
    fetch(group + stride, q1, s1);
    __builtin_amdgcn_sched_barrier(0);
    step(group, q0, s0);
    group += stride;
    if (group >= groups)
      break;
    fetch(group + stride, q0, s0);
    __builtin_amdgcn_sched_barrier(0);
    step(group, q1, s1);
    group += stride;
  }
}

// The convolution block's in projection with the decode convolution step
// (reference.cpp:85-101) in its epilogue: block g computes tiles g, g + T
// and g + 2T (T = hidden / 16) of the [B | C | X] projection, i.e. B, C and
// X of channels 16 g .. 16 g + 15, then applies ConvStepKernel's
// expressions to them, in the same order (for the same projection values,
// outputs and history equal lfm3_conv_step_ragged's bit for bit).
template<int W, bool kNorm = false>
__launch_bounds__((W + kNorm) * 64) __attribute__((amdgpu_waves_per_eu(2)))
__global__ void Q8GemvConvImage(const std::uint8_t* __restrict__ codes,
                                const Half* __restrict__ scales, int third_tiles,
                                int nchunks, const uint4* __restrict__ image,
                                const int* __restrict__ exps, int B,
                                const float* __restrict__ taps,
                                float* const* __restrict__ history, int L, int H,
                                float* __restrict__ y, int ldy, const FusedNorm fused) {
  constexpr int RT = 3, T = W * 64, kMaxWidth = 32;
  __shared__ float red[W * RT * 128 + RT * 128];
  __shared__ float s_hist[128][kMaxWidth - 1];
  __shared__ float s_taps[kTileRows][kMaxWidth];
  __shared__ unsigned s_ready;
  // A fused launch's first B blocks are the norm of its B rows; then wave W
  // of each block watches the rows' flags and leaves.
  if constexpr (kNorm) {
    if (int(blockIdx.x) < B) {
      NormImageRow<(W + 1) * 64, 1, true>(fused.args, blockIdx.x, fused.flags, fused.seq);
      return;
    }
    if (threadIdx.x == 0)
      s_ready = 0;
    __syncthreads();
    if ((threadIdx.x >> 6) == W) {
      WatchRows(fused.flags, fused.seq, fused.error, B, &s_ready);
      return;
    }
  }
  const int group = int(blockIdx.x) - (kNorm ? B : 0);
  // The step's history rows and taps do not depend on the projection: they
  // are staged before the weights stream, so the epilogue reads LDS only.
  for (int e = threadIdx.x; e < 128 * (L - 1); e += T) {
    const int o = e / (L - 1), t = e % (L - 1);
    const int tok = o / 16, ch = group * kTileRows + o % 16;
    if (tok < B && ch < H)
      s_hist[o][t] = history[tok][std::size_t(ch) * (L - 1) + t];
  }
  for (int e = threadIdx.x; e < kTileRows * L; e += T) {
    const int n = e / L, t = e % L, ch = group * kTileRows + n;
    if (ch < H)
      s_taps[n][t] = taps[std::size_t(ch) * L + t];
  }
  f4 total[RT];
  ImageGemvCore<W, RT, W >= 16 ? 2 : 4, kNorm>(
      codes, scales, 3 * third_tiles, nchunks, image, exps, B, 0, nchunks,
      [=](int r) { return group + r * third_tiles; }, total, &s_ready, fused.seq);
  const float* fin = ReduceWaves<W, RT>(total, red);  // its barriers publish s_hist
  for (int o = threadIdx.x; o < 128; o += T) {
#pragma clang fp contract(off)
    const int tok = o / 16, n = o % 16, ch = group * kTileRows + n;
    if (tok >= B || ch >= H)
      continue;
    const float b = fin[o], c = fin[128 + o], x = fin[256 + o];
    const float* own = s_hist[o];
    const float bx = b * x;
    const float* w = s_taps[n];
    float sum = 0.0f;
    for (int t = 0; t < L - 1; ++t)
      sum += w[t] * own[t];
    sum += w[L - 1] * bx;
    float* dst = history[tok] + std::size_t(ch) * (L - 1);
    for (int t = 1; t < L - 1; ++t)
      dst[t - 1] = own[t];
    dst[L - 2] = bx;
    y[std::size_t(tok) * ldy + ch] = sum * c;
  }
}

// The device's CU count (the first device queried; 256 on MI355X).
int CuCount() {
  static const int cus = [] {
    int device = 0, n = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        n <= 0)
      n = 256;
    return n;
  }();
  return cus;
}

// Past this many two-tile groups an operand-image GEMV whose K is one round
// runs as Q8GemvImageLoop, and a Q8Gemv whose K is one slice as Q8GemvLoop
// (the vocabulary head: 4000 groups).
constexpr int kLoopGroups = 1024;

template<int W, int SPW, int RT, bool kSwiGLU>
void LaunchPlan(const GemvPlan& p, const std::uint8_t* c, const Half* s, int K,
                const float* x, int ldx, int B, float* y, int ldy, int rows_out,
                hipStream_t stream) {
  if constexpr (!kSwiGLU && RT == 2 && W == 8 && SPW == 4) {
    if (p.parts == 1 && p.nchunks <= W * SPW && p.groups >= kLoopGroups) {
      // One block a CU, as the operand-image loop.
      Q8GemvLoop<W, RT, SPW><<<std::min(p.groups, CuCount()), W * 64, 0, stream>>>(
          c, s, p.row_tiles, p.nchunks, p.groups, K, x, ldx, B, y, ldy, rows_out);
      return;
    }
  }
  Q8Gemv<W, SPW, RT, kSwiGLU><<<dim3(p.groups, p.parts), W * 64, 0, stream>>>(
      c, s, p.row_tiles, p.nchunks, K, x, ldx, B, y, ldy, rows_out,
      std::size_t(ldy) * B);
}

template<int W, int SPW, bool kSwiGLU>
void LaunchRT(const GemvPlan& p, const std::uint8_t* c, const Half* s, int K,
              const float* x, int ldx, int B, float* y, int ldy, int rows_out,
              hipStream_t stream) {
  if constexpr (SPW > 4 || kSwiGLU) {  // one tile, or one gate/up pair
    LaunchPlan<W, SPW, kSwiGLU ? 2 : 1, kSwiGLU>(p, c, s, K, x, ldx, B, y, ldy, rows_out,
                                                stream);
  } else {
    if (p.RT == 1)
      LaunchPlan<W, SPW, 1, false>(p, c, s, K, x, ldx, B, y, ldy, rows_out, stream);
    else
      LaunchPlan<W, SPW, 2, false>(p, c, s, K, x, ldx, B, y, ldy, rows_out, stream);
  }
}

template<bool kSwiGLU>
int LaunchGemv(const void* codes, const void* scales, std::uint32_t rows,
               std::uint32_t cols, const float* x, std::uint32_t ldx, float* y,
               std::uint32_t ldy, std::uint32_t batch, hipStream_t stream,
               int parts = 1) {
  if (!codes || !scales || !x || !y || rows == 0 || cols == 0 ||
      cols % 32 || batch == 0 || batch > 8 || ldx % 4 || ldx < cols ||
      ldy < rows || (reinterpret_cast<std::uintptr_t>(x) & 15) || parts < 1 ||
      parts > int(Chunks(cols)) ||
      !BufferFits(std::size_t(RowTiles(rows) * (kSwiGLU ? 2 : 1)) * Chunks(cols) *
                  kTileCodeBytes) ||
      !BufferFits((std::size_t(batch - 1) * ldx + cols) * 4))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 GEMV shape");
  const GemvPlan p = PlanGemv(rows, cols, kSwiGLU, parts);
  const auto* c = static_cast<const std::uint8_t*>(codes);
  const auto* s = static_cast<const Half*>(scales);
  const int K = int(cols), B = int(batch), lx = int(ldx), ly = int(ldy), ro = int(rows);
  if (p.SPW == 5)
    LaunchRT<8, 5, kSwiGLU>(p, c, s, K, x, lx, B, y, ly, ro, stream);
  else if (p.W == 8)
    LaunchRT<8, 4, kSwiGLU>(p, c, s, K, x, lx, B, y, ly, ro, stream);
  else if (p.W == 4)
    LaunchRT<4, 4, kSwiGLU>(p, c, s, K, x, lx, B, y, ly, ro, stream);
  else if (p.W == 2)
    LaunchRT<2, 4, kSwiGLU>(p, c, s, K, x, lx, B, y, ly, ro, stream);
  else
    LaunchRT<1, 4, kSwiGLU>(p, c, s, K, x, lx, B, y, ly, ro, stream);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 GEMV launch");
}

// A fused launch's norm blocks have the GEMV's block size: one thread per 8
// columns (NormImageRow with G = 1) needs hidden / 8 <= threads; its
// operand image and flags must be given.
bool FusedNormFits(const FusedNorm& f, std::uint32_t cols, unsigned threads) {
  return f.flags && f.args.image && f.args.exps && f.args.x && f.args.weight &&
         f.args.H == int(cols) && Chunks(cols) * 8 <= threads;
}

template<int W, int RT, bool kSwiGLU>
void LaunchImagePlan(const GemvPlan& p, const std::uint8_t* c, const Half* s,
                     const uint4* image, const int* exps, int B, float* y,
                     int ldy, int rows_out, hipStream_t stream, float* const* y_rows,
                     unsigned long long* keys, const FusedNorm* fused) {
  constexpr int SPW = W >= 16 ? 2 : 4;
  if constexpr (!kSwiGLU && RT == 2 && W == 8) {
    if (p.parts == 1 && p.nchunks <= W * SPW && p.groups >= kLoopGroups) {
      // One block a CU (its 152 VGPRs a lane allow one), the norm blocks
      // included: a block past that would start only when a whole block
      // has finished its groups.
      const int lead = fused ? B : 0;
      const int blocks = std::min(p.groups, std::max(1, CuCount() - lead));
      if (fused)
        Q8GemvImageLoop<W, RT, SPW, true><<<blocks + lead, (W + 1) * 64, 0, stream>>>(
            c, s, p.row_tiles, p.nchunks, p.groups, image, exps, B, y, ldy, rows_out, y_rows,
            keys, *fused);
      else
        Q8GemvImageLoop<W, RT, SPW, false><<<blocks, W * 64, 0, stream>>>(
            c, s, p.row_tiles, p.nchunks, p.groups, image, exps, B, y, ldy, rows_out, y_rows,
            keys, FusedNorm{});
      return;
    }
  }
  if (fused)
    Q8GemvImage<W, RT, kSwiGLU, SPW, true>
        <<<dim3(p.groups + B, p.parts), (W + 1) * 64, 0, stream>>>(
            c, s, p.row_tiles, p.nchunks, image, exps, B, y, ldy, rows_out,
            std::size_t(ldy) * B, y_rows, keys, *fused);
  else
    Q8GemvImage<W, RT, kSwiGLU, SPW><<<dim3(p.groups, p.parts), W * 64, 0, stream>>>(
        c, s, p.row_tiles, p.nchunks, image, exps, B, y, ldy, rows_out,
        std::size_t(ldy) * B, y_rows, keys, FusedNorm{});
}

template<int W, bool kSwiGLU>
void LaunchImageRT(const GemvPlan& p, const std::uint8_t* c, const Half* s,
                   const uint4* image, const int* exps, int B, float* y, int ldy,
                   int rows_out, hipStream_t stream, float* const* y_rows,
                   unsigned long long* keys, const FusedNorm* fused) {
  if constexpr (kSwiGLU) {
    LaunchImagePlan<W, 2, true>(p, c, s, image, exps, B, y, ldy, rows_out, stream, y_rows, keys,
                                fused);
  } else {
    if (p.RT == 1)
      LaunchImagePlan<W, 1, false>(p, c, s, image, exps, B, y, ldy, rows_out, stream, y_rows,
                                   keys, fused);
    else
      LaunchImagePlan<W, 2, false>(p, c, s, image, exps, B, y, ldy, rows_out, stream, y_rows,
                                   keys, fused);
  }
}

GemvPlan PlanImage(std::uint32_t rows, std::uint32_t cols, bool swiglu, std::uint32_t parts) {
  GemvPlan p = PlanGemv(rows, cols, swiglu, int(parts));
  // Rounds of W * 4 chunks need no LDS: keep two tiles (one SwiGLU pair)
  // at most, so two blocks of eight waves fit a CU. With no operand
  // staging, a second tile only shares the cross-wave reduction, which
  // pays once the tiles outnumber the CUs: at 193 tiles (q | k | v | gate,
  // 3088 x 2048, 8 rows) one tile a block takes 4.8 us against 5.8 us with
  // two; at 8000 tiles (the vocabulary head) two take 60 us against 73 us
  // as one block a group (past kLoopGroups groups they run in
  // Q8GemvImageLoop).
  p.RT = swiglu ? 2 : p.row_tiles > 256 ? 2 : 1;
  p.groups = (p.row_tiles + p.RT - 1) / p.RT;
  return p;
}

template<bool kSwiGLU>
int LaunchGemvImage(const void* codes, const void* scales, std::uint32_t rows,
                    std::uint32_t cols, const void* image, const int* exps,
                    std::uint32_t batch, float* y, std::uint32_t ldy,
                    std::uint32_t parts, hipStream_t stream, float* const* y_rows = nullptr,
                    unsigned long long* keys = nullptr, const FusedNorm* fused = nullptr) {
  if (!codes || !scales || !image || !exps || (!y && !y_rows) || rows == 0 || cols == 0 ||
      cols % 32 || batch == 0 || batch > 8 || (!y_rows && ldy < rows) || parts < 1 ||
      parts > Chunks(cols) || (kSwiGLU && parts != 1) || ((y_rows || keys) && parts != 1) ||

      (reinterpret_cast<std::uintptr_t>(image) & 15) ||
      !BufferFits(std::size_t(RowTiles(rows) * (kSwiGLU ? 2 : 1)) * Chunks(cols) *
                  kTileCodeBytes))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 operand-image GEMV");
  const GemvPlan p = PlanImage(rows, cols, kSwiGLU, parts);
  if (fused && (parts != 1 || !FusedNormFits(*fused, cols, unsigned(p.W + 1) * 64)))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 fused norm + operand-image GEMV");
  const auto* c = static_cast<const std::uint8_t*>(codes);
  const auto* s = static_cast<const Half*>(scales);
  const auto* im = static_cast<const uint4*>(image);
  const int B = int(batch), ly = int(ldy), ro = int(rows);
  if (p.W == 8)
    LaunchImageRT<8, kSwiGLU>(p, c, s, im, exps, B, y, ly, ro, stream, y_rows, keys, fused);
  else if (p.W == 4)
    LaunchImageRT<4, kSwiGLU>(p, c, s, im, exps, B, y, ly, ro, stream, y_rows, keys, fused);
  else if (p.W == 2)
    LaunchImageRT<2, kSwiGLU>(p, c, s, im, exps, B, y, ly, ro, stream, y_rows, keys, fused);
  else
    LaunchImageRT<1, kSwiGLU>(p, c, s, im, exps, B, y, ly, ro, stream, y_rows, keys, fused);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 operand-image GEMV launch");
}

// Embedding rows from the tiled table: element k of row r sits in tile
// (r / 16, k / 64) at lane 16 (k % 32 / 8) + r % 16, byte 8 (k % 64 / 32)
// + k % 8.
__global__ void EmbedKernel(const std::uint8_t* __restrict__ codes,
                            const Half* __restrict__ scales, int nchunks,
                            int hidden, int vocab,
                            const std::uint32_t* __restrict__ tokens, int n,
                            float* __restrict__ out) {
  const int row = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= n || k >= hidden)
    return;
  std::uint32_t token = tokens[row];
  if (token >= std::uint32_t(vocab))
    token = 0;  // the host validates ids; never read out of bounds
  const int rt = token / kTileRows, nn = token % kTileRows;
  const int chunk = k / kChunk, within = k % kChunk, blk = within / 32;
  const int e = within % 32, g = e / 8, j = e % 8;
  const std::size_t tile = std::size_t(rt) * nchunks + chunk;
  const int q = int(codes[tile * kTileCodeBytes + (g * 16 + nn) * 16 + blk * 8 + j]) - 128;
  const float d = HalfBitsToFloat(scales[tile * kTileScales + nn * 2 + blk]);
  out[std::size_t(row) * hidden + k] = d * float(q);
}

}  // namespace

std::uint32_t HeadGemvGroups(std::uint32_t rows, std::uint32_t cols) {
  return std::uint32_t(PlanImage(rows, cols, false, 1).groups);
}

int LaunchHeadGemv(const void* codes, const void* scales, std::uint32_t rows,
                   std::uint32_t cols, const void* image, const int* exps, std::uint32_t batch,
                   float* const* y_rows, unsigned long long* keys, std::uint32_t* groups,
                   hipStream_t stream, const FusedNorm* fused) {
  if (!y_rows || !keys)
    return Fail(LFM3_E_INVALID, "LFM3 head GEMV needs its row table and key buffer");
  if (groups)
    *groups = HeadGemvGroups(rows, cols);
  return LaunchGemvImage<false>(codes, scales, rows, cols, image, exps, batch, nullptr, 0, 1,
                                stream, y_rows, keys, fused);
}

// A fused launch runs at most 8 compute waves a block (with its loader
// wave, at most 9 of the 16 a block may have).
template<int W>
void LaunchConvPlan(dim3 grid, const std::uint8_t* c, const Half* s, int third, int nchunks,
                    const uint4* im, const int* exps, int B, const float* taps,
                    float* const* history, int L, int H, float* y, int ly,
                    const FusedNorm* fused, hipStream_t st) {
  constexpr int WF = W > 8 ? 8 : W;
  if (fused)
    Q8GemvConvImage<WF, true><<<dim3(grid.x + B), (WF + 1) * 64, 0, st>>>(
        c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly, *fused);
  else
    Q8GemvConvImage<W><<<grid, W * 64, 0, st>>>(c, s, third, nchunks, im, exps, B, taps, history,
                                               L, H, y, ly, FusedNorm{});
}

int LaunchConvImage(const void* codes, const void* scales, std::uint32_t hidden,
                    const void* image, const int* exps, std::uint32_t batch, const float* taps,
                    float* const* history, std::uint32_t width, float* y, std::uint32_t ldy,
                    const FusedNorm* fused, hipStream_t st) {
  if (!codes || !scales || !image || !exps || !taps || !history || !y || !hidden ||
      hidden % kTileRows || batch == 0 || batch > 8 || width < 2 || width > 32 ||
      ldy < hidden || (reinterpret_cast<std::uintptr_t>(image) & 15) ||
      !BufferFits(std::size_t(RowTiles(3 * hidden)) * Chunks(hidden) * kTileCodeBytes))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 projection + convolution shape");
  const int third = int(hidden / kTileRows), nchunks = int(Chunks(hidden));
  // One block per 16 channels: few blocks, so each takes 16 waves (two
  // chunks each of a 32-chunk round) for more loads in flight per CU.
  const int W = nchunks <= 4 ? 1 : nchunks <= 8 ? 2 : nchunks <= 16 ? 4 : nchunks <= 24 ? 8 : 16;
  if (fused && !FusedNormFits(*fused, hidden, unsigned(std::min(W, 8) + 1) * 64))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 fused norm + convolution projection");
  const auto* c = static_cast<const std::uint8_t*>(codes);
  const auto* s = static_cast<const Half*>(scales);
  const auto* im = static_cast<const uint4*>(image);
  const dim3 grid(third);
  const int B = int(batch), L = int(width), H = int(hidden), ly = int(ldy);
  if (W == 16)
    LaunchConvPlan<16>(grid, c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly,
                       fused, st);
  else if (W == 8)
    LaunchConvPlan<8>(grid, c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly, fused,
                      st);
  else if (W == 4)
    LaunchConvPlan<4>(grid, c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly, fused,
                      st);
  else if (W == 2)
    LaunchConvPlan<2>(grid, c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly, fused,
                      st);
  else
    LaunchConvPlan<1>(grid, c, s, third, nchunks, im, exps, B, taps, history, L, H, y, ly, fused,
                      st);
  return HipStatus(hipGetLastError(), "LFM3 projection + convolution launch");
}

// Blocks of a fused launch that are resident at once: two (W + 1)-wave
// blocks a CU. Past that the last blocks wait for a second dispatch wave
// behind blocks that spin on the norm, and the norm in its own launch is
// faster (at FFN 8192: 512 + 8 blocks, round 1.177 ms fused against 1.160).
static int FusedSlots() { return 2 * CuCount(); }

int LaunchGemvImageFused(const void* codes, const void* scales, std::uint32_t rows,
                         std::uint32_t cols, const void* image, const int* exps,
                         std::uint32_t batch, float* y, std::uint32_t ldy, bool swiglu,
                         const FusedNorm& fused, hipStream_t stream) {
  if (PlanImage(rows, cols, swiglu, 1).groups + int(batch) > FusedSlots()) {
    // The same results from the norm's own launch and the plain GEMV.
    const int status = LaunchNormImage(fused.args, batch, stream);
    if (status != LFM3_OK)
      return status;
    return swiglu ? LaunchGemvImage<true>(codes, scales, rows, cols, image, exps, batch, y, ldy,
                                          1, stream)
                  : LaunchGemvImage<false>(codes, scales, rows, cols, image, exps, batch, y, ldy,
                                           1, stream);
  }
  return swiglu ? LaunchGemvImage<true>(codes, scales, rows, cols, image, exps, batch, y, ldy, 1,
                                        stream, nullptr, nullptr, &fused)
                : LaunchGemvImage<false>(codes, scales, rows, cols, image, exps, batch, y, ldy, 1,
                                         stream, nullptr, nullptr, &fused);
}
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

void lfm3_q8_tiled_bytes(std::uint32_t rows, std::uint32_t cols,
                         std::size_t* code_bytes, std::size_t* scale_bytes) {
  const std::size_t tiles = std::size_t(RowTiles(rows)) * Chunks(cols);
  if (code_bytes)
    *code_bytes = tiles * kTileCodeBytes;
  if (scale_bytes)
    *scale_bytes = tiles * kTileScales * sizeof(Half);
}

int lfm3_q8_pack_host(const void* gguf, std::uint32_t rows, std::uint32_t cols,
                      void* codes_out, void* scales_out,
                      std::uint32_t tile_offset, std::uint32_t tile_stride) {
  if (!gguf || !codes_out || !scales_out || !rows || !cols || cols % 32 ||
      !tile_stride)
    return Fail(LFM3_E_INVALID, "invalid LFM3 Q8_0 pack");
  const auto* src = static_cast<const Q8Block*>(gguf);
  auto* codes = static_cast<std::uint8_t*>(codes_out);
  auto* scales = static_cast<Half*>(scales_out);
  const std::uint32_t nchunks = Chunks(cols), blocks = cols / 32;
  const std::uint32_t tiles = RowTiles(rows);
  const auto work = [&](std::uint32_t t0, std::uint32_t t1) {
    for (std::uint32_t tile = t0; tile < t1; ++tile) {
      const std::size_t dst_tile = tile_offset + std::size_t(tile) * tile_stride;
      for (std::uint32_t chunk = 0; chunk < nchunks; ++chunk) {
        const std::size_t dst = dst_tile * nchunks + chunk;
        std::uint8_t* out = codes + dst * kTileCodeBytes;
        Half* sc = scales + dst * kTileScales;
        for (std::uint32_t n = 0; n < 16; ++n) {
          const std::uint32_t row = tile * 16 + n;
          for (int blk = 0; blk < 2; ++blk) {
            const std::uint32_t b = chunk * 2 + blk;
            const bool live = row < rows && b < blocks;
            const Q8Block* block = live ? src + std::size_t(row) * blocks + b : nullptr;
            sc[n * 2 + blk] = live ? block->d : 0;
            for (int g = 0; g < 4; ++g)
              for (int j = 0; j < 8; ++j)
                out[(g * 16 + n) * 16 + blk * 8 + j] =
                    std::uint8_t((live ? std::uint8_t(block->q[8 * g + j]) : 0) ^ kCodeBias);
          }
        }
      }
    }
  };
  const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (tiles < 64 || threads == 1) {
    work(0, tiles);
  } else {
    std::vector<std::thread> pool;
    for (unsigned w = 0; w < threads; ++w)
      pool.emplace_back(work, std::uint32_t(std::uint64_t(tiles) * w / threads),
                        std::uint32_t(std::uint64_t(tiles) * (w + 1) / threads));
    for (auto& th : pool)
      th.join();
  }
  return LFM3_OK;
}

int lfm3_q8_pack_device(const void* gguf, std::uint32_t rows, std::uint32_t cols,
                        void* codes, void* scales, std::uint32_t tile_offset,
                        std::uint32_t tile_stride, void* stream) {
  if (!gguf || !codes || !scales || !rows || !cols || cols % 32 || !tile_stride)
    return Fail(LFM3_E_INVALID, "invalid LFM3 Q8_0 pack");
  const std::uint32_t nchunks = Chunks(cols), tiles = RowTiles(rows);
  const std::size_t units = std::size_t(tiles) * nchunks * 64;
  PackKernel<<<unsigned((units + 255) / 256), 256, 0,
               static_cast<hipStream_t>(stream)>>>(
      static_cast<const std::uint8_t*>(gguf), rows, cols,
      static_cast<std::uint8_t*>(codes), static_cast<Half*>(scales), nchunks,
      tiles, tile_offset, tile_stride);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 pack launch");
}

std::size_t lfm3_gemv_workspace_bytes(std::uint32_t rows, std::uint32_t cols,
                                      std::uint32_t batch) {
  // Every block covers the whole of K, so no launch needs partial sums.
  (void)rows;
  (void)cols;
  (void)batch;
  return 0;
}

int lfm3_q8_gemv(const void* codes, const void* scales, std::uint32_t rows,
                 std::uint32_t cols, const float* x, std::uint32_t ldx,
                 float* y, std::uint32_t ldy, std::uint32_t batch,
                 void* workspace, std::size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return LaunchGemv<false>(codes, scales, rows, cols, x, ldx, y, ldy, batch,
                           static_cast<hipStream_t>(stream));
}

std::uint32_t lfm3_q8_gemv_parts(std::uint32_t rows, std::uint32_t cols) {
  if (!rows || !cols)
    return 1;
  return std::uint32_t(GemvParts(rows, cols));
}

int lfm3_q8_gemv_partials(const void* codes, const void* scales,
                          std::uint32_t rows, std::uint32_t cols,
                          const float* x, std::uint32_t ldx, float* y,
                          std::uint32_t ldy, std::uint32_t batch,
                          std::uint32_t parts, void* stream) {
  return LaunchGemv<false>(codes, scales, rows, cols, x, ldx, y, ldy, batch,
                           static_cast<hipStream_t>(stream), int(parts));
}

std::size_t lfm3_operand_image_bytes(std::uint32_t cols) {
  return std::size_t(Chunks(cols)) * 2 * 64 * 16;
}

int lfm3_q8_gemv_image(const void* codes, const void* scales,
                       std::uint32_t rows, std::uint32_t cols,
                       const void* image, const int* exps,
                       std::uint32_t batch, float* y, std::uint32_t ldy,
                       std::uint32_t parts, void* stream) {
  return LaunchGemvImage<false>(codes, scales, rows, cols, image, exps, batch,
                                y, ldy, parts, static_cast<hipStream_t>(stream));
}

int lfm3_q8_gemv_conv_image(const void* codes, const void* scales, std::uint32_t hidden,
                            const void* image, const int* exps, std::uint32_t batch,
                            const float* taps, float* const* history, std::uint32_t width,
                            float* y, std::uint32_t ldy, void* stream) {
  return LaunchConvImage(codes, scales, hidden, image, exps, batch, taps, history, width, y, ldy,
                         nullptr, static_cast<hipStream_t>(stream));
}

std::size_t lfm3_norm_flags_bytes(void) { return kFlagWords * sizeof(unsigned); }

namespace {
// The C-ABI's fused norm arguments (lfm3_residual_norm_image's), checked as
// that call checks them.
int FusedArgs(const float* branch, std::uint32_t parts, std::size_t part_stride,
              const float* post_norm, float* x, const float* norm, float eps, void* image,
              int* exps, unsigned* flags, std::uint32_t seq, unsigned* wait_error,
              std::uint32_t batch, std::uint32_t hidden, FusedNorm& f) {
  if (!x || !norm || !image || !exps || !flags || !seq || !batch || batch > 8 || !hidden ||
      hidden % 32 || !parts || parts > std::uint32_t(kNormParts) ||
      (branch && parts > 1 && part_stride < std::size_t(batch) * hidden))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 fused norm arguments");
  f.args.branch = branch;
  f.args.parts = int(parts);
  f.args.part_stride = part_stride;
  f.args.post = branch ? post_norm : nullptr;
  f.args.x = x;
  f.args.weight = norm;
  f.args.H = int(hidden);
  f.args.eps = eps;
  f.args.image = static_cast<uint4*>(image);
  f.args.exps = exps;
  f.flags = flags;
  f.seq = seq;
  f.error = wait_error;
  return LFM3_OK;
}
}  // namespace

int lfm3_q8_gemv_image_norm(const float* branch, std::uint32_t parts, std::size_t part_stride,
                            const float* post_norm, float* x, const float* norm, float eps,
                            void* image, int* exps, unsigned* flags, std::uint32_t seq,
                            unsigned* wait_error, const void* codes, const void* scales,
                            std::uint32_t rows, std::uint32_t cols, int swiglu,
                            std::uint32_t batch, float* y, std::uint32_t ldy, void* stream) {
  FusedNorm f;
  const int e = FusedArgs(branch, parts, part_stride, post_norm, x, norm, eps, image, exps, flags,
                          seq, wait_error, batch, cols, f);
  if (e)
    return e;
  return LaunchGemvImageFused(codes, scales, rows, cols, image, exps, batch, y, ldy, swiglu != 0,
                              f, static_cast<hipStream_t>(stream));
}

int lfm3_q8_gemv_conv_image_norm(const float* branch, std::uint32_t parts,
                                 std::size_t part_stride, const float* post_norm, float* x,
                                 const float* norm, float eps, void* image, int* exps,
                                 unsigned* flags, std::uint32_t seq, unsigned* wait_error,
                                 const void* codes, const void* scales, std::uint32_t hidden,
                                 std::uint32_t batch, const float* taps, float* const* history,
                                 std::uint32_t width, float* y, std::uint32_t ldy,
                                 void* stream) {
  FusedNorm f;
  const int e = FusedArgs(branch, parts, part_stride, post_norm, x, norm, eps, image, exps, flags,
                          seq, wait_error, batch, hidden, f);
  if (e)
    return e;
  return LaunchConvImage(codes, scales, hidden, image, exps, batch, taps, history, width, y, ldy,
                         &f, static_cast<hipStream_t>(stream));
}

int lfm3_q8_gemv_swiglu_image(const void* codes, const void* scales,
                              std::uint32_t rows, std::uint32_t cols,
                              const void* image, const int* exps,
                              std::uint32_t batch, float* y, std::uint32_t ldy,
                              void* stream) {
  return LaunchGemvImage<true>(codes, scales, rows, cols, image, exps, batch,
                               y, ldy, 1, static_cast<hipStream_t>(stream));
}

int lfm3_q8_gemv_swiglu(const void* codes, const void* scales,
                        std::uint32_t rows, std::uint32_t cols, const float* x,
                        std::uint32_t ldx, float* y, std::uint32_t ldy,
                        std::uint32_t batch, void* workspace,
                        std::size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return LaunchGemv<true>(codes, scales, rows, cols, x, ldx, y, ldy, batch,
                          static_cast<hipStream_t>(stream));
}

int lfm3_embed(const void* codes, const void* scales, std::uint32_t vocab,
               std::uint32_t hidden, const std::uint32_t* tokens,
               std::uint32_t n, float* out, void* stream) {
  if (!codes || !scales || !tokens || !out || !vocab || !hidden ||
      hidden % 32 || !n)
    return Fail(LFM3_E_INVALID, "invalid LFM3 embedding gather");
  const dim3 grid((hidden + 255) / 256, n);
  EmbedKernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const std::uint8_t*>(codes), static_cast<const Half*>(scales),
      int(Chunks(hidden)), int(hidden), int(vocab), tokens, int(n), out);
  return HipStatus(hipGetLastError(), "LFM3 embedding launch");
}

}  // extern "C"
