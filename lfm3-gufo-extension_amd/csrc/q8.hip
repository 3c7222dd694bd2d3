// Q8_0 weights on gfx950: tile repack, the skinny decode GEMV on MFMA, and
// the embedding gather.
//
// GEMV design (B <= 8 FP32 rows). Each wave owns a K range of the matrix
// and turns its slice of x into a pair of fp16 MFMA operands: per token a
// power-of-two scale 2^e puts the range's maximum in [2^14, 2^15), hi =
// fp16(x 2^e) and lo = fp16((x 2^e - hi) 2^11), so hi + lo 2^-11 carries
// about 22 bits of every element and each code x hi product is exact in
// FP32. The 16 A rows of v_mfma_f32_16x16x32_f16 are the 8 tokens' hi and
// lo parts; its B operand is 16 weight rows of one Q8_0 block decoded
// exactly to fp16, so one MFMA is the per-block dot of 16 rows and the
// block scale applies as acc = fma(d, c, acc), as in the reference's
// block-wise sums (hip/ops.hip:671-856: sums += scale * block_dot). The
// weights stream once from HBM with one 16-byte load per lane per tile.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "common.hpp"

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
      bytes[blk * 8 + j] = live ? block[2 + 8 * g + j] : 0;
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

// Launch shape of one GEMV: R row tiles per block, S K-slices across
// blocks (merged in slice order by the last block of each row group),
// W waves per block each taking up to CPW 64-column chunks of the slice.
struct GemvPlan {
  int row_tiles, nchunks, groups, R, S, W, CPW;
};

GemvPlan PlanGemv(std::uint32_t rows, std::uint32_t cols, bool swiglu) {
  GemvPlan p{};
  p.row_tiles = int(RowTiles(rows)) * (swiglu ? 2 : 1);
  p.nchunks = int(Chunks(cols));
  p.R = swiglu ? 2 : (p.row_tiles >= 4096 ? 2 : 1);
  p.groups = (p.row_tiles + p.R - 1) / p.R;
  p.S = 1;
  // Enough blocks for the 256 CUs; each slice keeps at least 2 chunks.
  while (p.groups * p.S < 256 && p.S < 8 && p.nchunks / (p.S * 2) >= 2)
    p.S *= 2;
  for (;;) {
    const int cps = (p.nchunks + p.S - 1) / p.S;
    p.CPW = 1;
    while (p.CPW < 4 && (cps + p.CPW - 1) / p.CPW > 8)
      p.CPW *= 2;
    p.W = (cps + p.CPW - 1) / p.CPW;
    if (p.W <= 16)
      break;
    p.S *= 2;  // long rows: more slices rather than wider blocks
  }
  return p;
}

constexpr int kMaxWaves = 16;
// Ticket words at the start of every GEMV workspace (one per row group).
constexpr int kTicketGroups = 16384;

template<int CPW, int R, bool kSwiGLU>
__launch_bounds__(1024) __global__
    void Q8Gemv(const std::uint8_t* __restrict__ codes,
                const Half* __restrict__ scales, int row_tiles, int nchunks,
                int K, const float* __restrict__ x, int ldx, int B,
                float* __restrict__ y, int ldy, int rows_out,
                float* __restrict__ partial, unsigned* __restrict__ tickets) {
  __shared__ float red[kMaxWaves * R * 128];
  __shared__ float fin[R * 128];
  __shared__ bool s_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int i = lane & 15, g = lane >> 4, t = i & 7, part = i >> 3;
  const int group = blockIdx.x, slice = blockIdx.y, slices = gridDim.y;
  const int slice_begin = slice * nchunks / slices;
  const int slice_end = (slice + 1) * nchunks / slices;
  const int c0 = slice_begin + wave * CPW;

  // x of this wave's chunks, token t: elements 8g..8g+7 of block 2c (A
  // operand of the chunk's first MFMA) and of block 2c + 1 (second MFMA).
  // The first pass finds the range maximum; the second re-reads the same
  // lines from L1 and converts, so no FP32 copy stays live.
  const auto load8 = [&](int c, int blk, float (&v)[8]) {
    const int chunk = c0 + c;
    const int k = chunk * kChunk + blk * 32 + 8 * g;
    float4 lo4 = make_float4(0, 0, 0, 0), hi4 = lo4;
    if (chunk < slice_end && t < B && k < K) {
      const float4* src = reinterpret_cast<const float4*>(x + std::size_t(t) * ldx + k);
      lo4 = src[0];
      hi4 = src[1];
    }
    v[0] = lo4.x; v[1] = lo4.y; v[2] = lo4.z; v[3] = lo4.w;
    v[4] = hi4.x; v[5] = hi4.y; v[6] = hi4.z; v[7] = hi4.w;
  };
  float maximum = 0.0f;
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      float v[8];
      load8(c, blk, v);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        maximum = fmaxf(maximum, fabsf(v[j]));
    }
  // Lanes of one token: same t, any part and group.
  maximum = fmaxf(maximum, __shfl_xor(maximum, 8, 64));
  maximum = fmaxf(maximum, __shfl_xor(maximum, 16, 64));
  maximum = fmaxf(maximum, __shfl_xor(maximum, 32, 64));
  const int e = maximum > 0.0f ? 14 - ilogbf(maximum) : 0;
  h8 a[CPW][2];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      float v[8];
      load8(c, blk, v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float s = ldexpf(v[j], e);
        const _Float16 hi = static_cast<_Float16>(s);
        a[c][blk][j] = part ? static_cast<_Float16>((s - float(hi)) * 2048.0f) : hi;
      }
    }
  // Exponent of each output token (lane t holds token t).
  int et[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
    et[k] = __builtin_amdgcn_readlane(e, k);

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = zero;
    const int tile = group * R + r;
    if (tile >= row_tiles)
      continue;
    uint4 q[CPW];
    unsigned sc[CPW];
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int chunk = c0 + c;
      if (chunk < slice_end) {
        const std::size_t off = std::size_t(tile) * nchunks + chunk;
        q[c] = *reinterpret_cast<const uint4*>(codes + off * kTileCodeBytes + lane * 16);
        sc[c] = *reinterpret_cast<const unsigned*>(scales + off * kTileScales + i * 2);
      }
    }
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      if (c0 + c < slice_end) {
        const h8 w0 = EightCodes(q[c].x, q[c].y), w1 = EightCodes(q[c].z, q[c].w);
        const f4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][0], w0, zero, 0, 0, 0);
        const f4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][1], w1, zero, 0, 0, 0);
        const float d0 = HalfBitsToFloat(sc[c] & 0xffffu);
        const float d1 = HalfBitsToFloat(sc[c] >> 16);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          acc[r][v] = fmaf(d0, p0[v], acc[r][v]);
          acc[r][v] = fmaf(d1, p1[v], acc[r][v]);
        }
      }
    }
  }
  // D layout: lane L holds A rows 4 (L / 16) + v (tokens hi 0-7, lo 0-7)
  // of weight row L % 16. Undo the power-of-two scales, add lo to hi.
  const int tok0 = (g & 1) * 4, lo = g >> 1;
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int ex = (g & 1) ? et[4 + v] : et[v];
      float val = ldexpf(acc[r][v], -(ex + (lo ? 11 : 0)));
      val += __shfl_xor(val, 32, 64);
      if (lane < 32)
        red[(wave * R + r) * 128 + (tok0 + v) * 16 + i] = val;
    }
  }
  __syncthreads();
  // Outputs of the block: R tiles x 8 tokens x 16 rows, summed over the
  // waves in wave order; a block may have fewer threads than outputs.
  const int tid = threadIdx.x, threads = blockDim.x;
  for (int o = tid; o < R * 128; o += threads) {
    const int r = o / 128, idx = o % 128;
    float sum = 0.0f;
    for (int w = 0; w < waves; ++w)
      sum += red[(w * R + r) * 128 + idx];
    fin[o] = sum;
  }
  __syncthreads();
  if (slices > 1) {
    // Slices merge in slice order, so the result does not depend on which
    // block finishes last.
    float* mine = partial + (std::size_t(group) * slices + slice) * (R * 128);
    for (int o = tid; o < R * 128; o += threads)
      mine[o] = fin[o];
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = atomicAdd(tickets + group, 1u);
      s_last = prev == unsigned(slices - 1);
      if (s_last)
        tickets[group] = 0;
    }
    __syncthreads();
    if (!s_last)
      return;
    __threadfence();
    const float* all = partial + std::size_t(group) * slices * (R * 128);
    for (int o = tid; o < R * 128; o += threads) {
      float sum = 0.0f;
      for (int s = 0; s < slices; ++s)
        sum += __builtin_nontemporal_load(all + s * (R * 128) + o);
      fin[o] = sum;
    }
    __syncthreads();
  }
  if constexpr (kSwiGLU) {
    // Tile 2j is gate, tile 2j + 1 is up: the same rows j*16 + n.
    for (int o = tid; o < 128; o += threads) {
      const int tok = o / 16, n = o % 16, row = group * kTileRows + n;
      const float gv = fin[o], uv = fin[128 + o];
      if (tok < B && row < rows_out)
        y[std::size_t(tok) * ldy + row] = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
    }
  } else {
    for (int o = tid; o < R * 128; o += threads) {
      const int r = o / 128, idx = o % 128, tok = idx / 16, n = idx % 16;
      const int row = (group * R + r) * kTileRows + n;
      if (tok < B && row < rows_out)
        y[std::size_t(tok) * ldy + row] = fin[o];
    }
  }
}

template<bool kSwiGLU>
int LaunchGemv(const void* codes, const void* scales, std::uint32_t rows,
               std::uint32_t cols, const float* x, std::uint32_t ldx, float* y,
               std::uint32_t ldy, std::uint32_t batch, void* workspace,
               std::size_t workspace_bytes, hipStream_t stream) {
  if (!codes || !scales || !x || !y || rows == 0 || cols == 0 ||
      cols % 32 || batch == 0 || batch > 8 || ldx % 4 || ldx < cols ||
      ldy < rows || (reinterpret_cast<std::uintptr_t>(x) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 GEMV shape");
  const GemvPlan p = PlanGemv(rows, cols, kSwiGLU);
  unsigned* tickets = nullptr;
  float* partial = nullptr;
  if (p.S > 1) {
    if (p.groups > kTicketGroups)
      return Fail(LFM3_E_INVALID, "LFM3 GEMV has too many row groups to split");
    if (workspace_bytes < lfm3_gemv_workspace_bytes(rows, cols, batch) ||
        !workspace)
      return Fail(LFM3_E_INVALID, "LFM3 GEMV workspace too small");
    // A fixed ticket region, so calls of different shapes can share one
    // workspace: partial sums never land where another shape's tickets are.
    tickets = static_cast<unsigned*>(workspace);
    partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kTicketGroups * 4);
  }
  const dim3 grid(p.groups, p.S), block(p.W * 64);
  const auto* c = static_cast<const std::uint8_t*>(codes);
  const auto* s = static_cast<const Half*>(scales);
  const int rows_out = int(rows);
#define LFM3_GEMV(CPW, R)                                                     \
  Q8Gemv<CPW, R, kSwiGLU><<<grid, block, 0, stream>>>(                        \
      c, s, p.row_tiles, p.nchunks, int(cols), x, int(ldx), int(batch), y,   \
      int(ldy), rows_out, partial, tickets)
  if constexpr (kSwiGLU) {
    switch (p.CPW) {
      case 1: LFM3_GEMV(1, 2); break;
      case 2: LFM3_GEMV(2, 2); break;
      default: LFM3_GEMV(4, 2); break;
    }
  } else if (p.R == 1) {
    switch (p.CPW) {
      case 1: LFM3_GEMV(1, 1); break;
      case 2: LFM3_GEMV(2, 1); break;
      default: LFM3_GEMV(4, 1); break;
    }
  } else {
    switch (p.CPW) {
      case 1: LFM3_GEMV(1, 2); break;
      case 2: LFM3_GEMV(2, 2); break;
      default: LFM3_GEMV(4, 2); break;
    }
  }
#undef LFM3_GEMV
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 GEMV launch");
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
  const auto q = static_cast<std::int8_t>(
      codes[tile * kTileCodeBytes + (g * 16 + nn) * 16 + blk * 8 + j]);
  const float d = HalfBitsToFloat(scales[tile * kTileScales + nn * 2 + blk]);
  out[std::size_t(row) * hidden + k] = d * float(q);
}

}  // namespace
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
                    live ? std::uint8_t(block->q[8 * g + j]) : 0;
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
  (void)batch;
  std::size_t most = 0;
  for (bool swiglu : {false, true}) {
    const GemvPlan p = PlanGemv(rows, cols, swiglu);
    if (p.S == 1)
      continue;
    most = std::max(most, std::size_t(kTicketGroups) * 4 +
                              std::size_t(p.groups) * p.S * p.R * 128 * 4);
  }
  return most;
}

int lfm3_q8_gemv(const void* codes, const void* scales, std::uint32_t rows,
                 std::uint32_t cols, const float* x, std::uint32_t ldx,
                 float* y, std::uint32_t ldy, std::uint32_t batch,
                 void* workspace, std::size_t workspace_bytes, void* stream) {
  return LaunchGemv<false>(codes, scales, rows, cols, x, ldx, y, ldy, batch,
                           workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

int lfm3_q8_gemv_swiglu(const void* codes, const void* scales,
                        std::uint32_t rows, std::uint32_t cols, const float* x,
                        std::uint32_t ldx, float* y, std::uint32_t ldy,
                        std::uint32_t batch, void* workspace,
                        std::size_t workspace_bytes, void* stream) {
  return LaunchGemv<true>(codes, scales, rows, cols, x, ldx, y, ldy, batch,
                          workspace, workspace_bytes,
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
