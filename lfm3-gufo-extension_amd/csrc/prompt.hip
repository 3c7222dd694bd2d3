// Prompt pass on gfx950: the Q8_0 x FP16 projection GEMM on MFMA and the
// FP16 row-scaled activations that feed it.
//
// Activations (hip/q8_prefill.hpp:13-74): each row is scaled by the power
// of two 2^e that puts its maximum magnitude in [2^14, 2^15) (e = 14 -
// ilogb(max), 0 for an all-zero row), rounded to fp16, and carries the
// scale 2^-e. Every element keeps 11 significant bits relative to itself.
//
// GEMM: Y[t][r] = scale[t] * sum_blk d[r][blk] * (sum_{k in blk} q[r][k] *
// a[t][k]): per Q8_0 block one v_mfma_f32_16x16x32_f16 gives the exact
// code x half products summed in FP32 (A operand = 16 tokens' activations,
// B operand = 16 weight rows decoded exactly from the tiled layout), and
// the block scale applies as acc = fma(d, dot, acc) (q8_prefill.hpp:
// 538-560). A block of WR x WT waves owns 16 RT WR weight rows and 16 TT WT
// tokens (16 RT rows and 16 TT tokens a wave). Each chunk's activations,
// weight tiles and scales arrive by direct-to-LDS loads into a two- or
// three-stage pipeline, so registers hold only the accumulators and the
// operands being multiplied. Narrow outputs split K
// across blockIdx.z into parts written separately; their consumer adds the
// parts in part order, so no launch merges blocks through memory.
#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace lfm3amd {
namespace {

// Block shapes: WR x WT waves; each wave owns kGemmRT weight tiles (16
// rows each) and 16 TT tokens (kGemmTT unless the shape says otherwise).
// The wide shape (4 x 2 waves) covers 256 weight rows and 128 tokens: 128
// FLOP per staged byte (2 M N / (M + 2 N) for 1-byte codes and 2-byte
// activations), about one block per CU for the 512-token pass. The narrow
// shape (2 x 2 waves, 128 rows x 128 tokens) does a quarter of that work a
// block and two blocks fit a CU: projections with few output rows fill the
// 256 CUs with fewer K parts, and each part costs a full FP32 output pass.
constexpr int kGemmRT = 4, kGemmTT = 4, kGemmStages = 3;

// A block shape and its pipeline stage: the block's activation rows for
// one 64-column chunk (kTokens rows x 8 16-byte slots; slot j of row t
// holds segment j ^ (t & 7), so the A reads of 8 consecutive rows hit
// distinct banks), the block's weight tiles for the chunk (1 KB each, lane
// order), and their scales (256 B per group of 4 tiles, row n's 4 tiles at
// 16 n).
// With kHalf the weight tiles are FP16 tiles (2 KB: the 16 codes a lane
// holds, decoded once at load into block 0's eight halves at byte 16 L and
// block 1's at 1024 + 16 L), so the loop feeds them to the MFMA without the
// per-chunk decode; the operands, and so every product, are the same.
template<int WR, int WT, bool kHalf = false, int kStageCount = kGemmStages, int TT = kGemmTT>
struct GemmShape {
  static constexpr int kWR = WR, kWT = WT, kTT = TT;
  static constexpr bool kHalfTiles = kHalf;
  static constexpr int kStages = kStageCount;  // LDS pipeline stages: 2 or 3
  static constexpr int kWaves = WR * WT, kThreads = 64 * kWaves;
  static constexpr int kTiles = WR * kGemmRT;  // weight tiles a block
  static constexpr int kTokens = WT * TT * 16;
  static constexpr int kTileW = kHalf ? 2 * kTileCodeBytes : kTileCodeBytes;
  static constexpr int kW = kTokens * 128;
  static constexpr int kS = kW + kTiles * kTileW;
  static constexpr int kBytes = kS + kTiles * kTileScales * 2;
};
using WideShape = GemmShape<4, 2>;
using NarrowShape = GemmShape<2, 2>;
// The same 256 x 128 block tile on FP16 tiles in 16 waves of 64 rows x 32
// tokens: four waves a SIMD instead of two hide more of the LDS and MFMA
// latency, for half again the LDS operand reads a MFMA (the SwiGLU GEMM
// 54.9-56.8 us against 57.6-59.5 with 8 waves of 64 x 64, the pass 0.7-1.2%
// faster). The code-tile shapes stay at 8 and 4 waves: 16 and 8 waves made
// their projections slower (6144 x 2048: 31.2 us against 28.0).
using WideHalfShape = GemmShape<4, 4, true, kGemmStages, 2>;
// The narrow 128 x 128 block tile on FP16 tiles in 8 waves of 64 rows x 32
// tokens and three stages (100 KB of LDS: one block a CU). With every
// narrow projection of the 512-token pass on it the pass takes 4.22-4.30 ms
// against 4.35-4.41 on code tiles in 4-wave blocks (two a CU); the same
// 8 waves with two stages (two blocks a CU) 4.45-4.47, the 8-wave shape on
// code tiles 4.48.
using NarrowHalfShape = GemmShape<2, 4, true, kGemmStages, 2>;

// One block per row: row maximum (scanned, or the maximum of max_blocks
// partial maxima), then fp16(x 2^e) and the scale 2^-e. The vector form
// (cols % 4 == 0, cols <= 8192, 16-byte aligned rows) holds the row in
// registers as float4 (one read) and stores four halves at a time.
constexpr int kHalfThreads = 256, kHalfVec = 8;  // float4 a thread: 8192 columns
constexpr int kHalfSplit = 4;  // blocks a row with known maxima: 2048 columns each

__device__ __forceinline__ float BlockMaximum256(float v, float* s_max) {
  v = WaveMax(v);
  if ((threadIdx.x & 63) == 0)
    s_max[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
}

// The row's maximum from max_blocks partial maxima: one load per thread,
// then a block maximum (a serial loop would chain max_blocks loads).
__device__ __forceinline__ float RowMaximum(const unsigned* __restrict__ row_max,
                                            int max_blocks, int rows, int row, float* s_max) {
  float maximum = 0.0f;
  for (int b = threadIdx.x; b < max_blocks; b += kHalfThreads)
    maximum = fmaxf(maximum, __uint_as_float(row_max[std::size_t(b) * rows + row]));
  return BlockMaximum256(maximum, s_max);
}

template<bool kVec>
__launch_bounds__(kHalfThreads) __global__
    void HalfRowsKernel(const float* __restrict__ x, int ldx,
                        const unsigned* __restrict__ row_max, int max_blocks,
                        Half* __restrict__ out, int lda,
                        float* __restrict__ scale, int K) {
  __shared__ float s_max[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* src = x + std::size_t(row) * ldx;
  Half* dst = out + std::size_t(row) * lda;
  if constexpr (kVec) {
    // With known maxima a row spreads over blocks of 2048 columns
    // (blockIdx.y); a scanned row is one block.
    const int per = gridDim.y == 1 ? K / 4 : kHalfThreads * kHalfVec / kHalfSplit;
    const int v0 = blockIdx.y * per;
    const int nv = min(K / 4, v0 + per);
    // Loads and stores through buffer resources, without branches (a
    // branch around a store makes the compiler wait for the stores before
    // the next one).
    const BufferResource src_res = MakeBuffer(src, unsigned(K) * 4u);
    const BufferResource dst_res = MakeBuffer(dst, unsigned((K + kChunk - 1) / kChunk * kChunk) * 2u);
    float4 v[kHalfVec];
#pragma unroll
    for (int j = 0; j < kHalfVec; ++j) {
      const int i = v0 + tid + kHalfThreads * j;
      v[j] = LoadF4(src_res, i < nv ? unsigned(i) * 16u : kOutOfRange);
    }
    float maximum;
    if (row_max) {
      maximum = RowMaximum(row_max, max_blocks, gridDim.x, row, s_max);
    } else {
      maximum = 0.0f;
#pragma unroll
      for (int j = 0; j < kHalfVec; ++j)
        maximum = fmaxf(maximum, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)),
                                       fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
      maximum = BlockMaximum256(maximum, s_max);
    }
    const int e = RowExponent(maximum);
    if (tid == 0 && blockIdx.y == 0)
      scale[row] = ldexpf(1.0f, -e);
#pragma unroll
    for (int j = 0; j < kHalfVec; ++j) {
      const int i = v0 + tid + kHalfThreads * j;
      StoreB64(dst_res, i < nv ? unsigned(i) * 8u : kOutOfRange,
               make_uint2(unsigned(ScaledHalf(v[j].x, e)) | (unsigned(ScaledHalf(v[j].y, e)) << 16),
                          unsigned(ScaledHalf(v[j].z, e)) | (unsigned(ScaledHalf(v[j].w, e)) << 16)));
    }
    if (blockIdx.y + 1 == gridDim.y)  // the zero tail of the last chunk
      for (int i = K / 4 + tid; i < (K + kChunk - 1) / kChunk * (kChunk / 4); i += kHalfThreads)
        StoreB64(dst_res, unsigned(i) * 8u, make_uint2(0u, 0u));
  } else {
    float maximum;
    if (row_max) {
      maximum = RowMaximum(row_max, max_blocks, gridDim.x, row, s_max);
    } else {
      maximum = 0.0f;
      for (int k = tid; k < K; k += kHalfThreads)
        maximum = fmaxf(maximum, fabsf(src[k]));
      maximum = BlockMaximum256(maximum, s_max);
    }
    const int e = RowExponent(maximum);
    if (tid == 0)
      scale[row] = ldexpf(1.0f, -e);
    for (int k = tid; k < (K + kChunk - 1) / kChunk * kChunk; k += kHalfThreads)
      dst[k] = k < K ? ScaledHalf(src[k], e) : Half(0);
  }
}

// Direct-to-LDS buffer loads (buffer_load_dword{,x4} ... lds): lane L's
// bytes land at the wave-uniform LDS base (M0) + L * size. Reads outside
// the resource's byte range return zero. Issued as inline assembly: the
// compiler's wait insertion cannot tell which stage a DMA load writes, and
// for the builtin it waited on the loads of later stages before reading an
// earlier one (vmcnt(0) every third chunk). The pipeline waits explicitly
// instead. One wait state separates the M0 write from the load.
typedef __attribute__((address_space(3))) void LdsVoid;
__device__ __forceinline__ unsigned LdsAddress(void* p) {
  return unsigned(reinterpret_cast<std::uintptr_t>((LdsVoid*)p));
}
__device__ __forceinline__ void BufferToLds16(BufferResource res, unsigned lane_offset,
                                              unsigned scalar_offset, void* lds_base) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(lane_offset), "s"(res), "s"(scalar_offset), "{m0}"(LdsAddress(lds_base))
               : "memory");
}
__device__ __forceinline__ void BufferToLds4(BufferResource res, unsigned lane_offset,
                                             unsigned scalar_offset, void* lds_base) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds"
               :
               : "v"(lane_offset), "s"(res), "s"(scalar_offset), "{m0}"(LdsAddress(lds_base))
               : "memory");
}


__device__ __forceinline__ void BlockBarrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Block b of a launch -> work item, XCD-major: blocks are dispatched to
// the 8 XCDs round robin (b % 8), so XCD x gets the consecutive items
// [first(x), first(x) + count(x)); items sharing weight rows are adjacent,
// so their tiles come from HBM once per XCD and then from its L2.
__device__ __forceinline__ int XcdMajorItem(int b, int blocks) {
  const int q = blocks / 8, rem = blocks % 8, x = b % 8, i = b / 8;
  return (x < rem ? x * (q + 1) : rem * (q + 1) + (x - rem) * q) + i;
}

// The SwiGLU GEMM's trailing blocks (lfm3_q8_gemm_swiglu_h16_rows): after
// the GEMM blocks of a launch (blockIdx.x < gemm_blocks), each further
// block converts kHiddenRows rows of the FFN hidden output into the down
// projection's FP16 row-scaled activations (HalfRowsKernel's expressions,
// the row maximum from the epilogue's partial maxima). A GEMM block stores
// its outputs and partial maxima through to memory (sc1), waits for them,
// and then stores `seq` into its flag (flags[tb * row_blocks + rb]); a
// converter block waits for the flags of every GEMM block of its token
// block. The converters come after every GEMM block in dispatch order and
// the GEMM blocks wait on nothing, so every wait ends; each is bounded
// (kGemmSpinLimit polls, then error set to 1 and the block goes on).
struct HiddenHalves {
  Half* out = nullptr;  // null: a plain SwiGLU launch
  int lda = 0;
  float* scale = nullptr;
  unsigned* flags = nullptr;
  unsigned seq = 0;
  unsigned* error = nullptr;
  int gemm_blocks = 0;
};
// Two rows a trailing block (256 blocks for 512 rows): the 512-token pass
// at 4.59 ms against 4.60 with 4 rows, 4.61 with 8 or 1, and 4.65 with the
// conversion as a launch of its own (three runs each, one box).
constexpr int kHiddenRows = 2, kHiddenMaxCols = 8192;
constexpr int kGemmSpinLimit = 1 << 20;

// A trailing block of the SwiGLU GEMM: rows r0 .. r0 + kHiddenRows - 1 of
// y (cols = the FFN width) once every GEMM block of their token block has
// published. Loads read memory (sc1), where the GEMM blocks wrote.
template<int T, int kTokens>
__device__ __forceinline__ void ConvertHidden(const HiddenHalves& t, const float* y, int ldy,
                                              int cols, int n, const unsigned* row_max,
                                              int row_blocks) {
  static_assert(kTokens % kHiddenRows == 0, "a converter's rows lie in one token block");
  constexpr int kHiddenLoads = kHiddenMaxCols / 4 / T;
  __shared__ float s_rmax[kHiddenRows][T / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r0 = (int(blockIdx.x) - t.gemm_blocks) * kHiddenRows;
  const int tb = r0 / kTokens;
  if (wave == 0) {
    const BufferResource f_res =
        MakeBuffer(t.flags + std::size_t(tb) * row_blocks, unsigned(row_blocks) * 4u);
    int spins = 0;
    for (;;) {
      bool mine = true;
      for (int k = lane; k < row_blocks; k += 64)
        mine = mine && __builtin_amdgcn_raw_buffer_load_b32(f_res, unsigned(k) * 4u, 0,
                                                            kCachePolicySc1) == t.seq;
      if (__all(mine))
        break;
      if (++spins >= kGemmSpinLimit) {
        if (lane == 0 && t.error)
          __hip_atomic_store(t.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(4);
    }
  }
  __syncthreads();
  // Each row's maximum over the partial maxima of the row blocks.
  const BufferResource m_res = MakeBuffer(row_max, unsigned(row_blocks) * unsigned(n) * 4u);
  float part[kHiddenRows];
#pragma unroll
  for (int i = 0; i < kHiddenRows; ++i) {
    const int r = r0 + i;
    float m = 0.0f;
    for (int b = tid; b < row_blocks; b += T)
      m = fmaxf(m, __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                       m_res, r < n ? unsigned(b * n + r) * 4u : kOutOfRange, 0,
                       kCachePolicySc1)));
    part[i] = WaveMax(m);
  }
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < kHiddenRows; ++i)
      s_rmax[i][wave] = part[i];
  __syncthreads();
  // Every row's values are loaded before the first conversion (at most
  // kHiddenLoads 16-byte loads a row and thread: cols <= kHiddenMaxCols), so
  // the block waits on memory once.
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const BufferResource y_res = MakeBuffer(y, unsigned(n) * unsigned(ldy) * 4u);
  u4 w[kHiddenRows][kHiddenLoads];
#pragma unroll
  for (int i = 0; i < kHiddenRows; ++i)
#pragma unroll
    for (int j = 0; j < kHiddenLoads; ++j) {
      const int r = r0 + i, v = tid + T * j;
      w[i][j] = __builtin_amdgcn_raw_buffer_load_b128(
          y_res, r < n && v < cols / 4 ? unsigned(std::size_t(r) * ldy + 4 * v) * 4u : kOutOfRange,
          0, kCachePolicySc1);
    }
  const int padded = (cols + kChunk - 1) / kChunk * kChunk;
#pragma unroll
  for (int i = 0; i < kHiddenRows; ++i) {
    const int r = r0 + i;
    if (r >= n)
      break;
    float maximum = 0.0f;
#pragma unroll
    for (int q = 0; q < T / 64; ++q)
      maximum = fmaxf(maximum, s_rmax[i][q]);
    const int e = RowExponent(maximum);
    if (tid == 0)
      t.scale[r] = ldexpf(1.0f, -e);
    Half* dst = t.out + std::size_t(r) * t.lda;
#pragma unroll
    for (int j = 0; j < kHiddenLoads; ++j) {
      const int v = tid + T * j;
      if (v < cols / 4)
        *reinterpret_cast<uint2*>(dst + 4 * v) = make_uint2(
            unsigned(ScaledHalf(__uint_as_float(w[i][j].x), e)) |
                (unsigned(ScaledHalf(__uint_as_float(w[i][j].y), e)) << 16),
            unsigned(ScaledHalf(__uint_as_float(w[i][j].z), e)) |
                (unsigned(ScaledHalf(__uint_as_float(w[i][j].w), e)) << 16));
    }
    for (int k = cols + tid; k < padded; k += T)  // the zero tail of the last chunk
      dst[k] = Half(0);
  }
}

// Pins 16 accumulators at this point: the FMAs producing them run before
// it and the values stay in their registers.
#define LFM3_PIN4(a) "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3])

template<bool kSwiGLU, class Shape>
__launch_bounds__(Shape::kThreads) __attribute__((amdgpu_waves_per_eu(2)))
__global__ void Q8GemmKernel(const std::uint8_t* __restrict__ codes,
                             const Half* __restrict__ scales, int row_tiles,
                             int nchunks, const Half* __restrict__ a, int lda,
                             const float* __restrict__ a_scale, int n,
                             float* __restrict__ y, int ldy, int rows_out,
                             int row_blocks, int token_blocks, int parts,
                             std::size_t part_stride,
                             unsigned* __restrict__ row_max, const HiddenHalves tail) {
  constexpr int RT = kGemmRT, TT = Shape::kTT;
  using Stage = Shape;
  constexpr int A_LOADS = Shape::kTokens * 8 / Shape::kThreads;  // 16-byte loads a lane
  constexpr int W_LOADS = Shape::kTiles / Shape::kWaves;         // tiles a wave loads
  constexpr int kTileW = Shape::kTileW;                           // bytes of a tile's chunk
  constexpr int W_PIECES = kTileW / kTileCodeBytes;               // 1 KB loads a tile
  static_assert(A_LOADS * Shape::kThreads == Shape::kTokens * 8, "A loads cover the rows");
  static_assert(W_LOADS * Shape::kWaves == Shape::kTiles, "W loads cover the tiles");
  static_assert(RT == 4 && Shape::kWR <= Shape::kWaves, "scale groups of four tiles");
  // One array per stage (not one indexed by stage) lets the compiler see
  // that a stage's reads never alias the other stages' loads in flight.
  __shared__ __attribute__((aligned(16))) std::uint8_t s_st0[Stage::kBytes];
  __shared__ __attribute__((aligned(16))) std::uint8_t s_st1[Stage::kBytes];
  __shared__ __attribute__((aligned(16))) std::uint8_t s_st2[Shape::kStages == 3 ? Stage::kBytes : 16];
  static_assert(Shape::kStages == 2 || Shape::kStages == 3, "two or three stage arrays");

  const bool publish = kSwiGLU && tail.out != nullptr;
  if constexpr (kSwiGLU) {
    if (publish && int(blockIdx.x) >= tail.gemm_blocks) {
      ConvertHidden<Shape::kThreads, Shape::kTokens>(tail, y, ldy, rows_out, n, row_max,
                                                     row_blocks);
      return;
    }
  }
  const int item = XcdMajorItem(blockIdx.x, publish ? tail.gemm_blocks : int(gridDim.x));
  const int tb = item % token_blocks, rb = (item / token_blocks) % row_blocks;
  const int part = item / (token_blocks * row_blocks);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave % Shape::kWR, wt = wave / Shape::kWR;
  const int btile0 = rb * Shape::kTiles;              // the block's first tile
  const int tile0 = btile0 + wr * RT;              // this wave's first tile
  const int tok0 = tb * Shape::kTokens;               // the block's first token
  const int c_begin = part * nchunks / parts, c_end = (part + 1) * nchunks / parts;
  y += std::size_t(part) * part_stride;

  // Sources as buffer resources (scalar registers), a scalar offset per
  // chunk and tile, and a 32-bit byte offset per lane: no 64-bit lane
  // addresses live across the loop. Rows past the last token and tiles
  // past the last tile read the last valid one; their results are
  // discarded. The host keeps every operand under 2 GiB.
  const BufferResource a_res = MakeBuffer(a + std::size_t(tok0) * lda,
                                          unsigned(n - tok0) * unsigned(lda) * 2u);
  const BufferResource w_res = MakeBuffer(codes, unsigned(row_tiles) * unsigned(nchunks) *
                                                     unsigned(kTileW));
  const BufferResource s_res = MakeBuffer(scales, unsigned(row_tiles) * unsigned(nchunks) *
                                                      unsigned(kTileScales * 2));
  unsigned a_off[A_LOADS];
#pragma unroll
  for (int j = 0; j < A_LOADS; ++j) {
    const int t = (wave * A_LOADS + j) * 8 + (lane >> 3);
    const int seg = (lane & 7) ^ (t & 7);
    a_off[j] = (unsigned(min(t, n - 1 - tok0)) * unsigned(lda) + unsigned(seg * 8)) * 2u;
  }
  unsigned w_tile[W_LOADS];  // byte offset of each loaded tile's chunk 0 (uniform)
#pragma unroll
  for (int j = 0; j < W_LOADS; ++j)
    w_tile[j] = unsigned(min(btile0 + wave * W_LOADS + j, row_tiles - 1)) *
                unsigned(nchunks * kTileW);
  const unsigned w_off = unsigned(lane) * 16u;
  // Scales: wave g < Shape::kWR loads group g; lane L brings tile 4 g + L % 4's
  // dword L / 4 (row L / 4's two block scales).
  const bool loads_scales = wave < Shape::kWR;
  const unsigned s_off =
      unsigned(min(btile0 + wave * 4 + (lane & 3), row_tiles - 1)) *
          unsigned(nchunks * kTileScales * 2) +
      unsigned((lane >> 2) * 4);
  const auto issue = [&](int c, std::uint8_t* stage) {
#pragma unroll
    for (int j = 0; j < A_LOADS; ++j)
      BufferToLds16(a_res, a_off[j], unsigned(c * kChunk * 2),
                    stage + (wave * A_LOADS + j) * 1024);
#pragma unroll
    for (int j = 0; j < W_LOADS; ++j)
#pragma unroll
      for (int piece = 0; piece < W_PIECES; ++piece)
        BufferToLds16(w_res, w_off, w_tile[j] + unsigned(c * kTileW + piece * kTileCodeBytes),
                      stage + Stage::kW + (wave * W_LOADS + j) * kTileW + piece * kTileCodeBytes);
    if (loads_scales)
      BufferToLds4(s_res, s_off, unsigned(c * kTileScales * 2),
                   stage + Stage::kS + wave * 4 * kTileScales * 2);
  };
  // Waits until at most one chunk's loads of this wave remain in flight.
  const auto wait_all_but_one_chunk = [&]() {
    if (loads_scales)
      __builtin_amdgcn_s_waitcnt(WaitVm(A_LOADS + W_LOADS * W_PIECES + 1));
    else
      __builtin_amdgcn_s_waitcnt(WaitVm(A_LOADS + W_LOADS * W_PIECES));
  };

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // Scalars, not f4: updating one lane of a 4-register tuple at a time
  // makes the register allocator copy whole tuples.
  float acc[RT][TT][4];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        acc[r][t][i] = 0.0f;

  // A read of lane L: row wt 16 TT + 16 t + L % 16, segment 4 blk + L / 16,
  // stored in slot segment ^ (L & 7).
  const int a_row = wt * TT * 16 + (lane & 15);
  // The previous chunk's last MFMA results and block scales, scaled into
  // acc[.][TT - 1] at the next chunk's first step (before the first chunk:
  // zero products at scale 0, which leave the zero accumulators as they
  // are).
  f4 last[RT];
  unsigned last_sc[RT];
  // acc += d * p, with d the block's fp16 scale (the low half of the
  // tile's scale dword d2 for block 0, the high half for block 1) read by
  // v_fma_mix_f32 as an exact FP32 value: one rounding, as the conversion
  // followed by an FMA, without the conversion and shift. Written as
  // assembly tied to the accumulator so it updates in place.
  const auto scale_fma = [](float& a, unsigned d2, float p, int blk) {
    if (blk)
      asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
          : "+v"(a) : "v"(d2), "v"(p));
    else
      asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,0,0] op_sel_hi:[1,0,0]"
          : "+v"(a) : "v"(d2), "v"(p));
  };
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    last[r] = zero;
    last_sc[r] = 0u;
  }
  const auto compute = [&](const std::uint8_t* stage) {
    uint4 q[RT];
    if constexpr (!Shape::kHalfTiles) {
#pragma unroll
      for (int r = 0; r < RT; ++r)
        q[r] = *reinterpret_cast<const uint4*>(stage + Stage::kW +
                                               (wr * RT + r) * kTileW + lane * 16);
    }
    // Q8_0 block blk's operands: the B operand of tile r, and the A operand
    // of token group t (lane L: row wt 16 TT + 16 t + L % 16, segment
    // 4 blk + L / 16, stored in slot segment ^ (L & 7)).
    const auto w_frag = [&](int blk, int r) -> h8 {
      if constexpr (Shape::kHalfTiles)
        return *reinterpret_cast<const h8*>(stage + Stage::kW + (wr * RT + r) * kTileW +
                                            blk * kTileCodeBytes + lane * 16);
      else
        return blk ? EightCodes(q[r].z, q[r].w) : EightCodes(q[r].x, q[r].y);
    };
    const auto a_frag = [&](int blk, int t) {
      const int slot = (blk * 4 + (lane >> 4)) ^ (lane & 7);
      return *reinterpret_cast<const h8*>(stage + (t * 16 + a_row) * 128 + slot * 16);
    };
    unsigned sc[4];
    // The first step's operands are read first, in the order the MFMAs
    // take them (the first MFMA waits for its A fragment and tile 0 only),
    // then the scales.
    h8 av = a_frag(0, 0);
    h8 w[RT], wn[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      __builtin_amdgcn_sched_barrier(0);
      w[r] = w_frag(0, r);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint4 sc4 = *reinterpret_cast<const uint4*>(
        stage + Stage::kS + wr * RT * kTileScales * 2 + (lane & 15) * 16);
    sc[0] = sc4.x;
    sc[1] = sc4.y;
    sc[2] = sc4.z;
    sc[3] = sc4.w;
    // One software pipeline over the chunk's 2 TT steps (block 0's token
    // groups, then block 1's): the MFMAs of step s issue beside the scale
    // FMAs of step s - 1, in a fixed order (the A read for s + 1, then each
    // MFMA of s followed by the 4 FMAs of s - 1 on the previous MFMA's
    // tile), so the matrix pipe runs while the VALU works; block 1's tiles
    // are read during block 0's second step. The FMAs of the chunk's last
    // step run in the next chunk's first step (last, last_sc), after the
    // block barrier, beside that chunk's first MFMAs; each accumulator still
    // takes its block products in K order. The scheduling barriers also
    // keep the compiler from hoisting every MFMA of the chunk (which would
    // hold 8 RT TT result registers).
    f4 prev[RT];
#pragma unroll
    for (int step = 0; step < 2 * TT; ++step) {
      const int blk = step / TT, t = step % TT;
      const int pblk = (step - 1) / TT, pt = (step + TT - 1) % TT;  // step - 1
      const h8 next = step + 1 < 2 * TT ? a_frag((step + 1) / TT, (step + 1) % TT) : av;
      if (step == 1) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
          wn[r] = w_frag(1, r);
      }
      if (step == TT) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
          w[r] = wn[r];
      }
      f4 cur[RT];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        cur[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, w[r], zero, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (step > 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            scale_fma(acc[r][pt][i], sc[r], prev[r][i], pblk);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            scale_fma(acc[r][TT - 1][i], last_sc[r], last[r][i], 1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < RT; ++r)
        prev[r] = cur[r];
      av = next;
      (void)blk;
      (void)t;
    }
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      last[r] = prev[r];
      last_sc[r] = sc[r];
    }
  };
  // Three-stage pipeline, unrolled so each stage is a fixed array. Step c:
  // wait until chunk c's loads are done (chunk c + 1's may remain in
  // flight), barrier (chunk c visible to every wave, and every wave done
  // with chunk c - 1), issue chunk c + 2 into chunk c - 1's stage, then
  // multiply chunk c. Loads get two chunks' compute to arrive.
  issue(c_begin, s_st0);
  if constexpr (Shape::kStages == 2) {
    // Two stages: step c waits for chunk c (the only loads in flight),
    // barrier (every wave done with chunk c - 1's stage), issues chunk
    // c + 1 into it, then multiplies chunk c.
    const auto step2 = [&](int c, std::uint8_t* stage, std::uint8_t* refill) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(WaitVm(0));
      BlockBarrier();
      if (c + 1 < c_end)
        issue(c + 1, refill);
      compute(stage);
      __builtin_amdgcn_sched_barrier(0);
    };
    int c = c_begin;
    for (; c + 2 <= c_end; c += 2) {
      step2(c, s_st0, s_st1);
      step2(c + 1, s_st1, s_st0);
    }
    if (c < c_end)
      step2(c, s_st0, s_st1);
  } else {
  if (c_begin + 1 < c_end)
    issue(c_begin + 1, s_st1);
  const auto step = [&](int c, std::uint8_t* stage, std::uint8_t* refill) {
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < c_end)
      wait_all_but_one_chunk();
    else
      __builtin_amdgcn_s_waitcnt(WaitVm(0));
    // Nothing counted by lgkmcnt is in flight here; the wait says so to the
    // compiler's wait insertion on every path into the step, so the step's
    // first MFMA waits for its own LDS operands, not for all of them.
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    BlockBarrier();
    if (c + 2 < c_end)
      issue(c + 2, refill);
    compute(stage);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Whole rounds of three chunks, then the ones left (no exits from inside
  // a round).
  int c = c_begin;
  for (; c + 3 <= c_end; c += 3) {
    step(c, s_st0, s_st2);
    step(c + 1, s_st1, s_st0);
    step(c + 2, s_st2, s_st1);
  }
  if (c < c_end)
    step(c, s_st0, s_st2);
  if (c + 1 < c_end)
    step(c + 1, s_st1, s_st0);
  }

  // The last chunk's last step.
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      scale_fma(acc[r][TT - 1][i], last_sc[r], last[r][i], 1);

  // D layout: lane L holds tokens 16 t + 4 (L / 16) + i of weight row L % 16.
  const int sub = lane & 15, quad = lane >> 4;
  const int wtok0 = tok0 + wt * TT * 16;
  // The lane's token scales (0 past the last token), all loaded before the
  // first store, and stores without branches (an output outside the
  // matrix goes to an offset the hardware drops): loads and stores share
  // one counter, and a load issued after stores, or a branch around them,
  // makes the compiler wait for every store.
  const BufferResource scale_res = MakeBuffer(a_scale, unsigned(n) * 4u);
  const BufferResource y_res = MakeBuffer(y, unsigned(n) * unsigned(ldy) * 4u);
  float s[TT][4];
  unsigned token_off[TT][4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int token = wtok0 + t * 16 + 4 * quad + i;
      s[t][i] = __uint_as_float(LoadB32(scale_res, unsigned(token) * 4u));
      token_off[t][i] = token < n ? unsigned(token) * unsigned(ldy) * 4u : kOutOfRange;
    }
  if constexpr (kSwiGLU) {
    // Each token's max |y| over the block's rows (LDS), stored once per
    // (row block, token) for the down projection's FP16 conversion.
    __shared__ unsigned s_max[Shape::kTokens];
    for (int i = tid; i < Shape::kTokens; i += Shape::kThreads)
      s_max[i] = 0;
    __syncthreads();
    // Tiles (2 j, 2 j + 1) are a (gate, up) pair for output rows j * 16 + n.
    unsigned row_off[RT / 2];
#pragma unroll
    for (int pr = 0; pr < RT / 2; ++pr) {
      const int row = (tile0 / 2 + pr) * kTileRows + sub;
      row_off[pr] = row < rows_out ? unsigned(row) * 4u : kOutOfRange;
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float m = 0.0f;
#pragma unroll
        for (int pr = 0; pr < RT / 2; ++pr) {
          const float g = acc[2 * pr][t][i] * s[t][i], u = acc[2 * pr + 1][t][i] * s[t][i];
          const float value = (g * (1.0f / (1.0f + expf(-g)))) * u;
          const bool inside = token_off[t][i] != kOutOfRange && row_off[pr] != kOutOfRange;
          const unsigned at = inside ? token_off[t][i] + row_off[pr] : kOutOfRange;
          if (publish)  // uniform
            StoreB32P<kCachePolicySc1>(y_res, at, __float_as_uint(value));
          else
            StoreF32(y_res, at, value);
          m = inside ? fmaxf(m, fabsf(value)) : m;
        }
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        if (sub == 0)
          atomicMax(&s_max[wt * TT * 16 + t * 16 + 4 * quad + i], __float_as_uint(m));
      }
    }
    __syncthreads();
    if (publish) {
      // The outputs and partial maxima through to memory, then the flag.
      const BufferResource m_res =
          MakeBuffer(row_max + std::size_t(rb) * n, unsigned(n) * 4u);
      for (int i = tid; i < Shape::kTokens; i += Shape::kThreads)
        StoreB32P<kCachePolicySc1>(m_res, tok0 + i < n ? unsigned(tok0 + i) * 4u : kOutOfRange,
                                   s_max[i]);
      __builtin_amdgcn_s_waitcnt(WaitVm(0));
      __syncthreads();
      if (tid == 0)
        __hip_atomic_store(tail.flags + tb * row_blocks + rb, tail.seq, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else if (row_max) {
      for (int i = tid; i < Shape::kTokens; i += Shape::kThreads)
        if (tok0 + i < n)
          row_max[std::size_t(rb) * n + tok0 + i] = s_max[i];
    }
  } else {
    unsigned row_off[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int row = (tile0 + r) * kTileRows + sub;
      row_off[r] = row < rows_out ? unsigned(row) * 4u : kOutOfRange;
    }
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < RT; ++r)
          StoreF32(y_res,
                   token_off[t][i] != kOutOfRange && row_off[r] != kOutOfRange
                       ? token_off[t][i] + row_off[r]
                       : kOutOfRange,
                   acc[r][t][i] * s[t][i]);
  }
}

// Code tiles -> FP16 tiles: the 16 codes lane L of a (tile, chunk) holds
// become block 0's eight halves at byte 16 L and block 1's at 1024 + 16 L
// of the 2 KB FP16 tile (the prompt GEMM's B operands, decoded once).
__global__ void HalfTilesKernel(const uint4* __restrict__ codes, uint4* __restrict__ out,
                                std::size_t units) {
  const std::size_t u = std::size_t(blockIdx.x) * 256 + threadIdx.x;  // (tile chunk, lane)
  if (u >= units)
    return;
  const uint4 q = codes[u];
  const std::size_t tc = u / 64;
  const unsigned lane = unsigned(u % 64);
  out[tc * 128 + lane] = __builtin_bit_cast(uint4, EightCodes(q.x, q.y));
  out[tc * 128 + 64 + lane] = __builtin_bit_cast(uint4, EightCodes(q.z, q.w));
}

// Adds K parts 1..parts-1 into part 0, in part order (the deterministic
// merge of split-K partial outputs, hip/ops.hip:2019-2119), for consumers
// that read one FP32 row.
__global__ void SumPartsKernel(float* __restrict__ y, std::size_t part_stride, int cols,
                               int ld, int parts) {
  const int row = blockIdx.y, col = blockIdx.x * blockDim.x + threadIdx.x;
  if (col >= cols)
    return;
  float* p = y + std::size_t(row) * ld + col;
  float sum = p[0];
  for (int k = 1; k < parts; ++k)
    sum += p[std::size_t(k) * part_stride];
  p[0] = sum;
}

// Blocks of one K part of a projection in the given shape.
template<class Shape>
int ShapeBlocks(int row_tiles, int tokens) {
  return (row_tiles + Shape::kTiles - 1) / Shape::kTiles *
         ((tokens + Shape::kTokens - 1) / Shape::kTokens);
}

// The block shape of a projection: wide when its blocks alone fill most of
// the 256 CUs, narrow (two blocks a CU) otherwise.
bool NarrowGemm(int row_tiles, int tokens) {
  return ShapeBlocks<WideShape>(row_tiles, tokens) < 192;
}

// K parts for a prompt GEMM: double while the blocks stay within 320
// (wide shape: one round on the 256 CUs with a quarter over) or 384
// (narrow shape) and each part keeps at least 4 chunks, at most 8 parts.
// Each part costs its consumer one more FP32 output pass; on the model's
// 512-token projections these limits give the fastest GEMM plus part
// reads (2048 x 2048: 4 parts; 6144 x 2048: 2; 2048 x 7680: 4).
int PromptParts(int row_tiles, int tokens, int nchunks) {
  const bool narrow = NarrowGemm(row_tiles, tokens);
  const int blocks = narrow ? ShapeBlocks<NarrowShape>(row_tiles, tokens)
                            : ShapeBlocks<WideShape>(row_tiles, tokens);
  const int limit = narrow ? 384 : 320;
  int parts = 1;
  while (parts < 8 && blocks * parts * 2 <= limit && nchunks / (parts * 2) >= 4)
    parts *= 2;
  return parts;
}

// The kernel addresses codes, scales, activations and each output part
// with 32-bit buffer offsets.
bool GemmOperandsFit(std::uint64_t row_tiles, std::uint64_t nchunks, std::uint64_t tokens,
                     std::uint64_t lda, std::uint64_t ldy, bool half) {
  return row_tiles * nchunks * kTileCodeBytes * (half ? 2 : 1) < (1ull << 31) &&
         tokens * lda * 2 < (1ull << 31) && tokens * ldy * 4 < (1ull << 31);
}

template<bool kSwiGLU, class Shape>
void LaunchGemm(const void* codes, const void* scales, int row_tiles, int nchunks,
                const std::uint16_t* a, std::uint32_t lda, const float* a_scale,
                std::uint32_t tokens, float* y, std::uint32_t ldy, std::uint32_t rows,
                int parts, std::size_t part_stride, unsigned* row_max, hipStream_t stream,
                HiddenHalves tail = HiddenHalves{}) {
  const int row_blocks = (row_tiles + Shape::kTiles - 1) / Shape::kTiles;
  const int token_blocks = (int(tokens) + Shape::kTokens - 1) / Shape::kTokens;
  const int gemm_blocks = row_blocks * token_blocks * parts;
  int blocks = gemm_blocks;
  if (tail.out) {
    tail.gemm_blocks = gemm_blocks;
    blocks += (int(tokens) + kHiddenRows - 1) / kHiddenRows;
  }
  Q8GemmKernel<kSwiGLU, Shape><<<blocks, Shape::kThreads, 0, stream>>>(
      static_cast<const std::uint8_t*>(codes), static_cast<const Half*>(scales), row_tiles,
      nchunks, reinterpret_cast<const Half*>(a), int(lda), a_scale, int(tokens), y, int(ldy),
      int(rows), row_blocks, token_blocks, parts, part_stride, row_max, tail);
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

int lfm3_half_rows(const float* x, std::uint32_t ldx, const unsigned* row_max,
                   std::uint32_t max_blocks, std::uint16_t* out, std::uint32_t lda,
                   float* scale, std::uint32_t rows, std::uint32_t cols, void* stream) {
  if (!x || !out || !scale || !rows || !cols || ldx < cols || lda < cols ||
      lda % 64 || (row_max && !max_blocks))
    return Fail(LFM3_E_INVALID, "invalid LFM3 fp16 row conversion");
  const bool vec = cols % 4 == 0 && ldx % 4 == 0 && cols <= 4 * kHalfThreads * kHalfVec &&
                   (reinterpret_cast<std::uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<std::uintptr_t>(out) & 7) == 0;
  const auto s = static_cast<hipStream_t>(stream);
  if (vec) {
    // Known maxima: a row's columns spread over blocks of 2048.
    const unsigned split =
        row_max ? (cols + 4 * kHalfThreads * kHalfVec / kHalfSplit - 1) /
                      (4 * kHalfThreads * kHalfVec / kHalfSplit)
                : 1;
    HalfRowsKernel<true><<<dim3(rows, split), kHalfThreads, 0, s>>>(
        x, int(ldx), row_max, int(max_blocks), out, int(lda), scale, int(cols));
  }
  else
    HalfRowsKernel<false><<<rows, kHalfThreads, 0, s>>>(x, int(ldx), row_max, int(max_blocks),
                                                        out, int(lda), scale, int(cols));
  return HipStatus(hipGetLastError(), "LFM3 fp16 row conversion launch");
}

std::uint32_t lfm3_q8_gemm_swiglu_max_blocks(std::uint32_t rows) {
  return (2 * RowTiles(rows) + WideShape::kTiles - 1) / WideShape::kTiles;
}

std::uint32_t lfm3_q8_gemm_parts(std::uint32_t rows, std::uint32_t cols,
                                 std::uint32_t tokens, int swiglu) {
  if (!rows || !cols || !tokens || swiglu)
    return 1;
  return std::uint32_t(PromptParts(int(RowTiles(rows)), int(tokens), int(Chunks(cols))));
}

std::size_t lfm3_q8_half_tiles_bytes(std::uint32_t rows, std::uint32_t cols) {
  return std::size_t(RowTiles(rows)) * Chunks(cols) * 2 * kTileCodeBytes;
}

int lfm3_q8_half_tiles(const void* codes, std::uint32_t rows, std::uint32_t cols, void* out,
                       void* stream) {
  if (!codes || !out || !rows || !cols || cols % 32 ||
      (reinterpret_cast<std::uintptr_t>(codes) & 15) ||
      (reinterpret_cast<std::uintptr_t>(out) & 15))
    return Fail(LFM3_E_INVALID, "invalid LFM3 FP16 tile conversion");
  const std::size_t units = std::size_t(RowTiles(rows)) * Chunks(cols) * 64;
  HalfTilesKernel<<<unsigned((units + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(codes), static_cast<uint4*>(out), units);
  return HipStatus(hipGetLastError(), "LFM3 FP16 tile conversion launch");
}

}  // extern "C"

namespace {

int Gemm(const void* tiles, bool half, const void* scales, std::uint32_t rows,
         std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda, const float* a_scale,
         std::uint32_t tokens, float* y, std::uint32_t ldy, std::uint32_t parts,
         void* stream) {
  if (!tiles || !scales || !a || !a_scale || !y || !rows || !cols ||
      cols % 32 || !tokens || lda % 64 || lda < Chunks(cols) * kChunk ||
      ldy < rows || !parts || parts > 8 || parts > Chunks(cols) ||
      (reinterpret_cast<std::uintptr_t>(a) & 15) ||
      !GemmOperandsFit(RowTiles(rows), Chunks(cols), tokens, lda, ldy, half))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 prompt GEMM shape");
  const bool narrow = NarrowGemm(int(RowTiles(rows)), int(tokens));
  const auto launch = half ? (narrow ? LaunchGemm<false, NarrowHalfShape>
                                     : LaunchGemm<false, WideHalfShape>)
                           : (narrow ? LaunchGemm<false, NarrowShape>
                                     : LaunchGemm<false, WideShape>);
  launch(tiles, scales, int(RowTiles(rows)), int(Chunks(cols)), a, lda, a_scale, tokens, y, ldy,
         rows, int(parts), std::size_t(ldy) * tokens, nullptr, static_cast<hipStream_t>(stream),
         HiddenHalves{});
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 prompt GEMM launch");
}

int GemmSwiGLU(const void* tiles, bool half, const void* scales, std::uint32_t rows,
               std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda,
               const float* a_scale, std::uint32_t tokens, float* y, std::uint32_t ldy,
               unsigned* row_max, void* stream, const HiddenHalves& tail = HiddenHalves{}) {
  if (!tiles || !scales || !a || !a_scale || !y || !rows || !cols ||
      cols % 32 || !tokens || lda % 64 || lda < Chunks(cols) * kChunk ||
      ldy < rows || (reinterpret_cast<std::uintptr_t>(a) & 15) ||
      !GemmOperandsFit(2 * RowTiles(rows), Chunks(cols), tokens, lda, ldy, half))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 prompt SwiGLU shape");
  const auto launch = half ? LaunchGemm<true, WideHalfShape> : LaunchGemm<true, WideShape>;
  launch(tiles, scales, int(2 * RowTiles(rows)), int(Chunks(cols)), a, lda, a_scale, tokens, y,
         ldy, rows, 1, 0, row_max, static_cast<hipStream_t>(stream), tail);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 prompt SwiGLU launch");
}

// Flags of a SwiGLU launch with trailing conversion blocks: one per GEMM block.
std::size_t SwiGLUFlags(std::uint32_t rows, std::uint32_t tokens) {
  const std::size_t row_blocks = (2 * RowTiles(rows) + WideHalfShape::kTiles - 1) /
                                 WideHalfShape::kTiles;
  const std::size_t token_blocks = (tokens + WideHalfShape::kTokens - 1) / WideHalfShape::kTokens;
  return row_blocks * token_blocks;
}

}  // namespace

extern "C" {

int lfm3_q8_gemm(const void* codes, const void* scales, std::uint32_t rows,
                 std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda,
                 const float* a_scale, std::uint32_t tokens, float* y,
                 std::uint32_t ldy, std::uint32_t parts, void* stream) {
  return Gemm(codes, false, scales, rows, cols, a, lda, a_scale, tokens, y, ldy, parts, stream);
}

std::size_t lfm3_q8_gemm_swiglu_flags_bytes(std::uint32_t rows, std::uint32_t tokens) {
  return rows && tokens ? SwiGLUFlags(rows, tokens) * sizeof(unsigned) : 0;
}

int lfm3_q8_gemm_swiglu_h16_rows(const void* halves, const void* scales, std::uint32_t rows,
                                 std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda,
                                 const float* a_scale, std::uint32_t tokens, float* y,
                                 std::uint32_t ldy, unsigned* row_max, std::uint16_t* out,
                                 std::uint32_t out_ld, float* out_scale, unsigned* flags,
                                 std::uint32_t seq, unsigned* error, void* stream) {
  if (!out || !out_scale || !row_max || !flags || !seq || rows % 4 || ldy % 4 ||
      out_ld % 64 || out_ld < rows || rows > std::uint32_t(kHiddenMaxCols) ||
      (reinterpret_cast<std::uintptr_t>(y) & 15) || (reinterpret_cast<std::uintptr_t>(out) & 7))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt SwiGLU with FP16 hidden rows");
  HiddenHalves tail;
  tail.out = reinterpret_cast<Half*>(out);
  tail.lda = int(out_ld);
  tail.scale = out_scale;
  tail.flags = flags;
  tail.seq = seq;
  tail.error = error;
  return GemmSwiGLU(halves, true, scales, rows, cols, a, lda, a_scale, tokens, y, ldy, row_max,
                    stream, tail);
}

int lfm3_q8_gemm_h16(const void* halves, const void* scales, std::uint32_t rows,
                     std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda,
                     const float* a_scale, std::uint32_t tokens, float* y,
                     std::uint32_t ldy, std::uint32_t parts, void* stream) {
  return Gemm(halves, true, scales, rows, cols, a, lda, a_scale, tokens, y, ldy, parts, stream);
}

int lfm3_sum_parts(float* y, std::size_t part_stride, std::uint32_t rows,
                   std::uint32_t cols, std::uint32_t ld, std::uint32_t parts, void* stream) {
  if (!y || !rows || !cols || ld < cols || !parts || parts > 8 ||
      (parts > 1 && part_stride < std::size_t(ld) * rows) || rows > 65535)
    return Fail(LFM3_E_INVALID, "invalid LFM3 part sum");
  if (parts == 1)
    return LFM3_OK;
  SumPartsKernel<<<dim3((cols + 255) / 256, rows), 256, 0, static_cast<hipStream_t>(stream)>>>(
      y, part_stride, int(cols), int(ld), int(parts));
  return HipStatus(hipGetLastError(), "LFM3 part sum launch");
}

int lfm3_q8_gemm_swiglu(const void* codes, const void* scales,
                        std::uint32_t rows, std::uint32_t cols,
                        const std::uint16_t* a, std::uint32_t lda,
                        const float* a_scale, std::uint32_t tokens, float* y,
                        std::uint32_t ldy, unsigned* row_max, void* stream) {
  return GemmSwiGLU(codes, false, scales, rows, cols, a, lda, a_scale, tokens, y, ldy, row_max,
                    stream);
}

int lfm3_q8_gemm_swiglu_h16(const void* halves, const void* scales,
                            std::uint32_t rows, std::uint32_t cols,
                            const std::uint16_t* a, std::uint32_t lda,
                            const float* a_scale, std::uint32_t tokens, float* y,
                            std::uint32_t ldy, unsigned* row_max, void* stream) {
  return GemmSwiGLU(halves, true, scales, rows, cols, a, lda, a_scale, tokens, y, ldy, row_max,
                    stream);
}

}  // extern "C"
