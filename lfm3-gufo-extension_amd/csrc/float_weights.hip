// Float weights (BF16, F16, F32) with exact products on gfx950: the
// numerical reference precision of the model (BF16, README.md:24-27) and
// the other float formats the reference binds (weights.cpp:30-37): the
// projections of gpu::Dense / gpu::LaunchGEMV for such tensors
// (hip/ops.hip:876-890 F16Dense, 1799-1825, 1917-2005, 2243-2244) and the
// embedding gather (hip/ops.hip:858-875).
//
// Weights are repacked at load into tiles of 16 rows x 32 columns: lane
// L = 16 g + n of a wave holds row n's columns 8g..8g+7 (16 bytes for the
// 16-bit formats, 1 KB a tile; two 16-byte planes for F32, columns
// 8g..8g+3 in the first 1 KB and 8g+4..8g+7 in the second). Tiles are
// stored [row tile][column block], rows padded to 16 and columns to 32
// with zeros.
//
// Every product runs on v_mfma_f32_16x16x32_bf16 with exact BF16 x BF16
// products. The FP32 inputs split exactly into three BF16 parts,
// x = hi + mid + lo (hi = x truncated to BF16, mid = (x - hi) truncated,
// lo = the rest, which has at most 8 significant bits). A BF16 weight is
// one part; an F16 weight (11 significant bits) is hi + lo with lo of at
// most 3 bits; an F32 weight splits like the inputs. So the 3 x (1, 2 or
// 3) MFMAs per 32-column block give the exact products of the weights
// with the FP32 inputs; only the FP32 accumulation order differs from a
// scalar loop. A block owns up to 16 tokens (A rows), RT row tiles and,
// per wave, a contiguous range of column blocks; the waves' sums meet in
// LDS and add in wave order.
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "internal.hpp"

namespace lfm3amd {
namespace {

constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kTileCols = 32, kTileElems = 16 * kTileCols;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

std::uint32_t ColBlocks(std::uint32_t cols) { return (cols + kTileCols - 1) / kTileCols; }
std::uint32_t RowTilesOf(std::uint32_t rows) { return (rows + 15) / 16; }

// x = hi + mid + lo exactly; returns the three BF16 bit patterns.
__device__ __forceinline__ void Split3(float x, unsigned& hi, unsigned& mid, unsigned& lo) {
  const unsigned b = __float_as_uint(x);
  const float r = x - __uint_as_float(b & 0xffff0000u);
  const unsigned rb = __float_as_uint(r);
  const float l = r - __uint_as_float(rb & 0xffff0000u);
  hi = b >> 16;
  mid = rb >> 16;
  lo = __float_as_uint(l) >> 16;
}

__device__ __forceinline__ f32x4 Mfma(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The A operands of one lane: 8 consecutive inputs of its token, split.
__device__ __forceinline__ void Operands(float4 p, float4 q, uint4& hi, uint4& mid, uint4& lo) {
  const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
  unsigned h[8], m[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    Split3(v[i], h[i], m[i], l[i]);
  hi = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
  mid = make_uint4(m[0] | m[1] << 16, m[2] | m[3] << 16, m[4] | m[5] << 16, m[6] | m[7] << 16);
  lo = make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
}

// Weight formats (GGML type ids) and their tile geometry.
constexpr int kF32 = LFM3_TYPE_F32, kF16 = LFM3_TYPE_F16, kBf16 = LFM3_TYPE_BF16;
constexpr int WordsOf(int wf) { return wf == kF32 ? 2 : 1; }       // 16-byte words a lane
constexpr int PartsOf(int wf) { return wf == kBf16 ? 1 : wf == kF16 ? 2 : 3; }  // BF16 parts
constexpr int ElemBytes(int wf) { return wf == kF32 ? 4 : 2; }

// Eight weights of a lane (its tile words) -> their exact BF16 parts.
template<int WF>
__device__ __forceinline__ void WeightParts(const uint4 (&w)[WordsOf(WF)],
                                            uint4 (&part)[PartsOf(WF)]) {
  if constexpr (WF == kBf16) {
    part[0] = w[0];
  } else if constexpr (WF == kF16) {
    // v = f16 exactly in FP32; hi keeps its top 8 significant bits, and
    // lo = v - hi (at most 3 significant bits) is exact in BF16.
    const unsigned in[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
    unsigned hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v0 = HalfBitsToFloat(in[i] & 0xffffu), v1 = HalfBitsToFloat(in[i] >> 16);
      const unsigned b0 = __float_as_uint(v0) & 0xffff0000u, b1 = __float_as_uint(v1) & 0xffff0000u;
      const unsigned l0 = __float_as_uint(v0 - __uint_as_float(b0)) >> 16;
      const unsigned l1 = __float_as_uint(v1 - __uint_as_float(b1)) >> 16;
      hi[i] = (b0 >> 16) | b1;
      lo[i] = l0 | (l1 << 16);
    }
    part[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    part[1] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  } else {
    const float4 p = __builtin_bit_cast(float4, w[0]), q = __builtin_bit_cast(float4, w[1]);
    Operands(p, q, part[0], part[1], part[2]);
  }
}

// y[p][t][r] for tokens t of blockIdx.y's group of 16, row tiles
// [blockIdx.x * RT, + RT) and K part p = blockIdx.z (column blocks
// [p * nkb / parts, (p + 1) * nkb / parts)). With kSwiGLU the row tiles
// come in gate/up pairs (tile 2j gate, 2j + 1 up of output tile j) and
// y = silu(gate) * up, as the reference's SwiGLU (g / (1 + exp(-g))) * u.
template<int RT, bool kSwiGLU, int WF>
__launch_bounds__(kThreads) __global__
    void FloatGemvKernel(const uint4* __restrict__ tiles, int row_tiles, int nkb,
                        const float* __restrict__ x, int ldx, int batch, float* __restrict__ y,
                        int ldy, int out_rows, int parts, std::size_t part_stride) {
  __shared__ f32x4 s_red[kWaves][RT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, m = lane & 15;
  const int tile0 = blockIdx.x * RT;
  const int token = blockIdx.y * 16 + m;
  const bool live = token < batch;
  const int part = blockIdx.z;
  const int p0 = part * nkb / parts, p1 = (part + 1) * nkb / parts;
  const int kb0 = p0 + wave * (p1 - p0) / kWaves, kb1 = p0 + (wave + 1) * (p1 - p0) / kWaves;
  const float* xr = x + std::size_t(live ? token : 0) * ldx + 8 * g;
  constexpr int NW = WordsOf(WF), NP = PartsOf(WF);
  // Tiles past the last one read the last one (unconditional 16-byte
  // loads); their rows are past out_rows, so their sums are never stored.
  const uint4* wt[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    wt[r] = tiles + (std::size_t(min(tile0 + r, row_tiles - 1)) * nkb) * 64 * NW + lane;

  f32x4 acc[3][RT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
    acc[0][r] = acc[1][r] = acc[2][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float4 zerof = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  // One block ahead: the next weights and inputs load while this block's
  // MFMAs run.
  uint4 wn[RT][NW];
  const auto load_w = [&](int kb, uint4 (&dst)[RT][NW]) {
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
        dst[r][q] = wt[r][std::size_t(kb) * 64 * NW + 64 * q];
  };
  float4 xa = zerof, xb = zerof;
  if (kb0 < kb1) {
    load_w(kb0, wn);
    if (live) {
      xa = *reinterpret_cast<const float4*>(xr + kb0 * kTileCols);
      xb = *reinterpret_cast<const float4*>(xr + kb0 * kTileCols + 4);
    }
  }
  for (int kb = kb0; kb < kb1; ++kb) {
    uint4 wc[RT][NW];
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int q = 0; q < NW; ++q)
        wc[r][q] = wn[r][q];
    const float4 ca = xa, cb = xb;
    if (kb + 1 < kb1) {
      load_w(kb + 1, wn);
      if (live) {
        xa = *reinterpret_cast<const float4*>(xr + (kb + 1) * kTileCols);
        xb = *reinterpret_cast<const float4*>(xr + (kb + 1) * kTileCols + 4);
      }
    }
    uint4 hi, mid, lo;
    Operands(ca, cb, hi, mid, lo);
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      uint4 wp[NP];
      WeightParts<WF>(wc[r], wp);
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        acc[0][r] = Mfma(hi, wp[j], acc[0][r]);
        acc[1][r] = Mfma(mid, wp[j], acc[1][r]);
        acc[2][r] = Mfma(lo, wp[j], acc[2][r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RT; ++r)
    s_red[wave][r][lane] = (acc[0][r] + acc[1][r]) + acc[2][r];
  __syncthreads();

  // Lane l of a tile holds tokens 4 (l >> 4) + i, weight row l & 15.
  float* yp = y + std::size_t(part) * part_stride;
  constexpr int kOut = kSwiGLU ? RT / 2 : RT;
  for (int e = threadIdx.x; e < kOut * 64; e += kThreads) {
    const int r = e >> 6, l = e & 63;
    const int t0 = blockIdx.y * 16 + 4 * (l >> 4);
    if (kSwiGLU) {
      f32x4 gs = s_red[0][2 * r][l], us = s_red[0][2 * r + 1][l];
      for (int v = 1; v < kWaves; ++v) {
        gs += s_red[v][2 * r][l];
        us += s_red[v][2 * r + 1][l];
      }
      const int row = ((tile0 >> 1) + r) * 16 + (l & 15);
      if (row >= out_rows)
        continue;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (t0 + i < batch)
          yp[std::size_t(t0 + i) * ldy + row] = (gs[i] / (1.0f + expf(-gs[i]))) * us[i];
    } else {
      f32x4 s = s_red[0][r][l];
      for (int v = 1; v < kWaves; ++v)
        s += s_red[v][r][l];
      const int row = (tile0 + r) * 16 + (l & 15);
      if (row >= out_rows)
        continue;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (t0 + i < batch)
          yp[std::size_t(t0 + i) * ldy + row] = s[i];
    }
  }
}

// Element (n, k) of a tile (row n < 16, column k < 32), in elements from
// the tile's start.
__host__ __device__ inline std::size_t TileIndex(int wf, int n, int k) {
  return wf == kF32 ? std::size_t(((k & 7) >> 2) * 256 + (16 * (k >> 3) + n) * 4 + (k & 3))
                    : std::size_t((16 * (k >> 3) + n) * 8 + (k & 7));
}

// Row gather from the tiles: out[i] = row tokens[i] (or, with a row table,
// inputs[i] when not null), as FP32 (hip/ops.hip:858-875 Value for F32,
// F16 and BF16). Ids at or past the vocabulary give zero rows (the host
// refuses them before a launch).
template<int WF>
__global__ void FloatEmbedKernel(const void* __restrict__ tiles, int nkb, int cols,
                                 std::uint32_t vocab, const std::uint32_t* __restrict__ tokens,
                                 const float* const* inputs, float* __restrict__ out) {
  const int i = blockIdx.y;
  const float* row_in = inputs ? inputs[i] : nullptr;
  const std::uint32_t t = row_in ? 0u : tokens[i];
  const std::size_t base = (std::size_t(t >> 4) * nkb) * kTileElems;
  const int n = int(t & 15u);
  for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x) {
    float v;
    if (row_in) {
      v = row_in[c];
    } else if (t >= vocab) {
      v = 0.0f;
    } else {
      const std::size_t at = base + std::size_t(c / kTileCols) * kTileElems +
                             TileIndex(WF, n, c % kTileCols);
      if constexpr (WF == kF32)
        v = static_cast<const float*>(tiles)[at];
      else if constexpr (WF == kF16)
        v = HalfBitsToFloat(static_cast<const std::uint16_t*>(tiles)[at]);
      else
        v = __uint_as_float(unsigned(static_cast<const std::uint16_t*>(tiles)[at]) << 16);
    }
    out[std::size_t(i) * cols + c] = v;
  }
}

template<int RT, bool kSwiGLU, int WF>
void Launch(const void* tiles, std::uint32_t row_tiles, std::uint32_t nkb, const float* x,
            std::uint32_t ldx, std::uint32_t batch, float* y, std::uint32_t ldy,
            std::uint32_t out_rows, std::uint32_t parts, hipStream_t stream) {
  const dim3 grid((row_tiles + RT - 1) / RT, (batch + 15) / 16, parts);
  FloatGemvKernel<RT, kSwiGLU, WF><<<grid, kThreads, 0, stream>>>(
      static_cast<const uint4*>(tiles), int(row_tiles), int(nkb), x, int(ldx), int(batch), y,
      int(ldy), int(out_rows), int(parts), std::size_t(batch) * ldy);
}

template<int WF>
void LaunchFormat(const void* tiles, std::uint32_t row_tiles, std::uint32_t nkb, const float* x,
                  std::uint32_t ldx, std::uint32_t batch, float* y, std::uint32_t ldy,
                  std::uint32_t out_rows, std::uint32_t parts, bool swiglu, hipStream_t s) {
  if (swiglu) {
    if (row_tiles >= 1024)
      Launch<4, true, WF>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, 1, s);
    else
      Launch<2, true, WF>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, 1, s);
  } else if (row_tiles >= 1024) {
    Launch<4, false, WF>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, s);
  } else if (row_tiles >= 512) {
    Launch<2, false, WF>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, s);
  } else {
    Launch<1, false, WF>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, s);
  }
}

bool FloatFormat(std::uint32_t type) {
  return type == LFM3_TYPE_BF16 || type == LFM3_TYPE_F16 || type == LFM3_TYPE_F32;
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

size_t lfm3_float_tiled_bytes(uint32_t type, uint32_t rows, uint32_t cols) {
  if (!FloatFormat(type))
    return 0;
  return std::size_t(RowTilesOf(rows)) * ColBlocks(cols) * kTileElems * ElemBytes(int(type));
}

int lfm3_float_pack_host(uint32_t type, const void* src, uint32_t rows, uint32_t cols,
                         void* tiles, uint32_t tile_offset, uint32_t tile_stride) {
  if (!FloatFormat(type) || !src || !tiles || !rows || !cols || !tile_stride)
    return Fail(LFM3_E_INVALID, "invalid LFM3 float-weight pack");
  const std::size_t eb = ElemBytes(int(type));
  const auto* in = static_cast<const std::uint8_t*>(src);
  auto* out = static_cast<std::uint8_t*>(tiles);
  const std::uint32_t nkb = ColBlocks(cols);
  for (std::uint32_t r = 0; r < rows; ++r) {
    const std::size_t tile = std::size_t(tile_offset) + std::size_t(r / 16) * tile_stride;
    const int n = int(r % 16);
    for (std::uint32_t c = 0; c < cols; ++c) {
      const std::size_t at = (tile * nkb + c / kTileCols) * kTileElems +
                             TileIndex(int(type), n, int(c % kTileCols));
      std::memcpy(out + at * eb, in + (std::size_t(r) * cols + c) * eb, eb);
    }
  }
  return LFM3_OK;
}

uint32_t lfm3_bf16_gemv_parts(uint32_t rows, uint32_t cols, uint32_t batch) {
  // Narrow outputs split K so that the grid reaches about 256 blocks; each
  // part keeps at least 16 column blocks (two a wave).
  const std::uint32_t tiles = RowTilesOf(rows), groups = (batch + 15) / 16;
  const std::uint32_t rt = tiles >= 1024 ? 4 : tiles >= 512 ? 2 : 1;
  std::uint32_t blocks = (tiles + rt - 1) / rt * std::max(groups, 1u), parts = 1;
  while (parts < 8 && blocks * parts * 2 <= 256 && ColBlocks(cols) / (parts * 2) >= 16)
    parts *= 2;
  return parts;
}

int lfm3_float_gemv(uint32_t type, const void* tiles, uint32_t rows, uint32_t cols,
                    const float* x, uint32_t ldx, float* y, uint32_t ldy, uint32_t batch,
                    uint32_t parts, int swiglu, void* stream) {
  const std::uint32_t out_rows = rows;
  const std::uint32_t row_tiles = RowTilesOf(rows) * (swiglu ? 2 : 1);
  if (!FloatFormat(type) || !tiles || !x || !y || !rows || !cols || cols % kTileCols ||
      ldx < cols || ldx % 4 || ldy < out_rows || !batch || !parts || parts > 8 ||
      parts > ColBlocks(cols) || (swiglu && parts != 1) ||
      (reinterpret_cast<std::uintptr_t>(x) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 float-weight GEMV shape");
  const auto s = static_cast<hipStream_t>(stream);
  const std::uint32_t nkb = ColBlocks(cols);
  if (type == LFM3_TYPE_BF16)
    LaunchFormat<kBf16>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, swiglu, s);
  else if (type == LFM3_TYPE_F16)
    LaunchFormat<kF16>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, swiglu, s);
  else
    LaunchFormat<kF32>(tiles, row_tiles, nkb, x, ldx, batch, y, ldy, out_rows, parts, swiglu, s);
  return HipStatus(hipGetLastError(), "LFM3 float-weight GEMV launch");
}

int lfm3_float_embed(uint32_t type, const void* tiles, uint32_t vocab, uint32_t cols,
                     const uint32_t* tokens, const float* const* inputs, uint32_t n, float* out,
                     void* stream) {
  if (!FloatFormat(type) || !tiles || !tokens || !out || !vocab || !cols || cols % kTileCols ||
      !n)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 float-weight embedding");
  const dim3 grid((cols + 255) / 256, n);
  const auto s = static_cast<hipStream_t>(stream);
  const int nkb = int(ColBlocks(cols));
  if (type == LFM3_TYPE_BF16)
    FloatEmbedKernel<kBf16><<<grid, 256, 0, s>>>(tiles, nkb, int(cols), vocab, tokens, inputs, out);
  else if (type == LFM3_TYPE_F16)
    FloatEmbedKernel<kF16><<<grid, 256, 0, s>>>(tiles, nkb, int(cols), vocab, tokens, inputs, out);
  else
    FloatEmbedKernel<kF32><<<grid, 256, 0, s>>>(tiles, nkb, int(cols), vocab, tokens, inputs, out);
  return HipStatus(hipGetLastError(), "LFM3 float-weight embedding launch");
}

// The BF16 forms (the reference precision) of the entry points above.
size_t lfm3_bf16_tiled_bytes(uint32_t rows, uint32_t cols) {
  return lfm3_float_tiled_bytes(LFM3_TYPE_BF16, rows, cols);
}

int lfm3_bf16_pack_host(const void* src, uint32_t rows, uint32_t cols, void* tiles,
                        uint32_t tile_offset, uint32_t tile_stride) {
  return lfm3_float_pack_host(LFM3_TYPE_BF16, src, rows, cols, tiles, tile_offset, tile_stride);
}

int lfm3_bf16_gemv(const void* tiles, uint32_t rows, uint32_t cols, const float* x,
                   uint32_t ldx, float* y, uint32_t ldy, uint32_t batch, uint32_t parts,
                   int swiglu, void* stream) {
  return lfm3_float_gemv(LFM3_TYPE_BF16, tiles, rows, cols, x, ldx, y, ldy, batch, parts, swiglu,
                         stream);
}

int lfm3_bf16_embed(const void* tiles, uint32_t vocab, uint32_t cols, const uint32_t* tokens,
                    const float* const* inputs, uint32_t n, float* out, void* stream) {
  return lfm3_float_embed(LFM3_TYPE_BF16, tiles, vocab, cols, tokens, inputs, n, out, stream);
}

}  // extern "C"
