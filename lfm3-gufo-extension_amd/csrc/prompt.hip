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
// 538-560). A block of 4 waves owns 64 RT weight rows (16 RT per wave,
// held in registers and prefetched a chunk ahead) and 16 TT tokens, whose
// activations are double-buffered through LDS. Narrow outputs split K
// across blockIdx.z into parts written separately; their consumer adds the
// parts in part order, so no launch merges blocks through memory.
#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace lfm3amd {
namespace {

constexpr int kGemmThreads = 256, kGemmWaves = 4;
constexpr int kRowPad = 8;  // halves of padding per LDS activation row

__device__ __forceinline__ int RowExponent(float maximum) {
  return maximum > 0.0f ? 14 - ilogbf(maximum) : 0;
}

// One block per row: row maximum, then fp16(x 2^e) and the scale 2^-e.
__launch_bounds__(256) __global__
    void HalfRowsKernel(const float* __restrict__ x, int ldx,
                        const unsigned* __restrict__ row_max,
                        Half* __restrict__ out, int lda,
                        float* __restrict__ scale, int K) {
  __shared__ float s_max[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* src = x + std::size_t(row) * ldx;
  float maximum;
  if (row_max) {
    maximum = __uint_as_float(row_max[row]);
  } else {
    maximum = 0.0f;
    for (int k = tid; k < K; k += 256)
      maximum = fmaxf(maximum, fabsf(src[k]));
    maximum = WaveMax(maximum);
    if ((tid & 63) == 0)
      s_max[tid >> 6] = maximum;
    __syncthreads();
    maximum = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  }
  const int e = RowExponent(maximum);
  if (tid == 0)
    scale[row] = ldexpf(1.0f, -e);
  for (int k = tid; k < lda; k += 256)
    out[std::size_t(row) * lda + k] =
        k < K ? FloatToHalfBits(ldexpf(src[k], e)) : Half(0);
}

template<int RT, int TT, bool kSwiGLU>
__launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(1)))
__global__ void Q8GemmKernel(const std::uint8_t* __restrict__ codes,
                             const Half* __restrict__ scales, int row_tiles,
                             int nchunks, const Half* __restrict__ a, int lda,
                             const float* __restrict__ a_scale, int n,
                             float* __restrict__ y, int ldy, int rows_out,
                             std::size_t part_stride,
                             unsigned* __restrict__ row_max) {
  constexpr int TOK = 16 * TT;                 // tokens per block
  constexpr int ROW_HALVES = kChunk + kRowPad; // LDS row stride (halves)
  constexpr int UNITS = TOK * 8 / kGemmThreads; // 16-byte A pieces per thread
  __shared__ __attribute__((aligned(16))) Half s_a[2][TOK * ROW_HALVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile0 = (blockIdx.x * kGemmWaves + wave) * RT;
  const int tok0 = blockIdx.y * TOK;
  const int c_begin = int(blockIdx.z) * nchunks / int(gridDim.z);
  const int c_end = (int(blockIdx.z) + 1) * nchunks / int(gridDim.z);
  y += std::size_t(blockIdx.z) * part_stride;

  uint4 q[RT], qn[RT];
  unsigned sc[RT], scn[RT];
  const auto fetch_w = [&](int c, uint4 (&qq)[RT], unsigned (&ss)[RT]) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int tile = tile0 + r;
      if (tile < row_tiles) {
        const std::size_t off = std::size_t(tile) * nchunks + c;
        qq[r] = *reinterpret_cast<const uint4*>(codes + off * kTileCodeBytes + lane * 16);
        ss[r] = *reinterpret_cast<const unsigned*>(scales + off * kTileScales + (lane & 15) * 2);
      } else {
        qq[r] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
        ss[r] = 0;
      }
    }
  };
  uint4 ar[UNITS];
  const auto fetch_a = [&](int c) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int idx = tid + u * kGemmThreads, t = idx >> 3, seg = idx & 7;
      const int token = tok0 + t;
      ar[u] = token < n ? *reinterpret_cast<const uint4*>(a + std::size_t(token) * lda + c * kChunk + seg * 8)
                        : make_uint4(0, 0, 0, 0);
    }
  };
  const auto commit_a = [&](int stage) {
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int idx = tid + u * kGemmThreads, t = idx >> 3, seg = idx & 7;
      *reinterpret_cast<uint4*>(&s_a[stage][t * ROW_HALVES + seg * 8]) = ar[u];
    }
  };

  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 acc[RT][TT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < TT; ++t)
      acc[r][t] = zero;

  fetch_w(c_begin, q, sc);
  fetch_a(c_begin);
  commit_a(0);
  __syncthreads();
  for (int c = c_begin; c < c_end; ++c) {
    const int stage = (c - c_begin) & 1;
    const bool more = c + 1 < c_end;
    if (more) {
      fetch_w(c + 1, qn, scn);
      fetch_a(c + 1);
    }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      h8 w[RT];
      float d[RT];
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        w[r] = blk ? EightCodes(q[r].z, q[r].w) : EightCodes(q[r].x, q[r].y);
        d[r] = HalfBitsToFloat(blk ? sc[r] >> 16 : sc[r] & 0xffffu);
      }
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        // A operand: lane L holds token 16 t + L % 16, elements 8 (L / 16)..
        const h8 av = *reinterpret_cast<const h8*>(
            &s_a[stage][(t * 16 + (lane & 15)) * ROW_HALVES + blk * 32 + 8 * (lane >> 4)]);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const f4 p = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, w[r], zero, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[r][t][i] = fmaf(d[r], p[i], acc[r][t][i]);
        }
      }
    }
    if (more) {
      commit_a(stage ^ 1);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        q[r] = qn[r];
        sc[r] = scn[r];
      }
    }
    __syncthreads();
  }

  // D layout: lane L holds tokens 16 t + 4 (L / 16) + i of weight row L % 16.
  const int sub = lane & 15, quad = lane >> 4;
  if constexpr (kSwiGLU) {
    // Tiles (2 j, 2 j + 1) are a (gate, up) pair for output rows j * 16 + n.
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int token = tok0 + t * 16 + 4 * quad + i;
        const float s = token < n ? a_scale[token] : 0.0f;
        float m = 0.0f;
#pragma unroll
        for (int pr = 0; pr < RT / 2; ++pr) {
          const int row = (tile0 / 2 + pr) * kTileRows + sub;
          const float g = acc[2 * pr][t][i] * s, u = acc[2 * pr + 1][t][i] * s;
          const float value = (g * (1.0f / (1.0f + expf(-g)))) * u;
          if (token < n && row < rows_out) {
            y[std::size_t(token) * ldy + row] = value;
            m = fmaxf(m, fabsf(value));
          }
        }
        // Row maxima for the down projection's fp16 conversion.
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        if (row_max && sub == 0 && token < n)
          atomicMax(row_max + token, __float_as_uint(m));
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int token = tok0 + t * 16 + 4 * quad + i;
        if (token >= n)
          continue;
        const float s = a_scale[token];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const int row = (tile0 + r) * kTileRows + sub;
          if (row < rows_out)
            y[std::size_t(token) * ldy + row] = acc[r][t][i] * s;
        }
      }
    }
  }
}

// K parts for a prompt GEMM: enough blocks for the 256 CUs (two resident
// each), keeping at least 4 chunks a part, at most 8 parts.
int PromptParts(int row_blocks, int token_blocks, int nchunks) {
  int parts = 1;
  while (parts < 8 && row_blocks * token_blocks * parts < 256 &&
         nchunks / (parts * 2) >= 4)
    parts *= 2;
  return parts;
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

int lfm3_half_rows(const float* x, std::uint32_t ldx, const unsigned* row_max,
                   std::uint16_t* out, std::uint32_t lda, float* scale,
                   std::uint32_t rows, std::uint32_t cols, void* stream) {
  if (!x || !out || !scale || !rows || !cols || ldx < cols || lda < cols ||
      lda % 64)
    return Fail(LFM3_E_INVALID, "invalid LFM3 fp16 row conversion");
  HalfRowsKernel<<<rows, 256, 0, static_cast<hipStream_t>(stream)>>>(
      x, int(ldx), row_max, out, int(lda), scale, int(cols));
  return HipStatus(hipGetLastError(), "LFM3 fp16 row conversion launch");
}

std::uint32_t lfm3_q8_gemm_parts(std::uint32_t rows, std::uint32_t cols,
                                 std::uint32_t tokens, int swiglu) {
  if (!rows || !cols || !tokens || swiglu)
    return 1;
  const int row_blocks = (int(RowTiles(rows)) + 15) / 16;
  const int token_blocks = (int(tokens) + 127) / 128;
  return std::uint32_t(PromptParts(row_blocks, token_blocks, int(Chunks(cols))));
}

int lfm3_q8_gemm(const void* codes, const void* scales, std::uint32_t rows,
                 std::uint32_t cols, const std::uint16_t* a, std::uint32_t lda,
                 const float* a_scale, std::uint32_t tokens, float* y,
                 std::uint32_t ldy, std::uint32_t parts, void* stream) {
  if (!codes || !scales || !a || !a_scale || !y || !rows || !cols ||
      cols % 32 || !tokens || lda % 64 || lda < Chunks(cols) * kChunk ||
      ldy < rows || !parts || parts > 8 || parts > Chunks(cols) ||
      (reinterpret_cast<std::uintptr_t>(a) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 prompt GEMM shape");
  const int row_tiles = int(RowTiles(rows)), nchunks = int(Chunks(cols));
  const dim3 grid((row_tiles + 15) / 16, (tokens + 127) / 128, parts);
  Q8GemmKernel<4, 8, false><<<grid, kGemmThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const std::uint8_t*>(codes), static_cast<const Half*>(scales),
      row_tiles, nchunks, reinterpret_cast<const Half*>(a), int(lda), a_scale,
      int(tokens), y, int(ldy), int(rows), std::size_t(ldy) * tokens, nullptr);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 prompt GEMM launch");
}

int lfm3_q8_gemm_swiglu(const void* codes, const void* scales,
                        std::uint32_t rows, std::uint32_t cols,
                        const std::uint16_t* a, std::uint32_t lda,
                        const float* a_scale, std::uint32_t tokens, float* y,
                        std::uint32_t ldy, unsigned* row_max, void* stream) {
  if (!codes || !scales || !a || !a_scale || !y || !rows || !cols ||
      cols % 32 || !tokens || lda % 64 || lda < Chunks(cols) * kChunk ||
      ldy < rows || (reinterpret_cast<std::uintptr_t>(a) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 Q8_0 prompt SwiGLU shape");
  const int row_tiles = 2 * int(RowTiles(rows)), nchunks = int(Chunks(cols));
  const dim3 grid((row_tiles + 15) / 16, (tokens + 127) / 128, 1);
  Q8GemmKernel<4, 8, true><<<grid, kGemmThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const std::uint8_t*>(codes), static_cast<const Half*>(scales),
      row_tiles, nchunks, reinterpret_cast<const Half*>(a), int(lda), a_scale,
      int(tokens), y, int(ldy), int(rows), 0, row_max);
  return HipStatus(hipGetLastError(), "LFM3 Q8_0 prompt SwiGLU launch");
}

}  // extern "C"
