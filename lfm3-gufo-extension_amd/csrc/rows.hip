// Row operations of the decode round on gfx950: residual + RMSNorm, the
// ragged gated short-convolution step, the ragged Q/K heads (per-head
// RMSNorm, paired RoPE, F16 K/V ring store) and greedy argmax.
#include <cmath>
#include <string>

#include <algorithm>

#include "common.hpp"
#include "internal.hpp"
#include "norm_image.hpp"

namespace lfm3amd {

namespace {
thread_local std::string g_error;
}
void SetError(const std::string& message) { g_error = message; }
int Fail(int status, const std::string& message) {
  g_error = message;
  return status;
}
int HipStatus(hipError_t e, const char* what) {
  if (e == hipSuccess)
    return LFM3_OK;
  g_error = std::string(what) + ": " + hipGetErrorString(e);
  return LFM3_E_HIP;
}

namespace {

constexpr int kNormThreads = 1024, kNormItems = 4;

// Block sum of one value per thread: wave butterflies then the wave sums
// in wave order.
__device__ float BlockSum(float v, float* scratch) {
  v = WaveSum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    scratch[wave] = v;
  __syncthreads();
  float total = 0.0f;
  for (int w = 0; w < kNormThreads / 64; ++w)
    total += scratch[w];
  return total;
}

// Writes one token's row (H floats in LDS) into a GEMV operand image (see
// lfm3_q8_gemv_image): exponent e puts the row maximum in [2^14, 2^15),
// and SplitPair gives hi and lo, as the FP32 GEMV stages them; columns past
// H (the tail of the last 64-column chunk) are written as zeros.
__device__ void WriteOperandRow(const float* __restrict__ s_row, int H, int t,
                                float maximum, uint4* __restrict__ image,
                                int* __restrict__ exps) {
  const int e = maximum > 0.0f ? 14 - ilogbf(maximum) : 0;
  if (threadIdx.x == 0)
    exps[t] = e;
  const int groups = (H + kChunk - 1) / kChunk * 8;
  for (int cg = threadIdx.x; cg < groups; cg += blockDim.x) {
    unsigned hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const int k = cg * 8 + i;
      SplitPair(k < H ? s_row[k] : 0.0f, k + 1 < H ? s_row[k + 1] : 0.0f, e, hi[i / 2],
                lo[i / 2]);
    }
    const int idx = ((cg >> 3) * 2 + ((cg >> 2) & 1)) * 64 + 16 * (cg & 3) + t;
    image[idx] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    image[idx + 8] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  }
}

__device__ float BlockMax(float v, float* scratch) {
  v = WaveMax(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    scratch[wave] = v;
  __syncthreads();
  float m = 0.0f;
  for (int w = 0; w < int(blockDim.x >> 6); ++w)
    m = fmaxf(m, scratch[w]);
  return m;
}

// reference.cpp:20-28 / hip/ops.hip:905-970 semantics: x += post(branch),
// then z = x / sqrt(mean(x^2) + eps) * w, each product rounded as the
// reference's x * scale * weight. The branch may arrive as `parts` K-part
// partial sums of a GEMV (lfm3_q8_gemv_partials), part_stride floats
// apart, added in part order. Every load, of every part, is issued before
// the first reduction, so the row costs one memory round trip.
// With an operand image, the normed row also goes out as the next GEMV's
// MFMA A operand (z may then be null).
__launch_bounds__(kNormThreads) __global__
    void ResidualNormKernel(const float* __restrict__ branch, int parts,
                            std::size_t part_stride,
                            const float* __restrict__ post,
                            float* __restrict__ x,
                            const float* __restrict__ weight,
                            float* __restrict__ z, int H, float eps,
                            uint4* __restrict__ image, int* __restrict__ exps,
                            Half* __restrict__ a16, int lda, float* __restrict__ a_scale) {
  __shared__ float scratch[kNormThreads / 64];
  __shared__ float s_row[kNormThreads * kNormItems];
  const int row = blockIdx.x, tid = threadIdx.x;
  float* xr = x + std::size_t(row) * H;
  float v[kNormItems], b[kNormParts][kNormItems], pw[kNormItems], nw[kNormItems];
#pragma unroll
  for (int i = 0; i < kNormItems; ++i) {
    const int k = tid + kNormThreads * i;
    const bool live = k < H;
    v[i] = live ? xr[k] : 0.0f;
    pw[i] = live && post ? post[k] : 0.0f;
    nw[i] = live && weight ? weight[k] : 0.0f;
#pragma unroll
    for (int p = 0; p < kNormParts; ++p)
      b[p][i] = live && branch && p < parts
                    ? branch[p * part_stride + std::size_t(row) * H + k]
                    : 0.0f;
  }
  if (branch) {
    float squares = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormItems; ++i) {
#pragma unroll
      for (int p = 1; p < kNormParts; ++p)
        b[0][i] += b[p][i];
      squares = fmaf(b[0][i], b[0][i], squares);
    }
    if (post) {
      const float scale = 1.0f / sqrtf(BlockSum(squares, scratch) / float(H) + eps);
#pragma unroll
      for (int i = 0; i < kNormItems; ++i)
        b[0][i] = (b[0][i] * scale) * pw[i];
    }
#pragma unroll
    for (int i = 0; i < kNormItems; ++i) {
      const int k = tid + kNormThreads * i;
      v[i] = v[i] + b[0][i];
      if (k < H)
        xr[k] = v[i];
    }
  }
  if (!weight)
    return;
  float squares = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormItems; ++i)
    squares = fmaf(v[i], v[i], squares);
  const float scale = 1.0f / sqrtf(BlockSum(squares, scratch) / float(H) + eps);
  float maximum = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormItems; ++i) {
    const int k = tid + kNormThreads * i;
    const float zv = (v[i] * scale) * nw[i];
    if (k < H) {
      if (z)
        z[std::size_t(row) * H + k] = zv;
      s_row[k] = zv;
      maximum = fmaxf(maximum, fabsf(zv));
    }
  }
  if (!image && !a16)
    return;
  maximum = BlockMax(maximum, scratch);  // its barriers publish s_row
  if (image)
    WriteOperandRow(s_row, H, row, maximum, image, exps);
  if (a16) {
    // The prompt GEMM's FP16 row (HalfRowsKernel's expressions), zero tail.
    const int e = RowExponent(maximum);
    if (tid == 0)
      a_scale[row] = ldexpf(1.0f, -e);
    // The zero tail of the last 64-column chunk; later columns are not read.
    for (int k = tid; k < (H + kChunk - 1) / kChunk * kChunk; k += kNormThreads)
      a16[std::size_t(row) * lda + k] = k < H ? ScaledHalf(s_row[k], e) : Half(0);
  }
}

// The decode round's norm as a launch of its own: one 256-thread block a
// row (NormImageRow, norm_image.hpp).
constexpr int kImageNormThreads = 256;
template<int G>
__launch_bounds__(kImageNormThreads) __global__ void NormImageKernel(const NormImageArgs a) {
  NormImageRow<kImageNormThreads, G, false>(a, blockIdx.x);
}

// reference.cpp:85-101: one owner per (row, channel); the window sum keeps
// the reference's order and separate roundings, so outputs and history are
// bit-identical to it for the same projection rows.
__global__ void ConvStepKernel(const float* __restrict__ p, int ldp,
                               const float* __restrict__ taps,
                               float* const* __restrict__ history,
                               float* __restrict__ y, int ldy, int H, int L) {
#pragma clang fp contract(off)
  const int ch = blockIdx.x * blockDim.x + threadIdx.x, row = blockIdx.y;
  if (ch >= H)
    return;
  const float* pr = p + std::size_t(row) * ldp;
  float* own = history[row] + std::size_t(ch) * (L - 1);
  const float bx = pr[ch] * pr[2 * H + ch];
  const float* w = taps + std::size_t(ch) * L;
  float sum = 0.0f;
  for (int t = 0; t < L - 1; ++t)
    sum += w[t] * own[t];
  sum += w[L - 1] * bx;
  for (int t = 1; t < L - 1; ++t)
    own[t - 1] = own[t];
  own[L - 2] = bx;
  y[std::size_t(row) * ldy + ch] = sum * pr[H + ch];
}

// ConvStepKernel with one block per row, writing the output row as the
// out projection's operand image (y, when given, also gets the FP32 row).
// Same expressions and order, so outputs and history stay bit-identical.
__launch_bounds__(kNormThreads) __global__
    void ConvRowImageKernel(const float* __restrict__ p, int ldp,
                            const float* __restrict__ taps,
                            float* const* __restrict__ history,
                            float* __restrict__ y, int ldy, int H, int L,
                            uint4* __restrict__ image, int* __restrict__ exps) {
#pragma clang fp contract(off)
  __shared__ float scratch[kNormThreads / 64];
  __shared__ float s_row[kNormThreads * kNormItems];
  const int row = blockIdx.x;
  const float* pr = p + std::size_t(row) * ldp;
  float maximum = 0.0f;
  for (int ch = threadIdx.x; ch < H; ch += kNormThreads) {
    float* own = history[row] + std::size_t(ch) * (L - 1);
    const float bx = pr[ch] * pr[2 * H + ch];
    const float* w = taps + std::size_t(ch) * L;
    float sum = 0.0f;
    for (int t = 0; t < L - 1; ++t)
      sum += w[t] * own[t];
    sum += w[L - 1] * bx;
    for (int t = 1; t < L - 1; ++t)
      own[t - 1] = own[t];
    own[L - 2] = bx;
    const float out = sum * pr[H + ch];
    if (y)
      y[std::size_t(row) * ldy + ch] = out;
    s_row[ch] = out;
    maximum = fmaxf(maximum, fabsf(out));
  }
  maximum = BlockMax(maximum, scratch);
  WriteOperandRow(s_row, H, row, maximum, image, exps);
}

// Per-head RMSNorm + paired RoPE of one head (the dim / 2 threads own the
// pairs (i, i + dim / 2)); writes the rotated head back and returns the
// pair. Sub-wave reductions cover one head (dim / 2 lanes).
template<int D>
__device__ __forceinline__ void NormRotateHead(float* __restrict__ xh,
                                               const float* __restrict__ w,
                                               const float* __restrict__ frequencies,
                                               const float* __restrict__ factors,
                                               std::uint32_t position, float eps, int pair,
                                               float& r0, float& r1, int parts = 1,
                                               std::size_t part_stride = 0) {
  constexpr int P = D / 2;
  // K parts of the projection added in part order (SumPartsKernel's sum).
  float x0 = xh[pair], x1 = xh[pair + P];
  for (int p = 1; p < parts; ++p) {
    x0 += xh[p * part_stride + pair];
    x1 += xh[p * part_stride + pair + P];
  }
  float squares = fmaf(x0, x0, x1 * x1);
#pragma unroll
  for (int m = P / 2; m; m >>= 1)
    squares += __shfl_xor(squares, m, P);
  const float scale = 1.0f / sqrtf(squares / float(D) + eps);
  const float a = (x0 * scale) * w[pair], b = (x1 * scale) * w[pair + P];
  float angle = float(position) * frequencies[pair];
  if (factors)
    angle /= factors[pair];
  float sn, cs;
  sincosf(angle, &sn, &cs);
  r0 = a * cs - b * sn;
  r1 = b * cs + a * sn;
  xh[pair] = r0;
  xh[pair + P] = r1;
}

// RoPE table (hip/ops.hip:1045-1050): theta^(-2i / dim) as a
// double-precision power of the FP32 exponent, rounded to FP32.
__global__ void RopeTableKernel(float* __restrict__ out, int dim, float theta) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim / 2; i += gridDim.x * blockDim.x) {
    const float exponent = -2.0f * float(i) / float(dim);
    out[i] = float(pow(double(theta), double(exponent)));
  }
}

// Standalone paired RoPE (hip/ops.hip:1052-1071 semantics): one thread per
// (row, head, pair) over a grid-stride walk; the pair (i, i + dim / 2) of
// row (t, h) turns by (position + t) * frequencies[i] (/ factors[i]).
__global__ void RopeRowsKernel(float* __restrict__ x, const float* __restrict__ frequencies,
                               const float* __restrict__ factors, std::size_t units,
                               int heads, int dim, std::uint32_t position) {
  const int half = dim / 2;
  for (std::size_t u = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x; u < units;
       u += std::size_t(gridDim.x) * blockDim.x) {
    const int pair = int(u % half);
    const std::size_t head_row = u / half;
    const std::uint32_t token = std::uint32_t(head_row / heads);
    float angle = float(position + token) * frequencies[pair];
    if (factors)
      angle /= factors[pair];
    float sn, cs;
    sincosf(angle, &sn, &cs);
    float* h = x + head_row * dim;
    const float a = h[pair], b = h[pair + half];
    h[pair] = a * cs - b * sn;
    h[pair + half] = b * cs + a * sn;
  }
}

// F16 rounding of K and V rows (round to nearest even), grid-stride.
__global__ void PackHalvesKernel(const float* __restrict__ k, const float* __restrict__ v,
                                 Half* __restrict__ k16, Half* __restrict__ v16,
                                 std::size_t count) {
  for (std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += std::size_t(gridDim.x) * blockDim.x) {
    k16[i] = FloatToHalfBits(k[i]);
    v16[i] = FloatToHalfBits(v[i]);
  }
}

// Decode heads: a block is one row (with its own position and ring) and
// blockIdx.x walks the query heads, then the KV heads, which also store K
// and V to the row's ring slot position % capacity.
template<int D>
__launch_bounds__(D / 2) __global__
    void HeadsKernel(float* __restrict__ q, float* __restrict__ k,
                     const float* __restrict__ v, int ld,
                     const float* __restrict__ q_norm,
                     const float* __restrict__ k_norm,
                     const float* __restrict__ frequencies,
                     const float* __restrict__ factors,
                     Half* const* __restrict__ cache_k,
                     Half* const* __restrict__ cache_v,
                     const std::uint32_t* __restrict__ positions,
                     const std::uint32_t* __restrict__ capacity, int heads,
                     int kv_heads, float eps) {
  constexpr int P = D / 2;
  const int head = blockIdx.x, row = blockIdx.y, pair = threadIdx.x;
  const bool is_key = head >= heads;
  const int kvh = head - heads;
  float* xh = is_key ? k + std::size_t(row) * ld + kvh * D
                     : q + std::size_t(row) * ld + head * D;
  const std::uint32_t position = positions[row];
  float r0, r1;
  NormRotateHead<D>(xh, is_key ? k_norm : q_norm, frequencies, factors, position, eps, pair,
                    r0, r1);
  if (!is_key)
    return;
  const std::size_t slot =
      std::size_t(position % capacity[row]) * kv_heads * D + std::size_t(kvh) * D;
  const float* vh = v + std::size_t(row) * ld + kvh * D;
  Half* ck = cache_k[row];
  Half* cv = cache_v[row];
  ck[slot + pair] = FloatToHalfBits(r0);
  ck[slot + pair + P] = FloatToHalfBits(r1);
  cv[slot + pair] = FloatToHalfBits(vh[pair]);
  cv[slot + pair + P] = FloatToHalfBits(vh[pair + P]);
}

// Prompt heads (hip/ops.hip:2407-2417 PromptHeads): row r of a chunk is at
// position + r and its K/V go to row r of k16/v16 (kv_heads * D halves a
// row), which is either a staging chunk or the cache rows themselves. A
// projection in K parts is summed here in part order: q (rotated) and the
// per-head gate g land in part 0, K and V go to the F16 rows.
template<int D>
__launch_bounds__(D / 2) __global__
    void PromptHeadsKernel(float* __restrict__ q, float* __restrict__ k,
                           const float* __restrict__ v, int ld,
                           const float* __restrict__ q_norm,
                           const float* __restrict__ k_norm,
                           const float* __restrict__ frequencies,
                           const float* __restrict__ factors, Half* __restrict__ k16,
                           Half* __restrict__ v16, int heads, int kv_heads,
                           std::uint32_t position, float eps, int parts,
                           std::size_t part_stride, float* __restrict__ g) {
  constexpr int P = D / 2;
  const int head = blockIdx.x, row = blockIdx.y, pair = threadIdx.x;
  const bool is_key = head >= heads;
  const int kvh = head - heads;
  float* xh = is_key ? k + std::size_t(row) * ld + kvh * D
                     : q + std::size_t(row) * ld + head * D;
  if (!is_key && parts > 1 && pair == 0) {
    float* gh = g + std::size_t(row) * ld + head;
    float sum = gh[0];
    for (int p = 1; p < parts; ++p)
      sum += gh[p * part_stride];
    gh[0] = sum;
  }
  float r0, r1;
  NormRotateHead<D>(xh, is_key ? k_norm : q_norm, frequencies, factors,
                    position + std::uint32_t(row), eps, pair, r0, r1, parts, part_stride);
  if (!is_key)
    return;
  const std::size_t slot = (std::size_t(row) * kv_heads + kvh) * D;
  const float* vh = v + std::size_t(row) * ld + kvh * D;
  float v0 = vh[pair], v1 = vh[pair + P];
  for (int p = 1; p < parts; ++p) {
    v0 += vh[p * part_stride + pair];
    v1 += vh[p * part_stride + pair + P];
  }
  k16[slot + pair] = FloatToHalfBits(r0);
  k16[slot + pair + P] = FloatToHalfBits(r1);
  v16[slot + pair] = FloatToHalfBits(v0);
  v16[slot + pair + P] = FloatToHalfBits(v1);
}

// StoreKV (hip/ops.hip:1737-1749, engine.cpp:467-470): rows 0..n-1 of a
// chunk at position + r go to ring slot (position + r) % capacity; only the
// last min(n, capacity) rows have distinct slots, so only they are copied.
__global__ void StoreRingKernel(const Half* __restrict__ k16, const Half* __restrict__ v16,
                                Half* __restrict__ ck, Half* __restrict__ cv, int n,
                                int stride, std::uint32_t position, std::uint32_t capacity) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int kept = min(n, int(capacity)), first = n - kept;
  if (i >= std::size_t(kept) * stride)
    return;
  const int r = first + int(i / stride);
  const std::size_t e = i % stride;
  const std::size_t src = std::size_t(r) * stride + e;
  const std::size_t dst = std::size_t((position + std::uint32_t(r)) % capacity) * stride + e;
  ck[dst] = k16[src];
  cv[dst] = v16[src];
}

// Prompt convolution over packed ragged segments (hip/ops.hip:990-1044
// ConvolutionWindow and ConvolutionHistory; engine.cpp:386-400): segment s
// is rows [begin, begin + rows) of p and y and continues its own history
// [H][L - 1] (oldest first). A thread slides one channel's window down
// kConvRows rows, forming each B x product once. The window sum keeps
// ConvStepKernel's expressions and order (reference.cpp:85-101), so n
// prompt rows give bit-identical outputs to n decode steps. For widths up
// to kConvRows + 1 only the threads of a segment's first row group read its
// old history, so they also write the new one (the segment's last L - 1
// products, reaching into the old history when the segment is shorter),
// after their own reads.
constexpr int kConvRows = 16;
constexpr int kMaxConvSegments = 8;
struct ConvSegments {
  float* history[kMaxConvSegments];
  int begin[kMaxConvSegments];
  int rows[kMaxConvSegments];
};

// The new history of channel ch of a segment of `rows` rows (ps: its first
// row of p): hist[j] = the B x product of row rows - (L - 1) + j, or the
// old entry for a row before the segment. Every old entry is read before
// the first write.
template<int kMaxL>
__device__ __forceinline__ void WriteConvHistory(const float* __restrict__ ps, int ldp, int H,
                                                 int ch, int rows, float* hist, int L) {
#pragma clang fp contract(off)
  float past[kMaxL - 1];
#pragma unroll
  for (int j = 0; j < kMaxL - 1; ++j) {
    const int r = rows - (L - 1) + j;
    if (j < L - 1)
      past[j] = r >= 0 ? ps[std::size_t(r) * ldp + ch] * ps[std::size_t(r) * ldp + 2 * H + ch]
                       : hist[(L - 1) + r];
  }
#pragma unroll
  for (int j = 0; j < kMaxL - 1; ++j)
    if (j < L - 1)
      hist[j] = past[j];
}

template<int L>
__global__ void PromptConvKernel(const float* __restrict__ p, int ldp,
                                 const float* __restrict__ taps, ConvSegments seg,
                                 float* __restrict__ y, int ldy, int H, int update_history) {
#pragma clang fp contract(off)
  const int s = blockIdx.z, ch = blockIdx.x * blockDim.x + threadIdx.x;
  const int first = blockIdx.y * kConvRows, rows = seg.rows[s];
  if (ch >= H || first >= rows)
    return;
  const float* ps = p + std::size_t(seg.begin[s]) * ldp;
  float* ys = y + std::size_t(seg.begin[s]) * ldy;
  float* hist = seg.history[s] + std::size_t(ch) * (L - 1);
  // Every load of the thread's rows is issued before any arithmetic: the
  // L - 1 products before the first row (from p, or the history before the
  // segment) and B, C, x of each of its rows.
  float w[L], pre[L - 1], bv[kConvRows], cv[kConvRows], xv[kConvRows];
#pragma unroll
  for (int t = 0; t < L; ++t)
    w[t] = taps[std::size_t(ch) * L + t];
#pragma unroll
  for (int t = 0; t < L - 1; ++t) {
    const int r = first - (L - 1) + t;
    pre[t] = r >= 0 ? ps[std::size_t(r) * ldp + ch] * ps[std::size_t(r) * ldp + 2 * H + ch]
                    : hist[(L - 1) + r];
  }
#pragma unroll
  for (int i = 0; i < kConvRows; ++i) {
    const int r = first + i;
    const bool live = r < rows;
    const float* pr = ps + std::size_t(live ? r : first) * ldp;
    bv[i] = pr[ch];
    cv[i] = pr[H + ch];
    xv[i] = pr[2 * H + ch];
  }
  // win[t] holds the product of row r - (L - 1) + t.
  float win[L];
#pragma unroll
  for (int t = 0; t < L - 1; ++t)
    win[t + 1] = pre[t];
#pragma unroll
  for (int i = 0; i < kConvRows; ++i) {
    const int r = first + i;
#pragma unroll
    for (int t = 0; t < L - 1; ++t)
      win[t] = win[t + 1];
    win[L - 1] = bv[i] * xv[i];
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < L; ++t)
      sum += w[t] * win[t];
    if (r < rows)
      ys[std::size_t(r) * ldy + ch] = sum * cv[i];
  }
  if (update_history && first == 0)
    WriteConvHistory<L>(ps, ldp, H, ch, rows, hist, L);
}

// The prompt convolution of one segment fused with the FP16 row-scaled
// activations of its output (the output projection's GEMM input,
// hip/q8_prefill.hpp:27-51): a block owns kConvHalfRows consecutive rows and
// every channel, so each output row is whole in the block. A thread takes V
// consecutive channels, keeps PromptConvKernel's expressions and order for
// every output, the block reduces each row's max |y|, and the row is stored
// as fp16(y 2^e) with scale 2^-e (HalfRowsKernel's expressions), so the FP16
// rows equal lfm3_conv_prompt followed by lfm3_half_rows bit for bit.
// Outputs of rows before `skip` are not stored (no later layer reads
// them); their products still feed the windows of the live rows. Block 0
// holds the lowest rows: it alone reads the old history (kConvHalfRows >=
// L - 1, so later blocks' windows start at row 0 or after), and it writes
// the new one after the block barrier that follows every thread's reads.
// Six rows a block (86 blocks for 512 rows; 8 rows: 9.5 us against 8.5
// for the 512-row pass shape) and four channels a thread (two: 9.5 us).
constexpr int kConvHalfRows = 6, kConvHalfV = 4;
constexpr int kConvHalfMaxHidden = 2048, kConvHalfMaxThreads = kConvHalfMaxHidden / kConvHalfV;
// Widths past 7 hold more than the 256 registers a lane has here.
constexpr int kConvHalfMaxWidth = 7;
static_assert(kConvHalfMaxWidth <= kConvHalfRows + 1, "window within the block's reach");

// V consecutive floats at a 4 V-byte aligned offset (zeros out of range).
template<int V>
__device__ __forceinline__ void LoadVec(BufferResource res, unsigned offset, float* v) {
  if constexpr (V == 4) {
    const float4 f = LoadF4(res, offset);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
  } else if constexpr (V == 2) {
    typedef unsigned u2 __attribute__((ext_vector_type(2)));
    const u2 f = __builtin_amdgcn_raw_buffer_load_b64(res, offset, 0, 0);
    v[0] = __uint_as_float(f.x);
    v[1] = __uint_as_float(f.y);
  } else {
    v[0] = __uint_as_float(LoadB32(res, offset));
  }
}

template<int L, int V>
__launch_bounds__(kConvHalfMaxThreads) __global__ void PromptConvHalfKernel(
    const float* __restrict__ p, int ldp, const float* __restrict__ taps,
    float* __restrict__ history, int rows, int skip, int first0, Half* __restrict__ out,
    int lda, float* __restrict__ scale, int H, int update_history) {
#pragma clang fp contract(off)
  static_assert(L >= 2 && L <= kConvHalfMaxWidth, "supported width");
  constexpr int R = kConvHalfRows;
  __shared__ float s_max[R][kConvHalfMaxThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int waves = int(blockDim.x) / 64;
  const int first = first0 + int(blockIdx.x) * R;
  const int padded = (H + kChunk - 1) / kChunk * kChunk;
  const bool live = tid * V < H;
  const int c0 = live ? tid * V : 0;
  // Buffer loads throughout: a row outside its range reads zeros without a
  // branch, and every load of a thread is issued before the first product.
  const BufferResource p_res = MakeBuffer(p, unsigned(std::size_t(rows) * ldp * 4));
  const BufferResource t_res = MakeBuffer(taps, unsigned(H * L * 4));
  const BufferResource h_res = MakeBuffer(history, unsigned(H * (L - 1) * 4));
  const bool history_block = update_history && blockIdx.x == 0;
  // The thread's taps (V L consecutive floats).
  float tw[V * L];
#pragma unroll
  for (int i = 0; i < L; ++i)
    LoadVec<V>(t_res, unsigned((c0 * L + V * i) * 4), tw + V * i);
  // The L - 1 products before the block's first row: for the block at row 0
  // the old history (every such row is before the segment; V (L - 1)
  // consecutive floats), taken as the entry times an exact 1; for any other
  // block (first >= kConvHalfRows >= L - 1) B x of rows of p.
  float pb[L - 1][V], px[L - 1][V], hv[V * (L - 1)];
  if (first == 0) {
#pragma unroll
    for (int i = 0; i < L - 1; ++i)
      LoadVec<V>(h_res, unsigned((c0 * (L - 1) + V * i) * 4), hv + V * i);
  } else {
#pragma unroll
    for (int t = 0; t < L - 1; ++t) {
      const unsigned at = unsigned((std::size_t(first - (L - 1) + t) * ldp + c0) * 4);
      LoadVec<V>(p_res, at, pb[t]);
      LoadVec<V>(p_res, at + unsigned(2 * H) * 4u, px[t]);
    }
  }
  // B, C, x of the block's rows (rows past the segment read zeros and are
  // not stored).
  float bv[R][V], cv[R][V], xv[R][V];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int r = first + i;
    const unsigned at = r < rows ? unsigned((std::size_t(r) * ldp + c0) * 4) : kOutOfRange;
    LoadVec<V>(p_res, at, bv[i]);
    LoadVec<V>(p_res, r < rows ? at + unsigned(H) * 4u : kOutOfRange, cv[i]);
    LoadVec<V>(p_res, r < rows ? at + unsigned(2 * H) * 4u : kOutOfRange, xv[i]);
  }
  // Block 0's new history (the segment's last L - 1 B x products, or old
  // entries for rows before the segment): B and x of those rows.
  float nb[L - 1][V], nx[L - 1][V];
  if (history_block) {
#pragma unroll
    for (int t = 0; t < L - 1; ++t) {
      const int r = rows - (L - 1) + t;
      const unsigned at = r >= 0 ? unsigned((std::size_t(r) * ldp + c0) * 4) : kOutOfRange;
      LoadVec<V>(p_res, at, nb[t]);
      LoadVec<V>(p_res, r >= 0 ? at + unsigned(2 * H) * 4u : kOutOfRange, nx[t]);
    }
  }
  // Keeps the products below every load: one memory round trip.
  __builtin_amdgcn_sched_barrier(0);
  if (first == 0) {
#pragma unroll
    for (int t = 0; t < L - 1; ++t)
#pragma unroll
      for (int c = 0; c < V; ++c) {
        pb[t][c] = hv[c * (L - 1) + t];
        px[t][c] = 1.0f;
      }
  }
  float win[L][V];
#pragma unroll
  for (int t = 0; t < L - 1; ++t)
#pragma unroll
    for (int c = 0; c < V; ++c)
      win[t + 1][c] = pb[t][c] * px[t][c];
  float y[R][V], row_max[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
#pragma unroll
    for (int t = 0; t < L - 1; ++t)
#pragma unroll
      for (int c = 0; c < V; ++c)
        win[t][c] = win[t + 1][c];
#pragma unroll
    for (int c = 0; c < V; ++c)
      win[L - 1][c] = bv[i][c] * xv[i][c];
    row_max[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < V; ++c) {
      float sum = 0.0f;
#pragma unroll
      for (int t = 0; t < L; ++t)
        sum += tw[c * L + t] * win[t][c];
      y[i][c] = sum * cv[i][c];
      row_max[i] = fmaxf(row_max[i], fabsf(y[i][c]));
    }
    if (!live)
      row_max[i] = 0.0f;
  }
  // Each row's maximum over the block (rows past the segment are unused).
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const float m = WaveMax(row_max[i]);
    if (lane == 0)
      s_max[i][wave] = m;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float m = 0.0f;
    for (int w = 0; w < waves; ++w)
      m = fmaxf(m, s_max[i][w]);
    row_max[i] = m;
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int r = first + i;
    if (r < skip || r >= rows)
      continue;
    const int e = RowExponent(row_max[i]);
    Half* dst = out + std::size_t(r - skip) * lda;
    if (tid == 0)
      scale[r - skip] = ldexpf(1.0f, -e);
    if (live) {
      unsigned h[(V + 1) / 2];
#pragma unroll
      for (int c = 0; c < V; c += 2)
        h[c / 2] = unsigned(ScaledHalf(y[i][c], e)) |
                   (c + 1 < V ? unsigned(ScaledHalf(y[i][c + 1], e)) << 16 : 0u);
      if constexpr (V == 4)
        *reinterpret_cast<uint2*>(dst + c0) = make_uint2(h[0], h[1]);
      else if constexpr (V == 2)
        *reinterpret_cast<unsigned*>(dst + c0) = h[0];
      else
        dst[c0] = Half(h[0]);
    }
    for (int k = H + tid; k < padded; k += int(blockDim.x))  // the chunk's zero tail
      dst[k] = Half(0);
  }
  if (history_block && live) {
    // WriteConvHistory's entries for the thread's channels: entry t of
    // channel c is the B x product of row rows - (L - 1) + t, or for a row
    // before the segment the old entry rows + t (loaded above: this block's
    // first row is 0 whenever rows < L - 1). Every old entry of these
    // channels was read by this thread.
    float e[V * (L - 1)];
#pragma unroll
    for (int t = 0; t < L - 1; ++t) {
      const int r = rows - (L - 1) + t;
#pragma unroll
      for (int c = 0; c < V; ++c)
        e[c * (L - 1) + t] = r >= 0 ? nb[t][c] * nx[t][c] : hv[c * (L - 1) + (rows + t)];
    }
#pragma unroll
    for (int i = 0; i < V * (L - 1); ++i)
      StoreF32(h_res, unsigned((c0 * (L - 1) + i) * 4), e[i]);
  }
}

// Any width: each output recomputes its window's products (same values and
// order as PromptConvKernel).
__global__ void PromptConvAnyKernel(const float* __restrict__ p, int ldp,
                                    const float* __restrict__ taps, ConvSegments seg,
                                    float* __restrict__ y, int ldy, int H, int L,
                                    int update_history) {
#pragma clang fp contract(off)
  const int s = blockIdx.z, ch = blockIdx.x * blockDim.x + threadIdx.x;
  const int first = blockIdx.y * kConvRows, rows = seg.rows[s];
  if (ch >= H || first >= rows)
    return;
  const float* ps = p + std::size_t(seg.begin[s]) * ldp;
  float* ys = y + std::size_t(seg.begin[s]) * ldy;
  float* hist = seg.history[s] + std::size_t(ch) * (L - 1);
  const int last = min(first + kConvRows, rows);
  for (int r = first; r < last; ++r) {
    float sum = 0.0f;
    for (int t = 0; t < L; ++t) {
      const int src = r - (L - 1) + t;
      const float b = src >= 0 ? ps[std::size_t(src) * ldp + ch] *
                                     ps[std::size_t(src) * ldp + 2 * H + ch]
                               : hist[(L - 1) + src];
      sum += taps[std::size_t(ch) * L + t] * b;
    }
    ys[std::size_t(r) * ldy + ch] = sum * ps[std::size_t(r) * ldp + H + ch];
  }
  if (update_history && first == 0)
    WriteConvHistory<32>(ps, ldp, H, ch, rows, hist, L);
}

// The history after a segment, as a launch of its own: for widths past
// kConvRows + 1 the second row group's windows also read the old history.
__global__ void PromptConvHistoryKernel(const float* __restrict__ p, int ldp,
                                        ConvSegments seg, int H, int L) {
  const int s = blockIdx.y, ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= H)
    return;
  WriteConvHistory<32>(p + std::size_t(seg.begin[s]) * ldp, ldp, H, ch, seg.rows[s],
                       seg.history[s] + std::size_t(ch) * (L - 1), L);
}

// Greedy argmax: one block per row scans the row with a 64-bit key per
// element (ordered value bits above the complemented index, so the largest
// key is the largest value at its first index, as std::max_element) and
// reduces it over the block; no cross-block merge.
constexpr int kArgmaxThreads = 1024;

__launch_bounds__(kArgmaxThreads) __global__
    void ArgmaxKernel(const float* __restrict__ logits, int cols,
                      std::uint32_t* __restrict__ ids) {
  __shared__ unsigned long long best[kArgmaxThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* lr = logits + std::size_t(row) * cols;
  unsigned long long key = 0;
  int c = tid * 4;
  for (; c + 3 < cols; c += kArgmaxThreads * 4) {
    const float4 v = *reinterpret_cast<const float4*>(lr + c);
    unsigned long long k = ArgKey(v.x, unsigned(c));
    key = k > key ? k : key;
    k = ArgKey(v.y, unsigned(c + 1));
    key = k > key ? k : key;
    k = ArgKey(v.z, unsigned(c + 2));
    key = k > key ? k : key;
    k = ArgKey(v.w, unsigned(c + 3));
    key = k > key ? k : key;
  }
  for (; c < cols; ++c) {  // the ragged tail (cols % 4)
    const unsigned long long k = ArgKey(lr[c], unsigned(c));
    key = k > key ? k : key;
  }
#pragma unroll
  for (int m = 32; m; m >>= 1) {
    const unsigned long long other = __shfl_xor(key, m, 64);
    key = other > key ? other : key;
  }
  if ((tid & 63) == 0)
    best[tid >> 6] = key;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w)
      key = best[w] > key ? best[w] : key;
    ids[row] = 0xffffffffu - unsigned(key & 0xffffffffu);
  }
}

// ids[t] from per-block candidate keys: keys[t * groups + j] is the best
// ArgKey of block j's rows for token t. A thread's keys (j = tid + 256 i)
// are loaded kKeysPer at a time, all in flight together: one memory round
// trip for up to 4096 groups (the vocabulary head's 4000), where a load
// per loop step waited for each in turn (5.2 us a launch). Keys are
// distinct (they hold the row), so the maximum does not depend on order.
constexpr int kKeysPer = 16;
__launch_bounds__(256) __global__
    void ArgmaxKeysKernel(const unsigned long long* __restrict__ keys, int groups,
                          std::uint32_t* __restrict__ ids) {
  __shared__ unsigned long long best[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const unsigned long long* kr = keys + std::size_t(t) * groups;
  unsigned long long key = 0;
  for (int j0 = tid; j0 < groups; j0 += 256 * kKeysPer) {
    unsigned long long v[kKeysPer];
#pragma unroll
    for (int i = 0; i < kKeysPer; ++i) {
      const int j = j0 + 256 * i;
      v[i] = j < groups ? kr[j] : 0ull;
    }
#pragma unroll
    for (int i = 0; i < kKeysPer; ++i)
      key = v[i] > key ? v[i] : key;
  }
#pragma unroll
  for (int m = 32; m; m >>= 1) {
    const unsigned long long other = __shfl_xor(key, m, 64);
    key = other > key ? other : key;
  }
  if ((tid & 63) == 0)
    best[tid >> 6] = key;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w)
      key = best[w] > key ? best[w] : key;
    ids[t] = 0xffffffffu - unsigned(key & 0xffffffffu);
  }
}

__global__ void ScatterRowsKernel(const float* __restrict__ src, std::size_t ld,
                                  float* const* __restrict__ dst,
                                  std::size_t count) {
  const int row = blockIdx.y;
  const std::size_t i = (std::size_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const float* s = src + row * ld;
  float* d = dst[row];
  if (i + 4 <= count) {
    *reinterpret_cast<float4*>(d + i) = *reinterpret_cast<const float4*>(s + i);
  } else {
    for (std::size_t k = i; k < count; ++k)
      d[k] = s[k];
  }
}

}  // namespace

int LaunchNormImage(const NormImageArgs& a, std::uint32_t rows, hipStream_t stream) {
  if (Chunks(unsigned(a.H)) * 8 <= kImageNormThreads)
    NormImageKernel<1><<<rows, kImageNormThreads, 0, stream>>>(a);
  else
    NormImageKernel<2><<<rows, kImageNormThreads, 0, stream>>>(a);
  return HipStatus(hipGetLastError(), "LFM3 residual norm launch");
}

int LaunchArgmaxKeys(const unsigned long long* keys, std::uint32_t rows, std::uint32_t groups,
                     std::uint32_t* ids, hipStream_t stream) {
  ArgmaxKeysKernel<<<rows, 256, 0, stream>>>(keys, int(groups), ids);
  return HipStatus(hipGetLastError(), "LFM3 argmax launch");
}

int LaunchScatterRows(const float* src, std::size_t ld, float* const* dst,
                      std::uint32_t rows, std::size_t count,
                      hipStream_t stream) {
  const std::size_t threads = (count + 3) / 4;
  const dim3 grid(unsigned((threads + 255) / 256), rows);
  ScatterRowsKernel<<<grid, 256, 0, stream>>>(src, ld, dst, count);
  return HipStatus(hipGetLastError(), "LFM3 row scatter launch");
}

}  // namespace lfm3amd

namespace lfm3amd {

void LaunchPromptHeads(float* q, float* k, const float* v, std::uint32_t ld, const float* q_norm,
                       const float* k_norm, const float* frequencies, const float* factors,
                       std::uint16_t* k16, std::uint16_t* v16, std::uint32_t rows,
                       std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
                       std::uint32_t position, float eps, std::uint32_t parts,
                       std::size_t part_stride, float* g, hipStream_t s) {
  const dim3 grid(heads + kv_heads, rows);
  if (dim == 128)
    PromptHeadsKernel<128><<<grid, 64, 0, s>>>(q, k, v, int(ld), q_norm, k_norm, frequencies,
                                               factors, k16, v16, int(heads), int(kv_heads),
                                               position, eps, int(parts), part_stride, g);
  else
    PromptHeadsKernel<64><<<grid, 32, 0, s>>>(q, k, v, int(ld), q_norm, k_norm, frequencies,
                                              factors, k16, v16, int(heads), int(kv_heads),
                                              position, eps, int(parts), part_stride, g);
}

}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

const char* lfm3_last_error(void) { return g_error.c_str(); }

int lfm3_residual_norm_parts(const float* branch, std::uint32_t parts,
                             std::size_t part_stride, const float* post_norm,
                             float* x, const float* norm, float* z,
                             std::uint32_t rows, std::uint32_t hidden,
                             float eps, void* stream) {
  if (!x || !rows || !hidden || hidden > kNormThreads * kNormItems ||
      (norm && !z) || !parts || parts > kNormParts ||
      (parts > 1 && part_stride < std::size_t(rows) * hidden))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 residual norm shape");
  ResidualNormKernel<<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      branch, int(parts), part_stride, branch ? post_norm : nullptr, x, norm, z,
      int(hidden), eps, nullptr, nullptr, nullptr, 0, nullptr);
  return HipStatus(hipGetLastError(), "LFM3 residual norm launch");
}

int lfm3_residual_norm_image(const float* branch, std::uint32_t parts,
                             std::size_t part_stride, const float* post_norm,
                             float* x, const float* norm, float* z, void* image,
                             int* exps, std::uint32_t rows,
                             std::uint32_t hidden, float eps, void* stream) {
  if (!x || !norm || !image || !exps || !rows || rows > 8 || !hidden ||
      hidden % 32 || hidden > kNormThreads * kNormItems || !parts ||
      parts > kNormParts || (parts > 1 && part_stride < std::size_t(rows) * hidden) ||
      (reinterpret_cast<std::uintptr_t>(image) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 residual norm image shape");
  const auto* post = branch ? post_norm : nullptr;
  auto* im = static_cast<uint4*>(image);
  const auto st = static_cast<hipStream_t>(stream);
  if (Chunks(hidden) * 8 > 2 * kImageNormThreads) {
    ResidualNormKernel<<<rows, kNormThreads, 0, st>>>(
        branch, int(parts), part_stride, post, x, norm, z, int(hidden), eps, im, exps,
        nullptr, 0, nullptr);
    return HipStatus(hipGetLastError(), "LFM3 residual norm launch");
  }
  NormImageArgs a{};
  a.branch = branch;
  a.parts = int(parts);
  a.part_stride = part_stride;
  a.post = post;
  a.x = x;
  a.weight = norm;
  a.z = z;
  a.H = int(hidden);
  a.eps = eps;
  a.image = im;
  a.exps = exps;
  return LaunchNormImage(a, rows, st);
}

int lfm3_residual_norm_half(const float* branch, std::uint32_t parts,
                            std::size_t part_stride, const float* post_norm, float* x,
                            const float* norm, float* z, std::uint16_t* a16,
                            std::uint32_t lda, float* scale, std::uint32_t rows,
                            std::uint32_t hidden, float eps, void* stream) {
  if (!x || !norm || !a16 || !scale || !rows || !hidden ||
      hidden > kNormThreads * kNormItems || lda < hidden || lda % 64 || !parts ||
      parts > kNormParts || (parts > 1 && part_stride < std::size_t(rows) * hidden))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 residual norm shape");
  const auto aligned = [](const void* p) {
    return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0;
  };
  if (Chunks(hidden) * 8 <= 2 * kImageNormThreads && hidden % 32 == 0 && aligned(a16) &&
      aligned(x) && aligned(z)) {
    NormImageArgs a{};
    a.branch = branch;
    a.parts = int(parts);
    a.part_stride = part_stride;
    a.post = branch ? post_norm : nullptr;
    a.x = x;
    a.weight = norm;
    a.z = z;
    a.H = int(hidden);
    a.eps = eps;
    a.a16 = a16;
    a.lda = int(lda);
    a.a_scale = scale;
    return LaunchNormImage(a, rows, static_cast<hipStream_t>(stream));
  }
  ResidualNormKernel<<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      branch, int(parts), part_stride, branch ? post_norm : nullptr, x, norm, z,
      int(hidden), eps, nullptr, nullptr, a16, int(lda), scale);
  return HipStatus(hipGetLastError(), "LFM3 residual norm launch");
}

int lfm3_conv_step_ragged_image(const float* p, std::uint32_t ldp,
                                const float* taps, float* const* history,
                                float* y, std::uint32_t ldy, void* image,
                                int* exps, std::uint32_t rows,
                                std::uint32_t hidden, std::uint32_t width,
                                void* stream) {
  if (!p || !taps || !history || !image || !exps || !rows || rows > 8 ||
      !hidden || hidden % 32 || hidden > kNormThreads * kNormItems ||
      width < 2 || width > 32 || ldp < 3 * hidden || (y && ldy < hidden) ||
      (reinterpret_cast<std::uintptr_t>(image) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 convolution image shape");
  ConvRowImageKernel<<<rows, kNormThreads, 0, static_cast<hipStream_t>(stream)>>>(
      p, int(ldp), taps, history, y, int(ldy), int(hidden), int(width),
      static_cast<uint4*>(image), exps);
  return HipStatus(hipGetLastError(), "LFM3 convolution launch");
}

int lfm3_residual_norm(const float* branch, const float* post_norm, float* x,
                       const float* norm, float* z, std::uint32_t rows,
                       std::uint32_t hidden, float eps, void* stream) {
  return lfm3_residual_norm_parts(branch, 1, 0, post_norm, x, norm, z, rows,
                                  hidden, eps, stream);
}

int lfm3_conv_step_ragged(const float* p, std::uint32_t ldp, const float* taps,
                          float* const* history, float* y, std::uint32_t ldy,
                          std::uint32_t rows, std::uint32_t hidden,
                          std::uint32_t width, void* stream) {
  if (!p || !taps || !history || !y || !rows || !hidden || width < 2 ||
      width > 32 || ldp < 3 * hidden || ldy < hidden)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 convolution shape");
  const dim3 grid((hidden + 255) / 256, rows);
  ConvStepKernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      p, int(ldp), taps, history, y, int(ldy), int(hidden), int(width));
  return HipStatus(hipGetLastError(), "LFM3 convolution launch");
}

int lfm3_decode_heads_ragged(float* q, float* k, const float* v,
                             std::uint32_t ld, const float* q_norm,
                             const float* k_norm, const float* frequencies,
                             const float* factors, std::uint16_t* const* cache_k,
                             std::uint16_t* const* cache_v,
                             const std::uint32_t* positions,
                             const std::uint32_t* capacity, std::uint32_t rows,
                             std::uint32_t heads, std::uint32_t kv_heads,
                             std::uint32_t dim, float eps, void* stream) {
  if (!q || !k || !v || !q_norm || !k_norm || !frequencies || !cache_k ||
      !cache_v || !positions || !capacity || !rows || !heads || !kv_heads ||
      heads % kv_heads || (dim != 64 && dim != 128))
    return Fail(LFM3_E_INVALID, "LFM3 decode heads need dimension 64 or 128");
  const dim3 grid(heads + kv_heads, rows);
  const auto s = static_cast<hipStream_t>(stream);
  if (dim == 128)
    HeadsKernel<128><<<grid, 64, 0, s>>>(q, k, v, int(ld), q_norm, k_norm,
                                         frequencies, factors, cache_k, cache_v,
                                         positions, capacity, int(heads),
                                         int(kv_heads), eps);
  else
    HeadsKernel<64><<<grid, 32, 0, s>>>(q, k, v, int(ld), q_norm, k_norm,
                                        frequencies, factors, cache_k, cache_v,
                                        positions, capacity, int(heads),
                                        int(kv_heads), eps);
  return HipStatus(hipGetLastError(), "LFM3 decode heads launch");
}

int lfm3_prompt_heads(float* q, float* k, const float* v, std::uint32_t ld,
                      const float* q_norm, const float* k_norm, const float* frequencies,
                      const float* factors, std::uint16_t* k16, std::uint16_t* v16,
                      std::uint32_t rows, std::uint32_t heads, std::uint32_t kv_heads,
                      std::uint32_t dim, std::uint32_t position, float eps, void* stream) {
  if (!q || !k || !v || !q_norm || !k_norm || !frequencies || !k16 || !v16 || !rows ||
      !heads || !kv_heads || heads % kv_heads || (dim != 64 && dim != 128) ||
      rows > 65535 || std::uint64_t(position) + rows > (1ull << 31))
    return Fail(LFM3_E_INVALID, "LFM3 prompt heads need dimension 64 or 128");
  LaunchPromptHeads(q, k, v, ld, q_norm, k_norm, frequencies, factors, k16, v16, rows, heads,
                    kv_heads, dim, position, eps, 1, 0, nullptr, static_cast<hipStream_t>(stream));
  return HipStatus(hipGetLastError(), "LFM3 prompt heads launch");
}

int lfm3_rope_frequencies(float* out, std::uint32_t dim, float theta, void* stream) {
  if (!out || dim < 2 || dim % 2 || dim > 1024 || !(theta > 0))
    return Fail(LFM3_E_INVALID, "invalid LFM3 RoPE table");
  RopeTableKernel<<<1, 512, 0, static_cast<hipStream_t>(stream)>>>(out, int(dim), theta);
  return HipStatus(hipGetLastError(), "LFM3 RoPE table launch");
}

int lfm3_rope(float* x, const float* frequencies, const float* factors, std::uint32_t n,
              std::uint32_t heads, std::uint32_t dim, std::uint32_t position, void* stream) {
  if (!x || !frequencies || !n || !heads || dim < 2 || dim % 2 || dim > 1024)
    return Fail(LFM3_E_INVALID, "invalid LFM3 RoPE shape");
  const std::size_t units = std::size_t(n) * heads * (dim / 2);
  const unsigned blocks = unsigned(std::min<std::size_t>((units + 255) / 256, 8192));
  RopeRowsKernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      x, frequencies, factors, units, int(heads), int(dim), position);
  return HipStatus(hipGetLastError(), "LFM3 RoPE launch");
}

int lfm3_pack_kv(const float* k, const float* v, std::uint16_t* k16, std::uint16_t* v16,
                 std::size_t count, void* stream) {
  if (!count)
    return LFM3_OK;
  if (!k || !v || !k16 || !v16)
    return Fail(LFM3_E_INVALID, "invalid LFM3 K/V pack");
  const unsigned blocks = unsigned(std::min<std::size_t>((count + 255) / 256, 8192));
  PackHalvesKernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(k, v, k16, v16, count);
  return HipStatus(hipGetLastError(), "LFM3 K/V pack launch");
}

int lfm3_store_kv(const std::uint16_t* k16, const std::uint16_t* v16, std::uint16_t* cache_k,
                  std::uint16_t* cache_v, std::uint32_t rows, std::uint32_t stride,
                  std::uint32_t position, std::uint32_t capacity, void* stream) {
  if (!k16 || !v16 || !cache_k || !cache_v || !rows || !stride || !capacity)
    return Fail(LFM3_E_INVALID, "invalid LFM3 K/V ring store");
  const std::size_t count = std::size_t(std::min(rows, capacity)) * stride;
  StoreRingKernel<<<(count + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
      k16, v16, cache_k, cache_v, int(rows), int(stride), position, capacity);
  return HipStatus(hipGetLastError(), "LFM3 K/V ring store launch");
}

int lfm3_conv_prompt_half(const float* p, std::uint32_t ldp, const float* taps,
                          float* history, std::uint32_t rows, std::uint32_t skip,
                          std::uint16_t* out, std::uint32_t lda, float* scale,
                          std::uint32_t hidden, std::uint32_t width, int update_history,
                          void* stream) {
  if (!p || !taps || !history || !out || !scale || !rows || skip >= rows || !hidden ||
      hidden % kConvHalfV || width < 2 || width > std::uint32_t(kConvHalfMaxWidth) ||
      ldp < 3 * hidden || lda % kChunk || lda < hidden ||
      hidden > std::uint32_t(kConvHalfMaxHidden) ||
      !BufferFits(std::size_t(rows) * ldp * 4))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt convolution (FP16 rows) shape");
  const auto s = static_cast<hipStream_t>(stream);
  const std::uint32_t first0 = skip / kConvHalfRows * kConvHalfRows;
  const unsigned blocks = (rows - first0 + kConvHalfRows - 1) / kConvHalfRows;
  const unsigned threads = (hidden / kConvHalfV + 63) / 64 * 64;
  const auto go = [&](auto kernel) {
    kernel<<<blocks, threads, 0, s>>>(p, int(ldp), taps, history, int(rows), int(skip),
                                      int(first0), out, int(lda), scale, int(hidden),
                                      update_history);
  };
  switch (width) {
    case 2: go(PromptConvHalfKernel<2, kConvHalfV>); break;
    case 3: go(PromptConvHalfKernel<3, kConvHalfV>); break;
    case 4: go(PromptConvHalfKernel<4, kConvHalfV>); break;
    case 5: go(PromptConvHalfKernel<5, kConvHalfV>); break;
    case 6: go(PromptConvHalfKernel<6, kConvHalfV>); break;
    default: go(PromptConvHalfKernel<7, kConvHalfV>); break;
  }
  return HipStatus(hipGetLastError(), "LFM3 prompt convolution (FP16 rows) launch");
}

int lfm3_conv_prompt(const float* p, std::uint32_t ldp, const float* taps,
                     float* const* history, const std::uint32_t* begin,
                     const std::uint32_t* rows, std::uint32_t segments, float* y,
                     std::uint32_t ldy, std::uint32_t hidden, std::uint32_t width,
                     int update_history, void* stream) {
  if (!p || !taps || !history || !begin || !rows || !y || !segments ||
      segments > kMaxConvSegments || !hidden || width < 2 || width > 32 ||
      ldp < 3 * hidden || ldy < hidden)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt convolution shape");
  ConvSegments seg{};
  std::uint32_t most = 0;
  for (std::uint32_t i = 0; i < segments; ++i) {
    if (!history[i] || !rows[i])
      return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt convolution shape");
    seg.history[i] = history[i];
    seg.begin[i] = int(begin[i]);
    seg.rows[i] = int(rows[i]);
    most = std::max(most, rows[i]);
  }
  const auto s = static_cast<hipStream_t>(stream);
  const dim3 grid((hidden + 127) / 128, (most + kConvRows - 1) / kConvRows, segments);
  // The first row group's threads move the history when only they read it.
  const bool in_kernel = width - 1 <= std::uint32_t(kConvRows);
  if (width == 7)
    PromptConvKernel<7><<<grid, 128, 0, s>>>(p, int(ldp), taps, seg, y, int(ldy), int(hidden),
                                             update_history);
  else
    PromptConvAnyKernel<<<grid, 128, 0, s>>>(p, int(ldp), taps, seg, y, int(ldy), int(hidden),
                                             int(width), update_history && in_kernel);
  if (update_history && !in_kernel)
    PromptConvHistoryKernel<<<dim3((hidden + 127) / 128, segments), 128, 0, s>>>(
        p, int(ldp), seg, int(hidden), int(width));
  return HipStatus(hipGetLastError(), "LFM3 prompt convolution launch");
}

std::size_t lfm3_argmax_workspace_bytes(std::uint32_t rows) {
  (void)rows;  // one block per row: no workspace
  return 0;
}

int lfm3_argmax(const float* logits, std::uint32_t rows, std::uint32_t cols,
                std::uint32_t* ids, void* workspace, std::size_t workspace_bytes,
                void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (!logits || !ids || !rows || !cols || cols % 4 ||
      (reinterpret_cast<std::uintptr_t>(logits) & 15))
    return Fail(LFM3_E_INVALID, "invalid LFM3 argmax");
  ArgmaxKernel<<<rows, kArgmaxThreads, 0, static_cast<hipStream_t>(stream)>>>(
      logits, int(cols), ids);
  return HipStatus(hipGetLastError(), "LFM3 argmax launch");
}

}  // extern "C"
