// Ragged decode attention on gfx950: one launch covers every session of a
// decode round. A work item is (row, key span); blockIdx.y is the KV head.
// Keys come from the row's own F16 ring (slot t % capacity), sliding
// layers reading only the last `window` positions (the item list encodes
// the window). Q, scores, probabilities and accumulation stay FP32, as in
// the reference decode (hip/ops.hip:1578-1691).
//
// Block = 4 waves. A wave splits into 128 / D sub-waves whose lanes own two
// dimensions each, so one dword load per lane reads a whole key row. A
// sub-wave takes batches of KB keys: the KB x G partial dots are reduced by
// a halving butterfly (each exchange halves the values a lane carries, so
// N values cost about 2N shuffles instead of N log2(lanes)), leaving each
// lane one (head, key) score; max and sum finish over the key bits, then
// the probabilities are broadcast back for the P.V update of every head.
// Streams merge through LDS; multi-span rows leave per-span partials that
// a second launch merges in span order, so results do not depend on block
// scheduling.
#include <cmath>

#include "common.hpp"

namespace lfm3amd {
namespace {

constexpr int kSpan = 256;       // keys per work item
constexpr int kAttnThreads = 256;

template<int LANES>
__device__ __forceinline__ float SubShfl(float v, int src_in_sub) {
  if constexpr (LANES == 64) {
    return __shfl(v, src_in_sub, 64);
  } else {
    const int base = threadIdx.x & 63 & ~(LANES - 1);
    return __shfl(v, base + src_in_sub, 64);
  }
}

template<int D, int G>
__launch_bounds__(kAttnThreads) __global__
    void DecodeAttentionKernel(const float* __restrict__ q, int ldq,
                               const float* __restrict__ gate, int ldg,
                               const Half* const* __restrict__ cache_k,
                               const Half* const* __restrict__ cache_v,
                               const std::uint32_t* __restrict__ capacity,
                               const lfm3_attention_item* __restrict__ items,
                               float* __restrict__ out, int ldo, int kv_heads,
                               float* __restrict__ partial) {
  constexpr int SUBS = 128 / D, LANES = 64 / SUBS;
  constexpr int KB = (LANES / G) < 8 ? (LANES / G) : 8;
  constexpr int N = KB * G;
  constexpr int LOG_LANES = LANES == 64 ? 6 : 5;
  constexpr int LOG_N = N == 64 ? 6 : N == 32 ? 5 : N == 16 ? 4 : N == 8 ? 3 : 2;
  constexpr int SH = LOG_LANES - LOG_N;
  constexpr int STREAMS = (kAttnThreads / 64) * SUBS;
  constexpr int LOG_KB = KB == 8 ? 3 : KB == 4 ? 2 : 1;

  __shared__ float s_acc[STREAMS][G][D];
  __shared__ float s_m[STREAMS][G], s_l[STREAMS][G];

  const lfm3_attention_item item = items[blockIdx.x];
  const int g = blockIdx.y;
  const int row = int(item.row);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub_lane = lane & (LANES - 1), sub = lane / LANES;
  const int stream = wave * SUBS + sub;
  const int d0 = 2 * sub_lane;
  const int stride = kv_heads * D;
  const std::uint32_t cap = capacity[row];
  const Half* ck = cache_k[row] + g * D + d0;
  const Half* cv = cache_v[row] + g * D + d0;
  const float scale = 1.0f / sqrtf(float(D));

  float qv[G][2];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float2 v2 = *reinterpret_cast<const float2*>(
        q + std::size_t(row) * ldq + (g * G + h) * D + d0);
    qv[h][0] = v2.x;
    qv[h][1] = v2.y;
  }
  const int idx = sub_lane >> SH, my_head = idx / KB;
  float m_own = -INFINITY, l_own = 0.0f;
  float acc[G][2];
#pragma unroll
  for (int h = 0; h < G; ++h)
    acc[h][0] = acc[h][1] = 0.0f;

  const int kb = int(item.key_begin), ke = int(item.key_end);
  for (int base = kb + stream * KB; base < ke; base += STREAMS * KB) {
    float k0[KB], k1[KB], v0[KB], v1[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      const int t = min(base + i, ke - 1);
      const std::size_t off = std::size_t(std::uint32_t(t) % cap) * stride;
      const unsigned kw = *reinterpret_cast<const unsigned*>(ck + off);
      const unsigned vw = *reinterpret_cast<const unsigned*>(cv + off);
      k0[i] = HalfBitsToFloat(kw & 0xffffu);
      k1[i] = HalfBitsToFloat(kw >> 16);
      v0[i] = HalfBitsToFloat(vw & 0xffffu);
      v1[i] = HalfBitsToFloat(vw >> 16);
    }
    float vals[N];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < KB; ++i)
        vals[h * KB + i] = fmaf(qv[h][1], k1[i], qv[h][0] * k0[i]);
    // Halving butterfly: after step s a lane carries N >> (s + 1) values.
#pragma unroll
    for (int s = 0; s < LOG_N; ++s) {
      const int mask = LANES >> (s + 1);
      const int half = N >> (s + 1);
      const bool upper = (sub_lane & mask) != 0;
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const float keep = upper ? vals[j + half] : vals[j];
        const float send = upper ? vals[j] : vals[j + half];
        vals[j] = keep + __shfl_xor(send, mask, 64);
      }
    }
    float dot = vals[0];
#pragma unroll
    for (int mask = (1 << SH) >> 1; mask; mask >>= 1)
      dot += __shfl_xor(dot, mask, 64);
    const int key = base + (idx % KB);
    const float score = key < ke ? dot * scale : -INFINITY;
    float top = score;
#pragma unroll
    for (int b = 0; b < LOG_KB; ++b)
      top = fmaxf(top, __shfl_xor(top, (1 << SH) << b, 64));
    const float m_new = fmaxf(m_own, top);
    const float shift = m_new == -INFINITY ? 0.0f : m_new;
    const float p = expf(score - shift);
    const float alpha = expf(m_own - shift);
    float psum = p;
#pragma unroll
    for (int b = 0; b < LOG_KB; ++b)
      psum += __shfl_xor(psum, (1 << SH) << b, 64);
    l_own = l_own * alpha + psum;
    m_own = m_new;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float a_h = SubShfl<LANES>(alpha, (h * KB) << SH);
      float x0 = acc[h][0] * a_h, x1 = acc[h][1] * a_h;
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        const float p_hi = SubShfl<LANES>(p, (h * KB + i) << SH);
        x0 = fmaf(p_hi, v0[i], x0);
        x1 = fmaf(p_hi, v1[i], x1);
      }
      acc[h][0] = x0;
      acc[h][1] = x1;
    }
  }
  // Merge the block's streams.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    s_acc[stream][h][d0] = acc[h][0];
    s_acc[stream][h][d0 + 1] = acc[h][1];
  }
  if ((sub_lane & ((1 << (SH + LOG_KB)) - 1)) == 0) {
    s_m[stream][my_head] = m_own;
    s_l[stream][my_head] = l_own;
  }
  __syncthreads();
  const bool split = item.parts > 1;
  float* part_out = partial + (std::size_t(blockIdx.x) * kv_heads + g) * G * (D + 2);
  for (int e = threadIdx.x; e < G * D; e += kAttnThreads) {
    const int h = e / D, d = e % D;
    float top = -INFINITY;
#pragma unroll
    for (int s = 0; s < STREAMS; ++s)
      top = fmaxf(top, s_m[s][h]);
    float l = 0.0f, a = 0.0f;
#pragma unroll
    for (int s = 0; s < STREAMS; ++s) {
      const float w = s_m[s][h] == -INFINITY ? 0.0f : expf(s_m[s][h] - top);
      l = fmaf(s_l[s][h], w, l);
      a = fmaf(s_acc[s][h][d], w, a);
    }
    const int head = g * G + h;
    if (!split) {
      out[std::size_t(row) * ldo + head * D + d] =
          (a / l) / (1.0f + expf(-gate[std::size_t(row) * ldg + head]));
    } else {
      float* po = part_out + h * (D + 2);
      if (d == 0) {
        po[0] = top;
        po[1] = l;
      }
      po[2 + d] = a;
    }
  }
}

// Merges the spans of every multi-span row in span order: block = (first
// item of a row, KV head); other items exit. A separate launch, so the
// partials of every span are visible without a device-scope fence.
template<int D, int G>
__launch_bounds__(kAttnThreads) __global__
    void CombineKernel(const float* __restrict__ gate, int ldg,
                       const lfm3_attention_item* __restrict__ items,
                       float* __restrict__ out, int ldo, int kv_heads,
                       const float* __restrict__ partial) {
  const lfm3_attention_item item = items[blockIdx.x];
  if (item.parts < 2 || item.first_item != blockIdx.x)
    return;
  const int g = blockIdx.y, row = int(item.row);
  for (int e = threadIdx.x; e < G * D; e += kAttnThreads) {
    const int h = e / D, d = e % D;
    float top = -INFINITY;
    for (std::uint32_t s = 0; s < item.parts; ++s) {
      const float* po = partial +
          ((std::size_t(item.first_item) + s) * kv_heads + g) * G * (D + 2) + h * (D + 2);
      top = fmaxf(top, po[0]);
    }
    float l = 0.0f, a = 0.0f;
    for (std::uint32_t s = 0; s < item.parts; ++s) {
      const float* po = partial +
          ((std::size_t(item.first_item) + s) * kv_heads + g) * G * (D + 2) + h * (D + 2);
      const float w = expf(po[0] - top);
      l = fmaf(po[1], w, l);
      a = fmaf(po[2 + d], w, a);
    }
    const int head = g * G + h;
    out[std::size_t(row) * ldo + head * D + d] =
        (a / l) / (1.0f + expf(-gate[std::size_t(row) * ldg + head]));
  }
}

template<int D, int G>
void LaunchGroup(dim3 grid, hipStream_t s, const float* q, int ldq,
                 const float* gate, int ldg, const Half* const* ck,
                 const Half* const* cv, const std::uint32_t* cap,
                 const lfm3_attention_item* items, float* out, int ldo, int kv,
                 float* partial) {
  DecodeAttentionKernel<D, G><<<grid, kAttnThreads, 0, s>>>(
      q, ldq, gate, ldg, ck, cv, cap, items, out, ldo, kv, partial);
  CombineKernel<D, G><<<grid, kAttnThreads, 0, s>>>(gate, ldg, items, out, ldo,
                                                     kv, partial);
}

template<int D>
int LaunchDim(int group, dim3 grid, hipStream_t s, const float* q, int ldq,
              const float* gate, int ldg, const Half* const* ck,
              const Half* const* cv, const std::uint32_t* cap,
              const lfm3_attention_item* items, float* out, int ldo, int kv,
              float* partial) {
  switch (group) {
    case 2:
      LaunchGroup<D, 2>(grid, s, q, ldq, gate, ldg, ck, cv, cap, items, out, ldo, kv, partial);
      break;
    case 4:
      LaunchGroup<D, 4>(grid, s, q, ldq, gate, ldg, ck, cv, cap, items, out, ldo, kv, partial);
      break;
    default:
      LaunchGroup<D, 8>(grid, s, q, ldq, gate, ldg, ck, cv, cap, items, out, ldo, kv, partial);
      break;
  }
  return HipStatus(hipGetLastError(), "LFM3 decode attention launch");
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

int lfm3_attention_plan(const std::uint32_t* positions, std::uint32_t rows,
                        std::uint32_t window, lfm3_attention_item* items,
                        std::uint32_t max_items) {
  if (!positions || !items)
    return Fail(LFM3_E_INVALID, "invalid LFM3 attention plan");
  std::uint32_t count = 0;
  for (std::uint32_t r = 0; r < rows; ++r) {
    const std::uint32_t p = positions[r];
    const std::uint32_t first = window && p + 1 > window ? p + 1 - window : 0;
    const std::uint32_t keys = p + 1 - first;
    const std::uint32_t parts = (keys + kSpan - 1) / kSpan;
    if (count + parts > max_items)
      return Fail(LFM3_E_INVALID, "LFM3 attention plan exceeds its item list");
    for (std::uint32_t s = 0; s < parts; ++s) {
      lfm3_attention_item& it = items[count + s];
      it.row = r;
      it.key_begin = first + s * kSpan;
      it.key_end = std::min(first + (s + 1) * kSpan, p + 1);
      it.first_item = count;
      it.parts = parts;
      it.reserved[0] = it.reserved[1] = it.reserved[2] = 0;
    }
    count += parts;
  }
  return int(count);
}

std::size_t lfm3_attention_workspace_bytes(std::uint32_t items,
                                           std::uint32_t rows,
                                           std::uint32_t heads,
                                           std::uint32_t kv_heads,
                                           std::uint32_t dim) {
  (void)rows;
  (void)kv_heads;
  return std::size_t(items) * heads * (dim + 2) * sizeof(float);
}

int lfm3_decode_attention_ragged(
    const float* q, std::uint32_t ldq, const float* gate, std::uint32_t ldg,
    const std::uint16_t* const* cache_k, const std::uint16_t* const* cache_v,
    const std::uint32_t* capacity, const lfm3_attention_item* items,
    std::uint32_t n_items, float* out, std::uint32_t ldo, std::uint32_t rows,
    std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
    void* workspace, std::size_t workspace_bytes, void* stream) {
  const std::uint32_t group = kv_heads ? heads / kv_heads : 0;
  if (!q || !gate || !cache_k || !cache_v || !capacity || !items || !out ||
      !rows || !kv_heads || heads % kv_heads ||
      (group != 2 && group != 4 && group != 8) || (dim != 64 && dim != 128) ||
      ldq % 2)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 attention shape");
  if (!n_items)
    return LFM3_OK;
  if (!workspace || workspace_bytes < lfm3_attention_workspace_bytes(
                                          n_items, rows, heads, kv_heads, dim))
    return Fail(LFM3_E_INVALID, "LFM3 attention workspace too small");
  auto* partial = static_cast<float*>(workspace);
  const dim3 grid(n_items, kv_heads);
  const auto s = static_cast<hipStream_t>(stream);
  const auto* ck = reinterpret_cast<const Half* const*>(cache_k);
  const auto* cv = reinterpret_cast<const Half* const*>(cache_v);
  if (dim == 128)
    return LaunchDim<128>(int(group), grid, s, q, int(ldq), gate, int(ldg), ck,
                          cv, capacity, items, out, int(ldo), int(kv_heads),
                          partial);
  return LaunchDim<64>(int(group), grid, s, q, int(ldq), gate, int(ldg), ck, cv,
                       capacity, items, out, int(ldo), int(kv_heads), partial);
}

}  // extern "C"
