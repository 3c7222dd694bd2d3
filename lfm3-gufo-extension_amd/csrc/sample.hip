// Token selection from logits rows on gfx950: greedy, or top-k /
// temperature sampling with a repetition penalty, one block per row.
//
// The serving loop's pick (runner.cpp:300-325, SelectNext) goes through the
// host sampler (sampling::SamplerState::Sample) with the defaults
// temperature 0.1, top_k 50, repeat_penalty 1.1 (runner.cpp:31-35). That
// sampler belongs to the Gufo host, which the reference does not carry, so
// this kernel follows the common definition of each step:
//   1. repetition penalty: the logit l of a token in the row's penalty list
//      becomes l / p when l > 0, else l * p (once per token, however often
//      it is listed; ids >= cols are padding);
//   2. top-k: the k largest logits, ties at the k-th value broken toward
//      the lower index (k == 0 or k >= cols: the whole vocabulary);
//   3. temperature T: weights w = exp((l - l_max) / T) in FP32;
//   4. the pick: target = u * sum(w) for the row's uniform u in [0, 1),
//      then the first candidate whose running weight sum exceeds it, the
//      candidates in descending logit order (lower index first on ties);
//      the whole vocabulary goes in index order.
// T <= 0 or k == 1 is greedy: the first index of the maximum, as
// std::max_element (tests/session_test.cpp:32-34).
//
// Work per row: the logits are read once for the maximum, four times for
// the radix select of the k-th largest key and once to gather the
// candidates, all from L2 (a 65536-entry row is 256 KB); the candidates (at
// most 1024) are sorted in LDS.
#include <cmath>

#include "common.hpp"
#include "internal.hpp"

namespace lfm3amd {
namespace {

constexpr int kThreads = 1024, kWaves = kThreads / 64;

// The float's bits made monotone as unsigned (larger value, larger key).
__device__ __forceinline__ unsigned OrderedBits(float v) {
  const unsigned b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct Row {
  const float* x;
  const unsigned* bits;  // penalty bitmap in LDS, or null
  float penalty;
  __device__ __forceinline__ float operator()(int t) const {
    const float l = x[t];
    if (bits && (bits[t >> 5] >> (t & 31) & 1u))
      return l > 0.0f ? l / penalty : l * penalty;
    return l;
  }
};

// Exclusive prefix over the block of one flag per thread, in thread order;
// returns the thread's offset and writes the block total.
__device__ __forceinline__ unsigned BlockPrefix(bool flag, unsigned* s_wave, unsigned* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned long long m = __ballot(flag);
  const unsigned below = __popcll(m & ((1ull << lane) - 1ull));
  __syncthreads();
  if (lane == 0)
    s_wave[wave] = __popcll(m);
  __syncthreads();
  unsigned before = 0, all = 0;
  for (int w = 0; w < kWaves; ++w) {
    const unsigned c = s_wave[w];
    before += w < wave ? c : 0u;
    all += c;
  }
  *total = all;
  return before + below;
}

__launch_bounds__(kThreads) __global__
    void SampleKernel(const float* __restrict__ logits, int ld, const float* const* row_ptrs,
                      int cols, float temperature, int top_k, float penalty,
                      const std::uint32_t* __restrict__ penalty_ids, int n_penalty,
                      const float* __restrict__ uniforms, std::uint32_t* __restrict__ ids) {
  __shared__ unsigned s_bits[kSampleMaxCols / 32];
  __shared__ unsigned s_hist[256];
  __shared__ float s_val[kSampleMaxTopK];
  __shared__ unsigned s_idx[kSampleMaxTopK];
  __shared__ float s_part[kThreads];
  __shared__ unsigned s_wave[kWaves];
  __shared__ unsigned long long s_key[kWaves];
  __shared__ unsigned s_prefix, s_need;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  Row value{row_ptrs ? row_ptrs[row] : logits + std::size_t(row) * ld, nullptr, penalty};
  if (penalty_ids && n_penalty > 0 && penalty != 1.0f) {
    for (int i = tid; i < (cols + 31) / 32; i += kThreads)
      s_bits[i] = 0u;
    __syncthreads();
    const std::uint32_t* pen = penalty_ids + std::size_t(row) * n_penalty;
    for (int i = tid; i < n_penalty; i += kThreads) {
      const std::uint32_t t = pen[i];
      if (t < std::uint32_t(cols))
        atomicOr(&s_bits[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
    value.bits = s_bits;
  }

  if (!(temperature > 0.0f) || top_k == 1) {
    unsigned long long best = 0;
    for (int t = tid; t < cols; t += kThreads)
      best = max(best, ArgKey(value(t), unsigned(t)));
    for (int m = 1; m < 64; m <<= 1) {
      const unsigned long long o = __shfl_xor(best, m, 64);
      best = o > best ? o : best;
    }
    if (lane == 0)
      s_key[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long b = 0;
      for (int w = 0; w < kWaves; ++w)
        b = max(b, s_key[w]);
      ids[row] = 0xffffffffu - unsigned(b & 0xffffffffu);
    }
    return;
  }

  float top = -INFINITY;
  for (int t = tid; t < cols; t += kThreads)
    top = fmaxf(top, value(t));
  top = WaveMax(top);
  if (lane == 0)
    s_part[wave] = top;
  __syncthreads();
  top = -INFINITY;
  for (int w = 0; w < kWaves; ++w)
    top = fmaxf(top, s_part[w]);
  __syncthreads();
  const float inv_t = 1.0f / temperature;
  const float u = uniforms[row];
  const auto weight = [&](float l) { return expf((l - top) * inv_t); };

  if (top_k <= 0 || top_k >= cols) {
    // Whole vocabulary, index order: thread i owns tokens [i*per, (i+1)*per);
    // the range sums are added in order, and the range that holds the
    // target is walked token by token.
    const int per = (cols + kThreads - 1) / kThreads;
    const int t0 = min(cols, tid * per), t1 = min(cols, t0 + per);
    float own = 0.0f;
    for (int t = t0; t < t1; ++t)
      own += weight(value(t));
    s_part[tid] = own;
    __syncthreads();
    if (tid == 0) {
      float total = 0.0f;
      for (int i = 0; i < kThreads; ++i)
        total += s_part[i];
      const float target = u * total;
      float run = 0.0f;
      int pick = -1, last = -1;
      for (int i = 0; i < kThreads && pick < 0; ++i) {
        if (s_part[i] > 0.0f)
          last = i;
        if (run + s_part[i] > target) {
          const int a = min(cols, i * per), b = min(cols, a + per);
          for (int t = a; t < b && pick < 0; ++t) {
            const float w = weight(value(t));
            run += w;
            if (w > 0.0f && run > target)
              pick = t;
          }
          if (pick < 0)  // rounding between the two sums: the range's last token
            for (int t = b - 1; t >= a && pick < 0; --t)
              if (weight(value(t)) > 0.0f)
                pick = t;
        } else {
          run += s_part[i];
        }
      }
      if (pick < 0 && last >= 0) {  // u * total rounded up to the total
        const int a = min(cols, last * per), b = min(cols, a + per);
        for (int t = b - 1; t >= a && pick < 0; --t)
          if (weight(value(t)) > 0.0f)
            pick = t;
      }
      ids[row] = unsigned(pick < 0 ? 0 : pick);
    }
    return;
  }

  // The k-th largest key, 8 bits a pass. The first pass sees few distinct
  // bins (sign and high exponent bits), so each wave adds its lanes per bin
  // with one atomic; later passes count only keys under the prefix.
  const int k = top_k;
  if (tid == 0) {
    s_prefix = 0u;
    s_need = unsigned(k);
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256)
      s_hist[tid] = 0u;
    __syncthreads();
    const unsigned prefix = s_prefix;
    const unsigned mask = pass ? 0xffffffffu << (32 - 8 * pass) : 0u;
    for (int base = 0; base < cols; base += kThreads) {
      const int t = base + tid;
      unsigned key = 0;
      bool hit = false;
      if (t < cols) {
        key = OrderedBits(value(t));
        hit = (key & mask) == prefix;
      }
      const unsigned bin = (key >> shift) & 255u;
      if (pass == 0) {
        bool left = hit;
        for (;;) {
          const unsigned long long act = __ballot(left);
          if (!act)
            break;
          const int leader = __ffsll(static_cast<long long>(act)) - 1;
          const unsigned lb = __shfl(bin, leader, 64);
          const unsigned long long same = __ballot(left && bin == lb);
          if (lane == leader)
            atomicAdd(&s_hist[lb], unsigned(__popcll(same)));
          if (bin == lb)
            left = false;
        }
      } else if (hit) {
        atomicAdd(&s_hist[bin], 1u);
      }
    }
    __syncthreads();
    if (tid == 0) {
      unsigned need = s_need;
      int b = 255;
      for (; b > 0; --b) {
        if (s_hist[b] >= need)
          break;
        need -= s_hist[b];
      }
      s_prefix = prefix | (unsigned(b) << shift);
      s_need = need;
    }
    __syncthreads();
  }
  const unsigned kth = s_prefix;  // key of the k-th largest logit
  const unsigned ties = s_need;   // keys equal to it that are kept (>= 1)
  // Candidates: every key above kth (k - ties of them), then the `ties`
  // lowest-index keys equal to it; block prefix sums keep index order.
  unsigned above = 0, equal = 0;
  for (int base = 0; base < cols; base += kThreads) {
    const int t = base + tid;
    const float v = t < cols ? value(t) : 0.0f;
    const unsigned key = t < cols ? OrderedBits(v) : 0u;
    const bool is_above = t < cols && key > kth, is_equal = t < cols && key == kth;
    unsigned n_above, n_equal;
    const unsigned a = BlockPrefix(is_above, s_wave, &n_above);
    if (is_above) {
      s_val[above + a] = v;
      s_idx[above + a] = unsigned(t);
    }
    const unsigned e = BlockPrefix(is_equal, s_wave, &n_equal);
    if (is_equal && equal + e < ties) {
      s_val[(unsigned(k) - ties) + equal + e] = v;
      s_idx[(unsigned(k) - ties) + equal + e] = unsigned(t);
    }
    above += n_above;
    equal += n_equal;
  }
  __syncthreads();
  // Bitonic sort of the k candidates: value descending, index ascending.
  int size = 1;
  while (size < k)
    size <<= 1;
  for (int i = k + tid; i < size; i += kThreads) {
    s_val[i] = -INFINITY;
    s_idx[i] = 0xffffffffu;
  }
  __syncthreads();
  const auto before = [&](int a, int b) {
    return s_val[a] > s_val[b] || (s_val[a] == s_val[b] && s_idx[a] < s_idx[b]);
  };
  for (int len = 2; len <= size; len <<= 1)
    for (int stride = len >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < size; i += kThreads) {
        const int j = i ^ stride;
        if (j > i && ((i & len) == 0 ? before(j, i) : before(i, j))) {
          const float tv = s_val[i];
          s_val[i] = s_val[j];
          s_val[j] = tv;
          const unsigned ti = s_idx[i];
          s_idx[i] = s_idx[j];
          s_idx[j] = ti;
        }
      }
      __syncthreads();
    }
  if (tid == 0) {
    float total = 0.0f;
    for (int i = 0; i < k; ++i)
      total += weight(s_val[i]);
    const float target = u * total;
    float run = 0.0f;
    int pick = 0;
    for (int i = 0; i < k; ++i) {
      const float w = weight(s_val[i]);
      if (w > 0.0f)
        pick = i;  // the last candidate with weight, should the sums round
      run += w;
      if (w > 0.0f && run > target)
        break;
    }
    ids[row] = s_idx[pick];
  }
}

}  // namespace

int CheckSample(const lfm3_sampling& p, std::uint32_t cols, std::uint32_t n_penalty,
                bool have_penalty, bool have_uniforms) {
  if (!cols || cols > kSampleMaxCols || n_penalty > kSampleMaxPenalty ||
      (n_penalty && !have_penalty) || !(p.repeat_penalty > 0.0f) ||
      !std::isfinite(p.repeat_penalty) || p.top_k > kSampleMaxTopK ||
      std::isnan(p.temperature) || (p.temperature > 0.0f && p.top_k != 1 && !have_uniforms))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 sampling parameters");
  return LFM3_OK;
}

int LaunchSample(const float* logits, std::uint32_t ld, const float* const* row_ptrs,
                 std::uint32_t rows, std::uint32_t cols, const lfm3_sampling& p,
                 const std::uint32_t* penalty_ids, std::uint32_t n_penalty,
                 const float* uniforms, std::uint32_t* ids, hipStream_t stream) {
  if (const int e = CheckSample(p, cols, n_penalty, penalty_ids != nullptr, uniforms != nullptr))
    return e;
  if ((!logits && !row_ptrs) || !ids || !rows || (logits && ld < cols))
    return Fail(LFM3_E_INVALID, "invalid LFM3 sampling shape");
  SampleKernel<<<rows, kThreads, 0, stream>>>(logits, int(ld), row_ptrs, int(cols),
                                              p.temperature, int(p.top_k), p.repeat_penalty,
                                              penalty_ids, int(n_penalty), uniforms, ids);
  return HipStatus(hipGetLastError(), "LFM3 sampling launch");
}

}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" int lfm3_sample(const float* logits, std::uint32_t rows, std::uint32_t cols,
                           std::uint32_t ld, const lfm3_sampling* params,
                           const std::uint32_t* penalty_ids, std::uint32_t n_penalty,
                           const float* uniforms, std::uint32_t* ids, void* stream) {
  if (!params)
    return Fail(LFM3_E_INVALID, "null LFM3 sampling parameters");
  return LaunchSample(logits, ld, nullptr, rows, cols, *params, penalty_ids, n_penalty,
                      uniforms, ids, static_cast<hipStream_t>(stream));
}
