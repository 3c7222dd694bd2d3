// Token selection from logits rows on gfx950: greedy, or top-k /
// temperature sampling with a repetition penalty.
//
// The serving loop's pick (runner.cpp:300-325, SelectNext) goes through the
// host sampler (sampling::SamplerState::Sample) with the defaults
// temperature 0.1, top_k 50, repeat_penalty 1.1 (runner.cpp:31-35). That
// sampler belongs to the Gufo host, which the reference does not carry, so
// this code follows the common definition of each step:
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
// Two launches. The first splits every row into slices of 4096 logits, one
// block each, so a batch of 8 rows of 128000 fills 256 CUs: the slice is
// read from HBM once into LDS (penalized there) and reduced to its best
// greedy key, its (max, weight sum), or its own top-k candidates in index
// order (keys above its k-th, then its lowest-index ties). The global top-k
// is among the slices' candidates, in global index order wherever keys tie.
// The second launch, one block per row, selects the k-th key among the
// candidates by radix select, sorts the k winners in LDS and picks; for
// the whole vocabulary it finds the slice that holds the target from the
// slices' sums and walks that slice's weights in index order.
#include <cmath>

#include "common.hpp"
#include "internal.hpp"

namespace lfm3amd {
namespace {

constexpr int kSliceLen = 4096, kSliceThreads = 256, kPickThreads = 1024;
constexpr unsigned kPadIndex = 0xffffffffu;

enum Mode { kGreedy = 0, kWhole = 1, kTopK = 2 };

int Slices(std::uint32_t cols) { return int((cols + kSliceLen - 1) / kSliceLen); }

int ModeOf(const lfm3_sampling& p, std::uint32_t cols) {
  if (!(p.temperature > 0.0f) || p.top_k == 1)
    return kGreedy;
  return p.top_k == 0 || p.top_k >= cols ? kWhole : kTopK;
}

// Workspace: per (row, slice) 16 bytes of statistics, then with top-k the
// slices' candidate values and indices (top_k each).
struct Layout {
  std::size_t stats = 0, values = 0, indices = 0, bytes = 0;
};
Layout LayoutOf(std::uint32_t rows, std::uint32_t cols, std::uint32_t cap) {
  const auto al = [](std::size_t n) { return (n + 255) / 256 * 256; };
  const std::size_t units = std::size_t(rows) * Slices(cols);
  Layout l;
  l.values = al(units * 16);
  l.indices = l.values + al(units * cap * 4);
  l.bytes = l.indices + al(units * cap * 4);
  return l;
}

// The float's bits made monotone as unsigned (larger value, larger key).
__device__ __forceinline__ unsigned OrderedBits(float v) {
  const unsigned b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float Penalized(float l, float p) { return l > 0.0f ? l / p : l * p; }

// Exclusive prefix over the block of one count per thread, in thread order;
// returns the thread's offset and writes the block total.
template<int kThreads>
__device__ __forceinline__ unsigned BlockScan(unsigned count, unsigned* s_wave, unsigned* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned incl = count;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned v = __shfl_up(incl, off, 64);
    if (lane >= off)
      incl += v;
  }
  __syncthreads();
  if (lane == 63)
    s_wave[wave] = incl;
  __syncthreads();
  unsigned before = 0, all = 0;
  for (int w = 0; w < kThreads / 64; ++w) {
    const unsigned c = s_wave[w];
    before += w < wave ? c : 0u;
    all += c;
  }
  *total = all;
  return before + incl - count;
}

// Counts packed for one scan: keys above the k-th (fewer than k <= 1024)
// in bits 20 and up, keys equal to it (at most 2^17) below.
constexpr int kUpShift = 20;
constexpr unsigned kEqMask = (1u << kUpShift) - 1u;

// Radix select over n keys key(i): the key of the k-th largest and how many
// keys equal to it are kept (the rest of the k are above it). Four passes
// of 8 bits; wave 0 finds each pass's bin from suffix sums of the
// histogram, 4 bins a lane.
template<int kThreads, class Key>
__device__ void SelectKth(int n, unsigned k, Key key, unsigned* s_hist, unsigned* s_sel,
                          unsigned& kth, unsigned& ties) {
  const int tid = threadIdx.x, lane = tid & 63;
  unsigned prefix = 0, need = k;
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    const unsigned mask = pass ? 0xffffffffu << (32 - 8 * pass) : 0u;
    for (int i = tid; i < 256; i += kThreads)
      s_hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
      const unsigned kv = key(i);
      if ((kv & mask) == prefix)
        atomicAdd(&s_hist[(kv >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      const unsigned h0 = s_hist[4 * lane], h1 = s_hist[4 * lane + 1];
      const unsigned h2 = s_hist[4 * lane + 2], h3 = s_hist[4 * lane + 3];
      const unsigned own = h0 + h1 + h2 + h3;
      unsigned incl = own;  // bins of this lane and every lane above it
      for (int off = 1; off < 64; off <<= 1) {
        const unsigned v = __shfl_down(incl, off, 64);
        if (lane + off < 64)
          incl += v;
      }
      unsigned above = incl - own;
      const unsigned h[4] = {h0, h1, h2, h3};
      for (int j = 3; j >= 0; --j) {
        if (above < need && need <= above + h[j]) {
          s_sel[0] = prefix | (unsigned(4 * lane + j) << shift);
          s_sel[1] = need - above;
        }
        above += h[j];
      }
    }
    __syncthreads();
    prefix = s_sel[0];
    need = s_sel[1];
    __syncthreads();
  }
  kth = prefix;
  ties = need;
}

__device__ __forceinline__ unsigned long long KeyMax(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

template<int kThreads>
__device__ unsigned long long BlockKeyMax(unsigned long long v, unsigned long long* s_key) {
  for (int m = 1; m < 64; m <<= 1)
    v = KeyMax(v, __shfl_xor(v, m, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    s_key[threadIdx.x >> 6] = v;
  __syncthreads();
  unsigned long long b = 0;
  for (int w = 0; w < kThreads / 64; ++w)
    b = KeyMax(b, s_key[w]);
  return b;
}

template<int kThreads>
__device__ float BlockMax(float v, float* s_f) {
  v = WaveMax(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    s_f[threadIdx.x >> 6] = v;
  __syncthreads();
  float b = -INFINITY;
  for (int w = 0; w < kThreads / 64; ++w)
    b = fmaxf(b, s_f[w]);
  return b;
}

template<int kThreads>
__device__ float BlockSum(float v, float* s_f) {
  v = WaveSum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
    s_f[threadIdx.x >> 6] = v;
  __syncthreads();
  float b = 0.0f;
  for (int w = 0; w < kThreads / 64; ++w)
    b += s_f[w];
  return b;
}

struct SliceArgs {
  const float* logits;
  int ld;
  const float* const* row_ptrs;
  int cols, mode, k;
  float inv_t, penalty;
  const std::uint32_t* penalty_ids;
  int n_penalty;
  std::uint8_t* ws;
  Layout layout;
};

// One slice of one row (blockIdx.x, blockIdx.y).
__launch_bounds__(kSliceThreads) __global__ void SliceKernel(SliceArgs a) {
  __shared__ __attribute__((aligned(16))) float s_v[kSliceLen];
  __shared__ unsigned s_bits[kSliceLen / 32];
  __shared__ unsigned s_hist[256];
  __shared__ unsigned s_sel[2];
  __shared__ unsigned s_wave[kSliceThreads / 64];
  __shared__ float s_f[kSliceThreads / 64];
  __shared__ unsigned long long s_key[kSliceThreads / 64];
  const int tid = threadIdx.x, row = blockIdx.y, slice = blockIdx.x;
  const int slices = gridDim.x;
  const int begin = slice * kSliceLen, len = min(kSliceLen, a.cols - begin);
  const float* x = (a.row_ptrs ? a.row_ptrs[row] : a.logits + std::size_t(row) * a.ld) + begin;
  const bool penalize = a.penalty_ids && a.n_penalty > 0 && a.penalty != 1.0f;
  if (penalize) {
    for (int i = tid; i < kSliceLen / 32; i += kSliceThreads)
      s_bits[i] = 0u;
    __syncthreads();
    const std::uint32_t* pen = a.penalty_ids + std::size_t(row) * a.n_penalty;
    for (int i = tid; i < a.n_penalty; i += kSliceThreads) {
      const std::uint32_t t = pen[i] - std::uint32_t(begin);
      if (pen[i] >= std::uint32_t(begin) && t < std::uint32_t(len))
        atomicOr(&s_bits[t >> 5], 1u << (t & 31));
    }
    __syncthreads();
  }
  for (int i = tid; i < len; i += kSliceThreads) {
    float l = x[i];
    if (penalize && (s_bits[i >> 5] >> (i & 31) & 1u))
      l = Penalized(l, a.penalty);
    s_v[i] = l;
  }
  __syncthreads();
  const std::size_t unit = std::size_t(row) * slices + slice;
  auto* stats = reinterpret_cast<float*>(a.ws + a.layout.stats) + unit * 4;

  if (a.mode == kGreedy) {
    unsigned long long best = 0;
    for (int i = tid; i < len; i += kSliceThreads)
      best = KeyMax(best, ArgKey(s_v[i], unsigned(begin + i)));
    best = BlockKeyMax<kSliceThreads>(best, s_key);
    if (tid == 0)
      *reinterpret_cast<unsigned long long*>(stats) = best;
    return;
  }
  if (a.mode == kWhole) {
    float m = -INFINITY;
    for (int i = tid; i < len; i += kSliceThreads)
      m = fmaxf(m, s_v[i]);
    m = BlockMax<kSliceThreads>(m, s_f);
    float z = 0.0f;
    for (int i = tid; i < len; i += kSliceThreads)
      z += expf((s_v[i] - m) * a.inv_t);
    z = BlockSum<kSliceThreads>(z, s_f);
    if (tid == 0) {
      stats[0] = m;
      stats[1] = z;
    }
    return;
  }

  // Top-k: this slice's k best in index order (keys above its k-th, then
  // its lowest-index ties), padded when the slice is shorter than k.
  const int k = a.k;
  float* out_v = reinterpret_cast<float*>(a.ws + a.layout.values) + unit * k;
  unsigned* out_i = reinterpret_cast<unsigned*>(a.ws + a.layout.indices) + unit * k;
  if (len <= k) {
    for (int i = tid; i < k; i += kSliceThreads) {
      out_v[i] = i < len ? s_v[i] : __uint_as_float(0xffffffffu);  // pad key 0
      out_i[i] = i < len ? unsigned(begin + i) : kPadIndex;
    }
    return;
  }
  unsigned kth, ties;
  SelectKth<kSliceThreads>(len, unsigned(k), [&](int i) { return OrderedBits(s_v[i]); },
                           s_hist, s_sel, kth, ties);
  // Thread t owns the kOwn consecutive elements from kOwn t: it counts its
  // keys above the k-th and equal to it, one block scan of the packed
  // counts gives its output offsets, and it writes its winners in index
  // order (the lowest-index ties first).
  constexpr int kOwn = kSliceLen / kSliceThreads;
  float vals[kOwn];
#pragma unroll
  for (int q = 0; q < kOwn / 4; ++q) {
    const float4 f = *reinterpret_cast<const float4*>(&s_v[tid * kOwn + 4 * q]);
    vals[4 * q] = f.x;
    vals[4 * q + 1] = f.y;
    vals[4 * q + 2] = f.z;
    vals[4 * q + 3] = f.w;
  }
  unsigned counts = 0;
#pragma unroll
  for (int j = 0; j < kOwn; ++j) {
    const unsigned key = OrderedBits(vals[j]);
    const bool live = tid * kOwn + j < len;
    counts += live && key > kth ? (1u << kUpShift) : live && key == kth ? 1u : 0u;
  }
  unsigned total;
  const unsigned at = BlockScan<kSliceThreads>(counts, s_wave, &total);
  unsigned up = at >> kUpShift, eq = at & kEqMask;
#pragma unroll
  for (int j = 0; j < kOwn; ++j) {
    const int i = tid * kOwn + j;
    const unsigned key = OrderedBits(vals[j]);
    if (i >= len)
      continue;
    if (key > kth) {
      out_v[up] = vals[j];
      out_i[up] = unsigned(begin + i);
      ++up;
    } else if (key == kth) {
      if (eq < ties) {
        out_v[unsigned(k) - ties + eq] = vals[j];
        out_i[unsigned(k) - ties + eq] = unsigned(begin + i);
      }
      ++eq;
    }
  }
}

struct PickArgs {
  const float* logits;
  int ld;
  const float* const* row_ptrs;
  int cols, mode, k, slices;
  float inv_t, penalty;
  const std::uint32_t* penalty_ids;
  int n_penalty;
  const float* uniforms;
  const std::uint8_t* ws;
  Layout layout;
  std::uint32_t* ids;
};

// One row: the pick from the slices' results.
__launch_bounds__(kPickThreads) __global__ void PickKernel(PickArgs a) {
  __shared__ float s_val[kSampleMaxTopK];
  __shared__ unsigned s_idx[kSampleMaxTopK];
  __shared__ unsigned s_hist[256];
  __shared__ unsigned s_sel[2];
  __shared__ unsigned s_wave[kPickThreads / 64];
  __shared__ float s_f[kPickThreads / 64];
  __shared__ unsigned long long s_key[kPickThreads / 64];
  __shared__ unsigned s_bits[kSliceLen / 32];
  __shared__ int s_slice, s_pick, s_last;
  __shared__ float s_target, s_top;
  const int tid = threadIdx.x, row = blockIdx.x;
  const float* stats = reinterpret_cast<const float*>(a.ws + a.layout.stats) +
                       std::size_t(row) * a.slices * 4;

  if (a.mode == kGreedy) {
    unsigned long long best = 0;
    for (int s = tid; s < a.slices; s += kPickThreads)
      best = KeyMax(best, *reinterpret_cast<const unsigned long long*>(stats + 4 * s));
    best = BlockKeyMax<kPickThreads>(best, s_key);
    if (tid == 0)
      a.ids[row] = 0xffffffffu - unsigned(best & 0xffffffffu);
    return;
  }
  const float u = a.uniforms[row];

  if (a.mode == kWhole) {
    // Slice sums rescaled to the row's maximum, added in slice order; the
    // slice whose running sum passes u * total is walked element by element.
    __shared__ float s_m[kSampleMaxCols / kSliceLen], s_z[kSampleMaxCols / kSliceLen];
    for (int s = tid; s < a.slices; s += kPickThreads) {
      s_m[s] = stats[4 * s];
      s_z[s] = stats[4 * s + 1];
    }
    __syncthreads();
    if (tid == 0) {
      float top = -INFINITY;
      for (int s = 0; s < a.slices; ++s)
        top = fmaxf(top, s_m[s]);
      float total = 0.0f;
      for (int s = 0; s < a.slices; ++s)
        total += s_z[s] * expf((s_m[s] - top) * a.inv_t);
      const float target = u * total;
      float run = 0.0f;
      int pick = -1, last = 0;
      for (int s = 0; s < a.slices; ++s) {
        const float z = s_z[s] * expf((s_m[s] - top) * a.inv_t);
        if (z > 0.0f)
          last = s;
        if (pick < 0 && run + z > target) {
          pick = s;
          break;
        }
        run += z;
      }
      if (pick < 0)
        pick = last;  // u * total rounded up to the total
      s_slice = pick;
      s_target = target - run;
      s_top = top;
      s_pick = 0x7fffffff;
      s_last = -1;
    }
    __syncthreads();
    const int slice = s_slice, begin = slice * kSliceLen;
    const int len = min(kSliceLen, a.cols - begin);
    const float top = s_top, target = s_target;
    const float* x = (a.row_ptrs ? a.row_ptrs[row] : a.logits + std::size_t(row) * a.ld) + begin;
    const bool penalize = a.penalty_ids && a.n_penalty > 0 && a.penalty != 1.0f;
    if (penalize) {
      for (int i = tid; i < kSliceLen / 32; i += kPickThreads)
        s_bits[i] = 0u;
      __syncthreads();
      const std::uint32_t* pen = a.penalty_ids + std::size_t(row) * a.n_penalty;
      for (int i = tid; i < a.n_penalty; i += kPickThreads) {
        const std::uint32_t t = pen[i] - std::uint32_t(begin);
        if (pen[i] >= std::uint32_t(begin) && t < std::uint32_t(len))
          atomicOr(&s_bits[t >> 5], 1u << (t & 31));
      }
      __syncthreads();
    }
    // Thread t owns elements 4t..4t+3 (a slice has at most 4096).
    float w[4];
    float own = 0.0f;
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * tid + j;
      float l = i < len ? x[i] : -INFINITY;
      if (i < len && penalize && (s_bits[i >> 5] >> (i & 31) & 1u))
        l = Penalized(l, a.penalty);
      w[j] = i < len ? expf((l - top) * a.inv_t) : 0.0f;
      own += w[j];
    }
    // Exclusive prefix of the threads' sums in thread order: wave scans,
    // then the waves' totals in order.
    const int lane = tid & 63, wave = tid >> 6;
    float incl = own;
    for (int off = 1; off < 64; off <<= 1) {
      const float v = __shfl_up(incl, off, 64);
      if (lane >= off)
        incl += v;
    }
    if (lane == 63)
      s_f[wave] = incl;
    __syncthreads();
    float before = incl - own;
    for (int v = 0; v < wave; ++v)
      before += s_f[v];
    float run = before;
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * tid + j;
      if (w[j] > 0.0f) {
        atomicMax(&s_last, i);
        if (run + w[j] > target)
          atomicMin(&s_pick, i);
      }
      run += w[j];
    }
    __syncthreads();
    if (tid == 0) {
      const int i = s_pick != 0x7fffffff ? s_pick : max(s_last, 0);
      a.ids[row] = unsigned(begin + i);
    }
    return;
  }

  // Top-k among the slices' candidates (global index order where keys tie).
  const int k = a.k, n = a.slices * k;
  const float* cv = reinterpret_cast<const float*>(a.ws + a.layout.values) +
                    std::size_t(row) * a.slices * k;
  const unsigned* ci = reinterpret_cast<const unsigned*>(a.ws + a.layout.indices) +
                       std::size_t(row) * a.slices * k;
  // The candidates' keys are read from the workspace once into LDS when
  // they fit, so the select's passes and the compaction read LDS.
  constexpr int kStagedKeys = 8192;
  __shared__ unsigned s_cand[kStagedKeys];
  const bool staged = n <= kStagedKeys;
  if (staged) {
    for (int i = tid; i < n; i += kPickThreads)
      s_cand[i] = OrderedBits(cv[i]);
    __syncthreads();
  }
  const auto key_of = [&](int i) { return staged ? s_cand[i] : OrderedBits(cv[i]); };
  unsigned kth, ties;
  SelectKth<kPickThreads>(n, unsigned(k), key_of, s_hist, s_sel, kth, ties);
  // Thread t owns `per` consecutive candidates (the slices' candidates in
  // slice order, so in global index order where keys tie): counts, one
  // block scan, then the winners in order.
  const int per = (n + kPickThreads - 1) / kPickThreads, i0 = tid * per;
  unsigned counts = 0;
  for (int j = 0; j < per; ++j) {
    const int i = i0 + j;
    if (i < n) {
      const unsigned key = key_of(i);
      counts += key > kth ? (1u << kUpShift) : key == kth ? 1u : 0u;
    }
  }
  unsigned total;
  const unsigned at = BlockScan<kPickThreads>(counts, s_wave, &total);
  unsigned up = at >> kUpShift, eq = at & kEqMask;
  for (int j = 0; j < per; ++j) {
    const int i = i0 + j;
    if (i >= n)
      break;
    const unsigned key = key_of(i);
    if (key > kth) {
      s_val[up] = cv[i];
      s_idx[up] = ci[i];
      ++up;
    } else if (key == kth) {
      if (eq < ties) {
        s_val[unsigned(k) - ties + eq] = cv[i];
        s_idx[unsigned(k) - ties + eq] = ci[i];
      }
      ++eq;
    }
  }
  __syncthreads();
  // Bitonic sort of the k winners: value descending, index ascending. Up to
  // 64 winners sort in one wave's registers (lane p holds position p;
  // exchanges by lane shuffles, no barriers); more sort in LDS.
  int size = 1;
  while (size < k)
    size <<= 1;
  if (size <= 64) {
    if (tid < 64) {
      float v = tid < k ? s_val[tid] : -INFINITY;
      unsigned ix = tid < k ? s_idx[tid] : kPadIndex;
      for (int len = 2; len <= 64; len <<= 1)
        for (int stride = len >> 1; stride > 0; stride >>= 1) {
          const float ov = __shfl_xor(v, stride, 64);
          const unsigned oi = unsigned(__shfl_xor(int(ix), stride, 64));
          // The lower lane of a pair keeps the first of the two in an
          // ascending run ((p & len) == 0), the upper lane in a descending one.
          const bool wants_first = ((tid & stride) == 0) == ((tid & len) == 0);
          const bool mine_first = v > ov || (v == ov && ix < oi);
          if (wants_first != mine_first) {
            v = ov;
            ix = oi;
          }
        }
      if (tid < k) {
        s_val[tid] = v;
        s_idx[tid] = ix;
      }
    }
    __syncthreads();
  } else {
    for (int i = k + tid; i < size; i += kPickThreads) {
      s_val[i] = -INFINITY;
      s_idx[i] = kPadIndex;
    }
    __syncthreads();
    const auto first = [&](int p, int q) {
      return s_val[p] > s_val[q] || (s_val[p] == s_val[q] && s_idx[p] < s_idx[q]);
    };
    for (int len = 2; len <= size; len <<= 1)
      for (int stride = len >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < size; i += kPickThreads) {
          const int j = i ^ stride;
          if (j > i && ((i & len) == 0 ? first(j, i) : first(i, j))) {
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
  }
  // The weights in parallel (the sorted maximum first), then the running
  // sums in candidate order on one thread.
  __shared__ float s_w[kSampleMaxTopK];
  const float top = s_val[0];
  for (int i = tid; i < k; i += kPickThreads)
    s_w[i] = expf((s_val[i] - top) * a.inv_t);
  __syncthreads();
  if (tid == 0) {
    float total = 0.0f;
    for (int i = 0; i < k; ++i)
      total += s_w[i];
    const float target = u * total;
    float run = 0.0f;
    int pick = 0;
    for (int i = 0; i < k; ++i) {
      const float w = s_w[i];
      if (w > 0.0f)
        pick = i;  // the last candidate with weight, should the sums round
      run += w;
      if (w > 0.0f && run > target)
        break;
    }
    a.ids[row] = s_idx[pick];
  }
}

}  // namespace

std::size_t SampleWorkspaceBytes(std::uint32_t rows, std::uint32_t cols, std::uint32_t top_k) {
  const bool topk = top_k > 1 && top_k < cols;
  return LayoutOf(rows, cols, topk ? top_k : 0).bytes;
}

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
                 const float* uniforms, std::uint32_t* ids, void* workspace,
                 std::size_t workspace_bytes, hipStream_t stream) {
  if (const int e = CheckSample(p, cols, n_penalty, penalty_ids != nullptr, uniforms != nullptr))
    return e;
  if ((!logits && !row_ptrs) || !ids || !rows || rows > 65535 || (logits && ld < cols) ||
      !workspace ||
      workspace_bytes < SampleWorkspaceBytes(rows, cols, p.top_k))
    return Fail(LFM3_E_INVALID, "invalid LFM3 sampling shape or workspace");
  const int mode = ModeOf(p, cols);
  const Layout layout = LayoutOf(rows, cols, mode == kTopK ? p.top_k : 0);
  const float inv_t = mode == kGreedy ? 0.0f : 1.0f / p.temperature;
  SliceArgs sa{logits, int(ld), row_ptrs, int(cols), mode, int(p.top_k), inv_t,
               p.repeat_penalty, penalty_ids, int(n_penalty),
               static_cast<std::uint8_t*>(workspace), layout};
  SliceKernel<<<dim3(Slices(cols), rows), kSliceThreads, 0, stream>>>(sa);
  PickArgs pa{logits, int(ld), row_ptrs, int(cols), mode, int(p.top_k), Slices(cols), inv_t,
              p.repeat_penalty, penalty_ids, int(n_penalty), uniforms,
              static_cast<const std::uint8_t*>(workspace), layout, ids};
  PickKernel<<<rows, kPickThreads, 0, stream>>>(pa);
  return HipStatus(hipGetLastError(), "LFM3 sampling launch");
}

}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" size_t lfm3_sample_workspace_bytes(uint32_t rows, uint32_t cols, uint32_t top_k) {
  return SampleWorkspaceBytes(rows, cols, top_k);
}

extern "C" int lfm3_sample(const float* logits, std::uint32_t rows, std::uint32_t cols,
                           std::uint32_t ld, const lfm3_sampling* params,
                           const std::uint32_t* penalty_ids, std::uint32_t n_penalty,
                           const float* uniforms, std::uint32_t* ids, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (!params)
    return Fail(LFM3_E_INVALID, "null LFM3 sampling parameters");
  return LaunchSample(logits, ld, nullptr, rows, cols, *params, penalty_ids, n_penalty,
                      uniforms, ids, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
}
