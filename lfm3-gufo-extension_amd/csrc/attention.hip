// Ragged decode attention on gfx950: one launch covers every session of a
// decode round. A work item is (row, key span); blockIdx.y is the KV head.
// Keys come from the row's own F16 ring (slot t % capacity), sliding
// layers reading only the last `window` positions (the item list encodes
// the window), as in the reference decode (hip/ops.hip:1578-1691;
// reference.cpp:109-144).
//
// Block = 4 waves (8 when every row is one item); wave w takes the 16-key
// groups w, w + 4, ... of its span.
// Scores S = Q K^T run on MFMA (v_mfma_f32_16x16x32_f16): the A operand
// holds each query head as an fp16 hi row and an fp16 lo row (hi + lo 2^-11
// keeps about 22 bits of the FP32 query; every half x half product is
// exact in FP32), the B operand is 16 keys' F16 rows read with one 16-byte
// load per lane per 32 dimensions. The softmax runs in (head, key) lanes
// with FP32 online maxima and sums; P V runs on the VALU, a lane owning
// eight dimensions of a quarter of the group's keys (one 16-byte V load per
// key), with the probabilities broadcast through LDS. The next group's K
// and V loads are issued before the current group is computed. Waves merge
// through LDS; rows with several spans leave per-span (max, sum, acc)
// partials, and the last span block of a (row, KV head) to arrive merges
// them in span order, so results do not depend on block scheduling. The
// partials go out as agent-scope stores (written through the XCD's L2),
// each thread waits for its stores, and one agent-scope atomic per block
// counts the arrivals; the block that brings the count to the row's span
// count resets it to zero and reads every span's partials with
// agent-scope loads. No device-scope fence is needed.
//
// With the heads fused in (lfm3_decode_heads_attention_ragged), every block
// also applies the per-head Q/K RMSNorm and paired RoPE of its row
// (hip/ops.hip:1072-1134) in its prologue. Each wave's first K/V group is
// issued right after the prologue's own loads, so it arrives while the
// norms and rotations compute. Exactly one block of a row writes the
// ring: the one whose span ends at the current position. It stores the
// row's F16 K/V to slot position % capacity for later rounds and takes
// that key from LDS for this one (the ring loads skip it, and the group
// holding it selects the LDS row in its place), so nothing waits for the
// store. No other span of the row covers the current position, so no
// other block reads the slot being written; on a sliding layer this
// relies on the ring holding at least the window (capacity = min(context,
// window) >= keys of any span), so the current slot is not an earlier key
// of another span.
//
// A row with several spans needs the merge. The 8-wave whole-row path runs
// only when the item count equals the row count (every row one item); an
// item with parts > 1 on that path (an item list that is not a plan over
// exactly `rows` rows) writes NaN to its row's outputs, so the misuse shows
// instead of leaving stale rows.
//
// Workspace: kCounterBytes of arrival counters (one per (first item, KV
// head); zero before the first call, and every call leaves them zero),
// then the span partials.
#include <algorithm>
#include <array>
#include <cmath>
#include <mutex>

#include "common.hpp"

namespace lfm3amd {

// Span partials of lfm3_decode_heads_attention_ragged_noalloc: a
// file-scope device array (one copy per GPU, held until the process ends)
// in place of a caller workspace. Host code reaches it only through the
// address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) float scratch[LFM3_ATTENTION_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kAttnThreads = 256, kAttnWaves = 4, kGroupKeys = 16, kWholeRowWaves = 8;
constexpr std::uint32_t kTargetItems = 128, kMinSpan = 64, kMaxSpan = 1024;
constexpr std::uint32_t kMaxParts = 256;
constexpr std::size_t kCounterBytes = 64 << 10;

__device__ __forceinline__ void AgentStore(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float AgentLoad(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The merge of a multi-span row's partials in span order (the last span
// block of (row, KV head g) runs it): span maxima, weights and
// denominators staged in LDS, then every output element sums its spans.
template<int D, int G, int T>
__device__ void MergeSpans(const lfm3_attention_item& item, int g, int kv_heads,
                           const float* partial, const float* s_gate, float* out, int ldo,
                           float (*s_w)[G], float (*s_lv)[G], float* s_top, float* s_den) {
  const int row = int(item.row), parts = int(item.parts), tid = threadIdx.x;
  const std::size_t span_stride = std::size_t(kv_heads) * G * (D + 2);
  const float* base = partial + (std::size_t(item.first_item) * kv_heads + g) * G * (D + 2);
  for (int e = tid; e < parts * G; e += T) {
    const int s = e / G, h = e % G;
    const float* po = base + s * span_stride + h * (D + 2);
    s_w[s][h] = AgentLoad(po);
    s_lv[s][h] = AgentLoad(po + 1);
  }
  __syncthreads();
  if (tid < G) {
    float top = -INFINITY;
    for (int s = 0; s < parts; ++s)
      top = fmaxf(top, s_w[s][tid]);
    s_top[tid] = top;
  }
  __syncthreads();
  for (int e = tid; e < parts * G; e += T) {
    const int s = e / G, h = e % G;
    s_w[s][h] = expf(s_w[s][h] - s_top[h]);
  }
  __syncthreads();
  if (tid < G) {
    float den = 0.0f;
    for (int s = 0; s < parts; ++s)
      den = fmaf(s_lv[s][tid], s_w[s][tid], den);
    s_den[tid] = den;
  }
  __syncthreads();
  // Every element's sum first, then the stores. The loads of kBatch spans
  // of every element a thread owns go out together (one memory round trip
  // a batch); the sums then run in span order. A batch's loads past the
  // last span repeat the last one and are not added.
  constexpr int EPT = (G * D + T - 1) / T, kBatch = 16;
  float av[EPT];
  const float* po[EPT];
  int hh[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = tid + T * j < G * D ? tid + T * j : 0;
    hh[j] = e / D;
    po[j] = base + hh[j] * (D + 2) + 2 + e % D;
    av[j] = 0.0f;
  }
  for (int s0 = 0; s0 < parts; s0 += kBatch) {
    float v[kBatch][EPT];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int s = min(s0 + b, parts - 1);
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        v[b][j] = AgentLoad(po[j] + s * span_stride);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
      if (s0 + b < parts)
#pragma unroll
        for (int j = 0; j < EPT; ++j)
          av[j] = fmaf(v[b][j], s_w[s0 + b][hh[j]], av[j]);
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = tid + T * j;
    if (e < G * D) {
      const int h = e / D, d = e % D;
      out[std::size_t(row) * ldo + (g * G + h) * D + d] = (av[j] / s_den[h]) / s_gate[h];
    }
  }
}

// Orders this wave's LDS writes before its later LDS reads by other lanes.
// The hardware keeps a wave's LDS operations in order; the fence stops the
// compiler from moving a store past a load that no single lane aliases
// (lanes here read rows other lanes wrote).
__device__ __forceinline__ void WaveSync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ int ngroups_of(int kb, int ke) {
  return (ke - kb + kGroupKeys - 1) / kGroupKeys;
}

template<int D, int G, bool kFused, int NW>
__launch_bounds__(NW * 64) __global__ void DecodeAttentionKernel(
    const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int ld, const float* __restrict__ gate,
    int ldg, const float* __restrict__ q_norm,
    const float* __restrict__ k_norm, const float* __restrict__ frequencies,
    const float* __restrict__ factors, Half* const* __restrict__ cache_k,
    Half* const* __restrict__ cache_v,
    const std::uint32_t* __restrict__ positions,
    const std::uint32_t* __restrict__ capacity,
    const lfm3_attention_item* __restrict__ items, float* __restrict__ out,
    int ldo, int kv_heads, float eps, float* __restrict__ partial,
    unsigned* __restrict__ counters) {
  static_assert(D == 64 || D == 128, "head dimension 64 or 128");
  static_assert(2 * G <= 16, "hi and lo rows of the group fit one MFMA tile");
  constexpr int S = D / 32;                // MFMA steps per key row
  constexpr int PAIRS = (16 * G + 63) / 64;
  __shared__ float s_q[G][D];
  __shared__ __attribute__((aligned(16))) Half s_kv[2][D];
  __shared__ float s_tile[NW][16][17];
  __shared__ float s_p[NW][kGroupKeys][G];
  __shared__ float s_alpha[NW][G];
  __shared__ __attribute__((aligned(16))) float s_acc[NW][G][D];
  __shared__ float s_m[NW][G], s_l[NW][G];
  __shared__ float s_gate[G];

  const lfm3_attention_item item = items[blockIdx.x];
  const int g = blockIdx.y, row = int(item.row);
  const int tid = threadIdx.x, lane = tid & 63;
  // The output gate, loaded before any store (a load after stores waits
  // for them); its divisor goes to LDS for the epilogue or the merge once
  // the first K/V group is in flight.
  const float gate_x = tid < G ? gate[std::size_t(row) * ldg + g * G + tid] : 0.0f;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int stride = kv_heads * D;
  const std::uint32_t cap = capacity[row];
  const int kb = int(item.key_begin), ke = int(item.key_end);
  const int pos = kFused ? int(positions[row]) : -1;
  Half* ck = cache_k[row];
  Half* cv = cache_v[row];

  // The span holds the current position (fused: this block writes its
  // key to the ring); that key is never read back through the ring.
  const int held = kFused && ke == pos + 1 ? 1 : 0;
  // P V layout: lane L owns dimensions 8 (L % DL) .. + 7 of keys
  // L / DL + KG i (i < KPL) of each 16-key group, one 16-byte V load per key.
  constexpr int DL = D / 8, KG = 64 / DL, KPL = 16 / KG;
  const int dg = lane % DL, kq = lane / DL;
  // The rings as buffers: a key past the span reads zeros, without a branch.
  const unsigned ring_bytes = cap * unsigned(stride) * 2;
  const BufferResource k_res = MakeBuffer(ck, ring_bytes);
  const BufferResource v_res = MakeBuffer(cv, ring_bytes);
  const int n = lane & 15, kg = lane >> 4;
  // Ring slots of keys base + o (o < 16) for the lane's K row (o = n) and V
  // rows (o = kq + KG i): one wave-uniform division per group, then the
  // wrap as an unsigned minimum (rings of 16 slots or more; smaller rings
  // take the remainder). Keys past the span, and groups past the wave's
  // last, read zeros from an offset the hardware drops (no traffic). The
  // offsets are selects, not branches around the loads.
  const int ngroups = ngroups_of(kb, ke);
  const unsigned row_bytes = unsigned(stride) * 2;
  const unsigned k_lane = unsigned(g * D + 8 * kg) * 2, v_lane = unsigned(g * D + 8 * dg) * 2;
  const auto fetch = [&](int j, uint4 (&kr)[S], uint4 (&vr)[KPL]) {
    const int base = kb + kGroupKeys * j;
    // Keys of the group inside the span; the current position's key (the
    // span's last when it holds it) comes from LDS instead (patch below).
    const int rem = j < ngroups ? ke - held - base : 0;
    const unsigned b0 = unsigned(base) % cap;
    unsigned sk = b0 + unsigned(n), sv[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      sv[i] = b0 + unsigned(kq + KG * i);
    if (cap >= 16) {
      sk = min(sk, sk - cap);
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        sv[i] = min(sv[i], sv[i] - cap);
    } else {
      sk %= cap;
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        sv[i] %= cap;
    }
    const unsigned koff = n < rem ? sk * row_bytes + k_lane : kOutOfRange;
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2)
      kr[s2] = LoadB128(k_res, koff + 64 * s2);
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      vr[i] = LoadB128(v_res, kq + KG * i < rem ? sv[i] * row_bytes + v_lane : kOutOfRange);
  };

  uint4 kr[S], vr[KPL];

  // Prologue: queries of the group (normed and rotated when fused). Its
  // own loads go out first, then the wave's first K/V group, so the
  // group's loads are in flight while the prologue computes (loads return
  // in issue order: issued the other way round, the prologue would wait
  // for the group).
  if constexpr (kFused) {
#pragma clang fp contract(off)
    constexpr int P = D / 2, SLOTS = (NW * 64) / P, ROUNDS = (G + SLOTS) / SLOTS;
    const int slot = tid / P, pair = tid % P;
    const float fp = frequencies[pair];
    const float fac = factors ? factors[pair] : 1.0f;
    // Loaded without a branch (a slot past the key head reads the key row
    // again and drops it): values loaded under a branch are copied at its
    // join, and each copy waits for its load.
    float x0s[ROUNDS], x1s[ROUNDS], w0s[ROUNDS], w1s[ROUNDS];
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      const int h = r * SLOTS + slot;  // h == G is the key head
      const float* src = h < G ? q + std::size_t(row) * ld + (g * G + h) * D
                               : k + std::size_t(row) * ld + g * D;
      const float* w = h < G ? q_norm : k_norm;
      x0s[r] = src[pair];
      x1s[r] = src[pair + P];
      w0s[r] = w[pair];
      w1s[r] = w[pair + P];
    }
    // A buffer load (zero past the row), not a branch: the compiler would
    // sink the F16 conversion into the branch and wait for the load there.
    const float vrow = __uint_as_float(
        LoadB32(MakeBuffer(v + std::size_t(row) * ld + g * D, D * 4),
                tid < D ? unsigned(tid) * 4 : kOutOfRange));
    fetch(wave, kr, vr);
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits on a load moves above
    if (tid < G)
      s_gate[tid] = 1.0f + expf(-gate_x);
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      const int h = r * SLOTS + slot;
      if (h <= G) {
        const float x0 = x0s[r], x1 = x1s[r];
        float squares = x0 * x0 + x1 * x1;
#pragma unroll
        for (int m = P / 2; m; m >>= 1)
          squares += __shfl_xor(squares, m, 64);
        const float inv = 1.0f / sqrtf(squares / float(D) + eps);
        const float a = (x0 * inv) * w0s[r], b = (x1 * inv) * w1s[r];
        float angle = float(pos) * fp;
        if (factors)
          angle /= fac;
        float sn, cs;
        sincosf(angle, &sn, &cs);
        const float r0 = a * cs - b * sn, r1 = b * cs + a * sn;
        if (h < G) {
          s_q[h][pair] = r0;
          s_q[h][pair + P] = r1;
        } else {
          s_kv[0][pair] = FloatToHalfBits(r0);
          s_kv[0][pair + P] = FloatToHalfBits(r1);
        }
      }
    }
    static_assert(D <= NW * 64, "a thread per dimension of the V row");
    if (tid < D)
      s_kv[1][tid] = FloatToHalfBits(vrow);
    __syncthreads();
    if (held && tid < D) {
      // The row goes to the ring for later rounds; this launch takes the
      // key from s_kv (no other span of the row covers the position, so no
      // block reads the slot being written). Global stores, not flat ones:
      // a flat store in flight makes the compiler wait for every load
      // before the next LDS read.
      using GlobalHalf = __attribute__((address_space(1))) Half;
      const std::size_t at = std::size_t(std::uint32_t(pos) % cap) * stride + g * D + tid;
      ((GlobalHalf*)ck)[at] = s_kv[0][tid];
      ((GlobalHalf*)cv)[at] = s_kv[1][tid];
    }
  } else {
    constexpr int QPT = (G * D + NW * 64 - 1) / (NW * 64);
    float qv[QPT];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + NW * 64 * i;
      qv[i] = e < G * D ? q[std::size_t(row) * ld + (g * G + e / D) * D + e % D] : 0.0f;
    }
    fetch(wave, kr, vr);
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits on a load moves above
    if (tid < G)
      s_gate[tid] = 1.0f + expf(-gate_x);
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int e = tid + NW * 64 * i;
      if (e < G * D)
        s_q[e / D][e % D] = qv[i];
    }
    __syncthreads();
  }

  // A operand: row m < G is head m's hi part, G <= m < 2G head m - G's lo.
  h8 a[S];
  {
    const int m = lane & 15, kg = lane >> 4;
    const int head = m < G ? m : m < 2 * G ? m - G : 0;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = s_q[head][32 * s + 8 * kg + i];
        const _Float16 hi = static_cast<_Float16>(x);
        const _Float16 lo = static_cast<_Float16>((x - float(hi)) * 2048.0f);
        a[s][i] = m < G ? hi : m < 2 * G ? lo : _Float16(0);
      }
  }

  const float root = sqrtf(float(D));
  float m_own[PAIRS], l_own[PAIRS];
#pragma unroll
  for (int r = 0; r < PAIRS; ++r) {
    m_own[r] = -INFINITY;
    l_own[r] = 0.0f;
  }
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      acc[h][i] = 0.0f;
  const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

  uint4 kn[S], vn[KPL];
  for (int j = wave; j < ngroups; j += NW) {
    const int base = kb + kGroupKeys * j;
    fetch(j + NW, kn, vn);  // past the span: zeros, no traffic
    if constexpr (kFused) {
      // The current key (key o of the group holding it; no lane matches in
      // other groups) from LDS, as selects: a branch here would leave the
      // compiler's wait counts for the loads in flight inexact, and it
      // then waits for all of them.
      const int o = held ? pos - base : -1;
#pragma unroll
      for (int s2 = 0; s2 < S; ++s2)
        kr[s2] = SelectU4(n == o, *reinterpret_cast<const uint4*>(&s_kv[0][32 * s2 + 8 * kg]),
                          kr[s2]);
      const uint4 cur_v = *reinterpret_cast<const uint4*>(&s_kv[1][8 * dg]);
#pragma unroll
      for (int i = 0; i < KPL; ++i)
        vr[i] = SelectU4(kq + KG * i == o, cur_v, vr[i]);
    }
    f4 sacc = zero;
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2)
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s2], __builtin_bit_cast(h8, kr[s2]), sacc, 0, 0, 0);
    // D layout: lane L holds rows 4 (L / 16) + i of key L % 16.
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s_tile[wave][4 * (lane >> 4) + i][lane & 15] = sacc[i];
    WaveSync();
    // Online softmax: lane owns (head, key) pairs idx = lane + 64 r.
#pragma unroll
    for (int r = 0; r < PAIRS; ++r) {
      const int idx = lane + 64 * r, h = idx >> 4, nn = idx & 15;
      if (h < G) {
        float sc = (s_tile[wave][h][nn] + s_tile[wave][G + h][nn] * (1.0f / 2048.0f)) / root;
        if (base + nn >= ke)
          sc = -INFINITY;
        const float m_new = fmaxf(m_own[r], GroupMax16(sc));
        const float shift = m_new == -INFINITY ? 0.0f : m_new;
        const float p = expf(sc - shift);
        const float alpha = expf(m_own[r] - shift);
        l_own[r] = l_own[r] * alpha + GroupSum16(p);
        m_own[r] = m_new;
        s_p[wave][nn][h] = p;
        if (nn == 0)
          s_alpha[wave][h] = alpha;
      }
    }
    WaveSync();
    // P V: lane owns dimensions 8 dg .. + 7 of every head of the group.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float al = s_alpha[wave][h];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[h][i] *= al;
    }
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int o = kq + KG * i;
      float vf[8];
      const unsigned w4[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        vf[2 * d] = HalfBitsToFloat(w4[d] & 0xffffu);
        vf[2 * d + 1] = HalfBitsToFloat(w4[d] >> 16);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = s_p[wave][o][h];
#pragma unroll
        for (int d = 0; d < 8; ++d)
          acc[h][d] = fmaf(p, vf[d], acc[h][d]);
      }
    }
    WaveSync();  // the next group rewrites s_tile, s_p and s_alpha
#pragma unroll
    for (int s2 = 0; s2 < S; ++s2)
      kr[s2] = kn[s2];
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      vr[i] = vn[i];
  }

  // Merge the key quarters (eighths for D = 64) across lanes, then the
  // waves, in a fixed order.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float t = acc[h][i];
      if constexpr (DL == 8)
        t = SumXor8(t);
      t = SumXor32(SumXor16(t));
      acc[h][i] = t;
    }
  if (kq == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float4* dst = reinterpret_cast<float4*>(&s_acc[wave][h][8 * dg]);
      dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
#pragma unroll
  for (int r = 0; r < PAIRS; ++r) {
    const int idx = lane + 64 * r, h = idx >> 4;
    if (h < G && (idx & 15) == 0) {
      s_m[wave][h] = m_own[r];
      s_l[wave][h] = l_own[r];
    }
  }
  __syncthreads();
  const bool split = item.parts > 1;
  float* part_out = partial + (std::size_t(blockIdx.x) * kv_heads + g) * G * (D + 2);
  // The whole-row shape has no merge launch behind it (see the file head).
  const bool unmerged = split && NW == kWholeRowWaves;
  for (int e = tid; e < G * D; e += (NW * 64)) {
    const int h = e / D, d = e % D;
    float top = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      top = fmaxf(top, s_m[w][h]);
    float l = 0.0f, av = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = s_m[w][h] == -INFINITY ? 0.0f : expf(s_m[w][h] - top);
      l = fmaf(s_l[w][h], wt, l);
      av = fmaf(s_acc[w][h][d], wt, av);
    }
    const int head = g * G + h;
    if (unmerged) {
      out[std::size_t(row) * ldo + head * D + d] = __builtin_nanf("");
    } else if (!split) {
      out[std::size_t(row) * ldo + head * D + d] = (av / l) / s_gate[h];
    } else {
      float* po = part_out + h * (D + 2);
      if (d == 0) {
        AgentStore(po, top);
        AgentStore(po + 1, l);
      }
      AgentStore(po + 2 + d, av);
    }
  }
  if constexpr (NW == kAttnWaves) {
    if (split) {  // uniform over the block
      __shared__ int s_last;
      __shared__ float s_w[kMaxParts][G], s_lv[kMaxParts][G], s_top[G], s_den[G];
      // Every thread's partial stores have completed before the arrival.
      // The hand-over is relaxed on purpose, and is ordered by how gfx950
      // carries out agent-scope accesses rather than by C++ release /
      // acquire: AgentStore writes through the XCD's L2 to the device's
      // coherence point, vmcnt(0) returns only once every store of this
      // thread is acknowledged there, the block barrier makes that true
      // for every thread before the atomic is issued, the atomic itself is
      // performed at that point, and the merging block issues its
      // AgentLoads (which read from that point, not from its own L2) only
      // after its atomic returned the final count (through LDS and a
      // block barrier, which the compiler does not move loads across). A
      // release / acquire pair would add an L2 write-back and an
      // invalidate to every arrival. The multi-span parity tests at
      // 16K-32K keys (many spans a row) would see a stale partial.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        unsigned* c = counters + std::size_t(item.first_item) * kv_heads + g;
        const unsigned arrived =
            __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
        const bool last = arrived == item.parts;
        if (last)
          __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
      }
      __syncthreads();
      if (s_last)
        MergeSpans<D, G, NW * 64>(item, g, kv_heads, partial, s_gate, out, ldo, s_w, s_lv,
                                  s_top, s_den);
    }
  }
}

struct AttentionArgs {
  const float *q = nullptr, *k = nullptr, *v = nullptr;
  int ld = 0;
  const float* gate = nullptr;
  int ldg = 0;
  const float *q_norm = nullptr, *k_norm = nullptr, *frequencies = nullptr,
              *factors = nullptr;
  Half* const* ck = nullptr;
  Half* const* cv = nullptr;
  const std::uint32_t *positions = nullptr, *capacity = nullptr;
  const lfm3_attention_item* items = nullptr;
  float* out = nullptr;
  int ldo = 0, kv = 0;
  float eps = 0.0f;
  float* partial = nullptr;
  unsigned* counters = nullptr;
};

template<int D, int G, int NW>
void LaunchWaves(const AttentionArgs& a, dim3 grid, hipStream_t s, bool fused) {
  if (fused)
    DecodeAttentionKernel<D, G, true, NW><<<grid, NW * 64, 0, s>>>(
        a.q, a.k, a.v, a.ld, a.gate, a.ldg, a.q_norm, a.k_norm, a.frequencies,
        a.factors, a.ck, a.cv, a.positions, a.capacity, a.items, a.out, a.ldo,
        a.kv, a.eps, a.partial, a.counters);
  else
    DecodeAttentionKernel<D, G, false, NW><<<grid, NW * 64, 0, s>>>(
        a.q, a.k, a.v, a.ld, a.gate, a.ldg, a.q_norm, a.k_norm, a.frequencies,
        a.factors, a.ck, a.cv, a.positions, a.capacity, a.items, a.out, a.ldo,
        a.kv, a.eps, a.partial, a.counters);
}

// Every row in one item (sliding windows, short histories): 8-wave
// blocks (two 16-key groups per wave for a 256-key window) and no merge.
// Otherwise 4-wave blocks over the spans, each row's last span block
// merging.
template<int D, int G>
void LaunchGroup(const AttentionArgs& a, dim3 grid, hipStream_t s, bool fused, bool whole_rows) {
  if (whole_rows)
    LaunchWaves<D, G, kWholeRowWaves>(a, grid, s, fused);
  else
    LaunchWaves<D, G, kAttnWaves>(a, grid, s, fused);
}

template<int D>
void LaunchDim(int group, const AttentionArgs& a, dim3 grid, hipStream_t s, bool fused,
               bool whole_rows) {
  switch (group) {
    case 2: LaunchGroup<D, 2>(a, grid, s, fused, whole_rows); break;
    case 4: LaunchGroup<D, 4>(a, grid, s, fused, whole_rows); break;
    default: LaunchGroup<D, 8>(a, grid, s, fused, whole_rows); break;
  }
}

int Launch(const AttentionArgs& a, std::uint32_t n_items, std::uint32_t rows,
           std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
           void* workspace, std::size_t workspace_bytes, void* stream,
           bool fused) {
  const std::uint32_t group = kv_heads ? heads / kv_heads : 0;
  if (!a.q || !a.gate || !a.ck || !a.cv || !a.capacity || !a.items || !a.out ||
      !rows || !kv_heads || heads % kv_heads ||
      (group != 2 && group != 4 && group != 8) || (dim != 64 && dim != 128) ||
      (fused && (!a.k || !a.v || !a.q_norm || !a.k_norm || !a.frequencies ||
                 !a.positions)))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 attention shape");
  if (!n_items)
    return LFM3_OK;
  if (!workspace || workspace_bytes < lfm3_attention_workspace_bytes(
                                          n_items, rows, heads, kv_heads, dim))
    return Fail(LFM3_E_INVALID, "LFM3 attention workspace too small");
  if (std::size_t(n_items) * kv_heads * sizeof(unsigned) > kCounterBytes)
    return Fail(LFM3_E_INVALID, "LFM3 attention plan has too many items for its counters");
  AttentionArgs args = a;
  args.kv = int(kv_heads);
  args.counters = static_cast<unsigned*>(workspace);
  args.partial = reinterpret_cast<float*>(static_cast<std::uint8_t*>(workspace) + kCounterBytes);
  const dim3 grid(n_items, kv_heads);
  const auto s = static_cast<hipStream_t>(stream);
  // Every plan item covers at least one row, so n_items == rows means one
  // item (no split) per row.
  const bool whole_rows = n_items == rows;
  if (dim == 128)
    LaunchDim<128>(int(group), args, grid, s, fused, whole_rows);
  else
    LaunchDim<64>(int(group), args, grid, s, fused, whole_rows);
  return HipStatus(hipGetLastError(), "LFM3 decode attention launch");
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
std::array<void*, kMaxDevices> g_scratch{};

// The current device's copy of `scratch`, looked up once per device.
int ScratchAddress(void** out) {
  int device = 0;
  int e = HipStatus(hipGetDevice(&device), "LFM3 attention scratch device");
  if (e)
    return e;
  if (device < 0 || device >= kMaxDevices)
    return Fail(LFM3_E_INVALID, "LFM3 attention scratch: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch[device]) {
    void* p = nullptr;
    e = HipStatus(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                  "LFM3 attention scratch address");
    if (e)
      return e;
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return LFM3_OK;
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
  // Span length: about kTargetItems items over the round, multiples of 64
  // keys between kMinSpan and kMaxSpan, and at most kMaxParts per row.
  std::uint64_t total = 0;
  std::uint32_t longest = 0;
  for (std::uint32_t r = 0; r < rows; ++r) {
    const std::uint32_t p = positions[r];
    const std::uint32_t first = window && p + 1 > window ? p + 1 - window : 0;
    total += p + 1 - first;
    longest = std::max(longest, p + 1 - first);
  }
  std::uint64_t span = (total + kTargetItems - 1) / kTargetItems;
  span = std::max<std::uint64_t>(span, (longest + kMaxParts - 1) / kMaxParts);
  span = (span + 63) / 64 * 64;
  span = std::min<std::uint64_t>(std::max<std::uint64_t>(span, kMinSpan), kMaxSpan);
  // A window of up to 256 keys is one item (an 8-wave block, no merge
  // launch).
  if (window && window <= 256)
    span = std::max<std::uint64_t>(span, window);
  if ((longest + span - 1) / span > kMaxParts)
    return Fail(LFM3_E_INVALID, "LFM3 attention row is too long");
  std::uint32_t count = 0;
  for (std::uint32_t r = 0; r < rows; ++r) {
    const std::uint32_t p = positions[r];
    const std::uint32_t first = window && p + 1 > window ? p + 1 - window : 0;
    const std::uint32_t keys = p + 1 - first;
    const std::uint32_t parts = std::uint32_t((keys + span - 1) / span);
    if (count + parts > max_items)
      return Fail(LFM3_E_INVALID, "LFM3 attention plan exceeds its item list");
    for (std::uint32_t s = 0; s < parts; ++s) {
      lfm3_attention_item& it = items[count + s];
      it.row = r;
      it.key_begin = first + std::uint32_t(s * span);
      it.key_end = std::uint32_t(std::min<std::uint64_t>(first + (s + 1) * span, p + 1));
      it.first_item = count;
      it.parts = parts;
      it.reserved[0] = it.reserved[1] = it.reserved[2] = 0;
    }
    count += parts;
  }
  return int(count);
}

std::size_t lfm3_attention_max_items(std::uint32_t rows,
                                     std::uint32_t max_position) {
  // A span is at least max(kMinSpan, total keys / kTargetItems) keys long
  // unless capped at kMaxSpan; rounding up costs at most one item per row.
  const std::uint64_t keys = std::uint64_t(max_position) + 1;
  return std::size_t(kTargetItems) + rows +
         std::size_t(rows) * std::size_t((keys + kMaxSpan - 1) / kMaxSpan);
}

std::size_t lfm3_attention_workspace_bytes(std::uint32_t items,
                                           std::uint32_t rows,
                                           std::uint32_t heads,
                                           std::uint32_t kv_heads,
                                           std::uint32_t dim) {
  (void)rows;
  (void)kv_heads;
  return kCounterBytes + std::size_t(items) * heads * (dim + 2) * sizeof(float);
}

int lfm3_decode_attention_ragged(
    const float* q, std::uint32_t ldq, const float* gate, std::uint32_t ldg,
    const std::uint16_t* const* cache_k, const std::uint16_t* const* cache_v,
    const std::uint32_t* capacity, const lfm3_attention_item* items,
    std::uint32_t n_items, float* out, std::uint32_t ldo, std::uint32_t rows,
    std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
    void* workspace, std::size_t workspace_bytes, void* stream) {
  AttentionArgs a;
  a.q = q;
  a.ld = int(ldq);
  a.gate = gate;
  a.ldg = int(ldg);
  // The unfused kernel only reads the rings.
  a.ck = const_cast<Half* const*>(reinterpret_cast<const Half* const*>(cache_k));
  a.cv = const_cast<Half* const*>(reinterpret_cast<const Half* const*>(cache_v));
  a.capacity = capacity;
  a.items = items;
  a.out = out;
  a.ldo = int(ldo);
  return Launch(a, n_items, rows, heads, kv_heads, dim, workspace,
                workspace_bytes, stream, false);
}

int lfm3_decode_heads_attention_ragged(
    const float* q, const float* k, const float* v, std::uint32_t ld,
    const float* gate, std::uint32_t ldg, const float* q_norm,
    const float* k_norm, const float* frequencies, const float* factors,
    std::uint16_t* const* cache_k, std::uint16_t* const* cache_v,
    const std::uint32_t* positions, const std::uint32_t* capacity,
    const lfm3_attention_item* items, std::uint32_t n_items, float* out,
    std::uint32_t ldo, std::uint32_t rows, std::uint32_t heads,
    std::uint32_t kv_heads, std::uint32_t dim, float eps, void* workspace,
    std::size_t workspace_bytes, void* stream) {
  AttentionArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.ld = int(ld);
  a.gate = gate;
  a.ldg = int(ldg);
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.frequencies = frequencies;
  a.factors = factors;
  a.ck = reinterpret_cast<Half* const*>(cache_k);
  a.cv = reinterpret_cast<Half* const*>(cache_v);
  a.positions = positions;
  a.capacity = capacity;
  a.items = items;
  a.out = out;
  a.ldo = int(ldo);
  a.eps = eps;
  return Launch(a, n_items, rows, heads, kv_heads, dim, workspace,
                workspace_bytes, stream, true);
}

}  // extern "C"

extern "C" int lfm3_decode_heads_attention_ragged_noalloc(
    const float* q, const float* k, const float* v, std::uint32_t ld, const float* gate,
    std::uint32_t ldg, const float* q_norm, const float* k_norm, const float* frequencies,
    const float* factors, std::uint16_t* const* cache_k, std::uint16_t* const* cache_v,
    const std::uint32_t* positions, const std::uint32_t* capacity,
    const lfm3_attention_item* items, std::uint32_t n_items, float* out, std::uint32_t ldo,
    std::uint32_t rows, std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
    float eps, void* stream) {
  const std::size_t need = lfm3_attention_workspace_bytes(n_items, rows, heads, kv_heads, dim);
  if (need > LFM3_ATTENTION_SCRATCH_BYTES)
    return Fail(LFM3_E_INVALID,
                "LFM3 attention plan needs " + std::to_string(need) +
                    " bytes of span partials, more than the library's " +
                    std::to_string(LFM3_ATTENTION_SCRATCH_BYTES) + "-byte scratch");
  void* ws = nullptr;
  const int e = ScratchAddress(&ws);
  if (e)
    return e;
  return lfm3_decode_heads_attention_ragged(q, k, v, ld, gate, ldg, q_norm, k_norm, frequencies,
                                            factors, cache_k, cache_v, positions, capacity, items,
                                            n_items, out, ldo, rows, heads, kv_heads, dim, eps, ws,
                                            LFM3_ATTENTION_SCRATCH_BYTES, stream);
}
