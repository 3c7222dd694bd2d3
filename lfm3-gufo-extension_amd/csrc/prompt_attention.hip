// Causal prompt attention on gfx950 MFMA: n query rows at positions
// position .. position + n - 1 over the F16 K/V of the chunk (keys at or
// after position) and of the ring (earlier keys), with an optional sliding
// window (hip/ops.hip:1355-1561 WmmaAttn, 1692-1709 PromptCombine,
// 2275-2280 PromptSplits, 2289-2333 Attention for n > 1).
//
// Numerics follow the reference's prompt path: Q is scaled by
// log2(e) / sqrt(D) in FP32 and rounded to F16; scores are FP32 sums of F16
// products in base-2 units; per 64-key tile the running maximum rescales the
// running sum and output; probabilities are rounded to F16 once and the sum
// adds the rounded values, so the weights applied to V are exactly
// normalized; out = (acc / sum) / (1 + e^-gate).
//
// A block of 8 waves owns one KV head's group of G query heads and 128 CT
// (query row, head) columns (128 CT / G rows x G heads); each wave owns CT
// tiles of 16 columns (two for long histories, so each K and V operand read
// from LDS feeds two MFMAs). K and V tiles of 64 keys are staged through
// LDS (double buffered, the next tile prefetched into registers) and shared
// by the 8 waves; the row blocks of one (span, KV head) run on one XCD, so
// its K/V tiles come from HBM once and then from that XCD's L2. Each wave
// computes S^T = K Q^T (v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims,
// B = Q^T) and O^T += V^T P^T (A = 16 dims x 32 keys of the transposed V
// tile, B = P^T). The K operand rows are permuted so that in
// the S^T accumulator lane L holds exactly the 8 keys that the P^T operand
// needs in lane L (keys 8 (L / 16) + j of a 32-key group): probabilities
// never cross lanes. A column's softmax state is per lane; its row maximum
// and final sum combine the 4 lanes of the column (L % 16) with two
// exchanges. Long global histories split keys across blockIdx.y into spans
// (SpanPlan: enough spans for about one block per CU, whole 64-key tiles,
// at least 1024 keys and at most 16 spans; the reference's PromptSplits
// instead fixes spans of at least 2048 keys, at most 8). Each span stores
// its maximum, sum and unnormalized output, merged by CombineSpansKernel.
#include <cmath>

#include "common.hpp"

namespace lfm3amd {
namespace {

constexpr int kPAWaves = 8, kPAThreads = 64 * kPAWaves;
constexpr int kPAKeys = 64;             // keys a tile

// Key spans of a long causal history (blockIdx.y of the tile launch): a
// launch of row blocks x KV heads blocks per span is cut into spans until
// it has about one block per CU, each span a whole number of 64-key tiles
// and at least kSpanFloorTiles tiles long, so the merge launch stays small
// next to the spans. A sliding window never splits.
constexpr int kFillBlocks = 256, kSpanFloorTiles = 16, kMaxSpans = 16;

int SpanPlan(int keys, int blocks_per_span, int& span_keys) {
  const int tiles = (keys + kPAKeys - 1) / kPAKeys;
  int spans = (kFillBlocks + blocks_per_span - 1) / std::max(blocks_per_span, 1);
  spans = std::min({spans, kMaxSpans, std::max(1, tiles / kSpanFloorTiles)});
  span_keys = (tiles + spans - 1) / spans * kPAKeys;
  return (keys + span_keys - 1) / span_keys;
}

// Keys visible to a query at absolute position p, clipped to a span
// [span_lo, span_hi]: the causal window [p + 1 - window, p] (from key 0
// without a window). Inclusive bounds; empty when lo > hi. Visible(p).lo
// and Visible(p).hi are both non-decreasing in p, so a run of consecutive
// queries sees the union {Visible(first).lo, Visible(last).hi} and every
// query of the run sees {Visible(last).lo, Visible(first).hi}.
struct KeyRange {
  int lo, hi;
};
__device__ __forceinline__ KeyRange Visible(int p, int window, int span_lo, int span_hi) {
  const int oldest = window > 0 ? p - window + 1 : 0;
  return KeyRange{max(oldest, span_lo), min(p, span_hi)};
}

// Slot of a key row's 16-byte segment: XOR swizzle chosen so that the 16
// keys one S^T operand read touches (keys 8 (r / 4) + (r % 4), r < 16, plus
// a constant) land in distinct banks.
template<int D>
__device__ __forceinline__ int KeySwizzle(int key) {
  if constexpr (D == 128)
    return (key & 3) | (((key >> 3) & 3) << 2);
  else
    return ((key >> 1) & 1) | (((key >> 3) & 3) << 1);
}

__device__ __forceinline__ unsigned PackHalves(float a, float b) {
  return unsigned(FloatToHalfBits(a)) | (unsigned(FloatToHalfBits(b)) << 16);
}

// Block b of a launch over (row blocks, splits, KV heads): blocks are
// dispatched to the 8 XCDs round robin, so the row blocks of one (split,
// KV head), which read the same K/V tiles, are placed on one XCD's L2.
__device__ __forceinline__ void PromptBlock(int b, int row_blocks, int& rb, int& pair) {
  const int xcd = b % 8, i = b / 8;
  rb = i % row_blocks;
  pair = xcd + 8 * (i / row_blocks);
}

template<int D, int G, int CT>
__launch_bounds__(kPAThreads) __global__ void PromptAttentionKernel(
    const float* __restrict__ q, int ldq, const Half* __restrict__ k,
    const Half* __restrict__ v, const float* __restrict__ gate, int ldg,
    const Half* __restrict__ ck, const Half* __restrict__ cv, float* __restrict__ out,
    int ldo, float* __restrict__ partial, int n, int heads, int kv_heads, int position,
    int capacity, int window, int span, int row_blocks, int splits) {
  static_assert(D == 64 || D == 128, "head dimension");
  constexpr int kCols = 16 * CT * kPAWaves;  // (row, head) columns a block
  static_assert(kCols % G == 0 && G >= 2 && G <= 8, "query group");
  constexpr int kRows = kCols / G;         // query rows a block
  constexpr int kSegs = D / 8;             // 16-byte segments a key row
  constexpr int kSteps = D / 32;           // MFMA K steps over dimensions
  constexpr int kDimBlocks = D / 16;       // O^T accumulators
  constexpr int kVPitch = kPAKeys + 8;     // halves a transposed V row
  constexpr int kKLoads = kPAKeys * kSegs / kPAThreads;     // K segments a thread
  constexpr int kVPairs = kPAKeys / 2 * kSegs;               // (key pair, segment) jobs
  static_assert(kKLoads * kPAThreads == kPAKeys * kSegs, "K staging");
  __shared__ __attribute__((aligned(16))) Half sK[2][kPAKeys * D];
  __shared__ __attribute__((aligned(16))) Half sV[2][D * kVPitch];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  int rb, pair;
  PromptBlock(blockIdx.x, row_blocks, rb, pair);
  // Past the last (split, KV head) pair: the grid rounds up to whole XCD
  // rows of row blocks.
  if (pair >= splits * kv_heads)
    return;
  const int g = pair / splits, split = pair % splits, q0 = rb * kRows;
  const int stride = kv_heads * D;
  // Column tile ct of this wave: columns wave 16 CT + 16 ct + L % 16.
  int row[CT], head[CT];
  bool live[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int c = (wave * CT + ct) * 16 + col;
    row[ct] = q0 + c / G;
    head[ct] = g * G + c % G;
    live[ct] = row[ct] < n;
  }
  // The output gate's divisor, loaded with the queries: a load after the
  // output stores would wait for them.
  float g_scale[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
    g_scale[ct] = partial || !live[ct]
                      ? 1.0f
                      : 1.0f + expf(-gate[std::size_t(row[ct]) * ldg + head[ct]]);

  // Q^T operands: lane L holds dims 32 s + 8 (L / 16) + j of its column,
  // scaled in FP32 and rounded to F16.
  const float scale = rsqrtf(float(D)) * 1.44269504088896341f;
  h8 qf[CT][kSteps];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float* qr = q + std::size_t(live[ct] ? row[ct] : 0) * ldq + head[ct] * D;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const float4 a = live[ct] ? *reinterpret_cast<const float4*>(qr + 32 * s + 8 * grp)
                                : make_float4(0, 0, 0, 0);
      const float4 b = live[ct] ? *reinterpret_cast<const float4*>(qr + 32 * s + 8 * grp + 4)
                                : make_float4(0, 0, 0, 0);
      const unsigned w[4] = {PackHalves(a.x * scale, a.y * scale),
                             PackHalves(a.z * scale, a.w * scale),
                             PackHalves(b.x * scale, b.y * scale),
                             PackHalves(b.z * scale, b.w * scale)};
      qf[ct][s] = __builtin_bit_cast(h8, w);
    }
  }

  // Visible keys of each column, of the block's rows (the tiles it walks)
  // and of the wave's rows: their union (tiles the wave computes) and their
  // intersection (tiles every column sees whole, where the mask is skipped).
  const int span_lo = split * span, span_hi = span_lo + span - 1;
  const auto visible = [&](int r) { return Visible(position + r, window, span_lo, span_hi); };
  KeyRange own[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
    own[ct] = visible(row[ct]);
  const KeyRange walk{visible(q0).lo, visible(min(q0 + kRows, n) - 1).hi};
  const int wave_r0 = q0 + wave * 16 * CT / G;
  const int wave_r1 = min(q0 + (wave * 16 * CT + 16 * CT - 1) / G, n - 1);
  const bool wave_live = wave_r0 < n;
  const KeyRange reach{visible(wave_r0).lo, visible(wave_r1).hi};
  const KeyRange whole{visible(wave_r1).lo, visible(wave_r0).hi};

  // Staging jobs of this thread: K job u is (key, segment) = (j / kSegs,
  // j % kSegs) with j = tid + kPAThreads u; V job i (threads below kVPairs)
  // is key 2 (tid % 32) + i of segment tid / 32. Keys at or after position
  // are the prompt's own rows (row t - position), older keys sit in ring
  // slot t mod capacity. Both are read as buffers: a key past the block's
  // last, or one that lies in the other source, gets an offset the hardware
  // drops and reads zeros, without a branch. Tiles are loaded in order, so
  // each job's ring offset advances by one tile's keys (mod the ring) with
  // an add and a conditional subtract instead of a division per load.
  constexpr int kJobs = kKLoads + 2;
  const unsigned row_bytes = unsigned(stride) * 2;
  const unsigned ring_bytes = unsigned(capacity) * row_bytes;
  const BufferResource rk = MakeBuffer(k, unsigned(n) * row_bytes);
  const BufferResource rv = MakeBuffer(v, unsigned(n) * row_bytes);
  const BufferResource rck = MakeBuffer(ck, ring_bytes);
  const BufferResource rcv = MakeBuffer(cv, ring_bytes);
  int job_key[kJobs];
  unsigned job_seg[kJobs], job_ring[kJobs];
#pragma unroll
  for (int u = 0; u < kKLoads; ++u) {
    const int j = tid + kPAThreads * u;
    job_key[u] = j / kSegs;
    job_seg[u] = unsigned(g * D + (j % kSegs) * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    job_key[kKLoads + i] = 2 * (tid % 32) + i;
    job_seg[kKLoads + i] = unsigned(g * D + (tid / 32 % kSegs) * 8) * 2;
  }
#pragma unroll
  for (int u = 0; u < kJobs; ++u)
    job_ring[u] = unsigned((walk.lo + job_key[u]) % capacity) * row_bytes + job_seg[u];
  const unsigned ring_step = unsigned(kPAKeys % capacity) * row_bytes;
  uint4 kr[kKLoads], vr[2];
  const auto load = [&](int base) {
    const int last = walk.hi - base, own = position - base;  // key offsets in the tile
    const bool from_ring = own > 0, mixed = own > 0 && own < kPAKeys;
    const BufferResource src_k = from_ring ? rck : rk;
    const BufferResource src_v = from_ring ? rcv : rv;
    const unsigned chunk0 = unsigned(base - position) * row_bytes;
    uint4 r[kJobs];
#pragma unroll
    for (int u = 0; u < kJobs; ++u) {
      const int key = job_key[u];
      const unsigned chunk = chunk0 + unsigned(key) * row_bytes + job_seg[u];
      const bool live = (u < kKLoads || tid < kVPairs) && key <= last, ring = key < own;
      const unsigned off = !live ? kOutOfRange : from_ring ? (ring ? job_ring[u] : kOutOfRange)
                                                           : chunk;
      r[u] = LoadB128(u < kKLoads ? src_k : src_v, off);
      if (mixed) {
        const uint4 c = LoadB128(u < kKLoads ? rk : rv, live && !ring ? chunk : kOutOfRange);
        r[u] = make_uint4(r[u].x | c.x, r[u].y | c.y, r[u].z | c.z, r[u].w | c.w);
      }
      job_ring[u] += ring_step;
      job_ring[u] -= job_ring[u] >= ring_bytes ? ring_bytes : 0u;
    }
#pragma unroll
    for (int u = 0; u < kKLoads; ++u)
      kr[u] = r[u];
    vr[0] = r[kKLoads];
    vr[1] = r[kKLoads + 1];
  };
  const auto store = [&](int st) {
#pragma unroll
    for (int u = 0; u < kKLoads; ++u) {
      const int j = tid + kPAThreads * u, key = j / kSegs, seg = j % kSegs;
      *reinterpret_cast<uint4*>(&sK[st][key * D + (seg ^ KeySwizzle<D>(key)) * 8]) = kr[u];
    }
    if (tid < kVPairs) {
      const int seg = tid / 32, key = 2 * (tid % 32);
      const unsigned a[4] = {vr[0].x, vr[0].y, vr[0].z, vr[0].w};
      const unsigned b[4] = {vr[1].x, vr[1].y, vr[1].z, vr[1].w};
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        // (key, key + 1) halves of dimension seg * 8 + d.
        const unsigned word = __builtin_amdgcn_perm(b[d / 2], a[d / 2],
                                                    (d & 1) ? 0x07060302u : 0x05040100u);
        *reinterpret_cast<unsigned*>(&sV[st][(seg * 8 + d) * kVPitch + key]) = word;
      }
    }
  };

  f4 acc[CT][kDimBlocks];
  float maximum[CT], sum[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
    for (int m = 0; m < kDimBlocks; ++m)
      acc[ct][m] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    maximum[ct] = -INFINITY;
    sum[ct] = 0.0f;
  }

  const auto compute = [&](int st, int base) {
    const Half* tk = sK[st];
    const Half* tv = sV[st];
    // S^T block kb: A row r <-> key 32 (kb / 2) + 8 (r / 4) + 4 (kb % 2) + r % 4.
    // Each K operand read feeds every column tile of the wave.
    f4 s[CT][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int key = 32 * (kb >> 1) + 8 * (col >> 2) + 4 * (kb & 1) + (col & 3);
      const int swz = KeySwizzle<D>(key);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        s[ct][kb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st2 = 0; st2 < kSteps; ++st2) {
        const int seg = 4 * st2 + grp;
        const h8 a = *reinterpret_cast<const h8*>(&tk[key * D + (seg ^ swz) * 8]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          s[ct][kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[ct][st2], s[ct][kb], 0, 0, 0);
      }
    }
    // Lane L's value i of block kb is key base + 32 (kb / 2) + 8 (L / 16) +
    // 4 (kb % 2) + i of its column.
    const bool open = base >= whole.lo && base + kPAKeys - 1 <= whole.hi;
    h8 p[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float tile_max = -INFINITY;
      if (open) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            tile_max = fmaxf(tile_max, s[ct][kb][i]);
      } else {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = base + 32 * (kb >> 1) + 8 * grp + 4 * (kb & 1) + i;
            s[ct][kb][i] = (t >= own[ct].lo && t <= own[ct].hi) ? s[ct][kb][i] : -INFINITY;
            tile_max = fmaxf(tile_max, s[ct][kb][i]);
          }
      }
      // The column's 4 lanes (L % 16 equal): L ^ 16 and L ^ 32.
      tile_max = MaxXor32(MaxXor16(tile_max));
      const float next = fmaxf(maximum[ct], tile_max);
      const float shift = next == -INFINITY ? 0.0f : next;
      const float alpha = __builtin_amdgcn_exp2f(maximum[ct] - shift);
      maximum[ct] = next;
      // Probabilities round to F16 once (two a v_cvt_pk_f16_f32); the sum
      // adds the rounded values, two a v_dot2 against (1, 1), whose
      // products are exact, in two chains.
      const h2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
      unsigned pw[4][2];
      float local[2] = {0.0f, 0.0f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          typedef float f2 __attribute__((ext_vector_type(2)));
          const f2 e = {__builtin_amdgcn_exp2f(s[ct][kb][2 * j] - shift),
                        __builtin_amdgcn_exp2f(s[ct][kb][2 * j + 1] - shift)};
          const h2 ph = __builtin_convertvector(e, h2);
          local[j] = __builtin_amdgcn_fdot2(ph, ones, local[j], false);
          pw[kb][j] = __builtin_bit_cast(unsigned, ph);
        }
      sum[ct] = sum[ct] * alpha + (local[0] + local[1]);
      // exp2(0) is exactly 1: when no lane's maximum moved, the rescale of
      // the accumulators is skipped for the whole wave.
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int m = 0; m < kDimBlocks; ++m)
          acc[ct][m] *= alpha;
      }
      // P^T operand: keys 32 c2 + 8 (L / 16) + j, j < 8, of column L % 16:
      // values 0..3 of block 2 c2 then of block 2 c2 + 1.
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const unsigned w[4] = {pw[2 * c2][0], pw[2 * c2][1], pw[2 * c2 + 1][0],
                               pw[2 * c2 + 1][1]};
        p[ct][c2] = __builtin_bit_cast(h8, w);
      }
    }
    // O^T += V^T P^T: each V operand read feeds every column tile.
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
#pragma unroll
      for (int m = 0; m < kDimBlocks; ++m) {
        const h8 a = *reinterpret_cast<const h8*>(
            &tv[(16 * m + col) * kVPitch + 32 * c2 + 8 * grp]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          acc[ct][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, p[ct][c2], acc[ct][m], 0, 0, 0);
      }
    }
  };

  // Tiles: write the prefetched tile to its stage, one barrier (the tile is
  // visible, and every wave is done with the stage written two tiles ago),
  // prefetch the next tile, multiply.
  if (walk.lo <= walk.hi)
    load(walk.lo);
  int it = 0;
  for (int base = walk.lo; base <= walk.hi; base += kPAKeys, ++it) {
    const int st = it & 1;
    store(st);
    __syncthreads();
    if (base + kPAKeys <= walk.hi)
      load(base + kPAKeys);
    if (!wave_live || base > reach.hi || base + kPAKeys <= reach.lo)
      continue;
    compute(st, base);
  }

#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float total = SumXor32(SumXor16(sum[ct]));
    if (!live[ct])
      continue;
    // Lane L holds dimensions 16 m + 4 (L / 16) + i of its column.
    if (partial) {
      float* part = partial + ((std::size_t(split) * n + row[ct]) * heads + head[ct]) * (D + 2);
      if (grp == 0) {
        part[0] = maximum[ct];
        part[1] = total;
      }
      // Records are D + 2 floats: plain float stores (no 16-byte alignment).
#pragma unroll
      for (int m = 0; m < kDimBlocks; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          part[2 + 16 * m + 4 * grp + i] = acc[ct][m][i];
      continue;
    }
    float* o = out + std::size_t(row[ct]) * ldo + head[ct] * D;
#pragma unroll
    for (int m = 0; m < kDimBlocks; ++m) {
      f4 r;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = (acc[ct][m][i] / total) / g_scale[ct];
      *reinterpret_cast<f4*>(o + 16 * m + 4 * grp) = r;
    }
  }
}

// hip/ops.hip:1692-1709: merges key spans (base-2 maxima); one block per
// (row, head), one thread per dimension.
template<int D>
__launch_bounds__(D) __global__
    void CombineSpansKernel(const float* __restrict__ partial, const float* __restrict__ gate,
                            int ldg, float* __restrict__ out, int ldo, int n, int heads,
                            int splits) {
  const int rh = blockIdx.x, d = threadIdx.x;
  const int row = rh / heads, head = rh % heads;
  const std::size_t rows = std::size_t(n) * heads;
  // Every load (each span's maximum, sum and output element, and the gate)
  // is issued before any arithmetic: one memory round trip.
  float m[kMaxSpans], l[kMaxSpans], a[kMaxSpans];
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s) {
    const float* part = partial + (s * rows + rh) * (D + 2);
    m[s] = s < splits ? part[0] : -INFINITY;
    l[s] = s < splits ? part[1] : 0.0f;
    a[s] = s < splits ? part[2 + d] : 0.0f;
  }
  const float g = gate[std::size_t(row) * ldg + head];
  float maximum = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s)
    maximum = fmaxf(maximum, m[s]);
  float sum = 0.0f, acc = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s) {
    if (s < splits) {
      const float w = __builtin_amdgcn_exp2f(m[s] - maximum);
      sum = fmaf(l[s], w, sum);
      acc = fmaf(a[s], w, acc);
    }
  }
  out[std::size_t(row) * ldo + head * D + d] = (acc / sum) / (1.0f + expf(-g));
}

// The span merge of one query row over all its heads, fused with the FP16
// row-scaled activations of the attention output (the output projection's
// GEMM input, hip/q8_prefill.hpp:27-51): a thread takes 4 dimensions of one
// head, merges the spans with CombineSpansKernel's expressions and order
// (a single span reduces to the tile kernel's own (acc / sum) / (1 +
// e^-gate)), the block reduces the row's max |out|, and the row is stored
// as fp16(out 2^e) with scale 2^-e (HalfRowsKernel's expressions).
constexpr int kCombineDims = 4;

template<int D>
__launch_bounds__(1024) __global__
    void CombineRowsHalfKernel(const float* __restrict__ partial, const float* __restrict__ gate,
                               int ldg, Half* __restrict__ out, int lda,
                               float* __restrict__ scale, int n, int heads, int splits) {
  __shared__ float s_max[16];
  const int row = blockIdx.x, tid = threadIdx.x;
  constexpr int kPerHead = D / kCombineDims;
  const bool live = tid < heads * kPerHead;
  const int head = live ? tid / kPerHead : 0, d0 = (tid % kPerHead) * kCombineDims;
  const std::size_t rh = std::size_t(row) * heads + head, rows = std::size_t(n) * heads;
  float m[kMaxSpans], l[kMaxSpans], a[kMaxSpans][kCombineDims];
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s) {
    const float* part = partial + (s * rows + rh) * (D + 2);
    const bool on = live && s < splits;
    // Records are D + 2 floats: 8-byte aligned pairs.
    const float2 ml = on ? *reinterpret_cast<const float2*>(part) : make_float2(-INFINITY, 0.0f);
    const float2 v0 = on ? *reinterpret_cast<const float2*>(part + 2 + d0) : make_float2(0, 0);
    const float2 v1 = on ? *reinterpret_cast<const float2*>(part + 4 + d0) : make_float2(0, 0);
    m[s] = ml.x;
    l[s] = ml.y;
    a[s][0] = v0.x;
    a[s][1] = v0.y;
    a[s][2] = v1.x;
    a[s][3] = v1.y;
  }
  const float g = live ? gate[std::size_t(row) * ldg + head] : 0.0f;
  float maximum = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s)
    maximum = fmaxf(maximum, m[s]);
  float sum = 0.0f, acc[kCombineDims] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < kMaxSpans; ++s) {
    if (s < splits) {
      const float w = __builtin_amdgcn_exp2f(m[s] - maximum);
      sum = fmaf(l[s], w, sum);
#pragma unroll
      for (int i = 0; i < kCombineDims; ++i)
        acc[i] = fmaf(a[s][i], w, acc[i]);
    }
  }
  float o[kCombineDims], largest = 0.0f;
#pragma unroll
  for (int i = 0; i < kCombineDims; ++i) {
    o[i] = (acc[i] / sum) / (1.0f + expf(-g));
    largest = live ? fmaxf(largest, fabsf(o[i])) : largest;
  }
  largest = WaveMax(largest);
  if ((tid & 63) == 0)
    s_max[tid >> 6] = largest;
  __syncthreads();
  float row_max = 0.0f;
  for (int w = 0; w < int(blockDim.x) / 64; ++w)
    row_max = fmaxf(row_max, s_max[w]);
  const int e = RowExponent(row_max);
  if (tid == 0)
    scale[row] = ldexpf(1.0f, -e);
  if (live)
    *reinterpret_cast<uint2*>(out + std::size_t(row) * lda + head * D + d0) =
        make_uint2(unsigned(ScaledHalf(o[0], e)) | (unsigned(ScaledHalf(o[1], e)) << 16),
                   unsigned(ScaledHalf(o[2], e)) | (unsigned(ScaledHalf(o[3], e)) << 16));
}

struct PromptArgs {
  const float* q;
  int ldq;
  const Half* k;
  const Half* v;
  const float* gate;
  int ldg;
  const Half* ck;
  const Half* cv;
  float* out;
  int ldo;
  float* partial;
  int n, heads, kv_heads, position, capacity, window, span, splits;
  // FP16 rows out (partials for every span, merged by CombineRowsHalfKernel).
  Half* out16 = nullptr;
  int lda = 0;
  float* scale = nullptr;
};

// Long histories: two column tiles a wave (each K / V operand read feeds two
// MFMAs); windows and short histories: one, for more blocks.
int ColumnTiles(int position, int n, int window) {
  return window == 0 && position + n > 4096 ? 2 : 1;
}

// The span plan of one call: span length and count for the tile launch of
// the chosen shape (spans > 1 only for a history without a window).
int PlanCall(int n, int position, int window, int group, int kv_heads, int& span) {
  const int keys = position + n;
  span = keys;
  if (window)
    return 1;
  const int rows = 16 * ColumnTiles(position, n, window) * kPAWaves / group;
  const int blocks_per_span = (n + rows - 1) / rows * kv_heads;
  const int spans = SpanPlan(keys, blocks_per_span, span);
  if (spans == 1)
    span = keys;
  return spans;
}

template<int D, int G, int CT>
void LaunchTiles(const PromptArgs& a, hipStream_t s) {
  constexpr int kRows = 16 * CT * kPAWaves / G;
  const int row_blocks = (a.n + kRows - 1) / kRows;
  // 8 XCD slots of row_blocks blocks per group of 8 (span, KV head) pairs.
  const int pairs = a.splits * a.kv_heads;
  const int blocks = (pairs + 7) / 8 * 8 * row_blocks;
  PromptAttentionKernel<D, G, CT><<<blocks, kPAThreads, 0, s>>>(
      a.q, a.ldq, a.k, a.v, a.gate, a.ldg, a.ck, a.cv, a.out, a.ldo,
      a.splits > 1 || a.out16 ? a.partial : nullptr, a.n, a.heads, a.kv_heads, a.position,
      a.capacity,
      a.window, a.span, row_blocks, a.splits);
}

template<int D, int G>
void LaunchPrompt(const PromptArgs& a, hipStream_t s) {
  if (ColumnTiles(a.position, a.n, a.window) == 2)
    LaunchTiles<D, G, 2>(a, s);
  else
    LaunchTiles<D, G, 1>(a, s);
  if (a.out16) {
    const int threads = (a.heads * (D / kCombineDims) + 63) / 64 * 64;
    CombineRowsHalfKernel<D><<<a.n, threads, 0, s>>>(a.partial, a.gate, a.ldg, a.out16, a.lda,
                                                     a.scale, a.n, a.heads, a.splits);
  } else if (a.splits > 1) {
    CombineSpansKernel<D><<<a.n * a.heads, D, 0, s>>>(a.partial, a.gate, a.ldg, a.out, a.ldo,
                                                       a.n, a.heads, a.splits);
  }
}

template<int D>
void LaunchPromptGroup(const PromptArgs& a, int group, hipStream_t s) {
  if (group == 2)
    LaunchPrompt<D, 2>(a, s);
  else if (group == 4)
    LaunchPrompt<D, 4>(a, s);
  else
    LaunchPrompt<D, 8>(a, s);
}

// Spans any call of these sizes may use, whatever its head grouping.
int MostSpans(std::uint32_t position, std::uint32_t n, std::uint32_t window) {
  if (window)
    return 1;
  const int tiles = int((std::uint64_t(position) + n + kPAKeys - 1) / kPAKeys);
  return std::min(kMaxSpans, std::max(1, tiles / kSpanFloorTiles));
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

std::size_t lfm3_prompt_attention_workspace_bytes(std::uint32_t rows, std::uint32_t heads,
                                                  std::uint32_t dim, std::uint32_t position,
                                                  std::uint32_t window) {
  const int spans = MostSpans(position, rows, window);
  return spans > 1 ? std::size_t(spans) * rows * heads * (dim + 2) * sizeof(float) : 0;
}

std::size_t lfm3_prompt_attention_half_workspace_bytes(std::uint32_t rows, std::uint32_t heads,
                                                       std::uint32_t dim, std::uint32_t position,
                                                       std::uint32_t window) {
  return std::size_t(MostSpans(position, rows, window)) * rows * heads * (dim + 2) *
         sizeof(float);
}

}  // extern "C"

namespace lfm3amd {
namespace {
// lfm3_prompt_attention (out, ldo) and lfm3_prompt_attention_half (out16,
// lda, scale): one check and plan.
int PromptAttention(const float* q, std::uint32_t ldq, const std::uint16_t* k,
                    const std::uint16_t* v, const float* gate, std::uint32_t ldg,
                    const std::uint16_t* cache_k, const std::uint16_t* cache_v, float* out,
                    std::uint32_t ldo, std::uint16_t* out16, std::uint32_t lda, float* scale,
                    std::uint32_t rows, std::uint32_t heads, std::uint32_t kv_heads,
                    std::uint32_t dim, std::uint32_t position, std::uint32_t capacity,
                    std::uint32_t window, void* workspace, std::size_t workspace_bytes,
                    void* stream) {
  const std::uint32_t group = kv_heads ? heads / kv_heads : 0;
  const bool half = out16 != nullptr;
  if (half ? (!scale || lda % kChunk || lda < heads * dim || heads * dim / kCombineDims > 1024)
           : (!out || ldo < heads * dim || ldo % 4))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt attention output");
  if (!q || !k || !v || !gate || !rows || !heads || !kv_heads || heads % kv_heads ||
      (group != 2 && group != 4 && group != 8) || (dim != 64 && dim != 128) ||
      ldq < heads * dim || ldg < heads || ldq % 4 ||
      (position && (!cache_k || !cache_v || !capacity)) ||
      (!window && position && capacity < position) ||
      // A sliding row at `position` reads the ring's last min(window - 1,
      // position) keys; a shorter ring would have overwritten some of them.
      (window && position && capacity < std::min(window - 1, position)) ||
      std::uint64_t(position) + rows > (1ull << 31) ||
      !BufferFits(std::size_t(rows) * kv_heads * dim * 2) ||
      !BufferFits(std::size_t(capacity) * kv_heads * dim * 2))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt attention shape");
  PromptArgs a{};
  a.splits = PlanCall(int(rows), int(position), int(window), int(group), int(kv_heads), a.span);
  const std::size_t need = a.splits > 1 || half
                               ? std::size_t(a.splits) * rows * heads * (dim + 2) * sizeof(float)
                               : 0;
  if (need && (!workspace || workspace_bytes < need))
    return Fail(LFM3_E_INVALID, "LFM3 prompt attention workspace too small");
  a.q = q;
  a.ldq = int(ldq);
  a.k = k;
  a.v = v;
  a.gate = gate;
  a.ldg = int(ldg);
  a.ck = cache_k;
  a.cv = cache_v;
  a.out = out;
  a.ldo = int(ldo);
  a.out16 = out16;
  a.lda = int(lda);
  a.scale = scale;
  a.partial = static_cast<float*>(workspace);
  a.n = int(rows);
  a.heads = int(heads);
  a.kv_heads = int(kv_heads);
  a.position = int(position);
  a.capacity = int(capacity ? capacity : 1);
  a.window = int(window);
  const auto s = static_cast<hipStream_t>(stream);
  if (dim == 128)
    LaunchPromptGroup<128>(a, int(group), s);
  else
    LaunchPromptGroup<64>(a, int(group), s);
  return HipStatus(hipGetLastError(), "LFM3 prompt attention launch");
}
}  // namespace
}  // namespace lfm3amd

extern "C" {

int lfm3_prompt_attention(const float* q, std::uint32_t ldq, const std::uint16_t* k,
                          const std::uint16_t* v, const float* gate, std::uint32_t ldg,
                          const std::uint16_t* cache_k, const std::uint16_t* cache_v,
                          float* out, std::uint32_t ldo, std::uint32_t rows,
                          std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
                          std::uint32_t position, std::uint32_t capacity,
                          std::uint32_t window, void* workspace, std::size_t workspace_bytes,
                          void* stream) {
  if (!out)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt attention output");
  return PromptAttention(q, ldq, k, v, gate, ldg, cache_k, cache_v, out, ldo, nullptr, 0,
                         nullptr, rows, heads, kv_heads, dim, position, capacity, window,
                         workspace, workspace_bytes, stream);
}

int lfm3_prompt_attention_half(const float* q, std::uint32_t ldq, const std::uint16_t* k,
                               const std::uint16_t* v, const float* gate, std::uint32_t ldg,
                               const std::uint16_t* cache_k, const std::uint16_t* cache_v,
                               std::uint16_t* out, std::uint32_t lda, float* scale,
                               std::uint32_t rows, std::uint32_t heads, std::uint32_t kv_heads,
                               std::uint32_t dim, std::uint32_t position, std::uint32_t capacity,
                               std::uint32_t window, void* workspace,
                               std::size_t workspace_bytes, void* stream) {
  if (!out)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 prompt attention output");
  return PromptAttention(q, ldq, k, v, gate, ldg, cache_k, cache_v, nullptr, 0, out, lda, scale,
                         rows, heads, kv_heads, dim, position, capacity, window, workspace,
                         workspace_bytes, stream);
}

}  // extern "C"
