// CPU oracle for the LFM3 decode step: TEST INFRASTRUCTURE ONLY (see
// oracle.h). A scalar FP32 restatement of reference.cpp built with
// -ffp-contract=off so every expression rounds in source order, as the
// reference's own scalar loops do. Nothing here is shipped or called by the
// product library.
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <new>
#include <thread>
#include <vector>

namespace {

// Worker threads of one matrix-vector product or attention read (1: the
// reference's serial loops). Each output row or head is still one thread's
// sequential sum in the reference's order, so results do not depend on the
// count; only the wall time does.
std::atomic<unsigned> g_threads{1};

// Runs body(begin, end) over [0, n) split into contiguous ranges, one per
// worker (the calling thread takes the first).
template<class Body>
void Split(size_t n, Body body) {
  const unsigned workers = unsigned(std::min<size_t>(g_threads.load(), n));
  if (workers <= 1) {
    body(size_t(0), n);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(workers - 1);
  for (unsigned w = 1; w < workers; ++w)
    pool.emplace_back(body, n * w / workers, n * (w + 1) / workers);
  body(size_t(0), n / workers);
  for (auto& t : pool)
    t.join();
}

// Textbook IEEE binary16 decoding: sign, 5-bit exponent (bias 15), 10-bit
// fraction; exponent 0 is subnormal (fraction * 2^-24), 31 is Inf/NaN.
float HalfToFloat(uint16_t h) {
  const uint32_t sign = uint32_t(h >> 15) << 31;
  const uint32_t exponent = (h >> 10) & 31, fraction = h & 1023;
  uint32_t bits;
  if (exponent == 0) {
    if (fraction == 0) {
      bits = sign;
    } else {
      float value = std::ldexp(float(fraction), -24);
      std::memcpy(&bits, &value, 4);
      bits |= sign;
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (fraction << 13);
  } else {
    bits = sign | ((exponent + 112) << 23) | (fraction << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

// Round-to-nearest-even binary32 -> binary16, including subnormals,
// overflow to infinity and NaN preservation.
uint16_t FloatToHalf(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t abs = x & 0x7fffffffu;
  if (abs >= 0x7f800000u)  // Inf or NaN
    return sign | (abs > 0x7f800000u ? uint16_t(0x7e00u | ((abs >> 13) & 0x3ffu))
                                     : uint16_t(0x7c00u));
  const int exponent = int(abs >> 23) - 127;
  if (exponent > 15)
    return sign | 0x7c00u;
  uint32_t mantissa = (abs & 0x7fffffu) | 0x800000u;  // 24 significant bits
  int shift;                                          // bits dropped
  uint32_t base;
  if (exponent >= -14) {
    shift = 13;
    base = uint32_t(exponent + 15) << 10;
    mantissa &= 0x7fffffu;  // implicit bit lives in the exponent field
  } else {
    if (abs == 0)
      return sign;
    shift = 13 + (-14 - exponent);
    base = 0;
    if (shift > 24)
      return sign;  // below half the smallest subnormal
  }
  const uint32_t kept = mantissa >> shift;
  const uint32_t rest = mantissa & ((1u << shift) - 1);
  const uint32_t half = 1u << (shift - 1);
  uint32_t out = base + kept;
  if (rest > half || (rest == half && (kept & 1)))
    ++out;  // may carry into the exponent, which is the correct result
  return sign | uint16_t(out);
}

struct Q8Block {
  uint16_t d;
  int8_t q[32];
};
static_assert(sizeof(Q8Block) == 34, "Q8_0 block is 34 bytes");

// weights.cpp:101-125 (Q8_0 via ggml's d * q, F32 by copy, F16 and BF16
// widened).
bool DecodeRow(const orc_tensor& t, uint32_t row, float* out) {
  if (row >= t.rows)
    return false;
  if (t.type == ORC_F32) {
    std::memcpy(out, static_cast<const float*>(t.data) + size_t(row) * t.cols,
                size_t(t.cols) * 4);
    return true;
  }
  if (t.type == ORC_F16) {
    const auto* h = static_cast<const uint16_t*>(t.data) + size_t(row) * t.cols;
    for (uint32_t i = 0; i < t.cols; ++i)
      out[i] = HalfToFloat(h[i]);
    return true;
  }
  if (t.type == ORC_BF16) {  // weights.cpp:116-117: the high half of an FP32
    const auto* h = static_cast<const uint16_t*>(t.data) + size_t(row) * t.cols;
    for (uint32_t i = 0; i < t.cols; ++i) {
      const uint32_t bits = uint32_t(h[i]) << 16;
      std::memcpy(&out[i], &bits, 4);
    }
    return true;
  }
  if (t.type == ORC_Q8_0 && t.cols % 32 == 0) {
    const auto* blocks =
        static_cast<const Q8Block*>(t.data) + size_t(row) * (t.cols / 32);
    for (uint32_t b = 0; b < t.cols / 32; ++b) {
      const float d = HalfToFloat(blocks[b].d);
      for (int j = 0; j < 32; ++j)
        out[b * 32 + j] = d * float(blocks[b].q[j]);
    }
    return true;
  }
  return false;
}

bool Decodable(const orc_tensor& t) {
  return t.type == ORC_F32 || t.type == ORC_F16 || t.type == ORC_BF16 ||
         (t.type == ORC_Q8_0 && t.cols % 32 == 0);
}

// reference.cpp:9-19 over n input rows at once: each weight row is decoded
// once and dotted with every input row. Every output is still its own
// sequential sum over k in the reference's order (sum += w[k] * x[k], no
// contraction), so each row's result is bit-identical to Mat on that row;
// only the loop order across independent sums differs. Tiles of 16 weight
// rows x 64 input rows keep the operands in cache; the inputs are
// transposed so the inner loop runs across input rows (vectorizable).
bool MatRows(const orc_tensor& t, const float* x, uint32_t n, float* y) {
  if (!Decodable(t))
    return false;
  constexpr uint32_t kRows = 16, kCols = 64;
  const size_t K = t.cols;
  const uint32_t col_blocks = (n + kCols - 1) / kCols;
  std::vector<float> xt(K * size_t(col_blocks) * kCols, 0.0F);
  // xt[block][k][j] = x[block * 64 + j][k]
  for (uint32_t i = 0; i < n; ++i)
    for (size_t k = 0; k < K; ++k)
      xt[(size_t(i / kCols) * K + k) * kCols + i % kCols] = x[size_t(i) * K + k];
  const size_t row_blocks = (t.rows + kRows - 1) / kRows;
  Split(row_blocks, [&](size_t b0, size_t b1) {
    std::vector<float> rows(kRows * K);
    for (size_t b = b0; b < b1; ++b) {
      const uint32_t r0 = uint32_t(b * kRows);
      const uint32_t nr = std::min<uint32_t>(kRows, t.rows - r0);
      std::fill(rows.begin(), rows.end(), 0.0F);
      for (uint32_t rr = 0; rr < nr; ++rr)
        DecodeRow(t, r0 + rr, rows.data() + rr * K);
      for (uint32_t cb = 0; cb < col_blocks; ++cb) {
        const float* xb = xt.data() + size_t(cb) * K * kCols;
        const uint32_t nc = std::min<uint32_t>(kCols, n - cb * kCols);
        for (uint32_t rr0 = 0; rr0 < nr; rr0 += 4) {
          // 4 weight rows x 64 input rows of sums, held in registers.
          float acc[4][kCols] = {};
          const float* w0 = rows.data() + rr0 * K;
          for (size_t k = 0; k < K; ++k) {
            const float* xk = xb + k * kCols;
            for (uint32_t q = 0; q < 4; ++q) {
              const float w = w0[q * K + k];
              for (uint32_t j = 0; j < kCols; ++j)
                acc[q][j] += w * xk[j];
            }
          }
          for (uint32_t q = 0; q < 4 && rr0 + q < nr; ++q)
            for (uint32_t j = 0; j < nc; ++j)
              y[size_t(cb * kCols + j) * t.rows + r0 + rr0 + q] = acc[q][j];
        }
      }
    }
  });
  return true;
}

// reference.cpp:9-19.
bool Mat(const orc_tensor& t, const float* x, float* y) {
  if (t.type != ORC_F32 && t.type != ORC_F16 && t.type != ORC_BF16 &&
      !(t.type == ORC_Q8_0 && t.cols % 32 == 0))
    return false;
  Split(t.rows, [&](size_t r0, size_t r1) {
    std::vector<float> row(t.cols);
    for (size_t r = r0; r < r1; ++r) {
      DecodeRow(t, uint32_t(r), row.data());
      float sum = 0;
      for (uint32_t k = 0; k < t.cols; ++k)
        sum += row[k] * x[k];
      y[r] = sum;
    }
  });
  return true;
}

// reference.cpp:20-28.
void Norm(float* x, size_t n, const float* weight, float eps) {
  float sum = 0;
  for (size_t i = 0; i < n; ++i)
    sum += x[i] * x[i];
  const float scale = 1 / std::sqrt(sum / float(n) + eps);
  for (size_t i = 0; i < n; ++i)
    x[i] = x[i] * scale * weight[i];
}

// reference.cpp:29-43: pairs (i, i + D/2), angle = position * theta^(-2i/D),
// divided by the factor on global layers.
void Rope(float* x, size_t count, uint32_t D, uint32_t position, float theta,
          bool sliding, const float* factors) {
  for (size_t h = 0; h < count; ++h) {
    float* head = x + h * D;
    for (uint32_t i = 0; i < D / 2; ++i) {
      float angle = float(position) * std::pow(theta, -2.0F * float(i) / float(D));
      if (!sliding)
        angle /= factors[i];
      const float a = head[i], b = head[i + D / 2];
      head[i] = a * std::cos(angle) - b * std::sin(angle);
      head[i + D / 2] = b * std::cos(angle) + a * std::sin(angle);
    }
  }
}

// reference.cpp:85-101.
void ConvStep(const float* p, const float* taps, float* history, float* y,
              uint32_t H, uint32_t L) {
  for (uint32_t ch = 0; ch < H; ++ch) {
    float* own = history + size_t(ch) * (L - 1);
    const float bx = p[ch] * p[2 * H + ch];
    float sum = 0;
    for (uint32_t t = 0; t < L; ++t)
      sum += taps[ch * L + t] * (t + 1 == L ? bx : own[t]);
    for (uint32_t t = 1; t < L - 1; ++t)
      own[t - 1] = own[t];
    if (L > 1)
      own[L - 2] = bx;
    y[ch] = sum * p[H + ch];
  }
}

// reference.cpp:109-144 (the read half): gated GQA of one query row over
// ring keys [first, position].
void AttentionRead(const float* q, const float* gate, const float* ck,
                   const float* cv, uint32_t heads, uint32_t kv_heads,
                   uint32_t D, uint32_t position, uint32_t capacity,
                   uint32_t window, float* out) {
  const size_t stride = size_t(kv_heads) * D;
  const uint32_t first =
      window && position + 1 > window ? position + 1 - window : 0;
  // Every score is its own sequential sum over d, and every output element
  // its own sequential sum over t, exactly as in the reference's loops; the
  // loops are only nested so the inner one runs across independent sums
  // (16 keys, or the D output elements), which the compiler vectorizes.
  const uint32_t count = position + 1 - first;
  Split(heads, [&](size_t h0, size_t h1) {
    std::vector<float> scores(count), sums(D);
    constexpr uint32_t kKeys = 16;
    for (uint32_t h = uint32_t(h0); h < h1; ++h) {
      const uint32_t kh = h / (heads / kv_heads);
      const float* qh = q + size_t(h) * D;
      for (uint32_t t0 = 0; t0 < count; t0 += kKeys) {
        const uint32_t m = std::min(kKeys, count - t0);
        const float* rows[kKeys];
        float acc[kKeys];
        for (uint32_t j = 0; j < m; ++j) {
          rows[j] = ck + size_t((first + t0 + j) % capacity) * stride + kh * D;
          acc[j] = 0;
        }
        for (uint32_t d = 0; d < D; ++d)
          for (uint32_t j = 0; j < m; ++j)
            acc[j] += qh[d] * rows[j][d];
        for (uint32_t j = 0; j < m; ++j)
          scores[t0 + j] = acc[j] / std::sqrt(float(D));
      }
      float max = -std::numeric_limits<float>::infinity();
      for (uint32_t t = 0; t < count; ++t)
        max = std::max(max, scores[t]);
      float den = 0;
      for (auto& score : scores) {
        score = std::exp(score - max);
        den += score;
      }
      std::fill(sums.begin(), sums.end(), 0.0F);
      for (uint32_t t = 0; t < count; ++t) {
        const float p = scores[t] / den;
        const float* vt = cv + size_t((first + t) % capacity) * stride + kh * D;
        for (uint32_t d = 0; d < D; ++d)
          sums[d] += p * vt[d];
      }
      for (uint32_t d = 0; d < D; ++d)
        out[h * D + d] = sums[d] / (1 + std::exp(-gate[h]));
    }
  });
}


// The reference's prompt-path attention read (hip/ops.hip:1355-1561
// WmmaAttn for n > 1 rows): q scaled by log2(e) / sqrt(D) in FP32 and
// rounded to F16; scores are sums of the F16 query times the F16 keys in
// base-2 units; probabilities exp2(s - max) rounded to F16, their sum and
// the weighted values taken over the rounded probabilities; out =
// (sum_t p_t v_t / sum_t p_t) / (1 + e^-gate). (The kernel rounds each
// probability against the running maximum of its 64-key tile walk; this
// restatement uses the row's final maximum, which moves a probability by at
// most its rounding.) Keys as AttentionRead's.
void AttentionReadPrompt(const float* q, const float* gate, const float* ck,
                         const float* cv, uint32_t heads, uint32_t kv_heads,
                         uint32_t D, uint32_t position, uint32_t capacity,
                         uint32_t window, float* out) {
  const size_t stride = size_t(kv_heads) * D;
  const uint32_t first =
      window && position + 1 > window ? position + 1 - window : 0;
  const uint32_t count = position + 1 - first;
  const float scale = (1.0F / std::sqrt(float(D))) * 1.44269504088896341F;
  Split(heads, [&](size_t h0, size_t h1) {
    std::vector<float> scores(count), sums(D), qs(D);
    constexpr uint32_t kKeys = 16;
    for (uint32_t h = uint32_t(h0); h < h1; ++h) {
      const uint32_t kh = h / (heads / kv_heads);
      for (uint32_t d = 0; d < D; ++d)
        qs[d] = HalfToFloat(FloatToHalf(q[size_t(h) * D + d] * scale));
      for (uint32_t t0 = 0; t0 < count; t0 += kKeys) {
        const uint32_t m = std::min(kKeys, count - t0);
        const float* rows[kKeys];
        float acc[kKeys];
        for (uint32_t j = 0; j < m; ++j) {
          rows[j] = ck + size_t((first + t0 + j) % capacity) * stride + kh * D;
          acc[j] = 0;
        }
        for (uint32_t d = 0; d < D; ++d)
          for (uint32_t j = 0; j < m; ++j)
            acc[j] += qs[d] * rows[j][d];
        for (uint32_t j = 0; j < m; ++j)
          scores[t0 + j] = acc[j];
      }
      float max = -std::numeric_limits<float>::infinity();
      for (uint32_t t = 0; t < count; ++t)
        max = std::max(max, scores[t]);
      float den = 0;
      for (auto& score : scores) {
        score = HalfToFloat(FloatToHalf(std::exp2(score - max)));
        den += score;
      }
      std::fill(sums.begin(), sums.end(), 0.0F);
      for (uint32_t t = 0; t < count; ++t) {
        const float p = scores[t];
        const float* vt = cv + size_t((first + t) % capacity) * stride + kh * D;
        for (uint32_t d = 0; d < D; ++d)
          sums[d] += p * vt[d];
      }
      for (uint32_t d = 0; d < D; ++d)
        out[h * D + d] = (sums[d] / den) / (1 + std::exp(-gate[h]));
    }
  });
}

// reference.cpp:102-146: per-head norms, RoPE and the F16 ring store, then
// the read (the prompt path's with `prompt_read`).
void AttentionStep(float* q, float* k, const float* v, const float* gate,
                   const float* q_norm, const float* k_norm,
                   const float* factors, float* ck, float* cv, uint32_t heads,
                   uint32_t kv_heads, uint32_t D, uint32_t position,
                   uint32_t capacity, uint32_t window, float theta,
                   bool sliding, float eps, bool f16, bool prompt_read,
                   float* out) {
  for (uint32_t h = 0; h < heads; ++h)
    Norm(q + size_t(h) * D, D, q_norm, eps);
  for (uint32_t h = 0; h < kv_heads; ++h)
    Norm(k + size_t(h) * D, D, k_norm, eps);
  Rope(q, heads, D, position, theta, sliding, factors);
  Rope(k, kv_heads, D, position, theta, sliding, factors);
  const size_t stride = size_t(kv_heads) * D;
  const size_t slot = position % capacity;
  for (size_t i = 0; i < stride; ++i) {
    ck[slot * stride + i] = f16 ? HalfToFloat(FloatToHalf(k[i])) : k[i];
    cv[slot * stride + i] = f16 ? HalfToFloat(FloatToHalf(v[i])) : v[i];
  }
  (prompt_read ? AttentionReadPrompt : AttentionRead)(
      q, gate, ck, cv, heads, kv_heads, D, position, capacity,
      sliding ? window : 0, out);
}

// Trailing-row pruning (engine.cpp:304-323): a prompt chunk's last layers
// compute only the rows later layers read. Walking back from the last
// layer: a sliding layer keeps every row; a full-attention layer keeps only
// the rows needed after it (its K/V still come from every row); a
// convolution needs width - 1 earlier rows. Layer i reads live_in[i] rows
// and produces live_out[i] (the last rows of the chunk).
void PruneRows(const orc_config& c, uint32_t n, std::vector<uint32_t>& live_in,
               std::vector<uint32_t>& live_out) {
  live_in.assign(c.n_layers, n);
  live_out.assign(c.n_layers, n);
  uint32_t need = 1;
  for (uint32_t i = c.n_layers; i-- > 0;) {
    if (c.layer_type[i] == ORC_SLIDING)
      break;
    live_out[i] = std::min(n, need);
    if (c.layer_type[i] == ORC_FULL)
      break;
    need = std::min(n, need + c.conv_width - 1);
    live_in[i] = need;
  }
}
}  // namespace

struct orc_model {
  orc_config config{};
  std::vector<uint32_t> kv_heads;
  std::vector<uint8_t> layer_type;
  std::vector<orc_tensor> tensors;
  const orc_tensor& global(int i) const { return tensors[i]; }
  const orc_tensor& layer(uint32_t l, int i) const {
    return tensors[ORC_GLOBALS + size_t(l) * ORC_PER_LAYER + i];
  }
};

struct orc_session {
  orc_model* model{};
  uint32_t context{}, position{};
  bool f16{};
  struct State {
    std::vector<float> conv, k, v;
    uint32_t capacity{};
  };
  std::vector<State> states;
};

extern "C" {

void orc_set_threads(unsigned threads) { g_threads.store(std::max(1u, threads)); }
unsigned orc_threads(void) { return g_threads.load(); }
unsigned orc_hardware_concurrency(void) { return std::thread::hardware_concurrency(); }

float orc_half_to_float(uint16_t h) { return HalfToFloat(h); }
uint16_t orc_float_to_half(float f) { return FloatToHalf(f); }
void orc_halves_to_floats(const uint16_t* h, float* f, size_t n) {
  for (size_t i = 0; i < n; ++i)
    f[i] = HalfToFloat(h[i]);
}
void orc_floats_to_halves(const float* f, uint16_t* h, size_t n) {
  for (size_t i = 0; i < n; ++i)
    h[i] = FloatToHalf(f[i]);
}

int orc_decode_row(const orc_tensor* t, uint32_t row, float* out) {
  return DecodeRow(*t, row, out) ? 0 : -1;
}
int orc_mat(const orc_tensor* t, const float* x, float* y) {
  return Mat(*t, x, y) ? 0 : -1;
}
int orc_mat_batch(const orc_tensor* t, const float* x, float* y,
                  uint32_t batch) {
  if (batch == 0)
    return 0;
  return MatRows(*t, x, batch, y) ? 0 : -1;
}
void orc_norm(float* x, size_t n, const float* weight, float eps) {
  Norm(x, n, weight, eps);
}
void orc_rope(float* x, size_t count, uint32_t dim, uint32_t position,
              float theta, int sliding, const float* factors) {
  Rope(x, count, dim, position, theta, sliding != 0, factors);
}
void orc_conv_step(const float* p, const float* taps, float* history, float* y,
                   uint32_t hidden, uint32_t width) {
  ConvStep(p, taps, history, y, hidden, width);
}
void orc_attention_read(const float* q, const float* gate, const float* ck,
                        const float* cv, uint32_t heads, uint32_t kv_heads,
                        uint32_t dim, uint32_t position, uint32_t capacity,
                        uint32_t window, float* out) {
  AttentionRead(q, gate, ck, cv, heads, kv_heads, dim, position, capacity,
                window, out);
}
// reference.cpp:102-146.
void orc_attention_step(float* q, float* k, const float* v, const float* gate,
                        const float* q_norm, const float* k_norm,
                        const float* factors, float* ck, float* cv,
                        uint32_t heads, uint32_t kv_heads, uint32_t D,
                        uint32_t position, uint32_t capacity, uint32_t window,
                        float theta, int sliding, float eps, int f16,
                        float* out) {
  AttentionStep(q, k, v, gate, q_norm, k_norm, factors, ck, cv, heads, kv_heads,
                D, position, capacity, window, theta, sliding != 0, eps,
                f16 != 0, false, out);
}
void orc_attention_read_prompt(const float* q, const float* gate,
                               const float* ck, const float* cv,
                               uint32_t heads, uint32_t kv_heads, uint32_t dim,
                               uint32_t position, uint32_t capacity,
                               uint32_t window, float* out) {
  AttentionReadPrompt(q, gate, ck, cv, heads, kv_heads, dim, position,
                      capacity, window, out);
}
void orc_half_rows(const float* x, size_t rows, size_t cols, float* inputs,
                   int* exps) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    float maximum = 0;
    for (size_t k = 0; k < cols; ++k)
      maximum = std::max(maximum, std::fabs(row[k]));
    const int e = maximum > 0 ? 14 - std::ilogb(maximum) : 0;
    if (exps)
      exps[r] = e;
    for (size_t k = 0; k < cols; ++k)
      inputs[r * cols + k] =
          std::ldexp(HalfToFloat(FloatToHalf(std::ldexp(row[k], e))), -e);
  }
}

void orc_swiglu(float* gate, const float* up, size_t n) {
  for (size_t i = 0; i < n; ++i)
    gate[i] = (gate[i] / (1 + std::exp(-gate[i]))) * up[i];
}
uint32_t orc_argmax(const float* x, size_t n) {
  return uint32_t(std::max_element(x, x + n) - x);
}

uint32_t orc_sample(const float* logits, size_t n, float temperature, uint32_t top_k,
                    float repeat_penalty, const uint32_t* penalty_ids, size_t n_penalty,
                    float u) {
  std::vector<float> l(logits, logits + n);
  std::vector<bool> hit(n, false);
  for (size_t i = 0; i < n_penalty; ++i)
    if (penalty_ids[i] < n && !hit[penalty_ids[i]]) {
      hit[penalty_ids[i]] = true;
      float& v = l[penalty_ids[i]];
      v = v > 0 ? v / repeat_penalty : v * repeat_penalty;
    }
  if (!(temperature > 0) || top_k == 1)
    return uint32_t(std::max_element(l.begin(), l.end()) - l.begin());
  const float top = *std::max_element(l.begin(), l.end());
  std::vector<uint32_t> order(n);
  for (size_t i = 0; i < n; ++i)
    order[i] = uint32_t(i);
  size_t k = n;
  if (top_k != 0 && top_k < n) {
    k = top_k;
    std::stable_sort(order.begin(), order.end(),
                     [&](uint32_t a, uint32_t b) { return l[a] > l[b]; });
    order.resize(k);
  }
  const float inv_t = 1.0f / temperature;
  float total = 0;
  for (size_t i = 0; i < k; ++i)
    total += std::exp((l[order[i]] - top) * inv_t);
  const float target = u * total;
  float run = 0;
  size_t pick = 0;
  for (size_t i = 0; i < k; ++i) {
    const float w = std::exp((l[order[i]] - top) * inv_t);
    if (w > 0)
      pick = i;
    run += w;
    if (w > 0 && run > target)
      break;
  }
  return order[pick];
}

orc_model* orc_model_create(const orc_config* config, const orc_tensor* tensors,
                            size_t count) {
  if (!config || count != ORC_GLOBALS + size_t(config->n_layers) * ORC_PER_LAYER)
    return nullptr;
  auto* m = new (std::nothrow) orc_model;
  if (!m)
    return nullptr;
  m->config = *config;
  m->kv_heads.assign(config->kv_heads, config->kv_heads + config->n_layers);
  m->layer_type.assign(config->layer_type,
                       config->layer_type + config->n_layers);
  m->config.kv_heads = m->kv_heads.data();
  m->config.layer_type = m->layer_type.data();
  m->tensors.assign(tensors, tensors + count);
  return m;
}
void orc_model_destroy(orc_model* m) { delete m; }

orc_session* orc_session_create(orc_model* m, uint32_t context, int f16) {
  if (!m || !context || context > m->config.context)
    return nullptr;
  auto* s = new (std::nothrow) orc_session;
  if (!s)
    return nullptr;
  const auto& c = m->config;
  s->model = m;
  s->context = context;
  s->f16 = f16 != 0;
  s->states.resize(c.n_layers);
  for (uint32_t i = 0; i < c.n_layers; ++i) {
    auto& st = s->states[i];
    if (c.layer_type[i] == ORC_CONV) {
      st.conv.assign(size_t(c.hidden) * (c.conv_width - 1), 0.0F);
    } else {
      // reference.cpp:53-62: sliding rings hold min(context, window) rows.
      st.capacity = c.layer_type[i] == ORC_SLIDING ? std::min(context, c.window)
                                                   : context;
      st.k.assign(size_t(st.capacity) * c.kv_heads[i] * c.head_dim, 0.0F);
      st.v.assign(st.k.size(), 0.0F);
    }
  }
  return s;
}
void orc_session_destroy(orc_session* s) { delete s; }
void orc_session_reset(orc_session* s) {
  s->position = 0;
  for (auto& st : s->states) {
    std::fill(st.conv.begin(), st.conv.end(), 0.0F);
    std::fill(st.k.begin(), st.k.end(), 0.0F);
    std::fill(st.v.begin(), st.v.end(), 0.0F);
  }
}
uint32_t orc_session_position(const orc_session* s) { return s->position; }
void orc_session_set_position(orc_session* s, uint32_t position) {
  s->position = position;
}
uint32_t orc_session_capacity(const orc_session* s, uint32_t layer) {
  return s->states[layer].capacity;
}
float* orc_session_conv(orc_session* s, uint32_t layer) {
  return s->states[layer].conv.empty() ? nullptr : s->states[layer].conv.data();
}
float* orc_session_k(orc_session* s, uint32_t layer) {
  return s->states[layer].k.empty() ? nullptr : s->states[layer].k.data();
}
float* orc_session_v(orc_session* s, uint32_t layer) {
  return s->states[layer].v.empty() ? nullptr : s->states[layer].v.data();
}

// reference.cpp:72-168.
}  // extern "C"

namespace {

// reference.cpp:72-168 from the step's input row x0 (the token's embedding
// row, or a caller's row in place of it: Session::ForwardBatchInputs,
// engine.cpp:1217-1299, copies such a row over the embedding).
int Step(orc_session* s, const float* x0, float* logits, float* hidden) {
  const orc_model& m = *s->model;
  const auto& c = m.config;
  if (s->position >= s->context)
    return -1;
  const uint32_t H = c.hidden, D = c.head_dim;
  std::vector<float> x(x0, x0 + H), z(H), out(H);
  for (uint32_t il = 0; il < c.n_layers; ++il) {
    auto& st = s->states[il];
    z = x;
    Norm(z.data(), H, static_cast<const float*>(m.layer(il, ORC_L_NORM).data),
         c.eps);
    if (c.layer_type[il] == ORC_CONV) {
      std::vector<float> p(3 * H), conv(H);
      Mat(m.layer(il, ORC_L_IN_PROJ), z.data(), p.data());
      ConvStep(p.data(),
               static_cast<const float*>(m.layer(il, ORC_L_CONV).data),
               st.conv.data(), conv.data(), H, c.conv_width);
      Mat(m.layer(il, ORC_L_OUT_PROJ), conv.data(), out.data());
    } else {
      const uint32_t kv = c.kv_heads[il];
      std::vector<float> q(size_t(c.heads) * D), k(size_t(kv) * D),
          v(size_t(kv) * D), gate(c.heads), a(size_t(c.heads) * D);
      Mat(m.layer(il, ORC_L_Q), z.data(), q.data());
      Mat(m.layer(il, ORC_L_K), z.data(), k.data());
      Mat(m.layer(il, ORC_L_V), z.data(), v.data());
      Mat(m.layer(il, ORC_L_ATTN_GATE), z.data(), gate.data());
      const bool sliding = c.layer_type[il] == ORC_SLIDING;
      orc_attention_step(
          q.data(), k.data(), v.data(), gate.data(),
          static_cast<const float*>(m.layer(il, ORC_L_Q_NORM).data),
          static_cast<const float*>(m.layer(il, ORC_L_K_NORM).data),
          static_cast<const float*>(m.global(ORC_ROPE_FREQS).data),
          st.k.data(), st.v.data(), c.heads, kv, D, s->position, st.capacity,
          c.window, sliding ? c.theta_swa : c.theta, sliding, c.eps, s->f16,
          a.data());
      Mat(m.layer(il, ORC_L_ATTN_OUT), a.data(), out.data());
    }
    const auto& post = m.layer(il, ORC_L_POST_NORM);
    if (post.data)
      Norm(out.data(), H, static_cast<const float*>(post.data), c.eps);
    for (uint32_t i = 0; i < H; ++i)
      x[i] += out[i];
    z = x;
    Norm(z.data(), H,
         static_cast<const float*>(m.layer(il, ORC_L_FFN_NORM).data), c.eps);
    std::vector<float> gate(c.intermediate), up(c.intermediate);
    Mat(m.layer(il, ORC_L_GATE), z.data(), gate.data());
    Mat(m.layer(il, ORC_L_UP), z.data(), up.data());
    for (uint32_t i = 0; i < c.intermediate; ++i)
      gate[i] = (gate[i] / (1 + std::exp(-gate[i]))) * up[i];
    Mat(m.layer(il, ORC_L_DOWN), gate.data(), out.data());
    const auto& post_ffn = m.layer(il, ORC_L_POST_FFN_NORM);
    if (post_ffn.data)
      Norm(out.data(), H, static_cast<const float*>(post_ffn.data), c.eps);
    for (uint32_t i = 0; i < H; ++i)
      x[i] += out[i];
  }
  if (logits || hidden) {
    Norm(x.data(), H, static_cast<const float*>(m.global(ORC_OUTPUT_NORM).data),
         c.eps);
    if (hidden)
      std::copy(x.begin(), x.end(), hidden);
    if (logits)
      Mat(m.global(ORC_OUTPUT), x.data(), logits);
  }
  ++s->position;
  return 0;
}

// reference.cpp:72-168 applied to n input rows in order, one layer at a time
// (the reference steps them one token at a time). Every row's arithmetic is
// Step's: its norms, its products (MatRows gives each row Mat's sums), its
// convolution step and its attention step at position + i. Rows meet only
// through the session state (conv history, K/V ring), which each layer
// reads and writes in row order, as n steps would. So the final state and
// the last row's logits are bit-identical to n calls of Step.
//
// With `prompt` set (and n > 1), the chunk takes the reference's prompt-path
// numerics (Session::Forward's chunk of n rows, engine.cpp:257-527): a
// projection over 16 rows or more (hip/ops.hpp:32) reads its inputs as FP16
// row-scaled values (orc_half_rows, q8_prefill.hpp:27-51), fewer rows stay
// FP32; the rows each layer computes follow the trailing-row pruning rule
// (PruneRows), which decides those counts; attention reads through the
// prompt path's F16 arithmetic (AttentionReadPrompt), except a full-attention
// layer left with one live row, which reads as a decode row (FP32). Rows
// that pruning drops are still computed here; nothing reads them.
int Steps(orc_session* s, const float* x0, uint32_t n, float* logits,
          float* hidden, bool prompt) {
  const orc_model& m = *s->model;
  const auto& c = m.config;
  if (n == 0 || s->position > s->context || n > s->context - s->position)
    return -1;
  if (n == 1)
    prompt = false;  // a one-row chunk is a decode row
  const uint32_t H = c.hidden, D = c.head_dim, base = s->position;
  constexpr uint32_t kPromptRows = 16;
  std::vector<uint32_t> live_in, live_out;
  PruneRows(c, n, live_in, live_out);
  std::vector<float> x(x0, x0 + size_t(n) * H), z(x.size()), out(x.size());
  auto norm_rows = [&](std::vector<float>& rows, const orc_tensor& w) {
    for (uint32_t i = 0; i < n; ++i)
      Norm(rows.data() + size_t(i) * H, H, static_cast<const float*>(w.data),
           c.eps);
  };
  // A projection's input rows as the chunk's path feeds them.
  auto input = [&](std::vector<float>& rows, size_t cols, uint32_t live) {
    if (prompt && live >= kPromptRows)
      orc_half_rows(rows.data(), n, cols, rows.data(), nullptr);
    return rows.data();
  };
  for (uint32_t il = 0; il < c.n_layers; ++il) {
    auto& st = s->states[il];
    const uint32_t rows_in = live_in[il], rows_out = live_out[il];
    z = x;
    norm_rows(z, m.layer(il, ORC_L_NORM));
    input(z, H, rows_in);
    if (c.layer_type[il] == ORC_CONV) {
      std::vector<float> p(size_t(n) * 3 * H), conv(size_t(n) * H);
      MatRows(m.layer(il, ORC_L_IN_PROJ), z.data(), n, p.data());
      for (uint32_t i = 0; i < n; ++i)
        ConvStep(p.data() + size_t(i) * 3 * H,
                 static_cast<const float*>(m.layer(il, ORC_L_CONV).data),
                 st.conv.data(), conv.data() + size_t(i) * H, H, c.conv_width);
      MatRows(m.layer(il, ORC_L_OUT_PROJ), input(conv, H, rows_out), n,
              out.data());
    } else {
      const uint32_t kv = c.kv_heads[il];
      const size_t qn = size_t(c.heads) * D, kn = size_t(kv) * D;
      std::vector<float> q(n * qn), k(n * kn), v(n * kn), gate(size_t(n) * c.heads),
          a(n * qn);
      MatRows(m.layer(il, ORC_L_Q), z.data(), n, q.data());
      MatRows(m.layer(il, ORC_L_K), z.data(), n, k.data());
      MatRows(m.layer(il, ORC_L_V), z.data(), n, v.data());
      MatRows(m.layer(il, ORC_L_ATTN_GATE), z.data(), n, gate.data());
      const bool sliding = c.layer_type[il] == ORC_SLIDING;
      const bool prompt_read = prompt && !(rows_out == 1 && !sliding);
      for (uint32_t i = 0; i < n; ++i)
        AttentionStep(
            q.data() + i * qn, k.data() + i * kn, v.data() + i * kn,
            gate.data() + size_t(i) * c.heads,
            static_cast<const float*>(m.layer(il, ORC_L_Q_NORM).data),
            static_cast<const float*>(m.layer(il, ORC_L_K_NORM).data),
            static_cast<const float*>(m.global(ORC_ROPE_FREQS).data),
            st.k.data(), st.v.data(), c.heads, kv, D, base + i, st.capacity,
            c.window, sliding ? c.theta_swa : c.theta, sliding, c.eps, s->f16,
            prompt_read, a.data() + i * qn);
      MatRows(m.layer(il, ORC_L_ATTN_OUT), input(a, qn, rows_out), n, out.data());
    }
    const auto& post = m.layer(il, ORC_L_POST_NORM);
    if (post.data)
      norm_rows(out, post);
    for (size_t i = 0; i < x.size(); ++i)
      x[i] += out[i];
    z = x;
    norm_rows(z, m.layer(il, ORC_L_FFN_NORM));
    input(z, H, rows_out);
    std::vector<float> gate(size_t(n) * c.intermediate), up(gate.size());
    MatRows(m.layer(il, ORC_L_GATE), z.data(), n, gate.data());
    MatRows(m.layer(il, ORC_L_UP), z.data(), n, up.data());
    for (size_t i = 0; i < gate.size(); ++i)
      gate[i] = (gate[i] / (1 + std::exp(-gate[i]))) * up[i];
    MatRows(m.layer(il, ORC_L_DOWN), input(gate, c.intermediate, rows_out), n,
            out.data());
    const auto& post_ffn = m.layer(il, ORC_L_POST_FFN_NORM);
    if (post_ffn.data)
      norm_rows(out, post_ffn);
    for (size_t i = 0; i < x.size(); ++i)
      x[i] += out[i];
  }
  if (logits || hidden) {
    float* last = x.data() + size_t(n - 1) * H;
    Norm(last, H, static_cast<const float*>(m.global(ORC_OUTPUT_NORM).data),
         c.eps);
    if (hidden)
      std::copy(last, last + H, hidden);
    if (logits)
      Mat(m.global(ORC_OUTPUT), last, logits);
  }
  s->position += n;
  return 0;
}

}  // namespace

extern "C" {

int orc_session_step(orc_session* s, uint32_t token, float* logits,
                     float* hidden) {
  const orc_model& m = *s->model;
  if (token >= m.config.vocab || s->position >= s->context)
    return -1;
  std::vector<float> x(m.config.hidden);
  DecodeRow(m.global(ORC_EMBEDDING), token, x.data());
  return Step(s, x.data(), logits, hidden);
}

int orc_session_step_row(orc_session* s, const float* row, float* logits,
                         float* hidden) {
  if (!row)
    return -1;
  return Step(s, row, logits, hidden);
}

int orc_session_steps_rows(orc_session* s, const float* rows, uint32_t n,
                           float* logits, float* hidden, int prompt_path) {
  if (!rows || n == 0)
    return -1;
  return Steps(s, rows, n, logits, hidden, prompt_path != 0);
}

int orc_session_steps(orc_session* s, const uint32_t* tokens, uint32_t n,
                      float* logits, float* hidden, int prompt_path) {
  const orc_model& m = *s->model;
  if (!tokens || n == 0)
    return -1;
  std::vector<float> x(size_t(n) * m.config.hidden);
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] >= m.config.vocab ||
        !DecodeRow(m.global(ORC_EMBEDDING), tokens[i],
                   x.data() + size_t(i) * m.config.hidden))
      return -1;
  return Steps(s, x.data(), n, logits, hidden, prompt_path != 0);
}

}  // extern "C"
