/*
 * CPU oracle for the LFM3 decode step: TEST INFRASTRUCTURE ONLY.
 *
 * A scalar FP32 restatement of the reference's one-token step
 * (reference.cpp:72-168) and of the row decoding it relies on
 * (weights.cpp:101-125), plus the two additions the GPU contract needs:
 *   - state injection: a session can start at any position with caller-filled
 *     convolution history and K/V rings (the reference only starts from zero);
 *   - an F16 switch that rounds the stored K/V row to IEEE binary16, as the
 *     GPU cache does (engine.cpp:60-77 allocates F16 rings; ops.hip stores
 *     with round-to-nearest-even).
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline may load
 * this library; the product never links it.
 *
 * Tensors use the GGUF layouts the reference binds (weights.hpp:7-12):
 * Q8_0 rows of 34-byte blocks (fp16 d, 32 x int8) or F32.
 */
#ifndef LFM3_ORACLE_H_
#define LFM3_ORACLE_H_
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_BF16 = 30 };
enum { ORC_CONV = 0, ORC_FULL = 1, ORC_SLIDING = 2 };

typedef struct {
  uint32_t hidden, intermediate, vocab, context, heads, head_dim, window,
      conv_width, n_layers;
  float eps, theta, theta_swa;
  const uint32_t* kv_heads;  /* per layer; 0 for convolution layers */
  const uint8_t* layer_type; /* ORC_CONV / ORC_FULL / ORC_SLIDING */
} orc_config;

typedef struct {
  const void* data;
  uint32_t type; /* ORC_F32 or ORC_Q8_0 */
  uint32_t cols, rows;
} orc_tensor;

/* Global tensors then 17 per layer, in weights.hpp:13-22 order. */
enum {
  ORC_EMBEDDING = 0,
  ORC_OUTPUT,
  ORC_OUTPUT_NORM,
  ORC_ROPE_FREQS,
  ORC_GLOBALS
};
enum {
  ORC_L_NORM = 0,
  ORC_L_FFN_NORM,
  ORC_L_POST_NORM,
  ORC_L_POST_FFN_NORM,
  ORC_L_GATE,
  ORC_L_UP,
  ORC_L_DOWN,
  ORC_L_CONV,
  ORC_L_IN_PROJ,
  ORC_L_OUT_PROJ,
  ORC_L_Q,
  ORC_L_K,
  ORC_L_V,
  ORC_L_Q_NORM,
  ORC_L_K_NORM,
  ORC_L_ATTN_GATE,
  ORC_L_ATTN_OUT,
  ORC_PER_LAYER
};

typedef struct orc_model orc_model;
typedef struct orc_session orc_session;

/* IEEE binary16 <-> binary32, round to nearest even. */
/* Worker threads per matrix-vector product (rows split into contiguous
   ranges) and per attention read (heads split): 1, the default, is the
   reference's serial loop. Every output row and head keeps its sequential
   sum, so results are identical for any count; process-wide. */
void orc_set_threads(unsigned threads);
unsigned orc_threads(void);
/* std::thread::hardware_concurrency() of the host. */
unsigned orc_hardware_concurrency(void);

float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);
void orc_halves_to_floats(const uint16_t* h, float* f, size_t n);
void orc_floats_to_halves(const float* f, uint16_t* h, size_t n);

/* weights.cpp:101-125: one decoded row of a tensor. */
int orc_decode_row(const orc_tensor* t, uint32_t row, float* out);
/* reference.cpp:9-19: y[r] = sequential FP32 sum of row[k] * x[k]. */
int orc_mat(const orc_tensor* t, const float* x, float* y);
/* Mat over `batch` input rows (row-major [batch][cols] -> [batch][rows]). */
int orc_mat_batch(const orc_tensor* t, const float* x, float* y,
                  uint32_t batch);
/* reference.cpp:20-28, in place over n values. */
void orc_norm(float* x, size_t n, const float* weight, float eps);
/* reference.cpp:29-43 over `count` heads of dim values (factors may be NULL
   for sliding layers). */
void orc_rope(float* x, size_t count, uint32_t dim, uint32_t position,
              float theta, int sliding, const float* factors);
/* reference.cpp:85-101: one decode row of the gated short convolution.
   p = [B | C | x] (3*hidden), history [hidden][width-1], y [hidden]. */
void orc_conv_step(const float* p, const float* taps, float* history,
                   float* y, uint32_t hidden, uint32_t width);
/* reference.cpp:102-146: per-head q/k norm, RoPE, K/V store at slot
   position % capacity, gated GQA over keys [first, position]. q [heads*dim],
   k/v [kv_heads*dim] are consumed (normed/rotated in place). With f16 set
   the stored K/V row is rounded to binary16. out [heads*dim]. */
void orc_attention_step(float* q, float* k, const float* v,
                        const float* gate, const float* q_norm,
                        const float* k_norm, const float* factors,
                        float* cache_k, float* cache_v, uint32_t heads,
                        uint32_t kv_heads, uint32_t dim, uint32_t position,
                        uint32_t capacity, uint32_t window, float theta,
                        int sliding, float eps, int f16, float* out);
/* The attention read alone (keys [first, position] of the ring, no store,
   no norm/RoPE): ops_test.cpp's operator contract at n == 1. */
void orc_attention_read(const float* q, const float* gate,
                        const float* cache_k, const float* cache_v,
                        uint32_t heads, uint32_t kv_heads, uint32_t dim,
                        uint32_t position, uint32_t capacity, uint32_t window,
                        float* out);
/* Prompt-path activations (hip/q8_prefill.hpp:27-51, as tests/ops_test.cpp
   :55-68 restates them): per row e = 14 - ilogb(max |x|) (0 for a zero
   row); inputs[k] = ldexp(float(binary16(ldexp(x[k], e))), -e). Writes the
   effective inputs and, when exps is not NULL, e per row. */
void orc_half_rows(const float* x, size_t rows, size_t cols, float* inputs,
                   int* exps);
/* reference.cpp:151-160 SwiGLU: (g / (1 + exp(-g))) * u. */
void orc_swiglu(float* gate, const float* up, size_t n);
/* First index of the maximum (std::max_element). */
uint32_t orc_argmax(const float* x, size_t n);
/* Token selection of the serving loop (SelectNext, runner.cpp:300-325;
   defaults temperature 0.1, top_k 50, repeat_penalty 1.1 at
   runner.cpp:31-35). The reference's sampler (Gufo's
   sampling::SamplerState) is not vendored, so this follows the common
   definition, step by step:
   repetition penalty over penalty_ids (l -> l / p if l > 0 else l * p,
   once per listed id < n), the top_k largest (ties: lower index; 0 or
   >= n keeps all), weights exp((l - max) / T) in float, then the first
   candidate (descending logit order, or index order when all are kept)
   whose running float sum exceeds u * total. T <= 0 or top_k == 1: the
   first index of the maximum. Parity unpinned against the Gufo sampler
   itself; pinned by the greedy cases and by frequency/closed-form checks
   in the tests. */
uint32_t orc_sample(const float* logits, size_t n, float temperature,
                    uint32_t top_k, float repeat_penalty,
                    const uint32_t* penalty_ids, size_t n_penalty, float u);

orc_model* orc_model_create(const orc_config* config,
                            const orc_tensor* tensors, size_t count);
void orc_model_destroy(orc_model* m);

/* A session with its own state; f16 rounds stored K/V rows (GPU contract). */
orc_session* orc_session_create(orc_model* m, uint32_t context, int f16);
void orc_session_destroy(orc_session* s);
void orc_session_reset(orc_session* s);
uint32_t orc_session_position(const orc_session* s);
void orc_session_set_position(orc_session* s, uint32_t position);
uint32_t orc_session_capacity(const orc_session* s, uint32_t layer);
/* Mutable state views: conv history [hidden][width-1] f32; K/V rings
   [capacity][kv_heads][dim] f32 (binary16-exact values when f16 is set). */
float* orc_session_conv(orc_session* s, uint32_t layer);
float* orc_session_k(orc_session* s, uint32_t layer);
float* orc_session_v(orc_session* s, uint32_t layer);
/* reference.cpp:72-168. Returns 0, or -1 on an invalid step (token out of
   range or context exhausted), leaving state untouched. logits may be NULL.
   hidden (may be NULL) receives the final-normed row. */
int orc_session_step(orc_session* s, uint32_t token, float* logits,
                     float* hidden);
/* The same step from a caller's FP32 input row (hidden floats) in place of
   the token's embedding row (Session::ForwardBatchInputs,
   engine.cpp:1217-1299). hidden receives the final-normed row whenever it
   is not NULL. */
int orc_session_step_row(orc_session* s, const float* row, float* logits,
                         float* hidden);
/* n tokens in order (a prompt), computed one layer at a time over all n
   rows: bit-identical to n calls of orc_session_step (each row's arithmetic
   is the step's; the state is read and written in row order). logits and
   hidden (each may be NULL) receive the last row's. Returns -1, leaving the
   state untouched, for n = 0, a token out of range or too short a context.
   With prompt_path set and n > 1, the n rows are one prompt chunk with the
   reference's prompt-path numerics (engine.cpp:257-527): projections over
   16 rows or more read FP16 row-scaled inputs (orc_half_rows), the rows a
   layer computes follow trailing-row pruning (engine.cpp:304-323), and
   attention reads through orc_attention_read_prompt except a full-attention
   layer left with one row, which reads as a decode row. */
int orc_session_steps(orc_session* s, const uint32_t* tokens, uint32_t n,
                      float* logits, float* hidden, int prompt_path);
/* The same from n caller FP32 input rows (n * hidden floats) in place of
   the tokens' embedding rows (Session::ForwardEmbeddings). */
int orc_session_steps_rows(orc_session* s, const float* rows, uint32_t n,
                           float* logits, float* hidden, int prompt_path);
/* The prompt path's attention read (hip/ops.hip:1355-1561): q scaled by
   log2(e)/sqrt(D) and rounded to F16, base-2 scores over the F16 query,
   probabilities exp2(s - max) rounded to F16, summed and applied as
   rounded; keys and output as orc_attention_read. */
void orc_attention_read_prompt(const float* q, const float* gate,
                               const float* ck, const float* cv,
                               uint32_t heads, uint32_t kv_heads, uint32_t dim,
                               uint32_t position, uint32_t capacity,
                               uint32_t window, float* out);

#ifdef __cplusplus
}
#endif
#endif
