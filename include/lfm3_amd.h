/*
 * lfm3_amd: the C-ABI boundary of the MI355X (gfx950) LFM3 continuous
 * batching step. Plain pointers, sizes and hipStream_t (passed as void*);
 * every call returns LFM3_OK or a negative status, with the message kept
 * per thread (lfm3_last_error). Kernel entry points are stream-ordered and
 * own nothing: weights, activations, state and workspaces are passed in,
 * as with the reference's ops (hip/ops.hpp:12-151).
 *
 * Status mapping to the reference's conventions:
 *   LFM3_E_INVALID  std::invalid_argument for unsupported shapes/inputs
 *                   (hip/ops.hip:2293-2294, 2402-2403; engine.cpp:908-914)
 *   LFM3_E_HIP      std::runtime_error(hipGetErrorString) from Check
 *                   (engine.cpp:23-26)
 *   LFM3_E_STATE    a poisoned session, which refuses work until Reset
 *                   (engine.cpp:905-907)
 */
#ifndef LFM3_AMD_H_
#define LFM3_AMD_H_
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define LFM3_OK 0
#define LFM3_E_INVALID (-1)
#define LFM3_E_HIP (-2)
#define LFM3_E_STATE (-3)
#define LFM3_E_NOMEM (-4)
/* A continuation hook refused the call (continuation_hooks.hpp:6-15: a
   hook may throw to refuse); nothing changed. */
#define LFM3_E_REFUSED (-5)

/* Message of the last failed call on this thread ("" if none). */
const char* lfm3_last_error(void);

/* ---------------------------------------------------------------------
 * Q8_0 weights in the device tile layout.
 *
 * GGUF Q8_0 rows (34-byte blocks: fp16 d, 32 x int8 q; weights.cpp:101-125)
 * are repacked once at load into tiles of 16 rows x 64 columns: 1024 code
 * bytes + 32 fp16 scales per tile, rows padded to 16 and columns to 64 with
 * zero codes and zero scales. Codes and scales are separate arrays.
 * Replaces: DeviceWeights::Add/Upload (upload.cpp:29-72), which copies the
 * GGUF bytes verbatim.
 * ------------------------------------------------------------------- */
/* Bytes of the tiled codes and scales of a rows x cols matrix. */
void lfm3_q8_tiled_bytes(uint32_t rows, uint32_t cols, size_t* code_bytes,
                         size_t* scale_bytes);
/* Host repack of GGUF Q8_0 rows into tiles. Source row tile i goes to
   destination row tile (tile_offset + i * tile_stride): stride 1 with an
   offset concatenates matrices; stride 2 interleaves two (FFN gate/up).
   cols must be a multiple of 32. */
int lfm3_q8_pack_host(const void* gguf, uint32_t rows, uint32_t cols,
                      void* codes, void* scales, uint32_t tile_offset,
                      uint32_t tile_stride);
/* The same repack on the device, from GGUF bytes already uploaded. */
int lfm3_q8_pack_device(const void* gguf, uint32_t rows, uint32_t cols,
                        void* codes, void* scales, uint32_t tile_offset,
                        uint32_t tile_stride, void* stream);

/* ---------------------------------------------------------------------
 * Q8_0 skinny GEMV for 1..8 FP32 rows: y[b][r] = sum_k W[r][k] x[b][k].
 * Replaces: gpu::LaunchGEMV (hip/ops.hip:1799-1825, B = 1) and
 * gpu::LaunchBatchedQuantGEMMFp32 (hip/ops.hip:1827-1915, B = 2..8), the
 * decode projections behind gpu::Dense / gpu::Project (hip/ops.hpp:44-64).
 * x: batch rows of ldx floats (ldx % 4 == 0, 16-byte aligned); y: batch
 * rows of ldy floats. Every block covers the whole of K, so no call needs
 * a workspace (lfm3_gemv_workspace_bytes returns 0; the arguments stay for
 * callers that pass one).
 * ------------------------------------------------------------------- */
size_t lfm3_gemv_workspace_bytes(uint32_t rows, uint32_t cols,
                                 uint32_t batch);
int lfm3_q8_gemv(const void* codes, const void* scales, uint32_t rows,
                 uint32_t cols, const float* x, uint32_t ldx, float* y,
                 uint32_t ldy, uint32_t batch, void* workspace,
                 size_t workspace_bytes, void* stream);
/* The same products split over K into `parts` contiguous ranges, one grid
   row of blocks each: part p writes its partial sums to y + p * batch *
   ldy (rows of ldy floats), and the consumer adds the parts in part order
   (lfm3_residual_norm_parts). No merge happens inside the launch, so
   narrow matrices fill the device without a device-scope fence.
   lfm3_q8_gemv_parts gives the number of parts (at most 8) this library
   picks for a shape (1 when one range fills the device).
   Replaces: the split-K tail of gpu::LaunchSplit (hip/ops.hip:2039-2069),
   which merges partial sums in the last block of each tile. */
uint32_t lfm3_q8_gemv_parts(uint32_t rows, uint32_t cols);
int lfm3_q8_gemv_partials(const void* codes, const void* scales, uint32_t rows,
                          uint32_t cols, const float* x, uint32_t ldx, float* y,
                          uint32_t ldy, uint32_t batch, uint32_t parts,
                          void* stream);
/* GEMV operand images. A producer that holds whole FP32 rows of x can
   hand them to the next GEMV already staged as its MFMA A operand: per
   token an exponent e (x = (hi + lo 2^-11) 2^-e, e puts the row maximum
   in [2^14, 2^15)), hi = fp16(x 2^e), lo = fp16((x 2^e - hi) 2^11), both
   truncated, laid out per 64-column chunk c and Q8_0 block b as 64 16-byte
   lane words at ((c * 2 + b) * 64 + L), lane L = 16 g + m holding elements
   8g..8g+7 of the block for A row m (m < 8: token m's hi part, m >= 8:
   token m - 8's lo part). exps holds 8 ints. The GEMV then reads its
   operands from L2 with no per-block staging; its result equals
   lfm3_q8_gemv on the same rows up to the order in which chunk sums add.
   No counterpart in the reference (its decode GEMVs read FP32 rows,
   hip/ops.hip:671-856). */
size_t lfm3_operand_image_bytes(uint32_t cols);
int lfm3_q8_gemv_image(const void* codes, const void* scales, uint32_t rows,
                       uint32_t cols, const void* image, const int* exps,
                       uint32_t batch, float* y, uint32_t ldy, uint32_t parts,
                       void* stream);
int lfm3_q8_gemv_swiglu_image(const void* codes, const void* scales,
                              uint32_t rows, uint32_t cols, const void* image,
                              const int* exps, uint32_t batch, float* y,
                              uint32_t ldy, void* stream);
/* The convolution block's in projection ([3 hidden x hidden], rows B | C |
   X in the usual tiled layout) on an operand image, with the decode
   convolution step in its epilogue: y[b][ch] and the history of row b
   (history[b], [hidden][width - 1]) as lfm3_conv_step_ragged leaves them
   after the projection (the step's expressions and order; the projection's
   chunk sums add in 16-wave order). hidden % 16 == 0, batch <= 8.
   Replaces: gpu::Project of in_proj then gpu::ShortConv for n == 1
   (engine.cpp:386-393, hip/ops.hip:2250-2264). */
int lfm3_q8_gemv_conv_image(const void* codes, const void* scales,
                            uint32_t hidden, const void* image, const int* exps,
                            uint32_t batch, const float* taps,
                            float* const* history, uint32_t width, float* y,
                            uint32_t ldy, void* stream);
/* FFN gate/up with the SwiGLU epilogue over a stride-2 interleaved pair
   (rows = rows of each of gate and up): y[b][r] = silu(g) * u.
   Replaces: gpu::ProjectSwiGLU (hip/ops.hip:2187-2204) and the decode half
   of gpu::ProjectFfn (hip/ops.hip:2205-2229). */
int lfm3_q8_gemv_swiglu(const void* codes, const void* scales, uint32_t rows,
                        uint32_t cols, const float* x, uint32_t ldx, float* y,
                        uint32_t ldy, uint32_t batch, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * Float weights (BF16, F16, F32): exact products with FP32 inputs. BF16 is
 * the reference precision (README.md:24-27); F16 and F32 are the other
 * float formats the reference binds (weights.cpp:30-37).
 *
 * `type` is LFM3_TYPE_BF16, LFM3_TYPE_F16 or LFM3_TYPE_F32. GGUF rows are
 * repacked at load into tiles of 16 rows x 32 columns (lane L = 16 g + n
 * holds row n, columns 8g..8g+7: one 1 KB plane for the 16-bit formats;
 * two for F32, columns 8g..8g+3 then 8g+4..8g+7), rows padded to 16 and
 * columns to 32 with zeros; the tile offset / stride arguments work as for
 * lfm3_q8_pack_host. The GEMV splits each FP32 input exactly into three
 * BF16 parts (hi + mid + lo) and each weight into one (BF16), two (F16) or
 * three (F32) BF16 parts, so that every product is exact on the BF16
 * matrix cores; sums are FP32 in block order. Any batch (tokens in groups
 * of 16); cols % 32 == 0, ldx % 4 == 0, x 16-byte aligned. parts > 1
 * splits K as lfm3_q8_gemv_partials does (part p at y + p * batch * ldy);
 * lfm3_bf16_gemv_parts gives this library's choice for any float type.
 * swiglu: the tiles hold gate/up pairs (tile stride 2), rows is the rows
 * of each, and y = silu(gate) * up (parts must be 1).
 * Replaces: gpu::LaunchExactBf16GEMMFp32SmallBatch (hip/ops.hip:1917-2005),
 * F16Dense (hip/ops.hip:876-890), the F32 / F16 / BF16 branches of
 * gpu::LaunchGEMV (hip/ops.hip:1799-1825) and of gpu::Dense
 * (hip/ops.hip:2230-2249).
 * ------------------------------------------------------------------- */
/* 0 for a type that is not a float format. */
size_t lfm3_float_tiled_bytes(uint32_t type, uint32_t rows, uint32_t cols);
int lfm3_float_pack_host(uint32_t type, const void* src, uint32_t rows,
                         uint32_t cols, void* tiles, uint32_t tile_offset,
                         uint32_t tile_stride);
uint32_t lfm3_bf16_gemv_parts(uint32_t rows, uint32_t cols, uint32_t batch);
int lfm3_float_gemv(uint32_t type, const void* tiles, uint32_t rows,
                    uint32_t cols, const float* x, uint32_t ldx, float* y,
                    uint32_t ldy, uint32_t batch, uint32_t parts, int swiglu,
                    void* stream);
/* out[i] = row tokens[i] of a tiled table as FP32 (vocab rows of cols), or
   inputs[i] (device FP32 rows) where the device pointer table inputs (may
   be NULL) has an entry. Ids >= vocab give zero rows.
   Replaces: gpu::Embedding on an F32, F16 or BF16 table
   (hip/ops.hip:858-875). */
int lfm3_float_embed(uint32_t type, const void* tiles, uint32_t vocab,
                     uint32_t cols, const uint32_t* tokens,
                     const float* const* inputs, uint32_t n, float* out,
                     void* stream);
/* The BF16 forms of the above (type LFM3_TYPE_BF16). */
size_t lfm3_bf16_tiled_bytes(uint32_t rows, uint32_t cols);
int lfm3_bf16_pack_host(const void* src, uint32_t rows, uint32_t cols,
                        void* tiles, uint32_t tile_offset, uint32_t tile_stride);
int lfm3_bf16_gemv(const void* tiles, uint32_t rows, uint32_t cols,
                   const float* x, uint32_t ldx, float* y, uint32_t ldy,
                   uint32_t batch, uint32_t parts, int swiglu, void* stream);
int lfm3_bf16_embed(const void* tiles, uint32_t vocab, uint32_t cols,
                    const uint32_t* tokens, const float* const* inputs,
                    uint32_t n, float* out, void* stream);

/* ---------------------------------------------------------------------
 * Prompt projections (n >= 16 rows of one session) on MFMA.
 * ------------------------------------------------------------------- */
/* FP16 row-scaled activations (hip/q8_prefill.hpp:27-74): per row
   e = 14 - ilogb(max |x|) (0 for a zero row), out = fp16(x 2^e), scale =
   2^-e. out rows have lda halves (lda % 64 == 0, lda >= cols); columns
   [cols, cols rounded up to 64) are zeroed (the GEMM's last chunk), later
   ones are not written. With row_max (max_blocks partial maxima of each row as FP32
   bits, row_max[b * rows + row], e.g. from lfm3_q8_gemm_swiglu) the row
   scan is skipped. Replaces: HalfRows / HalfRowsFromMax
   (q8_prefill.hpp:30-74). */
int lfm3_half_rows(const float* x, uint32_t ldx, const unsigned* row_max,
                   uint32_t max_blocks, uint16_t* out, uint32_t lda,
                   float* scale, uint32_t rows, uint32_t cols, void* stream);
/* Y[t][r] = scale[t] * sum over Q8_0 blocks of d * (exact code x fp16 dot
   in FP32), one FP32 fma per block; tokens rows of activations a (lda
   halves each, chunk tails zero) with their scales. K splits into `parts`
   (1..8) ranges written to y + p * tokens * ldy; the consumer adds the
   parts in part order. lfm3_q8_gemm_parts gives this library's choice.
   Replaces: gpu::Project / gpu::Dense for prompt rows (LaunchSplit,
   hip/ops.hip:2019-2119; RegQ8Gemm, q8_prefill.hpp:415-645). */
uint32_t lfm3_q8_gemm_parts(uint32_t rows, uint32_t cols, uint32_t tokens,
                            int swiglu);
int lfm3_q8_gemm(const void* codes, const void* scales, uint32_t rows,
                 uint32_t cols, const uint16_t* a, uint32_t lda,
                 const float* a_scale, uint32_t tokens, float* y, uint32_t ldy,
                 uint32_t parts, void* stream);
/* Adds K parts 1..parts-1 of a lfm3_q8_gemm output into part 0 in part
   order: y[r][c] += y[p][r][c] for p = 1.. (part_stride floats apart; row
   stride ld). For consumers that read one FP32 row (convolution, heads).
   Replaces: the deterministic split-K merge of LaunchSplit
   (hip/ops.hip:2019-2119). */
int lfm3_sum_parts(float* y, size_t part_stride, uint32_t rows, uint32_t cols,
                   uint32_t ld, uint32_t parts, void* stream);
/* Gate/up over a stride-2 interleaved pair with the SwiGLU epilogue
   (q8_prefill.hpp:622-635): y = silu(g) * u, and each token row's max |y|
   (FP32 bits) over each block of output rows stored to row_max[b * tokens
   + t], b < lfm3_q8_gemm_swiglu_max_blocks(rows) (NULL: skipped; plain
   stores, no zeroing needed): the partial maxima lfm3_half_rows reduces.
   The reference forms the same row maxima with atomicMax.
   Replaces: gpu::ProjectFfn's first half for prompt rows
   (hip/ops.hip:2205-2222). */
uint32_t lfm3_q8_gemm_swiglu_max_blocks(uint32_t rows);
int lfm3_q8_gemm_swiglu(const void* codes, const void* scales, uint32_t rows,
                        uint32_t cols, const uint16_t* a, uint32_t lda,
                        const float* a_scale, uint32_t tokens, float* y,
                        uint32_t ldy, unsigned* row_max, void* stream);
/* lfm3_q8_gemm_swiglu_h16 with the down projection's input in the same
   launch: after the GEMM blocks, trailing blocks convert the SwiGLU output
   rows (y, FP32, still written) into FP16 row-scaled activations, out +
   t * out_ld with out_scale[t] (lfm3_half_rows of y with these row maxima,
   bit for bit; chunk tails zeroed). A GEMM block writes y and its row
   maxima through to memory and then stores `seq` in its flag; a trailing
   block waits for the flags of its token block's GEMM blocks (bounded: a
   timeout stores 1 to *error, which may be NULL, and the block goes on).
   flags: lfm3_q8_gemm_swiglu_flags_bytes(rows, tokens), zeroed once; seq:
   nonzero and different from the previous call's on the same flags; calls
   on the same flags must not overlap. out must not alias a (the GEMM reads
   a while trailing blocks write out). rows % 4 == 0 and rows <= 8192, ldy
   % 4 == 0, out_ld % 64 == 0. Replaces: gpu::ProjectFfn's gate/up GEMM
   and the down projection's HalfRowsFromMax (q8_prefill.hpp:53-74;
   hip/ops.hip:2205-2222). */
size_t lfm3_q8_gemm_swiglu_flags_bytes(uint32_t rows, uint32_t tokens);
int lfm3_q8_gemm_swiglu_h16_rows(const void* halves, const void* scales, uint32_t rows,
                                 uint32_t cols, const uint16_t* a, uint32_t lda,
                                 const float* a_scale, uint32_t tokens, float* y,
                                 uint32_t ldy, unsigned* row_max, uint16_t* out,
                                 uint32_t out_ld, float* out_scale, unsigned* flags,
                                 uint32_t seq, unsigned* error, void* stream);
/* FP16 tiles of a tiled Q8_0 matrix: each code decoded exactly to fp16 in
   the order the prompt GEMM's MFMA takes it (2 KB per 16-row x 64-column
   tile; lfm3_q8_half_tiles_bytes). The scales stay in the Q8_0 scale
   array. Replaces: the per-chunk decode of Codes (q8_prefill.hpp:82-92),
   done once at load instead of in every prompt GEMM. */
size_t lfm3_q8_half_tiles_bytes(uint32_t rows, uint32_t cols);
int lfm3_q8_half_tiles(const void* codes, uint32_t rows, uint32_t cols,
                       void* halves, void* stream);
/* lfm3_q8_gemm and lfm3_q8_gemm_swiglu over FP16 tiles (the same
   operands, products and FP32 block fmas, so the outputs are identical).
   Replaces: as lfm3_q8_gemm and lfm3_q8_gemm_swiglu. */
int lfm3_q8_gemm_h16(const void* halves, const void* scales, uint32_t rows,
                     uint32_t cols, const uint16_t* a, uint32_t lda,
                     const float* a_scale, uint32_t tokens, float* y, uint32_t ldy,
                     uint32_t parts, void* stream);
int lfm3_q8_gemm_swiglu_h16(const void* halves, const void* scales, uint32_t rows,
                            uint32_t cols, const uint16_t* a, uint32_t lda,
                            const float* a_scale, uint32_t tokens, float* y,
                            uint32_t ldy, unsigned* row_max, void* stream);

/* ---------------------------------------------------------------------
 * Row operations.
 * ------------------------------------------------------------------- */
/* x[i] += post_norm(branch[i]) (branch/post may be NULL), then
   z[i] = RMSNorm(x[i]) * norm (norm may be NULL: x only). FP32.
   Replaces: gpu::ResidualNorm FP32 branch (hip/ops.hip:2158-2169) and
   gpu::LaunchBatchedRMSNorm (hip/ops.hip:1752-1764). */
int lfm3_residual_norm(const float* branch, const float* post_norm, float* x,
                       const float* norm, float* z, uint32_t rows,
                       uint32_t hidden, float eps, void* stream);
/* The same with the branch given as `parts` (at most 8) partial sums
   part_stride floats apart (lfm3_q8_gemv_partials output), added in part
   order. hidden <= 4096. */
int lfm3_residual_norm_parts(const float* branch, uint32_t parts,
                             size_t part_stride, const float* post_norm,
                             float* x, const float* norm, float* z,
                             uint32_t rows, uint32_t hidden, float eps,
                             void* stream);
/* lfm3_residual_norm_parts whose normed rows also go out as an operand
   image (z may be null). rows <= 8, hidden % 32 == 0. */
int lfm3_residual_norm_image(const float* branch, uint32_t parts,
                             size_t part_stride, const float* post_norm,
                             float* x, const float* norm, float* z, void* image,
                             int* exps, uint32_t rows, uint32_t hidden,
                             float eps, void* stream);
/* The decode round's residual norm and the GEMV that consumes its image in
   one launch: the launch's first `batch` blocks compute
   lfm3_residual_norm_image(branch, parts, part_stride, post_norm, x, norm,
   z = NULL, image, exps, batch, cols, eps) and publish each row through a
   flag; its GEMV blocks issue their weight loads, wait for the rows and
   compute lfm3_q8_gemv_image (swiglu 0) or lfm3_q8_gemv_swiglu_image
   (swiglu 1, rows of each of gate and up) on the image. Results equal the
   two calls made one after the other, bit for bit. flags: a device buffer
   of lfm3_norm_flags_bytes(), zeroed once; seq: a number no earlier call
   on these flags used (not 0); wait_error: NULL or a word the GPU can
   write (device or mapped host memory) that is set to 1 if a block's
   bounded wait for the rows timed out (its results are then undefined).
   Calls on the same flags must not overlap. Replaces: the residual_norm
   lambda of Session::Impl::Run followed by gpu::Project / ProjectSwiGLU
   (engine.cpp:327-350; hip/ops.hip:905-970, 2170-2204). */
size_t lfm3_norm_flags_bytes(void);
int lfm3_q8_gemv_image_norm(const float* branch, uint32_t parts,
                            size_t part_stride, const float* post_norm,
                            float* x, const float* norm, float eps,
                            void* image, int* exps, unsigned* flags,
                            uint32_t seq, unsigned* wait_error,
                            const void* codes, const void* scales,
                            uint32_t rows, uint32_t cols, int swiglu,
                            uint32_t batch, float* y, uint32_t ldy,
                            void* stream);
/* The same for the convolution block's in projection with its step
   (lfm3_q8_gemv_conv_image): norm, then projection and step, in one
   launch. Replaces: the residual_norm lambda, then gpu::Project of in_proj
   and gpu::ShortConv for n == 1 (engine.cpp:327-350, 386-393). */
int lfm3_q8_gemv_conv_image_norm(const float* branch, uint32_t parts,
                                 size_t part_stride, const float* post_norm,
                                 float* x, const float* norm, float eps,
                                 void* image, int* exps, unsigned* flags,
                                 uint32_t seq, unsigned* wait_error,
                                 const void* codes, const void* scales,
                                 uint32_t hidden, uint32_t batch,
                                 const float* taps, float* const* history,
                                 uint32_t width, float* y, uint32_t ldy,
                                 void* stream);
/* lfm3_residual_norm_parts whose normed rows also go out as the prompt
   GEMM's FP16 row-scaled activations (lfm3_half_rows of z: a16 rows of lda
   halves, scale per row); z may be NULL. Replaces: the FP16 split branch of
   ResidualNormKernel (hip/ops.hip:946-969). */
int lfm3_residual_norm_half(const float* branch, uint32_t parts,
                            size_t part_stride, const float* post_norm,
                            float* x, const float* norm, float* z,
                            uint16_t* a16, uint32_t lda, float* scale,
                            uint32_t rows, uint32_t hidden, float eps,
                            void* stream);
/* out[i] = d * q of row tokens[i] (tokens in device memory).
   Replaces: gpu::Embed (hip/ops.hip:2007-2011). */
int lfm3_embed(const void* codes, const void* scales, uint32_t vocab,
               uint32_t hidden, const uint32_t* tokens, uint32_t n,
               float* out, void* stream);
/* Greedy ids: first index of each row's maximum, as std::max_element
   (tests/session_test.cpp:32-34). ids in device memory; cols % 4 == 0 and
   logits 16-byte aligned. One block per row: no workspace
   (lfm3_argmax_workspace_bytes returns 0). Replaces: the host sampler's
   temperature-0 pick. */
size_t lfm3_argmax_workspace_bytes(uint32_t rows);
int lfm3_argmax(const float* logits, uint32_t rows, uint32_t cols,
                uint32_t* ids, void* workspace, size_t workspace_bytes,
                void* stream);
/* Sampler settings of the serving loop (runner.cpp:31-35 defaults:
   temperature 0.1, top_k 50, repeat_penalty 1.1). temperature <= 0 or
   top_k == 1 is the greedy pick; top_k 0 keeps the whole vocabulary. */
typedef struct {
  float temperature;
  uint32_t top_k;
  float repeat_penalty;
} lfm3_sampling;
#define LFM3_SAMPLE_MAX_TOP_K 1024u
#define LFM3_SAMPLE_MAX_PENALTY 4096u
#define LFM3_SAMPLE_MAX_COLS 262144u
/* One token id per logits row (at most 65535 rows of cols floats, ld
   floats apart), all in device memory. Each row: the repetition penalty over
   penalty_ids[row * n_penalty ...] (logit l -> l / p if l > 0 else l * p,
   once per listed token; ids >= cols are padding), the top_k largest
   logits (ties toward the lower index), weights exp((l - l_max) / T), and
   the first candidate, in descending logit order (index order when the
   whole vocabulary is kept), whose running weight sum exceeds
   uniforms[row] * total. uniforms (in [0, 1)) may be NULL for a greedy
   pick. Deterministic for given uniforms. The workspace (device memory,
   lfm3_sample_workspace_bytes(rows, cols, top_k) bytes) holds each
   4096-logit slice's statistics and top-k candidates between the two
   launches.
   Replaces: sampler.Sample(s.logits) in SelectNext (runner.cpp:300-325),
   the Gufo host sampler, which the reference does not carry. */
size_t lfm3_sample_workspace_bytes(uint32_t rows, uint32_t cols, uint32_t top_k);
int lfm3_sample(const float* logits, uint32_t rows, uint32_t cols, uint32_t ld,
                const lfm3_sampling* params, const uint32_t* penalty_ids,
                uint32_t n_penalty, const float* uniforms, uint32_t* ids,
                void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * Ragged decode rows: every row belongs to its own session; per-row
 * pointers and positions come from device index tables.
 * ------------------------------------------------------------------- */
/* One gated short-convolution step per row: p = [B | C | x] (row stride
   ldp), history[i] -> that row's [hidden][width - 1] FP32 history.
   Replaces: gpu::ShortConv with n == 1 (hip/ops.hip:2250-2255) called once
   per session (engine.cpp:394-400). */
int lfm3_conv_step_ragged(const float* p, uint32_t ldp, const float* taps,
                          float* const* history, float* y, uint32_t ldy,
                          uint32_t rows, uint32_t hidden, uint32_t width,
                          void* stream);
/* lfm3_conv_step_ragged with one block per row, writing the output rows
   as the out projection's operand image (y may be null). Outputs and
   history stay bit-identical. rows <= 8, hidden % 32 == 0. */
int lfm3_conv_step_ragged_image(const float* p, uint32_t ldp,
                                const float* taps, float* const* history,
                                float* y, uint32_t ldy, void* image, int* exps,
                                uint32_t rows, uint32_t hidden, uint32_t width,
                                void* stream);
/* Per-head Q/K RMSNorm, paired RoPE at positions[i] and the F16 K/V store
   to ring slot positions[i] % capacity[i] of cache_k[i] / cache_v[i]
   ([capacity][kv_heads][dim] F16). q/k/v rows have stride ld floats.
   frequencies: dim / 2 floats; factors: NULL on sliding layers.
   Replaces: gpu::DecodeHeads (hip/ops.hip:2397-2407) per session
   (engine.cpp:424-429). */
int lfm3_decode_heads_ragged(float* q, float* k, const float* v, uint32_t ld,
                             const float* q_norm, const float* k_norm,
                             const float* frequencies, const float* factors,
                             uint16_t* const* cache_k,
                             uint16_t* const* cache_v,
                             const uint32_t* positions,
                             const uint32_t* capacity, uint32_t rows,
                             uint32_t heads, uint32_t kv_heads, uint32_t dim,
                             float eps, void* stream);

/* Work list of ragged decode attention: one item per (row, key span). */
typedef struct {
  uint32_t row;        /* query row */
  uint32_t key_begin;  /* first key position of the span */
  uint32_t key_end;    /* one past the last key position */
  uint32_t first_item; /* index of this row's first item */
  uint32_t parts;      /* number of spans of this row */
  uint32_t reserved[3];
} lfm3_attention_item;
/* Host planning: positions[i] is row i's position (keys [first, position],
   first = max(0, position + 1 - window) when window > 0). Every row's keys
   split into contiguous spans of one length for the call: a multiple of 64
   keys between 64 and 1024, about (total keys) / 128, and long enough that
   no row has more than 256 spans (hip/ops.hip:2295-2311 splits each
   session's keys on its own). Writes up to max_items items and returns
   their count, or a negative status. */
int lfm3_attention_plan(const uint32_t* positions, uint32_t rows,
                        uint32_t window, lfm3_attention_item* items,
                        uint32_t max_items);
/* An item-list capacity that fits any plan of `rows` rows whose positions
   are at most max_position. */
size_t lfm3_attention_max_items(uint32_t rows, uint32_t max_position);
/* The decode attention workspace: 64 KiB of arrival counters (one per
   (first item, KV head) of a plan; they must be zero before a workspace's
   first call, and every call leaves them zero), then the partial sums of
   multi-span rows, items x heads x (dim + 2) floats. */
size_t lfm3_attention_workspace_bytes(uint32_t items, uint32_t rows,
                                      uint32_t heads, uint32_t kv_heads,
                                      uint32_t dim);
/* Gated GQA of one query per row over its session's F16 ring:
   out[i][h] = (softmax(q_h . K / sqrt(dim)) V) / (1 + exp(-gate[i][h])).
   q holds normed, rotated queries and the ring already holds the current
   K/V row (lfm3_decode_heads_ragged). q/gate/out rows have strides
   ldq/ldg/ldo floats; items and the per-row tables are in device memory.
   dim 64 or 128; heads % kv_heads == 0 with a group of 2, 4 or 8; each
   ring (capacity x kv_heads x dim F16) under 2 GiB. One
   launch: the last span block of a split row (counted with an agent-scope
   atomic in the workspace) merges the row's spans in span order, so
   outputs do not depend on scheduling. `items` must be an
   lfm3_attention_plan over exactly these `rows` rows: an item list whose
   count equals `rows` but holds a split row leaves that row's outputs NaN
   (the whole-row path has no merge).
   Replaces: gpu::Attention with n == 1 (hip/ops.hip:2289-2315:
   DecodeWaves + DecodeCombine) per session (engine.cpp:430-434). */
int lfm3_decode_attention_ragged(
    const float* q, uint32_t ldq, const float* gate, uint32_t ldg,
    const uint16_t* const* cache_k, const uint16_t* const* cache_v,
    const uint32_t* capacity, const lfm3_attention_item* items,
    uint32_t n_items, float* out, uint32_t ldo, uint32_t rows, uint32_t heads,
    uint32_t kv_heads, uint32_t dim, void* workspace, size_t workspace_bytes,
    void* stream);
/* lfm3_decode_heads_ragged and lfm3_decode_attention_ragged in one pass:
   q/k/v are the raw projection rows (stride ld floats, left unchanged);
   each block norms and rotates its row's queries and key; the one block
   whose span ends at the current position stores the row's F16 K/V to ring
   slot positions[i] % capacity[i], waits for the stores, and reads the key
   back through the ring with its other keys (no other span of the row
   covers that slot; sliding rings hold at least the window).
   Replaces: gpu::DecodeHeads + gpu::Attention (hip/ops.hip:2289-2315,
   2397-2407) per session (engine.cpp:424-436). */
int lfm3_decode_heads_attention_ragged(
    const float* q, const float* k, const float* v, uint32_t ld,
    const float* gate, uint32_t ldg, const float* q_norm, const float* k_norm,
    const float* frequencies, const float* factors, uint16_t* const* cache_k,
    uint16_t* const* cache_v, const uint32_t* positions,
    const uint32_t* capacity, const lfm3_attention_item* items,
    uint32_t n_items, float* out, uint32_t ldo, uint32_t rows, uint32_t heads,
    uint32_t kv_heads, uint32_t dim, float eps, void* workspace,
    size_t workspace_bytes, void* stream);

/* No counterpart in the reference. For callers that cannot allocate
   device memory (code under HIP graph capture, tight serving loops,
   harnesses that forbid hipMalloc): lfm3_decode_heads_attention_ragged
   with the span partials in a library-owned device array of
   LFM3_ATTENTION_SCRATCH_BYTES per GPU (held until the process ends)
   instead of a workspace argument; same kernels, same outputs. A plan
   whose partials (lfm3_attention_workspace_bytes) exceed the array is
   refused (LFM3_E_INVALID). Nothing in the array needs clearing: every
   partial a merge reads is written by its span first in the same call, and
   the arrival counters (the array's first 64 KiB, zero at load) return to
   zero at the end of every call.
   Every call on one GPU shares that GPU's array, so calls that overlap on
   one GPU (on different streams) race. Allocates nothing: the array's
   address is looked up once per device (hipGetSymbolAddress). */
#define LFM3_ATTENTION_SCRATCH_BYTES ((size_t)8 << 20)
int lfm3_decode_heads_attention_ragged_noalloc(
    const float* q, const float* k, const float* v, uint32_t ld,
    const float* gate, uint32_t ldg, const float* q_norm, const float* k_norm,
    const float* frequencies, const float* factors, uint16_t* const* cache_k,
    uint16_t* const* cache_v, const uint32_t* positions,
    const uint32_t* capacity, const lfm3_attention_item* items,
    uint32_t n_items, float* out, uint32_t ldo, uint32_t rows, uint32_t heads,
    uint32_t kv_heads, uint32_t dim, float eps, void* stream);

/* ---------------------------------------------------------------------
 * Prompt chunk rows: n consecutive rows of one session (or, for the
 * convolution, packed segments of several sessions).
 * ------------------------------------------------------------------- */
/* Gated short convolution over packed ragged prompt segments: segment s is
   rows [begin[s], begin[s] + rows[s]) of p ([B | C | x], stride ldp) and of
   y, and continues history[s] ([hidden][width - 1] FP32, oldest first).
   Each output keeps lfm3_conv_step_ragged's expressions and order, so a
   segment of n rows gives bit-identical outputs to n decode steps. With
   update_history the history becomes the segment's last width - 1 B x
   products. begin/rows/history are host arrays; segments <= 8.
   Replaces: gpu::ShortConv with n > 1 (hip/ops.hip:2250-2264:
   ConvolutionWindow + ConvolutionHistory) per prompt (engine.cpp:386-393). */
int lfm3_conv_prompt(const float* p, uint32_t ldp, const float* taps,
                     float* const* history, const uint32_t* begin,
                     const uint32_t* rows, uint32_t segments, float* y,
                     uint32_t ldy, uint32_t hidden, uint32_t width,
                     int update_history, void* stream);
/* lfm3_conv_prompt over one segment of `rows` rows fused with
   lfm3_half_rows of its output: rows r >= skip of the convolution output go
   to out + (r - skip) * lda as FP16 row-scaled activations with scale[r -
   skip] (bit-identical to the two calls; chunk tails zeroed), and no FP32
   output is written. Rows before skip only feed the windows. hidden % 4 ==
   0 and at most 2048, width 2..7, lda % 64 == 0. Replaces: gpu::ShortConv
   with n > 1 (hip/ops.hip:2250-2264) followed by the out projection's
   HalfRows (q8_prefill.hpp:30-51), for prompts of 16 rows or more. */
int lfm3_conv_prompt_half(const float* p, uint32_t ldp, const float* taps,
                          float* history, uint32_t rows, uint32_t skip,
                          uint16_t* out, uint32_t lda, float* scale,
                          uint32_t hidden, uint32_t width, int update_history,
                          void* stream);
/* Per-head Q/K RMSNorm and paired RoPE of `rows` chunk rows at positions
   position + r (q/k/v rows of stride ld floats, rotated in place), and the
   F16 K/V of row r stored to row r of k16/v16 (kv_heads * dim halves a
   row: a staging chunk, or the cache rows themselves for a full-attention
   ring that does not wrap). Replaces: gpu::PromptHeads
   (hip/ops.hip:2407-2417; engine.cpp:441-450). */
int lfm3_prompt_heads(float* q, float* k, const float* v, uint32_t ld,
                      const float* q_norm, const float* k_norm,
                      const float* frequencies, const float* factors,
                      uint16_t* k16, uint16_t* v16, uint32_t rows,
                      uint32_t heads, uint32_t kv_heads, uint32_t dim,
                      uint32_t position, float eps, void* stream);
/* gpu::RopeFrequencies (hip/ops.hpp:71; hip/ops.hip:1045-1050, 2265-2267):
   out[i] = fp32(theta^(-2i / dim)) for i < dim / 2, the power in double
   precision. dim even, at most 1024. */
int lfm3_rope_frequencies(float* out, uint32_t dim, float theta, void* stream);
/* gpu::Rope (hip/ops.hpp:72-73; hip/ops.hip:1052-1071, 2268-2274): rotates
   pairs (i, i + dim / 2) of n x heads rows of dim floats (row (t, h) at
   x + (t heads + h) dim) by angle (position + t) frequencies[i], divided
   by factors[i] when factors is not NULL. */
int lfm3_rope(float* x, const float* frequencies, const float* factors,
              uint32_t n, uint32_t heads, uint32_t dim, uint32_t position,
              void* stream);
/* gpu::PackKV (hip/ops.hpp:107-108; hip/ops.hip:1729-1736, 2387-2390):
   count values of k and v rounded to F16 (round to nearest even). */
int lfm3_pack_kv(const float* k, const float* v, uint16_t* k16, uint16_t* v16,
                 size_t count, void* stream);
/* Chunk rows 0..rows-1 at positions position + r into the F16 ring: row r
   goes to slot (position + r) % capacity; only the last min(rows, capacity)
   rows are copied (their slots are distinct). stride = kv_heads * dim.
   Replaces: gpu::StoreKV (hip/ops.hip:1737-1749, 2392-2396;
   engine.cpp:467-470). */
int lfm3_store_kv(const uint16_t* k16, const uint16_t* v16, uint16_t* cache_k,
                  uint16_t* cache_v, uint32_t rows, uint32_t stride,
                  uint32_t position, uint32_t capacity, void* stream);
/* Workspace of lfm3_prompt_attention: key spans of long global histories
   (whole 64-key tiles, at least 1024 keys each, at most 16, as many as
   bring the launch to about one block per CU) keep partial sums, rows x
   heads x (dim + 2) floats a span; this bounds any head grouping. 0 when
   the keys fit one span or window > 0. */
size_t lfm3_prompt_attention_workspace_bytes(uint32_t rows, uint32_t heads,
                                             uint32_t dim, uint32_t position,
                                             uint32_t window);
/* Causal gated GQA of `rows` query rows at positions position + r:
   out[r][h] = (softmax(q . K / sqrt(dim)) V) / (1 + exp(-gate[r][h])) over
   keys [first, position + r], first = max(0, position + r + 1 - window)
   when window > 0. Keys at or after position are rows of k/v (the chunk,
   row 0 at position), earlier keys come from cache_k/cache_v slot
   t % capacity ([capacity][kv_heads][dim] F16; unused when position is 0).
   q holds normed, rotated queries; q/gate/out rows have strides
   ldq/ldg/ldo floats (multiples of 4, 16-byte aligned rows). F16 Q (with
   the base-2 softmax scale), K, V and probabilities on the matrix cores,
   FP32 scores, sums and outputs. dim 64 or 128; group 2, 4 or 8; the
   chunk (rows) and the ring (capacity) each under 2 GiB of F16 rows.
   Replaces: gpu::Attention with n > 1 (hip/ops.hip:2316-2332: WmmaAttn +
   PromptCombine; engine.cpp:451-466). */
int lfm3_prompt_attention(const float* q, uint32_t ldq, const uint16_t* k,
                          const uint16_t* v, const float* gate, uint32_t ldg,
                          const uint16_t* cache_k, const uint16_t* cache_v,
                          float* out, uint32_t ldo, uint32_t rows,
                          uint32_t heads, uint32_t kv_heads, uint32_t dim,
                          uint32_t position, uint32_t capacity,
                          uint32_t window, void* workspace,
                          size_t workspace_bytes, void* stream);
/* lfm3_prompt_attention with its output written as the output projection's
   FP16 row-scaled activations: row r's heads * dim outputs (the same FP32
   values) go to out + r * lda as fp16(out 2^e) with scale[r] = 2^-e, e =
   14 - ilogb(max |row|) (lfm3_half_rows of the FP32 output, bit for bit).
   Every call keeps per-span partial sums in the workspace
   (lfm3_prompt_attention_half_workspace_bytes, at least one span); a
   per-row merge writes the rows. lda % 64 == 0, lda >= heads * dim.
   Replaces: gpu::Attention with n > 1 (hip/ops.hip:2316-2332) followed by
   the out projection's HalfRows (q8_prefill.hpp:30-51). */
size_t lfm3_prompt_attention_half_workspace_bytes(uint32_t rows, uint32_t heads,
                                                  uint32_t dim, uint32_t position,
                                                  uint32_t window);
int lfm3_prompt_attention_half(const float* q, uint32_t ldq, const uint16_t* k,
                               const uint16_t* v, const float* gate, uint32_t ldg,
                               const uint16_t* cache_k, const uint16_t* cache_v,
                               uint16_t* out, uint32_t lda, float* scale,
                               uint32_t rows, uint32_t heads, uint32_t kv_heads,
                               uint32_t dim, uint32_t position, uint32_t capacity,
                               uint32_t window, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------
 * Engine: Model / Session (engine.hpp:17-163).
 *
 * Threading: a model's sessions share its two streams and its round and
 * prompt scratch (the reference gives each session its own stream and
 * workspaces, engine.cpp:47-54, 180-190). Every engine call that uses
 * them takes the model's lock, so calls on sessions of one model may come
 * from several host threads and run one at a time, each with the results
 * it has alone. Continuation hooks run before the lock is taken and may
 * call back into the library. One session must not be used by two calls
 * at once (as in the reference, sessions are not thread-safe).
 * ------------------------------------------------------------------- */
enum { LFM3_LAYER_CONV = 0, LFM3_LAYER_FULL = 1, LFM3_LAYER_SLIDING = 2 };
/* GGML type ids (core::GgmlType). A model's projection matrices and its
   embedding all share one of Q8_0, BF16, F16 or F32 (one engine path per
   precision); norms, RoPE factors and convolution taps are F32. */
enum { LFM3_TYPE_F32 = 0, LFM3_TYPE_F16 = 1, LFM3_TYPE_Q8_0 = 8, LFM3_TYPE_BF16 = 30 };

/* config.hpp:9-20. */
typedef struct {
  uint32_t hidden, intermediate, vocab, context, heads, head_dim, window,
      conv_width, n_layers;
  float eps, theta, theta_swa;
  const uint32_t* kv_heads;  /* per layer; 0 for convolution layers */
  const uint8_t* layer_type; /* LFM3_LAYER_* per layer */
} lfm3_config;

/* weights.hpp:7-12 tensor view in host memory (GGUF layout). */
typedef struct {
  const void* data;
  uint32_t type; /* LFM3_TYPE_F32 / _F16 / _Q8_0 / _BF16 */
  uint32_t cols, rows;
} lfm3_tensor;

/* Tensor order: embedding, output, output_norm, rope_freqs, then per layer
   norm, ffn_norm, post_norm, post_ffn_norm, gate, up, down, conv, in_proj,
   out_proj, q, k, v, q_norm, k_norm, attn_gate, attn_out (weights.hpp:13-22;
   absent tensors have data == NULL). */
#define LFM3_GLOBAL_TENSORS 4
#define LFM3_LAYER_TENSORS 17

typedef struct lfm3_model lfm3_model;
typedef struct lfm3_session lfm3_session;

/* Binds and uploads the weights (Model::Load, engine.cpp:117-170, with the
   GGUF mapping replaced by caller-provided tensor views). */
int lfm3_model_load(const lfm3_config* config, const lfm3_tensor* tensors,
                    size_t count, lfm3_model** out);
void lfm3_model_destroy(lfm3_model* model);
/* Model::CreateSession (engine.cpp:195-236). */
int lfm3_session_create(lfm3_model* model, uint32_t context,
                        lfm3_session** out);
void lfm3_session_destroy(lfm3_session* session);
uint32_t lfm3_session_position(const lfm3_session* session);
int lfm3_session_reset(lfm3_session* session);
int lfm3_session_is_coherent(const lfm3_session* session);
uint32_t lfm3_session_ring_capacity(const lfm3_session* session,
                                    uint32_t layer);

/* Session state in device memory (Session::ContinuationData,
   engine.cpp:1341-1358): kind 0 logits (vocab f32), 1 frontier (hidden
   f32), 2 conv history (hidden * (width - 1) f32), 3 K ring, 4 V ring
   ([capacity][kv_heads][head_dim] F16). */
enum {
  LFM3_STATE_LOGITS = 0,
  LFM3_STATE_FRONTIER = 1,
  LFM3_STATE_CONV = 2,
  LFM3_STATE_KEY = 3,
  LFM3_STATE_VALUE = 4
};
int lfm3_session_state(lfm3_session* session, int kind, uint32_t layer,
                       void** data, size_t* bytes);
/* Session::BeginRestore (engine.cpp:1372-1377): waits for the session's
   work in flight and refuses further work (poisoned) until
   lfm3_session_set_position, so a caller can write every state row through
   lfm3_session_state. */
int lfm3_session_begin_restore(lfm3_session* session);
/* Session::FinishRestore (engine.cpp:1378-1384): the session resumes at
   `position` with the state rows the caller wrote, the logits row included
   (read_logits returns it as written; position 0 still has no logits). */
int lfm3_session_set_position(lfm3_session* session, uint32_t position);

/* Session::Forward (engine.cpp:882-938): n tokens of one session in
   chunks of 512 rows (engine.hpp:47); logits (vocab floats, may be NULL)
   receive the last token's logits. Refuses an empty or oversized token
   list, out-of-range tokens and a poisoned session without touching state;
   a device failure poisons the session. A chunk of 16 rows or more runs
   the prompt path (FP16 row-scaled projections on the matrix cores,
   packed convolution, prompt heads and MFMA prompt attention), with the
   reference's trailing-row pruning (engine.cpp:304-323); shorter chunks
   use the FP32 projections, and one token is one decode row. */
int lfm3_session_forward(lfm3_session* session, const uint32_t* tokens,
                         size_t n, float* logits);
/* Session::ForwardBatch (engine.cpp:1160-1216): one token per distinct
   session (at most 8), logits copied to host rows logits[i] (vocab floats
   each). On a device failure every session of the batch is poisoned. */
int lfm3_forward_batch(lfm3_session* const* sessions, size_t n,
                       const uint32_t* tokens, float* const* logits);
/* The same round with logits left in each session's device state and the
   greedy ids of the rows written to ids (host). The serving loop's form:
   no logits cross PCIe. */
int lfm3_forward_batch_greedy(lfm3_session* const* sessions, size_t n,
                              const uint32_t* tokens, uint32_t* ids);
/* The same round with the sampler's pick in place of the greedy one
   (lfm3_sample over each session's device logits row; the serving loop's
   SelectNext, runner.cpp:300-325, on the device). Host inputs: row i's
   penalty list penalty_ids[i * n_penalty ...] (the session's recent
   tokens; ids >= vocab are padding; may be NULL when n_penalty is 0) and
   its uniform uniforms[i] in [0, 1) (may be NULL for a greedy setting).
   ids (host) get the picks. Parameters are checked before any work. */
int lfm3_forward_batch_sample(lfm3_session* const* sessions, size_t n,
                              const uint32_t* tokens, const lfm3_sampling* params,
                              const uint32_t* penalty_ids, uint32_t n_penalty,
                              const float* uniforms, uint32_t* ids);
/* Session::ForwardBatchInputs (engine.cpp:1217-1299): the round of
   lfm3_forward_batch where rows[i], when not NULL, is a device FP32 row of
   hidden floats that stands in for session i's token embedding (tokens[i]
   is then not checked); NULL entries use the token. With want_logits 0 the
   vocabulary head is skipped: only the positions and the frontier rows
   (LFM3_STATE_FRONTIER, Session::DeviceHidden) advance, and the head runs
   on the frontier row when logits are first wanted
   (lfm3_session_prepare_logits, lfm3_session_read_logits). With
   want_logits set, logits (may be NULL) receive host copies. A device
   failure poisons every session of the batch. */
int lfm3_forward_batch_inputs(lfm3_session* const* sessions, size_t n,
                              const uint32_t* tokens, const float* const* rows,
                              int want_logits, float* const* logits);
/* Session::ReadLogits (engine.cpp:1433-1463) into host memory (vocab
   floats). Refuses a poisoned session or one at position 0; after a round
   or prompt without logits, the vocabulary head first runs on the
   frontier row (Session::Impl::EnsureLogits, engine.cpp:237-245). */
int lfm3_session_read_logits(const lfm3_session* session, float* logits);
/* Session::PrepareLogits (engine.hpp:146, engine.cpp:1369-1373): after a
   round or prompt that skipped the vocabulary head, runs the head on the
   frontier row on the model stream and waits for it, so the device logits
   row (LFM3_STATE_LOGITS) holds the frontier's logits; nothing is copied
   to the host, and logits already current cost nothing. Refuses a
   poisoned session or one at position 0. The continuation adapter calls
   it before it captures the logits component
   (continuation_adapter.cpp:369-370). */
int lfm3_session_prepare_logits(lfm3_session* session);
/* Snapshot v2 (Session::SnapshotBytes / SaveSnapshot / RestoreSnapshot,
   engine.cpp:1387-1574), byte-compatible with the reference's: a 32-byte
   header of little-endian words (0x334d464c, 2, context, position, hidden,
   vocab, layers, FNV-1a signature of the configuration), the frontier row
   and the logits (zeros at position 0), then per layer the convolution
   history or the first min(position, capacity) K ring slots then V slots
   in physical order. Save refuses a poisoned session (LFM3_E_STATE) and a
   buffer of another size; restore checks the whole header and the size
   before it changes anything (LFM3_E_INVALID), and a failed copy poisons
   the session. */
size_t lfm3_session_snapshot_bytes(const lfm3_session* session);
int lfm3_session_save_snapshot(lfm3_session* session, void* out, size_t bytes);
int lfm3_session_restore_snapshot(lfm3_session* session, const void* data,
                                  size_t bytes);
/* Stream of the model's batch rounds (Session::DeviceStream). */
void* lfm3_model_stream(lfm3_model* model);

/* One scheduler round (README.md:106-109: the decode batch and a prompt
   chunk a round): n decode rows of distinct sessions (as
   lfm3_forward_batch, at most 8; n may be 0) and a prompt of n_prompt
   tokens of another session of the same model (as lfm3_session_forward;
   n_prompt may be 0). The decode round runs on the model stream and the
   prompt pass on the model's second stream, both enqueued before either
   is waited on. ids (host, may be NULL) get the rows' greedy ids, logits
   (may be NULL) host copies of their logits; prompt_logits (may be NULL)
   the prompt's last logits. Every check and hook runs before any work;
   a device failure of the decode round poisons its sessions, one of the
   prompt poisons the prompt session. No counterpart call in the
   reference, whose runner issues the two one after the other. */
int lfm3_scheduler_round(lfm3_session* const* sessions, size_t n,
                         const uint32_t* tokens, uint32_t* ids,
                         float* const* logits, lfm3_session* prompt,
                         const uint32_t* prompt_tokens, size_t n_prompt,
                         float* prompt_logits);
/* Session::ForwardEmbeddings (engine.hpp:104-110, engine.cpp:939-985):
   n_rows input rows of hidden floats each in place of token embeddings, in
   passes of 512 rows (one row: a decode row), on host memory or, with
   on_device, device memory ordered before the call. logits (vocab floats,
   may be NULL) receive the last row's logits. Refusals and poisoning as
   lfm3_session_forward. */
int lfm3_session_forward_rows(lfm3_session* session, const float* rows,
                              size_t n_rows, int on_device, float* logits);
/* Session::Input (engine.hpp:111-115): a run of token ids or of input rows
   (hidden floats each, host memory); one of the two counts is 0. */
typedef struct {
  const uint32_t* tokens;
  size_t n_tokens;
  const float* rows;
  size_t n_rows;
} lfm3_input;
/* Session::ForwardInputs (engine.hpp:116-121, engine.cpp:986-1100): the
   runs in order, adjacent runs sharing their 512-row passes (a prompt that
   mixes text and embeddings reads the weights once per pass). A run with
   both tokens and rows, an out-of-range token or an empty total is
   refused without touching state. */
int lfm3_session_forward_inputs(lfm3_session* session, const lfm3_input* inputs,
                                size_t n_inputs, float* logits);
/* Session::ReadHidden (engine.hpp:122-123): the final-normed hidden row of
   the last advanced row (hidden floats, host memory). */
int lfm3_session_read_hidden(const lfm3_session* session, float* hidden);

/* ---------------------------------------------------------------------
 * Continuation hooks and state layout (continuation_hooks.hpp,
 * continuation_layout.hpp / .cpp).
 * ------------------------------------------------------------------- */
/* ContinuationHooks (continuation_hooks.hpp:6-15): host callbacks that run
   before the session changes state or submits device work. A nonzero
   return refuses the call (LFM3_E_REFUSED), leaving the session as it
   was. before_write gets the rows [first, end) about to be written (every
   forward entry; each session of a batch round, engine.cpp:1196-1199),
   before_reset runs first in lfm3_session_reset and before_restore first
   in lfm3_session_restore_snapshot (engine.cpp:1522-1524). NULL members
   are skipped; the table is copied. Session::SetContinuationHooks
   (engine.cpp:1338-1340). */
typedef struct {
  void* user;
  int (*before_write)(void* user, uint32_t first, uint32_t end);
  int (*before_reset)(void* user);
  int (*before_restore)(void* user);
} lfm3_hooks;
int lfm3_session_set_hooks(lfm3_session* session, const lfm3_hooks* hooks);

/* ContinuationPart (continuation_layout.hpp:12-25). */
enum {
  LFM3_PART_LOGITS = 0,
  LFM3_PART_FRONTIER = 1,
  LFM3_PART_METADATA = 2,
  LFM3_PART_CONVOLUTION = 3,
  LFM3_PART_SLIDING_WINDOW = 4, /* K then V of a sliding ring */
  LFM3_PART_KEY = 5,            /* full-attention K rows, final once written */
  LFM3_PART_VALUE = 6
};
/* The metadata part's bytes: uint32 version (1), uint32 position, zeros. */
#define LFM3_CONTINUATION_METADATA_BYTES 16
/* One component of the state inventory: append rows (row_bytes per
   position, state_bytes 0) or private state (state_bytes, row_bytes 0).
   Ids count from 1 in inventory order. */
typedef struct {
  uint32_t id, part, layer, reserved;
  size_t row_bytes, state_bytes;
} lfm3_continuation_component;
/* ContinuationLayout (continuation_layout.cpp:6-46): logits, frontier and
   metadata, then per layer its convolution history, its sliding ring (2 x
   kv_heads x head_dim x 2 x min(context, window) bytes) or its K and V
   rows. Writes up to `capacity` components and their total to *count.
   Refuses an invalid geometry (context 0 or past config->context). */
int lfm3_continuation_layout(const lfm3_config* config, uint32_t context,
                             lfm3_continuation_component* out, size_t capacity,
                             size_t* count);
/* PrivateBytes / RowBytes(position) (continuation_layout.cpp:56-69): the
   private state's bytes, and the append rows' bytes at a frontier
   (position <= context). */
int lfm3_continuation_bytes(const lfm3_config* config, uint32_t context,
                            uint32_t position, size_t* private_bytes,
                            size_t* row_bytes);

/* ---------------------------------------------------------------------
 * Deterministic synthetic inputs (benchmarks and parity tests). No
 * counterpart in the reference: they stand in for a GGUF checkpoint and
 * prefilled session state. Each value is a function of (seed, stream name,
 * index) only: SplitMix64 counters, Box-Muller normals in double precision.
 * ------------------------------------------------------------------- */
uint64_t lfm3_synth_key(uint64_t seed, const char* name);
void lfm3_synth_normal(uint64_t key, float mean, float stddev, float* out,
                       size_t n);
void lfm3_synth_uniform_u32(uint64_t key, uint32_t lo, uint32_t hi,
                            uint32_t* out, size_t n);
void lfm3_synth_half_normal(uint64_t key, uint16_t* out, size_t n);
/* GGUF Q8_0 rows: q uniform in [-127, 127], d = fp16(|N(0, d_std)| / 127). */
void lfm3_synth_q8(uint64_t key, uint32_t rows, uint32_t cols, float d_std,
                   void* out);

/* ---------------------------------------------------------------------
 * Device ceilings for the benchmark, reported beside the published peaks.
 * No counterpart in the reference (its benchmarks quote spec bandwidth).
 * ------------------------------------------------------------------- */
/* A streaming read of `bytes` (a multiple of 16, 16-byte aligned device
   memory) by `blocks` 512-thread blocks; sink[b] (device, `blocks` words)
   gets the XOR of every 32-bit word block b read, so the XOR over sink
   equals the XOR over the buffer. */
int lfm3_measure_stream_read(const void* buffer, size_t bytes, unsigned* sink,
                             uint32_t blocks, void* stream);
/* A register-only f16 MFMA loop: `blocks` blocks of 4 waves, each wave
   running 8 independent v_mfma_f32_16x16x32_f16 chains for `iterations`
   steps (at most 16384) over all-ones operands; sink (device, 4 * blocks
   floats) gets each wave's 1024 * iterations exactly. */
int lfm3_measure_mfma_f16(uint32_t iterations, uint32_t blocks, float* sink,
                          void* stream);
/* FLOPs of one lfm3_measure_mfma_f16 launch. */
uint64_t lfm3_measure_mfma_f16_flops(uint32_t iterations, uint32_t blocks);

#ifdef __cplusplus
}
#endif
#endif
