// Launchers used only inside the library (not part of the C-ABI).
#ifndef LFM3_AMD_INTERNAL_HPP_
#define LFM3_AMD_INTERNAL_HPP_
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/lfm3_amd.h"

namespace lfm3amd {
// Decode-round residual norm writing the next GEMV's operand image
// (lfm3_residual_norm_image) with the round's options: z rows through a
// device pointer table, and for the round's first norm x gathered from the
// tiled embedding table at tokens[r].
struct NormImageArgs {
  const float* branch = nullptr;
  int parts = 1;
  std::size_t part_stride = 0;
  const float* post = nullptr;
  float* x = nullptr;
  const float* weight = nullptr;
  float* z = nullptr;
  float* const* z_rows = nullptr;
  int H = 0;
  float eps = 0.0f;
  uint4* image = nullptr;
  int* exps = nullptr;
  const std::uint8_t* emb_codes = nullptr;
  const std::uint16_t* emb_scales = nullptr;
  const std::uint32_t* tokens = nullptr;
  int vocab = 0;
  // With tokens: row r's input is inputs[r] (H floats in device memory)
  // when the table entry is not null, else embedding row tokens[r].
  const float* const* inputs = nullptr;
  // The prompt GEMM's FP16 rows instead of (or beside) the image.
  std::uint16_t* a16 = nullptr;
  int lda = 0;
  float* a_scale = nullptr;
};
int LaunchNormImage(const NormImageArgs& a, std::uint32_t rows, hipStream_t stream);
// An operand-image GEMV launch that takes its norm along: its first `batch`
// blocks run the residual norm of `args` (one row each) and publish the
// image rows; its GEMV blocks wait for them (flags: kFlagWords words,
// norm_image.hpp; seq: a number no earlier launch on these flags used;
// error: a host-visible word set to 1 if a wait timed out).
struct FusedNorm {
  NormImageArgs args;
  unsigned* flags = nullptr;
  unsigned seq = 0;
  unsigned* error = nullptr;
};
int LaunchGemvImageFused(const void* codes, const void* scales, std::uint32_t rows,
                         std::uint32_t cols, const void* image, const int* exps,
                         std::uint32_t batch, float* y, std::uint32_t ldy, bool swiglu,
                         const FusedNorm& fused, hipStream_t stream);
// lfm3_q8_gemv_conv_image, fused with the norm when `fused` is not null.
int LaunchConvImage(const void* codes, const void* scales, std::uint32_t hidden,
                    const void* image, const int* exps, std::uint32_t batch, const float* taps,
                    float* const* history, std::uint32_t width, float* y, std::uint32_t ldy,
                    const FusedNorm* fused, hipStream_t stream);
// The vocabulary head on the final operand image: row t of the logits goes
// to y_rows[t], and keys[t * groups + j] gets the best ArgKey of block j's
// rows; returns the number of groups through *groups.
int LaunchHeadGemv(const void* codes, const void* scales, std::uint32_t rows,
                   std::uint32_t cols, const void* image, const int* exps, std::uint32_t batch,
                   float* const* y_rows, unsigned long long* keys, std::uint32_t* groups,
                   hipStream_t stream, const FusedNorm* fused = nullptr);
std::uint32_t HeadGemvGroups(std::uint32_t rows, std::uint32_t cols);
// ids[t] = the first index of token t's maximum from the head's keys.
int LaunchArgmaxKeys(const unsigned long long* keys, std::uint32_t rows, std::uint32_t groups,
                     std::uint32_t* ids, hipStream_t stream);
// lfm3_sample's limits, its parameter check (status, with the error text
// set), its workspace size and its launch over rows given by a device
// pointer table (row_ptrs) or by a base and stride (logits, ld).
constexpr int kSampleMaxCols = LFM3_SAMPLE_MAX_COLS, kSampleMaxTopK = LFM3_SAMPLE_MAX_TOP_K;
constexpr int kSampleMaxPenalty = LFM3_SAMPLE_MAX_PENALTY;
int CheckSample(const lfm3_sampling& p, std::uint32_t cols, std::uint32_t n_penalty,
                bool have_penalty, bool have_uniforms);
std::size_t SampleWorkspaceBytes(std::uint32_t rows, std::uint32_t cols, std::uint32_t top_k);
int LaunchSample(const float* logits, std::uint32_t ld, const float* const* row_ptrs,
                 std::uint32_t rows, std::uint32_t cols, const lfm3_sampling& p,
                 const std::uint32_t* penalty_ids, std::uint32_t n_penalty,
                 const float* uniforms, std::uint32_t* ids, void* workspace,
                 std::size_t workspace_bytes, hipStream_t stream);
// dst[i][0..count) = src + i * ld for rows i < rows, with dst pointers read
// from a device table (per-session logits / frontier rows of a round).
int LaunchScatterRows(const float* src, std::size_t ld, float* const* dst,
                      std::uint32_t rows, std::size_t count,
                      hipStream_t stream);
// lfm3_prompt_heads over a projection in K parts (part_stride floats
// apart): the parts are summed in part order, q and the per-head gate g
// (one float per head at g + row * ld) into part 0.
void LaunchPromptHeads(float* q, float* k, const float* v, std::uint32_t ld, const float* q_norm,
                       const float* k_norm, const float* frequencies, const float* factors,
                       std::uint16_t* k16, std::uint16_t* v16, std::uint32_t rows,
                       std::uint32_t heads, std::uint32_t kv_heads, std::uint32_t dim,
                       std::uint32_t position, float eps, std::uint32_t parts,
                       std::size_t part_stride, float* g, hipStream_t s);
}  // namespace lfm3amd
#endif
