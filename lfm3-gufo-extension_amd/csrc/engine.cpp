// Model / Session of the LFM3 continuous-batching step on one MI355X.
//
// Mirrors the reference engine (engine.hpp:17-163, engine.cpp): a model
// owns packed device weights shared by sessions; a session owns its
// recurrent state (convolution history, F16 K/V rings), logits and
// frontier row; ForwardBatch advances up to eight sessions by one token in
// one round that shares every projection across rows. Where the reference
// loops per session for the convolution and attention launches
// (engine.cpp:394-400, 424-436), a round here uploads one device index
// table (tokens, positions, per-layer state pointers, ring capacities and
// attention work lists) and every launch covers all rows.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "common.hpp"
#include "internal.hpp"
#include "norm_image.hpp"

namespace lfm3amd {
namespace {

constexpr std::uint32_t kMaxBatch = 8;       // engine.hpp:48
constexpr std::uint32_t kPrefillChunk = 512;  // engine.hpp:47
constexpr std::uint32_t kPromptRows = 16;     // hip/ops.hpp:32: FP16 GEMM from here

struct Error : std::runtime_error {
  int status;
  Error(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};
void Check(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw Error(LFM3_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}
void CheckStatus(int status) {
  if (status != LFM3_OK)
    throw Error(status, lfm3_last_error());
}
[[noreturn]] void Invalid(const std::string& m) { throw Error(LFM3_E_INVALID, m); }
// A continuation hook's refusal (a nonzero return) stops the call before
// the session changes state (continuation_hooks.hpp:6-15: hooks may throw).
void Hook(int rc, const char* what) {
  if (rc)
    throw Error(LFM3_E_REFUSED, std::string("LFM3 continuation hook refused ") + what);
}

struct Buffer {
  void* p = nullptr;
  std::size_t bytes = 0;
  Buffer() = default;
  explicit Buffer(std::size_t n, bool zero = true) : bytes(n) {
    if (n) {
      Check(hipMalloc(&p, n), "hipMalloc");
      if (zero)
        Check(hipMemset(p, 0, n), "hipMemset");
    }
  }
  ~Buffer() {
    if (p)
      (void)hipFree(p);
  }
  Buffer(Buffer&& b) noexcept : p(b.p), bytes(b.bytes) { b.p = nullptr; b.bytes = 0; }
  Buffer& operator=(Buffer&& b) noexcept {
    std::swap(p, b.p);
    std::swap(bytes, b.bytes);
    return *this;
  }
  Buffer(const Buffer&) = delete;
  template<class T> T* as() const { return static_cast<T*>(p); }
};

struct PinnedBuffer {
  void* p = nullptr;       // host address
  void* device = nullptr;  // the address kernels use (mapped buffers)
  explicit PinnedBuffer(std::size_t n, unsigned flags = hipHostMallocDefault) {
    Check(hipHostMalloc(&p, n, flags), "hipHostMalloc");
    if (flags & hipHostMallocMapped)
      Check(hipHostGetDevicePointer(&device, p, 0), "hipHostGetDevicePointer");
  }
  ~PinnedBuffer() {
    if (p)
      (void)hipHostFree(p);
  }
  PinnedBuffer(const PinnedBuffer&) = delete;
};

// A tiled Q8_0 matrix of rows x cols (several sources may share it). The
// prompt GEMMs read `halves`, the codes decoded to FP16 tiles, made with
// the model's prompt scratch; the decode GEMVs read the codes.
// A float matrix (BF16, F16 or F32: `exact` set, `type` its format) keeps
// its tiles in `codes` (lfm3_float_pack_host layout) and has no scales.
struct Matrix {
  Buffer codes, scales, halves;
  std::uint32_t rows = 0, cols = 0;
  std::uint32_t tiles = 0;  // row tiles stored (gate/up: two per 16 rows)
  bool exact = false;
  std::uint32_t type = LFM3_TYPE_Q8_0;
};

Buffer UploadFloats(const float* host, std::size_t n) {
  Buffer b(n * 4, false);
  Check(hipMemcpy(b.p, host, n * 4, hipMemcpyHostToDevice), "hipMemcpy");
  return b;
}

struct Part {
  const lfm3_tensor* t;
  std::uint32_t tile_offset, tile_stride;
};
// Packs sources into one tiled matrix of `tiles` row tiles.
Matrix PackMatrix(std::initializer_list<Part> parts, std::uint32_t tiles,
                  std::uint32_t rows, std::uint32_t cols) {
  Matrix m;
  m.rows = rows;
  m.cols = cols;
  m.tiles = tiles;
  const std::uint32_t type = parts.begin()->t->type;
  if (type != LFM3_TYPE_Q8_0) {
    m.exact = true;
    m.type = type;
    const std::size_t bytes = lfm3_float_tiled_bytes(type, tiles * kTileRows, cols);
    std::vector<std::uint8_t> host(bytes, 0);
    for (const auto& part : parts)
      CheckStatus(lfm3_float_pack_host(type, part.t->data, part.t->rows, part.t->cols,
                                       host.data(), part.tile_offset, part.tile_stride));
    m.codes = Buffer(bytes, false);
    Check(hipMemcpy(m.codes.p, host.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
    return m;
  }
  const std::size_t chunks = Chunks(cols);
  const std::size_t code_bytes = std::size_t(tiles) * chunks * kTileCodeBytes;
  const std::size_t scale_bytes = std::size_t(tiles) * chunks * kTileScales * 2;
  std::vector<std::uint8_t> codes(code_bytes, 0);
  std::vector<std::uint8_t> scales(scale_bytes, 0);
  for (const auto& part : parts)
    CheckStatus(lfm3_q8_pack_host(part.t->data, part.t->rows, part.t->cols,
                                  codes.data(), scales.data(), part.tile_offset,
                                  part.tile_stride));
  m.codes = Buffer(code_bytes, false);
  m.scales = Buffer(scale_bytes, false);
  Check(hipMemcpy(m.codes.p, codes.data(), code_bytes, hipMemcpyHostToDevice), "hipMemcpy");
  Check(hipMemcpy(m.scales.p, scales.data(), scale_bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return m;
}

struct Layer {
  int type = LFM3_LAYER_CONV;
  std::uint32_t kv = 0;
  Buffer norm, ffn_norm, post_norm, post_ffn_norm, conv, q_norm, k_norm;
  Matrix ffn;      // gate/up, interleaved by row tile (SwiGLU pairs)
  Matrix down;
  Matrix in_proj, out_proj;
  Matrix qkvg;     // q | k | v | gate, concatenated by row tile
  Matrix attn_out;
  std::uint32_t q_off = 0, k_off = 0, v_off = 0, g_off = 0, qkvg_ld = 0;
};

// Device index table of one round (uploaded once per round).
struct RoundTable {
  std::uint32_t tokens[kMaxBatch];
  std::uint32_t positions[kMaxBatch];
  float* logits[kMaxBatch];
  float* frontier[kMaxBatch];
  const float* inputs[kMaxBatch];  // FP32 input rows in place of tokens, or null
};

std::size_t Align(std::size_t n) { return (n + 255) / 256 * 256; }

// A sampled round's uploaded inputs: kMaxBatch uniforms, then up to
// kSampleMaxPenalty penalty ids a row.
inline std::size_t SampleTableBytes() {
  return Align(kMaxBatch * 4) + std::size_t(kMaxBatch) * kSampleMaxPenalty * 4;
}

// Scratch of one prompt chunk (kPrefillChunk rows), made on the first
// prompt and shared by the model's prompts (under the model's lock).
struct PromptBuffers {
  Buffer tokens, x, z, a16, scale, proj, mix, hid, out, row_max, chunk_k, chunk_v, attn_ws;
  // The FFN hidden rows as the down projection's FP16 rows (written by the
  // SwiGLU launch's trailing blocks), with the flags its GEMM blocks
  // publish (zeroed once) and the launch counter (0 skipped).
  Buffer hid16, hid_scale, swiglu_flags;
  std::uint32_t swiglu_seq = 0;
  // Set to 1 by a trailing block whose wait timed out (host-mapped; the
  // prompt checks it after its synchronization).
  std::unique_ptr<PinnedBuffer> wait_error;
  Buffer one_table;  // one decode-attention row: ring pointers, capacity, position, items
  Buffer one_ws;     // that row's span partials (apart from the decode round's)
  std::unique_ptr<PinnedBuffer> one_staging;
  std::size_t lda = 0, proj_ld = 0, attn_ws_bytes = 0, one_bytes = 0, one_items = 0;
  std::size_t one_ws_bytes = 0;
};

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

struct lfm3_session;

struct lfm3_model {
  std::vector<std::uint32_t> kv_heads;
  std::vector<std::uint8_t> layer_type;
  lfm3_config config{};
  std::vector<Layer> layers;
  Matrix embedding, output;
  bool tied = true;
  Buffer output_norm, factors, freq_global, freq_sliding;
  hipStream_t stream = nullptr;
  // The stream a scheduler round's prompt pass runs on, beside the decode
  // round on `stream` (both default priority).
  hipStream_t prompt_stream = nullptr;
  // Serializes every call that uses the model's streams or scratch, so
  // calls on sessions of one model may come from several host threads;
  // they run one at a time. (The reference gives each session its own
  // stream and workspaces, engine.cpp:47-54, 180-190; here the round and
  // prompt scratch are the model's.) Continuation hooks run before the
  // lock is taken, so a hook may call back into the library.
  std::mutex lock;
  // Round scratch, shared by the model's rounds (under `lock`).
  Buffer x, proj, a, hidden, out, gemv_ws, head_keys;
  // Float-weight models (exact set: BF16, F16 or F32 matrices): every
  // projection is an exact float x FP32 GEMV from FP32 normed rows z; the
  // head writes head_out, then the rows go to the sessions' logits.
  bool exact = false;
  std::uint32_t wtype = LFM3_TYPE_Q8_0;
  Buffer z, head_out;
  std::uint32_t head_groups = 0;
  Buffer image, exps;  // GEMV operand image of the current hidden-wide input
  // A decode round's norms run inside the GEMV launches that consume their
  // images (FusedNorm): the rows' flags, the launches' sequence numbers and
  // a host word that a timed-out wait sets (checked after every round).
  Buffer norm_flags;
  std::uint32_t norm_seq = 0;
  std::unique_ptr<PinnedBuffer> wait_error;
  Buffer one_row;      // a host input row of a one-row chunk, on the device
  std::size_t proj_ld = 0, gemv_ws_bytes = 0;
  // Per-round device tables: RoundTable, per-layer pointer rows, items.
  Buffer table;
  std::unique_ptr<PinnedBuffer> staging;
  std::unique_ptr<PinnedBuffer> logits_host;  // one logits row, pinned
  // A round's ids, written by its last kernel (the argmax or the sampler's
  // pick) straight into pinned host memory the device addresses, and the
  // logits rows on their way to the caller (pinned, made on first use,
  // copied on the model stream behind the round): the round and its
  // results take one synchronization and no copy for the ids.
  std::unique_ptr<PinnedBuffer> ids_host, rows_host;
  // The device's address of the ids. They are written by a kernel and read
  // on the host only after the model stream is synchronized (DeliverReadback).
  std::uint32_t* ids() const { return static_cast<std::uint32_t*>(ids_host->device); }
  // A sampled round's uniforms and penalty lists (made on first use), and
  // the sampler's workspace (greedy size at load, grown for top-k).
  Buffer sample_table, sample_ws;
  std::size_t sample_ws_bytes = 0;
  std::unique_ptr<PinnedBuffer> sample_staging;
  std::size_t table_bytes = 0, items_capacity = 0;
  Buffer attn_ws;
  std::size_t attn_ws_bytes = 0;
  std::uint32_t max_context = 0;
  std::unique_ptr<PromptBuffers> prompt;

  ~lfm3_model() {
    if (stream)
      (void)hipStreamDestroy(stream);
    if (prompt_stream)
      (void)hipStreamDestroy(prompt_stream);
  }
  const Matrix& head() const { return tied ? embedding : output; }
};

struct lfm3_session {
  lfm3_model* model = nullptr;
  std::uint32_t context = 0, position = 0;
  bool poisoned = false, logits_ready = false;
  // Continuation hooks (continuation_hooks.hpp:6-15); null members skip.
  lfm3_hooks hooks{};
  struct State {
    Buffer conv, k, v;
    std::uint32_t capacity = 0;
  };
  std::vector<State> states;
  Buffer logits, frontier;
};

namespace lfm3amd {
namespace {

void ValidateConfig(const lfm3_config& c) {
  if (!c.hidden || !c.intermediate || !c.vocab || !c.context || !c.heads ||
      !c.head_dim || !c.window || !c.n_layers || c.conv_width < 2 ||
      c.conv_width > 32 || !c.kv_heads || !c.layer_type ||
      (c.head_dim != 64 && c.head_dim != 128) || c.hidden % 64 ||
      c.intermediate % 64 || c.hidden > 4096 || !(c.eps > 0) ||
      !(c.theta > 0) || !(c.theta_swa > 0))
    Invalid("unsupported LFM3 dimensions");
  for (std::uint32_t i = 0; i < c.n_layers; ++i) {
    const auto h = c.kv_heads[i];
    const auto t = c.layer_type[i];
    if (t > LFM3_LAYER_SLIDING || (t == LFM3_LAYER_CONV) != (h == 0) ||
        (h && (c.heads % h || (c.heads / h != 2 && c.heads / h != 4 &&
                               c.heads / h != 8))))
      Invalid("invalid LFM3 layer heads/window");
    // The attention kernels address a layer's F16 K/V ring with 32-bit
    // buffer offsets: a ring of the full context stays under 2 GiB.
    if (h && !BufferFits(std::size_t(c.context) * h * c.head_dim * 2))
      Invalid("LFM3 context too long for its K/V rings");
  }
}

// `type` is LFM3_TYPE_F32 for vectors, else the model's matrix type.
void CheckTensor(const lfm3_tensor& t, std::uint32_t cols, std::uint32_t rows,
                 std::uint32_t type, const char* name) {
  if (!t.data || t.cols != cols || t.rows != rows || t.type != type)
    Invalid(std::string("invalid LFM3 tensor: ") + name);
}

// The model's matrix type: the embedding's, one of Q8_0, BF16, F16 and
// F32 (weights.cpp:30-37); every projection matrix must share it (one
// engine path per precision).
std::uint32_t MatrixType(const lfm3_tensor* tensors) {
  const std::uint32_t t = tensors[0].type;
  if (t != LFM3_TYPE_Q8_0 && t != LFM3_TYPE_BF16 && t != LFM3_TYPE_F16 && t != LFM3_TYPE_F32)
    Invalid("invalid LFM3 tensor: token_embd.weight (Q8_0, BF16, F16 or F32)");
  return t;
}

// weights.cpp:10-100 binding rules, checked before anything is uploaded.
void ValidateTensors(const lfm3_config& c, const lfm3_tensor* tensors) {
  const std::uint32_t H = c.hidden, F = c.intermediate, D = c.head_dim;
  const std::uint32_t mt = MatrixType(tensors);
  CheckTensor(tensors[0], H, c.vocab, mt, "token_embd.weight");
  if (tensors[1].data && tensors[1].data != tensors[0].data)
    CheckTensor(tensors[1], H, c.vocab, mt, "output.weight");
  CheckTensor(tensors[2], H, 1, LFM3_TYPE_F32, "output_norm.weight");
  CheckTensor(tensors[3], D / 2, 1, LFM3_TYPE_F32, "rope_freqs.weight");
  for (std::uint32_t i = 0; i < D / 2; ++i) {
    const float f = static_cast<const float*>(tensors[3].data)[i];
    if (!std::isfinite(f) || !(f > 0))
      Invalid("invalid LFM3 RoPE factor");
  }
  for (std::uint32_t i = 0; i < c.n_layers; ++i) {
    const lfm3_tensor* t = tensors + LFM3_GLOBAL_TENSORS + std::size_t(i) * LFM3_LAYER_TENSORS;
    CheckTensor(t[0], H, 1, LFM3_TYPE_F32, "attn_norm.weight");
    CheckTensor(t[1], H, 1, LFM3_TYPE_F32, "ffn_norm.weight");
    if (bool(t[2].data) != bool(t[3].data))
      Invalid("LFM3 requires both post norms or neither");
    if (t[2].data) {
      CheckTensor(t[2], H, 1, LFM3_TYPE_F32, "post_attention_norm.weight");
      CheckTensor(t[3], H, 1, LFM3_TYPE_F32, "post_ffw_norm.weight");
    }
    CheckTensor(t[4], H, F, mt, "ffn_gate.weight");
    CheckTensor(t[5], H, F, mt, "ffn_up.weight");
    CheckTensor(t[6], F, H, mt, "ffn_down.weight");
    if (c.layer_type[i] == LFM3_LAYER_CONV) {
      CheckTensor(t[7], c.conv_width, H, LFM3_TYPE_F32, "shortconv.conv.weight");
      CheckTensor(t[8], H, 3 * H, mt, "shortconv.in_proj.weight");
      CheckTensor(t[9], H, H, mt, "shortconv.out_proj.weight");
    } else {
      const std::uint32_t qr = c.heads * D, kr = c.kv_heads[i] * D;
      CheckTensor(t[10], H, qr, mt, "attn_q.weight");
      CheckTensor(t[11], H, kr, mt, "attn_k.weight");
      CheckTensor(t[12], H, kr, mt, "attn_v.weight");
      CheckTensor(t[13], D, 1, LFM3_TYPE_F32, "attn_q_norm.weight");
      CheckTensor(t[14], D, 1, LFM3_TYPE_F32, "attn_k_norm.weight");
      CheckTensor(t[15], H, c.heads, mt, "attn_gate.weight");
      CheckTensor(t[16], qr, H, mt, "attn_output.weight");
    }
  }
}

void EnsureRoundBuffers(lfm3_model& m, std::uint32_t max_context) {
  const auto& c = m.config;
  if (max_context <= m.max_context)
    return;
  m.items_capacity = lfm3_attention_max_items(kMaxBatch, max_context);
  const std::size_t L = c.n_layers;
  m.table_bytes = Align(sizeof(RoundTable)) +
                  Align(L * kMaxBatch * sizeof(void*)) * 3 +   // conv / k / v
                  Align(L * kMaxBatch * 4) +                   // capacity
                  Align(m.items_capacity * sizeof(lfm3_attention_item)) * 2;
  m.table = Buffer(m.table_bytes);
  m.staging = std::make_unique<PinnedBuffer>(m.table_bytes);
  m.attn_ws_bytes = lfm3_attention_workspace_bytes(
      std::uint32_t(m.items_capacity), kMaxBatch, c.heads, c.heads, c.head_dim);
  m.attn_ws = Buffer(m.attn_ws_bytes);
  m.max_context = max_context;
}

}  // namespace
}  // namespace lfm3amd

extern "C" {

int lfm3_model_load(const lfm3_config* config, const lfm3_tensor* tensors,
                    std::size_t count, lfm3_model** out) {
  if (!out)
    return Fail(LFM3_E_INVALID, "null model output");
  *out = nullptr;
  try {
    if (!config || !tensors)
      Invalid("null LFM3 config or tensors");
    const lfm3_config& c = *config;
    ValidateConfig(c);
    if (count != LFM3_GLOBAL_TENSORS + std::size_t(c.n_layers) * LFM3_LAYER_TENSORS)
      Invalid("LFM3 tensor list must describe every layer");
    auto m = std::make_unique<lfm3_model>();
    m->kv_heads.assign(c.kv_heads, c.kv_heads + c.n_layers);
    m->layer_type.assign(c.layer_type, c.layer_type + c.n_layers);
    m->config = c;
    m->config.kv_heads = m->kv_heads.data();
    m->config.layer_type = m->layer_type.data();
    const std::uint32_t H = c.hidden, F = c.intermediate, D = c.head_dim;
    ValidateTensors(c, tensors);
    const std::uint32_t mt = MatrixType(tensors);
    m->exact = mt != LFM3_TYPE_Q8_0;
    m->wtype = mt;
    Check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate");
    Check(hipStreamCreateWithFlags(&m->prompt_stream, hipStreamNonBlocking), "hipStreamCreate");

    const lfm3_tensor& emb = tensors[0];
    CheckTensor(emb, H, c.vocab, mt, "token_embd.weight");
    m->embedding = PackMatrix({{&emb, 0, 1}}, RowTiles(c.vocab), c.vocab, H);
    const lfm3_tensor& outw = tensors[1];
    m->tied = !outw.data || outw.data == emb.data;
    if (!m->tied) {
      CheckTensor(outw, H, c.vocab, mt, "output.weight");
      m->output = PackMatrix({{&outw, 0, 1}}, RowTiles(c.vocab), c.vocab, H);
    }
    CheckTensor(tensors[2], H, 1, LFM3_TYPE_F32, "output_norm.weight");
    m->output_norm = UploadFloats(static_cast<const float*>(tensors[2].data), H);
    CheckTensor(tensors[3], D / 2, 1, LFM3_TYPE_F32, "rope_freqs.weight");
    const auto* factors = static_cast<const float*>(tensors[3].data);
    for (std::uint32_t i = 0; i < D / 2; ++i)
      if (!std::isfinite(factors[i]) || !(factors[i] > 0))
        Invalid("invalid LFM3 RoPE factor");
    m->factors = UploadFloats(factors, D / 2);
    // reference.cpp:29-43: theta^(-2i/D) in FP32, as the oracle forms it.
    std::vector<float> fg(D / 2), fs(D / 2);
    for (std::uint32_t i = 0; i < D / 2; ++i) {
      fg[i] = std::pow(c.theta, -2.0F * float(i) / float(D));
      fs[i] = std::pow(c.theta_swa, -2.0F * float(i) / float(D));
    }
    m->freq_global = UploadFloats(fg.data(), D / 2);
    m->freq_sliding = UploadFloats(fs.data(), D / 2);

    std::uint32_t proj_rows = 3 * H;
    for (std::uint32_t i = 0; i < c.n_layers; ++i) {
      const lfm3_tensor* t = tensors + LFM3_GLOBAL_TENSORS + std::size_t(i) * LFM3_LAYER_TENSORS;
      Layer l;
      l.type = c.layer_type[i];
      l.kv = c.kv_heads[i];
      CheckTensor(t[0], H, 1, LFM3_TYPE_F32, "attn_norm.weight");
      CheckTensor(t[1], H, 1, LFM3_TYPE_F32, "ffn_norm.weight");
      l.norm = UploadFloats(static_cast<const float*>(t[0].data), H);
      l.ffn_norm = UploadFloats(static_cast<const float*>(t[1].data), H);
      if (bool(t[2].data) != bool(t[3].data))
        Invalid("LFM3 requires both post norms or neither");
      if (t[2].data) {
        CheckTensor(t[2], H, 1, LFM3_TYPE_F32, "post_attention_norm.weight");
        CheckTensor(t[3], H, 1, LFM3_TYPE_F32, "post_ffw_norm.weight");
        l.post_norm = UploadFloats(static_cast<const float*>(t[2].data), H);
        l.post_ffn_norm = UploadFloats(static_cast<const float*>(t[3].data), H);
      }
      CheckTensor(t[4], H, F, mt, "ffn_gate.weight");
      CheckTensor(t[5], H, F, mt, "ffn_up.weight");
      CheckTensor(t[6], F, H, mt, "ffn_down.weight");
      l.ffn = PackMatrix({{&t[4], 0, 2}, {&t[5], 1, 2}}, 2 * RowTiles(F), F, H);
      l.down = PackMatrix({{&t[6], 0, 1}}, RowTiles(H), H, F);
      if (l.type == LFM3_LAYER_CONV) {
        CheckTensor(t[7], c.conv_width, H, LFM3_TYPE_F32, "shortconv.conv.weight");
        CheckTensor(t[8], H, 3 * H, mt, "shortconv.in_proj.weight");
        CheckTensor(t[9], H, H, mt, "shortconv.out_proj.weight");
        l.conv = UploadFloats(static_cast<const float*>(t[7].data),
                              std::size_t(H) * c.conv_width);
        l.in_proj = PackMatrix({{&t[8], 0, 1}}, RowTiles(3 * H), 3 * H, H);
        l.out_proj = PackMatrix({{&t[9], 0, 1}}, RowTiles(H), H, H);
      } else {
        const std::uint32_t qr = c.heads * D, kr = l.kv * D;
        CheckTensor(t[10], H, qr, mt, "attn_q.weight");
        CheckTensor(t[11], H, kr, mt, "attn_k.weight");
        CheckTensor(t[12], H, kr, mt, "attn_v.weight");
        CheckTensor(t[13], D, 1, LFM3_TYPE_F32, "attn_q_norm.weight");
        CheckTensor(t[14], D, 1, LFM3_TYPE_F32, "attn_k_norm.weight");
        CheckTensor(t[15], H, c.heads, mt, "attn_gate.weight");
        CheckTensor(t[16], qr, H, mt, "attn_output.weight");
        const std::uint32_t tq = RowTiles(qr), tk = RowTiles(kr), tg = RowTiles(c.heads);
        l.q_off = 0;
        l.k_off = tq * kTileRows;
        l.v_off = (tq + tk) * kTileRows;
        l.g_off = (tq + 2 * tk) * kTileRows;
        l.qkvg_ld = (tq + 2 * tk + tg) * kTileRows;
        l.qkvg = PackMatrix({{&t[10], 0, 1}, {&t[11], tq, 1}, {&t[12], tq + tk, 1},
                             {&t[15], tq + 2 * tk, 1}},
                            tq + 2 * tk + tg, l.qkvg_ld, H);
        l.attn_out = PackMatrix({{&t[16], 0, 1}}, RowTiles(H), H, qr);
        l.q_norm = UploadFloats(static_cast<const float*>(t[13].data), D);
        l.k_norm = UploadFloats(static_cast<const float*>(t[14].data), D);
        proj_rows = std::max(proj_rows, l.qkvg_ld);
      }
      m->layers.push_back(std::move(l));
    }
    // Round scratch for up to kMaxBatch rows.
    m->proj_ld = (proj_rows + 3) / 4 * 4;
    const std::size_t B = kMaxBatch;
    m->x = Buffer(B * H * 4);
    m->proj = Buffer(B * m->proj_ld * 4);
    m->a = Buffer(B * std::max<std::size_t>(H, std::size_t(c.heads) * D) * 4);
    m->hidden = Buffer(B * F * 4);
    std::size_t out_parts = lfm3_q8_gemv_parts(H, F);
    out_parts = std::max<std::size_t>(out_parts, lfm3_q8_gemv_parts(H, H));
    out_parts = std::max<std::size_t>(out_parts, lfm3_q8_gemv_parts(H, c.heads * D));
    if (m->exact) {
      out_parts = std::max<std::size_t>(out_parts, lfm3_bf16_gemv_parts(H, F, B));
      out_parts = std::max<std::size_t>(out_parts, lfm3_bf16_gemv_parts(H, H, B));
      out_parts = std::max<std::size_t>(out_parts, lfm3_bf16_gemv_parts(H, c.heads * D, B));
      m->z = Buffer(B * H * 4);
      m->head_out = Buffer(B * std::size_t(c.vocab) * 4);
    }
    m->out = Buffer(out_parts * B * H * 4);
    std::size_t ws = lfm3_gemv_workspace_bytes(c.vocab, H, B);
    for (const auto& l : m->layers) {
      ws = std::max(ws, lfm3_gemv_workspace_bytes(F, H, B));
      ws = std::max(ws, lfm3_gemv_workspace_bytes(H, F, B));
      if (l.type == LFM3_LAYER_CONV) {
        ws = std::max(ws, lfm3_gemv_workspace_bytes(3 * H, H, B));
        ws = std::max(ws, lfm3_gemv_workspace_bytes(H, H, B));
      } else {
        ws = std::max(ws, lfm3_gemv_workspace_bytes(l.qkvg_ld, H, B));
        ws = std::max(ws, lfm3_gemv_workspace_bytes(H, c.heads * D, B));
      }
    }
    m->gemv_ws_bytes = std::max<std::size_t>(ws, 256);
    m->gemv_ws = Buffer(m->gemv_ws_bytes);
    m->head_groups = HeadGemvGroups(c.vocab, H);
    m->head_keys = Buffer(std::size_t(B) * m->head_groups * sizeof(unsigned long long));
    m->image = Buffer(lfm3_operand_image_bytes(H));
    m->exps = Buffer(kMaxBatch * sizeof(int));
    m->norm_flags = Buffer(kFlagWords * sizeof(unsigned));
    m->wait_error = std::make_unique<PinnedBuffer>(sizeof(unsigned),
                                                   hipHostMallocMapped | hipHostMallocCoherent);
    *static_cast<unsigned*>(m->wait_error->p) = 0;
    // Mapped and coherent (fine-grained): the last kernel's stores reach
    // host memory without a cache flush; the host reads them after the
    // stream synchronization that ends the round.
    m->ids_host = std::make_unique<PinnedBuffer>(std::size_t(B) * 4,
                                                 hipHostMallocMapped | hipHostMallocCoherent);
    // The sampler's workspace at its largest top-k (2 MB at vocab 128000)
    // and its input staging, made here so that no round allocates.
    m->sample_ws_bytes = SampleWorkspaceBytes(kMaxBatch, c.vocab, kSampleMaxTopK);
    m->sample_ws = Buffer(m->sample_ws_bytes);
    m->sample_table = Buffer(SampleTableBytes());
    m->sample_staging = std::make_unique<PinnedBuffer>(SampleTableBytes());
    m->one_row = Buffer(std::size_t(H) * 4);
    Check(hipDeviceSynchronize(), "model upload");
    *out = m.release();
    return LFM3_OK;
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  } catch (const std::bad_alloc&) {
    return Fail(LFM3_E_NOMEM, "out of host memory");
  } catch (const std::exception& e) {
    return Fail(LFM3_E_INVALID, e.what());
  }
}

void lfm3_model_destroy(lfm3_model* model) { delete model; }

void* lfm3_model_stream(lfm3_model* model) { return model ? model->stream : nullptr; }

int lfm3_session_create(lfm3_model* m, std::uint32_t context, lfm3_session** out) {
  if (!out)
    return Fail(LFM3_E_INVALID, "null session output");
  *out = nullptr;
  try {
    if (!m || !context || context > m->config.context)
      Invalid("invalid LFM3 context");
    const auto& c = m->config;
    auto s = std::make_unique<lfm3_session>();
    s->model = m;
    s->context = context;
    for (std::uint32_t i = 0; i < c.n_layers; ++i) {
      lfm3_session::State st;
      if (c.layer_type[i] == LFM3_LAYER_CONV) {
        st.conv = Buffer(std::size_t(c.hidden) * (c.conv_width - 1) * 4);
      } else {
        // engine.cpp:60-77: sliding rings keep min(context, window) rows.
        st.capacity = c.layer_type[i] == LFM3_LAYER_SLIDING
                          ? std::min(context, c.window)
                          : context;
        const std::size_t n = std::size_t(st.capacity) * c.kv_heads[i] * c.head_dim * 2;
        st.k = Buffer(n);
        st.v = Buffer(n);
      }
      s->states.push_back(std::move(st));
    }
    s->logits = Buffer(std::size_t(c.vocab) * 4);
    s->frontier = Buffer(std::size_t(c.hidden) * 4);
    std::lock_guard<std::mutex> guard(m->lock);
    EnsureRoundBuffers(*m, context);
    *out = s.release();
    return LFM3_OK;
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  } catch (const std::exception& e) {
    return Fail(LFM3_E_NOMEM, e.what());
  }
}

void lfm3_session_destroy(lfm3_session* s) { delete s; }

std::uint32_t lfm3_session_position(const lfm3_session* s) { return s ? s->position : 0; }

int lfm3_session_is_coherent(const lfm3_session* s) { return s && !s->poisoned; }

std::uint32_t lfm3_session_ring_capacity(const lfm3_session* s, std::uint32_t layer) {
  return s && layer < s->states.size() ? s->states[layer].capacity : 0;
}

// engine.cpp:1300-1332: zero the convolution history, position 0, healthy.
// The session's work runs on the model's non-blocking stream, which is not
// ordered against the null stream: the clears go on that stream, between
// two synchronizations, as the reference's Reset does.
int lfm3_session_reset(lfm3_session* s) {
  if (!s)
    return Fail(LFM3_E_INVALID, "null session");
  if (s->hooks.before_reset && s->hooks.before_reset(s->hooks.user))
    return Fail(LFM3_E_REFUSED, "LFM3 continuation hook refused the reset");
  const auto& c = s->model->config;
  const hipStream_t stream = s->model->stream;
  std::lock_guard<std::mutex> guard(s->model->lock);
  int e = HipStatus(hipStreamSynchronize(stream), "reset");
  for (auto& st : s->states)
    if (!e && st.conv.p)
      e = HipStatus(
          hipMemsetAsync(st.conv.p, 0, std::size_t(c.hidden) * (c.conv_width - 1) * 4, stream),
          "reset");
  if (!e)
    e = HipStatus(hipStreamSynchronize(stream), "reset");
  if (e)
    return e;
  s->position = 0;
  s->logits_ready = false;
  s->poisoned = false;
  return LFM3_OK;
}

int lfm3_session_state(lfm3_session* s, int kind, std::uint32_t layer,
                       void** data, std::size_t* bytes) {
  if (!s || !data)
    return Fail(LFM3_E_INVALID, "null session state query");
  Buffer* b = nullptr;
  switch (kind) {
    case LFM3_STATE_LOGITS: b = &s->logits; break;
    case LFM3_STATE_FRONTIER: b = &s->frontier; break;
    case LFM3_STATE_CONV:
    case LFM3_STATE_KEY:
    case LFM3_STATE_VALUE:
      if (layer >= s->states.size())
        return Fail(LFM3_E_INVALID, "LFM3 layer out of range");
      b = kind == LFM3_STATE_CONV ? &s->states[layer].conv
          : kind == LFM3_STATE_KEY ? &s->states[layer].k
                                   : &s->states[layer].v;
      break;
    default:
      return Fail(LFM3_E_INVALID, "unknown LFM3 state kind");
  }
  *data = b->p;
  if (bytes)
    *bytes = b->bytes;
  return b->p ? LFM3_OK : Fail(LFM3_E_INVALID, "LFM3 layer has no such state");
}

// Session::BeginRestore (engine.cpp:1372-1377): work in flight drains, and
// the session refuses work until lfm3_session_set_position.
int lfm3_session_begin_restore(lfm3_session* s) {
  if (!s)
    return Fail(LFM3_E_INVALID, "null session");
  std::lock_guard<std::mutex> guard(s->model->lock);
  const int e = HipStatus(hipStreamSynchronize(s->model->stream), "begin restore");
  if (e)
    return e;
  s->poisoned = true;
  return LFM3_OK;
}

// Session::FinishRestore (engine.cpp:1378-1384): the caller wrote every
// state row, the logits row included, so the logits are served as written.
int lfm3_session_set_position(lfm3_session* s, std::uint32_t position) {
  if (!s || position > s->context)
    return Fail(LFM3_E_INVALID, "invalid LFM3 position");
  s->position = position;
  s->poisoned = false;
  s->logits_ready = true;
  return LFM3_OK;
}

}  // extern "C"

namespace lfm3amd {
namespace {

// The vocabulary head on one FP32 row (the frontier), on stream s.
void HeadRow(lfm3_model& m, const float* row, float* logits, hipStream_t s) {
  const auto& c = m.config;
  const Matrix& head = m.head();
  if (head.exact)
    CheckStatus(lfm3_float_gemv(head.type, head.codes.p, c.vocab, c.hidden, row, c.hidden,
                                logits, c.vocab, 1, 1, 0, s));
  else
    CheckStatus(lfm3_q8_gemv(head.codes.p, head.scales.p, c.vocab, c.hidden, row, c.hidden,
                             logits, c.vocab, 1, nullptr, 0, s));
}

// Session::Impl::EnsureLogits (engine.cpp:237-245): a round or prompt that
// skipped the vocabulary head leaves the frontier row; the head runs on it
// when logits are first wanted.
void EnsureLogits(lfm3_session& se) {
  if (se.logits_ready)
    return;
  lfm3_model& m = *se.model;
  HeadRow(m, se.frontier.as<float>(), se.logits.as<float>(), m.stream);
  Check(hipStreamSynchronize(m.stream), "logits");
  se.logits_ready = true;
}

// Snapshot v2 (engine.cpp:1387-1574): a 32-byte header of little-endian
// words (magic "LFM3", version 2, context, position, hidden, vocab, layers,
// configuration signature), the frontier row and the logits (zeros at
// position 0), then per layer the convolution history [hidden][width - 1]
// f32, or the K rows then the V rows of the ring's first min(position,
// capacity) slots in physical order (F16 [slot][kv_heads][head_dim]).
constexpr std::uint32_t kSnapshotMagic = 0x334d464c, kSnapshotVersion = 2;
constexpr std::size_t kSnapshotHeaderBytes = 32;

// FNV-1a over the little-endian bytes of the configuration words
// (engine.cpp ConfigSignature): restores refuse a snapshot of another shape.
std::uint32_t ConfigSignature(const lfm3_config& c) {
  std::uint32_t hash = 2166136261u;
  const auto mix = [&](std::uint32_t value) {
    for (int i = 0; i < 4; ++i)
      hash = (hash ^ ((value >> (8 * i)) & 255u)) * 16777619u;
  };
  for (std::uint32_t value :
       {c.hidden, c.intermediate, c.vocab, c.heads, c.head_dim, c.window, c.conv_width,
        __builtin_bit_cast(std::uint32_t, c.eps), __builtin_bit_cast(std::uint32_t, c.theta),
        __builtin_bit_cast(std::uint32_t, c.theta_swa)})
    mix(value);
  for (std::uint32_t i = 0; i < c.n_layers; ++i) {
    mix(c.layer_type[i]);
    mix(c.kv_heads[i]);
  }
  return hash;
}

std::size_t RingBytes(const lfm3_config& c, std::uint32_t layer, std::uint32_t slots) {
  return std::size_t(slots) * c.kv_heads[layer] * c.head_dim * sizeof(Half);
}

std::size_t StateBytes(const lfm3_config& c, std::uint32_t position) {
  std::size_t bytes = kSnapshotHeaderBytes + (std::size_t(c.hidden) + c.vocab) * 4;
  for (std::uint32_t i = 0; i < c.n_layers; ++i)
    bytes += c.layer_type[i] == LFM3_LAYER_CONV
                 ? std::size_t(c.hidden) * (c.conv_width - 1) * 4
                 : 2 * RingBytes(c, i,
                                 c.layer_type[i] == LFM3_LAYER_SLIDING
                                     ? std::min(position, c.window)
                                     : position);
  return bytes;
}

void PutWord(std::uint8_t* p, std::size_t word, std::uint32_t value) {
  for (int i = 0; i < 4; ++i)
    p[word * 4 + i] = std::uint8_t(value >> (8 * i));
}
std::uint32_t GetWord(const std::uint8_t* p, std::size_t word) {
  std::uint32_t value = 0;
  for (int i = 0; i < 4; ++i)
    value |= std::uint32_t(p[word * 4 + i]) << (8 * i);
  return value;
}

}  // namespace
}  // namespace lfm3amd

extern "C" {

int lfm3_session_read_logits(const lfm3_session* s, float* logits) {
  if (!s || !logits)
    return Fail(LFM3_E_INVALID, "null logits");
  // engine.cpp Session::ReadLogits: a poisoned session or one without a
  // frontier row has no logits.
  if (s->poisoned || !s->position)
    return Fail(LFM3_E_INVALID, "invalid LFM3 logit frontier");
  std::lock_guard<std::mutex> guard(s->model->lock);
  try {
    EnsureLogits(const_cast<lfm3_session&>(*s));
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  const hipStream_t stream = s->model->stream;
  int e = HipStatus(hipMemcpyAsync(logits, s->logits.p, std::size_t(s->model->config.vocab) * 4,
                                   hipMemcpyDeviceToHost, stream),
                    "read logits");
  if (!e)
    e = HipStatus(hipStreamSynchronize(stream), "read logits");
  return e;
}

// Session::PrepareLogits (engine.hpp:146, engine.cpp:1369-1373): after a
// round or prompt that skipped the vocabulary head, the head runs on the
// frontier row on the model stream, so the device logits row
// (LFM3_STATE_LOGITS) holds the frontier's logits; nothing is copied to
// the host. The continuation adapter calls it before it captures the
// logits component (continuation_adapter.cpp:369-370).
int lfm3_session_prepare_logits(lfm3_session* s) {
  if (!s)
    return Fail(LFM3_E_INVALID, "null session");
  if (s->poisoned || !s->position)
    return Fail(LFM3_E_INVALID, "invalid LFM3 logit frontier");
  std::lock_guard<std::mutex> guard(s->model->lock);
  try {
    EnsureLogits(*s);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  return LFM3_OK;
}

std::size_t lfm3_session_snapshot_bytes(const lfm3_session* s) {
  return s ? StateBytes(s->model->config, s->position) : 0;
}

int lfm3_session_save_snapshot(lfm3_session* s, void* out, std::size_t bytes) {
  if (!s || !out || bytes != lfm3_session_snapshot_bytes(s))
    return Fail(LFM3_E_INVALID, "invalid LFM3 snapshot buffer");
  if (s->poisoned)
    return Fail(LFM3_E_STATE, "cannot snapshot a poisoned LFM3 session");
  const auto& c = s->model->config;
  auto* p = static_cast<std::uint8_t*>(out);
  std::lock_guard<std::mutex> guard(s->model->lock);
  try {
    if (s->position)
      EnsureLogits(*s);
    const std::uint32_t header[8] = {kSnapshotMagic, kSnapshotVersion, s->context,
                                     s->position,    c.hidden,         c.vocab,
                                     c.n_layers,     ConfigSignature(c)};
    for (std::size_t i = 0; i < 8; ++i)
      PutWord(p, i, header[i]);
    std::size_t offset = kSnapshotHeaderBytes;
    // Copies on the session stream, after its work and before the return.
    const hipStream_t stream = s->model->stream;
    Check(hipStreamSynchronize(stream), "snapshot");
    const auto copy = [&](const void* source, std::size_t size) {
      if (size)
        Check(hipMemcpyAsync(p + offset, source, size, hipMemcpyDeviceToHost, stream),
              "snapshot copy");
      offset += size;
    };
    if (s->position) {
      copy(s->frontier.p, std::size_t(c.hidden) * 4);
      copy(s->logits.p, std::size_t(c.vocab) * 4);
    } else {
      std::memset(p + offset, 0, (std::size_t(c.hidden) + c.vocab) * 4);
      offset += (std::size_t(c.hidden) + c.vocab) * 4;
    }
    for (std::uint32_t i = 0; i < c.n_layers; ++i) {
      const auto& st = s->states[i];
      if (st.conv.p) {
        copy(st.conv.p, std::size_t(c.hidden) * (c.conv_width - 1) * 4);
      } else {
        const std::size_t size = RingBytes(c, i, std::min(s->position, st.capacity));
        copy(st.k.p, size);
        copy(st.v.p, size);
      }
    }
    Check(hipStreamSynchronize(stream), "snapshot");
    return LFM3_OK;
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
}

int lfm3_session_restore_snapshot(lfm3_session* s, const void* data, std::size_t bytes) {
  if (!s || !data)
    return Fail(LFM3_E_INVALID, "invalid LFM3 snapshot payload");
  // engine.cpp:1522-1524: the hook runs before the header is checked.
  if (s->hooks.before_restore && s->hooks.before_restore(s->hooks.user))
    return Fail(LFM3_E_REFUSED, "LFM3 continuation hook refused the restore");
  const auto& c = s->model->config;
  const auto* p = static_cast<const std::uint8_t*>(data);
  // The whole header and the size are checked before any state changes.
  if (bytes < kSnapshotHeaderBytes || GetWord(p, 0) != kSnapshotMagic ||
      GetWord(p, 1) != kSnapshotVersion || GetWord(p, 2) != s->context ||
      GetWord(p, 3) > s->context || GetWord(p, 4) != c.hidden || GetWord(p, 5) != c.vocab ||
      GetWord(p, 6) != c.n_layers || GetWord(p, 7) != ConfigSignature(c) ||
      bytes != StateBytes(c, GetWord(p, 3)))
    return Fail(LFM3_E_INVALID, "invalid LFM3 snapshot payload");
  const std::uint32_t position = GetWord(p, 3);
  std::size_t offset = kSnapshotHeaderBytes;
  const hipStream_t stream = s->model->stream;
  std::lock_guard<std::mutex> guard(s->model->lock);
  try {
    Check(hipStreamSynchronize(stream), "restore");
    const auto copy = [&](void* destination, std::size_t size) {
      if (size)
        Check(hipMemcpyAsync(destination, p + offset, size, hipMemcpyHostToDevice, stream),
              "restore copy");
      offset += size;
    };
    copy(s->frontier.p, std::size_t(c.hidden) * 4);
    copy(s->logits.p, std::size_t(c.vocab) * 4);
    for (std::uint32_t i = 0; i < c.n_layers; ++i) {
      auto& st = s->states[i];
      if (st.conv.p) {
        copy(st.conv.p, std::size_t(c.hidden) * (c.conv_width - 1) * 4);
      } else {
        const std::size_t size = RingBytes(c, i, std::min(position, st.capacity));
        copy(st.k.p, size);
        copy(st.v.p, size);
      }
    }
    Check(hipStreamSynchronize(stream), "restore");
  } catch (const Error& e) {
    s->poisoned = true;  // a partial restore leaves no coherent state
    return Fail(e.status, e.what());
  }
  s->position = position;
  s->logits_ready = position != 0;
  s->poisoned = false;
  return LFM3_OK;
}

}  // extern "C"

namespace lfm3amd {
namespace {

// One decode round of n rows (engine.cpp:257-527, batch branch): every
// launch, enqueued on the model stream; FinishRound advances the sessions
// once the stream has drained.
void EnqueueRound(lfm3_model& m, lfm3_session* const* sessions, std::uint32_t n,
                  const std::uint32_t* tokens, bool greedy, const float* const* inputs,
                  bool head) {
  const auto& c = m.config;
  const std::uint32_t H = c.hidden, F = c.intermediate, D = c.head_dim;
  const std::uint32_t L = c.n_layers;
  const hipStream_t s = m.stream;
  std::uint32_t max_context = 0;
  for (std::uint32_t i = 0; i < n; ++i)
    max_context = std::max(max_context, sessions[i]->context);
  EnsureRoundBuffers(m, max_context);

  // Host side of the round's index tables, then one upload.
  auto* host = static_cast<std::uint8_t*>(m.staging->p);
  std::memset(host, 0, m.table_bytes);
  auto* rt = reinterpret_cast<RoundTable*>(host);
  std::size_t off = Align(sizeof(RoundTable));
  const std::size_t conv_off = off;
  off += Align(L * kMaxBatch * sizeof(void*));
  const std::size_t k_off = off;
  off += Align(L * kMaxBatch * sizeof(void*));
  const std::size_t v_off = off;
  off += Align(L * kMaxBatch * sizeof(void*));
  const std::size_t cap_off = off;
  off += Align(L * kMaxBatch * 4);
  const std::size_t items_full_off = off;
  off += Align(m.items_capacity * sizeof(lfm3_attention_item));
  const std::size_t items_swa_off = off;
  auto** conv_ptr = reinterpret_cast<float**>(host + conv_off);
  auto** k_ptr = reinterpret_cast<Half**>(host + k_off);
  auto** v_ptr = reinterpret_cast<Half**>(host + v_off);
  auto* cap = reinterpret_cast<std::uint32_t*>(host + cap_off);
  for (std::uint32_t i = 0; i < n; ++i) {
    lfm3_session& se = *sessions[i];
    rt->tokens[i] = tokens[i];
    rt->inputs[i] = inputs ? inputs[i] : nullptr;
    rt->positions[i] = se.position;
    rt->logits[i] = se.logits.as<float>();
    rt->frontier[i] = se.frontier.as<float>();
    for (std::uint32_t l = 0; l < L; ++l) {
      conv_ptr[l * kMaxBatch + i] = se.states[l].conv.as<float>();
      k_ptr[l * kMaxBatch + i] = se.states[l].k.as<Half>();
      v_ptr[l * kMaxBatch + i] = se.states[l].v.as<Half>();
      cap[l * kMaxBatch + i] = se.states[l].capacity;
    }
  }
  const int n_full = lfm3_attention_plan(
      rt->positions, n, 0,
      reinterpret_cast<lfm3_attention_item*>(host + items_full_off),
      std::uint32_t(m.items_capacity));
  const int n_swa = lfm3_attention_plan(
      rt->positions, n, c.window,
      reinterpret_cast<lfm3_attention_item*>(host + items_swa_off),
      std::uint32_t(m.items_capacity));
  if (n_full < 0 || n_swa < 0)
    throw Error(LFM3_E_INVALID, lfm3_last_error());
  auto* dev = m.table.as<std::uint8_t>();
  Check(hipMemcpyAsync(dev, host, m.table_bytes, hipMemcpyHostToDevice, s), "table upload");
  const auto* d_rt = reinterpret_cast<const RoundTable*>(dev);

  float* x = m.x.as<float>();
  float* proj = m.proj.as<float>();
  float* a = m.a.as<float>();
  float* hid = m.hidden.as<float>();
  float* out = m.out.as<float>();
  const std::uint32_t pld = std::uint32_t(m.proj_ld);

  if (m.exact) {
    // The float-weight round (every projection an exact float x FP32 GEMV,
    // hip/ops.hip:2230-2249): FP32 normed rows z feed the GEMVs; narrow
    // outputs split K into parts that the next norm adds.
    float* z = m.z.as<float>();
    const auto bgemv = [&](const Matrix& w, const float* in, std::uint32_t ldx, float* y,
                           std::uint32_t ldy, std::uint32_t parts, bool swiglu) {
      CheckStatus(lfm3_float_gemv(w.type, w.codes.p, w.rows, w.cols, in, ldx, y, ldy, n, parts,
                                  swiglu ? 1 : 0, s));
    };
    const auto bparts = [&](const Matrix& w, const float* in, std::uint32_t ldx) {
      const std::uint32_t parts = lfm3_bf16_gemv_parts(w.rows, w.cols, n);
      bgemv(w, in, ldx, out, H, parts, false);
      return parts;
    };
    const auto norm = [&](std::uint32_t parts, const float* post, const float* weight) {
      CheckStatus(lfm3_residual_norm_parts(parts ? out : nullptr, parts ? parts : 1,
                                           std::size_t(n) * H, parts ? post : nullptr, x, weight,
                                           z, n, H, c.eps, s));
    };
    CheckStatus(lfm3_float_embed(m.wtype, m.embedding.codes.p, c.vocab, H, d_rt->tokens,
                                 inputs ? d_rt->inputs : nullptr, n, x, s));
    norm(0, nullptr, m.layers[0].norm.as<float>());
    for (std::uint32_t il = 0; il < L; ++il) {
      const Layer& l = m.layers[il];
      std::uint32_t parts;
      if (l.type == LFM3_LAYER_CONV) {
        bgemv(l.in_proj, z, H, proj, 3 * H, 1, false);
        CheckStatus(lfm3_conv_step_ragged(
            proj, 3 * H, l.conv.as<float>(),
            reinterpret_cast<float* const*>(dev + conv_off) + il * kMaxBatch, a, H, n, H,
            c.conv_width, s));
        parts = bparts(l.out_proj, a, H);
      } else {
        const bool swa = l.type == LFM3_LAYER_SLIDING;
        bgemv(l.qkvg, z, H, proj, pld, 1, false);
        const auto* kp = reinterpret_cast<std::uint16_t* const*>(dev + k_off) + il * kMaxBatch;
        const auto* vp = reinterpret_cast<std::uint16_t* const*>(dev + v_off) + il * kMaxBatch;
        const auto* cp = reinterpret_cast<const std::uint32_t*>(dev + cap_off) + il * kMaxBatch;
        const auto* items = reinterpret_cast<const lfm3_attention_item*>(
            dev + (swa ? items_swa_off : items_full_off));
        CheckStatus(lfm3_decode_heads_attention_ragged(
            proj + l.q_off, proj + l.k_off, proj + l.v_off, pld, proj + l.g_off, pld,
            l.q_norm.as<float>(), l.k_norm.as<float>(),
            swa ? m.freq_sliding.as<float>() : m.freq_global.as<float>(),
            swa ? nullptr : m.factors.as<float>(), kp, vp, d_rt->positions, cp, items,
            std::uint32_t(swa ? n_swa : n_full), a, c.heads * D, n, c.heads, l.kv, D, c.eps,
            m.attn_ws.p, m.attn_ws_bytes, s));
        parts = bparts(l.attn_out, a, c.heads * D);
      }
      norm(parts, l.post_norm.as<float>(), l.ffn_norm.as<float>());
      bgemv(l.ffn, z, H, hid, F, 1, true);
      parts = bparts(l.down, hid, F);
      const bool last = il + 1 == L;
      norm(parts, l.post_ffn_norm.as<float>(),
           last ? m.output_norm.as<float>() : m.layers[il + 1].norm.as<float>());
    }
    // The final normed rows are the frontier rows (engine.cpp:505-511).
    CheckStatus(LaunchScatterRows(z, H, d_rt->frontier, n, H, s));
    if (head) {
      const Matrix& w = m.head();
      float* logits = m.head_out.as<float>();
      bgemv(w, z, H, logits, c.vocab, 1, false);
      CheckStatus(LaunchScatterRows(logits, c.vocab, d_rt->logits, n, c.vocab, s));
      if (greedy) {
        lfm3_sampling pick{0.0f, 1, 1.0f};
        CheckStatus(LaunchSample(logits, c.vocab, nullptr, n, c.vocab, pick, nullptr, 0,
                                 nullptr, m.ids(), m.sample_ws.p,
                                 m.sample_ws_bytes, s));
      }
    }
    Check(hipGetLastError(), "round launch");
    return;
  }

  // Narrow matrices (hidden rows) split K into parts whose partial sums the
  // following residual norm adds in part order.
  const auto partials = [&](const Matrix& w, const float* in,
                            std::uint32_t ldx) -> std::uint32_t {
    const std::uint32_t parts = lfm3_q8_gemv_parts(w.rows, w.cols);
    CheckStatus(lfm3_q8_gemv_partials(w.codes.p, w.scales.p, w.rows, w.cols, in,
                                      ldx, out, H, n, parts, s));
    return parts;
  };
  std::uint32_t mixer_parts = 1;

  // Normed rows go out as operand images; the convolution and attention
  // outputs and the FFN hidden state are staged by their GEMVs. Each norm
  // runs inside the launch of the GEMV that consumes its image: the
  // launch's first n blocks are the norm (one row each), and its GEMV
  // blocks stream their weights while they wait for the rows (FusedNorm).
  void* image = m.image.p;
  int* exps = m.exps.as<int>();
  FusedNorm fn;
  fn.args.part_stride = std::size_t(n) * H;
  fn.args.x = x;
  fn.args.H = int(H);
  fn.args.eps = c.eps;
  fn.args.image = static_cast<uint4*>(image);
  fn.args.exps = exps;
  fn.flags = m.norm_flags.as<unsigned>();
  fn.error = static_cast<unsigned*>(m.wait_error->device);
  // The next fused launch's norm: x += post(branch parts), then norm with
  // `weight` (and the FP32 rows to z_rows when given).
  const auto norm = [&](std::uint32_t parts, const float* post, const float* weight,
                        float* const* z_rows) {
    fn.args.branch = parts ? out : nullptr;
    fn.args.parts = parts ? int(parts) : 1;
    fn.args.post = parts ? post : nullptr;
    fn.args.weight = weight;
    fn.args.z_rows = z_rows;
    if (++m.norm_seq == 0)  // 0 is the flags' initial value
      m.norm_seq = 1;
    fn.seq = m.norm_seq;
  };

  // The first norm gathers the round's embedding rows into x.
  fn.args.emb_codes = static_cast<const std::uint8_t*>(m.embedding.codes.p);
  fn.args.emb_scales = static_cast<const std::uint16_t*>(m.embedding.scales.p);
  fn.args.tokens = d_rt->tokens;
  fn.args.inputs = inputs ? d_rt->inputs : nullptr;
  fn.args.vocab = int(c.vocab);
  norm(0, nullptr, m.layers[0].norm.as<float>(), nullptr);
  for (std::uint32_t il = 0; il < L; ++il) {
    const Layer& l = m.layers[il];
    if (l.type == LFM3_LAYER_CONV) {
      // The in projection with the convolution step in its epilogue; the
      // FP32 output is staged by the out projection.
      CheckStatus(LaunchConvImage(
          l.in_proj.codes.p, l.in_proj.scales.p, H, image, exps, n, l.conv.as<float>(),
          reinterpret_cast<float* const*>(dev + conv_off) + il * kMaxBatch, c.conv_width, a,
          H, &fn, s));
      mixer_parts = partials(l.out_proj, a, H);
    } else {
      const bool swa = l.type == LFM3_LAYER_SLIDING;
      CheckStatus(LaunchGemvImageFused(l.qkvg.codes.p, l.qkvg.scales.p, l.qkvg.rows,
                                       l.qkvg.cols, image, exps, n, proj, pld, false, fn, s));
      const auto* kp = reinterpret_cast<std::uint16_t* const*>(dev + k_off) + il * kMaxBatch;
      const auto* vp = reinterpret_cast<std::uint16_t* const*>(dev + v_off) + il * kMaxBatch;
      const auto* cp = reinterpret_cast<const std::uint32_t*>(dev + cap_off) + il * kMaxBatch;
      const auto* items = reinterpret_cast<const lfm3_attention_item*>(
          dev + (swa ? items_swa_off : items_full_off));
      CheckStatus(lfm3_decode_heads_attention_ragged(
          proj + l.q_off, proj + l.k_off, proj + l.v_off, pld, proj + l.g_off,
          pld, l.q_norm.as<float>(), l.k_norm.as<float>(),
          swa ? m.freq_sliding.as<float>() : m.freq_global.as<float>(),
          swa ? nullptr : m.factors.as<float>(), kp, vp, d_rt->positions, cp,
          items, std::uint32_t(swa ? n_swa : n_full), a, c.heads * D, n,
          c.heads, l.kv, D, c.eps, m.attn_ws.p, m.attn_ws_bytes, s));
      mixer_parts = partials(l.attn_out, a, c.heads * D);
    }
    fn.args.tokens = nullptr;
    fn.args.inputs = nullptr;
    norm(mixer_parts, l.post_norm.as<float>(), l.ffn_norm.as<float>(), nullptr);
    CheckStatus(LaunchGemvImageFused(l.ffn.codes.p, l.ffn.scales.p, F, H, image, exps, n, hid,
                                     F, true, fn, s));
    const std::uint32_t ffn_parts = partials(l.down, hid, F);
    const bool last = il + 1 == L;
    // The last norm's FP32 rows are the sessions' frontier rows
    // (engine.cpp:505-511), written in place.
    norm(ffn_parts, l.post_ffn_norm.as<float>(),
         last ? m.output_norm.as<float>() : m.layers[il + 1].norm.as<float>(),
         last ? d_rt->frontier : nullptr);
  }
  // LM head over the final-normed rows into each session's logits row, with
  // per-block greedy candidates; then the greedy ids from the candidates.
  // Without the head the final norm runs alone (the frontier rows).
  if (head) {
    const Matrix& w = m.head();
    auto* keys = m.head_keys.as<unsigned long long>();
    CheckStatus(LaunchHeadGemv(w.codes.p, w.scales.p, w.rows, w.cols, image, exps, n,
                               d_rt->logits, keys, nullptr, s, &fn));
    if (greedy)
      CheckStatus(LaunchArgmaxKeys(keys, n, m.head_groups, m.ids(), s));
  } else {
    CheckStatus(LaunchNormImage(fn.args, n, s));
  }
  Check(hipGetLastError(), "round launch");
}

// A fused launch's wait that timed out (FusedNorm) leaves the round's
// results undefined: the round fails as a device error. Call after the
// model stream has been synchronized.
void CheckRoundWaits(lfm3_model& m) {
  if (!m.wait_error)
    return;
  auto* word = static_cast<volatile unsigned*>(m.wait_error->p);
  if (*word) {
    *word = 0;
    throw Error(LFM3_E_HIP, "LFM3 decode round: a GEMV block's wait for its norm timed out");
  }
}

void FinishRound(lfm3_session* const* sessions, std::uint32_t n, bool head) {
  for (std::uint32_t i = 0; i < n; ++i) {
    ++sessions[i]->position;
    sessions[i]->logits_ready = head;
  }
}

void RunRound(lfm3_model& m, lfm3_session* const* sessions, std::uint32_t n,
              const std::uint32_t* tokens, bool greedy, const float* const* inputs = nullptr,
              bool head = true) {
  EnqueueRound(m, sessions, n, tokens, greedy, inputs, head);
  Check(hipStreamSynchronize(m.stream), "round");
  CheckRoundWaits(m);
  FinishRound(sessions, n, head);
}

// Device logits row -> caller's host row through the model's pinned
// staging row (a DMA copy, then a host memcpy), on the model stream.
void CopyLogits(lfm3_model& m, float* host, const void* device) {
  const std::size_t bytes = std::size_t(m.config.vocab) * 4;
  if (!m.logits_host)
    m.logits_host = std::make_unique<PinnedBuffer>(bytes);
  Check(hipMemcpyAsync(m.logits_host->p, device, bytes, hipMemcpyDeviceToHost, m.stream),
        "logits copy");
  Check(hipStreamSynchronize(m.stream), "logits copy");
  std::memcpy(host, m.logits_host->p, bytes);
}

// The sessions' logits rows into pinned staging, on the model stream
// behind the round's kernels (the round's ids are already written to
// pinned memory by its last kernel); the caller synchronizes the stream
// once and then calls DeliverReadback.
void EnqueueReadback(lfm3_model& m, lfm3_session* const* sessions, std::uint32_t n,
                     bool logits) {
  if (logits) {
    const std::size_t bytes = std::size_t(m.config.vocab) * 4;
    if (!m.rows_host)
      m.rows_host = std::make_unique<PinnedBuffer>(kMaxBatch * bytes);
    for (std::uint32_t i = 0; i < n; ++i)
      Check(hipMemcpyAsync(static_cast<std::uint8_t*>(m.rows_host->p) + i * bytes,
                           sessions[i]->logits.p, bytes, hipMemcpyDeviceToHost, m.stream),
            "logits copy");
  }
}

// Call only after the model stream has been synchronized: the ids are
// written by the round's last kernel, the logits rows by copies on the
// stream.
void DeliverReadback(lfm3_model& m, std::uint32_t n, std::uint32_t* ids, float* const* logits) {
  if (ids)
    std::memcpy(ids, m.ids_host->p, std::size_t(n) * 4);
  if (logits) {
    const std::size_t bytes = std::size_t(m.config.vocab) * 4;
    for (std::uint32_t i = 0; i < n; ++i)
      std::memcpy(logits[i], static_cast<const std::uint8_t*>(m.rows_host->p) + i * bytes, bytes);
  }
}

PromptBuffers& EnsurePromptBuffers(lfm3_model& m) {
  if (m.prompt)
    return *m.prompt;
  const auto& c = m.config;
  const std::size_t R = kPrefillChunk, H = c.hidden, F = c.intermediate, D = c.head_dim;
  auto b = std::make_unique<PromptBuffers>();
  std::size_t widest = std::max<std::size_t>({H, F, std::size_t(c.heads) * D});
  b->lda = (widest + 63) / 64 * 64;
  std::size_t proj_rows = 3 * H, kv_max = 0;
  for (const auto& l : m.layers)
    if (l.type != LFM3_LAYER_CONV) {
      proj_rows = std::max<std::size_t>(proj_rows, l.qkvg_ld);
      kv_max = std::max<std::size_t>(kv_max, l.kv);
    }
  b->proj_ld = (proj_rows + 3) / 4 * 4;
  b->tokens = Buffer(R * 4);
  b->x = Buffer(R * H * 4);
  b->z = Buffer(R * H * 4);
  b->a16 = Buffer(R * b->lda * 2);
  b->scale = Buffer(R * 4);
  b->hid16 = Buffer(R * ((F + 63) / 64 * 64) * 2, false);
  b->hid_scale = Buffer(R * 4, false);
  b->swiglu_flags = Buffer(lfm3_q8_gemm_swiglu_flags_bytes(std::uint32_t(F), std::uint32_t(R)));
  b->wait_error = std::make_unique<PinnedBuffer>(sizeof(unsigned),
                                                 hipHostMallocMapped | hipHostMallocCoherent);
  *static_cast<unsigned*>(b->wait_error->p) = 0;
  b->proj = Buffer(8 * R * b->proj_ld * 4);  // up to 8 K parts
  b->mix = Buffer(R * std::max<std::size_t>(H, std::size_t(c.heads) * D) * 4);
  b->hid = Buffer(R * F * 4);
  b->out = Buffer(8 * R * H * 4);
  b->row_max = Buffer(std::size_t(lfm3_q8_gemm_swiglu_max_blocks(c.intermediate)) * R * 4);
  b->chunk_k = Buffer(R * std::max<std::size_t>(kv_max, 1) * D * 2);
  b->chunk_v = Buffer(R * std::max<std::size_t>(kv_max, 1) * D * 2);
  b->attn_ws_bytes = std::max<std::size_t>(
      std::max(lfm3_prompt_attention_workspace_bytes(std::uint32_t(R), c.heads,
                                                     std::uint32_t(D), c.context, 0),
               lfm3_prompt_attention_half_workspace_bytes(std::uint32_t(R), c.heads,
                                                          std::uint32_t(D), c.context, 0)),
      256);
  b->attn_ws = Buffer(b->attn_ws_bytes);
  b->one_items = lfm3_attention_max_items(1, c.context);
  b->one_bytes = Align(4 * sizeof(void*)) + Align(b->one_items * sizeof(lfm3_attention_item));
  b->one_table = Buffer(b->one_bytes);
  b->one_ws_bytes = std::max<std::size_t>(
      lfm3_attention_workspace_bytes(std::uint32_t(b->one_items), 1, c.heads, c.heads,
                                     std::uint32_t(D)),
      256);
  b->one_ws = Buffer(b->one_ws_bytes);
  b->one_staging = std::make_unique<PinnedBuffer>(b->one_bytes);
  // FP16 tiles of every Q8_0 matrix the prompt GEMMs multiply (every
  // stored tile: gate/up two per 16 output rows), 2 bytes a weight: 2.9 GB
  // at the reference dims. Dropping the per-chunk code decode pays for the
  // doubled tile bytes: about 9% on the 512-token gate/up GEMM, 3% of the
  // pass on the other projections.
  for (auto& l : m.layers) {
    for (Matrix* wp : {&l.ffn, &l.down, &l.in_proj, &l.out_proj, &l.qkvg, &l.attn_out}) {
      Matrix& w = *wp;
      if (w.exact || !w.codes.p)
        continue;
      const std::uint32_t rows = w.tiles * kTileRows;
      w.halves = Buffer(lfm3_q8_half_tiles_bytes(rows, w.cols), false);
      CheckStatus(lfm3_q8_half_tiles(w.codes.p, rows, w.cols, w.halves.p, m.stream));
    }
  }
  Check(hipStreamSynchronize(m.stream), "FP16 tiles");
  m.prompt = std::move(b);
  return *m.prompt;
}

// Trailing-row pruning (engine.cpp:304-323): only the frontier row leaves
// the last layer, so trailing layers skip rows nothing reads. Walking back,
// a convolution needs conv_width - 1 earlier rows for its outputs and
// history, and an attention layer needs every row for its K/V (a sliding
// one also for its ring). Layer i reads the last live_in[i] rows and
// updates the last live_out[i] rows of the residual stream.
void PruneRows(const lfm3_config& c, std::uint32_t n, std::vector<std::uint32_t>& live_in,
               std::vector<std::uint32_t>& live_out) {
  live_in.assign(c.n_layers, n);
  live_out.assign(c.n_layers, n);
  std::uint32_t need = 1;
  for (std::uint32_t i = c.n_layers; i-- > 0;) {
    if (c.layer_type[i] == LFM3_LAYER_SLIDING)
      break;
    live_out[i] = std::min(n, need);
    if (c.layer_type[i] == LFM3_LAYER_FULL)
      break;
    need = std::min(n, need + c.conv_width - 1);
    live_in[i] = need;
  }
}

// One prompt chunk of n rows of one session (engine.cpp:257-527, the
// single-session branch; Session::Forward engine.cpp:882-938 calls it per
// kPrefillChunk tokens). Rows from kPromptRows on enter the projections as
// FP16 row-scaled activations on the MFMA GEMM; fewer rows use the FP32
// GEMV (hip/ops.hpp:32). The convolution continues the session's history;
// full-attention K/V rows are written in place into the cache (the ring
// does not wrap), sliding ones are staged and stored to the ring after
// attention read its history (engine.cpp:437-470).
// The input rows of a chunk, in row order: runs of token ids (host memory)
// and runs of FP32 rows of hidden floats (host memory, or device memory
// ordered before the call).
struct ChunkPart {
  std::uint32_t count = 0;
  const std::uint32_t* tokens = nullptr;
  const float* rows = nullptr;
  bool on_device = false;
};

void RunPrompt(lfm3_model& m, lfm3_session& se, const std::vector<ChunkPart>& input,
               std::uint32_t n, bool want_logits, hipStream_t s) {
  const auto& c = m.config;
  const std::uint32_t H = c.hidden, F = c.intermediate, D = c.head_dim;
  const std::uint32_t L = c.n_layers, position = se.position;
  PromptBuffers& b = EnsurePromptBuffers(m);
  std::vector<std::uint32_t> live_in, live_out;
  PruneRows(c, n, live_in, live_out);

  float* x = b.x.as<float>();
  float* z = b.z.as<float>();
  float* proj = b.proj.as<float>();
  float* mix = b.mix.as<float>();
  float* hid = b.hid.as<float>();
  float* out = b.out.as<float>();
  auto* a16 = b.a16.as<std::uint16_t>();
  float* scale = b.scale.as<float>();
  auto* row_max = b.row_max.as<unsigned>();
  const std::uint32_t lda = std::uint32_t(b.lda), pld = std::uint32_t(b.proj_ld);

  // a16 / scale hold FP16 row-scaled GEMM inputs. The residual norms write
  // them at the absolute chunk row (row r at a16 + r lda), so a pruned
  // consumer reads its last rows at the same offset; other GEMM inputs (the
  // convolution and attention outputs, the FFN hidden rows) are converted
  // into rows 0.. by `halves`.
  const std::uint32_t max_blocks = lfm3_q8_gemm_swiglu_max_blocks(F);
  const auto halves = [&](const float* in, std::uint32_t ldx, const unsigned* rmax,
                          std::uint32_t rows, std::uint32_t cols) {
    CheckStatus(lfm3_half_rows(in, ldx, rmax, rmax ? max_blocks : 0, a16, lda, scale, rows,
                               cols, s));
  };
  // Float-weight models run every projection through the exact float GEMV
  // over all rows at once (hip/ops.hip:2230-2249 for float tensors).
  const std::uint32_t mfma_rows = m.exact ? 0xffffffffu : kPromptRows;
  const auto gemv = [&](const Matrix& w, const float* in, std::uint32_t ldx, float* y,
                        std::uint32_t ldy, std::uint32_t rows, bool swiglu) {
    if (w.exact) {
      CheckStatus(lfm3_float_gemv(w.type, w.codes.p, swiglu ? F : w.rows, w.cols, in, ldx, y,
                                  ldy, rows, 1, swiglu ? 1 : 0, s));
      return;
    }
    for (std::uint32_t r = 0; r < rows; r += kMaxBatch) {
      const std::uint32_t k = std::min(kMaxBatch, rows - r);
      if (swiglu)
        CheckStatus(lfm3_q8_gemv_swiglu(w.codes.p, w.scales.p, F, H, in + std::size_t(r) * ldx,
                                        ldx, y + std::size_t(r) * ldy, ldy, k, nullptr, 0, s));
      else
        CheckStatus(lfm3_q8_gemv(w.codes.p, w.scales.p, w.rows, w.cols,
                                 in + std::size_t(r) * ldx, ldx, y + std::size_t(r) * ldy, ldy,
                                 k, nullptr, 0, s));
    }
  };
  const auto gemm_parts = [&](const Matrix& w, std::uint32_t a_row, std::uint32_t rows,
                              float* y, std::uint32_t ldy, std::uint32_t parts) {
    CheckStatus(lfm3_q8_gemm_h16(w.halves.p, w.scales.p, w.rows, w.cols,
                                 a16 + std::size_t(a_row) * lda, lda, scale + a_row, rows, y,
                                 ldy, parts, s));
  };
  const auto gemm = [&](const Matrix& w, std::uint32_t a_row, std::uint32_t rows, float* y,
                        std::uint32_t ldy) -> std::uint32_t {
    const std::uint32_t parts = lfm3_q8_gemm_parts(w.rows, w.cols, rows, 0);
    gemm_parts(w, a_row, rows, y, ldy, parts);
    return parts;
  };
  // A mixer's input projection over the last `rows` rows (FP32 rows of z
  // below kPromptRows, else the FP16 rows the residual norm left in a16).
  // With `single` one FP32 output (the convolution reads each value up to
  // width times); otherwise K parts that the heads kernel adds. Returns
  // the part count.
  const auto project = [&](const Matrix& w, std::uint32_t rows, float* y, std::uint32_t ldy,
                           bool single) -> std::uint32_t {
    const std::uint32_t first = n - rows;
    if (rows < mfma_rows) {
      gemv(w, z + std::size_t(first) * H, H, y, ldy, rows, false);
      return 1;
    }
    if (!single)
      return gemm(w, first, rows, y, ldy);
    gemm_parts(w, first, rows, y, ldy, 1);
    return 1;
  };
  // Hidden-wide outputs of FP32 rows `in` go to `out` as K parts that the
  // next residual norm adds in part order; returns the part count.
  const auto dense = [&](const Matrix& w, const float* in, std::uint32_t ldx,
                         std::uint32_t rows, const unsigned* rmax) -> std::uint32_t {
    if (rows < mfma_rows) {
      gemv(w, in, ldx, out, H, rows, false);
      return 1;
    }
    halves(in, ldx, rmax, rows, w.cols);
    return gemm(w, 0, rows, out, H);
  };
  // x += post(branch) over the last `rows` rows, then the next norm: FP16
  // rows into a16 when its consumer runs on the matrix cores (consumer
  // rows >= kPromptRows), else FP32 rows into z.
  const auto residual_norm = [&](std::uint32_t parts, const Buffer* post, const Buffer* next,
                                 std::uint32_t rows, std::uint32_t consumer_rows) {
    const std::size_t o = n - rows;
    const float* branch = parts ? out : nullptr;
    const float* pn = post && post->p ? post->as<float>() : nullptr;
    if (next && consumer_rows >= mfma_rows)
      CheckStatus(lfm3_residual_norm_half(branch, parts ? parts : 1, std::size_t(rows) * H, pn,
                                          x + o * H, next->as<float>(), nullptr, a16 + o * lda,
                                          lda, scale + o, rows, H, c.eps, s));
    else
      CheckStatus(lfm3_residual_norm_parts(branch, parts ? parts : 1, std::size_t(rows) * H, pn,
                                           x + o * H, next ? next->as<float>() : nullptr,
                                           z + o * H, rows, H, c.eps, s));
  };

  // x <- the chunk's input rows: token runs embedded from one upload of
  // their ids, row runs copied into place (engine.cpp:1066-1092). The ids
  // stay alive until the stream synchronizes at the end.
  std::vector<std::uint32_t> ids;
  for (const ChunkPart& part : input)
    if (part.tokens)
      ids.insert(ids.end(), part.tokens, part.tokens + part.count);
  if (!ids.empty())
    Check(hipMemcpyAsync(b.tokens.p, ids.data(), ids.size() * 4, hipMemcpyHostToDevice, s),
          "token upload");
  {
    std::size_t row = 0, id = 0;
    for (const ChunkPart& part : input) {
      if (part.tokens && m.exact) {
        CheckStatus(lfm3_float_embed(m.wtype, m.embedding.codes.p, c.vocab, H,
                                     b.tokens.as<std::uint32_t>() + id, nullptr, part.count,
                                     x + row * H, s));
        id += part.count;
      } else if (part.tokens) {
        CheckStatus(lfm3_embed(m.embedding.codes.p, m.embedding.scales.p, c.vocab, H,
                               b.tokens.as<std::uint32_t>() + id, part.count, x + row * H, s));
        id += part.count;
      } else {
        Check(hipMemcpyAsync(x + row * H, part.rows, std::size_t(part.count) * H * 4,
                             part.on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s),
              "input rows");
      }
      row += part.count;
    }
  }
  residual_norm(0, nullptr, &m.layers[0].norm, live_in[0], live_in[0]);
  for (std::uint32_t il = 0; il < L; ++il) {
    const Layer& l = m.layers[il];
    auto& state = se.states[il];
    const std::uint32_t rows_in = live_in[il], rows_out = live_out[il];
    const std::uint32_t o_in = n - rows_in, o = n - rows_out;
    std::uint32_t parts;
    if (l.type == LFM3_LAYER_CONV) {
      project(l.in_proj, rows_in, proj, 3 * H, true);
      // Rows before the first live one are not read: outputs that would
      // need them are not live either (engine.cpp:386-393).
      float* hist = state.conv.as<float>();
      if (rows_out >= mfma_rows && c.conv_width <= 7 && H % 4 == 0 && H <= 2048) {
        // The output projection's FP16 rows straight from the convolution.
        CheckStatus(lfm3_conv_prompt_half(proj, 3 * H, l.conv.as<float>(), hist, rows_in,
                                          o - o_in, a16, lda, scale, H, c.conv_width, 1, s));
        parts = gemm(l.out_proj, 0, rows_out, out, H);
      } else {
        const std::uint32_t begin = 0;
        CheckStatus(lfm3_conv_prompt(proj, 3 * H, l.conv.as<float>(), &hist, &begin, &rows_in,
                                     1, mix, H, H, c.conv_width, 1, s));
        parts = dense(l.out_proj, mix + std::size_t(o - o_in) * H, H, rows_out, nullptr);
      }
    } else {
      const bool swa = l.type == LFM3_LAYER_SLIDING;
      const std::uint32_t stride = l.kv * D;
      const std::uint32_t qparts = project(l.qkvg, n, proj, pld, false);
      const float* table = swa ? m.freq_sliding.as<float>() : m.freq_global.as<float>();
      const float* factors = swa ? nullptr : m.factors.as<float>();
      auto* ck = state.k.as<std::uint16_t>();
      auto* cv = state.v.as<std::uint16_t>();
      // Full-attention rows never wrap, so the chunk is packed in place; a
      // sliding ring is written only after attention read its history.
      std::uint16_t* kc = swa ? b.chunk_k.as<std::uint16_t>() : ck + std::size_t(position) * stride;
      std::uint16_t* vc = swa ? b.chunk_v.as<std::uint16_t>() : cv + std::size_t(position) * stride;
      LaunchPromptHeads(proj + l.q_off, proj + l.k_off, proj + l.v_off, pld,
                        l.q_norm.as<float>(), l.k_norm.as<float>(), table, factors, kc, vc, n,
                        c.heads, l.kv, D, position, c.eps, qparts, std::size_t(pld) * n,
                        proj + l.g_off, s);
      Check(hipGetLastError(), "LFM3 prompt heads launch");
      // Only the last rows_out queries are live.
      const std::uint32_t skip = n - rows_out;
      float* q_rows = proj + std::size_t(skip) * pld + l.q_off;
      float* g_rows = proj + std::size_t(skip) * pld + l.g_off;
      float* a_rows = mix + std::size_t(skip) * c.heads * D;
      if (rows_out == 1 && !swa) {
        // One live row reads the cache through the FP32 decode attention
        // (hip/ops.hip:2295-2315), as the reference's n == 1 call does.
        auto* host = static_cast<std::uint8_t*>(b.one_staging->p);
        auto** ptrs = reinterpret_cast<void**>(host);
        auto* nums = reinterpret_cast<std::uint32_t*>(host + 2 * sizeof(void*));
        ptrs[0] = ck;
        ptrs[1] = cv;
        nums[0] = state.capacity;
        nums[1] = position + skip;
        auto* items = reinterpret_cast<lfm3_attention_item*>(host + Align(4 * sizeof(void*)));
        const int count = lfm3_attention_plan(&nums[1], 1, 0, items,
                                              std::uint32_t(b.one_items));
        if (count < 0)
          throw Error(LFM3_E_INVALID, lfm3_last_error());
        auto* dev = b.one_table.as<std::uint8_t>();
        Check(hipMemcpyAsync(dev, host, b.one_bytes, hipMemcpyHostToDevice, s), "table upload");
        const std::size_t ws = lfm3_attention_workspace_bytes(std::uint32_t(count), 1, c.heads,
                                                              l.kv, D);
        if (ws > b.one_ws_bytes)
          throw Error(LFM3_E_INVALID, "LFM3 attention workspace too small");
        CheckStatus(lfm3_decode_attention_ragged(
            q_rows, pld, g_rows, pld, reinterpret_cast<const std::uint16_t* const*>(dev),
            reinterpret_cast<const std::uint16_t* const*>(dev + sizeof(void*)),
            reinterpret_cast<const std::uint32_t*>(dev + 2 * sizeof(void*)),
            reinterpret_cast<const lfm3_attention_item*>(dev + Align(4 * sizeof(void*))),
            std::uint32_t(count), a_rows, c.heads * D, 1, c.heads, l.kv, D, b.one_ws.p,
            b.one_ws_bytes, s));
        // The staging buffer is reused by the next layer's row.
        Check(hipStreamSynchronize(s), "decode attention row");
      } else if (rows_out >= mfma_rows) {
        // The output projection's FP16 rows straight from the attention.
        CheckStatus(lfm3_prompt_attention_half(
            q_rows, pld, kc + std::size_t(skip) * stride, vc + std::size_t(skip) * stride,
            g_rows, pld, ck, cv, a16, lda, scale, n - skip, c.heads, l.kv, D, position + skip,
            state.capacity, swa ? c.window : 0, b.attn_ws.p, b.attn_ws_bytes, s));
      } else {
        CheckStatus(lfm3_prompt_attention(
            q_rows, pld, kc + std::size_t(skip) * stride, vc + std::size_t(skip) * stride,
            g_rows, pld, ck, cv, a_rows, c.heads * D, n - skip, c.heads, l.kv, D,
            position + skip, state.capacity, swa ? c.window : 0, b.attn_ws.p,
            b.attn_ws_bytes, s));
      }
      if (swa)
        CheckStatus(lfm3_store_kv(kc, vc, ck, cv, n, stride, position, state.capacity, s));
      if (rows_out >= mfma_rows)
        parts = gemm(l.attn_out, 0, rows_out, out, H);
      else
        parts = dense(l.attn_out, mix + std::size_t(o) * c.heads * D, c.heads * D, rows_out,
                      nullptr);
    }
    residual_norm(parts, &l.post_norm, &l.ffn_norm, rows_out, rows_out);
    // FFN over the live rows: SwiGLU (with each row's max |y| per block of
    // output rows for the down projection's FP16 conversion), then down.
    if (rows_out < mfma_rows) {
      gemv(l.ffn, z + std::size_t(o) * H, H, hid, F, rows_out, true);
      parts = dense(l.down, hid, F, rows_out, nullptr);
    } else {
      // The hidden rows' FP16 conversion runs in the SwiGLU launch's
      // trailing blocks, into their own buffer (the launch still reads
      // a16).
      if (++b.swiglu_seq == 0)
        b.swiglu_seq = 1;
      const std::uint32_t hld = (F + 63) / 64 * 64;
      auto* h16 = b.hid16.as<std::uint16_t>();
      float* hscale = b.hid_scale.as<float>();
      CheckStatus(lfm3_q8_gemm_swiglu_h16_rows(
          l.ffn.halves.p, l.ffn.scales.p, F, H, a16 + std::size_t(o) * lda, lda, scale + o,
          rows_out, hid, F, row_max, h16, hld, hscale, b.swiglu_flags.as<unsigned>(),
          b.swiglu_seq, static_cast<unsigned*>(b.wait_error->device), s));
      const Matrix& w = l.down;
      const std::uint32_t dparts = lfm3_q8_gemm_parts(w.rows, w.cols, rows_out, 0);
      CheckStatus(lfm3_q8_gemm_h16(w.halves.p, w.scales.p, w.rows, w.cols, h16, hld, hscale,
                                   rows_out, out, H, dparts, s));
      parts = dparts;
    }
    const bool last = il + 1 == L;
    residual_norm(parts, &l.post_ffn_norm, last ? nullptr : &m.layers[il + 1].norm, rows_out,
                  last ? 0 : live_in[il + 1]);
  }
  // The frontier row: the last row normed by output_norm; logits from it.
  CheckStatus(lfm3_residual_norm(nullptr, nullptr, x + std::size_t(n - 1) * H,
                                 m.output_norm.as<float>(), se.frontier.as<float>(), 1, H,
                                 c.eps, s));
  if (want_logits)
    HeadRow(m, se.frontier.as<float>(), se.logits.as<float>(), s);
  Check(hipGetLastError(), "prompt launch");
  Check(hipStreamSynchronize(s), "prompt");
  auto* word = static_cast<volatile unsigned*>(b.wait_error->p);
  if (*word) {
    *word = 0;
    throw Error(LFM3_E_HIP, "LFM3 prompt: a SwiGLU conversion block's wait timed out");
  }
  se.position += n;
  se.logits_ready = want_logits;
}

// Session::Forward / ForwardEmbeddings / ForwardInputs (engine.cpp:882-1100):
// n input rows from `runs`, in chunks of kPrefillChunk rows that runs share
// (one pass reads the weights once whatever mixes in it); a chunk of one row
// is a decode row. The vocabulary head runs for the last chunk only when
// logits are wanted.
void ForwardRuns(lfm3_session& se, const std::vector<ChunkPart>& runs, std::size_t n,
                 bool want_logits, hipStream_t prompt_stream = nullptr) {
  lfm3_model& m = *se.model;
  if (!prompt_stream)
    prompt_stream = m.stream;
  const std::size_t H = m.config.hidden;
  std::size_t run = 0, at = 0;  // next input row: runs[run], row at
  for (std::size_t done = 0; done < n;) {
    const auto count = std::uint32_t(std::min<std::size_t>(kPrefillChunk, n - done));
    std::vector<ChunkPart> parts;
    for (std::uint32_t row = 0; row < count;) {
      const ChunkPart& r = runs[run];
      const auto take = std::uint32_t(std::min<std::size_t>(r.count - at, count - row));
      if (take) {
        ChunkPart p = r;
        p.count = take;
        if (r.tokens)
          p.tokens = r.tokens + at;
        else
          p.rows = r.rows + at * H;
        parts.push_back(p);
      }
      row += take;
      at += take;
      if (at == r.count) {
        ++run;
        at = 0;
      }
    }
    const bool head = want_logits && done + count == n;
    if (count == 1) {
      // One row is one decode row (engine.cpp:412-436).
      lfm3_session* one = &se;
      const ChunkPart& p = parts.front();
      if (p.tokens) {
        RunRound(m, &one, 1, p.tokens, false, nullptr, head);
      } else {
        const float* row = p.rows;
        if (!p.on_device) {
          Check(hipMemcpyAsync(m.one_row.p, p.rows, H * 4, hipMemcpyHostToDevice, m.stream),
                "input row");
          row = m.one_row.as<float>();
        }
        const std::uint32_t unused = 0;
        RunRound(m, &one, 1, &unused, false, &row, head);
      }
    } else {
      RunPrompt(m, se, parts, count, head, prompt_stream);
    }
    done += count;
  }
}

// Checks shared by the forward entries (engine.cpp:904-914), then the
// continuation hook for the rows about to be written.
void CheckForward(lfm3_session* se, std::size_t n) {
  if (!se)
    Invalid("null LFM3 session");
  if (se->poisoned)
    throw Error(LFM3_E_STATE, "LFM3 session requires Reset after a device error");
  if (n == 0 || n > se->context - se->position)
    Invalid("invalid LFM3 input/logit count or context exhausted");
}
void BeforeWrite(lfm3_session& se, std::size_t n) {
  if (se.hooks.before_write)
    Hook(se.hooks.before_write(se.hooks.user, se.position, se.position + std::uint32_t(n)),
         "the write");
}

// Runs a validated forward; a device failure poisons the session
// (engine.cpp:924-926).
int ForwardEntry(lfm3_session* se, const std::vector<ChunkPart>& runs, std::size_t n,
                 float* logits) {
  lfm3_model& m = *se->model;
  std::lock_guard<std::mutex> guard(m.lock);
  try {
    ForwardRuns(*se, runs, n, logits != nullptr);
    if (logits)
      CopyLogits(m, logits, se->logits.p);
    return LFM3_OK;
  } catch (const Error& e) {
    se->poisoned = true;
    return Fail(e.status, e.what());
  } catch (const std::exception& e) {
    se->poisoned = true;
    return Fail(LFM3_E_HIP, e.what());
  }
}

// engine.cpp:1178-1195; for ForwardBatchInputs (engine.cpp:1244-1259) a
// token is checked only where no input row stands in for it.
void ValidateBatch(lfm3_session* const* sessions, std::size_t n,
                   const std::uint32_t* tokens, const float* const* inputs = nullptr) {
  if (!sessions || !tokens || n == 0 || n > kMaxBatch)
    Invalid("invalid LFM3 decode batch shape");
  for (std::size_t i = 0; i < n; ++i) {
    lfm3_session* se = sessions[i];
    if (!se || std::find(sessions, sessions + i, se) != sessions + i)
      Invalid("duplicate or null LFM3 batch session");
    const bool row = inputs && inputs[i];
    if (se->poisoned || se->position >= se->context ||
        (!row && tokens[i] >= se->model->config.vocab) || se->model != sessions[0]->model)
      Invalid("incompatible LFM3 batch session");
  }
}

// The sampler's inputs for a round (host arrays): row i's penalty list at
// penalty_ids + i * n_penalty and its uniform at uniforms[i].
struct SampleArgs {
  const lfm3_sampling* params = nullptr;
  const std::uint32_t* penalty_ids = nullptr;
  std::uint32_t n_penalty = 0;
  const float* uniforms = nullptr;
};

// Uploads the sampler's inputs on the model stream and picks each row's id
// from its session's logits row into the pinned ids (m.ids()).
void EnqueueSample(lfm3_model& m, std::uint32_t n, const SampleArgs& a) {
  const std::size_t uni_bytes = Align(kMaxBatch * 4);
  auto* host = static_cast<std::uint8_t*>(m.sample_staging->p);
  if (a.uniforms)
    std::memcpy(host, a.uniforms, n * 4);
  if (a.n_penalty)
    std::memcpy(host + uni_bytes, a.penalty_ids, std::size_t(n) * a.n_penalty * 4);
  const std::size_t used = uni_bytes + std::size_t(n) * a.n_penalty * 4;
  auto* dev = m.sample_table.as<std::uint8_t>();
  Check(hipMemcpyAsync(dev, host, used, hipMemcpyHostToDevice, m.stream), "sampler upload");
  const std::size_t ws = SampleWorkspaceBytes(kMaxBatch, m.config.vocab, a.params->top_k);
  if (ws > m.sample_ws_bytes) {
    Check(hipStreamSynchronize(m.stream), "sampler workspace");
    m.sample_ws = Buffer(ws);
    m.sample_ws_bytes = ws;
  }
  const auto* rows = reinterpret_cast<const float* const*>(m.table.as<std::uint8_t>() +
                                                           offsetof(RoundTable, logits));
  CheckStatus(LaunchSample(nullptr, 0, rows, n, m.config.vocab, *a.params,
                           a.n_penalty ? reinterpret_cast<const std::uint32_t*>(dev + uni_bytes)
                                       : nullptr,
                           a.n_penalty, a.uniforms ? reinterpret_cast<const float*>(dev) : nullptr,
                           m.ids(), m.sample_ws.p, m.sample_ws_bytes,
                           m.stream));
}

int BatchEntry(lfm3_session* const* sessions, std::size_t n,
               const std::uint32_t* tokens, float* const* logits,
               std::uint32_t* ids, const float* const* inputs = nullptr, bool head = true,
               const SampleArgs* sample = nullptr) {
  try {
    ValidateBatch(sessions, n, tokens, inputs);
    if (logits)
      for (std::size_t i = 0; i < n; ++i)
        if (!logits[i])
          Invalid("invalid LFM3 decode batch shape");
    if (sample) {
      if (!sample->params ||
          CheckSample(*sample->params, sessions[0]->model->config.vocab, sample->n_penalty,
                      sample->penalty_ids != nullptr, sample->uniforms != nullptr))
        Invalid("unsupported LFM3 sampling parameters");
    }
    // engine.cpp:1196-1199: every session's hook before any work.
    for (std::size_t i = 0; i < n; ++i)
      BeforeWrite(*sessions[i], 1);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  lfm3_model& m = *sessions[0]->model;
  std::lock_guard<std::mutex> guard(m.lock);
  try {
    // The round, the pick, and the copies of its ids and logits rows; one
    // synchronization for all of them (engine.cpp:1201-1204 syncs, then
    // copies each logits row synchronously).
    EnqueueRound(m, sessions, std::uint32_t(n), tokens, ids != nullptr && !sample, inputs, head);
    if (sample)
      EnqueueSample(m, std::uint32_t(n), *sample);
    EnqueueReadback(m, sessions, std::uint32_t(n), logits != nullptr);
    Check(hipStreamSynchronize(m.stream), "round");
    CheckRoundWaits(m);
    FinishRound(sessions, std::uint32_t(n), head);
    DeliverReadback(m, std::uint32_t(n), ids, logits);
    return LFM3_OK;
  } catch (const Error& e) {
    for (std::size_t i = 0; i < n; ++i)
      sessions[i]->poisoned = true;  // engine.cpp:1205-1208
    return Fail(e.status, e.what());
  } catch (const std::exception& e) {
    for (std::size_t i = 0; i < n; ++i)
      sessions[i]->poisoned = true;
    return Fail(LFM3_E_HIP, e.what());
  }
}

}  // namespace
}  // namespace lfm3amd

extern "C" {

int lfm3_session_forward(lfm3_session* se, const std::uint32_t* tokens, std::size_t n,
                         float* logits) {
  try {
    CheckForward(se, n);
    if (!tokens)
      Invalid("invalid LFM3 token/logit count or context exhausted");
    for (std::size_t i = 0; i < n; ++i)
      if (tokens[i] >= se->model->config.vocab)
        Invalid("LFM3 token out of range");
    BeforeWrite(*se, n);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  ChunkPart run;
  run.count = std::uint32_t(n);
  run.tokens = tokens;
  return ForwardEntry(se, {run}, n, logits);
}

int lfm3_session_forward_rows(lfm3_session* se, const float* rows, std::size_t n_rows,
                              int on_device, float* logits) {
  try {
    CheckForward(se, n_rows);
    if (!rows)
      Invalid("invalid LFM3 embedding/logit count or context exhausted");
    BeforeWrite(*se, n_rows);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  ChunkPart run;
  run.count = std::uint32_t(n_rows);
  run.rows = rows;
  run.on_device = on_device != 0;
  return ForwardEntry(se, {run}, n_rows, logits);
}

int lfm3_session_forward_inputs(lfm3_session* se, const lfm3_input* inputs, std::size_t n_inputs,
                                float* logits) {
  std::vector<ChunkPart> runs;
  std::size_t n = 0;
  try {
    if (!se || (!inputs && n_inputs))
      Invalid("invalid LFM3 inputs");
    const std::uint32_t vocab = se->model->config.vocab;
    for (std::size_t i = 0; i < n_inputs; ++i) {
      const lfm3_input& in = inputs[i];
      if (in.n_tokens && in.n_rows)
        Invalid("an LFM3 input run is tokens or rows");
      if ((in.n_tokens && !in.tokens) || (in.n_rows && !in.rows))
        Invalid("invalid LFM3 inputs");
      for (std::size_t t = 0; t < in.n_tokens; ++t)
        if (in.tokens[t] >= vocab)
          Invalid("LFM3 token out of range");
      ChunkPart run;
      run.count = std::uint32_t(in.n_tokens + in.n_rows);
      run.tokens = in.n_tokens ? in.tokens : nullptr;
      run.rows = in.n_rows ? in.rows : nullptr;
      if (run.count)
        runs.push_back(run);
      n += in.n_tokens + in.n_rows;
    }
    CheckForward(se, n);
    BeforeWrite(*se, n);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  return ForwardEntry(se, runs, n, logits);
}

// ContinuationLayout (continuation_layout.cpp:6-46): the state inventory
// in the reference's order; ids count from 1.
int lfm3_continuation_layout(const lfm3_config* config, std::uint32_t context,
                             lfm3_continuation_component* out, std::size_t capacity,
                             std::size_t* count) {
  if (!config || !count || (capacity && !out) || !context || context > config->context ||
      !config->n_layers || !config->hidden || !config->vocab || !config->head_dim ||
      !config->conv_width || !config->kv_heads || !config->layer_type)
    return Fail(LFM3_E_INVALID, "invalid LFM3 continuation geometry");
  const lfm3_config& c = *config;
  std::size_t n = 0;
  const auto add = [&](std::uint32_t part, std::size_t row, std::size_t state,
                       std::uint32_t layer) {
    if (n < capacity) {
      lfm3_continuation_component& x = out[n];
      x.id = std::uint32_t(n + 1);
      x.part = part;
      x.layer = layer;
      x.reserved = 0;
      x.row_bytes = row;
      x.state_bytes = state;
    }
    ++n;
  };
  add(LFM3_PART_LOGITS, 0, std::size_t(c.vocab) * 4, 0);
  add(LFM3_PART_FRONTIER, 0, std::size_t(c.hidden) * 4, 0);
  add(LFM3_PART_METADATA, 0, LFM3_CONTINUATION_METADATA_BYTES, 0);
  for (std::uint32_t l = 0; l < c.n_layers; ++l) {
    const std::size_t row = std::size_t(c.kv_heads[l]) * c.head_dim * sizeof(Half);
    switch (c.layer_type[l]) {
      case LFM3_LAYER_CONV:
        add(LFM3_PART_CONVOLUTION, 0, std::size_t(c.hidden) * (c.conv_width - 1) * 4, l);
        break;
      case LFM3_LAYER_SLIDING:
        add(LFM3_PART_SLIDING_WINDOW, 0, 2 * row * std::min(context, c.window), l);
        break;
      default:
        add(LFM3_PART_KEY, row, 0, l);
        add(LFM3_PART_VALUE, row, 0, l);
        break;
    }
  }
  *count = n;
  return LFM3_OK;
}

// PrivateBytes and RowBytes(position) (continuation_layout.cpp:56-69).
int lfm3_continuation_bytes(const lfm3_config* config, std::uint32_t context,
                            std::uint32_t position, std::size_t* private_bytes,
                            std::size_t* row_bytes) {
  std::size_t n = 0;
  int e = lfm3_continuation_layout(config, context, nullptr, 0, &n);
  if (e)
    return e;
  if (position > context)
    return Fail(LFM3_E_INVALID, "invalid LFM3 continuation frontier");
  std::vector<lfm3_continuation_component> parts(n);
  e = lfm3_continuation_layout(config, context, parts.data(), n, &n);
  if (e)
    return e;
  std::size_t priv = 0, rows = 0;
  for (const auto& x : parts) {
    priv += x.state_bytes;
    rows += x.row_bytes * position;
  }
  if (private_bytes)
    *private_bytes = priv;
  if (row_bytes)
    *row_bytes = rows;
  return LFM3_OK;
}

// One scheduler round (README.md:106-109; runner.cpp drives the decode
// batch and a prompt chunk each round): the decode rows of `sessions` on
// the model stream and the prompt pass on the model's prompt stream, both
// enqueued before either is waited on, so the bandwidth-bound decode GEMVs
// run beside the matrix-core prompt GEMMs. The decode round's greedy ids
// (ids) and logits (logits) and the prompt's last logits are as from
// lfm3_forward_batch_greedy / lfm3_forward_batch and lfm3_session_forward.
int lfm3_scheduler_round(lfm3_session* const* sessions, std::size_t n,
                         const std::uint32_t* tokens, std::uint32_t* ids, float* const* logits,
                         lfm3_session* prompt, const std::uint32_t* prompt_tokens,
                         std::size_t n_prompt, float* prompt_logits) {
  lfm3_model* model = nullptr;
  try {
    if (!n && !n_prompt)
      Invalid("empty LFM3 scheduler round");
    if (n) {
      ValidateBatch(sessions, n, tokens);
      if (logits)
        for (std::size_t i = 0; i < n; ++i)
          if (!logits[i])
            Invalid("invalid LFM3 decode batch shape");
      model = sessions[0]->model;
    }
    if (n_prompt) {
      CheckForward(prompt, n_prompt);
      if (!prompt_tokens)
        Invalid("invalid LFM3 token/logit count or context exhausted");
      if (model && prompt->model != model)
        Invalid("LFM3 prompt session of another model");
      if (n && std::find(sessions, sessions + n, prompt) != sessions + n)
        Invalid("an LFM3 session cannot decode and prefill in one round");
      for (std::size_t i = 0; i < n_prompt; ++i)
        if (prompt_tokens[i] >= prompt->model->config.vocab)
          Invalid("LFM3 token out of range");
      model = prompt->model;
    }
    for (std::size_t i = 0; i < n; ++i)
      BeforeWrite(*sessions[i], 1);
    if (n_prompt)
      BeforeWrite(*prompt, n_prompt);
  } catch (const Error& e) {
    return Fail(e.status, e.what());
  }
  lfm3_model& m = *model;
  std::lock_guard<std::mutex> guard(m.lock);
  const auto poison_batch = [&] {
    for (std::size_t i = 0; i < n; ++i)
      sessions[i]->poisoned = true;
  };
  int status = LFM3_OK;
  std::string message;
  bool enqueued = false;
  try {
    if (n_prompt)
      EnsurePromptBuffers(m);
    // A prompt whose last chunk is one row runs that row as a decode round
    // on the model stream: then the two run one after the other.
    const bool overlap = n && n_prompt && n_prompt % kPrefillChunk != 1;
    if (n) {
      EnqueueRound(m, sessions, std::uint32_t(n), tokens, ids != nullptr, nullptr, true);
      EnqueueReadback(m, sessions, std::uint32_t(n), logits != nullptr);
      enqueued = true;
      if (!overlap) {
        Check(hipStreamSynchronize(m.stream), "round");
        CheckRoundWaits(m);
        FinishRound(sessions, std::uint32_t(n), true);
        enqueued = false;
      }
    }
    if (n_prompt) {
      ChunkPart run;
      run.count = std::uint32_t(n_prompt);
      run.tokens = prompt_tokens;
      try {
        ForwardRuns(*prompt, {run}, n_prompt, prompt_logits != nullptr, m.prompt_stream);
      } catch (const std::exception& e) {
        prompt->poisoned = true;  // engine.cpp:924-926
        (void)hipStreamSynchronize(m.prompt_stream);
        const auto* err = dynamic_cast<const Error*>(&e);
        status = err ? err->status : LFM3_E_HIP;
        message = e.what();
      }
    }
    if (enqueued) {
      Check(hipStreamSynchronize(m.stream), "round");
      CheckRoundWaits(m);
      FinishRound(sessions, std::uint32_t(n), true);
      enqueued = false;
    }
    if (n)
      DeliverReadback(m, std::uint32_t(n), ids, logits);
    if (status == LFM3_OK && n_prompt && prompt_logits)
      CopyLogits(m, prompt_logits, prompt->logits.p);
  } catch (const std::exception& e) {
    if (enqueued)
      (void)hipStreamSynchronize(m.stream);
    poison_batch();  // engine.cpp:1205-1208
    const auto* err = dynamic_cast<const Error*>(&e);
    return Fail(err ? err->status : LFM3_E_HIP, e.what());
  }
  return status == LFM3_OK ? LFM3_OK : Fail(status, message);
}

int lfm3_session_set_hooks(lfm3_session* se, const lfm3_hooks* hooks) {
  if (!se)
    return Fail(LFM3_E_INVALID, "null session");
  se->hooks = hooks ? *hooks : lfm3_hooks{};
  return LFM3_OK;
}

int lfm3_session_read_hidden(const lfm3_session* se, float* hidden) {
  if (!se || !hidden)
    return Fail(LFM3_E_INVALID, "null hidden row");
  if (se->poisoned || !se->position)
    return Fail(LFM3_E_INVALID, "invalid LFM3 hidden frontier");
  std::lock_guard<std::mutex> guard(se->model->lock);
  const hipStream_t stream = se->model->stream;
  int e = HipStatus(hipMemcpyAsync(hidden, se->frontier.p, std::size_t(se->model->config.hidden) * 4,
                                   hipMemcpyDeviceToHost, stream),
                    "read hidden");
  if (!e)
    e = HipStatus(hipStreamSynchronize(stream), "read hidden");
  return e;
}

int lfm3_forward_batch(lfm3_session* const* sessions, std::size_t n,
                       const std::uint32_t* tokens, float* const* logits) {
  if (!logits)
    return Fail(LFM3_E_INVALID, "invalid LFM3 decode batch shape");
  return BatchEntry(sessions, n, tokens, logits, nullptr);
}

int lfm3_forward_batch_greedy(lfm3_session* const* sessions, std::size_t n,
                              const std::uint32_t* tokens, std::uint32_t* ids) {
  if (!ids)
    return Fail(LFM3_E_INVALID, "null greedy ids");
  return BatchEntry(sessions, n, tokens, nullptr, ids);
}

int lfm3_forward_batch_sample(lfm3_session* const* sessions, std::size_t n,
                              const std::uint32_t* tokens, const lfm3_sampling* params,
                              const std::uint32_t* penalty_ids, std::uint32_t n_penalty,
                              const float* uniforms, std::uint32_t* ids) {
  if (!ids || !params)
    return Fail(LFM3_E_INVALID, "null sampled ids or sampling parameters");
  SampleArgs a;
  a.params = params;
  a.penalty_ids = penalty_ids;
  a.n_penalty = n_penalty;
  a.uniforms = uniforms;
  return BatchEntry(sessions, n, tokens, nullptr, ids, nullptr, true, &a);
}

int lfm3_forward_batch_inputs(lfm3_session* const* sessions, std::size_t n,
                              const std::uint32_t* tokens, const float* const* rows,
                              int want_logits, float* const* logits) {
  if (!rows || (logits && !want_logits))
    return Fail(LFM3_E_INVALID, "invalid LFM3 decode batch shape");
  return BatchEntry(sessions, n, tokens, logits, nullptr, rows, want_logits != 0);
}

}  // extern "C"
