// The decode round's residual norm with the operand image, as a device
// function: its own launch (NormImageKernel, rows.hip) or the leading
// blocks of the GEMV that consumes the image (q8.hip), which then waits
// for the rows through a flag per row (NormImageRow with kPublish, WatchRows).
#ifndef LFM3_AMD_NORM_IMAGE_HPP_
#define LFM3_AMD_NORM_IMAGE_HPP_
#include "common.hpp"
#include "internal.hpp"

namespace lfm3amd {

// Decode-round residual norm with the operand image (rows <= 8): the same
// expressions as ResidualNormKernel on one block of T threads per row.
// Thread t owns column groups g = t + T i (columns 8g..8g+7) and holds them
// in registers from the loads to the image write, so the block needs no row
// staging; every load (x, norm weights, every K part) is issued before the
// first reduction. Run by NormImageKernel (a launch of its own) and by the
// first blocks of an operand-image GEMV that takes its norm along
// (kPublish: the hand-over below).
constexpr int kNormParts = 8;

// A block barrier for LDS exchanges only: this wave's LDS operations
// complete, then the waves meet. Global stores in flight are not waited
// for (a __syncthreads would drain them first).
__device__ __forceinline__ void LdsBarrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template<int N>
__device__ __forceinline__ float SmallBlockSum(float v, float* slots) {
  v = WaveSum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0)
    slots[wave] = v;
  LdsBarrier();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < N; ++w)
    total += slots[w];
  return total;
}

// The flags a fused launch's norm blocks publish: kFlagCopies copies,
// kFlagStride words apart, one for each XCD's blocks to poll.
constexpr int kFlagCopies = 8, kFlagStride = 1024;
constexpr std::size_t kFlagWords = std::size_t(kFlagCopies) * kFlagStride;

// With kPublish (the norm blocks of a fused launch), the image row and its
// exponent go out first with sc1 stores (through the XCD's L2 to memory,
// where the GEMV blocks of every XCD read them); once every wave's stores
// are acknowledged, one thread per copy stores `seq` into the row's flag;
// the FP32 rows (x, z) are stored last, so the hand-over waits for none of
// them.
template<int T, int G, bool kPublish>
__device__ __forceinline__ void NormImageRow(const NormImageArgs& a, int row,
                                             unsigned* flags = nullptr, unsigned seq = 0) {
  constexpr int kWaves = T / 64;
  // Image words of a fused launch go through the L2 to memory (sc1), where
  // the consumer blocks of other XCDs read them.
  constexpr int kImagePolicy = kPublish ? kCachePolicySc1 : 0;
  __shared__ float s_red[3][kWaves];
  const int tid = threadIdx.x, H = a.H;
  const unsigned row_bytes = unsigned(H) * 4;
  float* x = a.x;
  const BufferResource x_res = MakeBuffer(x + std::size_t(row) * H, a.tokens ? 0u : row_bytes);
  const BufferResource w_res = MakeBuffer(a.weight, row_bytes);
  const BufferResource p_res = MakeBuffer(a.post ? a.post : a.weight, a.post ? row_bytes : 0u);
  float v[G][8], pw[G][8], nw[G][8], b[kNormParts][G][8];
  const auto load8 = [](BufferResource r, unsigned off, float* out) {
    const float4 lo = LoadF4(r, off), hi = LoadF4(r, off + 16);
    out[0] = lo.x; out[1] = lo.y; out[2] = lo.z; out[3] = lo.w;
    out[4] = hi.x; out[5] = hi.y; out[6] = hi.z; out[7] = hi.w;
  };
  // Every load is issued before the first store: loads and stores share
  // one counter, so a load after stores would wait for all of them.
  float* const zrow = a.z_rows ? a.z_rows[row] : a.z ? a.z + std::size_t(row) * H : nullptr;
  // The round's first norm gathers its rows from the tiled embedding table
  // (EmbedKernel's layout: columns 8G..8G+7 of row r are 8 consecutive code
  // bytes of one lane word) and writes them to x.
  std::uint32_t token = 0;
  const float* input = nullptr;  // an FP32 input row in place of the token
  if (a.tokens) {
    token = a.tokens[row];
    if (token >= std::uint32_t(a.vocab))
      token = 0;  // the host validates ids; never read out of bounds
    if (a.inputs)
      input = a.inputs[row];
  }
  const BufferResource in_res = MakeBuffer(input, input ? row_bytes : 0u);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + T * i;
    const unsigned off = g * 8 < H ? unsigned(g) * 32 : kOutOfRange;
    if (input) {
      load8(in_res, off, v[i]);
    } else if (a.tokens) {
      const int chunk = g / 8, blk = (g % 8) / 4, lg = g % 4;
      const std::size_t tile = std::size_t(token / kTileRows) * ((H + kChunk - 1) / kChunk) + chunk;
      const int nn = int(token % kTileRows);
      unsigned lo = 0, hi = 0;
      float d = 0.0f;
      if (g * 8 < H) {
        const uint2 q = *reinterpret_cast<const uint2*>(
            a.emb_codes + tile * kTileCodeBytes + (lg * 16 + nn) * 16 + blk * 8);
        lo = q.x;
        hi = q.y;
        d = HalfBitsToFloat(a.emb_scales[tile * kTileScales + nn * 2 + blk]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        v[i][k] = d * float(int((lo >> (8 * k)) & 0xffu) - 128);
        v[i][4 + k] = d * float(int((hi >> (8 * k)) & 0xffu) - 128);
      }
    } else {
      load8(x_res, off, v[i]);
    }
    load8(w_res, off, nw[i]);
    load8(p_res, off, pw[i]);
  }
  if (a.branch) {
#pragma unroll
    for (int p = 0; p < kNormParts; ++p) {
      if (p < a.parts) {  // uniform: only the parts that exist are read
        const BufferResource b_res =
            MakeBuffer(a.branch + p * a.part_stride + std::size_t(row) * H, row_bytes);
#pragma unroll
        for (int i = 0; i < G; ++i) {
          const int g = tid + T * i;
          load8(b_res, g * 8 < H ? unsigned(g) * 32 : kOutOfRange, b[p][i]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
          for (int k = 0; k < 8; ++k)
            b[p][i][k] = 0.0f;
      }
    }
  }
  // Every load has landed before the first store, on every path: stores
  // and loads share one counter, and a wait the compiler places after a
  // store (for a load still in flight on another path) drains the stores.
  __builtin_amdgcn_s_waitcnt(WaitVm(0));
  // Stores go through buffer resources at offsets that are dropped past
  // the row, without branches: the compiler's waits after a branch around
  // a store drain every store in flight.
  const BufferResource x_out = MakeBuffer(x + std::size_t(row) * H, row_bytes);
  const auto store8 = [](BufferResource r, unsigned off, const float* in) {
    StoreF4(r, off, in[0], in[1], in[2], in[3]);
    StoreF4(r, off + 16, in[4], in[5], in[6], in[7]);
  };
  if (a.branch) {
    float squares = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
#pragma unroll
        for (int p = 1; p < kNormParts; ++p)
          b[0][i][k] += b[p][i][k];
        squares = fmaf(b[0][i][k], b[0][i][k], squares);
      }
    if (a.post) {
      const float scale =
          1.0f / sqrtf(SmallBlockSum<kWaves>(squares, s_red[0]) / float(H) + a.eps);
#pragma unroll
      for (int i = 0; i < G; ++i)
#pragma unroll
        for (int k = 0; k < 8; ++k)
          b[0][i][k] = (b[0][i][k] * scale) * pw[i][k];
    }
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[i][k] = v[i][k] + b[0][i][k];
  }
  // The residual row (the gathered embedding row, or x + post(branch)),
  // stored at the end.
  float xv[G][8];
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k)
      xv[i][k] = v[i][k];
  const bool store_x = a.tokens || a.branch;
  float squares = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i)
#pragma unroll
    for (int k = 0; k < 8; ++k)
      squares = fmaf(v[i][k], v[i][k], squares);
  const float scale =
      1.0f / sqrtf(SmallBlockSum<kWaves>(squares, s_red[1]) / float(H) + a.eps);
  float maximum = 0.0f;
  const BufferResource z_out = MakeBuffer(zrow, zrow ? row_bytes : 0u);
#pragma unroll
  for (int i = 0; i < G; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      v[i][k] = (v[i][k] * scale) * nw[i][k];  // zero past H
      maximum = fmaxf(maximum, fabsf(v[i][k]));
    }
  }
  maximum = WaveMax(maximum);
  if ((tid & 63) == 0)
    s_red[2][tid >> 6] = maximum;
  LdsBarrier();
  maximum = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    maximum = fmaxf(maximum, s_red[2][w]);
  const int e = RowExponent(maximum);
  // Every group of the row's 64-column chunks, zeros past H.
  const int groups = (H + kChunk - 1) / kChunk * 8;
  if (a.image) {
    // groups / 8 chunks of two 16-byte (hi, lo) planes of 64 lanes.
    const BufferResource image_out = MakeBuffer(a.image, unsigned(groups) * 256u);
    StoreB32P<kImagePolicy>(MakeBuffer(a.exps + row, 4u), tid == 0 ? 0u : kOutOfRange,
                            unsigned(e));
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int cg = tid + T * i;
      unsigned hi[4], lo[4];
#pragma unroll
      for (int k = 0; k < 8; k += 2)
        SplitPair(v[i][k], v[i][k + 1], e, hi[k / 2], lo[k / 2]);
      const unsigned idx = unsigned(((cg >> 3) * 2 + ((cg >> 2) & 1)) * 64 + 16 * (cg & 3) + row);
      StoreB128P<kImagePolicy>(image_out, cg < groups ? idx * 16u : kOutOfRange,
                               make_uint4(hi[0], hi[1], hi[2], hi[3]));
      StoreB128P<kImagePolicy>(image_out, cg < groups ? (idx + 8) * 16u : kOutOfRange,
                               make_uint4(lo[0], lo[1], lo[2], lo[3]));
    }
  }
  if (a.a16) {
    // The prompt GEMM's FP16 row (HalfRowsKernel's expressions).
    const BufferResource a16_out =
        MakeBuffer(a.a16 + std::size_t(row) * a.lda, unsigned(groups) * 16u);
    StoreF32(MakeBuffer(a.a_scale + row, 4u), tid == 0 ? 0u : kOutOfRange, ldexpf(1.0f, -e));
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int cg = tid + T * i;
      unsigned h[4];
#pragma unroll
      for (int k = 0; k < 8; k += 2)
        h[k / 2] = unsigned(ScaledHalf(v[i][k], e)) | (unsigned(ScaledHalf(v[i][k + 1], e)) << 16);
      StoreB128(a16_out, cg < groups ? unsigned(cg) * 16u : kOutOfRange,
                make_uint4(h[0], h[1], h[2], h[3]));
    }
  }
  if constexpr (kPublish) {
    __builtin_amdgcn_s_waitcnt(WaitVm(0));
    LdsBarrier();
    if (tid < kFlagCopies)
      __hip_atomic_store(flags + tid * kFlagStride + row, seq, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + T * i;
    const unsigned off = g * 8 < H ? unsigned(g) * 32 : kOutOfRange;
    if (store_x)  // uniform
      store8(x_out, off, xv[i]);
    store8(z_out, off, v[i]);
  }
}


// A fused GEMV block's watcher wave (one wave beside the compute waves):
// it polls the flags of the block's XCD copy (lanes < rows, loads through
// to memory) with short sleeps until every row carries `seq`, at most
// kSpinLimit times (past it, it records the failure in *error, host memory
// the caller checks after the launch, and goes on, so every wave leaves),
// then writes `seq` into the block's LDS word *ready. The compute waves
// issue their weight loads first and then wait on that LDS word
// (AwaitReady): a wait for a memory flag inside a compute wave would also
// wait for its weights (vector loads return in issue order), an LDS read
// does not.
constexpr int kSpinLimit = 1 << 17;
__device__ __forceinline__ void WatchRows(const unsigned* flags, unsigned seq, unsigned* error,
                                          int rows, unsigned* ready) {
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const int lane = threadIdx.x & 63;
  const BufferResource f = MakeBuffer(flags + (xcc % kFlagCopies) * kFlagStride, 4u * 8u);
  const unsigned f_off = lane < rows ? unsigned(lane) * 4u : kOutOfRange;
  unsigned got = __builtin_amdgcn_raw_buffer_load_b32(f, f_off, 0, kCachePolicySc1);
  int spins = 0;
  while (__any(lane < rows && got != seq) && spins < kSpinLimit) {
    __builtin_amdgcn_s_sleep(4);
    got = __builtin_amdgcn_raw_buffer_load_b32(f, f_off, 0, kCachePolicySc1);
    ++spins;
  }
  if (spins == kSpinLimit && lane == 0 && error)
    __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (lane == 0)
    __hip_atomic_store(ready, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// A compute wave's wait for its block's watcher: its image loads come
// after it (the compiler barrier keeps them there).
__device__ __forceinline__ void AwaitReady(const unsigned* ready, unsigned seq) {
  while (__hip_atomic_load(ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != seq)
    __builtin_amdgcn_s_sleep(1);
  asm volatile("" ::: "memory");
}

}  // namespace lfm3amd
#endif
