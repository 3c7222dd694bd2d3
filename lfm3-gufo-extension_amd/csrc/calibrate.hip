// Device ceilings measured beside the published MI355X peaks: a plain
// streaming read of a large buffer (what HBM delivers to a kernel that only
// loads) and a register-only f16 MFMA loop (what the matrix cores deliver
// with no operand traffic). The bench reports every roofline fraction
// against the published peak and these two beside it.
//
// Both results are checkable: the read folds every 32-bit word it loads
// into one XOR per block, and the MFMA loop multiplies all-ones operands,
// so each accumulator holds 32 x iterations exactly.
#include "common.hpp"

namespace lfm3amd {
namespace {

constexpr int kReadThreads = 512, kReadDepth = 8;  // 16-byte loads in flight a lane
constexpr int kMfmaThreads = 256, kMfmaChains = 8;  // independent accumulators a wave

__device__ __forceinline__ unsigned Fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// Grid-stride read, kReadDepth loads issued before any is folded; lane
// XORs reduce through the wave, and each wave's result XORs into the
// block's word through LDS, written by one vector store.
__launch_bounds__(kReadThreads) __global__
    void StreamReadKernel(const uint4* __restrict__ p, std::size_t n, unsigned* __restrict__ sink) {
  __shared__ unsigned s_fold[kReadThreads / 64];
  const std::size_t stride = std::size_t(gridDim.x) * kReadThreads;
  std::size_t i = std::size_t(blockIdx.x) * kReadThreads + threadIdx.x;
  unsigned acc = 0;
  for (; i + (kReadDepth - 1) * stride < n; i += kReadDepth * stride) {
    uint4 v[kReadDepth];
#pragma unroll
    for (int d = 0; d < kReadDepth; ++d)
      v[d] = p[i + d * stride];
#pragma unroll
    for (int d = 0; d < kReadDepth; ++d)
      acc ^= Fold(v[d]);
  }
  for (; i < n; i += stride)
    acc ^= Fold(p[i]);
#pragma unroll
  for (int m = 32; m; m >>= 1)
    acc ^= unsigned(__shfl_xor(int(acc), m, 64));
  if ((threadIdx.x & 63) == 0)
    s_fold[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned total = 0;
    for (int w = 0; w < kReadThreads / 64; ++w)
      total ^= s_fold[w];
    sink[blockIdx.x] = total;
  }
}

// kMfmaChains independent v_mfma_f32_16x16x32_f16 chains a wave over
// all-ones operands; each wave writes the sum of its accumulators' lane 0
// elements (4 kMfmaChains x 32 x iterations, `origin` being 0). The
// chains are named variables (an indexed array of accumulators makes the
// register allocator copy them through VGPRs every step), and each starts
// from its own multiple of the runtime `origin`, so the compiler cannot
// merge chains it would otherwise prove equal.
__launch_bounds__(kMfmaThreads) __global__
    void MfmaLoopKernel(int iterations, float origin, float* __restrict__ sink) {
  static_assert(kMfmaChains == 8, "eight named chains");
  h8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    ones[i] = static_cast<_Float16>(1.0f);
  const f4 o = {origin, origin, origin, origin};
  f4 c0 = o, c1 = 2.0f * o, c2 = 3.0f * o, c3 = 4.0f * o, c4 = 5.0f * o, c5 = 6.0f * o,
     c6 = 7.0f * o, c7 = 8.0f * o;
  for (int it = 0; it < iterations; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c3, 0, 0, 0);
    c4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c4, 0, 0, 0);
    c5 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c5, 0, 0, 0);
    c6 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c6, 0, 0, 0);
    c7 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ones, c7, 0, 0, 0);
  }
  const f4 t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
  if ((threadIdx.x & 63) == 0)
    sink[std::size_t(blockIdx.x) * (kMfmaThreads / 64) + (threadIdx.x >> 6)] =
        (t[0] + t[1]) + (t[2] + t[3]);
}

}  // namespace
}  // namespace lfm3amd

using namespace lfm3amd;

extern "C" {

int lfm3_measure_stream_read(const void* buffer, std::size_t bytes, unsigned* sink,
                             std::uint32_t blocks, void* stream) {
  if (!buffer || !sink || !bytes || bytes % 16 || !blocks || blocks > 65535 ||
      (reinterpret_cast<std::uintptr_t>(buffer) & 15))
    return Fail(LFM3_E_INVALID, "unsupported LFM3 stream-read measurement");
  StreamReadKernel<<<blocks, kReadThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(buffer), bytes / 16, sink);
  return HipStatus(hipGetLastError(), "LFM3 stream-read launch");
}

int lfm3_measure_mfma_f16(std::uint32_t iterations, std::uint32_t blocks, float* sink,
                          void* stream) {
  // 32 x iterations x 4 x kMfmaChains stays an exact FP32 integer.
  if (!sink || !iterations || iterations > (1u << 14) || !blocks || blocks > 65535)
    return Fail(LFM3_E_INVALID, "unsupported LFM3 MFMA measurement");
  MfmaLoopKernel<<<blocks, kMfmaThreads, 0, static_cast<hipStream_t>(stream)>>>(
      int(iterations), 0.0f, sink);
  return HipStatus(hipGetLastError(), "LFM3 MFMA loop launch");
}

std::uint64_t lfm3_measure_mfma_f16_flops(std::uint32_t iterations, std::uint32_t blocks) {
  return std::uint64_t(blocks) * (kMfmaThreads / 64) * kMfmaChains * iterations * 16384ull;
}

}  // extern "C"
