// Shared device helpers and status plumbing for the gfx950 LFM3 kernels.
#ifndef LFM3_AMD_COMMON_HPP_
#define LFM3_AMD_COMMON_HPP_
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/lfm3_amd.h"

namespace lfm3amd {

using Half = std::uint16_t;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Q8_0 tile geometry of the device weight layout: a tile is 16 weight rows
// by one 64-column chunk (two Q8_0 blocks). Its 1024 code bytes are one
// 16-byte load per lane of a wave: lane L = 16 g + n holds row n, bytes
// [0, 8) = elements 8g..8g+7 of the chunk's first block and bytes [8, 16)
// = elements 8g..8g+7 of its second block, which is the B operand of two
// v_mfma_f32_16x16x32_f16 (one per Q8_0 block). Codes are stored biased,
// u = q + 128 (q ^ 0x80), so they decode with one byte permute and one
// packed half add. The tile's 32 fp16 scales follow as [row][block].
constexpr int kTileRows = 16;
constexpr int kChunk = 64;
constexpr int kTileCodeBytes = kTileRows * kChunk;     // 1024
constexpr int kTileScales = kTileRows * 2;             // 32 halves
constexpr std::uint8_t kCodeBias = 0x80;

inline std::uint32_t RowTiles(std::uint32_t rows) {
  return (rows + kTileRows - 1) / kTileRows;
}
inline std::uint32_t Chunks(std::uint32_t cols) {
  return (cols + kChunk - 1) / kChunk;
}

// Thread-local message of the last failed C-ABI call.
void SetError(const std::string& message);
int Fail(int status, const std::string& message);
int HipStatus(hipError_t e, const char* what);

__device__ __forceinline__ float HalfBitsToFloat(unsigned bits) {
  return float(__builtin_bit_cast(_Float16, static_cast<unsigned short>(bits)));
}
__device__ __forceinline__ Half FloatToHalfBits(float x) {
  return __builtin_bit_cast(Half, static_cast<_Float16>(x));
}

// Four biased codes (one dword) -> four exact fp16 values as two packed
// dwords. v_perm_b32 places each code byte u under an 0x64 high byte,
// which reads as 1024 + u = 1152 + q; the packed add of -1152 leaves q.
__device__ __forceinline__ void CodesToHalves(unsigned codes, unsigned& lo,
                                              unsigned& hi) {
  const h2 bias = {static_cast<_Float16>(-1152.0f),
                   static_cast<_Float16>(-1152.0f)};
  const unsigned p0 = __builtin_amdgcn_perm(codes, 0x64646464u, 0x01050004u);
  const unsigned p1 = __builtin_amdgcn_perm(codes, 0x64646464u, 0x03070206u);
  lo = __builtin_bit_cast(unsigned, __builtin_bit_cast(h2, p0) + bias);
  hi = __builtin_bit_cast(unsigned, __builtin_bit_cast(h2, p1) + bias);
}
// Eight biased codes (two dwords) -> one MFMA operand of eight fp16 values.
__device__ __forceinline__ h8 EightCodes(unsigned a, unsigned b) {
  unsigned w[4];
  CodesToHalves(a, w[0], w[1]);
  CodesToHalves(b, w[2], w[3]);
  return __builtin_bit_cast(h8, w);
}

// GEMV operand split of x0, x1 scaled by 2^e (the row or slice maximum in
// [2^14, 2^15)): hi = fp16(x 2^e) and lo = fp16((x 2^e - hi) 2^11), both
// truncated, two values per conversion instruction. x 2^e - hi is exact in
// FP32, so hi + lo 2^-11 keeps about 21 bits of x.
__device__ __forceinline__ void SplitPair(float x0, float x1, int e, unsigned& hi,
                                          unsigned& lo) {
  const auto hp = __builtin_amdgcn_cvt_pkrtz(ldexpf(x0, e), ldexpf(x1, e));
  const float r0 = fmaf(float(hp[0]), -2048.0f, ldexpf(x0, e + 11));
  const float r1 = fmaf(float(hp[1]), -2048.0f, ldexpf(x1, e + 11));
  hi = __builtin_bit_cast(unsigned, hp);
  lo = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_pkrtz(r0, r1));
}

// Prompt activations (hip/q8_prefill.hpp:27-51): a row with maximum
// magnitude m is scaled by 2^e, e = 14 - ilogb(m) (0 for a zero row), which
// puts m in [2^14, 2^15), rounded to fp16, and carries the scale 2^-e.
__device__ __forceinline__ int RowExponent(float maximum) {
  return maximum > 0.0f ? 14 - ilogbf(maximum) : 0;
}
__device__ __forceinline__ Half ScaledHalf(float x, int e) {
  return FloatToHalfBits(ldexpf(x, e));
}

// Raw buffer resources over one tensor (at most 2^31 bytes). A lane whose
// byte offset is past the range reads zeros, so guarded loads need no
// branch and the compiler's wait counts stay exact across them.
using BufferResource = __amdgpu_buffer_rsrc_t;
constexpr int kBufferWord3 = 0x00020000;  // 32-bit data format, raw access
constexpr unsigned kOutOfRange = 0x80000000u;
inline bool BufferFits(std::size_t bytes) { return bytes < std::size_t(kOutOfRange); }
__device__ __forceinline__ BufferResource MakeBuffer(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), kBufferWord3);
}
__device__ __forceinline__ uint4 LoadB128(BufferResource res, unsigned offset) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_amdgcn_raw_buffer_load_b128(res, offset, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 LoadF4(BufferResource res, unsigned offset) {
  const uint4 v = LoadB128(res, offset);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                     __uint_as_float(v.w));
}
__device__ __forceinline__ unsigned LoadB32(BufferResource res, unsigned offset) {
  return __builtin_amdgcn_raw_buffer_load_b32(res, offset, 0, 0);
}
// s_waitcnt immediates (vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt
// 11:8), issued through the builtin so the compiler's own wait insertion
// sees them.
constexpr int WaitVm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int kWaitLgkm0 = 15 | (3 << 14) | (7 << 4);

// Per-component select (a select of whole vectors in a register array can
// become a select of addresses into scratch memory).
__device__ __forceinline__ uint4 SelectU4(bool p, uint4 a, uint4 b) {
  return make_uint4(p ? a.x : b.x, p ? a.y : b.y, p ? a.z : b.z, p ? a.w : b.w);
}

// A store at kOutOfRange (or any offset past the resource) is dropped.
__device__ __forceinline__ void StoreF32(BufferResource res, unsigned offset, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), res, offset, 0, 0);
}
__device__ __forceinline__ void StoreB32(BufferResource res, unsigned offset, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, res, offset, 0, 0);
}
__device__ __forceinline__ void StoreB64(BufferResource res, unsigned offset, uint2 v) {
  typedef unsigned u2 __attribute__((ext_vector_type(2)));
  const u2 w = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(w, res, offset, 0, 0);
}
__device__ __forceinline__ void StoreB128(BufferResource res, unsigned offset, uint4 v) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, res, offset, 0, 0);
}
// Buffer stores with a cache policy: kCachePolicySc1 writes through the
// XCD's L2 to memory (the coherence point of every XCD); a load with it
// reads from there.
constexpr int kCachePolicySc1 = 16;
template<int kPolicy>
__device__ __forceinline__ void StoreB32P(BufferResource res, unsigned offset, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, res, offset, 0, kPolicy);
}
template<int kPolicy>
__device__ __forceinline__ void StoreB128P(BufferResource res, unsigned offset, uint4 v) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, res, offset, 0, kPolicy);
}
__device__ __forceinline__ void StoreF4(BufferResource res, unsigned offset, float a, float b,
                                        float c, float d) {
  StoreB128(res, offset,
            make_uint4(__float_as_uint(a), __float_as_uint(b), __float_as_uint(c),
                       __float_as_uint(d)));
}

// Greedy-pick order key: the float's bits made monotone as unsigned, then
// the inverted index, so the largest key is the first index of the maximum
// (std::max_element).
__device__ __forceinline__ unsigned long long ArgKey(float value, unsigned index) {
  unsigned bits = __float_as_uint(value);
  bits = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<unsigned long long>(bits) << 32) | (0xffffffffu - index);
}


// Cross-lane moves without the LDS crossbar: DPP within 16-lane rows
// (quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror, row_mirror,
// row_ror 8) and gfx950's permlane swaps across rows. Every lane of a
// reduced group ends with the same value (the pairs add commutatively).
template<int kCtrl>
__device__ __forceinline__ float Dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float GroupMax16(float v) {
  v = fmaxf(v, Dpp<0xB1>(v));
  v = fmaxf(v, Dpp<0x4E>(v));
  v = fmaxf(v, Dpp<0x141>(v));
  return fmaxf(v, Dpp<0x140>(v));
}
__device__ __forceinline__ float GroupSum16(float v) {
  v += Dpp<0xB1>(v);
  v += Dpp<0x4E>(v);
  v += Dpp<0x141>(v);
  return v + Dpp<0x140>(v);
}
// v of lane L plus v of lane L ^ 8 (within a row), L ^ 16, L ^ 32.
__device__ __forceinline__ float SumXor8(float v) { return v + Dpp<0x128>(v); }
// The row swaps as inline assembly: this compiler folds the sum of the two
// results of __builtin_amdgcn_permlane{16,32}_swap(v, v) into twice the
// first. Two wait states after the VALU writes of the operands.
__device__ __forceinline__ float SumXor16(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float SumXor32(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// Maxima of v over lanes L, L ^ 8 (within a row), L ^ 16 and L ^ 32.
__device__ __forceinline__ float MaxXor8(float v) { return fmaxf(v, Dpp<0x128>(v)); }
__device__ __forceinline__ float MaxXor16(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
__device__ __forceinline__ float MaxXor32(float v) {
  unsigned a = __builtin_bit_cast(unsigned, v), b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}

// Wave-wide sum and maximum through DPP and the row swaps (no LDS
// crossbar); every lane ends with the same value.
__device__ __forceinline__ float WaveSum(float v) { return SumXor32(SumXor16(GroupSum16(v))); }
__device__ __forceinline__ float WaveMax(float v) { return MaxXor32(MaxXor16(GroupMax16(v))); }

}  // namespace lfm3amd
#endif
