// Launchers used only inside the library (not part of the C-ABI).
#ifndef LFM3_AMD_INTERNAL_HPP_
#define LFM3_AMD_INTERNAL_HPP_
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace lfm3amd {
// dst[i][0..count) = src + i * ld for rows i < rows, with dst pointers read
// from a device table (per-session logits / frontier rows of a round).
int LaunchScatterRows(const float* src, std::size_t ld, float* const* dst,
                      std::uint32_t rows, std::size_t count,
                      hipStream_t stream);
}  // namespace lfm3amd
#endif
