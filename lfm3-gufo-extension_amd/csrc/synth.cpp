// Deterministic synthetic inputs for benchmarks and parity tests. They stand
// in for a GGUF checkpoint and for prefilled session state, which the
// build cannot download. Every value is a pure function of (seed, stream
// name, element index): SplitMix64 of a counter gives the bits, uniform
// integers take them modulo the range, normals use Box-Muller in double
// precision. Results do not depend on the thread count.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/lfm3_amd.h"

namespace {

std::uint64_t SplitMix(std::uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
std::uint64_t Bits(std::uint64_t key, std::uint64_t i) {
  return SplitMix(key ^ SplitMix(i + 0x632BE59BD9B4E019ull));
}
double Uniform01(std::uint64_t key, std::uint64_t i) {  // (0, 1]
  return double((Bits(key, i) >> 11) + 1) * 0x1.0p-53;
}
double Normal(std::uint64_t key, std::uint64_t i) {
  const double u1 = Uniform01(key, 2 * i), u2 = Uniform01(key, 2 * i + 1);
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

template<class F>
void Parallel(std::size_t n, F f) {
  const unsigned threads =
      n < (1u << 16) ? 1u : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (threads == 1) {
    f(std::size_t(0), n);
    return;
  }
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; ++t)
    pool.emplace_back(f, n * t / threads, n * (t + 1) / threads);
  for (auto& th : pool)
    th.join();
}

std::uint16_t ToHalf(float x) {
  return __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(x));
}

}  // namespace

extern "C" {

std::uint64_t lfm3_synth_key(std::uint64_t seed, const char* name) {
  std::uint64_t h = 1469598103934665603ull;  // FNV-1a of the stream name
  for (const char* p = name; p && *p; ++p)
    h = (h ^ std::uint8_t(*p)) * 1099511628211ull;
  return SplitMix(seed ^ SplitMix(h));
}

void lfm3_synth_normal(std::uint64_t key, float mean, float stddev, float* out,
                       std::size_t n) {
  Parallel(n, [&](std::size_t a, std::size_t b) {
    for (std::size_t i = a; i < b; ++i)
      out[i] = float(double(mean) + double(stddev) * Normal(key, i));
  });
}

void lfm3_synth_uniform_u32(std::uint64_t key, std::uint32_t lo,
                            std::uint32_t hi, std::uint32_t* out, std::size_t n) {
  const std::uint64_t span = std::uint64_t(hi) - lo + 1;
  Parallel(n, [&](std::size_t a, std::size_t b) {
    for (std::size_t i = a; i < b; ++i)
      out[i] = lo + std::uint32_t(Bits(key, i) % span);
  });
}

void lfm3_synth_half_normal(std::uint64_t key, std::uint16_t* out, std::size_t n) {
  Parallel(n, [&](std::size_t a, std::size_t b) {
    for (std::size_t i = a; i < b; ++i)
      out[i] = ToHalf(float(Normal(key, i)));
  });
}

// GGUF Q8_0 rows: q uniform in [-127, 127]; d = fp16(|N(0, d_std)| / 127).
void lfm3_synth_q8(std::uint64_t key, std::uint32_t rows, std::uint32_t cols,
                   float d_std, void* out) {
  const std::size_t blocks = std::size_t(rows) * (cols / 32);
  auto* bytes = static_cast<std::uint8_t*>(out);
  const std::uint64_t dkey = SplitMix(key ^ 0xD1B54A32D192ED03ull);
  Parallel(blocks, [&](std::size_t a, std::size_t b) {
    for (std::size_t blk = a; blk < b; ++blk) {
      std::uint8_t* o = bytes + blk * 34;
      const float d = float(std::fabs(double(d_std) * Normal(dkey, blk)) / 127.0);
      const std::uint16_t h = ToHalf(d);
      std::memcpy(o, &h, 2);
      for (int j = 0; j < 32; ++j)
        o[2 + j] = std::uint8_t(std::int8_t(int(Bits(key, blk * 32 + j) % 255) - 127));
    }
  });
}

}  // extern "C"
