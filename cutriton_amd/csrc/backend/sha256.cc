// SHA-256 per FIPS 180-4 (section 6.2): 64-byte blocks, big-endian message
// schedule, the first 32 bits of the fractional parts of the cube roots of
// the first 64 primes as round constants and of the square roots of the
// first 8 primes as the initial hash.
#include <array>
#include <cmath>
#include <cstdint>
#include <string>

#include "cutriton/backend/kernel_artifact.h"

namespace cutriton {
namespace {

// Derives the FIPS 180-4 constant tables from their definition instead of
// transcribing them: frac(p^(1/3)) and frac(p^(1/2)) of the leading primes,
// computed exactly with integer cube/square roots of p * 2^96 / p * 2^64.
struct Tables {
  std::array<std::uint32_t, 64> k{};
  std::array<std::uint32_t, 8> h0{};
  Tables() {
    int primes[64];
    int count = 0;
    for (int n = 2; count < 64; ++n) {
      bool prime = true;
      for (int d = 2; d * d <= n; ++d) {
        if (n % d == 0) {
          prime = false;
          break;
        }
      }
      if (prime) primes[count++] = n;
    }
    for (int i = 0; i < 64; ++i) k[static_cast<std::size_t>(i)] = FracRoot(primes[i], 3);
    for (int i = 0; i < 8; ++i) h0[static_cast<std::size_t>(i)] = FracRoot(primes[i], 2);
  }
  // First 32 fractional bits of p^(1/degree), by integer root search on
  // p * 2^(32*degree) (exact; no floating point rounding involved).
  static std::uint32_t FracRoot(int p, int degree) {
    using u128 = unsigned __int128;
    const u128 target = static_cast<u128>(p) << (32 * degree);
    // root = floor(target^(1/degree)); bounded by p * 2^32.
    u128 lo = 0;
    u128 hi = static_cast<u128>(p) << 32;
    while (lo < hi) {
      const u128 mid = lo + (hi - lo + 1) / 2;
      u128 power = 1;
      bool over = false;
      for (int d = 0; d < degree; ++d) {
        if (power > target / mid) {
          over = true;
          break;
        }
        power *= mid;
      }
      if (over || power > target) hi = mid - 1; else lo = mid;
    }
    return static_cast<std::uint32_t>(lo & 0xffffffffu);
  }
};

const Tables& Constants() {
  static const Tables tables;
  return tables;
}

inline std::uint32_t Rotr(std::uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

}  // namespace

std::string Sha256Hex(const std::string& data) {
  const Tables& t = Constants();
  std::array<std::uint32_t, 8> h = t.h0;
  std::string message = data;
  const std::uint64_t bit_length = static_cast<std::uint64_t>(data.size()) * 8u;
  message.push_back(static_cast<char>(0x80));
  while (message.size() % 64 != 56) message.push_back('\0');
  for (int shift = 56; shift >= 0; shift -= 8) {
    message.push_back(static_cast<char>((bit_length >> shift) & 0xffu));
  }
  std::uint32_t w[64];
  for (std::size_t block = 0; block < message.size(); block += 64) {
    for (int i = 0; i < 16; ++i) {
      const auto* p = reinterpret_cast<const unsigned char*>(message.data() + block + 4 * i);
      w[i] = (std::uint32_t{p[0]} << 24) | (std::uint32_t{p[1]} << 16) |
             (std::uint32_t{p[2]} << 8) | std::uint32_t{p[3]};
    }
    for (int i = 16; i < 64; ++i) {
      const std::uint32_t s0 = Rotr(w[i - 15], 7) ^ Rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const std::uint32_t s1 = Rotr(w[i - 2], 17) ^ Rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    std::uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
      const std::uint32_t big1 = Rotr(e, 6) ^ Rotr(e, 11) ^ Rotr(e, 25);
      const std::uint32_t choose = (e & f) ^ (~e & g);
      const std::uint32_t t1 = hh + big1 + choose + t.k[static_cast<std::size_t>(i)] + w[i];
      const std::uint32_t big0 = Rotr(a, 2) ^ Rotr(a, 13) ^ Rotr(a, 22);
      const std::uint32_t majority = (a & b) ^ (a & c) ^ (b & c);
      const std::uint32_t t2 = big0 + majority;
      hh = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d;
    h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  static const char* hex = "0123456789abcdef";
  std::string out;
  out.reserve(64);
  for (const std::uint32_t word : h) {
    for (int shift = 28; shift >= 0; shift -= 4) out.push_back(hex[(word >> shift) & 0xfu]);
  }
  return out;
}

}  // namespace cutriton
