// test_util.hpp -- seeded inputs and comparators for the project's C++
// parity suites over the lh:: drop-in.
#ifndef LONGHORN_TESTS_TEST_UTIL_HPP
#define LONGHORN_TESTS_TEST_UTIL_HPP

#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace lh_test {

// splitmix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number
// generators", 2014): a 64-bit counter-based stream, identical on every
// platform, so a seed names the same inputs everywhere.
inline uint64_t splitmix64(uint64_t& state) {
    uint64_t z = (state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// n floats uniform in [lo, hi): the top 24 bits of each draw scaled to [0, 1).
inline std::vector<float> uniform(int64_t n, uint64_t seed, float lo = -1.0f, float hi = 1.0f) {
    uint64_t st = seed * 0x2545f4914f6cdd1dull + 1;
    std::vector<float> out(static_cast<size_t>(n));
    for (float& v : out) {
        const float u = static_cast<float>(splitmix64(st) >> 40) * (1.0f / 16777216.0f);
        v = lo + (hi - lo) * u;
    }
    return out;
}

// n ints uniform in [0, bound).
inline std::vector<int32_t> uniform_ids(int64_t n, int32_t bound, uint64_t seed) {
    uint64_t st = seed ^ 0x5851f42d4c957f2dull;
    std::vector<int32_t> out(static_cast<size_t>(n));
    for (int32_t& v : out) v = static_cast<int32_t>(splitmix64(st) % static_cast<uint64_t>(bound));
    return out;
}

// Relative Frobenius error ||got - want|| / ||want||, in double.
inline double rel_frobenius(const std::vector<float>& got, const std::vector<float>& want) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < want.size(); ++i) {
        const double d = static_cast<double>(got[i]) - want[i];
        num += d * d;
        den += static_cast<double>(want[i]) * want[i];
    }
    return den > 0.0 ? std::sqrt(num / den) : std::sqrt(num);
}

// Bitwise equality of two float / integer buffers.
template <typename T>
inline ::testing::AssertionResult BitEqual(const std::vector<T>& a, const std::vector<T>& b) {
    if (a.size() != b.size()) return ::testing::AssertionFailure() << "size mismatch";
    for (size_t i = 0; i < a.size(); ++i)
        if (std::memcmp(&a[i], &b[i], sizeof(T)) != 0)
            return ::testing::AssertionFailure() << "first difference at index " << i << ": " << +a[i] << " vs "
                                                 << +b[i];
    return ::testing::AssertionSuccess();
}

}  // namespace lh_test

#endif  // LONGHORN_TESTS_TEST_UTIL_HPP
