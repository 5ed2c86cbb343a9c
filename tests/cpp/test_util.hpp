// test_util.hpp -- seeded inputs and comparators for the C++ suites; the
// same helpers the reference suites use (lh_test::random_vector, random_ids,
// AllClose; tests/test_util.hpp:17-57), plus the relative Frobenius error
// the parity bounds are stated in.
#ifndef LONGHORN_TESTS_TEST_UTIL_HPP
#define LONGHORN_TESTS_TEST_UTIL_HPP

#include <gtest/gtest.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

namespace lh_test {

constexpr float kAtolF32 = 1e-4f;
constexpr float kRtolF32 = 1e-4f;

// Uniform floats in [lo, hi) from a 32-bit Mersenne twister with `seed`.
inline std::vector<float> random_vector(int64_t n, uint32_t seed, float lo = -1.0f, float hi = 1.0f) {
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> u(lo, hi);
    std::vector<float> out(static_cast<size_t>(n));
    for (float& v : out) v = u(gen);
    return out;
}

inline std::vector<int32_t> random_ids(int64_t n, int32_t vocab, uint32_t seed) {
    std::mt19937 gen(seed);
    std::uniform_int_distribution<int32_t> u(0, vocab - 1);
    std::vector<int32_t> out(static_cast<size_t>(n));
    for (int32_t& v : out) v = u(gen);
    return out;
}

// |a - b| <= atol + rtol*|b| everywhere (NaN fails).
inline ::testing::AssertionResult AllClose(const std::vector<float>& a, const std::vector<float>& b,
                                           float atol = kAtolF32, float rtol = kRtolF32) {
    if (a.size() != b.size())
        return ::testing::AssertionFailure() << "size mismatch: " << a.size() << " vs " << b.size();
    for (size_t i = 0; i < a.size(); ++i) {
        const float d = std::fabs(a[i] - b[i]);
        const float tol = atol + rtol * std::fabs(b[i]);
        if (!(d <= tol))
            return ::testing::AssertionFailure() << "mismatch at index " << i << ": " << a[i] << " vs " << b[i]
                                                 << " (|diff|=" << d << ", tol=" << tol << ")";
    }
    return ::testing::AssertionSuccess();
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
