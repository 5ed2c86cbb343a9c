// gtest/gtest.h -- a small GoogleTest-compatible test harness.
//
// GoogleTest is not installed in this environment and cannot be fetched, so
// the C++ suites build against this header instead.  It implements the part
// of the GoogleTest API the LonghornAI kernel suites use: TEST, the
// EXPECT_* / ASSERT_* comparison macros with streamed messages,
// ::testing::AssertionResult / AssertionSuccess / AssertionFailure, and a
// runner (RUN_ALL_TESTS, --gtest_filter=Suite.Name patterns with '*').
#ifndef LONGHORN_GTEST_COMPAT_H
#define LONGHORN_GTEST_COMPAT_H

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

namespace testing {

class AssertionResult {
public:
    explicit AssertionResult(bool ok) : ok_(ok) {}
    AssertionResult(const AssertionResult& o) : ok_(o.ok_), msg_(o.msg_.str()) {}
    explicit operator bool() const { return ok_; }
    template <typename T> AssertionResult& operator<<(const T& v) {
        msg_ << v;
        return *this;
    }
    std::string message() const { return msg_.str(); }

private:
    bool ok_;
    std::ostringstream msg_;
};
inline AssertionResult AssertionSuccess() { return AssertionResult(true); }
inline AssertionResult AssertionFailure() { return AssertionResult(false); }

namespace internal {

struct TestInfo {
    std::string suite, name;
    std::function<void()> body;
};
inline std::vector<TestInfo>& registry() {
    static std::vector<TestInfo> r;
    return r;
}
inline bool& current_failed() {
    static bool f = false;
    return f;
}
struct Registrar {
    Registrar(const char* suite, const char* name, std::function<void()> body) {
        registry().push_back({suite, name, std::move(body)});
    }
};

// Failure reporting: `FailSink(file, line, text) = Message() << ...`.  The
// assignment binds looser than `<<`, so the whole streamed message is built
// first; operator= records the failure and returns void, which also lets
// ASSERT_* write `return FailSink(...) = ...`.
class Message {
public:
    Message() = default;
    Message(const Message& o) : s_(o.s_.str()) {}
    template <typename T> Message& operator<<(const T& v) {
        s_ << v;
        return *this;
    }
    std::string str() const { return s_.str(); }

private:
    std::ostringstream s_;
};
class FailSink {
public:
    FailSink(const char* file, int line, std::string text) : file_(file), line_(line), text_(std::move(text)) {}
    void operator=(const Message& m) const {
        current_failed() = true;
        const std::string extra = m.str();
        std::printf("%s:%d: Failure\n%s%s%s\n", file_, line_, text_.c_str(), extra.empty() ? "" : "\n",
                    extra.c_str());
    }

private:
    const char* file_;
    int line_;
    std::string text_;
};

// EXPECT_TRUE / EXPECT_FALSE on a bool or an AssertionResult.
struct BoolCheck {
    bool ok;
    std::string msg;
    BoolCheck(bool v, bool want) : ok(v == want) {}
    BoolCheck(const AssertionResult& r, bool want) : ok(bool(r) == want), msg(r.message()) {}
    explicit operator bool() const { return ok; }
    std::string text(const char* expr) const {
        return std::string("Value of: ") + expr + (msg.empty() ? std::string() : "\n" + msg);
    }
};

template <typename A, typename B>
std::string cmp_text(const char* ea, const char* eb, const char* op, const A& a, const B& b) {
    std::ostringstream s;
    s << "Expected: (" << ea << ") " << op << " (" << eb << "), actual: " << a << " vs " << b;
    return s.str();
}

inline bool glob(const char* p, const char* s) {
    if (*p == '\0') return *s == '\0';
    if (*p == '*') return glob(p + 1, s) || (*s && glob(p, s + 1));
    return *s && (*p == '?' || *p == *s) && glob(p + 1, s + 1);
}
inline bool filter_match(const std::string& filter, const std::string& full) {
    // ':'-separated positive patterns, optional '-'-prefixed negative list
    std::string pos = filter, neg;
    const size_t dash = filter.find('-');
    if (dash != std::string::npos) {
        pos = filter.substr(0, dash);
        neg = filter.substr(dash + 1);
    }
    auto any = [&](const std::string& list) {
        std::stringstream ss(list);
        std::string pat;
        while (std::getline(ss, pat, ':'))
            if (!pat.empty() && glob(pat.c_str(), full.c_str())) return true;
        return false;
    };
    return (pos.empty() || any(pos)) && !(neg.size() && any(neg));
}

struct Options {
    std::string filter;
};
inline Options& options() {
    static Options o;
    return o;
}

}  // namespace internal

inline void InitGoogleTest(int* argc, char** argv) {
    for (int i = 1; i < *argc; ++i) {
        const char* a = argv[i];
        if (std::strncmp(a, "--gtest_filter=", 15) == 0) internal::options().filter = a + 15;
    }
}

}  // namespace testing

inline int RUN_ALL_TESTS() {
    using namespace testing::internal;
    int run = 0, failed = 0;
    std::vector<std::string> failures;
    for (auto& t : registry()) {
        const std::string full = t.suite + "." + t.name;
        if (!filter_match(options().filter, full)) continue;
        std::printf("[ RUN      ] %s\n", full.c_str());
        std::fflush(stdout);
        current_failed() = false;
        t.body();
        ++run;
        if (current_failed()) {
            ++failed;
            failures.push_back(full);
            std::printf("[  FAILED  ] %s\n", full.c_str());
        } else {
            std::printf("[       OK ] %s\n", full.c_str());
        }
        std::fflush(stdout);
    }
    std::printf("[==========] %d tests ran.\n[  PASSED  ] %d tests.\n", run, run - failed);
    for (auto& f : failures) std::printf("[  FAILED  ] %s\n", f.c_str());
    return failed ? 1 : 0;
}

#define LHG_CAT2(a, b) a##b
#define LHG_CAT(a, b) LHG_CAT2(a, b)
#define TEST(suite, name)                                                              \
    static void LHG_CAT(lhg_test_##suite##_, name)();                                  \
    static ::testing::internal::Registrar LHG_CAT(lhg_reg_##suite##_, name)(           \
        #suite, #name, &LHG_CAT(lhg_test_##suite##_, name));                           \
    static void LHG_CAT(lhg_test_##suite##_, name)()

// `if (ok) ; else <report>` keeps a trailing `<< msg` attached to the report.
#define LHG_REPORT(text) ::testing::internal::FailSink(__FILE__, __LINE__, text) = ::testing::internal::Message()
#define LHG_NONFATAL
#define LHG_FATAL return
#define LHG_CHECK(ok, text, kind) \
    if (ok)                       \
        ;                         \
    else                          \
        kind LHG_REPORT(text)

#define LHG_CMP(a, b, op, kind) LHG_CHECK(((a)op(b)), ::testing::internal::cmp_text(#a, #b, #op, (a), (b)), kind)
#define EXPECT_EQ(a, b) LHG_CMP(a, b, ==, LHG_NONFATAL)
#define EXPECT_NE(a, b) LHG_CMP(a, b, !=, LHG_NONFATAL)
#define EXPECT_LT(a, b) LHG_CMP(a, b, <, LHG_NONFATAL)
#define EXPECT_LE(a, b) LHG_CMP(a, b, <=, LHG_NONFATAL)
#define EXPECT_GT(a, b) LHG_CMP(a, b, >, LHG_NONFATAL)
#define EXPECT_GE(a, b) LHG_CMP(a, b, >=, LHG_NONFATAL)
#define ASSERT_EQ(a, b) LHG_CMP(a, b, ==, LHG_FATAL)
#define ASSERT_NE(a, b) LHG_CMP(a, b, !=, LHG_FATAL)
#define ASSERT_LT(a, b) LHG_CMP(a, b, <, LHG_FATAL)
#define ASSERT_LE(a, b) LHG_CMP(a, b, <=, LHG_FATAL)
#define ASSERT_GT(a, b) LHG_CMP(a, b, >, LHG_FATAL)
#define ASSERT_GE(a, b) LHG_CMP(a, b, >=, LHG_FATAL)

#define LHG_BOOL(cond, want, kind)                                          \
    if (const ::testing::internal::BoolCheck lhg_c{(cond), want})           \
        ;                                                                   \
    else                                                                    \
        kind LHG_REPORT(lhg_c.text(#cond))
#define EXPECT_TRUE(c) LHG_BOOL(c, true, LHG_NONFATAL)
#define EXPECT_FALSE(c) LHG_BOOL(c, false, LHG_NONFATAL)
#define ASSERT_TRUE(c) LHG_BOOL(c, true, LHG_FATAL)
#define ASSERT_FALSE(c) LHG_BOOL(c, false, LHG_FATAL)

#define LHG_NEAR(a, b, tol, kind)                                                        \
    LHG_CHECK(std::fabs(static_cast<double>(a) - static_cast<double>(b)) <= (tol),     \
              ::testing::internal::cmp_text(#a, #b, "~=", (a), (b)), kind)
#define EXPECT_NEAR(a, b, tol) LHG_NEAR(a, b, tol, LHG_NONFATAL)
#define ASSERT_NEAR(a, b, tol) LHG_NEAR(a, b, tol, LHG_FATAL)

#endif  // LONGHORN_GTEST_COMPAT_H
