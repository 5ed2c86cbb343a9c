// bench_util.hpp -- timing harness of the MI355X backend's benchmark driver.
//
// Same shape as the reference's bench harness (bench/bench_util.hpp: named
// specs with a per-iteration FLOP and byte count, warm-up then timed
// iterations, percentiles, a roofline classification and CSV output), with
// a second timing mode for device work:
//   Host: steady_clock around a host callable, as the reference times its
//         CPU kernels (bench_util.hpp:98-127).  Used for the synchronous lh::
//         drop-in, whose calls include host<->device copies.
//   Hip:  a device callable enqueues one launch on a stream; every timed
//         launch is bracketed by HIP events on that stream (per-launch
//         percentiles), and one more event pair around all timed launches
//         gives the steady-state mean without per-launch gaps.
// Rooflines use MI355X's published peaks: HBM 8 TB/s, dense bf16 MFMA
// 2.5 PFLOP/s, dense int8 MFMA 5.0 POP/s.
#ifndef LONGHORN_MI355X_BENCH_UTIL_HPP
#define LONGHORN_MI355X_BENCH_UTIL_HPP

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <functional>
#include <iomanip>
#include <ostream>
#include <string>
#include <vector>

namespace lh_bench {

constexpr double kHbmPeakBytes = 8.0e12;
constexpr double kBf16PeakFlops = 2.5e15;
constexpr double kInt8PeakOps = 5.0e15;
constexpr double kFp8PeakFlops = 5.0e15;

enum class Timing { Host, Hip };

struct BenchSpec {
    std::string name;
    std::function<void()> host_fn;                  // Host timing
    std::function<void(hipStream_t, int)> dev_fn;  // Hip timing: enqueue launch number i
    double flops = 0.0;       // per iteration
    double bytes = 0.0;       // per iteration (algorithmic)
    double peak_flops = kBf16PeakFlops;  // the MFMA roof this work runs on
    int warmup = 5;
    int iters = 50;
};

struct BenchResult {
    std::string name;
    Timing timing = Timing::Host;
    double p50_us = 0, p90_us = 0, p99_us = 0, min_us = 0, max_us = 0, mean_us = 0;
    double flops = 0, bytes = 0, peak_flops = kBf16PeakFlops;
    double tflops() const { return mean_us > 0 ? flops / (mean_us * 1e-6) / 1e12 : 0; }
    double gbps() const { return mean_us > 0 ? bytes / (mean_us * 1e-6) / 1e9 : 0; }
};

// Arithmetic intensity against the ridge of the roof the work runs on.
struct Roofline {
    double ai = 0, ridge = 0, mfma_frac = 0, hbm_frac = 0;
    const char* bound = "memory";
};

inline Roofline roofline(const BenchResult& r) {
    Roofline o;
    o.ai = r.bytes > 0 ? r.flops / r.bytes : 0;
    o.ridge = r.peak_flops / kHbmPeakBytes;
    o.mfma_frac = r.tflops() * 1e12 / r.peak_flops;
    o.hbm_frac = r.gbps() * 1e9 / kHbmPeakBytes;
    o.bound = o.ai >= o.ridge ? "compute" : "memory";
    return o;
}

inline double percentile(std::vector<double> v, double q) {
    if (v.empty()) return 0;
    std::sort(v.begin(), v.end());
    const double pos = q * (v.size() - 1);
    const size_t lo = static_cast<size_t>(pos);
    const size_t hi = std::min(lo + 1, v.size() - 1);
    return v[lo] + (pos - lo) * (v[hi] - v[lo]);
}

inline void fill_stats(BenchResult& r, const std::vector<double>& us) {
    r.p50_us = percentile(us, 0.5);
    r.p90_us = percentile(us, 0.9);
    r.p99_us = percentile(us, 0.99);
    r.min_us = *std::min_element(us.begin(), us.end());
    r.max_us = *std::max_element(us.begin(), us.end());
}

inline bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "lh_bench: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

inline bool run_host(const BenchSpec& s, BenchResult& r) {
    for (int i = 0; i < s.warmup; ++i) s.host_fn();
    std::vector<double> us;
    double sum = 0;
    for (int i = 0; i < s.iters; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        s.host_fn();
        const auto t1 = std::chrono::steady_clock::now();
        us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count());
        sum += us.back();
    }
    fill_stats(r, us);
    r.mean_us = sum / s.iters;
    return true;
}

inline bool run_hip(const BenchSpec& s, BenchResult& r, hipStream_t st) {
    for (int i = 0; i < s.warmup; ++i) s.dev_fn(st, i);
    if (!hip_ok(hipStreamSynchronize(st), "warm-up")) return false;
    // per-launch event pairs
    std::vector<hipEvent_t> ev(2 * s.iters + 2);
    for (auto& e : ev)
        if (!hip_ok(hipEventCreate(&e), "hipEventCreate")) return false;
    bool ok = true;
    for (int i = 0; i < s.iters; ++i) {
        ok &= hip_ok(hipEventRecord(ev[2 * i], st), "hipEventRecord");
        s.dev_fn(st, s.warmup + i);
        ok &= hip_ok(hipEventRecord(ev[2 * i + 1], st), "hipEventRecord");
    }
    // back-to-back launches between one event pair
    ok &= hip_ok(hipEventRecord(ev[2 * s.iters], st), "hipEventRecord");
    for (int i = 0; i < s.iters; ++i) s.dev_fn(st, s.warmup + s.iters + i);
    ok &= hip_ok(hipEventRecord(ev[2 * s.iters + 1], st), "hipEventRecord");
    ok &= hip_ok(hipStreamSynchronize(st), "timed launches");
    std::vector<double> us;
    for (int i = 0; ok && i < s.iters; ++i) {
        float ms = 0;
        ok = hip_ok(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]), "hipEventElapsedTime");
        us.push_back(ms * 1e3);
    }
    float total = 0;
    if (ok) ok = hip_ok(hipEventElapsedTime(&total, ev[2 * s.iters], ev[2 * s.iters + 1]), "hipEventElapsedTime");
    for (auto& e : ev) (void)hipEventDestroy(e);
    if (!ok) return false;
    fill_stats(r, us);
    r.mean_us = total * 1e3 / s.iters;
    return true;
}

inline void print_header(std::ostream& os, Timing t) {
    os << std::left << std::setw(44) << (t == Timing::Hip ? "benchmark (hip events)" : "benchmark (host clock)")
       << std::right << std::setw(11) << "mean us" << std::setw(11) << "p50 us" << std::setw(11) << "p90 us"
       << std::setw(12) << "TFLOP/s" << std::setw(11) << "GB/s" << "\n";
    os << std::string(44 + 11 * 4 + 12, '-') << "\n";
}

inline void print_row(std::ostream& os, const BenchResult& r) {
    os << std::left << std::setw(44) << r.name << std::right << std::fixed << std::setprecision(2) << std::setw(11)
       << r.mean_us << std::setw(11) << r.p50_us << std::setw(11) << r.p90_us << std::setprecision(1) << std::setw(12)
       << r.tflops() << std::setw(11) << r.gbps() << "\n";
}

inline void print_roofline(std::ostream& os, const std::vector<BenchResult>& rs) {
    os << std::left << std::setw(44) << "roofline (MI355X peaks)" << std::right << std::setw(10) << "AI"
       << std::setw(10) << "ridge" << std::setw(10) << "bound" << std::setw(12) << "% MFMA" << std::setw(10)
       << "% HBM" << "\n";
    os << std::string(44 + 10 * 3 + 22, '-') << "\n";
    for (const auto& r : rs) {
        const Roofline f = roofline(r);
        os << std::left << std::setw(44) << r.name << std::right << std::fixed << std::setprecision(1)
           << std::setw(10) << f.ai << std::setw(10) << f.ridge << std::setw(10) << f.bound << std::setw(12)
           << 100.0 * f.mfma_frac << std::setw(10) << 100.0 * f.hbm_frac << "\n";
    }
}

inline bool write_csv(const std::string& path, const std::vector<BenchResult>& rs) {
    FILE* f = std::fopen(path.c_str(), "w");
    if (!f) return false;
    std::fprintf(f, "name,timing,mean_us,p50_us,p90_us,p99_us,min_us,max_us,tflops,gbps\n");
    for (const auto& r : rs)
        std::fprintf(f, "%s,%s,%.3f,%.3f,%.3f,%.3f,%.3f,%.3f,%.3f,%.3f\n", r.name.c_str(),
                     r.timing == Timing::Hip ? "hip" : "host", r.mean_us, r.p50_us, r.p90_us, r.p99_us, r.min_us,
                     r.max_us, r.tflops(), r.gbps());
    return std::fclose(f) == 0;
}

inline bool write_roofline_csv(const std::string& path, const std::vector<BenchResult>& rs) {
    FILE* f = std::fopen(path.c_str(), "w");
    if (!f) return false;
    std::fprintf(f, "name,flops,bytes,ai,ridge,bound,tflops,gbps,mfma_frac,hbm_frac\n");
    for (const auto& r : rs) {
        const Roofline o = roofline(r);
        std::fprintf(f, "%s,%.6g,%.6g,%.4f,%.2f,%s,%.3f,%.3f,%.4f,%.4f\n", r.name.c_str(), r.flops, r.bytes, o.ai,
                     o.ridge, o.bound, r.tflops(), r.gbps(), o.mfma_frac, o.hbm_frac);
    }
    return std::fclose(f) == 0;
}

class BenchSuite {
public:
    void add(BenchSpec s) { specs_.push_back(std::move(s)); }
    size_t size() const { return specs_.size(); }

    // Runs every spec whose name contains `filter`; a spec without a callable
    // for the chosen timing is skipped.
    std::vector<BenchResult> run(std::ostream& os, Timing t, const std::string& filter, int iters_override,
                                 int warmup_override) {
        std::vector<BenchResult> out;
        hipStream_t st = nullptr;
        if (t == Timing::Hip && !hip_ok(hipStreamCreate(&st), "hipStreamCreate")) return out;
        print_header(os, t);
        for (auto& s : specs_) {
            if (!filter.empty() && s.name.find(filter) == std::string::npos) continue;
            if ((t == Timing::Hip && !s.dev_fn) || (t == Timing::Host && !s.host_fn)) continue;
            if (iters_override > 0) s.iters = iters_override;
            if (warmup_override >= 0) s.warmup = warmup_override;
            BenchResult r;
            r.name = s.name;
            r.timing = t;
            r.flops = s.flops;
            r.bytes = s.bytes;
            r.peak_flops = s.peak_flops;
            const bool ok = t == Timing::Hip ? run_hip(s, r, st) : run_host(s, r);
            if (!ok) continue;
            print_row(os, r);
            out.push_back(r);
        }
        if (st) (void)hipStreamDestroy(st);
        return out;
    }

private:
    std::vector<BenchSpec> specs_;
};

}  // namespace lh_bench

#endif  // LONGHORN_MI355X_BENCH_UTIL_HPP
