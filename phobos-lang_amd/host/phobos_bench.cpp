// phobos-bench for the MI355X backend: a native host of the C ABI in
// include/phobos_hip.h, the counterpart of phobos-bench/src/main.rs (with
// autotune.rs and report.rs), as a Rust caller of the backend would run it.
// It links nothing but libphobos_hip.so: no HIP headers, no Python.
//
// Kept from the reference bench:
//   * the command line (main.rs:36-160): --bench NAME, --autotune "NAME=VALUE
//     ...", --csv [PATH], --peak-fp32 / --peak-fp16tc / --peak-fp16tcf32acc
//     TFLOPS, --help, and its error texts;
//   * the problems (main.rs:461-1309): saxpy n = 2^25, alpha 2; the three
//     4096^3 GEMMs with C = 0 and (alpha, beta) = (1.5, 2.5) for gemm_fp32,
//     (1, 1) for the f16 ones; one head of 4096 x 4096 x 64 flash attention
//     at scale 1/8; inputs uniform in [-1, 1), from the in-tree Lcg
//     (phobos-base/src/rng.rs) in place of rand's SmallRng(42), seeds
//     x, A, Q = 1; y, B, K = 2; V = 3;
//   * each launch through the kernel's .ph file and entry name with the
//     caller's exploded-memref void** list, index width as the kernel's ABI
//     (launch_gemm / launch_flash, main.rs:290-371), and the reference's own
//     grid and block; the backend substitutes its geometry (phx_launch);
//   * the two-stage autotuner (autotune.rs:98-230): verify on the first
//     launch, short probes of every plan, then the fastest four timed
//     round-robin after a joint warmup, the fastest minimum wins.  The dims
//     are this backend's launch plan (phx_plan: splits, variant), pinned with
//     phx_plan_pin in place of compiling a tile config;
//   * bench() (main.rs:238-262): 10 warmups, the fastest of 100 host-timed
//     launches, each followed by a stream synchronize;
//   * the checks (main.rs:386-445, 638-679, 869-920, 1176-1188): sampled f64
//     GEMM and flash replays at the xorshift64 points, saxpy exact;
//   * the results CSV (report.rs:71-88) with MI355X peaks derived from the
//     device's CU count and clock (256 f32 and 4096 f16 matrix flops per CU
//     per clock) unless overridden.
// Not kept: the cuBLAS comparison rows (bench.py --vendor has the vendor
// library rows on ROCm).
#include "phobos_hip.h"

#include <algorithm>
#include <cctype>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

void check(int rc, const char *what) {
    if (rc) throw Error(fmt("%s: %s", what, phx_last_error()));
}

void info(const std::string &s) { printf("[phobos-bench] %s\n", s.c_str()); fflush(stdout); }

const char *const BENCHES[] = {"saxpy_fp32", "gemm_fp32", "gemm_fp16tc_fp32acc",
                               "gemm_fp16", "flash_fp32", "flash_fp16"};
const char *const DEFAULT_CSV = "phobos-bench.csv";
const int PROBES_SHORT = 5, PROBES_LONG = 30, FINALISTS = 4, WARMUP = 10, BENCH_N = 100;

std::string bench_list() {
    std::string s;
    for (const char *b : BENCHES) s += (s.empty() ? "" : ", ") + std::string(b);
    return s;
}

// ------------------------------------------------------------------ options
struct Options {
    std::string bench;  // empty: all
    std::map<std::string, int64_t> pins;
    std::string csv;  // empty: no CSV
    double peak_fp32 = 0, peak_fp16tc = 0, peak_fp16tcf32acc = 0;  // TFLOP/s, 0 = derive
    bool wants(const char *name) const { return bench.empty() || bench == name; }
};

double parse_peak(const std::string &flag, const char *value) {
    if (!value) throw Error(flag + " needs a value in TFLOP/s");
    char *end = nullptr;
    const double t = strtod(value, &end);
    if (end == value || *end) throw Error(fmt("%s value '%s' is not a number", flag.c_str(), value));
    if (!(t > 0.0)) throw Error(flag + " value must be positive");
    return t;
}

void parse_pins(const std::string &spec, std::map<std::string, int64_t> *pins) {
    std::string tok;
    auto flush = [&]() {
        if (tok.empty()) return;
        const size_t eq = tok.find('=');
        if (eq == std::string::npos)
            throw Error(fmt("bad autotune pin '%s', expected NAME=VALUE", tok.c_str()));
        const std::string name = tok.substr(0, eq), val = tok.substr(eq + 1);
        char *end = nullptr;
        const long long v = strtoll(val.c_str(), &end, 10);
        if (val.empty() || *end)
            throw Error(fmt("autotune pin '%s' has a non-integer value '%s'", name.c_str(),
                            val.c_str()));
        (*pins)[name] = v;
        tok.clear();
    };
    for (char c : spec) {
        if (c == ',' || isspace((unsigned char)c))
            flush();
        else
            tok += c;
    }
    flush();
}

Options parse(int argc, char **argv) {
    Options o;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        const char *next = i + 1 < argc ? argv[i + 1] : nullptr;
        if (a == "--bench" || a == "-bench") {
            if (!next) throw Error(a + " needs a benchmark name");
            o.bench = argv[++i];
        } else if (a == "--autotune" || a == "-autotune") {
            if (!next) throw Error(a + " needs a \"NAME=VALUE ...\" spec");
            parse_pins(argv[++i], &o.pins);
        } else if (a == "--csv" || a == "-csv") {
            o.csv = (next && next[0] != '-') ? argv[++i] : DEFAULT_CSV;
        } else if (a == "--peak-fp32" || a == "-peak-fp32") {
            o.peak_fp32 = parse_peak(a, next), ++i;
        } else if (a == "--peak-fp16tc" || a == "-peak-fp16tc") {
            o.peak_fp16tc = parse_peak(a, next), ++i;
        } else if (a == "--peak-fp16tcf32acc" || a == "-peak-fp16tcf32acc") {
            o.peak_fp16tcf32acc = parse_peak(a, next), ++i;
        } else if (a == "--help" || a == "-h") {
            printf("usage: phobos-bench [--bench NAME] [--autotune \"DIM=VAL ...\"] [--csv [PATH]] "
                   "[--peak-fp32 TFLOPS] [--peak-fp16tc TFLOPS] [--peak-fp16tcf32acc TFLOPS]\n\n"
                   "  --bench NAME                run only one benchmark: %s\n"
                   "  --autotune SPEC             pin the launch plan (skips the search), e.g.\n"
                   "                              --bench gemm_fp32 --autotune \"splits=1 variant=0\"\n"
                   "  --csv [PATH]                write a results CSV (default %s) of achieved\n"
                   "                              GFLOP/s vs theoretical peak\n"
                   "  --peak-fp32         TFLOPS  override the derived f32 matrix peak\n"
                   "  --peak-fp16tc       TFLOPS  override the derived f16 matrix peak\n"
                   "  --peak-fp16tcf32acc TFLOPS  override the derived f16 matrix f32-acc peak\n",
                   bench_list().c_str(), DEFAULT_CSV);
            exit(0);
        } else {
            throw Error(fmt("unknown argument '%s' (try --help)", a.c_str()));
        }
    }
    if (!o.bench.empty() &&
        std::none_of(std::begin(BENCHES), std::end(BENCHES),
                     [&](const char *b) { return o.bench == b; }))
        throw Error(fmt("unknown --bench '%s'; available: %s", o.bench.c_str(),
                        bench_list().c_str()));
    if (!o.pins.empty() && o.bench.empty())
        throw Error("--autotune pins are kernel-specific; pass --bench to pick one");
    return o;
}

// ------------------------------------------------------------------ report
enum class Precision { F32, F16Tc, F16TcF32 };
const char *label(Precision p) {
    return p == Precision::F32 ? "f32" : p == Precision::F16Tc ? "f16-tc" : "f16-tc-f32-acc";
}
struct Record {
    std::string bench;
    Precision prec;
    double gflops;
};
struct Peaks {
    double fp32, fp16tc, fp16tcf32;  // GFLOP/s
    double of(Precision p) const {
        return p == Precision::F32 ? fp32 : p == Precision::F16Tc ? fp16tc : fp16tcf32;
    }
};

Peaks detect_peaks(const Options &o) {
    char name[256] = {0};
    int cus = 0, clk = 0, lds = 0;
    size_t hbm = 0;
    check(phx_device_info(name, sizeof name, &cus, &clk, &hbm, &lds), "phx_device_info");
    const double hz = clk * 1e3;
    Peaks p{cus * 256.0 * hz / 1e9, cus * 4096.0 * hz / 1e9, cus * 4096.0 * hz / 1e9};
    if (o.peak_fp32 > 0) p.fp32 = o.peak_fp32 * 1e3;
    if (o.peak_fp16tc > 0) p.fp16tc = o.peak_fp16tc * 1e3;
    if (o.peak_fp16tcf32acc > 0) p.fp16tcf32 = o.peak_fp16tcf32acc * 1e3;
    info(fmt("gpu: %s (%d CUs @ %.2f GHz)", name, cus, hz / 1e9));
    info(fmt("theoretical peak: fp32 %.1f TFLOP/s%s, fp16-tc %.1f TFLOP/s%s, fp16-tc-f32-acc "
             "%.1f TFLOP/s%s",
             p.fp32 / 1e3, o.peak_fp32 > 0 ? " (override)" : "", p.fp16tc / 1e3,
             o.peak_fp16tc > 0 ? " (override)" : "", p.fp16tcf32 / 1e3,
             o.peak_fp16tcf32acc > 0 ? " (override)" : ""));
    return p;
}

void write_csv(const std::string &path, const std::vector<Record> &rs, const Peaks &pk) {
    FILE *f = fopen(path.c_str(), "w");
    if (!f) throw Error("cannot write " + path);
    fprintf(f, "benchmark,impl,precision,gflops,peak_gflops,pct_of_peak\n");
    for (const Record &r : rs) {
        const double peak = pk.of(r.prec);
        fprintf(f, "%s,phobos,%s,%.1f,%.1f,%.1f\n", r.bench.c_str(), label(r.prec), r.gflops, peak,
                100.0 * r.gflops / peak);
    }
    fclose(f);
    info(fmt("wrote %zu rows to %s", rs.size(), path.c_str()));
}

// ------------------------------------------------------------------ device
struct Buf {
    uint64_t ptr = 0;
    size_t bytes = 0;
    explicit Buf(size_t n) : bytes(n) { check(phx_malloc(&ptr, n), "phx_malloc"); }
    template <typename T>
    explicit Buf(const std::vector<T> &v) : Buf(v.size() * sizeof(T)) {
        check(phx_memcpy_h2d(ptr, v.data(), bytes), "phx_memcpy_h2d");
    }
    template <typename T>
    void to(std::vector<T> *v) const {
        check(phx_memcpy_d2h(v->data(), ptr, v->size() * sizeof(T)), "phx_memcpy_d2h");
    }
    ~Buf() {
        if (ptr) phx_free(ptr);
    }
    Buf(const Buf &) = delete;
    Buf &operator=(const Buf &) = delete;
};

std::vector<float> uniform(uint64_t seed, size_t n) {
    std::vector<float> v(n);
    check(phx_lcg_fill_f32(seed, n, v.data()), "phx_lcg_fill_f32");
    return v;
}
std::vector<uint16_t> to_f16(const std::vector<float> &x) {
    std::vector<uint16_t> h(x.size());
    check(phx_f32_to_f16(x.size(), x.data(), h.data()), "phx_f32_to_f16");
    return h;
}
std::vector<float> from_f16(const std::vector<uint16_t> &h) {
    std::vector<float> x(h.size());
    check(phx_f16_to_f32(h.size(), h.data(), x.data()), "phx_f16_to_f32");
    return x;
}
std::vector<float> f16_round(const std::vector<float> &x) { return from_f16(to_f16(x)); }

// The exploded-memref void** list of a launch: each tensor<T>[d0, d1] as
// (alloc, aligned, offset, size0, size1, stride0, stride1) at the kernel's
// index width, then the f32 scalars (launch_gemm / launch_flash,
// main.rs:290-371; saxpy's rank-1 tensors at main.rs:1230-1235).
struct Args {
    std::vector<std::vector<uint8_t>> store;
    std::vector<void *> ptrs;
    template <typename T>
    void push(T v) {
        store.emplace_back(sizeof(T));
        memcpy(store.back().data(), &v, sizeof(T));
    }
    void idx(int bits, int64_t v) {
        if (bits == 64)
            push<int64_t>(v);
        else
            push<int32_t>((int32_t)v);
    }
    void tensor(int bits, uint64_t p, std::initializer_list<int64_t> sizes) {
        push(p);
        push(p);
        idx(bits, 0);
        const std::vector<int64_t> sz(sizes);
        for (int64_t s : sz) idx(bits, s);
        std::vector<int64_t> stride(sz.size(), 1);  // row-major
        for (size_t d = sz.size() - 1; d-- > 0;) stride[d] = stride[d + 1] * sz[d + 1];
        for (int64_t s : stride) idx(bits, s);
    }
    void **list() {
        ptrs.clear();
        for (auto &s : store) ptrs.push_back(s.data());
        return ptrs.data();
    }
};

int index_bits(const char *ph, const char *entry) {
    phx_kernel k;
    check(phx_kernel_by_name(&k, ph, entry), "phx_kernel_by_name");
    int bits;
    uint32_t block[3];
    check(phx_kernel_abi(k, &bits, block), "phx_kernel_abi");
    return bits;
}

double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// ------------------------------------------------------------------ autotune
using Plan = std::pair<int, int>;  // (splits, variant)

std::string plan_str(const Plan &p) { return fmt("splits=%d variant=%d", p.first, p.second); }

// Every distinct chunk count the runtime can run over `units` K steps or key
// blocks (whole units per chunk, no empty chunk), as the runtime rounds a
// requested count.
std::vector<Plan> split_space(int64_t units, bool variant1) {
    std::vector<Plan> out;
    for (int sp : {1, 2, 3, 4, 6, 8, 12, 16}) {
        int64_t e = std::min<int64_t>(sp, units);
        if (e >= 2) {
            const int64_t per = (units + e - 1) / e;
            e = (units + per - 1) / per;
        } else {
            e = 1;
        }
        if (std::find(out.begin(), out.end(), Plan{(int)e, 0}) == out.end())
            out.push_back({(int)e, 0});
    }
    if (variant1) out.push_back({1, 1});
    return out;
}

// gemm_fp32's tilings by plan variant (TILE_M, TILE_N, TILE_K), as
// include/phobos_hip.h lists them: the .ph file's @autotune dims.
const int64_t kS32Tilings[][3] = {{256, 256, 16}, {256, 128, 16}, {128, 256, 16}, {128, 128, 16},
                                  {128, 128, 32}, {128, 128, 8},  {256, 256, 8},  {64, 64, 16}};
constexpr int kS32Count = (int)(sizeof kS32Tilings / sizeof kS32Tilings[0]);

// Narrows the space to the pinned values (autotune.rs:38-58).  gemm_fp32
// also takes TILE_M / TILE_N / TILE_K (dims not given keep the built-in
// tiling's value), which select its tiling variant.
std::vector<Plan> pin_space(std::vector<Plan> space, const std::map<std::string, int64_t> &pins,
                            bool tiles = false) {
    for (auto &kv : pins) {
        const bool tile_dim = kv.first == "TILE_M" || kv.first == "TILE_N" || kv.first == "TILE_K";
        if (kv.first != "splits" && kv.first != "variant" && !(tiles && tile_dim))
            throw Error(fmt("autotune pin '%s' is not a search dim of this kernel (dims: splits, "
                            "variant%s)",
                            kv.first.c_str(), tiles ? ", TILE_M, TILE_N, TILE_K" : ""));
    }
    if (pins.empty()) return space;
    Plan p{1, 0};
    if (pins.count("splits")) p.first = (int)pins.at("splits");
    if (pins.count("variant")) p.second = (int)pins.at("variant");
    if (tiles && (pins.count("TILE_M") || pins.count("TILE_N") || pins.count("TILE_K"))) {
        const char *names[3] = {"TILE_M", "TILE_N", "TILE_K"};
        int64_t want[3];
        for (int d = 0; d < 3; ++d) want[d] = pins.count(names[d]) ? pins.at(names[d]) : kS32Tilings[0][d];
        p.second = -1;
        for (int v = 0; v < kS32Count; ++v)
            if (want[0] == kS32Tilings[v][0] && want[1] == kS32Tilings[v][1] &&
                want[2] == kS32Tilings[v][2])
                p.second = v;
        if (p.second < 0)
            throw Error(fmt("no gemm_fp32 tiling TILE_M=%lld TILE_N=%lld TILE_K=%lld",
                            (long long)want[0], (long long)want[1], (long long)want[2]));
    }
    return {p};
}

// A plan as the log names it: gemm_fp32 with its tile dims.
std::string plan_str(phx_kernel k, const Plan &p) {
    if (k == PHX_GEMM_FP32 && p.second >= 0 && p.second < kS32Count)
        return fmt("splits=%d variant=%d (TILE_M=%lld TILE_N=%lld TILE_K=%lld)", p.first, p.second,
                   (long long)kS32Tilings[p.second][0], (long long)kS32Tilings[p.second][1],
                   (long long)kS32Tilings[p.second][2]);
    return plan_str(p);
}

struct Tuner {
    phx_kernel kernel;
    std::vector<int64_t> dims;
    std::function<void()> launch;  // one launch, synchronized
    std::function<void()> verify;  // throws on a wrong result

    void pin(const Plan &p) {
        phx_plan pl{p.first, p.second};
        check(phx_plan_pin(kernel, dims.data(), (int)dims.size(), &pl), "phx_plan_pin");
    }
    double probe() {
        const double t0 = now_s();
        launch();
        return now_s() - t0;
    }
    // Stage 1: verify and short-probe every plan; stage 2: the fastest four
    // round-robin, one launch each per round after a joint warmup, so they
    // share clocks and heat; the fastest minimum wins and stays pinned.
    Plan run(const std::vector<Plan> &space) {
        info(fmt("autotune: %zu configs", space.size()));
        std::vector<std::pair<double, Plan>> cand;
        for (const Plan &p : space) {
            try {
                pin(p);
                launch();
                verify();
                for (int w = 0; w < WARMUP; ++w) launch();
                double best = 1e30;
                for (int i = 0; i < PROBES_SHORT; ++i) best = std::min(best, probe());
                info(fmt("  %s: %.2f us", plan_str(kernel, p).c_str(), best * 1e6));
                cand.push_back({best, p});
            } catch (const Error &e) {
                info(fmt("  %s: skipped (%s)", plan_str(kernel, p).c_str(), e.what()));
            }
        }
        if (cand.empty()) throw Error("autotune: no config works");
        std::sort(cand.begin(), cand.end());
        if ((int)cand.size() > FINALISTS) cand.resize(FINALISTS);
        info(fmt("autotune: long probe of the top %zu", cand.size()));
        for (auto &c : cand) {
            pin(c.second);
            for (int w = 0; w < WARMUP; ++w) launch();
        }
        std::vector<double> mn(cand.size(), 1e30), mx(cand.size(), 0.0);
        for (int r = 0; r < PROBES_LONG; ++r)
            for (size_t i = 0; i < cand.size(); ++i) {
                pin(cand[i].second);
                const double t = probe();
                mn[i] = std::min(mn[i], t);
                mx[i] = std::max(mx[i], t);
            }
        size_t best = 0;
        for (size_t i = 0; i < cand.size(); ++i) {
            info(fmt("  %s: %.2f us (spread %.2f us)", plan_str(kernel, cand[i].second).c_str(),
                     mn[i] * 1e6, (mx[i] - mn[i]) * 1e6));
            if (mn[i] < mn[best]) best = i;
        }
        pin(cand[best].second);
        info("autotune winner: " + plan_str(kernel, cand[best].second));
        return cand[best].second;
    }
};

// The fastest of BENCH_N launches after 10 warmups (main.rs:238-262).
double bench(const char *name, const std::function<void()> &launch) {
    for (int w = 0; w < 10; ++w) launch();
    double mn = 1e30, mx = 0;
    for (int i = 0; i < BENCH_N; ++i) {
        const double t0 = now_s();
        launch();
        const double t = now_s() - t0;
        mn = std::min(mn, t);
        mx = std::max(mx, t);
    }
    info(fmt("%s: %.2f us (spread %.2f us)", name, mn * 1e6, (mx - mn) * 1e6));
    return mn;
}

// ------------------------------------------------------------------ checks
// xorshift64 sample points, the first two forced to the corners
// (main.rs:400-412).
struct Sampler {
    uint64_t state = 0x243F6A8885A308D3ull;
    size_t next(size_t limit) {
        state ^= state << 13;
        state ^= state >> 7;
        state ^= state << 17;
        return (size_t)(state % limit);
    }
};

// f64 sampled GEMM check (main.rs:386-445): A, B as given (already f16-rounded
// for the tensor-core kernels), rel = |got - want| / max(|want|, floor).
void verify_matmul(const std::vector<float> &c, const std::vector<float> &a,
                   const std::vector<float> &b, double alpha, double beta, size_t M, size_t N,
                   size_t K, bool fp16) {
    const double tol = fp16 ? 1e-2 : 1e-3, floor = fp16 ? std::sqrt((double)K) / 3.0 : 2.2250738585072014e-308;
    Sampler s;
    for (int n = 0; n < 64; ++n) {
        size_t i, j;
        if (n == 0) i = 0, j = 0;
        else if (n == 1) i = M - 1, j = N - 1;
        else i = s.next(M), j = s.next(N);
        double dot = 0;
        for (size_t k = 0; k < K; ++k) dot += (double)a[i * K + k] * (double)b[k * N + j];
        const double want = alpha * dot + beta * 0.0, got = c[i * N + j];
        const double rel = std::fabs(got - want) / std::max(std::fabs(want), floor);
        if (!(rel < tol))
            throw Error(fmt("c[%zu,%zu] = %e, want ~ %e (rel err %.2e)", i, j, got, want, rel));
    }
}

// The fp16-accumulate GEMM check (main.rs:638-679): every input and every
// step of the K sum rounded to f16 (a sequential model of the reference's
// f16 fragments), output rounded to f16, tol 1.5e-1 relative to
// max(|want|, sqrt(K)/3).  This backend accumulates in f32, which is closer
// to the exact value than the model.
void verify_matmul_fp16acc(const std::vector<float> &c, const std::vector<float> &a,
                           const std::vector<float> &b, float alpha, size_t M, size_t N,
                           size_t K) {
    const double tol = 1.5e-1, floor = std::sqrt((double)K) / 3.0;
    auto r16 = [](float x) {
        uint16_t h;
        float y;
        phx_f32_to_f16(1, &x, &h);
        phx_f16_to_f32(1, &h, &y);
        return y;
    };
    Sampler s;
    for (int n = 0; n < 64; ++n) {
        size_t i, j;
        if (n == 0) i = 0, j = 0;
        else if (n == 1) i = M - 1, j = N - 1;
        else i = s.next(M), j = s.next(N);
        float acc = 0.0f;
        for (size_t k = 0; k < K; ++k) {
            const float p = a[i * K + k] * b[k * N + j];  // a, b are f16 values already
            acc = r16(acc + p);
        }
        const double want = r16(alpha * acc), got = c[i * N + j];
        const double rel = std::fabs(got - want) / std::max(std::fabs(want), floor);
        if (!(rel < tol))
            throw Error(fmt("c[%zu,%zu] = %e, want ~ %e (rel err %.2e)", i, j, got, want, rel));
    }
}

// f64 replay of the online softmax at 64 sampled outputs (main.rs:869-920),
// |err| / max(|want|, 0.1) < 2e-2.
void verify_flash(const std::vector<float> &o, const std::vector<float> &q,
                  const std::vector<float> &k, const std::vector<float> &v, double scale,
                  size_t Nq, size_t Nk, size_t D) {
    Sampler s;
    for (int n = 0; n < 64; ++n) {
        size_t i, d;
        if (n == 0) i = 0, d = 0;
        else if (n == 1) i = Nq - 1, d = D - 1;
        else i = s.next(Nq), d = s.next(D);
        double m = -INFINITY, l = 0, acc = 0;
        for (size_t j = 0; j < Nk; ++j) {
            double sc = 0;
            for (size_t e = 0; e < D; ++e) sc += (double)q[i * D + e] * (double)k[j * D + e];
            sc *= scale;
            const double mn = std::max(m, sc), corr = std::exp(m - mn), p = std::exp(sc - mn);
            l = l * corr + p;
            acc = acc * corr + p * v[j * D + d];
            m = mn;
        }
        const double want = acc / l, got = o[i * D + d];
        const double rel = std::fabs(got - want) / std::max(std::fabs(want), 0.1);
        if (!(rel < 2e-2))
            throw Error(fmt("O[%zu,%zu] = %e, want ~ %e (rel err %.2e)", i, d, got, want, rel));
    }
}

// ------------------------------------------------------------------ benches
constexpr int PHX_SPLIT_CHUNKS_MAX = 16;  // the most chunks phx_plan_pin takes

// A device buffer bound as the split workspace of a stream while it lives.
struct Workspace {
    Buf buf;
    phx_stream s;
    Workspace(phx_stream st, size_t bytes) : buf(bytes), s(st) {
        check(phx_stream_set_workspace(s, buf.ptr, bytes), "phx_stream_set_workspace");
    }
    ~Workspace() { phx_stream_set_workspace(s, 0, 0); }
};

struct Ctx {
    const Options &opt;
    phx_stream stream;
    std::vector<Record> results;
};

void bench_saxpy(Ctx &cx) {
    if (!cx.opt.pins.empty())  // saxpy has one launch plan
        throw Error(fmt("autotune pin '%s' is not a search dim of this kernel (dims: none)",
                        cx.opt.pins.begin()->first.c_str()));
    const int64_t n = 1 << 25;
    const float alpha = 2.0f;
    const auto x = uniform(1, n), y = uniform(2, n);
    std::vector<float> out(n);
    Buf xd(x), yd(y), od(out.size() * 4);
    const int bits = index_bits("saxpy_fp32", "saxpy");
    Args a;
    a.tensor(bits, xd.ptr, {n});
    a.tensor(bits, yd.ptr, {n});
    a.tensor(bits, od.ptr, {n});
    a.push(alpha);
    void **args = a.list();
    const uint32_t block[3] = {1024, 1, 1};  // main.rs:1216
    const uint32_t grid[3] = {(uint32_t)((n + 1023) / 1024), 1, 1};
    Tuner t{PHX_SAXPY_FP32, {n}, [&] {
                check(phx_launch_by_name("saxpy_fp32", "saxpy", grid, block, cx.stream, args),
                      "saxpy launch");
                check(phx_stream_synchronize(cx.stream), "sync");
            },
            [&] {
                od.to(&out);
                for (int64_t i = 0; i < n; ++i) {
                    const float want = alpha * x[i] + y[i];  // separately rounded, no FMA
                    if (memcmp(&out[i], &want, 4))
                        throw Error(fmt("expected %g, got %g at index %lld", want, out[i],
                                        (long long)i));
                }
            }};
    // saxpy has no plan choices: the search is a single verified plan
    t.launch();
    t.verify();
    const double s = bench("phobos saxpy", t.launch);
    t.verify();
    info(fmt("check: %lld elements, correct", (long long)n));
    const double gflop = 2.0 * n / 1e9;
    info(fmt("phobos saxpy: %.1f GFLOP/s (%.1f GB/s)", gflop / s, 12.0 * n / s / 1e9));
    cx.results.push_back({"saxpy_fp32", Precision::F32, gflop / s});
}

void bench_gemm(Ctx &cx, const char *name, const char *ph, phx_kernel kern, bool f16_storage,
                bool f16_inputs, float alpha, float beta, Precision prec) {
    const int64_t M = 4096, N = 4096, K = 4096;
    auto a = uniform(1, M * K), b = uniform(2, K * N);
    if (f16_inputs) a = f16_round(a), b = f16_round(b);
    const size_t esz = f16_storage ? 2 : 4;
    std::unique_ptr<Buf> ad, bd;
    if (f16_storage)
        ad.reset(new Buf(to_f16(a))), bd.reset(new Buf(to_f16(b)));
    else
        ad.reset(new Buf(a)), bd.reset(new Buf(b));
    Buf cd(M * N * esz);
    const int bits = index_bits(ph, "gemm");
    Args ar;
    ar.tensor(bits, ad->ptr, {M, K});
    ar.tensor(bits, bd->ptr, {K, N});
    ar.tensor(bits, cd.ptr, {M, N});
    ar.push(alpha);
    ar.push(beta);
    void **args = ar.list();
    const uint32_t block[3] = {256, 1, 1}, grid[3] = {(uint32_t)(M / 128), (uint32_t)(N / 128), 1};
    // the split plans' partial sums: a buffer this host owns, bound to its
    // stream, enough for the largest split the search tries
    Workspace ws(cx.stream, (size_t)PHX_SPLIT_CHUNKS_MAX * M * N * 4);
    Tuner t{kern, {M, N, K},
            [&] {  // C starts at zero on every launch (main.rs:511)
                check(phx_memset_async(cd.ptr, 0, M * N * esz, cx.stream), "memset");
                check(phx_launch_by_name(ph, "gemm", grid, block, cx.stream, args), "gemm launch");
                check(phx_stream_synchronize(cx.stream), "sync");
            },
            [&] {
                std::vector<float> c(M * N);
                if (f16_storage) {
                    std::vector<uint16_t> h(M * N);
                    cd.to(&h);
                    c = from_f16(h);
                    verify_matmul_fp16acc(c, a, b, alpha, M, N, K);
                } else {
                    cd.to(&c);
                    verify_matmul(c, a, b, alpha, beta, M, N, K, f16_inputs);
                }
            }};
    std::vector<Plan> space = split_space(K / 32, kern == PHX_GEMM_FP16TC_FP32ACC);
    if (kern == PHX_GEMM_FP32)  // the other tilings, unsplit
        for (int v = 1; v < kS32Count; ++v) space.push_back({1, v});
    t.run(pin_space(space, cx.opt.pins, kern == PHX_GEMM_FP32));
    const double s = bench(fmt("phobos %s", name).c_str(), t.launch);
    t.verify();
    info(fmt("check: %lld elements sampled at 64 points, correct", (long long)(M * N)));
    const double gflop = (2.0 * M * N * K + (double)M * N) / 1e9;
    info(fmt("phobos %s: %.1f GFLOP/s", name, gflop / s));
    cx.results.push_back({name, prec, gflop / s});
}

void bench_flash(Ctx &cx, const char *name, const char *ph, phx_kernel kern, bool f16,
                 Precision prec) {
    const int64_t Nq = 4096, Nk = 4096, D = 64;
    const float scale = 1.0f / std::sqrt((float)D);
    auto q = uniform(1, Nq * D), k = uniform(2, Nk * D), v = uniform(3, Nk * D);
    if (f16) q = f16_round(q), k = f16_round(k), v = f16_round(v);
    std::unique_ptr<Buf> qd, kd, vd;
    if (f16)
        qd.reset(new Buf(to_f16(q))), kd.reset(new Buf(to_f16(k))), vd.reset(new Buf(to_f16(v)));
    else
        qd.reset(new Buf(q)), kd.reset(new Buf(k)), vd.reset(new Buf(v));
    Buf od(Nq * D * (f16 ? 2 : 4));
    const int bits = index_bits(ph, "flash_attention");
    Args ar;
    ar.tensor(bits, qd->ptr, {Nq, D});
    ar.tensor(bits, kd->ptr, {Nk, D});
    ar.tensor(bits, vd->ptr, {Nk, D});
    ar.tensor(bits, od.ptr, {Nq, D});
    ar.push(scale);
    void **args = ar.list();
    // @launch(128) and Nq / BR blocks with BR = 128 (main.rs:974-981)
    const uint32_t block[3] = {128, 1, 1}, grid[3] = {(uint32_t)(Nq / 128), 1, 1};
    Workspace ws(cx.stream, (size_t)PHX_SPLIT_CHUNKS_MAX * Nq * (D + 2) * 4);
    Tuner t{kern, {Nq, Nk, D},
            [&] {
                check(phx_launch_by_name(ph, "flash_attention", grid, block, cx.stream, args),
                      "flash launch");
                check(phx_stream_synchronize(cx.stream), "sync");
            },
            [&] {
                std::vector<float> o(Nq * D);
                if (f16) {
                    std::vector<uint16_t> h(Nq * D);
                    od.to(&h);
                    o = from_f16(h);
                } else {
                    od.to(&o);
                }
                verify_flash(o, q, k, v, scale, Nq, Nk, D);
            }};
    t.run(pin_space(split_space((Nk + 63) / 64, false), cx.opt.pins));
    const double s = bench(fmt("phobos %s", name).c_str(), t.launch);
    t.verify();
    info("check: 64 probes, correct");
    const double gflop = 4.0 * Nq * Nk * D / 1e9;
    info(fmt("phobos %s: %.1f GFLOP/s", name, gflop / s));
    cx.results.push_back({name, prec, gflop / s});
}

}  // namespace

int main(int argc, char **argv) {
    Options opt;
    try {
        opt = parse(argc, argv);
    } catch (const Error &e) {
        fprintf(stderr, "Error: %s\n", e.what());
        return 2;
    }
    try {
        check(phx_init(0, nullptr), "phx_init");
        Ctx cx{opt, nullptr, {}};
        check(phx_stream_create(&cx.stream), "phx_stream_create");
        if (opt.wants("saxpy_fp32")) bench_saxpy(cx);
        if (opt.wants("gemm_fp32"))
            bench_gemm(cx, "gemm_fp32", "gemm_fp32", PHX_GEMM_FP32, false, false, 1.5f, 2.5f,
                       Precision::F32);
        if (opt.wants("gemm_fp16tc_fp32acc"))
            bench_gemm(cx, "gemm_fp16tc_fp32acc", "gemm_fp16tc_fp32acc", PHX_GEMM_FP16TC_FP32ACC,
                       false, true, 1.0f, 1.0f, Precision::F16TcF32);
        if (opt.wants("gemm_fp16"))
            bench_gemm(cx, "gemm_fp16", "gemm_fp16", PHX_GEMM_FP16, true, true, 1.0f, 1.0f,
                       Precision::F16Tc);
        if (opt.wants("flash_fp32"))
            bench_flash(cx, "flash_fp32", "flash_attention_fp32", PHX_FLASH_FP32, false,
                        Precision::F32);
        if (opt.wants("flash_fp16"))
            bench_flash(cx, "flash_fp16", "flash_attention_fp16", PHX_FLASH_FP16, true,
                        Precision::F16TcF32);
        if (!opt.csv.empty()) write_csv(opt.csv, cx.results, detect_peaks(opt));
        phx_stream_destroy(cx.stream);
        phx_shutdown();
    } catch (const Error &e) {
        fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
    return 0;
}
