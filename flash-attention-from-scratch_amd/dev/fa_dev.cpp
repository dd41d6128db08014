// fa_dev -- standalone driver of the attention forward, without Python or PyTorch.
//
//   fa_dev [B H N D causal iters variant] [--lib PATH] [--warmup-ms MS] [--seed S] [--json]
//          [--std X] [--boost-keys FRAC:FACTOR] [--sink NATS] [--splitkv S] [--probe PATH]
//          defaults:  4 8 4096 128 0 20 opt,  --lib <this dir>/../fa/libfa_hip.so
//   variant: base | baseline | opt | fp16acc
//   --std X                 inputs ~ N(0, X^2) instead of N(0, 1)
//   --boost-keys FRAC:FAC   multiply floor(FRAC * N) key rows of every head (a seeded random
//                           choice) by FAC, as the benchmark's many-heads config does
//                           (--std 0.5 --boost-keys 0.01:8): row maxima then jump mid-sequence
//   --sink NATS             an attention sink: feature 0 of every query set to 4 and of key 0
//                           of every head to NATS * sqrt(D) / 4, so that key 0 scores about
//                           NATS above the other keys for every query (as tests/
//                           test_softmax_model.py's sink_qkv)
//   --splitkv S             run the split-KV entry point (fa_flash_fwd_splitkv) with S key
//                           ranges per query block (0 = the library's automatic plan) and a
//                           workspace of the plan's size; the timing covers both launches
//   --probe PATH            (a library built with FA_PROBE=1, e.g. dev/ab.py build probe
//                           --define FA_PROBE=1) after the timed launches, one more launch
//                           with the ping-pong's timeline stamps cleared before it; writes
//                           them to PATH (32 uint64 per workgroup; dev/probe.py reads them)
//
// Loads the kernel library at run time (dlopen) and calls only its C ABI (include/fa_hip.h),
// as any foreign caller would: that lets the tuning sweep (dev/tune.py) time libraries built
// with other tile tables, and keeps rocprofv3 traces free of a Python process.
// It draws fp16 inputs from a seeded generator (approximately N(0, 1)), runs one checked
// launch (a sample of output rows against an fp64 restatement of the softmax-attention row
// formula, tolerance |got - ref| <= 2e-3 + 1e-2 |ref|), then times `iters` launches with HIP
// events on a stream of its own after a warmup of at least `warmup-ms` of launches, and prints
// the median.
// Exit status: 0 ok, 1 check failed, 2 usage or runtime error.
//
// Counterpart of the reference's csrc/dev/main.cu:82-188 (same positional arguments, defaults,
// sampled-row fp64 check and event timing); the row formula follows csrc/dev/main.cu:31-63.

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "fa_hip.h"

namespace {

constexpr double kPeakTflops = 2516.6;  // MI355X dense fp16 MFMA: 256 CU x 2.4 GHz x 4096

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    }
}

struct Api {
    decltype(&fa_flash_fwd) flash_fwd = nullptr;
    decltype(&fa_last_error) last_error = nullptr;
    decltype(&fa_tile_config) tile_config = nullptr;
    decltype(&fa_version) version = nullptr;
    decltype(&fa_splitkv_plan) splitkv_plan = nullptr;
    decltype(&fa_flash_fwd_splitkv) flash_fwd_splitkv = nullptr;
};

template <class F>
F symbol(void* h, const char* name) {
    void* p = dlsym(h, name);
    if (p == nullptr) throw std::runtime_error(std::string("missing symbol ") + name);
    return reinterpret_cast<F>(p);
}

Api load_api(const std::string& path) {
    void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (h == nullptr) throw std::runtime_error(std::string("dlopen: ") + dlerror());
    Api a;
    a.flash_fwd = symbol<decltype(a.flash_fwd)>(h, "fa_flash_fwd");
    a.last_error = symbol<decltype(a.last_error)>(h, "fa_last_error");
    a.tile_config = symbol<decltype(a.tile_config)>(h, "fa_tile_config");
    a.version = symbol<decltype(a.version)>(h, "fa_version");
    a.splitkv_plan = symbol<decltype(a.splitkv_plan)>(h, "fa_splitkv_plan");
    a.flash_fwd_splitkv = symbol<decltype(a.flash_fwd_splitkv)>(h, "fa_flash_fwd_splitkv");
    return a;
}

std::string default_lib(const char* argv0) {
    std::string exe(argv0);
    const auto slash = exe.rfind('/');
    const std::string dir = slash == std::string::npos ? "." : exe.substr(0, slash);
    return dir + "/../fa/libfa_hip.so";
}

// splitmix64 (S. Vigna, public domain): one 64-bit draw per element, fast enough to fill
// hundreds of millions of inputs in a second.
uint64_t splitmix64(uint64_t& state) {
    uint64_t z = (state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Irwin-Hall: the sum of four uniform [0, 1) variates (the four 16-bit fields of one draw) has
// mean 2 and variance 1/3; centred and scaled it has mean 0, variance 1, support [-2√3, 2√3].
_Float16 normalish(uint64_t& state) {
    const uint64_t r = splitmix64(state);
    float sum = 0.0F;
    for (int f = 0; f < 4; ++f) {
        sum += static_cast<float>((r >> (16 * f)) & 0xFFFF) * (1.0F / 65536.0F);
    }
    return static_cast<_Float16>((sum - 2.0F) * 1.7320508F);
}

int parse_variant(const std::string& s) {
    if (s == "base" || s == "baseline") return FA_VARIANT_BASELINE;
    if (s == "opt") return FA_VARIANT_OPT;
    if (s == "fp16acc") return FA_VARIANT_FP16ACC;
    throw std::invalid_argument("variant must be base, opt or fp16acc, got " + s);
}

// Exact attention of query row i of head bh in double precision: scores q.k * scale over the
// visible keys, shifted by their maximum, exponentiated, normalised, and the weighted sum of V.
std::vector<double> reference_row(const std::vector<_Float16>& q, const std::vector<_Float16>& k,
                                  const std::vector<_Float16>& v, size_t bh, size_t n, size_t d,
                                  size_t i, bool causal, double scale) {
    const size_t base = bh * n * d;
    const size_t visible = causal ? i + 1 : n;
    std::vector<double> s(visible);
    double mx = -INFINITY;
    for (size_t j = 0; j < visible; ++j) {
        double dot = 0.0;
        for (size_t c = 0; c < d; ++c) {
            dot += static_cast<double>(q[base + i * d + c]) * static_cast<double>(k[base + j * d + c]);
        }
        s[j] = dot * scale;
        mx = std::max(mx, s[j]);
    }
    double sum = 0.0;
    for (double& x : s) {
        x = std::exp(x - mx);
        sum += x;
    }
    std::vector<double> out(d, 0.0);
    for (size_t j = 0; j < visible; ++j) {
        const double p = s[j] / sum;
        for (size_t c = 0; c < d; ++c) out[c] += p * static_cast<double>(v[base + j * d + c]);
    }
    return out;
}

struct Options {
    int batch = 4, heads = 8, seqlen = 4096, head_dim = 128, causal = 0, iters = 20;
    std::string variant = "opt";
    std::string lib;
    double warmup_ms = 200.0;
    uint64_t seed = 42;
    bool json = false;
    float std = 1.0F;
    double boost_frac = 0.0;
    float boost = 1.0F;
    float sink = 0.0F;  // 0: no sink
    int splitkv = -1;  // < 0: fa_flash_fwd; else fa_flash_fwd_splitkv with this many ranges
    std::string probe;  // "": no timeline dump
};

Options parse(int argc, char** argv) {
    Options o;
    o.lib = default_lib(argv[0]);
    std::vector<std::string> pos;
    for (int a = 1; a < argc; ++a) {
        const std::string s = argv[a];
        auto value = [&]() -> std::string {
            if (a + 1 >= argc) throw std::invalid_argument(s + " needs a value");
            return argv[++a];
        };
        if (s == "--lib") {
            o.lib = value();
        } else if (s == "--warmup-ms") {
            o.warmup_ms = std::stod(value());
        } else if (s == "--seed") {
            o.seed = std::stoull(value());
        } else if (s == "--json") {
            o.json = true;
        } else if (s == "--splitkv") {
            o.splitkv = std::stoi(value());
            if (o.splitkv < 0) throw std::invalid_argument("--splitkv must be >= 0");
        } else if (s == "--std") {
            o.std = std::stof(value());
        } else if (s == "--sink") {
            o.sink = std::stof(value());
        } else if (s == "--probe") {
            o.probe = value();
        } else if (s == "--boost-keys") {
            const std::string v = value();
            const auto colon = v.find(':');
            if (colon == std::string::npos) throw std::invalid_argument("--boost-keys wants FRAC:FACTOR");
            o.boost_frac = std::stod(v.substr(0, colon));
            o.boost = std::stof(v.substr(colon + 1));
            if (o.boost_frac < 0.0 || o.boost_frac > 1.0) {
                throw std::invalid_argument("--boost-keys fraction must be in [0, 1]");
            }
        } else if (s == "-h" || s == "--help") {
            throw std::invalid_argument("usage");
        } else {
            pos.push_back(s);
        }
    }
    if (pos.size() > 7) throw std::invalid_argument("too many positional arguments");
    int* ints[] = {&o.batch, &o.heads, &o.seqlen, &o.head_dim, &o.causal, &o.iters};
    for (size_t i = 0; i < pos.size() && i < 6; ++i) *ints[i] = std::stoi(pos[i]);
    if (pos.size() == 7) o.variant = pos[6];
    if (o.iters < 1) throw std::invalid_argument("iters must be >= 1");
    return o;
}

int run(const Options& o) {
    const Api api = load_api(o.lib);
    const int variant = parse_variant(o.variant);
    const bool causal = o.causal != 0;

    fa_params shape{};
    shape.batch = o.batch;
    shape.heads = o.heads;
    shape.seqlen = o.seqlen;
    shape.head_dim = o.head_dim;
    shape.causal = causal ? 1 : 0;
    shape.variant = static_cast<uint8_t>(variant);
    fa_tile_info tile{};
    if (api.tile_config(&shape, &tile) != FA_OK) throw std::invalid_argument(api.last_error());
    const size_t elems = static_cast<size_t>(o.batch) * o.heads * o.seqlen * o.head_dim;
    const size_t bytes = elems * sizeof(_Float16);

    uint64_t state = o.seed;
    std::vector<_Float16> hq(elems), hk(elems), hv(elems), ho(elems);
    for (auto* t : {&hq, &hk, &hv}) {
        for (auto& x : *t) x = static_cast<_Float16>(o.std * static_cast<float>(normalish(state)));
    }
    const size_t n_boost = static_cast<size_t>(o.boost_frac * o.seqlen);
    if (n_boost > 0) {
        std::mt19937_64 choose(o.seed + 3);
        std::vector<size_t> rows(static_cast<size_t>(o.seqlen));
        const size_t nbh = static_cast<size_t>(o.batch) * o.heads;
        for (size_t bh = 0; bh < nbh; ++bh) {
            for (size_t r = 0; r < rows.size(); ++r) rows[r] = r;
            for (size_t r = 0; r < n_boost; ++r) {  // partial Fisher-Yates: n_boost distinct rows
                std::swap(rows[r], rows[r + choose() % (rows.size() - r)]);
                _Float16* row = hk.data() + (bh * o.seqlen + rows[r]) * o.head_dim;
                for (int c = 0; c < o.head_dim; ++c) {
                    row[c] = static_cast<_Float16>(static_cast<float>(row[c]) * o.boost);
                }
            }
        }
    }

    if (o.sink != 0.0F) {
        const size_t nbh = static_cast<size_t>(o.batch) * o.heads;
        for (size_t r = 0; r < nbh * o.seqlen; ++r) hq[r * o.head_dim] = static_cast<_Float16>(4.0F);
        for (size_t bh = 0; bh < nbh; ++bh) {
            hk[bh * o.seqlen * o.head_dim] =
                static_cast<_Float16>(o.sink * std::sqrt(static_cast<float>(o.head_dim)) / 4.0F);
        }
    }

    void *dq = nullptr, *dk = nullptr, *dv = nullptr, *dout = nullptr;
    hip_check(hipMalloc(&dq, bytes), "hipMalloc q");
    hip_check(hipMalloc(&dk, bytes), "hipMalloc k");
    hip_check(hipMalloc(&dv, bytes), "hipMalloc v");
    hip_check(hipMalloc(&dout, bytes), "hipMalloc o");
    hip_check(hipMemcpy(dq, hq.data(), bytes, hipMemcpyHostToDevice), "copy q");
    hip_check(hipMemcpy(dk, hk.data(), bytes, hipMemcpyHostToDevice), "copy k");
    hip_check(hipMemcpy(dv, hv.data(), bytes, hipMemcpyHostToDevice), "copy v");
    hipStream_t stream = nullptr;
    hip_check(hipStreamCreate(&stream), "hipStreamCreate");

    fa_params p{};
    p.q = dq;
    p.k = dk;
    p.v = dv;
    p.o = dout;
    p.batch = o.batch;
    p.heads = o.heads;
    p.seqlen = o.seqlen;
    p.head_dim = o.head_dim;
    p.softmax_scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(o.head_dim)));
    p.causal = causal ? 1 : 0;
    p.variant = static_cast<uint8_t>(variant);
    fa_splitkv_info plan{};
    void* workspace = nullptr;
    if (o.splitkv >= 0) {
        if (api.splitkv_plan(&p, o.splitkv, &plan) != FA_OK) {
            throw std::invalid_argument(api.last_error());
        }
        hip_check(hipMalloc(&workspace, plan.workspace_bytes), "hipMalloc workspace");
        tile.block_q = plan.block_q;
        tile.block_k = plan.block_k;
    }
    auto launch = [&]() {
        const int rc = o.splitkv >= 0
                           ? api.flash_fwd_splitkv(&p, nullptr, o.splitkv, workspace,
                                                   plan.workspace_bytes, stream)
                           : api.flash_fwd(&p, stream);
        if (rc != FA_OK) throw std::runtime_error(api.last_error());
    };

    // One checked launch: rows 0, N/3 and N-1 of the first and last head, plus four more rows.
    launch();
    hip_check(hipStreamSynchronize(stream), "checked launch");
    hip_check(hipMemcpy(ho.data(), dout, bytes, hipMemcpyDeviceToHost), "copy o");
    const size_t nbh = static_cast<size_t>(o.batch) * o.heads;
    const size_t n = o.seqlen, d = o.head_dim;
    std::vector<std::pair<size_t, size_t>> rows;
    for (size_t bh : {size_t{0}, nbh - 1}) {
        for (size_t i : {size_t{0}, n / 3, n - 1}) rows.emplace_back(bh, i);
    }
    std::mt19937_64 pick(o.seed + 1);
    for (int r = 0; r < 4; ++r) rows.emplace_back(pick() % nbh, pick() % n);
    double max_err = 0.0, worst_excess = -INFINITY;
    for (const auto& [bh, i] : rows) {
        const auto ref = reference_row(hq, hk, hv, bh, n, d, i, causal, p.softmax_scale);
        for (size_t c = 0; c < d; ++c) {
            const double got = static_cast<double>(ho[(bh * n + i) * d + c]);
            const double err = std::fabs(got - ref[c]);
            max_err = std::max(max_err, std::isnan(err) ? INFINITY : err);
            worst_excess = std::max(worst_excess, err - (2e-3 + 1e-2 * std::fabs(ref[c])));
        }
    }
    const bool ok = worst_excess <= 0.0 && std::isfinite(max_err);

    // Warmup until the clock has settled, then `iters` timed launches.
    const auto t0 = std::chrono::steady_clock::now();
    int warm = 0;
    while (warm < 3 || std::chrono::duration<double, std::milli>(
                           std::chrono::steady_clock::now() - t0).count() < o.warmup_ms) {
        launch();
        hip_check(hipStreamSynchronize(stream), "warmup");
        ++warm;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hip_check(hipEventCreate(&e0), "hipEventCreate");
    hip_check(hipEventCreate(&e1), "hipEventCreate");
    std::vector<float> times;
    for (int it = 0; it < o.iters; ++it) {
        hip_check(hipEventRecord(e0, stream), "hipEventRecord");
        launch();
        hip_check(hipEventRecord(e1, stream), "hipEventRecord");
        hip_check(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms = 0.0F;
        hip_check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        times.push_back(ms);
    }
    std::vector<float> sorted = times;
    std::sort(sorted.begin(), sorted.end());
    const double median = sorted[sorted.size() / 2];
    double mean = 0.0;
    for (float t : times) mean += t;
    mean /= static_cast<double>(times.size());
    const double flops = 4.0 * static_cast<double>(elems) * n / (causal ? 2.0 : 1.0);
    const double tf = flops / (median * 1e-3) / 1e12;

    if (o.json) {
        std::printf(
            "{\"lib\": \"%s\", \"version\": \"%s\", \"variant\": \"%s\", \"B\": %d, \"H\": %d, "
            "\"N\": %d, \"D\": %d, \"causal\": %d, \"block_q\": %d, \"block_k\": %d, "
            "\"waves\": %d, \"schedule\": %d, \"max_abs_err\": %.3e, \"check\": \"%s\", \"iters\": %d, "
            "\"median_ms\": %.5f, \"mean_ms\": %.5f, \"min_ms\": %.5f, \"tflops\": %.2f, "
            "\"frac_of_peak\": %.4f, \"splitkv\": %d, \"n_splits\": %d, "
            "\"tiles_per_split\": %d}\n",
            o.lib.c_str(), api.version(), o.variant.c_str(), o.batch, o.heads, o.seqlen,
            o.head_dim, causal ? 1 : 0, tile.block_q, tile.block_k, tile.waves, tile.schedule,
            max_err, ok ? "ok" : "FAILED", o.iters, median, mean, static_cast<double>(sorted.front()), tf,
            tf / kPeakTflops, o.splitkv, plan.num_splits, plan.tiles_per_split);
    } else {
        std::printf("%s B=%d H=%d N=%d D=%d causal=%d tile=%dx%d/%dw sched=%d  "
                    "max_abs_err=%.2e  median=%.4f ms  %.1f TFLOPS (%.1f%% of peak)\n",
                    o.variant.c_str(), o.batch, o.heads, o.seqlen, o.head_dim, causal ? 1 : 0,
                    tile.block_q, tile.block_k, tile.waves, tile.schedule, max_err, median, tf,
                    100.0 * tf / kPeakTflops);
    }
    if (!ok) std::printf("FAILED: |err| above 2e-3 + 1e-2 |ref| on a sampled row\n");

    if (!o.probe.empty()) {
        // The stamps of one more launch (workgroups [0, 65536), kProbeSlots each), written up
        // to the last workgroup that stamped.
        constexpr size_t kProbeSlots = 32;
        void* h = dlopen(o.lib.c_str(), RTLD_NOW | RTLD_LOCAL | RTLD_NOLOAD);
        auto* clear = h ? reinterpret_cast<int (*)()>(dlsym(h, "fa_probe_clear")) : nullptr;
        auto* read = h ? reinterpret_cast<int (*)(void*, uint64_t)>(dlsym(h, "fa_probe_read"))
                       : nullptr;
        if (clear == nullptr || read == nullptr) {
            throw std::runtime_error("--probe needs a library built with FA_PROBE=1");
        }
        hip_check(hipStreamSynchronize(stream), "probe: drain");
        if (clear() != 0) throw std::runtime_error("fa_probe_clear failed");
        launch();
        hip_check(hipStreamSynchronize(stream), "probe launch");
        std::vector<uint64_t> stamps((size_t{1} << 16) * kProbeSlots);
        if (read(stamps.data(), stamps.size() * sizeof(uint64_t)) != 0) {
            throw std::runtime_error("fa_probe_read failed");
        }
        size_t used = 0;
        for (size_t i = 0; i < stamps.size(); ++i) {
            if (stamps[i] != 0) used = i / kProbeSlots + 1;
        }
        FILE* f = std::fopen(o.probe.c_str(), "wb");
        if (f == nullptr) throw std::runtime_error("cannot write " + o.probe);
        const size_t wrote =
            std::fwrite(stamps.data(), sizeof(uint64_t), used * kProbeSlots, f);
        std::fclose(f);
        if (wrote != used * kProbeSlots) throw std::runtime_error("short write to " + o.probe);
        std::printf("probe: %zu workgroups -> %s\n", used, o.probe.c_str());
    }

    hip_check(hipEventDestroy(e0), "hipEventDestroy");
    hip_check(hipEventDestroy(e1), "hipEventDestroy");
    hip_check(hipStreamDestroy(stream), "hipStreamDestroy");
    for (void* ptr : {dq, dk, dv, dout}) hip_check(hipFree(ptr), "hipFree");
    if (workspace != nullptr) hip_check(hipFree(workspace), "hipFree workspace");
    return ok ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(parse(argc, argv));
    } catch (const std::invalid_argument& e) {
        std::fprintf(stderr,
                     "error: %s\nusage: fa_dev [B H N D causal iters variant] [--lib PATH] "
                     "[--warmup-ms MS] [--seed S] [--json] [--std X] [--boost-keys FRAC:FAC] [--sink NATS] "
                     "[--splitkv S] [--probe PATH]\n",
                     e.what());
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 2;
    }
}
