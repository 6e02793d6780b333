// gemv_timeline -- where a GEMV launch's time goes, per wave.
//
// Runs the timeline instances of zlm_gemv_timeline.hip (the library's
// configs[1] gate/up kernel and the decode step's normed gate_up, the same
// template instantiations with per-wave s_memrealtime points) back to back
// over weight copies rotated past the 256 MiB Infinity Cache, then prints, for
// one launch out of 16 traced ones:
//   * the spread of the waves' start times and the gap from the previous
//     launch's last wave to this launch's first wave;
//   * the time each wave spent staging x (plus the norm), on its first tile
//     (the plain kernel) and on the rest;
//   * the waves' end times, overall, by the order in which a CU received its
//     workgroups (dispatch slot = workgroup index / workgroups per slot) and
//     as waves ending per 0.5 us.
// The points sit outside the tile loops (a point inside them changed the
// compiled loop: 117 -> 64 VGPRs and 10.4 -> 11.4 us for the plain kernel),
// so the timeline instances keep the library kernels' register counts.
// The weights are pseudo-random bytes with small fp16 scales: the kernels'
// timing does not depend on the values.  Usage:
//   gemv_timeline [c1|normpair] [path to zlm_gemv_timeline_gfx950.hsaco]
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "gemv_timeline: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

// Host mirror of GemvArgs (gemv_impl.h).
struct Args {
    const void* w0;
    const void* d0;
    const void* w1;
    const void* d1;
    const float* x;
    const float* xw;
    float* y;
    const float* res;
    uint32_t rows, nb;
    float eps;
    uint32_t act;
};

double pct(std::vector<double> v, double p) {
    std::sort(v.begin(), v.end());
    const size_t i = std::min(v.size() - 1, static_cast<size_t>(p / 100.0 * static_cast<double>(v.size() - 1) + 0.5));
    return v[i];
}

void row(const char* name, const std::vector<double>& v) {
    printf("  %-40s p0 %6.0f  p10 %6.0f  p50 %6.0f  p90 %6.0f  p100 %6.0f ns\n", name, pct(v, 0), pct(v, 10),
           pct(v, 50), pct(v, 90), pct(v, 100));
}

}  // namespace

int main(int argc, char** argv) {
    const std::string which = argc > 1 ? argv[1] : "c1";
    std::string path = argc > 2 ? argv[2] : "";
    if (path.empty()) {
        std::string self = argv[0];
        const size_t slash = self.rfind('/');
        path = (slash == std::string::npos ? std::string(".") : self.substr(0, slash)) + "/zlm_gemv_timeline_gfx950.hsaco";
    }
    const bool pair = which == "normpair";
    if (!pair && which != "c1") {
        fprintf(stderr, "usage: gemv_timeline [c1|normpair] [code object]\n");
        return 2;
    }
    // c1: Q8_0 12288 x 4096, 4-wave workgroups at 4 per CU (the library's grid);
    // normpair: Q4_0 gate and up 12288 x 4096, 16-wave workgroups at one per CU.
    const uint32_t rows = 12288, nb = 128, bpb = pair ? 16 : 32;
    int cus = 0;
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0), "device");
    const unsigned threads = pair ? 1024 : 256;
    const unsigned grid = pair ? static_cast<unsigned>(cus) : 4u * static_cast<unsigned>(cus);
    const unsigned per_slot = static_cast<unsigned>(cus);  // workgroups dealt before a CU gets its next one
    const unsigned waves = grid * threads / 64;

    hipModule_t mod;
    check(hipModuleLoad(&mod, path.c_str()), path.c_str());
    hipFunction_t f;
    check(hipModuleGetFunction(&f, mod, pair ? "zlm_tl_q4_0_normpair_s2_pfqw16" : "zlm_tl_q8_0_r1_s4"), "kernel");

    const size_t pay = static_cast<size_t>(rows) * nb * bpb, sc = static_cast<size_t>(rows) * nb * 2;
    const int copies = static_cast<int>((512ull << 20) / (pay + sc)) + 2;
    std::vector<uint8_t> hp(pay);
    std::vector<uint16_t> hs(rows * static_cast<size_t>(nb));
    uint64_t s = 0x5A4C4D01u;
    for (auto& b : hp) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        b = static_cast<uint8_t>(s >> 56);
    }
    for (auto& d : hs) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        d = static_cast<uint16_t>(0x1c00u | ((s >> 40) & 0x3ffu));  // fp16 in [2^-8, 2^-7)
    }
    std::vector<uint8_t*> W(copies);
    std::vector<uint16_t*> D(copies);
    for (int c = 0; c < copies; c++) {
        check(hipMalloc(reinterpret_cast<void**>(&W[c]), pay), "hipMalloc");
        check(hipMalloc(reinterpret_cast<void**>(&D[c]), sc), "hipMalloc");
        check(hipMemcpy(W[c], hp.data(), pay, hipMemcpyHostToDevice), "upload");
        check(hipMemcpy(D[c], hs.data(), sc, hipMemcpyHostToDevice), "upload");
    }
    std::vector<float> hx(4096), hw(4096, 1.0f);
    for (auto& v : hx) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        v = static_cast<float>(static_cast<int64_t>(s >> 40) - (1ll << 23)) / static_cast<float>(1 << 23);
    }
    float *x, *xw, *y;
    check(hipMalloc(reinterpret_cast<void**>(&x), 4096 * 4), "hipMalloc");
    check(hipMalloc(reinterpret_cast<void**>(&xw), 4096 * 4), "hipMalloc");
    check(hipMalloc(reinterpret_cast<void**>(&y), rows * 4), "hipMalloc");
    check(hipMemcpy(x, hx.data(), 4096 * 4, hipMemcpyHostToDevice), "upload");
    check(hipMemcpy(xw, hw.data(), 4096 * 4, hipMemcpyHostToDevice), "upload");
    constexpr int kTraced = 16;
    uint64_t* tl;
    const size_t tl_words = static_cast<size_t>(kTraced) * waves * 8;
    check(hipMalloc(reinterpret_cast<void**>(&tl), tl_words * 8), "hipMalloc");
    check(hipMemset(tl, 0, tl_words * 8), "memset");
    hipStream_t st;
    check(hipStreamCreate(&st), "stream");

    auto launch = [&](int c, uint64_t* t) {
        if (pair) {
            Args a = {W[(2 * c) % copies], D[(2 * c) % copies], W[(2 * c + 1) % copies], D[(2 * c + 1) % copies],
                      x, xw, y, nullptr, rows, nb, 1e-6f, 0u};
            void* args[] = {&a, &t};
            check(hipModuleLaunchKernel(f, grid, 1, 1, threads, 1, 1, 0, st, args, nullptr), "launch");
        } else {
            uint32_t r = rows, n = nb;
            void* args[] = {&W[c % copies], &D[c % copies], &x, &y, &r, &n, &t};
            check(hipModuleLaunchKernel(f, grid, 1, 1, threads, 1, 1, 0, st, args, nullptr), "launch");
        }
    };
    uint64_t* none = nullptr;
    for (int i = 0; i < 3000; i++) launch(i, none);  // clocks up
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "event");
    check(hipEventCreate(&e1), "event");
    check(hipEventRecord(e0, st), "record");
    for (int i = 0; i < 2000; i++) launch(i, none);
    check(hipEventRecord(e1, st), "record");
    check(hipEventSynchronize(e1), "sync");
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
    for (int i = 0; i < kTraced; i++) launch(i, tl + static_cast<size_t>(i) * waves * 8);
    check(hipStreamSynchronize(st), "sync");
    std::vector<uint64_t> h(tl_words);
    check(hipMemcpy(h.data(), tl, tl_words * 8, hipMemcpyDeviceToHost), "download");

    const double tick = 10.0;  // ns per s_memrealtime tick (100 MHz)
    const double row_bytes = pair ? 2.0 * 4096 * 18 / 32 : 4096.0 * 34 / 32;
    printf("%s: %s, grid %u x %u threads, %d weight copies; untimed-launch period %.3f us (HIP events, 2000 launches)\n",
           which.c_str(), pair ? "Q4_0 RMSNorm + gate/up + SiLU 2 x 12288 x 4096" : "Q8_0 12288 x 4096", grid, threads,
           copies, ms * 1000.0 / 2000);
    // launch gaps over the traced launches
    std::vector<double> gaps, spans;
    uint64_t prev_end = 0;
    for (int L = 0; L < kTraced; L++) {
        const uint64_t* w = h.data() + static_cast<size_t>(L) * waves * 8;
        uint64_t s0 = UINT64_MAX, e = 0;
        for (unsigned v = 0; v < waves; v++) {
            s0 = std::min(s0, w[v * 8]);
            for (int i = 7; i >= 1; i--)
                if (w[v * 8 + i]) {
                    e = std::max(e, w[v * 8 + i]);
                    break;
                }
        }
        if (L > 0) gaps.push_back((static_cast<double>(s0) - static_cast<double>(prev_end)) * tick);
        spans.push_back(static_cast<double>(e - s0) * tick);
        prev_end = e;
    }
    printf("  first wave start -> last wave end: median %.0f ns; last wave end -> next launch's first wave start: "
           "median %.0f ns (min %.0f)\n",
           pct(spans, 50), pct(gaps, 50), pct(gaps, 0));
    const int L = kTraced / 2;
    const uint64_t* w = h.data() + static_cast<size_t>(L) * waves * 8;
    uint64_t s0 = UINT64_MAX;
    for (unsigned v = 0; v < waves; v++) s0 = std::min(s0, w[v * 8]);
    std::vector<double> start, staged, first, rest, end;
    std::vector<std::vector<double>> end_by_slot(8);
    const unsigned wpg = threads / 64;
    for (unsigned v = 0; v < waves; v++) {
        const uint64_t* p = w + v * 8;
        // points: start, x staged, [first tile done,] end
        const int np = p[3] ? 4 : 3;
        start.push_back(static_cast<double>(p[0] - s0) * tick);
        staged.push_back(static_cast<double>(p[1] - p[0]) * tick);
        if (np == 4) {
            first.push_back(static_cast<double>(p[2] - p[1]) * tick);
            rest.push_back(static_cast<double>(p[3] - p[2]) * tick);
        } else {
            rest.push_back(static_cast<double>(p[2] - p[1]) * tick);
        }
        const double e = static_cast<double>(p[np - 1] - s0) * tick;
        end.push_back(e);
        const unsigned slot = (v / wpg) / per_slot;
        if (slot < 8) end_by_slot[slot].push_back(e);
    }
    printf("launch %d of %d (%u waves, %.0f bytes of weights per wave):\n", L, kTraced, waves,
           row_bytes * rows / waves);
    row("wave start (after the first wave's)", start);
    row("x staged (after the wave's start)", staged);
    if (!first.empty()) row("first tile (after x staged)", first);
    row(first.empty() ? "all tiles (after x staged)" : "other tiles (after the first)", rest);
    row("wave end (after the first wave's start)", end);
    printf("  wave end by the CU's dispatch slot (median ns):");
    for (int i = 0; i < 8; i++)
        if (!end_by_slot[i].empty()) printf(" slot %d %.0f", i, pct(end_by_slot[i], 50));
    printf("\n  waves ending per 0.5 us after the first wave's start:\n   ");
    double tmax = 0;
    for (double t : end) tmax = std::max(tmax, t);
    const int bins = static_cast<int>(tmax / 500.0) + 1;
    std::vector<int> hist(bins, 0);
    for (double t : end) hist[static_cast<int>(t / 500.0)]++;
    for (int i = 0; i < bins; i++) printf(" %d", hist[i]);
    printf("\n");
    return 0;
}
