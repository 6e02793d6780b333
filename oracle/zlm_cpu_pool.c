/*
 * zlm_cpu_pool.c -- the CPU baseline's thread pool and width dispatch.
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's CPU baseline.  Nothing in zlm_amd/
 * links or calls this file.
 *
 * A persistent pool restating zlm's runtime/pool.zig: helper threads pinned
 * one per physical core (utils/cpu.zig), a job slot guarded by a mutex and two
 * conditions with a bounded spin before a helper sleeps (pool.zig:34-44,
 * :103-134), rows split by rangeOf (pool.zig:52-66) with the caller running
 * part 0 and helper h part h + 1.  The sweep itself is zlm_cpu_sweep.c, built
 * for 8 lanes (AVX2) and 16 lanes (AVX-512); `lanes` 0 picks the width zlm's
 * `simd.native` would on this host (kernels/simd.zig:30-41).
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "zlm_oracle.h"

int orc_sweep_matvec_l8(uint32_t, const uint8_t *, size_t, size_t, size_t, const float *, float *, size_t, size_t);
int orc_sweep_matvec_l16(uint32_t, const uint8_t *, size_t, size_t, size_t, const float *, float *, size_t, size_t);
int orc_sweep_matvec_int_q8_l8(uint32_t, const uint8_t *, size_t, size_t, size_t, const int8_t *, const float *,
                               const int32_t *, float *, size_t, size_t);
int orc_sweep_matvec_int_q8_l16(uint32_t, const uint8_t *, size_t, size_t, size_t, const int8_t *, const float *,
                                const int32_t *, float *, size_t, size_t);

int orc_fast_native_lanes(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512dq"))
        return 16;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 8;
    return 0;
}

static int pick_lanes(int lanes) {
    const int native = orc_fast_native_lanes();
    if (lanes == 0) return native;
    if (lanes == 16 && native != 16) return 0;
    if (lanes == 8 && native == 0) return 0;
    return (lanes == 8 || lanes == 16) ? lanes : 0;
}

int orc_fast_matvec(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, const float *x, float *out,
                    size_t begin, size_t end, int lanes) {
    switch (pick_lanes(lanes)) {
    case 8: return orc_sweep_matvec_l8(t, w, w_len, k, rows, x, out, begin, end);
    case 16: return orc_sweep_matvec_l16(t, w, w_len, k, rows, x, out, begin, end);
    default: return ORC_E_UNSUPPORTED;
    }
}

/* The int sweep of one token (orc_matvec_int's arithmetic; Q4_0 and Q8_0). */
int orc_fast_matvec_int(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, const float *x,
                        float *out, size_t begin, size_t end, int lanes) {
    const int l = pick_lanes(lanes);
    if (!l) return ORC_E_UNSUPPORTED;
    if (k % 32 != 0) return ORC_E_SHAPE;
    const size_t chunks = k / 32;
    if (chunks > 2048) return orc_fast_matvec(t, w, w_len, k, rows, x, out, begin, end, l);
    int8_t qx[2048 * 32];
    float dx[2048];
    int32_t sums[2048];
    orc_quantize_act_q8(x, chunks, qx, dx, sums);
    return l == 16 ? orc_sweep_matvec_int_q8_l16(t, w, w_len, k, rows, qx, dx, sums, out, begin, end)
                   : orc_sweep_matvec_int_q8_l8(t, w, w_len, k, rows, qx, dx, sums, out, begin, end);
}

/* ---- physical cores of this process's affinity mask ------------------- */

static int read_int(const char *path) {
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    int v = -1;
    if (fscanf(f, "%d", &v) != 1) v = -1;
    fclose(f);
    return v;
}

/* One logical CPU per (package, core) pair among the CPUs this process may
 * run on, in CPU order; returns the count written to cpus (at most max). */
int orc_physical_cores(int *cpus, int max) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof set, &set) != 0) return 0;
    int n = 0, keys[1024];
    for (int c = 0; c < CPU_SETSIZE && n < max && n < 1024; c++) {
        if (!CPU_ISSET(c, &set)) continue;
        char p[128];
        snprintf(p, sizeof p, "/sys/devices/system/cpu/cpu%d/topology/core_id", c);
        const int core = read_int(p);
        snprintf(p, sizeof p, "/sys/devices/system/cpu/cpu%d/topology/physical_package_id", c);
        const int pkg = read_int(p);
        const int key = (core < 0 || pkg < 0) ? -1 - c : pkg * 65536 + core;
        int seen = 0;
        for (int i = 0; i < n; i++) seen |= keys[i] == key;
        if (seen) continue;
        keys[n] = key;
        cpus[n++] = c;
    }
    return n;
}

/* ---- the pool ------------------------------------------------------------ */

typedef struct {
    int mode; /* 0 fp GEMV, 1 int GEMM over m tokens */
    uint32_t t;
    const uint8_t *w;
    size_t w_len, k, rows, m;
    const float *x;
    float *out;
    int lanes;
} pool_job;

#define MAX_HELPERS 255
#define SPIN_ITERS 3000

static struct {
    pthread_mutex_t mu;
    pthread_cond_t work, done;
    pthread_t tid[MAX_HELPERS];
    int helpers, parts;
    int cpus[MAX_HELPERS + 1];
    int shutdown;
    _Atomic unsigned long generation;
    _Atomic int finished;
    pool_job job;
    int started;
} P = {.mu = PTHREAD_MUTEX_INITIALIZER, .work = PTHREAD_COND_INITIALIZER, .done = PTHREAD_COND_INITIALIZER};

static void run_part(const pool_job *j, size_t part, size_t parts) {
    size_t b, e;
    orc_range_of(j->rows, parts, part, &b, &e);
    if (b >= e) return;
    if (j->mode == 0) {
        orc_fast_matvec(j->t, j->w, j->w_len, j->k, j->rows, j->x, j->out, b, e, j->lanes);
    } else {
        for (size_t tok = 0; tok < j->m; tok++)
            orc_fast_matvec_int(j->t, j->w, j->w_len, j->k, j->rows, j->x + tok * j->k, j->out + tok * j->rows, b,
                                e, j->lanes);
    }
}

static void pin(int cpu) {
    if (cpu < 0) return;
    cpu_set_t s;
    CPU_ZERO(&s);
    CPU_SET(cpu, &s);
    pthread_setaffinity_np(pthread_self(), sizeof s, &s);
}

static void *helper_main(void *arg) {
    const int index = (int)(intptr_t)arg;
    pin(P.cpus[index + 1]);
    unsigned long seen = 0;
    for (;;) {
        int spins = 0;
        while (atomic_load_explicit(&P.generation, memory_order_acquire) == seen && spins < SPIN_ITERS) {
            __builtin_ia32_pause();
            spins++;
        }
        pthread_mutex_lock(&P.mu);
        while (!P.shutdown && atomic_load(&P.generation) == seen) pthread_cond_wait(&P.work, &P.mu);
        if (P.shutdown) {
            pthread_mutex_unlock(&P.mu);
            return NULL;
        }
        seen = atomic_load(&P.generation);
        const pool_job job = P.job;
        const int parts = P.parts;
        pthread_mutex_unlock(&P.mu);
        run_part(&job, (size_t)index + 1, (size_t)parts);
        if (atomic_fetch_add_explicit(&P.finished, 1, memory_order_acq_rel) + 1 == parts - 1) {
            pthread_mutex_lock(&P.mu);
            pthread_cond_signal(&P.done);
            pthread_mutex_unlock(&P.mu);
        }
    }
}

static void pool_stop(void) {
    if (!P.started) return;
    pthread_mutex_lock(&P.mu);
    P.shutdown = 1;
    pthread_cond_broadcast(&P.work);
    pthread_mutex_unlock(&P.mu);
    for (int i = 0; i < P.helpers; i++) pthread_join(P.tid[i], NULL);
    P.started = 0;
    P.shutdown = 0;
    P.helpers = 0;
}

/* Start (or restart) the pool with `threads` workers, the caller included,
 * pinned one per physical core; returns the worker count. */
int orc_pool_start(int threads) {
    int cpus[MAX_HELPERS + 1];
    const int n = orc_physical_cores(cpus, MAX_HELPERS + 1);
    if (threads < 1) threads = 1;
    if (n > 0 && threads > n) threads = n;
    if (threads > MAX_HELPERS + 1) threads = MAX_HELPERS + 1;
    if (P.started && P.helpers + 1 == threads) return threads;
    pool_stop();
    for (int i = 0; i < threads; i++) P.cpus[i] = n > 0 ? cpus[i % n] : -1;
    P.helpers = threads - 1;
    atomic_store(&P.generation, 0);
    for (int i = 0; i < P.helpers; i++) pthread_create(&P.tid[i], NULL, helper_main, (void *)(intptr_t)i);
    P.started = 1;
    return threads;
}

void orc_pool_stop(void) { pool_stop(); }

static void pool_run(const pool_job *job) {
    const int parts = P.helpers + 1;
    if (parts > 1) {
        pthread_mutex_lock(&P.mu);
        P.job = *job;
        P.parts = parts;
        atomic_store(&P.finished, 0);
        atomic_fetch_add_explicit(&P.generation, 1, memory_order_release);
        pthread_cond_broadcast(&P.work);
        pthread_mutex_unlock(&P.mu);
    }
    run_part(job, 0, (size_t)parts);
    if (parts > 1) {
        int spins = 0;
        while (atomic_load_explicit(&P.finished, memory_order_acquire) < parts - 1 && spins < SPIN_ITERS * 100) {
            __builtin_ia32_pause();
            spins++;
        }
        pthread_mutex_lock(&P.mu);
        while (atomic_load(&P.finished) < parts - 1) pthread_cond_wait(&P.done, &P.mu);
        pthread_mutex_unlock(&P.mu);
    }
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Min-of-`reps` wall seconds of one pooled call, the calling thread pinned to
 * the first physical core for the duration (its mask restored after).  Call r
 * reads weight copy r % n_copies: copies whose total exceeds the host's last
 * level cache make every call stream its weights from DRAM, as a decode step
 * streaming gigabytes of distinct weights does. */
static double time_pooled(const pool_job *job, const uint8_t *const *copies, int n_copies, int threads, int reps) {
    orc_pool_start(threads);
    cpu_set_t saved;
    const int have_saved = sched_getaffinity(0, sizeof saved, &saved) == 0;
    if (P.cpus[0] >= 0) pin(P.cpus[0]);
    double best = 1e30;
    pool_job j = *job;
    for (int r = 0; r < reps; r++) {
        if (copies && n_copies > 0) j.w = copies[r % n_copies];
        const double t0 = now_s();
        pool_run(&j);
        const double dt = now_s() - t0;
        if (dt < best) best = dt;
    }
    if (have_saved) sched_setaffinity(0, sizeof saved, &saved);
    return best;
}

/* The production sweep of one GEMV split over the pool (zlm's matvec job),
 * rotating over n_copies weight copies of w_len bytes each. */
double orc_fast_time_matvec_copies(uint32_t t, const uint8_t *const *ws, int n_copies, size_t w_len, size_t k,
                                   size_t rows, const float *x, float *out, int threads, int reps, int lanes) {
    if (!ws || n_copies < 1) return -1.0;
    const pool_job job = {0, t, ws[0], w_len, k, rows, 1, x, out, pick_lanes(lanes)};
    if (!job.lanes) return -1.0;
    return time_pooled(&job, ws, n_copies, threads, reps);
}

double orc_fast_time_matvec(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, const float *x,
                            float *out, int threads, int reps, int lanes) {
    return orc_fast_time_matvec_copies(t, &w, 1, w_len, k, rows, x, out, threads, reps, lanes);
}

/* The int path over m tokens (each worker its row range for every token). */
double orc_fast_time_matmul_int(uint32_t t, const uint8_t *w, size_t w_len, size_t k, size_t rows, size_t m,
                                const float *x, float *out, int threads, int reps, int lanes) {
    const pool_job job = {1, t, w, w_len, k, rows, m, x, out, pick_lanes(lanes)};
    if (!job.lanes || (t != ORC_Q4_0 && t != ORC_Q8_0)) return -1.0;
    return time_pooled(&job, NULL, 0, threads, reps);
}

/* The threads a started pool runs (0 before the first timed call). */
int orc_pool_threads(void) { return P.started ? P.helpers + 1 : 0; }
