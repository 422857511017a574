/*
 * Seeded, platform-independent input generators (counter-based: element i
 * depends only on (seed, i), so any thread split gives the same bits).  The
 * reference fills inputs with glibc rand() inside OpenMP loops
 * (src/rpl_core.c:88-93), which is neither portable nor reproducible, so
 * tests and benchmarks use these instead.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <unistd.h>

#include "rpl.h"

/* Static-partition parallel loop over [0, n) on plain pthreads (the library
 * carries no OpenMP runtime of its own). */
typedef void (*range_fn)(uint64_t lo, uint64_t hi, void* ctx);
typedef struct {
    range_fn fn;
    void* ctx;
    uint64_t lo, hi;
} RangeJob;

static void* range_thread(void* p) {
    RangeJob* j = (RangeJob*)p;
    j->fn(j->lo, j->hi, j->ctx);
    return NULL;
}

static void parallel_range(uint64_t n, range_fn fn, void* ctx) {
    long nt = sysconf(_SC_NPROCESSORS_ONLN);
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    if (n < (1u << 16)) nt = 1;
    pthread_t th[64];
    RangeJob jobs[64];
    int started[64] = {0};
    for (long t = 0; t < nt; t++) {
        jobs[t].fn = fn;
        jobs[t].ctx = ctx;
        jobs[t].lo = n * t / nt;
        jobs[t].hi = n * (t + 1) / nt;
        if (t > 0) started[t] = pthread_create(&th[t], NULL, range_thread, &jobs[t]) == 0;
    }
    fn(jobs[0].lo, jobs[0].hi, ctx);
    for (long t = 1; t < nt; t++) {
        if (started[t])
            pthread_join(th[t], NULL);
        else
            fn(jobs[t].lo, jobs[t].hi, ctx);
    }
}

static inline uint64_t splitmix64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Top 24 bits -> [0, 1) with a 2^-24 step (exact in float). */
static inline double u24(uint64_t x) { return (double)(x >> 40) * (1.0 / 16777216.0); }

typedef struct {
    float* out;
    uint32_t* labels;
    uint64_t seed;
    double a, b; /* uniform: lo, hi - lo; normal: mean, std */
    uint32_t classes;
} FillCtx;

static void uniform_range(uint64_t lo, uint64_t hi, void* p) {
    FillCtx* c = (FillCtx*)p;
    for (uint64_t i = lo; i < hi; i++) c->out[i] = (float)(c->a + c->b * u24(splitmix64(c->seed, i)));
}

static void normal_range(uint64_t lo, uint64_t hi, void* p) {
    FillCtx* c = (FillCtx*)p;
    for (uint64_t i = lo; i < hi; i++) {
        /* u1 in (0, 1] from 53 bits, u2 in [0, 1). */
        double u1 = ((double)(splitmix64(c->seed, 2 * i) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix64(c->seed, 2 * i + 1) >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        c->out[i] = (float)(c->a + c->b * z);
    }
}

static void labels_range(uint64_t lo, uint64_t hi, void* p) {
    FillCtx* c = (FillCtx*)p;
    for (uint64_t i = lo; i < hi; i++) {
        uint32_t k = (uint32_t)((splitmix64(c->seed, i) >> 32) % c->classes);
        if (c->labels) c->labels[i] = k;
        if (c->out)
            for (uint32_t j = 0; j < c->classes; j++) c->out[i * c->classes + j] = (j == k) ? 1.0f : 0.0f;
    }
}

void rpl_fill_uniform(float* out, uint64_t n, uint64_t seed, float lo, float hi) {
    FillCtx c = {out, NULL, seed, (double)lo, (double)hi - (double)lo, 0};
    parallel_range(n, uniform_range, &c);
}

void rpl_fill_normal(float* out, uint64_t n, uint64_t seed, float mean, float std) {
    FillCtx c = {out, NULL, seed, (double)mean, (double)std, 0};
    parallel_range(n, normal_range, &c);
}

void rpl_fill_labels(uint32_t* labels, float* one_hot, uint64_t n, uint64_t seed, uint32_t classes) {
    if (classes == 0) return;
    FillCtx c = {one_hot, labels, seed, 0.0, 0.0, classes};
    parallel_range(n, labels_range, &c);
}
