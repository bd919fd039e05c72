/*
 * inputs.c -- seeded synthetic inputs for the benchmark configurations
 * (libtrs_inputs.so, host only).
 *
 * The reference has no RNG (tensors enter through torch_rs.tensor(buffer),
 * src/python.rs:4139-4170), so the configs are realised with a counter-based
 * generator whose output does not depend on thread count:
 *   Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 *   easy as 1, 2, 3", SC'11), key = {seed, stream}, counter = {block, 0, 0, 0},
 *   four 32-bit words per block;
 *   uniform u = (w >> 8) * 2^-24 in [0, 1);
 *   normal  = Box-Muller on (u1' = ((w0 >> 8) + 1) * 2^-24, u2) in double,
 *             z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), then mean + std*z
 *             rounded once to f32;
 *   keep-mask = (u < keep) as uint8 0/1.
 * Element i uses word i of the stream (normals use words 2j, 2j+1 for the
 * pair j = i/2).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline void mulhilo(uint32_t a, uint32_t b, uint32_t *hi, uint32_t *lo) {
    uint64_t p = (uint64_t)a * b;
    *hi = (uint32_t)(p >> 32);
    *lo = (uint32_t)p;
}

void trs_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; r++) {
        if (r > 0) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint32_t hi0, lo0, hi1, lo1;
        mulhilo(0xD2511F53u, c0, &hi0, &lo0);
        mulhilo(0xCD9E8D57u, c2, &hi1, &lo1);
        uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static inline void block_words(uint64_t seed, uint32_t stream, uint64_t block, uint32_t w[4]) {
    uint32_t ctr[4] = {(uint32_t)block, (uint32_t)(block >> 32), 0u, 0u};
    uint32_t key[2] = {(uint32_t)seed, stream};
    trs_philox4x32_10(ctr, key, w);
}

static inline uint32_t word_at(uint64_t seed, uint32_t stream, uint64_t i) {
    uint32_t w[4];
    block_words(seed, stream, i >> 2, w);
    return w[i & 3];
}

static inline double unit_u(uint32_t w) { return (double)(w >> 8) * (1.0 / 16777216.0); }

enum { KIND_UNIFORM = 0, KIND_NORMAL = 1, KIND_MASK = 2 };

typedef struct {
    int kind;
    uint64_t seed;
    uint32_t stream;
    double a, b;  /* uniform: [a, b); normal: mean a, std b; mask: keep a */
    void *out;
    uint64_t begin, end;
} job_t;

static void run_range(const job_t *j) {
    if (j->kind == KIND_UNIFORM) {
        float *out = (float *)j->out;
        uint64_t i = j->begin;
        while (i < j->end) {
            uint32_t w[4];
            block_words(j->seed, j->stream, i >> 2, w);
            for (uint64_t q = i & 3; q < 4 && i < j->end; q++, i++)
                out[i] = (float)(j->a + (j->b - j->a) * unit_u(w[q]));
        }
    } else if (j->kind == KIND_MASK) {
        uint8_t *out = (uint8_t *)j->out;
        uint64_t i = j->begin;
        while (i < j->end) {
            uint32_t w[4];
            block_words(j->seed, j->stream, i >> 2, w);
            for (uint64_t q = i & 3; q < 4 && i < j->end; q++, i++)
                out[i] = unit_u(w[q]) < j->a ? 1u : 0u;
        }
    } else {
        float *out = (float *)j->out;
        const double two_pi = 6.283185307179586476925286766559;
        for (uint64_t i = j->begin; i < j->end; i++) {
            uint64_t pair = i >> 1;
            uint32_t w0 = word_at(j->seed, j->stream, 2 * pair);
            uint32_t w1 = word_at(j->seed, j->stream, 2 * pair + 1);
            double u1 = (double)((w0 >> 8) + 1u) * (1.0 / 16777216.0);
            double u2 = unit_u(w1);
            double r = sqrt(-2.0 * log(u1));
            double z = (i & 1) ? r * sin(two_pi * u2) : r * cos(two_pi * u2);
            out[i] = (float)(j->a + j->b * z);
        }
    }
}

static void *thread_main(void *arg) {
    run_range((const job_t *)arg);
    return NULL;
}

static int run(int kind, uint64_t seed, uint32_t stream, double a, double b, void *out, uint64_t n,
               int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if ((uint64_t)threads > n / 65536 + 1) threads = (int)(n / 65536 + 1);
    job_t jobs[64];
    pthread_t tids[64];
    uint64_t per = (n + threads - 1) / threads;
    per = (per + 3) & ~(uint64_t)3;
    int launched = 0;
    for (int t = 0; t < threads; t++) {
        jobs[t].kind = kind;
        jobs[t].seed = seed;
        jobs[t].stream = stream;
        jobs[t].a = a;
        jobs[t].b = b;
        jobs[t].out = out;
        jobs[t].begin = (uint64_t)t * per < n ? (uint64_t)t * per : n;
        jobs[t].end = (uint64_t)(t + 1) * per < n ? (uint64_t)(t + 1) * per : n;
    }
    for (int t = 1; t < threads; t++) {
        if (pthread_create(&tids[t], NULL, thread_main, &jobs[t]) != 0) break;
        launched = t;
    }
    run_range(&jobs[0]);
    for (int t = 1; t <= launched; t++) pthread_join(tids[t], NULL);
    for (int t = launched + 1; t < threads; t++) run_range(&jobs[t]);
    return 0;
}

int trs_gen_uniform_f32(uint64_t seed, uint32_t stream, double lo, double hi, float *out, uint64_t n,
                        int threads) {
    return run(KIND_UNIFORM, seed, stream, lo, hi, out, n, threads);
}

int trs_gen_normal_f32(uint64_t seed, uint32_t stream, double mean, double std, float *out, uint64_t n,
                       int threads) {
    return run(KIND_NORMAL, seed, stream, mean, std, out, n, threads);
}

int trs_gen_mask_u8(uint64_t seed, uint32_t stream, double keep, uint8_t *out, uint64_t n, int threads) {
    return run(KIND_MASK, seed, stream, keep, 0.0, out, n, threads);
}
