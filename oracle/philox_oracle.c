/*
 * CPU oracle for the Philox noise path.  TEST INFRASTRUCTURE ONLY: this file
 * is compiled into oracle/libltx_oracle.so, which only tests/, the smoke check
 * and bench.py's CPU-baseline leg load.  The product path never links it.
 *
 * Restates, in plain scalar C:
 *   - Philox4x32-10 (Salmon et al., "Parallel Random Numbers: As Easy as
 *     1, 2, 3", SC'11; the Random123 round function and Weyl key schedule).
 *   - The counter/offset/thread layout of the reference's torch-compatible
 *     randn: cuda_c_standalone/common/philox.cu:19-35 (element li =
 *     linear_index + T*ii, one Philox block per grid-stride iteration per
 *     thread, subsequence = thread id, counter = offset/4 + iteration) and the
 *     offset advance of philox.cu:6-17,47-61 (4*ceil(n/(4T))).
 *   - The Box-Muller transform in the form published by rocRAND
 *     (rocrand_normal.h, box_muller): u = 2^-32 + x*2^-32,
 *     v = 2pi*2^-32 + y*2pi*2^-32, both in fp32, then
 *     (sqrt(-2 ln u) sin v, sqrt(-2 ln u) cos v).  The oracle evaluates the
 *     transcendental part in fp64 and rounds once to fp32, so it is the
 *     correctly-rounded value of that formula at the fp32 (u, v).
 *
 * Pinned by: the Random123 known-answer vectors, rocRAND's host-callable
 * philox4x32_10 engine (vectors committed under tests/golden/), and the
 * reference's bf16 golden noise (cuda_c_standalone/artifacts/m1_philox/).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define PHILOX_M0 0xD2511F53u
#define PHILOX_M1 0xCD9E8D57u
#define PHILOX_W0 0x9E3779B9u
#define PHILOX_W1 0xBB67AE85u

/* Philox4x32-10 on one 128-bit counter block. ctr[4] in, out[4] out. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += PHILOX_W0;
            k1 += PHILOX_W1;
        }
        uint64_t p0 = (uint64_t)PHILOX_M0 * c0;
        uint64_t p1 = (uint64_t)PHILOX_M1 * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* The block for (seed, subsequence tid, block index blk). */
static void block_for(uint64_t seed, uint64_t tid, uint64_t blk, uint32_t out[4])
{
    uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), (uint32_t)tid, (uint32_t)(tid >> 32)};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    oracle_philox4x32_10(ctr, key, out);
}

/* 4*ceil(n/(4T)): the offset advance after drawing n values with T threads. */
int64_t oracle_offset_advance(int64_t n, int64_t total_threads)
{
    if (n <= 0) return 0;
    return ((n - 1) / (total_threads * 4) + 1) * 4;
}

/* The thread count torch's grid-stride policy picks (philox.cu:6-17). */
int64_t oracle_policy_threads(int64_t n, int64_t multiprocessors, int64_t max_threads_per_mp)
{
    int64_t block = 256;
    int64_t grid = (n + block - 1) / block;
    int64_t cap = multiprocessors * (max_threads_per_mp / block);
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    return grid * block;
}

/* Raw uint32 stream in element order: out[e] = lane (e/T)%4 of the block of
 * thread e%T at iteration e/(4T).  Elements [first, first+count). */
void oracle_philox_u32(uint32_t *out, int64_t first, int64_t count, uint64_t seed, uint64_t offset,
                       int64_t total_threads)
{
    const int64_t T = total_threads;
    for (int64_t i = 0; i < count; ++i) {
        int64_t e = first + i;
        int64_t iter = e / (4 * T);
        int64_t r = e - iter * 4 * T;
        int64_t lane = r / T;
        int64_t tid = r - lane * T;
        uint32_t b[4];
        block_for(seed, (uint64_t)tid, offset / 4 + (uint64_t)iter, b);
        out[i] = b[lane];
    }
}

/* Box-Muller pair from two uint32 draws: fp32 (u, v) per the published
 * formula, transcendental part in fp64, one rounding to fp32. */
static void box_muller_ref(uint32_t x, uint32_t y, float *s_sin, float *s_cos)
{
    const float inv32 = 2.3283064e-10f;    /* 2^-32 */
    const float inv32_2pi = 1.46291807e-09f; /* 2pi * 2^-32 */
    volatile float xf = (float)x;           /* uint32 -> fp32, RNE */
    volatile float yf = (float)y;
    volatile float um = xf * inv32;          /* separate fp32 mul and add */
    volatile float vm = yf * inv32_2pi;
    float u = inv32 + um;
    float v = inv32_2pi + vm;
    double s = sqrt(-2.0 * log((double)u));
    *s_sin = (float)(s * sin((double)v));
    *s_cos = (float)(s * cos((double)v));
}

/* Exposed for tests: the fp32 (u, v) pair the formula produces. */
void oracle_box_muller_uv(uint32_t x, uint32_t y, float *u, float *v)
{
    const float inv32 = 2.3283064e-10f;
    const float inv32_2pi = 1.46291807e-09f;
    volatile float xf = (float)x, yf = (float)y;
    volatile float um = xf * inv32, vm = yf * inv32_2pi;
    *u = inv32 + um;
    *v = inv32_2pi + vm;
}

/* N(0,1) values in element order (fp32), elements [first, first+count). */
void oracle_philox_normal(float *out, int64_t first, int64_t count, uint64_t seed, uint64_t offset,
                          int64_t total_threads)
{
    const int64_t T = total_threads;
    int64_t i = 0;
    while (i < count) {
        int64_t e = first + i;
        int64_t iter = e / (4 * T);
        int64_t r = e - iter * 4 * T;
        int64_t lane = r / T;
        int64_t tid = r - lane * T;
        uint32_t b[4];
        block_for(seed, (uint64_t)tid, offset / 4 + (uint64_t)iter, b);
        float n[4];
        box_muller_ref(b[0], b[1], &n[0], &n[1]);
        box_muller_ref(b[2], b[3], &n[2], &n[3]);
        out[i] = n[lane];
        ++i;
    }
}

/* Same stream, blocked by Philox block instead of by element: computes every
 * block once and scatters its 4 values.  out has n elements; used for whole
 * tensors (each block is evaluated once instead of four times). */
void oracle_philox_normal_full(float *out, int64_t n, uint64_t seed, uint64_t offset, int64_t total_threads)
{
    const int64_t T = total_threads;
    const int64_t iters = n > 0 ? (n - 1) / (4 * T) + 1 : 0;
    for (int64_t it = 0; it < iters; ++it) {
        for (int64_t tid = 0; tid < T; ++tid) {
            int64_t base = it * 4 * T + tid;
            if (base >= n) break;
            uint32_t b[4];
            block_for(seed, (uint64_t)tid, offset / 4 + (uint64_t)it, b);
            float v[4];
            box_muller_ref(b[0], b[1], &v[0], &v[1]);
            box_muller_ref(b[2], b[3], &v[2], &v[3]);
            for (int l = 0; l < 4; ++l) {
                int64_t e = base + (int64_t)l * T;
                if (e < n) out[e] = v[l];
            }
        }
    }
}

/* fp32 -> bf16 bits, round to nearest even (NaN kept quiet). */
static uint16_t f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void oracle_f32_to_bf16(const float *in, uint16_t *out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}

/* Euler update x <- x + dt*v in fp32 with the product rounded before the add
 * (the reference evaluates `x + v*dt` as two tensor ops). */
void oracle_euler_update_f32(float *x, const float *v, int64_t n, float dt)
{
    for (int64_t i = 0; i < n; ++i) {
        volatile float p = v[i] * dt;
        x[i] = x[i] + p;
    }
}
