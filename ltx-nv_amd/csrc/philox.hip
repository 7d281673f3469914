// Philox4x32-10 Gaussian noise in the reference's counter/offset layout.
//
// Layout (cuda_c_standalone/common/philox.cu:19-35): a launch of T logical
// threads; logical thread `tid` draws Philox blocks with key = seed and
// counter = (offset/4 + iter, tid) for iter = 0, 1, ...; block `iter` of
// thread `tid` fills elements iter*4T + lane*T + tid for lane 0..3.  The
// physical launch here is free: each hardware thread evaluates G consecutive
// logical threads of one iteration, so each of its four lanes lands in G
// consecutive elements and is written with one 16-byte (fp32) or 8/16-byte
// (bf16) store.  Output is a pure function of (seed, offset, T, n).
//
// Philox4x32-10: Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As
// Easy as 1, 2, 3" (SC'11).  Box-Muller in rocRAND's published form
// (rocrand_normal.h box_muller): u = 2^-32 + x*2^-32 and
// v = 2pi*2^-32 + y*2pi*2^-32 in fp32, pair (s*sin v, s*cos v),
// s = sqrt(-2 ln u).
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr uint32_t kM0 = 0xD2511F53u;
constexpr uint32_t kM1 = 0xCD9E8D57u;
constexpr uint32_t kW0 = 0x9E3779B9u;
constexpr uint32_t kW1 = 0xBB67AE85u;

struct Block4 {
    uint32_t v[4];
};

__device__ __forceinline__ Block4 philox10(uint64_t blk, uint64_t tid, uint32_t k0, uint32_t k1)
{
    uint32_t c0 = static_cast<uint32_t>(blk), c1 = static_cast<uint32_t>(blk >> 32);
    uint32_t c2 = static_cast<uint32_t>(tid), c3 = static_cast<uint32_t>(tid >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(kM0) * c0;
        const uint64_t p1 = static_cast<uint64_t>(kM1) * c2;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(p1);
        c3 = static_cast<uint32_t>(p0);
        c0 = n0;
        c2 = n2;
        k0 += kW0;
        k1 += kW1;
    }
    return Block4{{c0, c1, c2, c3}};
}

// The transcendental part is evaluated in fp64 from the fp32 (u, v) and
// rounded once, so each normal is within 1 ulp fp32 of the formula's value
// (the product of three separately rounded fp32 functions reached 3 ulp).
// That needs the fp64 factors to about 2^-28 relative, not fp64's 2^-53, and
// the argument ranges are known (u in [2^-32, 1], v in (0, 2pi]), so the fp64
// functions are reduced-range forms sized for that (fp64 FMAs issue at the
// unpacked fp32 rate on this part: the cost is the operation count):
//
//   ln u = e ln2 + ln m,  u = m 2^e, m in [1/sqrt2, sqrt2) from u's bits;
//          ln m = 2 atanh f = 2 (f + f^3/3 + ... + f^11/11), f = (m-1)/(m+1)
//          (hardware reciprocal, measured within 2^-24.4, + one Newton step),
//          |f| <= 0.1716: truncation below 2e-10 relative;
//   sqrt   x * rsqrt(x) (hardware seed, measured within 2^-24, + one Newton
//          step);
//   sin v, cos v: k = rint(v 2/pi) in 0..4, r = v - k pi/2 with pi/2 split in
//          three parts (the first two of 33 bits, so k times them is exact),
//          |r| <= pi/4; Taylor series to r^11 (sin) and r^10 (cos),
//          truncation below 1e-10; the quadrant k mod 4 swaps and negates.
//
// On the host (same operations, seeds perturbed by 2^-22) 0.005 % of 237 M
// normals differ from the correctly rounded formula, by 1 ulp.
__device__ __forceinline__ double log_unit(float u)
{
    constexpr double kLn2Hi = 0x1.62e42fefa2000p-1;  // 40 bits: e * kLn2Hi is exact
    constexpr double kLn2Lo = 0x1.9ef35793c7673p-41;
    const uint32_t bits = __float_as_uint(u);  // u >= 2^-32: normal, positive
    const uint32_t man = bits & 0x7fffffu;
    const bool hi = man > 0x3504f3u;  // m > sqrt2: halve it
    const int e = static_cast<int>(bits >> 23) - 127 + (hi ? 1 : 0);
    const double m = static_cast<double>(__uint_as_float(man | (hi ? 0x3f000000u : 0x3f800000u)));
    const double den = m + 1.0;
    double rc = __builtin_amdgcn_rcp(den);
    rc = __builtin_fma(__builtin_fma(-den, rc, 1.0), rc, rc);
    const double f = (m - 1.0) * rc;
    const double f2 = f * f;
    double p = 1.0 / 11.0;
    p = __builtin_fma(p, f2, 1.0 / 9.0);
    p = __builtin_fma(p, f2, 1.0 / 7.0);
    p = __builtin_fma(p, f2, 1.0 / 5.0);
    p = __builtin_fma(p, f2, 1.0 / 3.0);
    const double f_2 = 2.0 * f;
    const double ln_m = __builtin_fma(f_2 * f2, p, f_2);
    const double de = static_cast<double>(e);
    return __builtin_fma(de, kLn2Hi, __builtin_fma(de, kLn2Lo, ln_m));
}

// sqrt(x) for x >= 0 (x = 0 when u = 1).
__device__ __forceinline__ double sqrt_nonneg(double x)
{
    const double h = 0.5 * x;
    double y = __builtin_amdgcn_rsq(x > 0.0 ? x : 1.0);
    y = y * __builtin_fma(-h * y, y, 1.5);
    return x > 0.0 ? x * y : 0.0;
}

__device__ __forceinline__ void sincos_angle(float v, double &sn, double &cs)
{
    constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
    constexpr double kP1 = 0x1.921fb54400000p+0;  // pi/2 = kP1 + kP2 + kP3
    constexpr double kP2 = 0x1.0b4611a600000p-34;
    constexpr double kP3 = 0x1.3198a2e037073p-69;
    const double x = static_cast<double>(v);
    const double k = __builtin_rint(x * kTwoOverPi);
    double r = __builtin_fma(-k, kP1, x);
    r = __builtin_fma(-k, kP2, r);
    r = __builtin_fma(-k, kP3, r);
    const double r2 = r * r;
    double ps = -1.0 / 39916800.0;  // -1/11!
    ps = __builtin_fma(ps, r2, 1.0 / 362880.0);
    ps = __builtin_fma(ps, r2, -1.0 / 5040.0);
    ps = __builtin_fma(ps, r2, 1.0 / 120.0);
    ps = __builtin_fma(ps, r2, -1.0 / 6.0);
    const double s = __builtin_fma(r * r2, ps, r);
    double pc = -1.0 / 3628800.0;  // -1/10!
    pc = __builtin_fma(pc, r2, 1.0 / 40320.0);
    pc = __builtin_fma(pc, r2, -1.0 / 720.0);
    pc = __builtin_fma(pc, r2, 1.0 / 24.0);
    pc = __builtin_fma(pc, r2, -0.5);
    const double c = __builtin_fma(r2, pc, 1.0);
    const int q = static_cast<int>(k) & 3;
    const double s1 = (q & 1) ? c : s;
    const double c1 = (q & 1) ? s : c;
    sn = (q & 2) ? -s1 : s1;
    cs = ((q + 1) & 2) ? -c1 : c1;
}

__device__ __forceinline__ void box_muller(uint32_t x, uint32_t y, float &a, float &b)
{
    const float inv32 = 2.3283064e-10f;      // 2^-32
    const float inv32_2pi = 1.46291807e-09f;  // 2pi * 2^-32
    // Separate fp32 multiply and add (the TU is built without contraction).
    const float u = inv32 + static_cast<float>(x) * inv32;
    const float v = inv32_2pi + static_cast<float>(y) * inv32_2pi;
    const double s = sqrt_nonneg(-2.0 * log_unit(u));
    double sn, cs;
    sincos_angle(v, sn, cs);
    a = static_cast<float>(s * sn);
    b = static_cast<float>(s * cs);
}

template <typename Out>
struct Store;

template <>
struct Store<float> {
    static constexpr int G = 4;  // logical threads per hardware thread
    __device__ static void vec(float *p, const float v[G])
    {
        st16f_stream(p, v[0], v[1], v[2], v[3]);
    }
    __device__ static void one(float *p, float v) { *p = v; }
};

template <>
struct Store<uint16_t> {
    static constexpr int G = 8;
    __device__ static void vec(uint16_t *p, const float v[G]) { st16_stream(p, pack8(v)); }
    __device__ static void one(uint16_t *p, float v) { *p = f32_to_bf16(v); }
};

// Vector path: T % G == 0.  Hardware thread p covers logical threads
// [G*q, G*q + G) of iteration it, with (it, q) = divmod(p, T/G).
template <typename Out>
__global__ void __launch_bounds__(256) philox_normal_vec(Out *__restrict__ out, int64_t n, uint32_t k0, uint32_t k1,
                                                         uint64_t blk0, int64_t T, int64_t quads_per_iter,
                                                         int64_t total_quads)
{
    constexpr int G = Store<Out>::G;
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= total_quads) return;
    const int64_t it = p / quads_per_iter;
    const int64_t tid0 = (p - it * quads_per_iter) * G;
    float vals[4][G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid0 + g), k0, k1);
        box_muller(r.v[0], r.v[1], vals[0][g], vals[1][g]);
        box_muller(r.v[2], r.v[3], vals[2][g], vals[3][g]);
    }
    const int64_t base = it * 4 * T + tid0;
#pragma unroll
    for (int lane = 0; lane < 4; ++lane) {
        const int64_t e = base + lane * T;
        if (e + G <= n) {
            Store<Out>::vec(out + e, vals[lane]);
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g)
                if (e + g < n) Store<Out>::one(out + e + g, vals[lane][g]);
        }
    }
}

// General path (any T): one logical thread per hardware thread.
template <typename Out>
__global__ void __launch_bounds__(256) philox_normal_any(Out *__restrict__ out, int64_t n, uint32_t k0, uint32_t k1,
                                                         uint64_t blk0, int64_t T, int64_t total)
{
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= total) return;
    const int64_t it = p / T;
    const int64_t tid = p - it * T;
    const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid), k0, k1);
    float v[4];
    box_muller(r.v[0], r.v[1], v[0], v[1]);
    box_muller(r.v[2], r.v[3], v[2], v[3]);
#pragma unroll
    for (int lane = 0; lane < 4; ++lane) {
        const int64_t e = it * 4 * T + lane * T + tid;
        if (e < n) Store<Out>::one(out + e, v[lane]);
    }
}

__global__ void __launch_bounds__(256) philox_u32_kernel(uint32_t *__restrict__ out, int64_t n, uint32_t k0,
                                                         uint32_t k1, uint64_t blk0, int64_t T, int64_t total)
{
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= total) return;
    const int64_t it = p / T;
    const int64_t tid = p - it * T;
    const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid), k0, k1);
#pragma unroll
    for (int lane = 0; lane < 4; ++lane) {
        const int64_t e = it * 4 * T + lane * T + tid;
        if (e < n) out[e] = r.v[lane];
    }
}

int check_common(const void *out, int64_t n, uint64_t offset, int64_t T, const char *what)
{
    if (n < 0) return fail(LTXK_E_ARG, "%s: n must be >= 0 (got %lld)", what, (long long)n);
    if (n > 0 && !out) return fail(LTXK_E_ARG, "%s: null output", what);
    if (T <= 0) return fail(LTXK_E_ARG, "%s: total_threads must be > 0 (got %lld)", what, (long long)T);
    if (offset % 4 != 0)
        return fail(LTXK_E_ARG, "%s: offset must be a multiple of 4 (got %llu)", what, (unsigned long long)offset);
    return LTXK_OK;
}

int64_t iterations(int64_t n, int64_t T) { return n > 0 ? (n - 1) / (4 * T) + 1 : 0; }

template <typename Out>
int launch_normal(Out *out, int64_t n, uint64_t seed, uint64_t offset, int64_t T, hipStream_t stream)
{
    constexpr int G = Store<Out>::G;
    const uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
    const int64_t iters = iterations(n, T);
    const uint64_t blk0 = offset / 4;
    if (T % G == 0 && aligned16(out)) {
        const int64_t qpi = T / G;
        const int64_t total = qpi * iters;
        const int64_t grid = (total + 255) / 256;
        if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "philox_normal: launch too large");
        philox_normal_vec<Out><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream>>>(out, n, k0, k1, blk0, T,
                                                                                          qpi, total);
    } else {
        const int64_t total = T * iters;
        const int64_t grid = (total + 255) / 256;
        if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "philox_normal: launch too large");
        philox_normal_any<Out><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream>>>(out, n, k0, k1, blk0, T,
                                                                                          total);
    }
    return check_launch("philox_normal");
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int64_t ltxk_philox_policy_threads(int64_t n, int64_t multiprocessors, int64_t max_threads_per_mp)
{
    const int64_t block = 256;
    int64_t grid = (n + block - 1) / block;
    const int64_t cap = multiprocessors * (max_threads_per_mp / block);
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    return grid * block;
}

extern "C" int64_t ltxk_philox_offset_advance(int64_t n, int64_t total_threads)
{
    if (n <= 0 || total_threads <= 0) return 0;
    return iterations(n, total_threads) * 4;
}

extern "C" int ltxk_philox_normal(void *out, int dtype, int64_t n, uint64_t seed, uint64_t offset,
                                  int64_t total_threads, void *stream)
{
    clear_error();
    int rc = check_common(out, n, offset, total_threads, "philox_normal");
    if (rc) return rc;
    if (n == 0) return LTXK_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == LTXK_DTYPE_F32) return launch_normal(static_cast<float *>(out), n, seed, offset, total_threads, s);
    if (dtype == LTXK_DTYPE_BF16)
        return launch_normal(static_cast<uint16_t *>(out), n, seed, offset, total_threads, s);
    return fail(LTXK_E_DTYPE, "philox_normal: unsupported dtype %d", dtype);
}

extern "C" int ltxk_philox_u32(uint32_t *out, int64_t n, uint64_t seed, uint64_t offset, int64_t total_threads,
                               void *stream)
{
    clear_error();
    int rc = check_common(out, n, offset, total_threads, "philox_u32");
    if (rc) return rc;
    if (n == 0) return LTXK_OK;
    const int64_t total = total_threads * iterations(n, total_threads);
    const int64_t grid = (total + 255) / 256;
    if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "philox_u32: launch too large");
    philox_u32_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
        out, n, static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32), offset / 4, total_threads, total);
    return check_launch("philox_u32");
}
