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

#include "philox_tables.h"

constexpr uint32_t kM0 = 0xD2511F53u;
constexpr uint32_t kM1 = 0xCD9E8D57u;
constexpr uint32_t kW0 = 0x9E3779B9u;
constexpr uint32_t kW1 = 0xBB67AE85u;

struct Block4 {
    uint32_t v[4];
};

// a ^ b ^ c in one instruction: gfx950's three-input bitwise op with the
// truth table of odd parity (bit i of 0x96 is set when i has an odd number of
// ones), in place of two v_xor_b32.
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c)
{
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ Block4 philox10(uint64_t blk, uint64_t tid, uint32_t k0, uint32_t k1)
{
    uint32_t c0 = static_cast<uint32_t>(blk), c1 = static_cast<uint32_t>(blk >> 32);
    uint32_t c2 = static_cast<uint32_t>(tid), c3 = static_cast<uint32_t>(tid >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(kM0) * c0;
        const uint64_t p1 = static_cast<uint64_t>(kM1) * c2;
        const uint32_t n0 = xor3(static_cast<uint32_t>(p1 >> 32), c1, k0);
        const uint32_t n2 = xor3(static_cast<uint32_t>(p0 >> 32), c3, k1);
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
// functions are table-driven reduced-range forms sized for that (fp64 FMAs
// issue at the unpacked fp32 rate on this part: the cost is the operation
// count; the tables, philox_tables.h, sit in LDS):
//
//   ln u = e ln2 + ln c_i + ln(1 + r),  u = m 2^e from u's bits, bin i = the
//          top 7 bits of m's fraction, r = m/c_i - 1 (one FMA with the
//          table's 1/c_i), |r| < 2^-7; ln(1+r) to r^4 (truncation below
//          2e-10 relative).  Bins of m above 1 + 53/128 use the next binade
//          (e + 1, c_i/2 in [0.707, 1)) centred on their upper edge, so as u
//          -> 1 the table term is 0 and ln u = ln(1 + r) loses nothing; u = 1
//          gives exactly 0;
//   sqrt   x * rsqrt(x) (hardware seed, measured within 2^-24, + one Newton
//          step);
//   sin v, cos v: k = rint(v 32/pi) in 0..64, r = v - k pi/32 with pi/32
//          split in three parts (the first two of 45 and 46 bits, so k times
//          them is exact), |r| <= pi/64; sin r to r^5, cos r to r^4
//          (truncation below 3e-11 relative), then the angle sum with the
//          table's sin and cos of k pi/32 (exact zeros and ones where the
//          angle has them, so sin v near pi and 2pi and cos v near pi/2 and
//          3pi/2 keep their relative accuracy).
//
// On the host (the same operations from the same tables, the rsqrt seed
// perturbed by 2^-22) 0.0034 % of 200 M normals differ from the correctly
// rounded formula, by 1 ulp (the previous series forms: 0.005 %).
struct BoxMullerTabs {
    double2 log[128];    // {1/c_i, ln c_i or ln(c_i/2)}
    double2 sincos[64];  // {sin, cos} of k pi/32
};

__device__ __forceinline__ double log_unit(float u, const BoxMullerTabs &tb)
{
    constexpr double kLn2Hi = 0x1.62e42fefa3a00p-1;  // 44 bits: e * kLn2Hi is exact for |e| <= 64
    constexpr double kLn2Lo = -0x1.0ca86c3898d00p-49;
    const uint32_t bits = __float_as_uint(u);  // u >= 2^-32: normal, positive
    const uint32_t man = bits & 0x7fffffu;
    const int i = static_cast<int>(man >> 16);
    const int e = static_cast<int>(bits >> 23) - 127 + (i >= kLogHi ? 1 : 0);
    const double m = static_cast<double>(__uint_as_float(man | 0x3f800000u));  // in [1, 2)
    const double2 t = tb.log[i];
    const double r = __builtin_fma(m, t.x, -1.0);
    double p = __builtin_fma(r, -0.25, 1.0 / 3.0);
    p = __builtin_fma(p, r, -0.5);
    p = __builtin_fma(p, r, 1.0);
    const double de = static_cast<double>(e);
    return __builtin_fma(de, kLn2Hi, __builtin_fma(de, kLn2Lo, __builtin_fma(r, p, t.y)));
}

// sqrt(x) for x >= 0 (x = 0 when u = 1).  The seed is taken at max(x,
// 2^-1000), finite for every x, so x = 0 gives 0 * finite = 0 with no
// select (the same values as guarding both ends with x > 0).
__device__ __forceinline__ double sqrt_nonneg(double x)
{
    const double h = 0.5 * x;
    double y = __builtin_amdgcn_rsq(__builtin_fmax(x, 0x1p-1000));
    y = y * __builtin_fma(-h * y, y, 1.5);
    return x * y;
}

__device__ __forceinline__ void sincos_angle(float v, const BoxMullerTabs &tb, double &sn, double &cs)
{
    constexpr double k32OverPi = 0x1.45f306dc9c883p+3;
    constexpr double kP1 = 0x1.921fb54442d00p-4;  // pi/32 = kP1 + kP2 + kP3
    constexpr double kP2 = 0x1.8469898cc5180p-52;
    constexpr double kP3 = -0x1.fc8f8cbb5bf6cp-101;
    const double x = static_cast<double>(v);
    const double k = __builtin_rint(x * k32OverPi);
    double r = __builtin_fma(-k, kP1, x);
    r = __builtin_fma(-k, kP2, r);
    r = __builtin_fma(-k, kP3, r);
    const double2 t = tb.sincos[static_cast<int>(k) & 63];
    const double r2 = r * r;
    const double sr = __builtin_fma(r * r2, __builtin_fma(r2, 1.0 / 120.0, -1.0 / 6.0), r);
    const double cr = __builtin_fma(r2, __builtin_fma(r2, 1.0 / 24.0, -0.5), 1.0);
    sn = __builtin_fma(t.x, cr, t.y * sr);
    cs = __builtin_fma(t.y, cr, -(t.x * sr));
}

__device__ __forceinline__ void box_muller(uint32_t x, uint32_t y, const BoxMullerTabs &tb, float &a, float &b)
{
    const float inv32 = 2.3283064e-10f;      // 2^-32
    const float inv32_2pi = 1.46291807e-09f;  // 2pi * 2^-32
    // Separate fp32 multiply and add (the TU is built without contraction).
    const float u = inv32 + static_cast<float>(x) * inv32;
    const float v = inv32_2pi + static_cast<float>(y) * inv32_2pi;
    const double s = sqrt_nonneg(-2.0 * log_unit(u, tb));
    double sn, cs;
    sincos_angle(v, tb, sn, cs);
    a = static_cast<float>(s * sn);
    b = static_cast<float>(s * cs);
}

// The tables into the workgroup's LDS (every thread of the workgroup calls it
// before any returns: it ends with a barrier).
__device__ __forceinline__ void load_tabs(BoxMullerTabs &tb)
{
    for (int i = threadIdx.x; i < 128 + 64; i += blockDim.x) {
        if (i < 128)
            tb.log[i] = double2{kLogTab[i][0], kLogTab[i][1]};
        else
            tb.sincos[i - 128] = double2{kSinCosTab[i - 128][0], kSinCosTab[i - 128][1]};
    }
    __syncthreads();
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
    __shared__ BoxMullerTabs tb;
    load_tabs(tb);
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= total_quads) return;
    const int64_t it = p / quads_per_iter;
    const int64_t tid0 = (p - it * quads_per_iter) * G;
    const int64_t base = it * 4 * T + tid0;
    // a Box-Muller pair whose two lanes land past the tensor is not evaluated
    // (with T above n/4 lanes 2 and 3 of every item do: the thread policy's
    // T = 524288 for 786432 values); no value of it is stored
    // (the branch is outside the unrolled loop, so either body keeps its G
    // independent chains interleaved)
    float vals[4][G] = {};
    if (base + 2 * T < n) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid0 + g), k0, k1);
            box_muller(r.v[0], r.v[1], tb, vals[0][g], vals[1][g]);
            box_muller(r.v[2], r.v[3], tb, vals[2][g], vals[3][g]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid0 + g), k0, k1);
            box_muller(r.v[0], r.v[1], tb, vals[0][g], vals[1][g]);
        }
    }
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
    __shared__ BoxMullerTabs tb;
    load_tabs(tb);
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= total) return;
    const int64_t it = p / T;
    const int64_t tid = p - it * T;
    const Block4 r = philox10(blk0 + static_cast<uint64_t>(it), static_cast<uint64_t>(tid), k0, k1);
    float v[4] = {};
    box_muller(r.v[0], r.v[1], tb, v[0], v[1]);
    if (it * 4 * T + 2 * T + tid < n) box_muller(r.v[2], r.v[3], tb, v[2], v[3]);  // lanes 2, 3 in the tensor
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
