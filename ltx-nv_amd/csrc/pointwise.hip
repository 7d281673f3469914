// Flat elementwise kernels: GELU-tanh and the flow-matching Euler updates.
// Each thread streams kChunks 16-byte vectors through the workgroup's buffer
// range (streamed loads and streamed stores); the last partial vector of the
// tensor is handled element by element by the thread that owns it.  Streamed
// (nt) stores instead of write-through: GELU on [6144, 16384] 62.1 us either
// way alone, but the 48-block chain, where the FFN's GELU runs beside the
// audio stream's kernels, 16.72-16.74 against 16.92-16.99 ms (graph replays
// 16.49-16.57 against 16.78-16.86) and the full denoise step unchanged within
// its run-to-run spread.  The Euler updates store with nt alone (below).
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kChunks = 2;  // 16-byte vectors per thread
constexpr int kEulerStore = 2;  // aux cache-policy bits of the Euler updates' stores: nt

// gelu_tanh(x) = 0.5 x (1 + tanh(y)), y = sqrt(2/pi) (x + 0.044715 x^3),
// evaluated as x * sigmoid(2y) = x / (1 + 2^(-2y log2 e)), the same function
// written with one exp2 and one reciprocal.
__device__ __forceinline__ float gelu_tanh_f(float x)
{
    constexpr float kBeta = 0.7978845608028654f;  // sqrt(2/pi)
    constexpr float kKappa = 0.044715f;
    constexpr float kC1 = -2.0f * 1.4426950408889634f * kBeta;  // -2 log2(e) sqrt(2/pi)
    constexpr float kC2 = kC1 * kKappa;
    const float x2 = x * x;
    const float q = __builtin_fmaf(kC2, x2, kC1);
    const float e = __builtin_amdgcn_exp2f(x * q);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

template <typename T>
struct Vec;

// 16 bytes of T as a native 4 x u32 vector <-> N floats.
template <>
struct Vec<uint16_t> {
    static constexpr int N = 8;
    __device__ static void unpack(const u32x4 &r, float f[N]) { unpack8v(r, f); }
    __device__ static u32x4 pack(const float f[N]) { return pack8v(f); }
    __device__ static float get(const uint16_t *p) { return bf16_to_f32(*p); }
    __device__ static void put(uint16_t *p, float f) { *p = f32_to_bf16(f); }
    __device__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
};

template <>
struct Vec<float> {
    static constexpr int N = 4;
    __device__ static void unpack(const u32x4 &r, float f[N])
    {
#pragma unroll
        for (int i = 0; i < N; ++i) f[i] = __uint_as_float(r[i]);
    }
    __device__ static u32x4 pack(const float f[N])
    {
        return u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
    }
    __device__ static float get(const float *p) { return *p; }
    __device__ static void put(float *p, float f) { *p = f; }
    __device__ static float round(float f) { return f; }
};

// op 0: y = gelu(a) ; 1: a <- a + dt*b ; 2: y = a + round((a - b)/sigma)*dt
template <int OP, typename T>
struct Op {
    float dt, sigma;
    __device__ float operator()(float a, float b) const
    {
        if (OP == 0) return gelu_tanh_f(a);
        if (OP == 1) return a + b * dt;
        const float vel = Vec<T>::round((a - b) / sigma);
        return a + vel * dt;
    }
};

template <int OP, typename T>
__global__ void __launch_bounds__(kBlock) flat_kernel(T *y, const T *a, const T *b, int64_t n,
                                                      Op<OP, T> op)
{
    constexpr int N = Vec<T>::N;
    constexpr int64_t kPerBlock = static_cast<int64_t>(kBlock) * kChunks;  // 16-byte vectors per workgroup
    const int64_t nvec = n / N;
    // The workgroup's span of whole vectors as one buffer range: vectors past
    // the end read zeros and their stores are dropped, so every load is issued
    // unconditionally before the first use.
    const int64_t v0 = static_cast<int64_t>(blockIdx.x) * kPerBlock;
    const int64_t left = nvec - v0;
    const uint32_t bytes = left <= 0 ? 0u : static_cast<uint32_t>((left < kPerBlock ? left : kPerBlock) * 16);
    const int64_t base = (left > 0 ? v0 : 0) * N;
    const rsrc_t ra = make_rsrc(a + base, bytes);
    const rsrc_t rb = make_rsrc((OP != 0 ? b : a) + base, OP != 0 ? bytes : 0u);
    const rsrc_t ry = make_rsrc(y + base, bytes);
    u32x4 ra_v[kChunks], rb_v[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const uint32_t off = (static_cast<uint32_t>(c) * kBlock + threadIdx.x) * 16u;
        ra_v[c] = ldb(ra, off);
        if (OP != 0) rb_v[c] = ldb(rb, off);
    }
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const uint32_t off = (static_cast<uint32_t>(c) * kBlock + threadIdx.x) * 16u;
        float av[N], bv[N], o[N];
        Vec<T>::unpack(ra_v[c], av);
        if (OP != 0) Vec<T>::unpack(rb_v[c], bv);
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = op(av[i], OP != 0 ? bv[i] : 0.f);
        // GELU: streaming stores (nt | sc1); the Euler updates' outputs are
        // the next step's latents: nt alone (the config-0 update 2.63 us
        // against 3.19 with nt | sc1 and 2.68 written through)
        __builtin_amdgcn_raw_buffer_store_b128(Vec<T>::pack(o), ry, off, 0, OP == 0 ? kStoreStream : kEulerStore);
        // the last partial vector of the tensor, element by element, by the
        // thread that would own vector nvec
        if (v0 + static_cast<int64_t>(c) * kBlock + threadIdx.x == nvec) {
            for (int64_t e = nvec * N; e < n; ++e) {
                const float bv1 = OP != 0 ? Vec<T>::get(b + e) : 0.f;
                Vec<T>::put(y + e, op(Vec<T>::get(a + e), bv1));
            }
        }
    }
}

template <int OP, typename T>
int launch_flat(T *y, const T *a, const T *b, int64_t n, Op<OP, T> op, hipStream_t s, const char *what)
{
    constexpr int N = Vec<T>::N;
    const int64_t nvec = n / N + 1;  // +1: the tail owner
    const int64_t per_block = static_cast<int64_t>(kBlock) * kChunks;
    const int64_t grid = (nvec + per_block - 1) / per_block;
    if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "%s: tensor too large", what);
    flat_kernel<OP, T><<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), 0, s>>>(y, a, b, n, op);
    return check_launch(what);
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int ltxk_gelu_tanh(void *y, const void *x, int64_t n, void *stream)
{
    static const char *what = "gelu_tanh";
    clear_error();
    if (n < 0) return fail(LTXK_E_ARG, "%s: n < 0", what);
    if (n == 0) return LTXK_OK;
    if (!y || !x) return fail(LTXK_E_ARG, "%s: null pointer", what);
    if (!aligned16(y) || !aligned16(x)) return fail(LTXK_E_ALIGN, "%s: buffers must be 16-byte aligned", what);
    Op<0, uint16_t> op{0.f, 1.f};
    return launch_flat<0, uint16_t>(static_cast<uint16_t *>(y), static_cast<const uint16_t *>(x), nullptr, n, op,
                                    static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_euler_update(void *x, const void *v, int64_t n, int dtype, float dt, void *stream)
{
    static const char *what = "euler_update";
    clear_error();
    if (n < 0) return fail(LTXK_E_ARG, "%s: n < 0", what);
    if (n == 0) return LTXK_OK;
    if (!x || !v) return fail(LTXK_E_ARG, "%s: null pointer", what);
    if (!aligned16(x) || !aligned16(v)) return fail(LTXK_E_ALIGN, "%s: buffers must be 16-byte aligned", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == LTXK_DTYPE_F32) {
        Op<1, float> op{dt, 1.f};
        return launch_flat<1, float>(static_cast<float *>(x), static_cast<const float *>(x),
                                     static_cast<const float *>(v), n, op, s, what);
    }
    if (dtype == LTXK_DTYPE_BF16) {
        Op<1, uint16_t> op{dt, 1.f};
        return launch_flat<1, uint16_t>(static_cast<uint16_t *>(x), static_cast<const uint16_t *>(x),
                                        static_cast<const uint16_t *>(v), n, op, s, what);
    }
    return fail(LTXK_E_DTYPE, "%s: unsupported dtype %d", what, dtype);
}

extern "C" int ltxk_euler_step(void *out, const void *sample, const void *denoised, int64_t n, int dtype,
                               float sigma, float dt, void *stream)
{
    static const char *what = "euler_step";
    clear_error();
    if (n < 0) return fail(LTXK_E_ARG, "%s: n < 0", what);
    if (n == 0) return LTXK_OK;
    if (!out || !sample || !denoised) return fail(LTXK_E_ARG, "%s: null pointer", what);
    if (!aligned16(out) || !aligned16(sample) || !aligned16(denoised))
        return fail(LTXK_E_ALIGN, "%s: buffers must be 16-byte aligned", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == LTXK_DTYPE_F32) {
        Op<2, float> op{dt, sigma};
        return launch_flat<2, float>(static_cast<float *>(out), static_cast<const float *>(sample),
                                     static_cast<const float *>(denoised), n, op, s, what);
    }
    if (dtype == LTXK_DTYPE_BF16) {
        Op<2, uint16_t> op{dt, sigma};
        return launch_flat<2, uint16_t>(static_cast<uint16_t *>(out), static_cast<const uint16_t *>(sample),
                                        static_cast<const uint16_t *>(denoised), n, op, s, what);
    }
    return fail(LTXK_E_DTYPE, "%s: unsupported dtype %d", what, dtype);
}
