// Flat elementwise kernels: GELU-tanh and the flow-matching Euler updates.
// Each thread streams CHUNKS 16-byte vectors; the last partial vector of the
// tensor is handled element by element by the thread that owns it.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kChunks = 2;  // 16-byte vectors per thread

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

template <>
struct Vec<uint16_t> {
    static constexpr int N = 8;
    using Raw = uint4;
    __device__ static Raw fetch(const uint16_t *p) { return ld16_stream(p); }
    __device__ static void unpack(const Raw &r, float f[N]) { unpack8(r, f); }
    __device__ static void store(uint16_t *p, const float f[N]) { st16_stream(p, pack8(f)); }
    __device__ static float get(const uint16_t *p) { return bf16_to_f32(*p); }
    __device__ static void put(uint16_t *p, float f) { *p = f32_to_bf16(f); }
    __device__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
};

template <>
struct Vec<float> {
    static constexpr int N = 4;
    using Raw = f32x4;
    __device__ static Raw fetch(const float *p) { return ld16f_stream(p); }
    __device__ static void unpack(const Raw &v, float f[N])
    {
        f[0] = v.x;
        f[1] = v.y;
        f[2] = v.z;
        f[3] = v.w;
    }
    __device__ static void store(float *p, const float f[N])
    {
        st16f_stream(p, f[0], f[1], f[2], f[3]);
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
    const int64_t nvec = n / N;
    const int64_t v0 = (static_cast<int64_t>(blockIdx.x) * kBlock * kChunks) + threadIdx.x;
    // Every vector load is issued before the first use, from a clamped index;
    // only the stores are conditional.  (A condition around a chunk's whole
    // work lets the compiler sink its loads under it, behind a wait for the
    // previous chunk.)
    typename Vec<T>::Raw ra[kChunks], rb[kChunks];
    if (nvec > 0) {
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int64_t v = v0 + static_cast<int64_t>(c) * kBlock;
            const int64_t vc = v < nvec ? v : nvec - 1;
            ra[c] = Vec<T>::fetch(a + vc * N);
            if (OP != 0) rb[c] = Vec<T>::fetch(b + vc * N);
        }
    }
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int64_t v = v0 + static_cast<int64_t>(c) * kBlock;
        if (nvec > 0) {
            float av[N], bv[N], o[N];
            Vec<T>::unpack(ra[c], av);
            if (OP != 0) Vec<T>::unpack(rb[c], bv);
#pragma unroll
            for (int i = 0; i < N; ++i) o[i] = op(av[i], OP != 0 ? bv[i] : 0.f);
            if (v < nvec) Vec<T>::store(y + v * N, o);
        }
        if (v == nvec) {
            for (int64_t e = nvec * N; e < n; ++e) {
                const float bv = OP != 0 ? Vec<T>::get(b + e) : 0.f;
                Vec<T>::put(y + e, op(Vec<T>::get(a + e), bv));
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
