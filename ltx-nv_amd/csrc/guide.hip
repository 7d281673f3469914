// The guidance tail of one denoising step, fused (standalone/ltx_dit.py:551-562,
// 592-598, 602-606):
//
//   x0_p     = round(latent - v_p * ts_p)               p = cond, uncond, ptb, mod
//   pred     = c + (cfg-1)(c - u) + stg (c - p) + (mod-1)(c - m)     (fp32, c = x0_cond)
//   pred    *= r * std(c) / std(pred) + (1 - r)          (only when r != 0)
//   denoised = round(pred)
//   next     = round(latent + round((latent - denoised) / sigma) * dt)
//
// The latent is read once for all four passes (the reference repeats it four
// times).  With r != 0 the two standard deviations are global reductions, so
// the work is two launches: a statistics pass writing one fp64 partial
// (sum, sum of squares of c and pred) per block into the caller's workspace,
// and the output pass, whose every block folds those partials (at most
// kStatBlocks of them, an 8 KB cache-resident read, while its own inputs are
// loading) and then recomputes its elements from the inputs and writes them.  Recomputing costs one extra read
// of the small latent-sized inputs and avoids an fp32 scratch copy of pred.
// Without rescale it is the output pass alone.
//
// Every fp32 operation is the reference's, in its order and with one rounding
// each (no contraction; the build passes -ffp-contract=off), so only the two
// standard deviations (fp64 sums here) can differ from an eager evaluation.
#include <math.h>

#include <mutex>

#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kStatBlocks = 256;  // partials; the output pass folds one per thread
constexpr int kPasses = 4;

struct GuideArgs {
    const uint16_t *lat;   // [n]
    const uint16_t *vel;   // [kPasses][n]
    const float *ts;       // ts[p * ts_ps + row * ts_rs]
    uint16_t *den;         // [n] or null
    uint16_t *x0;          // [kPasses][n] or null
    uint16_t *next;        // [n] or null
    double *part;          // [stat_blocks][4]
    int64_t n, dim, ts_ps, ts_rs, chunks;
    int stat_blocks;
    int rescale;
    float a_cfg, a_stg, a_mod;  // cfg-1, stg, mod-1 as the reference's fp32 scalars
    float r, one_minus_r;
    float sigma, dt;
};

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

struct Chunk {
    float x[8];
    float x0[kPasses][8];
    float pred[8];
};

// The raw inputs of one chunk: 8 latent elements, the 4 passes' velocities
// (or x0) and timesteps.
struct Raw {
    uint4 v[1 + kPasses];
    float t[kPasses];
};

// Issues the loads of chunk `ch` (one latent row never splits a chunk:
// dim % 8 == 0); nothing waits for them here.
__device__ __forceinline__ void load_chunk(const GuideArgs &a, int64_t ch, Raw &r)
{
    // the four passes' velocities as one buffer range: streamed loads
    const rsrc_t rv = make_rsrc(a.vel, static_cast<uint32_t>(a.n * kPasses * 2));
    const int64_t e = ch * 8;
    const int64_t row = udiv32(e, a.dim);
    r.v[0] = a.lat ? ld16(a.lat + e) : uint4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        r.v[1 + p] = ldb4(rv, static_cast<uint32_t>((p * a.n + e) * 2));
        r.t[p] = a.ts ? a.ts[p * a.ts_ps + row * a.ts_rs] : 0.0f;
    }
}

// x0 of every pass and the guided prediction of a loaded chunk.  Without
// timesteps the second operand already holds the four x0.
__device__ __forceinline__ void eval_chunk(const GuideArgs &a, const Raw &r, Chunk &c)
{
    unpack8(r.v[0], c.x);
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        float v[8];
        unpack8(r.v[1 + p], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) c.x0[p][i] = a.ts ? round_bf16(c.x[i] - v[i] * r.t[p]) : v[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float cc = c.x0[0][i];
        float pr = cc + a.a_cfg * (cc - c.x0[1][i]);
        pr = pr + a.a_stg * (cc - c.x0[2][i]);
        pr = pr + a.a_mod * (cc - c.x0[3][i]);
        c.pred[i] = pr;
    }
}

// Block-wide sum of four doubles; the totals are returned in every thread.
__device__ __forceinline__ void block_sum4(double s[4], double *lds /* [kBlock/64][4] */)
{
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s[k] += __shfl_xor(s[k], o, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int k = 0; k < 4; ++k) lds[wave * 4 + k] = s[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) t += lds[w * 4 + k];
        s[k] = t;
    }
    __syncthreads();
}

// A thread's chunks are ch, ch + stride, ...; two of them have their loads
// in flight before either is evaluated (with 256 blocks the latent-sized
// inputs of a [6144, 128] step are 1.5 chunks a thread: one round trip to
// memory instead of two).  The sums run over the chunks in the same order.
__global__ void __launch_bounds__(kBlock) guide_stats_kernel(GuideArgs a)
{
    __shared__ double lds[kBlock / 64 * 4];
    double s[4] = {0.0, 0.0, 0.0, 0.0};
    auto add = [&](const Raw &r) {
        Chunk c;
        eval_chunk(a, r, c);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const double cc = c.x0[0][i], pp = c.pred[i];
            s[0] += cc;
            s[1] += cc * cc;
            s[2] += pp;
            s[3] += pp * pp;
        }
    };
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t ch = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; ch < a.chunks; ch += 2 * stride) {
        const bool two = ch + stride < a.chunks;
        Raw r0, r1;
        load_chunk(a, ch, r0);
        if (two) load_chunk(a, ch + stride, r1);
        add(r0);
        if (two) add(r1);
    }
    block_sum4(s, lds);
    if (threadIdx.x < 4) a.part[blockIdx.x * 4 + threadIdx.x] = s[threadIdx.x];
}

// Unbiased standard deviation (torch.std's default) from fp64 sums, as fp32.
__device__ __forceinline__ float std_from_sums(double sum, double sumsq, double n)
{
    const double var = (sumsq - sum * sum / n) / (n - 1.0);
    return static_cast<float>(sqrt(var > 0.0 ? var : 0.0));
}

// The chunk's loads are issued before the partials are folded, so the two
// memory round trips overlap.
__global__ void __launch_bounds__(kBlock) guide_apply_kernel(GuideArgs a)
{
    __shared__ double lds[kBlock / 64 * 4];
    const int64_t ch = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const bool live = ch < a.chunks;
    Raw raw;
    if (live) load_chunk(a, ch, raw);
    float factor = 1.0f;
    if (a.rescale) {
        double s[4] = {0.0, 0.0, 0.0, 0.0};
        if (static_cast<int>(threadIdx.x) < a.stat_blocks)
#pragma unroll
            for (int k = 0; k < 4; ++k) s[k] = a.part[threadIdx.x * 4 + k];
        block_sum4(s, lds);
        const double n = static_cast<double>(a.n);
        const float ratio = std_from_sums(s[0], s[1], n) / std_from_sums(s[2], s[3], n);
        factor = a.r * ratio + a.one_minus_r;
    }
    if (!live) return;
    Chunk c;
    eval_chunk(a, raw, c);
    const int64_t e = ch * 8;
    float den[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) den[i] = round_bf16(a.rescale ? c.pred[i] * factor : c.pred[i]);
    // outputs as buffer ranges (empty when not requested): write-through stores
    const uint32_t nb = static_cast<uint32_t>(a.n * 2);
    const rsrc_t rden = make_rsrc(a.den, a.den ? nb : 0u);
    const rsrc_t rx0 = make_rsrc(a.x0, a.x0 ? nb * kPasses : 0u);
    const rsrc_t rnext = make_rsrc(a.next, a.next ? nb : 0u);
    const uint32_t eb = static_cast<uint32_t>(e * 2);
    if (a.den) stb(rden, eb, pack8v(den));
    if (a.x0)
#pragma unroll
        for (int p = 0; p < kPasses; ++p) stb(rx0, p * nb + eb, pack8v(c.x0[p]));
    if (a.next) {
        float nx[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float vel = round_bf16((c.x[i] - den[i]) / a.sigma);
            nx[i] = c.x[i] + vel * a.dt;
        }
        stb(rnext, eb, pack8v(nx));
    }
}

int stat_blocks_for(int64_t chunks)
{
    const int64_t g = (chunks + kBlock - 1) / kBlock;
    return static_cast<int>(g < kStatBlocks ? (g > 0 ? g : 1) : kStatBlocks);
}

}  // namespace
}  // namespace ltxk

// Partial sums of ltxk_guide_noalloc: the library's own device memory, one
// copy per GPU, held until the process ends.  Its size covers every input
// ltxk_guide accepts (at most kStatBlocks partials of four doubles).  Host
// code never passes this name to a kernel (on the host it is a stand-in, not
// a device address): the address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) double scratch[ltxk::kStatBlocks * 4];

namespace ltxk {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, looked up once

// The address of `scratch` on the current device (looked up on the first call
// there, with that device current).
int device_scratch(void **out, const char *what)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(LTXK_E_HIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(LTXK_E_ARG, "%s: device %d beyond %d", what, dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(LTXK_E_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return LTXK_OK;
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int64_t ltxk_guide_workspace_bytes(int64_t n)
{
    if (n < 0) return 0;
    return static_cast<int64_t>(stat_blocks_for(n / 8)) * 4 * static_cast<int64_t>(sizeof(double));
}

extern "C" int ltxk_guide(void *denoised, void *x0, void *next, const void *latent, const void *velocity,
                          const float *timesteps, int64_t ts_pass_stride, int64_t ts_row_stride, int64_t rows,
                          int64_t dim, const ltxk_guidance *g, float sigma, float dt, void *workspace,
                          int64_t workspace_bytes, void *stream)
{
    static const char *what = "guide";
    clear_error();
    if (!g) return fail(LTXK_E_ARG, "%s: guidance parameters are required", what);
    if (rows < 0 || dim <= 0 || dim % 8) return fail(LTXK_E_ARG, "%s: dim must be a positive multiple of 8", what);
    if (rows == 0 || (!denoised && !x0 && !next)) return LTXK_OK;
    // the four passes' tensors are addressed by 32-bit byte offsets
    if (rows * dim > (int64_t{1} << 28)) return fail(LTXK_E_ARG, "%s: more than 2^28 elements", what);
    if (!velocity) return fail(LTXK_E_ARG, "%s: velocity (or x0) is required", what);
    if (!latent && (timesteps || next))
        return fail(LTXK_E_ARG, "%s: the latent is required with timesteps or an Euler step", what);
    for (const void *p : {static_cast<const void *>(denoised), static_cast<const void *>(x0),
                          static_cast<const void *>(next), latent, velocity})
        if (!aligned16(p)) return fail(LTXK_E_ALIGN, "%s: bf16 buffers must be 16-byte aligned", what);
    if (ts_pass_stride < 0 || ts_row_stride < 0) return fail(LTXK_E_ARG, "%s: negative timestep stride", what);

    GuideArgs a{};
    a.lat = static_cast<const uint16_t *>(latent);
    a.vel = static_cast<const uint16_t *>(velocity);
    a.ts = timesteps;
    a.den = static_cast<uint16_t *>(denoised);
    a.x0 = static_cast<uint16_t *>(x0);
    a.next = static_cast<uint16_t *>(next);
    a.n = rows * dim;
    a.dim = dim;
    a.ts_ps = ts_pass_stride;
    a.ts_rs = ts_row_stride;
    a.chunks = a.n / 8;
    a.stat_blocks = stat_blocks_for(a.chunks);
    a.rescale = g->rescale_scale != 0.0;
    // Python float scalars meet fp32 tensors as fp32 values (torch's scalar rule).
    a.a_cfg = static_cast<float>(g->cfg_scale - 1.0);
    a.a_stg = static_cast<float>(g->stg_scale);
    a.a_mod = static_cast<float>(g->modality_scale - 1.0);
    a.r = static_cast<float>(g->rescale_scale);
    a.one_minus_r = static_cast<float>(1.0 - g->rescale_scale);
    a.sigma = sigma;
    a.dt = dt;
    const int64_t apply_blocks = (a.chunks + kBlock - 1) / kBlock;
    if (apply_blocks > 0x7fffffff) return fail(LTXK_E_ARG, "%s: too many elements", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (a.rescale) {
        const int64_t need = ltxk_guide_workspace_bytes(a.n);
        if (!workspace || workspace_bytes < need)
            return fail(LTXK_E_ARG, "%s: rescale needs a workspace of %lld bytes (got %lld)", what, (long long)need,
                        (long long)workspace_bytes);
        if (reinterpret_cast<uintptr_t>(workspace) & 7u)
            return fail(LTXK_E_ALIGN, "%s: workspace must be 8-byte aligned", what);
        a.part = static_cast<double *>(workspace);
        guide_stats_kernel<<<dim3(a.stat_blocks), dim3(kBlock), 0, s>>>(a);
        int rc = check_launch(what);
        if (rc) return rc;
    }
    guide_apply_kernel<<<dim3(static_cast<unsigned>(apply_blocks)), dim3(kBlock), 0, s>>>(a);
    return check_launch(what);
}

extern "C" int ltxk_guide_noalloc(void *denoised, void *x0, void *next, const void *latent, const void *velocity,
                                  const float *timesteps, int64_t ts_pass_stride, int64_t ts_row_stride,
                                  int64_t rows, int64_t dim, const ltxk_guidance *g, float sigma, float dt,
                                  void *stream)
{
    static const char *what = "guide_noalloc";
    clear_error();
    if (rows < 0 || dim <= 0 || rows * dim > (int64_t{1} << 28))
        return fail(LTXK_E_ARG, "%s: rows*dim must be in [0, 2^28] with dim > 0 (got %lld x %lld)", what,
                    (long long)rows, (long long)dim);
    // The partials need no clearing: the statistics launch writes every one
    // that the output launch reads, within this call.
    void *ws = nullptr;
    if (g && g->rescale_scale != 0.0) {
        const int rc = device_scratch(&ws, what);
        if (rc) return rc;
    }
    const int64_t need = ltxk_guide_workspace_bytes(rows * dim);
    if (need > static_cast<int64_t>(sizeof(scratch)))
        return fail(LTXK_E_ARG, "%s: needs %lld bytes of partials, the library holds %lld", what, (long long)need,
                    (long long)sizeof(scratch));
    return ltxk_guide(denoised, x0, next, latent, velocity, timesteps, ts_pass_stride, ts_row_stride, rows, dim, g,
                      sigma, dt, ws, ws ? static_cast<int64_t>(sizeof(scratch)) : 0, stream);
}
