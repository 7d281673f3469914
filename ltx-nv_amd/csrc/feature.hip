// Multi-layer feature normalisation of the text-encoder connector path
// (FeatureExtractorV2, standalone/ltx_te.py:167-184, up to its two
// projections):
//
//   n_l[r, :]          = round(x_l[r, :] * rsqrt(mean(x_l[r, :]^2) + eps))
//   out_k[r, d*L + l]  = keep[r] ? round(n_l[r, d] * scale_k) : 0      k = 0, 1
//
// for the L hidden states x_l [rows, D] of the language model.  The reference
// stacks the L tensors on a new last axis (a full copy), normalises over D and
// flattens to [rows, D*L], so output element d*L + l interleaves the layers.
//
// One launch; a workgroup owns a row at a time (rows strided over a grid of
// resident workgroups).  Its waves first reduce the row's L layer rows, two at
// a time per wave with sixteen 16-byte loads per lane in flight, into L
// reciprocal RMS values in LDS.  The workgroup then writes the row's output in
// tiles of kSuper hidden columns: the tile's L x kSuper values are read,
// normalised and staged in LDS (layer rows padded so one column's values fall
// in different banks), and written back as the tile's kSuper*L contiguous
// interleaved outputs with 16-byte stores, once per output scale.  The next
// tile's loads are in flight while the current one is written.  The tile loads
// read the layer rows a second time (a row is 376 KB at 49 x 3840, more than
// LDS holds; the measured fetch shows the second read coming from HBM), so
// rows that fit in the registers of a 1024-thread workgroup take the resident
// form below, which reads them once.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxLayers = 64;
constexpr int kSuper = 512;  // hidden columns per LDS tile (a multiple of 8)

struct FeatureArgs {
    const uint16_t *layers[kMaxLayers];
    uint16_t *out0;
    uint16_t *out1;
    const uint8_t *keep;
    int64_t rows, dim;
    int n_layers;
    float eps, s0, s1;
    float fdim;         // dim as a float (the mean's divisor)
    uint32_t cu_magic;  // ceil(2^32 / (dim / 8)): chunk -> layer by one multiply-high
    uint32_t l_magic;   // ceil(2^32 / n_layers): output element -> hidden column
};

// Sums of squares of two layer rows at once (16 loads per lane in flight):
// the row pair's totals land in s[0], s[1] of every lane.
__device__ __forceinline__ void layer_sumsq2(const uint16_t *x0, const uint16_t *x1, int64_t units, int lane,
                                             float s[2])
{
    s[0] = s[1] = 0.f;
    for (int64_t base = 0; base < units; base += 8 * 64) {
        uint4 r[2][8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t u = base + lane + k * 64;
            const int64_t off = (u < units ? u : 0) * 8;
            r[0][k] = ld16(x0 + off);
            r[1][k] = ld16(x1 + off);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                float v[8];
                unpack8(r[j][k], v);
                const bool in = base + lane + k * 64 < units;
#pragma unroll
                for (int i = 0; i < 8; ++i) s[j] = __builtin_fmaf(in ? v[i] : 0.f, in ? v[i] : 0.f, s[j]);
            }
    }
    s[0] = wave_sum64(s[0]);
    s[1] = wave_sum64(s[1]);
}

// The whole operation (see the top of the file); `sw` is the tile width,
// kSuper or kSuper / 2 when L rows of kSuper + 8 values exceed 64 KB of LDS.
__global__ void __launch_bounds__(kBlock) feature_norm_kernel(FeatureArgs a, int sw)
{
    constexpr int NT = kBlock;
    constexpr int Q = kMaxLayers * (kSuper / 8) / NT;  // tile chunks per thread, at most
    extern __shared__ __align__(16) uint16_t stage[];  // [L][sw + 8]
    __shared__ float rinv[kMaxLayers];
    const int L = a.n_layers;
    const int stride = sw + 8;  // padded: the layer rows of one column fall in different banks
    const int lane = threadIdx.x & 63;
    const int64_t units = a.dim / 8;
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
        for (int l = threadIdx.x >> 6; l < L; l += 2 * (NT / 64)) {
            const int l2 = l + NT / 64 < L ? l + NT / 64 : l;  // wave-uniform
            float sq[2];
            layer_sumsq2(a.layers[l] + row * a.dim, a.layers[l2] + row * a.dim, units, lane, sq);
            if (lane == 0) {
                rinv[l] = rsqrtf(sq[0] / static_cast<float>(a.dim) + a.eps);
                rinv[l2] = rsqrtf(sq[1] / static_cast<float>(a.dim) + a.eps);
            }
        }
        const bool keep = a.keep ? a.keep[row] != 0 : true;
        uint4 raw[Q];
        // loads of the tile at column d0; indexes clamped, so every load is in bounds
        auto fetch = [&](int64_t d0) {
            const int wu = static_cast<int>(a.dim - d0 < sw ? a.dim - d0 : sw) / 8;
            const int n = L * wu;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int i = threadIdx.x + q * NT < n ? threadIdx.x + q * NT : n - 1;
                const int l = static_cast<int>(udiv32(i, wu));
                raw[q] = ld16(a.layers[l] + row * a.dim + d0 + (i - l * wu) * 8);
            }
        };
        fetch(0);
        __syncthreads();  // rinv complete
        for (int64_t d0 = 0; d0 < a.dim; d0 += sw) {
            const int w = static_cast<int>(a.dim - d0 < sw ? a.dim - d0 : sw);  // multiple of 8
            const int wu = w / 8;
            const int n = L * wu;
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int i = threadIdx.x + q * NT;
                const int l = static_cast<int>(udiv32(i < n ? i : n - 1, wu));
                float v[8];
                unpack8(raw[q], v);
                const float r = rinv[l];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = v[k] * r;  // rounded by pack8: the reference's bf16 normed
                if (i < n) *reinterpret_cast<uint4 *>(&stage[l * stride + (i - l * wu) * 8]) = pack8(v);
            }
            __syncthreads();
            // next tile's loads (at the last tile, the same tile again: never used)
            fetch(d0 + sw < a.dim ? d0 + sw : d0);
            const int chunks = w * L / 8;
            uint16_t *t0 = a.out0 + row * a.dim * L + d0 * L;
            uint16_t *t1 = a.out1 ? a.out1 + row * a.dim * L + d0 * L : nullptr;
            for (int i = threadIdx.x; i < chunks; i += NT) {
                int d = udiv32(i * 8, L), l = i * 8 - d * L;
                float v0[8], v1[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float nv = bf16_to_f32(stage[l * stride + d]);
                    v0[k] = keep ? nv * a.s0 : 0.f;  // masked rows are +0 (torch.where before the scale)
                    v1[k] = keep ? nv * a.s1 : 0.f;
                    if (++l == L) l = 0, ++d;
                }
                st16_stream(t0 + i * 8, pack8(v0));
                if (t1) st16_stream(t1 + i * 8, pack8(v1));
            }
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------- resident --
// Rows whose L x D/8 16-byte chunks fit in the registers of one 1024-thread
// workgroup (kResident chunks per thread: 49 x 3840 is 23,520 chunks, 23 per
// thread) are read once.  Chunk c = i * 1024 + thread (layer c / (D/8),
// column chunk c % (D/8)) stays in registers from its load to its staging
// tile: the sums of squares are formed per chunk, reduced per wave in two
// parts split at the layer boundary inside the wave's 64 chunks (D >= 512
// keeps it to at most one boundary), and the parts of each layer are added in
// chunk order (deterministic).  The normalised bf16 values replace the raw
// ones in the same registers, then go to the output through LDS tiles of `tw`
// hidden columns as in feature_norm_kernel.  After the last tile is staged the
// registers are free and the workgroup's next row is loaded while the tile is
// written.
constexpr int kWide = 1024;
constexpr int kWideWaves = kWide / 64;
constexpr int kResident = 24;  // chunks per thread, at most

typedef const __attribute__((address_space(1))) u32x4 GlobalChunk;

// c / (dim / 8) for c < 2^15 and dim / 8 < 2^15 (a resident row has at most
// 24,576 chunks): exact with the rounded-up reciprocal, since
// c * (magic * (dim / 8) - 2^32) < 2^15 * 2^15 < 2^32.
__device__ __forceinline__ int layer_of(const FeatureArgs &a, int c)
{
    return static_cast<int>(__umulhi(static_cast<uint32_t>(c), a.cu_magic));
}

// threadIdx.x through an empty asm: values derived from it are recomputed in
// each phase instead of being hoisted out of the row loop, where they would
// hold registers the row's data needs.
__device__ __forceinline__ int fresh_tid()
{
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

template <int NCH>
__global__ void __launch_bounds__(kWide) feature_norm_resident_kernel(FeatureArgs a, int tw)
{
    extern __shared__ __align__(16) uint16_t stage[];  // [L][tw + 8]
    __shared__ const GlobalChunk *lptr[kMaxLayers];  // global-space pointers: global (not flat) loads
    __shared__ float rinv[kMaxLayers];
    __shared__ float part[NCH * kWideWaves * 2];  // per 64-chunk block: first layer, next layer
    const int lane = threadIdx.x & 63;
    const int L = a.n_layers;
    const int cu = static_cast<int>(a.dim / 8);  // chunks per layer row, >= 64
    const int U = L * cu;
    const int stride = tw + 8;
    if (threadIdx.x < L) lptr[threadIdx.x] = (const GlobalChunk *)(a.layers[threadIdx.x]);  // generic -> global
    int64_t row = blockIdx.x;
    if (row >= a.rows) return;  // uniform over the workgroup
    __syncthreads();
    u32x4 x[NCH];
    auto load = [&](int64_t r) {
        const int tid = fresh_tid();
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = i * kWide + tid < U ? i * kWide + tid : U - 1;  // clamped: in bounds
            const int l = layer_of(a, c);
            x[i] = __builtin_nontemporal_load(lptr[l] + r * cu + (c - l * cu));
        }
    };
    load(row);
    for (;;) {
        int tid = fresh_tid();
        const int wbase = __builtin_amdgcn_readfirstlane(tid & ~63);  // the wave's first thread (scalar)
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = i * kWide + tid;
            float v[8];
            unpack8v(x[i], v);
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = __builtin_fmaf(v[e], v[e], s);
            if (c >= U) s = 0.f;
            const int l0 = layer_of(a, i * kWide + wbase);  // scalar
            const bool first = layer_of(a, c < U ? c : U - 1) == l0;
            const float s0 = wave_sum64(first ? s : 0.f);
            const float s1 = wave_sum64(first ? 0.f : s);
            if (lane == 0) {
                part[(i * kWideWaves + wbase / 64) * 2] = s0;
                part[(i * kWideWaves + wbase / 64) * 2 + 1] = s1;
            }
        }
        __syncthreads();
        if (tid < L) {
            const int lo = tid * cu, hi = lo + cu - 1;
            float t = 0.f;
            for (int b = lo / 64; b <= hi / 64; ++b) t += part[b * 2 + (layer_of(a, b * 64) == tid ? 0 : 1)];
            rinv[tid] = rsqrtf(t / a.fdim + a.eps);
        }
        __syncthreads();
        tid = fresh_tid();
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = i * kWide + tid < U ? i * kWide + tid : U - 1;
            const float r = rinv[layer_of(a, c)];
            // the raw words, not the floats the sums unpacked, stay live across
            // the barriers: unpack again from an opaque copy
            asm volatile("" : "+v"(x[i]));
            float v[8];
            unpack8v(x[i], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = v[e] * r;
            x[i] = pack8v(v);  // rounded: the reference's bf16 normed
        }
        const bool keep = a.keep ? a.keep[row] != 0 : true;
        const int64_t next = row + gridDim.x;
        for (int d0 = 0; d0 < a.dim; d0 += tw) {
            const int w = a.dim - d0 < tw ? static_cast<int>(a.dim - d0) : tw;  // multiple of 8
            tid = fresh_tid();
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int c = i * kWide + tid;
                const int cc = c < U ? c : U - 1;
                const int l = layer_of(a, cc);
                const int j = (cc - l * cu) * 8 - d0;
                if (c < U && j >= 0 && j < w) *reinterpret_cast<u32x4 *>(&stage[l * stride + j]) = x[i];
            }
            __syncthreads();
            if (d0 + tw >= a.dim && next < a.rows) load(next);  // registers free: next row in flight
            const int chunks = w * L / 8;
            uint16_t *t0 = a.out0 + row * a.dim * L + static_cast<int64_t>(d0) * L;
            uint16_t *t1 = a.out1 ? a.out1 + row * a.dim * L + static_cast<int64_t>(d0) * L : nullptr;
            for (int q = tid; q < chunks; q += kWide) {
                // q * 8 < tw * L <= LDS bytes / 2 < 2^17 and L <= 64: exact as in layer_of
                int d = static_cast<int>(__umulhi(static_cast<uint32_t>(q * 8), a.l_magic)), l = q * 8 - d * L;
                uint16_t h[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    h[k] = stage[l * stride + d];
                    if (++l == L) l = 0, ++d;
                }
                // one output at a time: few live registers beside the row's data
                float v[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) v[k] = keep ? bf16_to_f32(h[k]) * a.s0 : 0.f;  // masked rows are +0
                st16_stream(t0 + q * 8, pack8(v));
                if (t1) {
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = keep ? bf16_to_f32(h[k]) * a.s1 : 0.f;
                    st16_stream(t1 + q * 8, pack8(v));
                }
            }
            __syncthreads();
        }
        row = next;
        if (row >= a.rows) break;
    }
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int ltxk_feature_norm(void *out0, void *out1, const void *const *layers, int64_t n_layers,
                                 const uint8_t *keep, int64_t rows, int64_t dim, float eps, float scale0,
                                 float scale1, void *stream)
{
    static const char *what = "feature_norm";
    clear_error();
    if (n_layers < 1 || n_layers > kMaxLayers)
        return fail(LTXK_E_ARG, "%s: 1..%d layers supported (got %lld)", what, kMaxLayers, (long long)n_layers);
    if (rows < 0 || dim <= 0 || dim % 8) return fail(LTXK_E_ARG, "%s: dim must be a positive multiple of 8", what);
    if (rows == 0) return LTXK_OK;
    if (!out0 || !layers) return fail(LTXK_E_ARG, "%s: out0 and layers are required", what);
    FeatureArgs a{};
    for (int64_t l = 0; l < n_layers; ++l) {
        if (!layers[l] || !aligned16(layers[l]))
            return fail(LTXK_E_ALIGN, "%s: layer %lld is null or not 16-byte aligned", what, (long long)l);
        a.layers[l] = static_cast<const uint16_t *>(layers[l]);
    }
    if (!aligned16(out0) || !aligned16(out1)) return fail(LTXK_E_ALIGN, "%s: outputs must be 16-byte aligned", what);
    a.out0 = static_cast<uint16_t *>(out0);
    a.out1 = static_cast<uint16_t *>(out1);
    a.keep = keep;
    a.rows = rows;
    a.dim = dim;
    a.n_layers = static_cast<int>(n_layers);
    a.eps = eps;
    a.s0 = scale0;
    a.s1 = scale1;
    a.fdim = static_cast<float>(dim);
    a.cu_magic = static_cast<uint32_t>(((uint64_t(1) << 32) + dim / 8 - 1) / (dim / 8));
    a.l_magic = static_cast<uint32_t>(((uint64_t(1) << 32) + n_layers - 1) / n_layers);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    const int64_t chunks = n_layers * (dim / 8);
    if (dim >= 512 && chunks <= static_cast<int64_t>(kResident) * kWide) {
        // the resident form: tiles as wide as the LDS allows (multiples of 64 columns)
        int lds_max = 0;
        if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            lds_max <= 0)
            lds_max = 65536;
        const int fixed = 4096;  // the kernel's static LDS, rounded up
        int64_t tw = ((lds_max - fixed) / (2 * n_layers) - 8) / 64 * 64;
        if (tw > dim) tw = (dim + 63) / 64 * 64;
        if (tw >= 64) {
            const size_t lds = static_cast<size_t>(n_layers) * (tw + 8) * sizeof(uint16_t);
            const int64_t grid = cus < rows ? cus : rows;
            auto go = [&](auto kernel) {
                (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
                kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kWide), lds, st>>>(a, static_cast<int>(tw));
            };
            if (chunks <= 8 * kWide)
                go(feature_norm_resident_kernel<8>);
            else if (chunks <= 16 * kWide)
                go(feature_norm_resident_kernel<16>);
            else
                go(feature_norm_resident_kernel<kResident>);
            return check_launch(what);
        }
    }
    const int sw = n_layers * (kSuper + 8) * 2 <= 65536 ? kSuper : kSuper / 2;
    const size_t lds = static_cast<size_t>(n_layers) * (sw + 8) * sizeof(uint16_t);
    // as many workgroups as can be resident (compute units x occupancy), at most one per row
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, feature_norm_kernel, kBlock, lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const int64_t grid = static_cast<int64_t>(cus) * per_cu < rows ? static_cast<int64_t>(cus) * per_cu : rows;
    feature_norm_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), lds, st>>>(a, sw);
    return check_launch(what);
}
