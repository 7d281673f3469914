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
                const int i0 = static_cast<int>(threadIdx.x) + q * NT;
                const int i = i0 < n ? i0 : n - 1;
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
// workgroup are read once.  A row is cut into T <= 3 tiles of hidden columns
// (49 x 3840: three of 1280), and tile t's L x (columns / 8) chunks are held
// in its own kTileChunks registers per thread (tile-local chunk k = j * 1024
// + thread: layer k / groups, column group k % groups), so that every index
// into the register array is known at compile time.  Per tile:
//  1. stage: each thread normalises the tile's chunks it holds and scatters
//     their 8 values into LDS in output order: a group of 8 columns is its 8L
//     interleaved outputs, padded by one dword, so the 64 lanes of a wave
//     (consecutive column groups of one layer, 4L + 1 dwords apart) write 64
//     different banks;
//  2. after a barrier, output: the tile's contiguous outputs are read back 16
//     bytes at a time, scaled and stored (no index arithmetic per element),
//     and the tile's registers are loaded with the same chunks of the
//     workgroup's next row: behind the stores (measured faster than
//     interleaved with them or ahead of them), except in the last tile, where
//     they go ahead so that the next row's statistics need not wait for the
//     stores (measured 3 % faster).
// The sums of squares of the next row's tile t are formed in the next tile's
// stage phase (into LDS, one float per chunk) and a wave per layer adds them
// in a fixed order, so the statistics of the next row are complete one short
// phase after the current row's last stores are issued.
constexpr int kWide = 1024;
constexpr int kWideWaves = kWide / 64;
constexpr int kTileChunks = 8;  // chunks per thread per tile
constexpr int kMaxTiles = 3;
constexpr int kResident = kTileChunks * kMaxTiles;  // chunks per thread, at most

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

// keep[row] != 0 for a workgroup-uniform row, read through the scalar cache
// (a vector load would have to be waited for behind the stores in flight):
// the aligned dword that holds the byte, which lies in the byte's page.
__device__ __forceinline__ bool keep_row(const uint8_t *keep, int64_t row)
{
    if (!keep) return true;
    const uintptr_t p = reinterpret_cast<uintptr_t>(keep + row);
    const auto *w = reinterpret_cast<const __attribute__((address_space(4))) uint32_t *>(p & ~uintptr_t(3));
    return ((*w >> ((p & 3) * 8)) & 0xffu) != 0;
}

struct ResidentTiles {
    int gw;              // column groups (8 columns) per tile, the last tile excepted
    int gw_last;         // column groups of the last tile
    uint32_t gw_magic;   // ceil(2^32 / gw)
    uint32_t gwl_magic;  // ceil(2^32 / gw_last)
};

template <int T>
__global__ void __launch_bounds__(kWide) feature_norm_resident_kernel(FeatureArgs a, ResidentTiles tl)
{
    constexpr int R = kTileChunks;
    // LDS: one staged tile (tl.gw groups of 4L + 1 dwords), then one tile's
    // per-chunk sums of squares (R * 1024 floats)
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ const GlobalChunk *lptr[kMaxLayers];  // global-space pointers: global (not flat) loads
    __shared__ float rinv[kMaxLayers];
    __shared__ float lsum[T][kMaxLayers];  // per tile, per layer: sum of squares of the next row
    const int L = a.n_layers;
    const int cu = static_cast<int>(a.dim / 8);  // chunks per layer row
    const int gs = 4 * L + 1;                    // dwords per staged group of 8 columns
    float *part = reinterpret_cast<float *>(lds + tl.gw * gs);
    if (static_cast<int>(threadIdx.x) < L) lptr[threadIdx.x] = (const GlobalChunk *)(a.layers[threadIdx.x]);  // generic -> global
    int64_t row = blockIdx.x;
    if (row >= a.rows) return;  // uniform over the workgroup
    __syncthreads();
    u32x4 x[T][R];  // tile t's chunks of the current row, then (once staged) of the next row

    // tile-local chunk k of tile t: layer k / gw, column group k % gw (groups t * tl.gw + ...)
    auto groups = [&](int t) { return t == T - 1 ? tl.gw_last : tl.gw; };
    auto layer = [&](int t, int k) {  // k < 2^13, gw < 2^13: exact, as in layer_of
        return static_cast<int>(__umulhi(static_cast<uint32_t>(k), t == T - 1 ? tl.gwl_magic : tl.gw_magic));
    };
    // every lane issues its R loads (past the tile's end: its last chunk again; no row or a masked one: one fixed
    // chunk) and the output loop its 2R stores: the same count on every path, so no wait is conservative
    auto load_tile = [&](int t, int64_t r, bool real) {
        const int gw = groups(t), nq = L * gw, tid = fresh_tid();
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int k = j * kWide + tid < nq ? j * kWide + tid : nq - 1;
            const int l = layer(t, k);
            x[t][j] = __builtin_nontemporal_load(real ? lptr[l] + r * cu + t * tl.gw + (k - l * gw) : lptr[0]);
        }
    };
    auto sums = [&](int t) {  // tile t's chunks of the row in registers -> part[k]
        const int nq = L * groups(t), tid = fresh_tid();
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int k = j * kWide + tid;
            if (k < nq) {
                float v[8];
                unpack8v(x[t][j], v);
                float s = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) s = __builtin_fmaf(v[e], v[e], s);
                part[k] = s;
            }
        }
    };
    // a wave per layer: each lane in column order, then across the wave; the last tile's pass adds the
    // tiles' sums in tile order and leaves the reciprocal RMS of the row
    auto layer_sums = [&](int t) {
        const int gw = groups(t), tid = fresh_tid(), lane = tid & 63;
        for (int l = __builtin_amdgcn_readfirstlane(tid >> 6); l < L; l += kWideWaves) {
            float s = 0.f;
            for (int m = lane; m < gw; m += 64) s += part[l * gw + m];
            s = wave_sum64(s);
            if (lane == 0) {
                if (t < T - 1) {
                    lsum[t][l] = s;
                } else {
                    float tot = 0.f;
#pragma unroll
                    for (int u = 0; u < T - 1; ++u) tot += lsum[u][l];
                    rinv[l] = rsqrtf((tot + s) / a.fdim + a.eps);
                }
            }
        }
    };
    // normalise tile t's chunks into LDS in output order
    auto stage = [&](int t) {
        const int gw = groups(t), nq = L * gw, tid = fresh_tid();
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int k = j * kWide + tid;
            if (k < nq) {
                const int l = layer(t, k);
                const int g = k - l * gw;  // column group in the tile
                float v[8];
                unpack8v(x[t][j], v);
                const float r = rinv[l];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = v[e] * r;
                const u32x4 p = pack8v(v);  // rounded: the reference's bf16 normed
                uint16_t *s = reinterpret_cast<uint16_t *>(lds + g * gs) + l;  // column 8g + e at s[e * L]
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s[2 * e * L] = static_cast<uint16_t>(p[e]);
                    s[(2 * e + 1) * L] = static_cast<uint16_t>(p[e] >> 16);
                }
            }
        }
    };
    auto output = [&](int t, int64_t r, uint32_t keep_mask) {
        const int nq = L * groups(t), tid = fresh_tid();
        const int64_t base = r * a.dim * L + static_cast<int64_t>(t) * tl.gw * 8 * L;
        uint16_t *t0 = a.out0 + base;
        uint16_t *t1 = a.out1 ? a.out1 + base : t0;  // no second output: the first stored twice
        const float s1 = a.out1 ? a.s1 : a.s0;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int q = j * kWide + tid < nq ? j * kWide + tid : nq - 1;  // past the end: the last again
            // q < 2^13 and L <= 64: q / L exact with the rounded-up reciprocal
            const int g = static_cast<int>(__umulhi(static_cast<uint32_t>(q), a.l_magic));
            const uint32_t *s = lds + g * gs + 4 * (q - g * L);
            const u32x4 h = {s[0], s[1], s[2], s[3]};
            float v[8], o[8];
            unpack8v(h, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = v[e] * a.s0;
            u32x4 p = pack8v(o) & keep_mask;  // masked rows are +0 (torch.where before the scale)
            st16_stream(t0 + q * 8, uint4{p[0], p[1], p[2], p[3]});
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = v[e] * s1;
            p = pack8v(o) & keep_mask;
            st16_stream(t1 + q * 8, uint4{p[0], p[1], p[2], p[3]});
        }
    };

    // a masked row's outputs are +0 whatever its inputs: they are not read (the fixed chunk instead)
    bool kept = keep_row(a.keep, row);
#pragma unroll
    for (int t = 0; t < T; ++t) load_tile(t, row, kept);
#pragma unroll
    for (int t = 0; t < T; ++t) {
        sums(t);
        __syncthreads();
        layer_sums(t);  // the last tile's leaves rinv
        __syncthreads();
    }
    for (;;) {
        const int64_t next = row + gridDim.x;
        const bool more = next < a.rows;
        const bool next_kept = more && keep_row(a.keep, next);
        const uint32_t keep_mask = kept ? 0xffffffffu : 0u;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            stage(t);
            if (t > 0) sums(t - 1);  // the next row's chunks loaded one tile ago
            __syncthreads();
            // tile t's registers are free: the next row's chunks, behind the tile's stores, except for
            // the last tile, whose loads the next row's statistics wait for at once
            if (t == T - 1) load_tile(t, next, next_kept);
            output(t, row, keep_mask);
            if (t < T - 1) load_tile(t, next, next_kept);
            if (t > 0) layer_sums(t - 1);
            __syncthreads();
        }
        sums(T - 1);
        __syncthreads();
        layer_sums(T - 1);  // the next row's rinv (the current row's last use was stage(T - 1))
        __syncthreads();
        row = next;
        kept = next_kept;
        if (!more) break;
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
    int dev = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const int cus = device_cus();
    const int64_t chunks = n_layers * (dim / 8);
    // (one layer takes the streamed form: ceil(2^32 / n_layers) does not fit 32 bits for n_layers = 1)
    if (n_layers >= 2 && dim >= 512 && chunks <= static_cast<int64_t>(kResident) * kWide) {
        // the resident form: the fewest tiles of equal width (multiples of 8 columns) whose chunks fit
        // kTileChunks per thread and whose staged outputs fit the LDS beside one tile's sums
        int lds_max = 0;
        if (hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            lds_max <= 0)
            lds_max = 65536;
        const int64_t fixed = 2048;                          // the kernel's static LDS, rounded up
        const int64_t group_bytes = (8 * n_layers + 2) * 2;  // 8 columns x L outputs + one dword of padding
        const int64_t part_bytes = static_cast<int64_t>(kTileChunks) * kWide * 4;
        const int64_t groups = dim / 8;
        for (int tiles = 1; tiles <= kMaxTiles; ++tiles) {
            const int64_t gw = (groups + tiles - 1) / tiles;
            const int64_t gw_last = groups - (tiles - 1) * gw;
            const int64_t lds = gw * group_bytes + part_bytes;
            // (gw_last >= 2: the rounded-up reciprocals below fit 32 bits; dim >= 512 gives at least 20)
            if (gw_last < 2 || n_layers * gw > static_cast<int64_t>(kTileChunks) * kWide || lds > lds_max - fixed)
                continue;
            ResidentTiles tl;
            tl.gw = static_cast<int>(gw);
            tl.gw_last = static_cast<int>(gw_last);
            tl.gw_magic = static_cast<uint32_t>(((uint64_t(1) << 32) + gw - 1) / gw);
            tl.gwl_magic = static_cast<uint32_t>(((uint64_t(1) << 32) + gw_last - 1) / gw_last);
            const int64_t grid = cus < rows ? cus : rows;
            auto go = [&](auto kernel) {
                (void)hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
                kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kWide), static_cast<size_t>(lds), st>>>(a, tl);
            };
            if (tiles == 1)
                go(feature_norm_resident_kernel<1>);
            else if (tiles == 2)
                go(feature_norm_resident_kernel<2>);
            else
                go(feature_norm_resident_kernel<3>);
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
