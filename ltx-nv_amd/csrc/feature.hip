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
// read the layer rows a second time: a row is 376 KB at 49 x 3840, too much to
// keep on chip for the reduction, and the measured fetch shows the second read
// coming from HBM.
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
    const int sw = n_layers * (kSuper + 8) * 2 <= 65536 ? kSuper : kSuper / 2;
    const size_t lds = static_cast<size_t>(n_layers) * (sw + 8) * sizeof(uint16_t);
    // as many workgroups as can be resident (compute units x occupancy), at most one per row
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, feature_norm_kernel, kBlock, lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const int64_t grid = static_cast<int64_t>(cus) * per_cu < rows ? static_cast<int64_t>(cus) * per_cu : rows;
    feature_norm_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kBlock), lds, static_cast<hipStream_t>(stream)>>>(
        a, sw);
    return check_launch(what);
}
