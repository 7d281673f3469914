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
// Two launches.  The statistics launch gives each (row, layer) pair to one
// wave, which streams the row (8 loads per lane in flight at D = 3840) and
// leaves rsqrt(mean + eps) in the caller's workspace.  The output launch gives
// each (row, kTile-column tile) to one workgroup: it stages the L x kTile
// normalised values in LDS and writes the tile's kTile*L contiguous
// interleaved outputs with 16-byte stores, once per output scale.  The output
// launch walks the rows in reverse, so its first rows are the ones the
// statistics launch read last and may still find in the MALL.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxLayers = 64;
constexpr int kTile = 64;  // hidden columns per output workgroup (multiple of 8)

struct FeatureArgs {
    const uint16_t *layers[kMaxLayers];
    uint16_t *out0;
    uint16_t *out1;
    const uint8_t *keep;
    float *rinv;  // [rows][n_layers]
    int64_t rows, dim;
    int n_layers, tiles;
    float eps, s0, s1;
};

__global__ void __launch_bounds__(kBlock) feature_stats_kernel(FeatureArgs a)
{
    const int64_t task = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t tasks = a.rows * a.n_layers;
    const bool active = task < tasks;
    const int64_t t = active ? task : tasks - 1;
    const int64_t row = udiv32(t, a.n_layers);
    // one (row, layer) task per wave: the layer index is wave-uniform, so its
    // pointer comes through the scalar cache
    const int l = __builtin_amdgcn_readfirstlane(static_cast<int>(t - row * a.n_layers));
    const uint16_t *x = a.layers[l] + row * a.dim;
    const int64_t units = a.dim / 8;
    float s = 0.f;
    int64_t u = lane;
    for (; u + 3 * 64 < units; u += 4 * 64) {  // four loads in flight per step
        uint4 r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = ld16_stream(x + (u + k * 64) * 8);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float v[8];
            unpack8(r[k], v);
#pragma unroll
            for (int i = 0; i < 8; ++i) s = __builtin_fmaf(v[i], v[i], s);
        }
    }
    for (; u < units; u += 64) {
        float v[8];
        unpack8(ld16_stream(x + u * 8), v);
#pragma unroll
        for (int i = 0; i < 8; ++i) s = __builtin_fmaf(v[i], v[i], s);
    }
    s = wave_sum64(s);
    if (active && lane == 0) a.rinv[t] = rsqrtf(s / static_cast<float>(a.dim) + a.eps);
}

__global__ void __launch_bounds__(kBlock) feature_write_kernel(FeatureArgs a)
{
    __shared__ __align__(16) uint16_t tile[kMaxLayers * kTile];
    const int L = a.n_layers;
    const int64_t rblk = blockIdx.x / a.tiles;
    const int64_t row = a.rows - 1 - rblk;  // reverse order: see above
    const int64_t d0 = static_cast<int64_t>(blockIdx.x - rblk * a.tiles) * kTile;
    const int w = static_cast<int>(a.dim - d0 < kTile ? a.dim - d0 : kTile);  // multiple of 8
    const int wu = w / 8;
    for (int i = threadIdx.x; i < L * wu; i += kBlock) {
        const int l = i / wu, u = i - l * wu;
        float v[8];
        unpack8(ld16(a.layers[l] + row * a.dim + d0 + u * 8), v);
        const float r = a.rinv[row * L + l];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = v[k] * r;  // rounded by pack8: the reference's bf16 normed
        *reinterpret_cast<uint4 *>(&tile[l * kTile + u * 8]) = pack8(v);
    }
    __syncthreads();
    const bool keep = a.keep ? a.keep[row] != 0 : true;
    const int chunks = w * L / 8;
    uint16_t *t0 = a.out0 + row * a.dim * L + d0 * L;
    uint16_t *t1 = a.out1 ? a.out1 + row * a.dim * L + d0 * L : nullptr;
    for (int i = threadIdx.x; i < chunks; i += kBlock) {
        int d = (i * 8) / L, l = i * 8 - d * L;
        float v0[8], v1[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float nv = bf16_to_f32(tile[l * kTile + d]);
            v0[k] = keep ? nv * a.s0 : 0.f;  // masked rows are +0 (torch.where before the scale)
            v1[k] = keep ? nv * a.s1 : 0.f;
            if (++l == L) l = 0, ++d;
        }
        st16_stream(t0 + i * 8, pack8(v0));
        if (t1) st16_stream(t1 + i * 8, pack8(v1));
    }
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int64_t ltxk_feature_norm_workspace_bytes(int64_t rows, int64_t n_layers)
{
    if (rows <= 0 || n_layers <= 0) return 0;
    return rows * n_layers * static_cast<int64_t>(sizeof(float));
}

extern "C" int ltxk_feature_norm(void *out0, void *out1, const void *const *layers, int64_t n_layers,
                                 const uint8_t *keep, int64_t rows, int64_t dim, float eps, float scale0,
                                 float scale1, void *workspace, int64_t workspace_bytes, void *stream)
{
    static const char *what = "feature_norm";
    clear_error();
    if (n_layers < 1 || n_layers > kMaxLayers)
        return fail(LTXK_E_ARG, "%s: 1..%d layers supported (got %lld)", what, kMaxLayers, (long long)n_layers);
    if (rows < 0 || dim <= 0 || dim % 8) return fail(LTXK_E_ARG, "%s: dim must be a positive multiple of 8", what);
    const int64_t tiles = (dim + kTile - 1) / kTile;
    if (rows * n_layers > 0x7fffffff || rows * tiles > 0x7fffffff) return fail(LTXK_E_ARG, "%s: too many rows", what);
    if (rows == 0) return LTXK_OK;
    if (!out0 || !layers) return fail(LTXK_E_ARG, "%s: out0 and layers are required", what);
    const int64_t need = ltxk_feature_norm_workspace_bytes(rows, n_layers);
    if (!workspace || workspace_bytes < need)
        return fail(LTXK_E_ARG, "%s: needs a workspace of %lld bytes (got %lld)", what, (long long)need,
                    (long long)workspace_bytes);
    if (reinterpret_cast<uintptr_t>(workspace) & 3u)
        return fail(LTXK_E_ALIGN, "%s: workspace not 4-byte aligned", what);
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
    a.rinv = static_cast<float *>(workspace);
    a.rows = rows;
    a.dim = dim;
    a.n_layers = static_cast<int>(n_layers);
    a.tiles = static_cast<int>(tiles);
    a.eps = eps;
    a.s0 = scale0;
    a.s1 = scale1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t stat_blocks = (rows * n_layers + (kBlock / 64) - 1) / (kBlock / 64);
    feature_stats_kernel<<<dim3(static_cast<unsigned>(stat_blocks)), dim3(kBlock), 0, s>>>(a);
    int rc = check_launch(what);
    if (rc) return rc;
    feature_write_kernel<<<dim3(static_cast<unsigned>(rows * tiles)), dim3(kBlock), 0, s>>>(a);
    return check_launch(what);
}
