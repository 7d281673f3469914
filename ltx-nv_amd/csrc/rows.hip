// Row kernels over token-major activations [rows, dim] (bf16):
//   norm_modulate       y(,y2) = norm(x) * (1 + scale) + shift
//   add_norm_modulate   x' = x + f*gate*mask ; y = rms(x') * (1 + scale) + shift
//   modulate            y = x * (1 + scale) + shift
//   gated_residual      out = x + f*gate*mask
//   head_gate           out[r,h,:] = x[r,h,:] * 2*sigmoid(logit[r,h])
//   x0                  x0 = latent - v * ts[b,t]
//
// One row per group of `tpr` threads; each thread holds up to MAXC 16-byte
// chunks (8 bf16) of its row in registers, so every activation makes exactly
// one HBM round trip.  Row sums use wave shuffles, plus LDS for the partials
// of the 2..4 waves that share a row.  fp32 arithmetic, one rounding per output.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;

struct RowGeom {
    int64_t rows;
    int64_t tokens;  // tokens per batch item: (b, t) = divmod(row, tokens)
    int64_t dim;
    int64_t units;   // dim / 8
    int tpr;
    int rows_per_block;
};

inline RowGeom make_geom(int64_t rows, int64_t tokens, int64_t dim)
{
    RowGeom g;
    g.rows = rows;
    g.tokens = tokens;
    g.dim = dim;
    g.units = dim / 8;
    RowLayout l = row_layout(g.units, kBlock);
    g.tpr = l.tpr;
    g.rows_per_block = l.rows_per_block;
    return g;
}

inline int per_thread(const RowGeom &g) { return static_cast<int>((g.units + g.tpr - 1) / g.tpr); }

inline unsigned grid_for(const RowGeom &g)
{
    return static_cast<unsigned>((g.rows + g.rows_per_block - 1) / g.rows_per_block);
}

struct RowPos {
    int64_t row;
    int lane;
    bool active;
};

__device__ __forceinline__ RowPos row_pos(const RowGeom &g)
{
    RowPos p;
    const int lrow = threadIdx.x / g.tpr;
    p.lane = threadIdx.x - lrow * g.tpr;
    p.row = static_cast<int64_t>(blockIdx.x) * g.rows_per_block + lrow;
    p.active = p.row < g.rows;
    return p;
}

// ------------------------------------------------------------ norm_modulate --
struct NormModParams {
    RowGeom g;
    uint16_t *y;
    uint16_t *y2;
    const uint16_t *x;
    const uint16_t *w;  // optional elementwise weight applied after the norm
    Ada shift, scale, shift2, scale2;
    float eps;
    int layer;  // 1: LayerNorm (mean-centred), 0: RMSNorm
};

template <int MAXC>
__global__ void __launch_bounds__(kBlock) norm_modulate_kernel(NormModParams p)
{
    __shared__ float lds[kBlock / 64];
    const RowGeom &g = p.g;
    const RowPos rp = row_pos(g);
    float v[MAXC][8];
    float s1 = 0.f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int64_t u = rp.lane + static_cast<int64_t>(k) * g.tpr;
        if (rp.active && u < g.units) {
            unpack8(ld16_stream(p.x + rp.row * g.dim + u * 8), v[k]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
        }
    }
    float mean = 0.f;
    if (p.layer) {
#pragma unroll
        for (int k = 0; k < MAXC; ++k)
#pragma unroll
            for (int i = 0; i < 8; ++i) s1 += v[k][i];
        mean = group_sum(s1, g.tpr, lds) / static_cast<float>(g.dim);
    }
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int64_t u = rp.lane + static_cast<int64_t>(k) * g.tpr;
        if (u < g.units) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float c = v[k][i] - mean;
                s2 += c * c;
            }
        }
    }
    const float var = group_sum(s2, g.tpr, lds) / static_cast<float>(g.dim);
    const float r = rsqrtf(var + p.eps);
    if (!rp.active) return;
    const int64_t b = rp.row / g.tokens, t = rp.row - (rp.row / g.tokens) * g.tokens;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int64_t u = rp.lane + static_cast<int64_t>(k) * g.tpr;
        if (u >= g.units) continue;
        float nv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) nv[i] = (v[k][i] - mean) * r;
        if (p.w) {
            float wv[8];
            unpack8(ld16(p.w + u * 8), wv);
#pragma unroll
            for (int i = 0; i < 8; ++i) nv[i] = nv[i] * wv[i];
        }
        float sh[8], sc[8], o[8];
        ada_load8(p.shift, b, t, u * 8, 0.f, sh);
        ada_load8(p.scale, b, t, u * 8, 0.f, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
        st16_stream(p.y + rp.row * g.dim + u * 8, pack8(o));
        if (p.y2) {
            ada_load8(p.shift2, b, t, u * 8, 0.f, sh);
            ada_load8(p.scale2, b, t, u * 8, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
            st16_stream(p.y2 + rp.row * g.dim + u * 8, pack8(o));
        }
    }
}

// -------------------------------------------------------- add_norm_modulate --
struct AddNormParams {
    RowGeom g;
    uint16_t *x_out;
    uint16_t *y;
    const uint16_t *x;
    const uint16_t *f;
    const uint16_t *mask;
    Ada gate, shift, scale;
    float eps;
};

template <int MAXC>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_kernel(AddNormParams p)
{
    __shared__ float lds[kBlock / 64];
    const RowGeom &g = p.g;
    const RowPos rp = row_pos(g);
    const int64_t b = rp.active ? rp.row / g.tokens : 0;
    const int64_t t = rp.active ? rp.row - b * g.tokens : 0;
    const float m = (rp.active && p.mask) ? bf16_to_f32(p.mask[b]) : 1.0f;
    float v[MAXC][8];
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int64_t u = rp.lane + static_cast<int64_t>(k) * g.tpr;
        if (rp.active && u < g.units) {
            float xv[8], fv[8], gv[8];
            unpack8(ld16_stream(p.x + rp.row * g.dim + u * 8), xv);
            unpack8(ld16_stream(p.f + rp.row * g.dim + u * 8), fv);
            ada_load8(p.gate, b, t, u * 8, 1.0f, gv);
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gv[i]) * m;
            const uint4 packed = pack8(xv);
            st16_stream(p.x_out + rp.row * g.dim + u * 8, packed);
            unpack8(packed, v[k]);  // the norm sees the rounded residual
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 += v[k][i] * v[k][i];
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
        }
    }
    if (!p.y) return;  // uniform over the launch
    const float r = rsqrtf(group_sum(s2, g.tpr, lds) / static_cast<float>(g.dim) + p.eps);
    if (!rp.active) return;
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
        const int64_t u = rp.lane + static_cast<int64_t>(k) * g.tpr;
        if (u >= g.units) continue;
        float sh[8], sc[8], o[8];
        ada_load8(p.shift, b, t, u * 8, 0.f, sh);
        ada_load8(p.scale, b, t, u * 8, 0.f, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[k][i] * r) * (1.0f + sc[i]) + sh[i];
        st16_stream(p.y + rp.row * g.dim + u * 8, pack8(o));
    }
}

// ------------------------------------------- modulate / residual / head gate --
struct PointRowParams {
    RowGeom g;
    uint16_t *out;
    const uint16_t *x;
    const uint16_t *f;       // residual branch (gated_residual) or logits (head_gate)
    const uint16_t *mask;
    const float *ts;         // x0 timesteps
    int64_t ts_bs, ts_ts;
    Ada a0, a1;              // modulate: shift, scale ; residual: gate
    int64_t heads, head_dim;
    int64_t xbs, xts, xhs;   // head gate: input strides (batch, token, head)
};

// op 0: modulate, 1: gated residual, 2: head gate, 3: x0
template <int OP>
__global__ void __launch_bounds__(kBlock) point_row_kernel(PointRowParams p)
{
    const RowGeom &g = p.g;
    const RowPos rp = row_pos(g);
    if (!rp.active) return;
    const int64_t b = rp.row / g.tokens;
    const int64_t t = rp.row - b * g.tokens;
    const float m = (OP == 1 && p.mask) ? bf16_to_f32(p.mask[b]) : 1.0f;
    float tsv = 0.f;
    if (OP == 3) tsv = p.ts[b * p.ts_bs + t * p.ts_ts];
    for (int64_t u = rp.lane; u < g.units; u += g.tpr) {
        const int64_t off = rp.row * g.dim + u * 8;
        float xv[8], o[8];
        if (OP == 2) {
            const int64_t h = (u * 8) / p.head_dim;
            const int64_t d = u * 8 - h * p.head_dim;
            unpack8(ld16_stream(p.x + b * p.xbs + t * p.xts + h * p.xhs + d), xv);
        } else {
            unpack8(ld16_stream(p.x + off), xv);
        }
        if (OP == 0) {
            float sh[8], sc[8];
            ada_load8(p.a0, b, t, u * 8, 0.f, sh);
            ada_load8(p.a1, b, t, u * 8, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * (1.0f + sc[i]) + sh[i];
        } else if (OP == 1) {
            float fv[8], gv[8];
            unpack8(ld16_stream(p.f + off), fv);
            ada_load8(p.a0, b, t, u * 8, 1.0f, gv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] + (fv[i] * gv[i]) * m;
        } else if (OP == 2) {
            const int64_t h = (u * 8) / p.head_dim;
            const float l = bf16_to_f32(p.f[rp.row * p.heads + h]);
            // 2*sigmoid(l) = 2 / (1 + e^-l)
            const float gate = 2.0f / (1.0f + expf(-l));
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * gate;
        } else {
            float vv[8];
            unpack8(ld16_stream(p.f + off), vv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] - vv[i] * tsv;
        }
        st16_stream(p.out + off, pack8(o));
    }
}

int check_rows(int64_t rows, int64_t tokens, int64_t dim, const char *what)
{
    if (rows < 0 || dim <= 0 || tokens <= 0)
        return fail(LTXK_E_ARG, "%s: bad shape rows=%lld tokens=%lld dim=%lld", what, (long long)rows,
                    (long long)tokens, (long long)dim);
    if (dim % 8) return fail(LTXK_E_ARG, "%s: dim must be a multiple of 8 (got %lld)", what, (long long)dim);
    if (dim > 8 * kBlock * 8) return fail(LTXK_E_ARG, "%s: dim %lld above 16384", what, (long long)dim);
    if (rows % tokens) return fail(LTXK_E_ARG, "%s: rows %lld not a multiple of tokens %lld", what,
                                   (long long)rows, (long long)tokens);
    return LTXK_OK;
}

int check_ptrs(const char *what, std::initializer_list<const void *> ptrs)
{
    for (const void *q : ptrs)
        if (q && !aligned16(q)) return fail(LTXK_E_ALIGN, "%s: buffer %p not 16-byte aligned", what, q);
    return LTXK_OK;
}

int check_ada(const Ada &a, const char *what, const char *name)
{
    if (!ada_aligned(a))
        return fail(LTXK_E_ALIGN, "%s: %s operand not 16-byte aligned (pointers and strides)", what, name);
    return LTXK_OK;
}

template <template <int> class K, typename P>
int launch_maxc(const P &p, hipStream_t s, const char *what)
{
    const int pt = per_thread(p.g);
    const dim3 grid(grid_for(p.g)), block(kBlock);
    if (pt <= 1)
        K<1>::launch(grid, block, s, p);
    else if (pt <= 2)
        K<2>::launch(grid, block, s, p);
    else if (pt <= 4)
        K<4>::launch(grid, block, s, p);
    else
        K<8>::launch(grid, block, s, p);
    return check_launch(what);
}

template <int MAXC>
struct NormModLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const NormModParams &p)
    {
        norm_modulate_kernel<MAXC><<<g, b, 0, s>>>(p);
    }
};

template <int MAXC>
struct AddNormLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const AddNormParams &p)
    {
        add_norm_modulate_kernel<MAXC><<<g, b, 0, s>>>(p);
    }
};

template <int OP>
int launch_point(const PointRowParams &p, hipStream_t s, const char *what)
{
    point_row_kernel<OP><<<dim3(grid_for(p.g)), dim3(kBlock), 0, s>>>(p);
    return check_launch(what);
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int ltxk_norm_modulate(void *y, void *y2, const void *x, int64_t rows, int64_t tokens, int64_t dim,
                                  int norm, float eps, const ltxk_ada *shift, const ltxk_ada *scale,
                                  const ltxk_ada *shift2, const ltxk_ada *scale2, void *stream)
{
    static const char *what = "norm_modulate";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!y || !x) return fail(LTXK_E_ARG, "%s: null x or y", what);
    if (norm != LTXK_NORM_RMS && norm != LTXK_NORM_LAYER) return fail(LTXK_E_ARG, "%s: bad norm kind %d", what, norm);
    if ((rc = check_ptrs(what, {y, y2, x}))) return rc;
    NormModParams p{};
    p.g = make_geom(rows, tokens, dim);
    p.y = static_cast<uint16_t *>(y);
    p.y2 = static_cast<uint16_t *>(y2);
    p.x = static_cast<const uint16_t *>(x);
    p.shift = make_ada(shift);
    p.scale = make_ada(scale);
    p.shift2 = make_ada(shift2);
    p.scale2 = make_ada(scale2);
    p.eps = eps;
    p.layer = norm == LTXK_NORM_LAYER;
    if ((rc = check_ada(p.shift, what, "shift")) || (rc = check_ada(p.scale, what, "scale")) ||
        (rc = check_ada(p.shift2, what, "shift2")) || (rc = check_ada(p.scale2, what, "scale2")))
        return rc;
    return launch_maxc<NormModLaunch>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_add_norm_modulate(void *x_out, void *y, const void *x, const void *f, const ltxk_ada *gate,
                                      const void *mask, int64_t rows, int64_t tokens, int64_t dim, float eps,
                                      const ltxk_ada *shift, const ltxk_ada *scale, void *stream)
{
    static const char *what = "add_norm_modulate";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!x_out || !x || !f) return fail(LTXK_E_ARG, "%s: null x_out, x or f", what);
    if ((rc = check_ptrs(what, {x_out, y, x, f}))) return rc;
    AddNormParams p;
    p.g = make_geom(rows, tokens, dim);
    p.x_out = static_cast<uint16_t *>(x_out);
    p.y = static_cast<uint16_t *>(y);
    p.x = static_cast<const uint16_t *>(x);
    p.f = static_cast<const uint16_t *>(f);
    p.mask = static_cast<const uint16_t *>(mask);
    p.gate = make_ada(gate);
    p.shift = make_ada(shift);
    p.scale = make_ada(scale);
    p.eps = eps;
    if ((rc = check_ada(p.gate, what, "gate")) || (rc = check_ada(p.shift, what, "shift")) ||
        (rc = check_ada(p.scale, what, "scale")))
        return rc;
    return launch_maxc<AddNormLaunch>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_rms_norm(void *y, const void *x, const void *weight, int64_t rows, int64_t dim, float eps,
                             void *stream)
{
    static const char *what = "rms_norm";
    clear_error();
    int rc = check_rows(rows, 1, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!y || !x) return fail(LTXK_E_ARG, "%s: null x or y", what);
    if ((rc = check_ptrs(what, {y, x, weight}))) return rc;
    NormModParams p{};
    p.g = make_geom(rows, 1, dim);
    p.y = static_cast<uint16_t *>(y);
    p.x = static_cast<const uint16_t *>(x);
    p.w = static_cast<const uint16_t *>(weight);
    p.eps = eps;
    return launch_maxc<NormModLaunch>(p, static_cast<hipStream_t>(stream), what);
}

static PointRowParams point_params(void *out, const void *x, const void *f, int64_t rows, int64_t tokens,
                                   int64_t dim)
{
    PointRowParams p{};
    p.g = make_geom(rows, tokens, dim);
    p.out = static_cast<uint16_t *>(out);
    p.x = static_cast<const uint16_t *>(x);
    p.f = static_cast<const uint16_t *>(f);
    return p;
}

extern "C" int ltxk_modulate(void *y, const void *x, int64_t rows, int64_t tokens, int64_t dim,
                             const ltxk_ada *shift, const ltxk_ada *scale, void *stream)
{
    static const char *what = "modulate";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!y || !x) return fail(LTXK_E_ARG, "%s: null x or y", what);
    if ((rc = check_ptrs(what, {y, x}))) return rc;
    PointRowParams p = point_params(y, x, nullptr, rows, tokens, dim);
    p.a0 = make_ada(shift);
    p.a1 = make_ada(scale);
    if ((rc = check_ada(p.a0, what, "shift")) || (rc = check_ada(p.a1, what, "scale"))) return rc;
    return launch_point<0>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_gated_residual(void *out, const void *x, const void *f, const ltxk_ada *gate, const void *mask,
                                   int64_t rows, int64_t tokens, int64_t dim, void *stream)
{
    static const char *what = "gated_residual";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!out || !x || !f) return fail(LTXK_E_ARG, "%s: null out, x or f", what);
    if ((rc = check_ptrs(what, {out, x, f}))) return rc;
    PointRowParams p = point_params(out, x, f, rows, tokens, dim);
    p.mask = static_cast<const uint16_t *>(mask);
    p.a0 = make_ada(gate);
    if ((rc = check_ada(p.a0, what, "gate"))) return rc;
    return launch_point<1>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_head_gate(void *out, const void *x, int64_t x_bstride, int64_t x_tstride, int64_t x_hstride,
                              const void *logits, int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                              void *stream)
{
    static const char *what = "head_gate";
    clear_error();
    if (heads <= 0 || head_dim <= 0 || head_dim % 8)
        return fail(LTXK_E_ARG, "%s: heads must be > 0 and head_dim a multiple of 8 (got %lld, %lld)", what,
                    (long long)heads, (long long)head_dim);
    if (batch < 0) return fail(LTXK_E_ARG, "%s: batch < 0", what);
    const int64_t dim = heads * head_dim;
    const int64_t rows = batch * tokens;
    int rc = check_rows(rows, tokens > 0 ? tokens : 1, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!out || !x || !logits) return fail(LTXK_E_ARG, "%s: null out, x or logits", what);
    if ((rc = check_ptrs(what, {out, x}))) return rc;
    if (x_bstride % 8 || x_tstride % 8 || x_hstride % 8)
        return fail(LTXK_E_ALIGN, "%s: input strides must be multiples of 8 elements", what);
    PointRowParams p = point_params(out, x, logits, rows, tokens, dim);
    p.heads = heads;
    p.head_dim = head_dim;
    p.xbs = x_bstride;
    p.xts = x_tstride;
    p.xhs = x_hstride;
    return launch_point<2>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_x0(void *x0, const void *latent, const void *velocity, const float *ts, int64_t ts_batch_stride,
                       int64_t ts_token_stride, int64_t rows, int64_t tokens, int64_t dim, void *stream)
{
    static const char *what = "x0";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!x0 || !latent || !velocity || !ts) return fail(LTXK_E_ARG, "%s: null pointer", what);
    if ((rc = check_ptrs(what, {x0, latent, velocity}))) return rc;
    PointRowParams p = point_params(x0, latent, velocity, rows, tokens, dim);
    p.ts = ts;
    p.ts_bs = ts_batch_stride;
    p.ts_ts = ts_token_stride;
    return launch_point<3>(p, static_cast<hipStream_t>(stream), what);
}
