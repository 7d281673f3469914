// Row kernels over token-major activations [rows, dim] (bf16):
//   norm_modulate       y(,y2) = norm(x)[*w] * (1 + scale) + shift
//   add_norm_modulate   x' = x + f*gate*mask ; y(,y2) = rms(x') * (1 + scale) + shift
//   modulate            y = x * (1 + scale) + shift
//   gated_residual      out = x + f*gate*mask
//   head_gate           out[r,h,:] = x[r,h,:] * 2*sigmoid(logit[r,h])
//   x0                  x0 = latent - v * ts[b,t]
//
// Two kernel forms:
//   per-row     workgroup w owns RPB = 256/TPR consecutive rows; a row of
//               dim/8 16-byte chunks is owned by TPR threads (the next power
//               of two >= dim/8, at most 256), C chunks each (chunk u = lane +
//               k*TPR, so for every k a wave reads one contiguous 1 KiB span).
//               Any modulation operand (per batch item, per token, indexed).
//   streaming   persistent workgroups (two per CU) over whole rows (TPR 256)
//               when every modulation operand is one row per batch item: the
//               item's modulation is combined into registers once, then rows
//               w, w + G, ... stream with the next row's loads in flight while
//               the current row is reduced and written.
// Activations go through buffer resources (ltxk_common.h): a row group's (or
// row's) byte range, so chunks past the end of a row read zeros and their
// stores are dropped by the hardware, without clamps or predicates; the
// prefetch past a workgroup's last row uses an empty range and reads nothing.
// Modulation rows (table + timestep embedding) are cache-resident and use
// ordinary loads.  Row sums use DPP inside a wave and LDS across the (up to
// four) waves of a row.  fp32 arithmetic, one rounding per output, each
// activation read and written once.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;

struct RowGeom {
    int64_t rows;
    int64_t tokens;  // tokens per batch item: (b, t) = divmod(row, tokens)
    int64_t dim;
    int64_t units;   // dim / 8
};

// This thread's place in a per-row launch: rows [row0, row0 + nrows) belong
// to the workgroup; `row` is the thread's row, clamped into range so operand
// fetches stay valid for the threads of a missing row.
template <int TPR>
struct Group {
    int64_t row0, row;
    int nrows, lrow, lane;
    bool active;
    __device__ explicit Group(int64_t rows)
    {
        constexpr int RPB = kBlock / TPR;
        lrow = threadIdx.x / TPR;
        lane = threadIdx.x % TPR;
        row0 = static_cast<int64_t>(blockIdx.x) * RPB;
        const int64_t left = rows - row0;
        nrows = left < RPB ? static_cast<int>(left) : RPB;
        active = lrow < nrows;
        row = active ? row0 + lrow : rows - 1;
    }
};

// Buffer range over the workgroup's rows of a [rows, dim] bf16 tensor.
__device__ __forceinline__ rsrc_t group_rsrc(const uint16_t *base, const RowGeom &g, int64_t row0, int nrows)
{
    return make_rsrc(base + row0 * g.dim, static_cast<uint32_t>(nrows * g.dim * 2));
}

// Byte offset of chunk k of this thread inside its group's range; kOOB past
// the end of its row (the load returns zeros, the store is dropped).
template <int TPR>
__device__ __forceinline__ uint32_t chunk_off(const RowGeom &g, int lrow, int lane, int k)
{
    const int64_t u = lane + static_cast<int64_t>(k) * TPR;
    return u < g.units ? static_cast<uint32_t>((lrow * g.dim + u * 8) * 2) : kOOB;
}

// Column of chunk k of this thread, clamped into the row (operand fetches).
template <int TPR>
__device__ __forceinline__ int64_t chunk_col(int lane, int k, int64_t units)
{
    const int64_t u = lane + static_cast<int64_t>(k) * TPR;
    return (u < units ? u : units - 1) * 8;
}

template <int TPR>
__device__ __forceinline__ bool chunk_valid(int lane, int k, int64_t units)
{
    return lane + static_cast<int64_t>(k) * TPR < units;
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

template <int TPR, int C>
__global__ void __launch_bounds__(kBlock) norm_modulate_kernel(NormModParams p)
{
    __shared__ float lds[kBlock / 64];
    const RowGeom &g = p.g;
    const Group<TPR> s(g.rows);
    const int64_t b = udiv32(s.row, g.tokens), t = s.row - b * g.tokens;
    // Issue order: modulation rows (cache hits) first, then the activation
    // (HBM); waiting for the former leaves the latter in flight.
    AdaRaw rsh[C], rsc[C];
    uint4 rw[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        rsh[k] = ada_fetch(p.shift, b, t, s.row, d);
        rsc[k] = ada_fetch(p.scale, b, t, s.row, d);
        rw[k] = ld16((p.w ? p.w : g_ada_zeros) + d);
    }
    const rsrc_t rx = group_rsrc(p.x, g, s.row0, s.nrows);
    u32x4 raw[C];
#pragma unroll
    for (int k = 0; k < C; ++k) raw[k] = ldb(rx, chunk_off<TPR>(g, s.lrow, s.lane, k));
    float v[C][8];
#pragma unroll
    for (int k = 0; k < C; ++k) unpack8v(raw[k], v[k]);  // chunks past the row read zeros
    if (p.layer) {
        float s1 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k)
#pragma unroll
            for (int i = 0; i < 8; ++i) s1 += v[k][i];
        const float mean = row_sum<TPR>(s1, lds) / static_cast<float>(g.dim);
#pragma unroll
        for (int k = 0; k < C; ++k)
            if (chunk_valid<TPR>(s.lane, k, g.units))
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] -= mean;
    }
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < C; ++k)
#pragma unroll
        for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
    const float r = rsqrtf(row_sum<TPR>(s2, lds) / static_cast<float>(g.dim) + p.eps);
    if (!s.active) return;
    const rsrc_t ry = group_rsrc(p.y, g, s.row0, s.nrows);
    const rsrc_t ry2 = group_rsrc(p.y2 ? p.y2 : p.y, g, s.row0, p.y2 ? s.nrows : 0);
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!chunk_valid<TPR>(s.lane, k, g.units)) continue;
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        const uint32_t off = chunk_off<TPR>(g, s.lrow, s.lane, k);
        float nv[8], wv[8], sh[8], sc[8], o[8];
        unpack8(rw[k], wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) nv[i] = p.w ? (v[k][i] * r) * wv[i] : v[k][i] * r;
        ada_finish(p.shift, rsh[k], 0.f, sh);
        ada_finish(p.scale, rsc[k], 0.f, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
        stb(ry, off, pack8v(o));
        if (p.y2) {
            ada_load8(p.shift2, b, t, s.row, d, 0.f, sh);
            ada_load8(p.scale2, b, t, s.row, d, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
            stb(ry2, off, pack8v(o));
        }
    }
}

// -------------------------------------------------------- add_norm_modulate --
struct AddNormParams {
    RowGeom g;
    uint16_t *x_out;
    uint16_t *y;
    uint16_t *y2;  // optional second modulation of the same normalised row
    const uint16_t *x;
    const uint16_t *f;  // NULL: the addend is the gate operand itself (x + gate*mask)
    const uint16_t *mask;
    Ada gate, shift, scale, shift2, scale2;
    float eps;
};

template <int TPR, int C>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_kernel(AddNormParams p)
{
    __shared__ float lds[kBlock / 64];
    const RowGeom &g = p.g;
    const Group<TPR> s(g.rows);
    const int64_t b = udiv32(s.row, g.tokens), t = s.row - b * g.tokens;
    AdaRaw rg[C], rsh[C], rsc[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        rg[k] = ada_fetch(p.gate, b, t, s.row, d);
        rsh[k] = ada_fetch(p.shift, b, t, s.row, d);
        rsc[k] = ada_fetch(p.scale, b, t, s.row, d);
    }
    const rsrc_t rx = group_rsrc(p.x, g, s.row0, s.nrows);
    const rsrc_t rf = group_rsrc(p.f ? p.f : p.x, g, s.row0, p.f ? s.nrows : 0);
    u32x4 cx[C], cf[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const uint32_t off = chunk_off<TPR>(g, s.lrow, s.lane, k);
        cx[k] = ldb(rx, off);
        cf[k] = ldb(rf, off);
    }
    const float m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;  // after the streamed loads are issued
    const rsrc_t rxo = group_rsrc(p.x_out, g, s.row0, s.nrows);  // a missing row's offsets lie past the range
    float v[C][8];
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const uint32_t off = chunk_off<TPR>(g, s.lrow, s.lane, k);
        float xv[8], fv[8], gv[8];
        unpack8v(cx[k], xv);
        unpack8v(cf[k], fv);
        ada_finish(p.gate, rg[k], 1.0f, gv);
        if (p.f) {
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gv[i]) * m;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + gv[i] * m;
        }
        const u32x4 packed = pack8v(xv);
        stb(rxo, off, packed);  // dropped past the row and for missing rows
        unpack8v(packed, v[k]);  // the norm sees the rounded residual
        if (!chunk_valid<TPR>(s.lane, k, g.units))
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
    }
    if (!p.y) return;  // uniform over the launch
    const float r = rsqrtf(row_sum<TPR>(s2, lds) / static_cast<float>(g.dim) + p.eps);
    if (!s.active) return;
    const rsrc_t ry = group_rsrc(p.y, g, s.row0, s.nrows);
    const rsrc_t ry2 = group_rsrc(p.y2 ? p.y2 : p.y, g, s.row0, p.y2 ? s.nrows : 0);
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!chunk_valid<TPR>(s.lane, k, g.units)) continue;
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        const uint32_t off = chunk_off<TPR>(g, s.lrow, s.lane, k);
        float sh[8], sc[8], o[8], nv[8];
        ada_finish(p.shift, rsh[k], 0.f, sh);
        ada_finish(p.scale, rsc[k], 0.f, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * r;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
        stb(ry, off, pack8v(o));
        if (p.y2) {
            ada_load8(p.shift2, b, t, s.row, d, 0.f, sh);
            ada_load8(p.scale2, b, t, s.row, d, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
            stb(ry2, off, pack8v(o));
        }
    }
}

// ------------------------------------------- modulate / residual / head gate --
struct PointRowParams {
    RowGeom g;
    uint16_t *out;
    const uint16_t *x;
    const uint16_t *f;       // residual branch (gated_residual), logits (head_gate), velocity (x0)
    const uint16_t *mask;
    const float *ts;         // x0 timesteps
    int64_t ts_bs, ts_ts;
    Ada a0, a1;              // modulate: shift, scale ; residual: gate
    int64_t heads, head_dim;
    int64_t xbs, xts, xhs;   // head gate: input strides (batch, token, head)
    uint32_t xspan;          // head gate: bytes of x the strides can reach
    const uint16_t *v;       // head gate: value rows blended in where the keep-mask is 0
};

// op 0: modulate, 1: gated residual, 2: head gate, 3: x0, 4: head gate with
// perturbation blend (v and its keep-mask set)
template <int OP, int TPR, int C>
__global__ void __launch_bounds__(kBlock) point_row_kernel(PointRowParams p)
{
    const RowGeom &g = p.g;
    const Group<TPR> s(g.rows);
    if (!s.active) return;  // no barriers below
    const int64_t b = udiv32(s.row, g.tokens);
    const int64_t t = s.row - b * g.tokens;
    constexpr bool kGate = OP == 2 || OP == 4;
    AdaRaw r0[C], r1[C];
    float lg[C];
    if (OP == 0 || OP == 1) {
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
            r0[k] = ada_fetch(p.a0, b, t, s.row, d);
            if (OP == 0) r1[k] = ada_fetch(p.a1, b, t, s.row, d);
        }
    }
    if (kGate) {
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const int64_t h = static_cast<uint32_t>(chunk_col<TPR>(s.lane, k, g.units)) /
                              static_cast<uint32_t>(p.head_dim);
            lg[k] = ld_bf16_or_zero(p.f, s.row * p.heads + h);
        }
    }
    const float tsv = OP == 3 ? p.ts[b * p.ts_bs + t * p.ts_ts] : 0.f;
    // the per-batch keep value before the streamed loads, so waiting for it
    // does not wait for them (the blend always has its mask; for the residual
    // a branch on a missing mask measured faster than loading a constant 1)
    const float m = OP == 4 ? bf16_to_f32(p.mask[b]) : ((OP == 1 && p.mask) ? bf16_to_f32(p.mask[b]) : 1.0f);
    const rsrc_t rx = kGate ? make_rsrc(p.x, p.xspan) : group_rsrc(p.x, g, s.row0, s.nrows);
    const rsrc_t rf = group_rsrc(OP == 4 ? p.v : p.f, g, s.row0, (OP == 1 || OP == 3 || OP == 4) ? s.nrows : 0);
    u32x4 rxv[C], rfv[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const uint32_t off = chunk_off<TPR>(g, s.lrow, s.lane, k);
        if (kGate) {
            const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
            const int64_t h = static_cast<uint32_t>(d) / static_cast<uint32_t>(p.head_dim);
            const int64_t e = b * p.xbs + t * p.xts + h * p.xhs + (d - h * p.head_dim);
            rxv[k] = ldb(rx, off == kOOB ? kOOB : static_cast<uint32_t>(e * 2));
        } else {
            rxv[k] = ldb(rx, off);
        }
        if (OP == 1 || OP == 3 || OP == 4) rfv[k] = ldb(rf, off);
    }
    const rsrc_t ro = group_rsrc(p.out, g, s.row0, s.nrows);
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!kGate && !chunk_valid<TPR>(s.lane, k, g.units)) continue;
        float xv[8], o[8];
        unpack8v(rxv[k], xv);
        if (OP == 0) {
            float sh[8], sc[8];
            ada_finish(p.a0, r0[k], 0.f, sh);
            ada_finish(p.a1, r1[k], 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * (1.0f + sc[i]) + sh[i];
        } else if (OP == 1) {
            float fv[8], gv[8];
            unpack8v(rfv[k], fv);
            ada_finish(p.a0, r0[k], 1.0f, gv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] + (fv[i] * gv[i]) * m;
        } else if (kGate) {
            // 2*sigmoid(l) = 2 / (1 + e^-l); no logits: l = 0 from the zero row, gate exactly 1
            const float gate = 2.0f / (1.0f + expf(-lg[k]));
            if (OP == 4) {  // perturbation blend: attn*m + v*(1-m), m one 0/1 keep value per batch item
                float vv[8];
                unpack8v(rfv[k], vv);
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = xv[i] * m + vv[i] * (1.0f - m);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * gate;
        } else {
            float vv[8];
            unpack8v(rfv[k], vv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] - vv[i] * tsv;
        }
        // Head gate: every chunk is computed and the store range drops the
        // ones past the row, because a condition around the computation lets
        // the compiler sink that chunk's loads under it, behind a wait.
        stb(ro, chunk_off<TPR>(g, s.lrow, s.lane, k), pack8v(o));
    }
}

// ----------------------------------------------------- modulate, per block --
// The text-context modulation of every block of a step from one read of the
// context: out[l, row] = round(x[row] * (1 + scale_l) + shift_l), the layer-l
// operands reading their table (and embedding) rows l * stride further on.
struct ModLayersParams {
    uint16_t *out;
    const uint16_t *x;
    int64_t rows, tokens, dim;
    uint32_t units;          // dim / 8
    Ada shift, scale;
    int64_t tab_ls, emb_ls;  // elements between consecutive layers' table / embedding rows
};

// Workgroup w = row + rows * g: row `row` for the layers [g*kLayersPerGroup,
// ...): the x row is loaded once into registers and written out modulated
// once per layer.  With rows a multiple of 8 a row's workgroups land on the
// same XCD (the dispatcher deals workgroups round-robin over the eight), so
// the groups after the first read the x row from that XCD's L2; x loads keep
// the default cache policy for that reason.  Up to 16384 / 8 / 256 = 8 chunks
// of x per thread.
constexpr int kLayersPerGroup = 8;

// EMB_SHARED: every layer reads the same embedding rows (emb_layer_stride 0,
// the step's prompt timestep): they are fetched once, before the layer loop,
// and a layer loads only its table rows.
template <int C, bool EMB_SHARED>
__global__ void __launch_bounds__(kBlock) modulate_layers_kernel(ModLayersParams p, int64_t layers)
{
    const int64_t w = blockIdx.x;
    const int64_t grp = udiv32(w, p.rows);
    const int64_t row = w - grp * p.rows;
    const int64_t b = udiv32(row, p.tokens);
    const int64_t t = row - b * p.tokens;
    const uint32_t nb = static_cast<uint32_t>(p.dim * 2);
    const rsrc_t rx = make_rsrc(p.x + row * p.dim, nb);
    float xv[C][8];
    uint4 esh[C], esc[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const uint32_t u = threadIdx.x + k * kBlock;
        // past the row: the range returns zeros and the stores below are dropped
        unpack8v(__builtin_amdgcn_raw_buffer_load_b128(rx, u < p.units ? u * 16 : kOOB, 0, 0), xv[k]);
        if constexpr (EMB_SHARED) {
            const int64_t d = u < p.units ? static_cast<int64_t>(u) * 8 : 0;
            esh[k] = ada_fetch(p.shift, b, t, row, d).emb;
            esc[k] = ada_fetch(p.scale, b, t, row, d).emb;
        }
    }
    const int64_t l0 = grp * kLayersPerGroup;
    const int64_t l1 = l0 + kLayersPerGroup < layers ? l0 + kLayersPerGroup : layers;
    for (int64_t layer = l0; layer < l1; ++layer) {
        Ada sh = p.shift, sc = p.scale;
        if (sh.tab) sh.tab += layer * p.tab_ls;
        if (sh.emb) sh.emb += layer * p.emb_ls;
        if (sc.tab) sc.tab += layer * p.tab_ls;
        if (sc.emb) sc.emb += layer * p.emb_ls;
        const rsrc_t ro = make_rsrc(p.out + (layer * p.rows + row) * p.dim, nb);
        AdaRaw r0[C], r1[C];
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const uint32_t u = threadIdx.x + k * kBlock;
            const int64_t d = u < p.units ? static_cast<int64_t>(u) * 8 : 0;
            if constexpr (EMB_SHARED) {
                r0[k] = AdaRaw{ld16((sh.tab ? sh.tab : g_ada_zeros) + d), esh[k]};
                r1[k] = AdaRaw{ld16((sc.tab ? sc.tab : g_ada_zeros) + d), esc[k]};
            } else {
                r0[k] = ada_fetch(sh, b, t, row, d);
                r1[k] = ada_fetch(sc, b, t, row, d);
            }
        }
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const uint32_t u = threadIdx.x + k * kBlock;
            float shv[8], scv[8], o[8];
            ada_finish(sh, r0[k], 0.f, shv);
            ada_finish(sc, r1[k], 0.f, scv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[k][i] * (1.0f + scv[i]) + shv[i];
            // non-temporal, not write-through: this kernel is almost all writes,
            // and for it the streaming store measured faster (79-89 against
            // 97-99 us for the 48 x [1024,4096] outputs)
            stb_stream(ro, u < p.units ? u * 16 : kOOB, pack8v(o));
        }
    }
}

// Tiled form, for operands whose value depends on the layer and the batch item
// only (no index, no per-token embedding rows: the text-context modulation's
// prompt table + prompt timestep).  Workgroup w = row block rb of the layers
// [lg*LG, lg*LG + LG): the LG layers' (1 + scale, shift) of the block's batch
// item are computed once into registers (again only where the block crosses
// into another batch item), then each row is loaded once (the next row's
// load in flight) and written out LG times.  A per-row recomputation of the
// modulation (a bf16 rounding per element and layer) made the per-row form
// ALU-bound.
// Tile of the tiled form: rows per workgroup and layers per workgroup (for
// rows of at most 4096).  Measured on 48 x [1024, 4096] (µs, two boxes):
// 16 rows x 2 layers 75.3, 8 x 2 73.3, 4 x 2 71.8, 16 x 1 73.7, 8 x 1
// 70.7-73.6, 4 x 1 78.1, 2 x 1 97.6, 1 x 1 147.1, 16 x 4 78.1; streaming
// stores 78.2 (16 x 2).
#ifndef LTXK_MODL_ROWS
#define LTXK_MODL_ROWS 8
#endif
#ifndef LTXK_MODL_LG
#define LTXK_MODL_LG 1
#endif
#ifndef LTXK_MODL_STORE
#define LTXK_MODL_STORE 16
#endif
constexpr int kModRows = LTXK_MODL_ROWS;  // rows per workgroup of the tiled form

template <int C, int LG>
__global__ void __launch_bounds__(kBlock) modulate_layers_tiled_kernel(ModLayersParams p, int64_t layers,
                                                                       int64_t row_blocks)
{
    const int64_t w = blockIdx.x;
    const int64_t lg = udiv32(w, row_blocks);
    const int64_t rb = w - lg * row_blocks;
    const int64_t r0 = rb * kModRows;
    const int64_t r1 = r0 + kModRows < p.rows ? r0 + kModRows : p.rows;
    const uint32_t nb = static_cast<uint32_t>(p.dim * 2);
    uint32_t off[C];
    int64_t col[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const uint32_t u = threadIdx.x + k * kBlock;
        off[k] = u < p.units ? u * 16 : kOOB;  // past the row: zeros in, stores dropped
        col[k] = u < p.units ? static_cast<int64_t>(u) * 8 : 0;
    }
    float one_sc[LG][C][8], shv[LG][C][8];
    int64_t cur_b = -1;
    u32x4 nxt[C];
    {
        const rsrc_t rx = make_rsrc(p.x + r0 * p.dim, nb);
#pragma unroll
        for (int k = 0; k < C; ++k) nxt[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off[k], 0, 0);
    }
    for (int64_t row = r0; row < r1; ++row) {
        u32x4 cur[C];
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = nxt[k];
        {
            // the next row of the block (past its end: an empty range, zeros)
            const rsrc_t rx = make_rsrc(p.x + (row + 1) * p.dim, row + 1 < r1 ? nb : 0u);
#pragma unroll
            for (int k = 0; k < C; ++k) nxt[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, off[k], 0, 0);
        }
        const int64_t b = udiv32(row, p.tokens);
        if (b != cur_b) {  // uniform: the same row for the whole workgroup
#pragma unroll
            for (int j = 0; j < LG; ++j) {
                const int64_t lj = lg * LG + j < layers ? lg * LG + j : layers - 1;
                Ada sh = p.shift, sc = p.scale;
                if (sh.tab) sh.tab += lj * p.tab_ls;
                if (sh.emb) sh.emb += lj * p.emb_ls;
                if (sc.tab) sc.tab += lj * p.tab_ls;
                if (sc.emb) sc.emb += lj * p.emb_ls;
#pragma unroll
                for (int k = 0; k < C; ++k) {
                    float scv[8];
                    ada_load8(sh, b, 0, row, col[k], 0.f, shv[j][k]);
                    ada_load8(sc, b, 0, row, col[k], 0.f, scv);
#pragma unroll
                    for (int i = 0; i < 8; ++i) one_sc[j][k][i] = 1.0f + scv[i];
                }
            }
            cur_b = b;
        }
        float xv[C][8];
#pragma unroll
        for (int k = 0; k < C; ++k) unpack8v(cur[k], xv[k]);
#pragma unroll
        for (int j = 0; j < LG; ++j) {
            const int64_t layer = lg * LG + j;
            const rsrc_t ro = make_rsrc(p.out + (layer * p.rows + row) * p.dim, layer < layers ? nb : 0u);
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = xv[k][i] * one_sc[j][k][i] + shv[j][k][i];
                // write-through, as the other kernels (measured 75.5-76 us here
                // against 78.2 for streaming stores and 79.3 for write-back)
                __builtin_amdgcn_raw_buffer_store_b128(pack8v(o), ro, off[k], 0, LTXK_MODL_STORE);
            }
        }
    }
}

template <int C>
__device__ __forceinline__ void item_mod(const Ada &a, int64_t b, float absent, int lane, int64_t units,
                                         float (&out)[C][8])
{
    const uint16_t *tp = a.tab ? a.tab : g_ada_zeros;
    const uint16_t *ep = a.emb ? a.emb + b * a.bs : g_ada_zeros;
    u32x4 tr[C], er[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t col = chunk_col<kBlock>(lane, k, units);
        tr[k] = *reinterpret_cast<const u32x4 *>(tp + col);
        er[k] = *reinterpret_cast<const u32x4 *>(ep + col);
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
        float tv[8], ev[8];
        unpack8v(tr[k], tv);
        unpack8v(er[k], ev);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[k][i] = (absent != 0.f && !a.kind) ? absent : bf16_to_f32(f32_to_bf16(tv[i] + ev[i]));
    }
}

// Sum of v over the workgroup; partials double-buffered by the row parity so
// one barrier per row suffices.
__device__ __forceinline__ float block_sum(float v, float (&lds)[2][kBlock / 64], int parity)
{
    const float w = wave_sum64(v);
    if ((threadIdx.x & 63) == 0) lds[parity][threadIdx.x >> 6] = w;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kBlock / 64; ++q) tot += lds[parity][q];
    return tot;
}

// First row of batch item [lo, hi) that workgroup w handles when the rows of
// every item are dealt out as r = w, w + G, ... over the whole tensor.
__device__ __forceinline__ int first_row(int lo, int w, int G)
{
    return lo > w ? w + ((lo - w + G - 1) / G) * G : w;
}

// Register stages of the streaming kernels: each holds one row's loads, so
// a workgroup has kRowStages rows in flight while it reduces and writes the
// current one.  A stage is refilled as soon as its row has been unpacked
// (the stages are used in turn, so no register is copied from a load still
// in flight).
#ifndef LTXK_ROW_STAGES
#define LTXK_ROW_STAGES 1
#endif
constexpr int kRowStages = LTXK_ROW_STAGES;

// Loads row `r` of a [rows, dim] tensor into C registers (one 16-byte chunk
// per kBlock lanes); an empty range (`ok` false) reads zeros and no memory.
template <int C>
__device__ __forceinline__ void row_load(u32x4 (&v)[C], const uint16_t *base, int r, bool ok, int64_t dim,
                                         uint32_t rbytes, int lane)
{
    const rsrc_t rs = make_rsrc(base + static_cast<int64_t>(r) * dim, ok ? rbytes : 0u);
#pragma unroll
    for (int k = 0; k < C; ++k) v[k] = ldb(rs, (lane + k * kBlock) * 16u);
}

// norm_modulate over rows owned by a whole workgroup with one modulation row
// per batch item: workgroup w walks rows w, w + G, ... of each item with
// kRowStages rows in flight.  The first rows' loads are issued before the
// item's modulation rows are fetched and combined, so the two latencies
// overlap.
template <int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) norm_modulate_stream_kernel(NormModParams p)
{
    __shared__ float lds[2][kBlock / 64];
    const int lane = threadIdx.x;
    // rows * dim * 2 bytes fit in device memory, so rows < 2^26 and row
    // indices plus the grid stay far inside int.
    const int rows = static_cast<int>(p.g.rows), tokens = static_cast<int>(p.g.tokens);
    const int G = static_cast<int>(gridDim.x), w = static_cast<int>(blockIdx.x);
    const int64_t dim = p.g.dim;
    const uint32_t rbytes = static_cast<uint32_t>(dim * 2);
    int parity = 0;
    for (int lo = 0; lo < rows; lo += tokens) {
        const int hi = lo + tokens;
        int r = first_row(lo, w, G);
        if (r >= hi) continue;  // uniform over the workgroup
        const int64_t b = lo / tokens;
        u32x4 st[kRowStages][C];
#pragma unroll
        for (int j = 0; j < kRowStages; ++j) row_load<C>(st[j], p.x, r + j * G, r + j * G < hi, dim, rbytes, lane);
        float sh[C][8], sc[C][8], sh2[DUAL ? C : 1][8], sc2[DUAL ? C : 1][8];
        item_mod<C>(p.shift, b, 0.f, lane, p.g.units, sh);
        item_mod<C>(p.scale, b, 0.f, lane, p.g.units, sc);
        if constexpr (DUAL) {
            item_mod<C>(p.shift2, b, 0.f, lane, p.g.units, sh2);
            item_mod<C>(p.scale2, b, 0.f, lane, p.g.units, sc2);
        }
        // row r from stage st: unpack, refill the stage with row r + kRowStages*G,
        // reduce, write; false after the item's last row of this workgroup
        auto step = [&](u32x4 (&cur)[C]) {
            float v[C][8];
            float s2 = 0.f;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                unpack8v(cur[k], v[k]);  // chunks past the row read zeros
#pragma unroll
                for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
            }
            const int ra = r + kRowStages * G;
            row_load<C>(cur, p.x, ra < hi ? ra : r, ra < hi, dim, rbytes, lane);
            const float rs = rsqrtf(block_sum(s2, lds, parity) / static_cast<float>(dim) + p.eps);
            parity ^= 1;
            const rsrc_t ry = make_rsrc(p.y + static_cast<int64_t>(r) * dim, rbytes);
            const rsrc_t ry2 = make_rsrc((DUAL ? p.y2 : p.y) + static_cast<int64_t>(r) * dim, DUAL ? rbytes : 0u);
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float nv[8], o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[k][i]) + sh[k][i];
                stb(ry, (lane + k * kBlock) * 16u, pack8v(o));
                if constexpr (DUAL) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2[k][i]) + sh2[k][i];
                    stb(ry2, (lane + k * kBlock) * 16u, pack8v(o));
                }
            }
            r += G;
            return r < hi;
        };
        bool more = true;
        while (more) {
#pragma unroll
            for (int j = 0; j < kRowStages; ++j)
                if (more) more = step(st[j]);
        }
    }
}

// add_norm_modulate in the streaming form: x_out = x + f * gate * mask, then
// the norm and modulation(s) of the rounded x_out when y is set.  Same walk
// and stages as norm_modulate_stream_kernel, each stage holding a row of x
// and of f.
template <int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_stream_kernel(AddNormParams p)
{
    __shared__ float lds[2][kBlock / 64];
    const int lane = threadIdx.x;
    const int rows = static_cast<int>(p.g.rows), tokens = static_cast<int>(p.g.tokens);
    const int G = static_cast<int>(gridDim.x), w = static_cast<int>(blockIdx.x);
    const int64_t dim = p.g.dim;
    const uint32_t rbytes = static_cast<uint32_t>(dim * 2);
    int parity = 0;
    for (int lo = 0; lo < rows; lo += tokens) {
        const int hi = lo + tokens;
        int r = first_row(lo, w, G);
        if (r >= hi) continue;
        const int64_t b = lo / tokens;
        u32x4 sx[kRowStages][C], sf[kRowStages][C];
#pragma unroll
        for (int j = 0; j < kRowStages; ++j) {
            row_load<C>(sx[j], p.x, r + j * G, r + j * G < hi, dim, rbytes, lane);
            row_load<C>(sf[j], p.f, r + j * G, r + j * G < hi, dim, rbytes, lane);
        }
        float gt[C][8], sh[C][8], sc[C][8], sh2[DUAL ? C : 1][8], sc2[DUAL ? C : 1][8];
        item_mod<C>(p.gate, b, 1.0f, lane, p.g.units, gt);
        item_mod<C>(p.shift, b, 0.f, lane, p.g.units, sh);
        item_mod<C>(p.scale, b, 0.f, lane, p.g.units, sc);
        if constexpr (DUAL) {
            item_mod<C>(p.shift2, b, 0.f, lane, p.g.units, sh2);
            item_mod<C>(p.scale2, b, 0.f, lane, p.g.units, sc2);
        }
        const float m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;
        auto step = [&](u32x4 (&cx)[C], u32x4 (&cf)[C]) {
            float v[C][8];
            u32x4 packed[C];
            float s2 = 0.f;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float xv[8], fv[8];
                unpack8v(cx[k], xv);
                unpack8v(cf[k], fv);
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gt[k][i]) * m;
                packed[k] = pack8v(xv);
                unpack8v(packed[k], v[k]);  // the norm sees the rounded residual (zeros past the row)
#pragma unroll
                for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
            }
            const int ra = r + kRowStages * G;
            row_load<C>(cx, p.x, ra < hi ? ra : r, ra < hi, dim, rbytes, lane);
            row_load<C>(cf, p.f, ra < hi ? ra : r, ra < hi, dim, rbytes, lane);
            const rsrc_t rxo = make_rsrc(p.x_out + static_cast<int64_t>(r) * dim, rbytes);
#pragma unroll
            for (int k = 0; k < C; ++k) stb(rxo, (lane + k * kBlock) * 16u, packed[k]);
            if (p.y) {  // uniform over the launch
                const float rs = rsqrtf(block_sum(s2, lds, parity) / static_cast<float>(dim) + p.eps);
                parity ^= 1;
                const rsrc_t ry = make_rsrc(p.y + static_cast<int64_t>(r) * dim, rbytes);
                const rsrc_t ry2 = make_rsrc((DUAL ? p.y2 : p.y) + static_cast<int64_t>(r) * dim, DUAL ? rbytes : 0u);
#pragma unroll
                for (int k = 0; k < C; ++k) {
                    float nv[8], o[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[k][i]) + sh[k][i];
                    // streaming stores for the modulated outputs (x_out, which
                    // the next residual reads back, is written through): 32.8 /
                    // 41.6 us for one / two outputs against 36.6 / 47.3 with
                    // write-through ones; the 48-block chain 16.68-16.80 against
                    // 16.65-16.74 ms (graph replays 16.53-16.69 against
                    // 16.48-16.61) and the full denoise step unchanged within its
                    // spread (200.7-203.4 against 200.4-202.0 ms).  x_out
                    // streamed as well: the chain 17.69 ms.
                    stb_stream(ry, (lane + k * kBlock) * 16u, pack8v(o));
                    if constexpr (DUAL) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2[k][i]) + sh2[k][i];
                        stb_stream(ry2, (lane + k * kBlock) * 16u, pack8v(o));
                    }
                }
            }
            r += G;
            return r < hi;
        };
        bool more = true;
        while (more) {
#pragma unroll
            for (int j = 0; j < kRowStages; ++j)
                if (more) more = step(sx[j], sf[j]);
        }
    }
}

// ------------------------------------------------------------- wave rows --
// norm_modulate with one wave per row, for rows of up to 4096 elements with
// one modulation row per batch item (the model's broadcast AdaLN).  Lane l owns
// the 16-byte chunks l + 64k (k < CW), so every load and store instruction
// covers one contiguous 1 KiB span, and a row's sum is one wave reduction:
// the row loop has no barrier.  Persistent waves walk rows w, w + NW, ... of
// each batch item with two rows loaded ahead (all of a [6144, 4096] activation
// is in flight from the start at 16 waves per CU); as each 16-byte chunk of a
// row's outputs is stored, the register that held it is refilled with the
// same chunk of the wave's next row.  The item's modulation rows are combined
// (table + embedding, rounded) once per workgroup into LDS, which every wave
// reads per row.
//
// Measured on the headline [6144, 4096] with buffers rotating past the MALL
// (us): this form 17.4-17.6; the workgroup-per-row streaming form above 19.4.
// Variants: the modulation in registers 18.1; refill after the whole row
// instead of per chunk 17.5; 512- or 1024-thread workgroups 18.6 / 20.7; 2
// workgroups per CU with 2 stages 21.0 (a wave's third row waits for its
// first); one row per wave (5-8 workgroups per CU) 24-26.  Issuing a row's
// eight loads back to back is slower than spacing them by two s_nop 7 each
// (18.1 against 17.4-17.5; one nop 17.7, three 17.7, six 18.1; nops between
// stores make it slower: 18.2-19.1).  Streaming (nt) stores instead of
// write-through: 17.29-17.32 against 17.44-17.48 us (the workgroup-per-row
// form was slower with them); the 48-block chain and the full denoise step
// unchanged within their run-to-run spread.
// The residual forms (add_norm_modulate) keep the workgroup-per-row kernel:
// in this form (x and f held per stage; two or three workgroups per CU) they
// measured 36.1 / 45.5 us alone against 36.5 / 47.4 (one / two outputs), but
// the 48-block chain with them ran 17.75 against 17.11-17.14 ms (in the
// chain their inputs are partly cache-resident, and the audio stream's
// kernels share the CUs, which the workgroup-per-row form tolerates better).
constexpr int kWaveBlock = 256;

constexpr int kWaveStages = 2;

// Launch shape and memory-op schedule of the wave-row kernel.
struct NormTune {
    static constexpr int per_cu = 4;            // workgroups per CU
    static constexpr bool chunk_refill = true;  // refill per chunk, as it is stored
    static constexpr int load_nops = 2;         // s_nop 7 after each activation load
};

template <int N>
__device__ __forceinline__ void load_spacing()
{
#pragma unroll
    for (int q = 0; q < N; ++q) asm volatile("s_nop 7");
}

// Chunk u of one modulation operand of batch item b: round(tab + emb) (an
// absent part reads zeros).
__device__ __forceinline__ u32x4 mod_chunk(const Ada &a, int64_t b, int64_t u)
{
    const uint16_t *tp = a.tab ? a.tab + u * 8 : g_ada_zeros;
    const uint16_t *ep = a.emb ? a.emb + b * a.bs + u * 8 : g_ada_zeros;
    float tv[8], ev[8], o[8];
    unpack8v(*reinterpret_cast<const u32x4 *>(tp), tv);
    unpack8v(*reinterpret_cast<const u32x4 *>(ep), ev);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = tv[i] + ev[i];
    return pack8v(o);
}

// Operands a0..a4 (those of index < NM) of batch item b into lmod[m][u]
// (u < CW*64; chunks past the row hold zeros).  Every thread of the
// workgroup calls it; it ends with a barrier.
template <int NM, int CW>
__device__ __forceinline__ void stage_mod(u32x4 (&lmod)[NM][CW * 64], const Ada &a0, const Ada &a1,
                                          const Ada &a2, const Ada &a3, const Ada &a4, int64_t b, int64_t units)
{
    for (int u = threadIdx.x; u < CW * 64; u += kWaveBlock) {
        const bool ok = u < units;
        const int64_t uu = ok ? u : 0;
        constexpr u32x4 z = {0, 0, 0, 0};
        lmod[0][u] = ok ? mod_chunk(a0, b, uu) : z;
        if constexpr (NM > 1) lmod[1][u] = ok ? mod_chunk(a1, b, uu) : z;
        if constexpr (NM > 2) lmod[2][u] = ok ? mod_chunk(a2, b, uu) : z;
        if constexpr (NM > 3) lmod[3][u] = ok ? mod_chunk(a3, b, uu) : z;
        if constexpr (NM > 4) lmod[4][u] = ok ? mod_chunk(a4, b, uu) : z;
    }
    __syncthreads();
}

// Buffer resource over row r of a [rows, dim] tensor, or an empty range (reads
// zeros and no memory, drops stores) when `ok` is false.
__device__ __forceinline__ rsrc_t row_rsrc(const uint16_t *base, int r, bool ok, int64_t dim, uint32_t rbytes)
{
    return make_rsrc(base + static_cast<int64_t>(ok ? r : 0) * dim, ok ? rbytes : 0u);
}

// Chunk lane + 64k of a row into v[k].
template <int CW, int NOPS>
__device__ __forceinline__ void wave_row_load(u32x4 (&v)[CW], rsrc_t rs, int lane)
{
#pragma unroll
    for (int k = 0; k < CW; ++k) {
        v[k] = ldb(rs, (lane + k * 64) * 16u);
        load_spacing<NOPS>();
    }
}

// This wave's index in the launch: wave-uniform (read from lane 0), so rows
// and buffer resources stay in scalar registers.
__device__ __forceinline__ int wave_index()
{
    return static_cast<int>(blockIdx.x) * (kWaveBlock / 64) +
           __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// y (, y2) = rms(x) * (1 + scale) + shift, one wave per row.
template <int CW, bool DUAL>
__global__ void __launch_bounds__(kWaveBlock, NormTune::per_cu) norm_modulate_wave_kernel(NormModParams p)
{
    using T = NormTune;
    constexpr int NM = DUAL ? 4 : 2;
    __shared__ u32x4 lmod[NM][CW * 64];
    const int lane = threadIdx.x & 63;
    // rows * dim * 2 bytes fit in device memory: rows < 2^26
    const int rows = static_cast<int>(p.g.rows), tokens = static_cast<int>(p.g.tokens);
    const int NW = static_cast<int>(gridDim.x) * (kWaveBlock / 64);
    const int w = wave_index();
    const int64_t dim = p.g.dim;
    const uint32_t rbytes = static_cast<uint32_t>(dim * 2);
    for (int lo = 0; lo < rows; lo += tokens) {
        const int hi = lo + tokens;
        int r = first_row(lo, w, NW);
        u32x4 st[kWaveStages][CW];
#pragma unroll
        for (int j = 0; j < kWaveStages; ++j)
            wave_row_load<CW, T::load_nops>(st[j], row_rsrc(p.x, r + j * NW, r + j * NW < hi, dim, rbytes), lane);
        stage_mod<NM, CW>(lmod, p.shift, p.scale, p.shift2, p.scale2, p.scale2, lo / tokens, p.g.units);
        auto step = [&](u32x4 (&cur)[CW]) {
            float s2 = 0.f;
#pragma unroll
            for (int k = 0; k < CW; ++k) {
                float v[8];
                unpack8v(cur[k], v);  // chunks past the row read zeros
#pragma unroll
                for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[i], v[i], s2);
            }
            const float rs = rsqrtf(wave_sum64(s2) / static_cast<float>(dim) + p.eps);
            const rsrc_t ry = make_rsrc(p.y + static_cast<int64_t>(r) * dim, rbytes);
            const rsrc_t ry2 = make_rsrc((DUAL ? p.y2 : p.y) + static_cast<int64_t>(r) * dim, DUAL ? rbytes : 0u);
            const int ra = r + kWaveStages * NW;
            const rsrc_t rn = row_rsrc(p.x, ra, ra < hi, dim, rbytes);
#pragma unroll
            for (int k = 0; k < CW; ++k) {
                // the row stays packed between its two uses (unpacking it once
                // for both would hold 8 * CW more registers)
                asm volatile("" : "+v"(cur[k]));
                float v[8], sh[8], sc[8], nv[8], o[8];
                unpack8v(cur[k], v);
                unpack8v(lmod[0][lane + k * 64], sh);
                unpack8v(lmod[1][lane + k * 64], sc);
#pragma unroll
                for (int i = 0; i < 8; ++i) nv[i] = v[i] * rs;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
                stb_stream(ry, (lane + k * 64) * 16u, pack8v(o));
                if constexpr (DUAL) {
                    unpack8v(lmod[2][lane + k * 64], sh);
                    unpack8v(lmod[3][lane + k * 64], sc);
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
                    stb_stream(ry2, (lane + k * 64) * 16u, pack8v(o));
                }
                if constexpr (T::chunk_refill) {
                    cur[k] = ldb(rn, (lane + k * 64) * 16u);
                    load_spacing<T::load_nops>();
                }
            }
            if constexpr (!T::chunk_refill) wave_row_load<CW, T::load_nops>(cur, rn, lane);
            r += NW;
            return r < hi;
        };
        bool more = r < hi;
        while (more) {
#pragma unroll
            for (int j = 0; j < kWaveStages; ++j)
                if (more) more = step(st[j]);
        }
        __syncthreads();  // every wave is done with this item's modulation
    }
}

// ----------------------------------------------------------------- launch --
#ifndef LTXK_ROWS_PER_CU
#define LTXK_ROWS_PER_CU 2
#endif
constexpr int kStreamPerCU = LTXK_ROWS_PER_CU;  // workgroups per CU of the streaming kernels
constexpr int kStreamItems = 64; // most batch items a streaming launch walks
constexpr int kStreamMaxC = 4;   // streaming form up to dim 8192 (register budget)

struct Choice {
    int tpr;
    int c;
};

inline Choice choose(int64_t units)
{
    // TPR = min(next power of two >= units, 256) threads per row; C chunks each.
    int tpr = 8;
    while (tpr < units && tpr < kBlock) tpr <<= 1;
    const int64_t c = (units + tpr - 1) / tpr;
    return {tpr, c <= 1 ? 1 : c <= 2 ? 2 : c <= 4 ? 4 : 8};
}

inline unsigned grid_for(int64_t rows, int tpr)
{
    return static_cast<unsigned>((rows + (kBlock / tpr) - 1) / (kBlock / tpr));
}

// Workgroups of a streaming launch: kStreamPerCU per compute unit (cached per
// device), never more than there are rows.
unsigned stream_grid(int64_t rows)
{
    const int64_t blocks = static_cast<int64_t>(device_cus()) * kStreamPerCU;
    return static_cast<unsigned>(rows < blocks ? rows : blocks);
}

// Workgroups of a wave-row launch: per_cu per compute unit, at most one wave
// per row.
unsigned wave_grid(int64_t rows, int per_cu)
{
    const int64_t full = static_cast<int64_t>(stream_grid(int64_t{1} << 30)) / kStreamPerCU * per_cu;
    const int64_t need = (rows + kWaveBlock / 64 - 1) / (kWaveBlock / 64);
    return static_cast<unsigned>(need < full ? need : full);
}

// True when every operand is one row per batch item (or absent).
inline bool broadcast_only(std::initializer_list<const Ada *> ops)
{
    for (const Ada *a : ops)
        if (a->emb && (a->ts != 0 || a->idx)) return false;
    return true;
}

// The streaming form applies: rows owned by a whole workgroup, at most
// kStreamMaxC chunks per thread, few batch items, broadcast modulation.
inline bool streaming(const RowGeom &g, const Choice &c)
{
    return c.tpr == kBlock && c.c <= kStreamMaxC && g.rows / g.tokens <= kStreamItems;
}

// Instantiates kernel K<TPR, C> for the chosen geometry.
template <template <int, int> class K, typename P>
int dispatch(const P &p, hipStream_t s, const char *what)
{
    const Choice c = choose(p.g.units);
    const dim3 block(kBlock);
    const dim3 grid(grid_for(p.g.rows, c.tpr));
#define LTXK_CASE(T, CC) \
    if (c.tpr == T && c.c == CC) { K<T, CC>::launch(grid, block, s, p); return check_launch(what); }
    LTXK_CASE(8, 1)
    LTXK_CASE(16, 1)
    LTXK_CASE(32, 1)
    LTXK_CASE(64, 1)
    LTXK_CASE(128, 1)
    LTXK_CASE(256, 1)
    LTXK_CASE(256, 2)
    LTXK_CASE(256, 4)
    LTXK_CASE(256, 8)
#undef LTXK_CASE
    return fail(LTXK_E_ARG, "%s: no kernel geometry for dim %lld", what, (long long)(p.g.units * 8));
}

// Launchers: the wave-row kernel for broadcast modulation of rows up to 4096
// elements (CW = 4 or 8 chunks a lane), the workgroup-row streaming kernel
// for wider rows, the per-row kernel otherwise (per-token or indexed
// timestep embeddings, layer norm, weighted norm, many batch items).
template <int TPR, int C>
struct NormModLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const NormModParams &p)
    {
        if constexpr (TPR == kBlock && C <= kStreamMaxC) {
            if (!p.layer && !p.w && streaming(p.g, Choice{TPR, C}) &&
                broadcast_only({&p.shift, &p.scale, &p.shift2, &p.scale2})) {
                if constexpr (C <= 2) {
                    constexpr int CW = 4 * C;
                    auto k = p.y2 ? norm_modulate_wave_kernel<CW, true> : norm_modulate_wave_kernel<CW, false>;
                    k<<<dim3(wave_grid(p.g.rows, NormTune::per_cu)), dim3(kWaveBlock), 0, s>>>(p);
                } else {
                    auto k = p.y2 ? norm_modulate_stream_kernel<C, true> : norm_modulate_stream_kernel<C, false>;
                    k<<<dim3(stream_grid(p.g.rows)), b, 0, s>>>(p);
                }
                return;
            }
        }
        norm_modulate_kernel<TPR, C><<<g, b, 0, s>>>(p);
    }
};

template <int TPR, int C>
struct AddNormLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const AddNormParams &p)
    {
        if constexpr (TPR == kBlock && C <= kStreamMaxC) {
            if (p.f && streaming(p.g, Choice{TPR, C}) &&
                broadcast_only({&p.gate, &p.shift, &p.scale, &p.shift2, &p.scale2})) {
                auto k = (p.y2 && p.y) ? add_norm_modulate_stream_kernel<C, true>
                                       : add_norm_modulate_stream_kernel<C, false>;
                k<<<dim3(stream_grid(p.g.rows)), b, 0, s>>>(p);
                return;
            }
        }
        add_norm_modulate_kernel<TPR, C><<<g, b, 0, s>>>(p);
    }
};

template <int OP>
struct PointLaunch {
    template <int TPR, int C>
    struct K {
        static void launch(dim3 g, dim3 b, hipStream_t s, const PointRowParams &p)
        {
            point_row_kernel<OP, TPR, C><<<g, b, 0, s>>>(p);
        }
    };
};

int check_rows(int64_t rows, int64_t tokens, int64_t dim, const char *what)
{
    if (rows < 0 || dim <= 0 || tokens <= 0)
        return fail(LTXK_E_ARG, "%s: bad shape rows=%lld tokens=%lld dim=%lld", what, (long long)rows,
                    (long long)tokens, (long long)dim);
    if (dim % 8) return fail(LTXK_E_ARG, "%s: dim must be a multiple of 8 (got %lld)", what, (long long)dim);
    if (dim > 16384) return fail(LTXK_E_ARG, "%s: dim %lld above 16384", what, (long long)dim);
    if (rows % tokens) return fail(LTXK_E_ARG, "%s: rows %lld not a multiple of tokens %lld", what,
                                   (long long)rows, (long long)tokens);
    if (rows > 0x7fffffff) return fail(LTXK_E_ARG, "%s: too many rows", what);
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
    if (a.idx && (a.idx_rows == 0 || a.idx_rows > 0x7fffffffu))
        return fail(LTXK_E_ARG, "%s: %s operand has an index but emb_rows %u is not in [1, 2^31)", what, name,
                    a.idx_rows);
    return LTXK_OK;
}

RowGeom make_geom(int64_t rows, int64_t tokens, int64_t dim)
{
    return RowGeom{rows, tokens, dim, dim / 8};
}

PointRowParams point_params(void *out, const void *x, const void *f, int64_t rows, int64_t tokens, int64_t dim)
{
    PointRowParams p{};
    p.g = make_geom(rows, tokens, dim);
    p.out = static_cast<uint16_t *>(out);
    p.x = static_cast<const uint16_t *>(x);
    p.f = static_cast<const uint16_t *>(f);
    return p;
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
    return dispatch<NormModLaunch>(p, static_cast<hipStream_t>(stream), what);
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
    return dispatch<NormModLaunch>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_add_norm_modulate(void *x_out, void *y, void *y2, const void *x, const void *f,
                                      const ltxk_ada *gate, const void *mask, int64_t rows, int64_t tokens,
                                      int64_t dim, float eps, const ltxk_ada *shift, const ltxk_ada *scale,
                                      const ltxk_ada *shift2, const ltxk_ada *scale2, void *stream)
{
    static const char *what = "add_norm_modulate";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (rows == 0) return LTXK_OK;
    if (!x_out || !x) return fail(LTXK_E_ARG, "%s: null x_out or x", what);
    if (!f && !(gate && (gate->tab || gate->emb)))
        return fail(LTXK_E_ARG, "%s: without f the gate operand is the addend and must be present", what);
    if ((rc = check_ptrs(what, {x_out, y, y2, x, f}))) return rc;
    if (y2 && !y) return fail(LTXK_E_ARG, "%s: y2 needs y", what);
    AddNormParams p{};
    p.g = make_geom(rows, tokens, dim);
    p.x_out = static_cast<uint16_t *>(x_out);
    p.y = static_cast<uint16_t *>(y);
    p.x = static_cast<const uint16_t *>(x);
    p.f = static_cast<const uint16_t *>(f);
    p.mask = static_cast<const uint16_t *>(mask);
    p.gate = make_ada(gate);
    p.shift = make_ada(shift);
    p.scale = make_ada(scale);
    p.y2 = static_cast<uint16_t *>(y2);
    p.shift2 = make_ada(shift2);
    p.scale2 = make_ada(scale2);
    p.eps = eps;
    if ((rc = check_ada(p.gate, what, "gate")) || (rc = check_ada(p.shift, what, "shift")) ||
        (rc = check_ada(p.scale, what, "scale")) || (rc = check_ada(p.shift2, what, "shift2")) ||
        (rc = check_ada(p.scale2, what, "scale2")))
        return rc;
    return dispatch<AddNormLaunch>(p, static_cast<hipStream_t>(stream), what);
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
    return dispatch<PointLaunch<0>::K>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_modulate_layers(void *y, const void *x, int64_t layers, int64_t rows, int64_t tokens,
                                    int64_t dim, const ltxk_ada *shift, const ltxk_ada *scale,
                                    int64_t tab_layer_stride, int64_t emb_layer_stride, void *stream)
{
    static const char *what = "modulate_layers";
    clear_error();
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (layers < 0) return fail(LTXK_E_ARG, "%s: negative layer count %lld", what, (long long)layers);
    if (rows == 0 || layers == 0) return LTXK_OK;
    if (!y || !x) return fail(LTXK_E_ARG, "%s: null x or y", what);
    if (layers * rows > 0x7fffffff)
        return fail(LTXK_E_ARG, "%s: layers*rows %lld above 2^31", what, (long long)(layers * rows));
    if (tab_layer_stride < 0 || emb_layer_stride < 0 || tab_layer_stride % 8 || emb_layer_stride % 8)
        return fail(LTXK_E_ALIGN, "%s: layer strides must be non-negative multiples of 8 elements", what);
    if ((rc = check_ptrs(what, {y, x}))) return rc;
    ModLayersParams p{};
    p.out = static_cast<uint16_t *>(y);
    p.x = static_cast<const uint16_t *>(x);
    p.rows = rows;
    p.tokens = tokens;
    p.dim = dim;
    p.units = static_cast<uint32_t>(dim / 8);
    p.shift = make_ada(shift);
    p.scale = make_ada(scale);
    p.tab_ls = tab_layer_stride;
    p.emb_ls = emb_layer_stride;
    if ((rc = check_ada(p.shift, what, "shift")) || (rc = check_ada(p.scale, what, "scale"))) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t c = (p.units + kBlock - 1) / kBlock;  // chunks per thread, dim <= 16384: at most 8
    if (!p.shift.idx && !p.scale.idx && p.shift.ts == 0 && p.scale.ts == 0) {
        // per-(layer, batch item) operands: the tiled form
        const int64_t row_blocks = (rows + kModRows - 1) / kModRows;
        const int lgs = c <= 2 ? LTXK_MODL_LG : 1;
        const int64_t lgroups = (layers + lgs - 1) / lgs;
        if (lgroups * row_blocks > 0x7fffffff) return fail(LTXK_E_ARG, "%s: grid too large", what);
        const dim3 tgrid(static_cast<unsigned>(lgroups * row_blocks)), tblock(kBlock);
        if (c <= 1) modulate_layers_tiled_kernel<1, LTXK_MODL_LG><<<tgrid, tblock, 0, s>>>(p, layers, row_blocks);
        else if (c <= 2)
            modulate_layers_tiled_kernel<2, LTXK_MODL_LG><<<tgrid, tblock, 0, s>>>(p, layers, row_blocks);
        else if (c <= 4) modulate_layers_tiled_kernel<4, 1><<<tgrid, tblock, 0, s>>>(p, layers, row_blocks);
        else modulate_layers_tiled_kernel<8, 1><<<tgrid, tblock, 0, s>>>(p, layers, row_blocks);
        return check_launch(what);
    }
    const int64_t groups = (layers + kLayersPerGroup - 1) / kLayersPerGroup;
    const dim3 grid(static_cast<unsigned>(groups * rows)), block(kBlock);
    auto go = [&](auto shared, auto separate) {
        if (emb_layer_stride == 0) shared<<<grid, block, 0, s>>>(p, layers);
        else separate<<<grid, block, 0, s>>>(p, layers);
    };
    if (c <= 1) go(modulate_layers_kernel<1, true>, modulate_layers_kernel<1, false>);
    else if (c <= 2) go(modulate_layers_kernel<2, true>, modulate_layers_kernel<2, false>);
    else if (c <= 4) go(modulate_layers_kernel<4, true>, modulate_layers_kernel<4, false>);
    else go(modulate_layers_kernel<8, true>, modulate_layers_kernel<8, false>);
    return check_launch(what);
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
    return dispatch<PointLaunch<1>::K>(p, static_cast<hipStream_t>(stream), what);
}

extern "C" int ltxk_head_gate(void *out, const void *x, int64_t x_bstride, int64_t x_tstride, int64_t x_hstride,
                              const void *logits, const void *v, const void *mask, int64_t batch, int64_t tokens,
                              int64_t heads, int64_t head_dim, void *stream)
{
    static const char *what = "head_gate";
    clear_error();
    if (heads <= 0 || head_dim <= 0 || head_dim % 8)
        return fail(LTXK_E_ARG, "%s: heads must be > 0 and head_dim a multiple of 8 (got %lld, %lld)", what,
                    (long long)heads, (long long)head_dim);
    if (batch < 0 || tokens < 0) return fail(LTXK_E_ARG, "%s: negative batch or tokens", what);
    const int64_t dim = heads * head_dim;
    const int64_t rows = batch * tokens;
    if (rows == 0) return LTXK_OK;
    int rc = check_rows(rows, tokens, dim, what);
    if (rc) return rc;
    if (!out || !x) return fail(LTXK_E_ARG, "%s: null out or x", what);
    if (v && !mask) return fail(LTXK_E_ARG, "%s: a value blend needs its keep-mask", what);
    if ((rc = check_ptrs(what, {out, x, v}))) return rc;
    if (x_bstride % 8 || x_tstride % 8 || x_hstride % 8)
        return fail(LTXK_E_ALIGN, "%s: input strides must be multiples of 8 elements", what);
    if (x_bstride < 0 || x_tstride < 0 || x_hstride < 0)
        return fail(LTXK_E_ARG, "%s: input strides must be non-negative", what);
    // the input is addressed by 32-bit byte offsets from its start
    const int64_t span = ((batch - 1) * x_bstride + (tokens - 1) * x_tstride + (heads - 1) * x_hstride + head_dim) * 2;
    if (span >= static_cast<int64_t>(kOOB))
        return fail(LTXK_E_ARG, "%s: input spans %lld bytes, above 2^31", what, (long long)span);
    PointRowParams p = point_params(out, x, logits, rows, tokens, dim);
    p.heads = heads;
    p.head_dim = head_dim;
    p.xbs = x_bstride;
    p.xts = x_tstride;
    p.xhs = x_hstride;
    p.xspan = static_cast<uint32_t>(span);
    p.v = static_cast<const uint16_t *>(v);
    p.mask = v ? static_cast<const uint16_t *>(mask) : nullptr;
    if (v) return dispatch<PointLaunch<4>::K>(p, static_cast<hipStream_t>(stream), what);
    return dispatch<PointLaunch<2>::K>(p, static_cast<hipStream_t>(stream), what);
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
    return dispatch<PointLaunch<3>::K>(p, static_cast<hipStream_t>(stream), what);
}
