// Row kernels over token-major activations [rows, dim] (bf16):
//   norm_modulate       y(,y2) = norm(x)[*w] * (1 + scale) + shift
//   add_norm_modulate   x' = x + f*gate*mask ; y = rms(x') * (1 + scale) + shift
//   modulate            y = x * (1 + scale) + shift
//   gated_residual      out = x + f*gate*mask
//   head_gate           out[r,h,:] = x[r,h,:] * 2*sigmoid(logit[r,h])
//   x0                  x0 = latent - v * ts[b,t]
//
// Geometry (compile time): a row of dim/8 16-byte chunks is owned by TPR
// consecutive threads (TPR = the next power of two >= dim/8, at most 256),
// C chunks each (chunk u = lane + k*TPR, so for every k a wave reads one
// contiguous 1 KiB span).  Every load of a thread is issued before the first
// use, from clamped addresses, cache-resident modulation rows first and the
// streamed activation last, so all of them are in flight together; ragged
// tails are zeroed by select, not by branches.  Row sums use DPP inside a
// wave and LDS across the (up to four) waves of a row.  fp32 arithmetic, one
// rounding per output, each activation read and written once.
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

// Position of this thread: its row (clamped into range so every load is
// valid), whether the row exists, and its lane within the row group.
template <int TPR>
struct Slot {
    int64_t row;
    bool active;
    int lane;
    __device__ Slot(int64_t rows)
    {
        constexpr int RPB = kBlock / TPR;
        const int lrow = threadIdx.x / TPR;
        lane = threadIdx.x % TPR;
        const int64_t r = static_cast<int64_t>(blockIdx.x) * RPB + lrow;
        active = r < rows;
        row = active ? r : rows - 1;
    }
};

template <int TPR, int C>
__device__ __forceinline__ void load_row(const uint16_t *base, int lane, int64_t units, uint4 v[C])
{
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t u = lane + static_cast<int64_t>(k) * TPR;
        v[k] = ld16_stream(base + (u < units ? u : units - 1) * 8);
    }
}

// Column of chunk k of this thread, clamped into the row so loads stay valid.
template <int TPR>
__device__ __forceinline__ int64_t chunk_col(int lane, int k, int64_t units)
{
    const int64_t u = lane + static_cast<int64_t>(k) * TPR;
    return (u < units ? u : units - 1) * 8;
}

template <int TPR, int C>
__device__ __forceinline__ bool chunk_valid(int lane, int k, int64_t units)
{
    // Known true at compile time when TPR*C == units; otherwise one compare.
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
    const Slot<TPR> s(g.rows);
    const int64_t b = udiv32(s.row, g.tokens), t = s.row - b * g.tokens;
    // Issue order: modulation rows (cache hits) first, then the activation
    // (HBM); waiting for the former leaves the latter in flight.
    AdaRaw rsh[C], rsc[C];
    uint4 rw[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        rsh[k] = ada_fetch(p.shift, b, t, d);
        rsc[k] = ada_fetch(p.scale, b, t, d);
        rw[k] = ld16((p.w ? p.w : g_ada_zeros) + d);
    }
    uint4 raw[C];
    load_row<TPR, C>(p.x + s.row * g.dim, s.lane, g.units, raw);
    float v[C][8];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        unpack8(raw[k], v[k]);
        if (!chunk_valid<TPR, C>(s.lane, k, g.units))
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
    }
    float mean = 0.f;
    if (p.layer) {
        float s1 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k)
#pragma unroll
            for (int i = 0; i < 8; ++i) s1 += v[k][i];
        mean = row_sum<TPR>(s1, lds) / static_cast<float>(g.dim);
#pragma unroll
        for (int k = 0; k < C; ++k)
            if (chunk_valid<TPR, C>(s.lane, k, g.units))
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
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!chunk_valid<TPR, C>(s.lane, k, g.units)) continue;
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        float nv[8], wv[8], sh[8], sc[8], o[8];
        unpack8(rw[k], wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) nv[i] = p.w ? (v[k][i] * r) * wv[i] : v[k][i] * r;
        ada_finish(p.shift, rsh[k], 0.f, sh);
        ada_finish(p.scale, rsc[k], 0.f, sc);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
        st16_stream(p.y + s.row * g.dim + d, pack8(o));
        if (p.y2) {
            ada_load8(p.shift2, b, t, d, 0.f, sh);
            ada_load8(p.scale2, b, t, d, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
            st16_stream(p.y2 + s.row * g.dim + d, pack8(o));
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
    const uint16_t *f;
    const uint16_t *mask;
    Ada gate, shift, scale, shift2, scale2;
    float eps;
};

template <int TPR, int C>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_kernel(AddNormParams p)
{
    __shared__ float lds[kBlock / 64];
    const RowGeom &g = p.g;
    const Slot<TPR> s(g.rows);
    const int64_t b = udiv32(s.row, g.tokens), t = s.row - b * g.tokens;
    AdaRaw rg[C], rsh[C], rsc[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        rg[k] = ada_fetch(p.gate, b, t, d);
        rsh[k] = ada_fetch(p.shift, b, t, d);
        rsc[k] = ada_fetch(p.scale, b, t, d);
    }
    uint4 rx[C], rf[C];
    load_row<TPR, C>(p.x + s.row * g.dim, s.lane, g.units, rx);
    load_row<TPR, C>(p.f + s.row * g.dim, s.lane, g.units, rf);
    const float m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;  // after the streamed loads are issued
    float v[C][8];
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const bool ok = chunk_valid<TPR, C>(s.lane, k, g.units);
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        float xv[8], fv[8], gv[8];
        unpack8(rx[k], xv);
        unpack8(rf[k], fv);
        ada_finish(p.gate, rg[k], 1.0f, gv);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gv[i]) * m;
        const uint4 packed = pack8(xv);
        if (ok && s.active) st16_stream(p.x_out + s.row * g.dim + d, packed);
        unpack8(packed, v[k]);  // the norm sees the rounded residual
        if (!ok)
#pragma unroll
            for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
    }
    if (!p.y) return;  // uniform over the launch
    const float r = rsqrtf(row_sum<TPR>(s2, lds) / static_cast<float>(g.dim) + p.eps);
    if (!s.active) return;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!chunk_valid<TPR, C>(s.lane, k, g.units)) continue;
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        float sh[8], sc[8], o[8];
        ada_finish(p.shift, rsh[k], 0.f, sh);
        ada_finish(p.scale, rsc[k], 0.f, sc);
        float nv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * r;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
        st16_stream(p.y + s.row * g.dim + d, pack8(o));
        if (p.y2) {
            ada_load8(p.shift2, b, t, d, 0.f, sh);
            ada_load8(p.scale2, b, t, d, 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[i]) + sh[i];
            st16_stream(p.y2 + s.row * g.dim + d, pack8(o));
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
    const uint16_t *v;       // head gate: value rows blended in where the keep-mask is 0
};

// op 0: modulate, 1: gated residual, 2: head gate, 3: x0, 4: head gate with
// perturbation blend (v and its keep-mask set)
template <int OP, int TPR, int C>
__global__ void __launch_bounds__(kBlock) point_row_kernel(PointRowParams p)
{
    const RowGeom &g = p.g;
    const Slot<TPR> s(g.rows);
    if (!s.active) return;  // no barriers below
    const int64_t b = udiv32(s.row, g.tokens);
    const int64_t t = s.row - b * g.tokens;
    AdaRaw r0[C], r1[C];
    float lg[C];
    if (OP == 0 || OP == 1) {
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
            r0[k] = ada_fetch(p.a0, b, t, d);
            if (OP == 0) r1[k] = ada_fetch(p.a1, b, t, d);
        }
    }
    if (OP == 2 || OP == 4) {
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
    uint4 rx[C], rf[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        if (OP == 2 || OP == 4) {
            const int64_t h = static_cast<uint32_t>(d) / static_cast<uint32_t>(p.head_dim);
            rx[k] = ld16_stream(p.x + b * p.xbs + t * p.xts + h * p.xhs + (d - h * p.head_dim));
        } else {
            rx[k] = ld16_stream(p.x + s.row * g.dim + d);
        }
        if (OP == 1 || OP == 3) rf[k] = ld16_stream(p.f + s.row * g.dim + d);
        if (OP == 4) rf[k] = ld16_stream(p.v + s.row * g.dim + d);
    }
    // Head gate: every chunk is computed (out-of-range ones on clamped, valid
    // data) and only the store is conditional, because a condition around the
    // computation lets the compiler sink that chunk's loads under it, behind a
    // wait (measured: 20.4 -> 18.5 us at [6144, 4096]).  The other ops measured
    // faster with the skip.
    constexpr bool kGate = OP == 2 || OP == 4;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        if (!kGate && !chunk_valid<TPR, C>(s.lane, k, g.units)) continue;
        const int64_t d = chunk_col<TPR>(s.lane, k, g.units);
        float xv[8], o[8];
        unpack8(rx[k], xv);
        if (OP == 0) {
            float sh[8], sc[8];
            ada_finish(p.a0, r0[k], 0.f, sh);
            ada_finish(p.a1, r1[k], 0.f, sc);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * (1.0f + sc[i]) + sh[i];
        } else if (OP == 1) {
            float fv[8], gv[8];
            unpack8(rf[k], fv);
            ada_finish(p.a0, r0[k], 1.0f, gv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] + (fv[i] * gv[i]) * m;
        } else if (OP == 2 || OP == 4) {
            // 2*sigmoid(l) = 2 / (1 + e^-l); no logits: l = 0 from the zero row, gate exactly 1
            const float gate = 2.0f / (1.0f + expf(-lg[k]));
            if (OP == 4) {  // perturbation blend: attn*m + v*(1-m), m one 0/1 keep value per batch item
                float vv[8];
                unpack8(rf[k], vv);
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = xv[i] * m + vv[i] * (1.0f - m);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] * gate;
        } else {
            float vv[8];
            unpack8(rf[k], vv);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = xv[i] - vv[i] * tsv;
        }
        if (!kGate || chunk_valid<TPR, C>(s.lane, k, g.units)) st16_stream(p.out + s.row * g.dim + d, pack8(o));
    }
}

// ------------------------------------------- broadcast-modulation kernels --
// When every AdaLN operand is the same for all tokens of a batch item (table
// row + per-batch timestep embedding: emb_tstride == 0), the kernels below
// run persistent workgroups.  Each thread always owns the same C chunks of
// its row, so it combines the modulation rows for its columns once into
// registers (as fp32, after the reference's bf16 rounding of table +
// timestep) and then streams rows: the next row group's activation is
// requested before the current one is reduced and written.  Per element this
// leaves the unpack, the sum of squares, the normalise/modulate arithmetic
// and the pack.

template <int TPR, int C>
struct ModRegs {
    float v[C][8];
};

// Loads N modulation operands for batch item b: every fetch is issued before
// the first one is combined, so the N*C cache round trips overlap.
template <int TPR, int C, int N>
__device__ __forceinline__ void load_mods(const Ada *const (&ops)[N], const float (&absent)[N], int64_t b, int lane,
                                          int64_t units, ModRegs<TPR, C> *(&out)[N])
{
    AdaRaw raw[N][C];
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int k = 0; k < C; ++k) raw[n][k] = ada_fetch(*ops[n], b, 0, chunk_col<TPR>(lane, k, units));
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
        for (int k = 0; k < C; ++k) ada_finish(*ops[n], raw[n][k], absent[n], out[n]->v[k]);
}

// Row r of group `grp` for this thread (clamped), and whether it exists.
template <int TPR>
__device__ __forceinline__ int64_t group_row(int64_t grp, int64_t rows, bool &exists)
{
    const int64_t r = grp * (kBlock / TPR) + threadIdx.x / TPR;
    exists = r < rows;
    return exists ? r : rows - 1;
}

template <int TPR, int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) norm_modulate_bcast_kernel(NormModParams p)
{
    __shared__ float lds[2 * (kBlock / 64)];
    const RowGeom &g = p.g;
    const int lane = threadIdx.x % TPR;
    const int64_t groups = (g.rows + (kBlock / TPR) - 1) / (kBlock / TPR);
    int64_t grp = blockIdx.x;
    bool exists;
    int64_t row = group_row<TPR>(grp, g.rows, exists);
    int64_t cur_b = udiv32(row, g.tokens);
    ModRegs<TPR, C> sh, sc, sh2, sc2;
    if constexpr (DUAL) {
        const Ada *ops[4] = {&p.shift, &p.scale, &p.shift2, &p.scale2};
        ModRegs<TPR, C> *dst[4] = {&sh, &sc, &sh2, &sc2};
        load_mods<TPR, C, 4>(ops, {0.f, 0.f, 0.f, 0.f}, cur_b, lane, g.units, dst);
    } else {
        const Ada *ops[2] = {&p.shift, &p.scale};
        ModRegs<TPR, C> *dst[2] = {&sh, &sc};
        load_mods<TPR, C, 2>(ops, {0.f, 0.f}, cur_b, lane, g.units, dst);
    }
    uint4 cur[C];
    load_row<TPR, C>(p.x + row * g.dim, lane, g.units, cur);
    for (int it = 0; grp < groups; ++it) {
        const int64_t ngrp = grp + gridDim.x;
        bool nexists;
        const int64_t nrow = group_row<TPR>(ngrp < groups ? ngrp : grp, g.rows, nexists);
        uint4 nxt[C];
        // past the last group the prefetch reads cached zeros instead of HBM
        load_row<TPR, C>(ngrp < groups ? p.x + nrow * g.dim : g_ada_zeros, lane, g.units, nxt);
        const int64_t b = udiv32(row, g.tokens);
        if (b != cur_b) {  // batch boundary inside the stream: refresh the modulation
            cur_b = b;
            if constexpr (DUAL) {
                const Ada *ops[4] = {&p.shift, &p.scale, &p.shift2, &p.scale2};
                ModRegs<TPR, C> *dst[4] = {&sh, &sc, &sh2, &sc2};
                load_mods<TPR, C, 4>(ops, {0.f, 0.f, 0.f, 0.f}, b, lane, g.units, dst);
            } else {
                const Ada *ops[2] = {&p.shift, &p.scale};
                ModRegs<TPR, C> *dst[2] = {&sh, &sc};
                load_mods<TPR, C, 2>(ops, {0.f, 0.f}, b, lane, g.units, dst);
            }
        }
        float v[C][8];
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            unpack8(cur[k], v[k]);
            if (!chunk_valid<TPR, C>(lane, k, g.units))
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
        }
        float tot;
        if constexpr (TPR <= 64) {
            tot = row_sum<TPR>(s2, lds);
        } else {
            // partials double-buffered by iteration parity: one barrier per row
            const float w = wave_sum64(s2);
            float *buf = lds + (it & 1) * (kBlock / 64);
            if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = w;
            __syncthreads();
            tot = 0.f;
            const int w0 = (threadIdx.x / TPR) * (TPR / 64);  // first wave of this row
#pragma unroll
            for (int q = 0; q < TPR / 64; ++q) tot += buf[w0 + q];
        }
        const float r = rsqrtf(tot / static_cast<float>(g.dim) + p.eps);
        if (exists) {
#pragma unroll
            for (int k = 0; k < C; ++k) {
                if (!chunk_valid<TPR, C>(lane, k, g.units)) continue;
                const int64_t d = chunk_col<TPR>(lane, k, g.units);
                float nv[8], o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * r;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc.v[k][i]) + sh.v[k][i];
                st16_stream(p.y + row * g.dim + d, pack8(o));
                if constexpr (DUAL) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2.v[k][i]) + sh2.v[k][i];
                    st16_stream(p.y2 + row * g.dim + d, pack8(o));
                }
            }
        }
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = nxt[k];
        row = nrow;
        exists = nexists;
        grp = ngrp;
    }
}

// The broadcast norm for rows owned by a whole workgroup (TPR == kBlock),
// the shape of every DiT activation (dim >= 2048).  Workgroup w streams rows
// w, w + G, ... (G = gridDim.x) batch item by batch item: the modulation of an
// item is loaded before its rows, so the row loop issues no other loads and
// the wait for a row never waits for anything but that row (and, through the
// prefetch copy, the next one).  Measured on [6144, 4096]: 2 workgroups per CU
// stream fastest (the fewest rows in flight that still hide the latency).
// FULL: dim == C * kBlock * 8 (every chunk of every thread in range: dim 2048,
// 4096, 8192, 16384), which drops the per-chunk range handling from the loop.
template <int C, bool DUAL, bool FULL>
__global__ void __launch_bounds__(kBlock) norm_modulate_seg_kernel(NormModParams p)
{
    __shared__ float lds[2 * (kBlock / 64)];
    const RowGeom &g = p.g;
    const int lane = threadIdx.x;
    const int64_t G = gridDim.x;
    int64_t col[C];  // this thread's chunk columns (clamped into the row)
    bool valid[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        col[k] = chunk_col<kBlock>(lane, k, g.units);
        valid[k] = FULL || chunk_valid<kBlock, C>(lane, k, g.units);
    }
    int parity = 0;
    for (int64_t lo = 0; lo < g.rows; lo += g.tokens) {
        const int64_t hi = lo + g.tokens;
        const int64_t skip = lo > blockIdx.x ? (lo - blockIdx.x + G - 1) / G : 0;
        int64_t r = blockIdx.x + skip * G;  // this workgroup's first row of the item
        if (r >= hi) continue;              // uniform over the workgroup
        const int64_t b = udiv32(lo, g.tokens);
        ModRegs<kBlock, C> sh, sc, sh2, sc2;
        if constexpr (DUAL) {
            const Ada *ops[4] = {&p.shift, &p.scale, &p.shift2, &p.scale2};
            ModRegs<kBlock, C> *dst[4] = {&sh, &sc, &sh2, &sc2};
            load_mods<kBlock, C, 4>(ops, {0.f, 0.f, 0.f, 0.f}, b, lane, g.units, dst);
        } else {
            const Ada *ops[2] = {&p.shift, &p.scale};
            ModRegs<kBlock, C> *dst[2] = {&sh, &sc};
            load_mods<kBlock, C, 2>(ops, {0.f, 0.f}, b, lane, g.units, dst);
        }
        uint4 cur[C];
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = ld16_stream(p.x + r * g.dim + col[k]);
        for (;;) {
            const int64_t rn = r + G;  // workgroup-uniform: row addresses are scalar
            const bool more = rn < hi;
            const uint16_t *nx = more ? p.x + rn * g.dim : g_ada_zeros;  // past the item: cached zeros
            uint4 nxt[C];
#pragma unroll
            for (int k = 0; k < C; ++k) nxt[k] = ld16_stream(nx + (more ? col[k] : 0));
            float v[C][8];
            float s2 = 0.f;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                unpack8(cur[k], v[k]);
                if (!FULL && !valid[k])
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
            }
            // partials double-buffered by parity: one barrier per row
            const float w = wave_sum64(s2);
            float *buf = lds + parity * (kBlock / 64);
            if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = w;
            __syncthreads();
            float tot = 0.f;
#pragma unroll
            for (int q = 0; q < kBlock / 64; ++q) tot += buf[q];
            parity ^= 1;
            const float rs = rsqrtf(tot / static_cast<float>(g.dim) + p.eps);
            uint16_t *y = p.y + r * g.dim;
            uint16_t *y2 = DUAL ? p.y2 + r * g.dim : nullptr;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float nv[8], o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc.v[k][i]) + sh.v[k][i];
                if (valid[k]) st16_stream(y + col[k], pack8(o));
                if constexpr (DUAL) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2.v[k][i]) + sh2.v[k][i];
                    if (valid[k]) st16_stream(y2 + col[k], pack8(o));
                }
            }
            if (!more) break;
#pragma unroll
            for (int k = 0; k < C; ++k) cur[k] = nxt[k];
            r = rn;
        }
    }
}

// Modulation of batch item 0 for the item kernels below: round(table +
// timestep row) for the C chunks of this thread, `absent` for an operand with
// neither part.  An absent part reads the zero row.
template <int C>
__device__ __forceinline__ void item_mod(const Ada &a, float absent, int lane, float (&out)[C][8])
{
    const u32x4 *tp = reinterpret_cast<const u32x4 *>(a.tab ? a.tab : g_ada_zeros);
    const u32x4 *ep = reinterpret_cast<const u32x4 *>(a.emb ? a.emb : g_ada_zeros);
    u32x4 tr[C], er[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        tr[k] = tp[lane + k * kBlock];
        er[k] = ep[lane + k * kBlock];
    }
#pragma unroll
    for (int k = 0; k < C; ++k) {
        float tv[8], ev[8];
        unpack8v(tr[k], tv);
        unpack8v(er[k], ev);
#pragma unroll
        for (int i = 0; i < 8; ++i)  // absent == 0: the zero rows give 0 without a select
            out[k][i] = (absent != 0.f && !a.kind) ? absent : bf16_to_f32(f32_to_bf16(tv[i] + ev[i]));
    }
}

// Sum of v over the workgroup; partials double-buffered by the row parity so
// one barrier per row suffices.
__device__ __forceinline__ float item_row_sum(float v, float (&lds)[2][kBlock / 64], int it)
{
    const float w = wave_sum64(v);
    if ((threadIdx.x & 63) == 0) lds[it & 1][threadIdx.x >> 6] = w;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kBlock / 64; ++q) tot += lds[it & 1][q];
    return tot;
}

// norm_modulate of one batch item whose rows are exactly C * kBlock chunks
// wide (dim 2048, 4096, 8192, 16384) with broadcast modulation: the shape of
// the DiT's norms at batch 1.  Workgroup w streams rows w, w + G, ... with the
// next row's loads issued before the current row is reduced; past the last
// row it re-reads its own row (a cache hit) so no branch guards the loads.
// Same arithmetic as norm_modulate_seg_kernel<C, DUAL, true>.
template <int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) norm_modulate_item_kernel(NormModParams p)
{
    constexpr int kStride = C * kBlock;  // 16-byte chunks per row
    __shared__ float lds[2][kBlock / 64];
    const int lane = threadIdx.x;
    float sh[C][8], sc[C][8], sh2[DUAL ? C : 1][8], sc2[DUAL ? C : 1][8];
    item_mod<C>(p.shift, 0.f, lane, sh);
    item_mod<C>(p.scale, 0.f, lane, sc);
    if constexpr (DUAL) {
        item_mod<C>(p.shift2, 0.f, lane, sh2);
        item_mod<C>(p.scale2, 0.f, lane, sc2);
    }
    const u32x4 *src = reinterpret_cast<const u32x4 *>(p.x);
    // rows * dim * 2 bytes fit in device memory, so rows < 2^26 and row
    // indices plus the grid stay far inside int.
    const int rows = static_cast<int>(p.g.rows);
    const int G = static_cast<int>(gridDim.x);
    int r = blockIdx.x;
    if (r >= rows) return;  // uniform over the workgroup
    u32x4 buf[C];
#pragma unroll
    for (int k = 0; k < C; ++k)
        buf[k] = __builtin_nontemporal_load(src + static_cast<int64_t>(r) * kStride + lane + k * kBlock);
    for (int it = 0; r < rows; ++it) {
        u32x4 cur[C];
#pragma unroll
        for (int k = 0; k < C; ++k) cur[k] = buf[k];
        {
            const int rn = r + G < rows ? r + G : r;
#pragma unroll
            for (int k = 0; k < C; ++k)
                buf[k] = __builtin_nontemporal_load(src + static_cast<int64_t>(rn) * kStride + lane + k * kBlock);
        }
        float v[C][8];
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            unpack8v(cur[k], v[k]);
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
        }
        const float rs = rsqrtf(item_row_sum(s2, lds, it) / static_cast<float>(kStride * 8) + p.eps);
        const int64_t at = static_cast<int64_t>(r) * kStride + lane;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            float nv[8], o[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[k][i]) + sh[k][i];
            __builtin_nontemporal_store(pack8v(o), reinterpret_cast<u32x4 *>(p.y) + at + k * kBlock);
            if constexpr (DUAL) {
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2[k][i]) + sh2[k][i];
                __builtin_nontemporal_store(pack8v(o), reinterpret_cast<u32x4 *>(p.y2) + at + k * kBlock);
            }
        }
        r += G;
    }
}

// add_norm_modulate in the form of norm_modulate_item_kernel (one batch item,
// full rows, broadcast gate/shift/scale): x_out = x + f * gate * mask, then
// the norm and modulation(s) of the rounded x_out when y is set.  Same
// arithmetic as add_norm_modulate_seg_kernel<C, DUAL, true>.  Launched for
// two outputs (46.1 us against 47.0 on [6144, 4096]); with one output it
// measured no faster than the segmented kernel (36.2 against 36.0 us).
template <int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_item_kernel(AddNormParams p)
{
    constexpr int kStride = C * kBlock;
    __shared__ float lds[2][kBlock / 64];
    const int lane = threadIdx.x;
    float gt[C][8], sh[C][8], sc[C][8], sh2[DUAL ? C : 1][8], sc2[DUAL ? C : 1][8];
    item_mod<C>(p.gate, 1.0f, lane, gt);
    item_mod<C>(p.shift, 0.f, lane, sh);
    item_mod<C>(p.scale, 0.f, lane, sc);
    if constexpr (DUAL) {
        item_mod<C>(p.shift2, 0.f, lane, sh2);
        item_mod<C>(p.scale2, 0.f, lane, sc2);
    }
    const float m = p.mask ? bf16_to_f32(p.mask[0]) : 1.0f;
    const u32x4 *xs = reinterpret_cast<const u32x4 *>(p.x);
    const u32x4 *fs = reinterpret_cast<const u32x4 *>(p.f);
    const int rows = static_cast<int>(p.g.rows);  // < 2^26, as above
    const int G = static_cast<int>(gridDim.x);
    int r = blockIdx.x;
    if (r >= rows) return;
    u32x4 bx[C], bfv[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        bx[k] = __builtin_nontemporal_load(xs + static_cast<int64_t>(r) * kStride + lane + k * kBlock);
        bfv[k] = __builtin_nontemporal_load(fs + static_cast<int64_t>(r) * kStride + lane + k * kBlock);
    }
    for (int it = 0; r < rows; ++it) {
        u32x4 cx[C], cf[C];
#pragma unroll
        for (int k = 0; k < C; ++k) {
            cx[k] = bx[k];
            cf[k] = bfv[k];
        }
        {
            const int rn = r + G < rows ? r + G : r;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                bx[k] = __builtin_nontemporal_load(xs + static_cast<int64_t>(rn) * kStride + lane + k * kBlock);
                bfv[k] = __builtin_nontemporal_load(fs + static_cast<int64_t>(rn) * kStride + lane + k * kBlock);
            }
        }
        const int64_t at = static_cast<int64_t>(r) * kStride + lane;
        float v[C][8];
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            float xv[8], fv[8];
            unpack8v(cx[k], xv);
            unpack8v(cf[k], fv);
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gt[k][i]) * m;
            const u32x4 packed = pack8v(xv);
            __builtin_nontemporal_store(packed, reinterpret_cast<u32x4 *>(p.x_out) + at + k * kBlock);
            unpack8v(packed, v[k]);  // the norm sees the rounded residual
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
        }
        if (p.y) {  // uniform over the launch
            const float rs = rsqrtf(item_row_sum(s2, lds, it) / static_cast<float>(kStride * 8) + p.eps);
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float nv[8], o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc[k][i]) + sh[k][i];
                __builtin_nontemporal_store(pack8v(o), reinterpret_cast<u32x4 *>(p.y) + at + k * kBlock);
                if constexpr (DUAL) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2[k][i]) + sh2[k][i];
                    __builtin_nontemporal_store(pack8v(o), reinterpret_cast<u32x4 *>(p.y2) + at + k * kBlock);
                }
            }
        }
        r += G;
    }
}

// add_norm_modulate for rows owned by a whole workgroup, in the segmented
// form of norm_modulate_seg_kernel: gate, shift and scale of a batch item (and
// its mask value) are loaded before the item's rows; the row loop streams x
// and f with a one-row prefetch.
template <int C, bool DUAL, bool FULL>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_seg_kernel(AddNormParams p)
{
    __shared__ float lds[2 * (kBlock / 64)];
    const RowGeom &g = p.g;
    const int lane = threadIdx.x;
    const int64_t G = gridDim.x;
    int64_t col[C];
    bool valid[C];
#pragma unroll
    for (int k = 0; k < C; ++k) {
        col[k] = chunk_col<kBlock>(lane, k, g.units);
        valid[k] = FULL || chunk_valid<kBlock, C>(lane, k, g.units);
    }
    int parity = 0;
    for (int64_t lo = 0; lo < g.rows; lo += g.tokens) {
        const int64_t hi = lo + g.tokens;
        const int64_t skip = lo > blockIdx.x ? (lo - blockIdx.x + G - 1) / G : 0;
        int64_t r = blockIdx.x + skip * G;
        if (r >= hi) continue;  // uniform over the workgroup
        const int64_t b = udiv32(lo, g.tokens);
        ModRegs<kBlock, C> gt, sh, sc, sh2, sc2;
        if constexpr (DUAL) {
            const Ada *ops[5] = {&p.gate, &p.shift, &p.scale, &p.shift2, &p.scale2};
            ModRegs<kBlock, C> *dst[5] = {&gt, &sh, &sc, &sh2, &sc2};
            load_mods<kBlock, C, 5>(ops, {1.0f, 0.f, 0.f, 0.f, 0.f}, b, lane, g.units, dst);
        } else {
            const Ada *ops[3] = {&p.gate, &p.shift, &p.scale};
            ModRegs<kBlock, C> *dst[3] = {&gt, &sh, &sc};
            load_mods<kBlock, C, 3>(ops, {1.0f, 0.f, 0.f}, b, lane, g.units, dst);
        }
        const float m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;
        uint4 cx[C], cf[C];
#pragma unroll
        for (int k = 0; k < C; ++k) {
            cx[k] = ld16_stream(p.x + r * g.dim + col[k]);
            cf[k] = ld16_stream(p.f + r * g.dim + col[k]);
        }
        for (;;) {
            const int64_t rn = r + G;  // workgroup-uniform
            const bool more = rn < hi;
            const uint16_t *nxp = more ? p.x + rn * g.dim : g_ada_zeros;  // past the item: cached zeros
            const uint16_t *nfp = more ? p.f + rn * g.dim : g_ada_zeros;
            uint4 nx[C], nf[C];
#pragma unroll
            for (int k = 0; k < C; ++k) {
                nx[k] = ld16_stream(nxp + (more ? col[k] : 0));
                nf[k] = ld16_stream(nfp + (more ? col[k] : 0));
            }
            float v[C][8];
            float s2 = 0.f;
            uint16_t *xo = p.x_out + r * g.dim;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                float xv[8], fv[8];
                unpack8(cx[k], xv);
                unpack8(cf[k], fv);
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gt.v[k][i]) * m;
                const uint4 packed = pack8(xv);
                if (valid[k]) st16_stream(xo + col[k], packed);
                unpack8(packed, v[k]);  // the norm sees the rounded residual
                if (!FULL && !valid[k])
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
            }
            if (p.y) {  // uniform over the launch
                const float w = wave_sum64(s2);
                float *buf = lds + parity * (kBlock / 64);
                if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = w;
                __syncthreads();
                float tot = 0.f;
#pragma unroll
                for (int q = 0; q < kBlock / 64; ++q) tot += buf[q];
                parity ^= 1;
                const float rs = rsqrtf(tot / static_cast<float>(g.dim) + p.eps);
                uint16_t *y = p.y + r * g.dim;
                uint16_t *y2 = DUAL ? p.y2 + r * g.dim : nullptr;
#pragma unroll
                for (int k = 0; k < C; ++k) {
                    float nv[8], o[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * rs;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc.v[k][i]) + sh.v[k][i];
                    if (valid[k]) st16_stream(y + col[k], pack8(o));
                    if constexpr (DUAL) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2.v[k][i]) + sh2.v[k][i];
                        if (valid[k]) st16_stream(y2 + col[k], pack8(o));
                    }
                }
            }
            if (!more) break;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                cx[k] = nx[k];
                cf[k] = nf[k];
            }
            r = rn;
        }
    }
}

template <int TPR, int C, bool DUAL>
__global__ void __launch_bounds__(kBlock) add_norm_modulate_bcast_kernel(AddNormParams p)
{
    __shared__ float lds[2 * (kBlock / 64)];
    const RowGeom &g = p.g;
    const int lane = threadIdx.x % TPR;
    const int64_t groups = (g.rows + (kBlock / TPR) - 1) / (kBlock / TPR);
    int64_t grp = blockIdx.x;
    bool exists;
    int64_t row = group_row<TPR>(grp, g.rows, exists);
    int64_t cur_b = udiv32(row, g.tokens);
    constexpr int NM = DUAL ? 5 : 3;
    ModRegs<TPR, C> gt, sh, sc, sh2, sc2;
    const Ada *ops[NM];
    ModRegs<TPR, C> *dst[NM];
    float absent[NM];
    ops[0] = &p.gate, ops[1] = &p.shift, ops[2] = &p.scale;
    dst[0] = &gt, dst[1] = &sh, dst[2] = &sc;
    absent[0] = 1.0f, absent[1] = 0.f, absent[2] = 0.f;
    if constexpr (DUAL) {
        ops[3] = &p.shift2, ops[4] = &p.scale2;
        dst[3] = &sh2, dst[4] = &sc2;
        absent[3] = 0.f, absent[4] = 0.f;
    }
    load_mods<TPR, C, NM>(ops, absent, cur_b, lane, g.units, dst);
    float m = p.mask ? bf16_to_f32(p.mask[cur_b]) : 1.0f;
    uint4 cx[C], cf[C];
    load_row<TPR, C>(p.x + row * g.dim, lane, g.units, cx);
    load_row<TPR, C>(p.f + row * g.dim, lane, g.units, cf);
    for (int it = 0; grp < groups; ++it) {
        const int64_t ngrp = grp + gridDim.x;
        bool nexists;
        const int64_t nrow = group_row<TPR>(ngrp < groups ? ngrp : grp, g.rows, nexists);
        uint4 nx[C], nf[C];
        // past the last group the prefetch reads cached zeros instead of HBM
        load_row<TPR, C>(ngrp < groups ? p.x + nrow * g.dim : g_ada_zeros, lane, g.units, nx);
        load_row<TPR, C>(ngrp < groups ? p.f + nrow * g.dim : g_ada_zeros, lane, g.units, nf);
        const int64_t b = udiv32(row, g.tokens);
        if (b != cur_b) {
            cur_b = b;
            load_mods<TPR, C, NM>(ops, absent, b, lane, g.units, dst);
            m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;
        }
        float v[C][8];
        float s2 = 0.f;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            const bool ok = chunk_valid<TPR, C>(lane, k, g.units);
            float xv[8], fv[8];
            unpack8(cx[k], xv);
            unpack8(cf[k], fv);
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + (fv[i] * gt.v[k][i]) * m;
            const uint4 packed = pack8(xv);
            if (ok && exists) st16_stream(p.x_out + row * g.dim + chunk_col<TPR>(lane, k, g.units), packed);
            unpack8(packed, v[k]);  // the norm sees the rounded residual
            if (!ok)
#pragma unroll
                for (int i = 0; i < 8; ++i) v[k][i] = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[k][i], v[k][i], s2);
        }
        if (p.y) {  // uniform over the launch
            float tot;
            if constexpr (TPR <= 64) {
                tot = row_sum<TPR>(s2, lds);
            } else {
                const float w = wave_sum64(s2);
                float *buf = lds + (it & 1) * (kBlock / 64);
                if ((threadIdx.x & 63) == 0) buf[threadIdx.x >> 6] = w;
                __syncthreads();
                tot = 0.f;
                const int w0 = (threadIdx.x / TPR) * (TPR / 64);  // first wave of this row
#pragma unroll
                for (int q = 0; q < TPR / 64; ++q) tot += buf[w0 + q];
            }
            const float r = rsqrtf(tot / static_cast<float>(g.dim) + p.eps);
            if (exists) {
#pragma unroll
                for (int k = 0; k < C; ++k) {
                    if (!chunk_valid<TPR, C>(lane, k, g.units)) continue;
                    float nv[8], o[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) nv[i] = v[k][i] * r;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc.v[k][i]) + sh.v[k][i];
                    st16_stream(p.y + row * g.dim + chunk_col<TPR>(lane, k, g.units), pack8(o));
                    if constexpr (DUAL) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) o[i] = nv[i] * (1.0f + sc2.v[k][i]) + sh2.v[k][i];
                        st16_stream(p.y2 + row * g.dim + chunk_col<TPR>(lane, k, g.units), pack8(o));
                    }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < C; ++k) {
            cx[k] = nx[k];
            cf[k] = nf[k];
        }
        row = nrow;
        exists = nexists;
        grp = ngrp;
    }
}

// op 0: modulate (a0 shift, a1 scale), 1: gated residual (a0 gate, mask)
template <int OP, int TPR, int C>
__global__ void __launch_bounds__(kBlock) point_row_bcast_kernel(PointRowParams p)
{
    const RowGeom &g = p.g;
    const int lane = threadIdx.x % TPR;
    const int64_t groups = (g.rows + (kBlock / TPR) - 1) / (kBlock / TPR);
    int64_t grp = blockIdx.x;
    bool exists;
    int64_t row = group_row<TPR>(grp, g.rows, exists);
    int64_t cur_b = udiv32(row, g.tokens);
    ModRegs<TPR, C> m0, m1;
    const Ada *ops[2] = {&p.a0, &p.a1};
    ModRegs<TPR, C> *dst[2] = {&m0, &m1};
    const float absent[2] = {OP == 1 ? 1.0f : 0.f, 0.f};
    load_mods<TPR, C, OP == 0 ? 2 : 1>(reinterpret_cast<const Ada *const(&)[OP == 0 ? 2 : 1]>(ops),
                                       reinterpret_cast<const float(&)[OP == 0 ? 2 : 1]>(absent), cur_b, lane,
                                       g.units, reinterpret_cast<ModRegs<TPR, C> *(&)[OP == 0 ? 2 : 1]>(dst));
    float m = (OP == 1 && p.mask) ? bf16_to_f32(p.mask[cur_b]) : 1.0f;
    uint4 cx[C], cf[C];
    load_row<TPR, C>(p.x + row * g.dim, lane, g.units, cx);
    if (OP == 1) load_row<TPR, C>(p.f + row * g.dim, lane, g.units, cf);
    while (grp < groups) {
        const int64_t ngrp = grp + gridDim.x;
        bool nexists;
        const int64_t nrow = group_row<TPR>(ngrp < groups ? ngrp : grp, g.rows, nexists);
        uint4 nx[C], nf[C];
        // past the last group the prefetch reads cached zeros instead of HBM
        load_row<TPR, C>(ngrp < groups ? p.x + nrow * g.dim : g_ada_zeros, lane, g.units, nx);
        if (OP == 1) load_row<TPR, C>(ngrp < groups ? p.f + nrow * g.dim : g_ada_zeros, lane, g.units, nf);
        const int64_t b = udiv32(row, g.tokens);
        if (b != cur_b) {
            cur_b = b;
            load_mods<TPR, C, OP == 0 ? 2 : 1>(reinterpret_cast<const Ada *const(&)[OP == 0 ? 2 : 1]>(ops),
                                               reinterpret_cast<const float(&)[OP == 0 ? 2 : 1]>(absent), b, lane,
                                               g.units, reinterpret_cast<ModRegs<TPR, C> *(&)[OP == 0 ? 2 : 1]>(dst));
            if (OP == 1) m = p.mask ? bf16_to_f32(p.mask[b]) : 1.0f;
        }
        if (exists) {
#pragma unroll
            for (int k = 0; k < C; ++k) {
                if (!chunk_valid<TPR, C>(lane, k, g.units)) continue;
                float xv[8], o[8];
                unpack8(cx[k], xv);
                if (OP == 0) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = xv[i] * (1.0f + m1.v[k][i]) + m0.v[k][i];
                } else {
                    float fv[8];
                    unpack8(cf[k], fv);
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = xv[i] + (fv[i] * m0.v[k][i]) * m;
                }
                st16_stream(p.out + row * g.dim + chunk_col<TPR>(lane, k, g.units), pack8(o));
            }
        }
#pragma unroll
        for (int k = 0; k < C; ++k) {
            cx[k] = nx[k];
            if (OP == 1) cf[k] = nf[k];
        }
        row = nrow;
        exists = nexists;
        grp = ngrp;
    }
}

// ----------------------------------------------------------------- launch --
constexpr int kSegPerCU = 2;    // workgroups per CU of the segmented kernels
constexpr int kSegItems = 64;   // most batch items a segmented launch walks
// Geometry choice: TPR threads per row, C chunks per thread.
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

// Workgroups of a persistent launch: as many as can be resident at once
// (compute units x occupancy of this kernel), never more than row groups.
template <typename Kernel>
unsigned persistent_grid(Kernel kernel, int64_t rows, int tpr, int max_per_cu = 0)
{
    struct Entry {
        const void *fn;
        int dev;
        int blocks;
    };
    static thread_local Entry cache[32];
    static thread_local int used = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const void *fn = reinterpret_cast<const void *>(kernel);
    int blocks = 0;
    for (int i = 0; i < used; ++i)
        if (cache[i].fn == fn && cache[i].dev == dev) blocks = cache[i].blocks;
    if (blocks == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kBlock, 0) != hipSuccess || per_cu <= 0)
            per_cu = 2;
        blocks = cus * per_cu;
        if (used < 32) cache[used++] = Entry{fn, dev, blocks};
    }
    if (max_per_cu > 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (blocks > cus * max_per_cu) blocks = cus * max_per_cu;
    }
    const int64_t groups = grid_for(rows, tpr);
    return static_cast<unsigned>(groups < blocks ? groups : blocks);
}

// True when none of the operands varies across the tokens of a batch item.
inline bool broadcast_only(std::initializer_list<const Ada *> ops)
{
    for (const Ada *a : ops)
        if (a->emb && a->ts != 0) return false;
    return true;
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

// Launchers: the persistent broadcast kernel when the modulation allows it,
// the per-row kernel otherwise (per-token timestep embeddings, layer norm,
// weighted norm).
template <int TPR, int C>
struct NormModLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const NormModParams &p)
    {
        if (!p.layer && !p.w && broadcast_only({&p.shift, &p.scale, &p.shift2, &p.scale2})) {
            if constexpr (TPR == kBlock) {
                if (p.g.rows / p.g.tokens <= kSegItems) {  // few batch items: the segmented kernel
                    const bool full = p.g.units == static_cast<int64_t>(C) * kBlock;
                    if (full && p.g.rows == p.g.tokens) {  // one item, whole rows
                        auto k = p.y2 ? norm_modulate_item_kernel<C, true> : norm_modulate_item_kernel<C, false>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    } else if (p.y2) {
                        auto k = full ? norm_modulate_seg_kernel<C, true, true>
                                      : norm_modulate_seg_kernel<C, true, false>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    } else {
                        auto k = full ? norm_modulate_seg_kernel<C, false, true>
                                      : norm_modulate_seg_kernel<C, false, false>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    }
                    return;
                }
            }
            if (p.y2) {
                auto k = norm_modulate_bcast_kernel<TPR, C, true>;
                k<<<dim3(persistent_grid(k, p.g.rows, TPR)), b, 0, s>>>(p);
            } else {
                auto k = norm_modulate_bcast_kernel<TPR, C, false>;
                k<<<dim3(persistent_grid(k, p.g.rows, TPR)), b, 0, s>>>(p);
            }
        } else
            norm_modulate_kernel<TPR, C><<<g, b, 0, s>>>(p);
    }
};

template <int TPR, int C>
struct AddNormLaunch {
    static void launch(dim3 g, dim3 b, hipStream_t s, const AddNormParams &p)
    {
        if (broadcast_only({&p.gate, &p.shift, &p.scale, &p.shift2, &p.scale2})) {
            if constexpr (TPR == kBlock) {
                if (p.g.rows / p.g.tokens <= kSegItems) {  // few batch items: the segmented kernel
                    const bool full = p.g.units == static_cast<int64_t>(C) * kBlock;
                    if (full && p.y2 && p.y && p.g.rows == p.g.tokens) {  // one item, whole rows, two outputs
                        auto k = add_norm_modulate_item_kernel<C, true>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    } else if (p.y2 && p.y) {
                        auto k = full ? add_norm_modulate_seg_kernel<C, true, true>
                                      : add_norm_modulate_seg_kernel<C, true, false>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    } else {
                        auto k = full ? add_norm_modulate_seg_kernel<C, false, true>
                                      : add_norm_modulate_seg_kernel<C, false, false>;
                        k<<<dim3(persistent_grid(k, p.g.rows, TPR, kSegPerCU)), b, 0, s>>>(p);
                    }
                    return;
                }
            }
            if (p.y2 && p.y) {
                auto k = add_norm_modulate_bcast_kernel<TPR, C, true>;
                k<<<dim3(persistent_grid(k, p.g.rows, TPR)), b, 0, s>>>(p);
            } else {
                auto k = add_norm_modulate_bcast_kernel<TPR, C, false>;
                k<<<dim3(persistent_grid(k, p.g.rows, TPR)), b, 0, s>>>(p);
            }
        } else
            add_norm_modulate_kernel<TPR, C><<<g, b, 0, s>>>(p);
    }
};

template <int OP>
struct PointLaunch {
    template <int TPR, int C>
    struct K {
        static void launch(dim3 g, dim3 b, hipStream_t s, const PointRowParams &p)
        {
            // Only the modulate op runs persistent: the gated residual has no
            // reduction to amortise and streams best as one row group per
            // workgroup.
            if constexpr (OP == 0) {
                if (broadcast_only({&p.a0, &p.a1})) {
                    auto k = point_row_bcast_kernel<OP, TPR, C>;
                    k<<<dim3(persistent_grid(k, p.g.rows, TPR)), b, 0, s>>>(p);
                    return;
                }
            }
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
    if (!x_out || !x || !f) return fail(LTXK_E_ARG, "%s: null x_out, x or f", what);
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
    PointRowParams p = point_params(out, x, logits, rows, tokens, dim);
    p.heads = heads;
    p.head_dim = head_dim;
    p.xbs = x_bstride;
    p.xts = x_tstride;
    p.xhs = x_hstride;
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
