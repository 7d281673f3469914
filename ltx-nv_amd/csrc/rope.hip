// q/k preparation: RMSNorm over the whole inner dim with a weight, then
// LTXRopeType.SPLIT rotation per head, in place, one HBM round trip.
//
// A row is one token of x [batch*tokens, heads*head_dim].  It is cut into
// "slots": slot s covers 8 rotation pairs of one head, i.e. the 8 elements at
// h*Dh + 8j (first half) and the 8 at h*Dh + Dh/2 + 8j (second half) for
// h = s / (Dh/16), j = s % (Dh/16).  A thread owns whole slots, so the pair
// partner of every element it rotates is already in its registers.
//
// Rotation tables come in two forms:
//   full     (batch, heads, tokens, Dh/2) cos/sin as precompute_freqs_cis
//            builds them (standalone/ltx_nn.py:63-96): 16 contiguous bytes of
//            each table per slot, streamed from HBM with the activations;
//   compact  rows [R, inner/2] holding, for one coordinate value of one
//            position axis, cos/sin at that axis' pairs and 0 elsewhere (plus
//            the identity padding in axis 0's rows), and a per-token index of
//            one row per axis.  Exactly one axis row is non-zero at a pair, so
//            combining the axis rows gives the full table's value bit for bit;
//            the rows are a few hundred KB and stay in L2.
//
// When q and k share tables and token count (self-attention), one launch
// handles both for the same token and fetches each table chunk once.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;

struct QKDev {
    uint16_t *x;
    const uint16_t *w;
    const uint16_t *cos;
    const uint16_t *sin;
    const int32_t *idx;  // compact tables: [rows, n_axes] table rows per token
    int64_t rows;
    int64_t tokens;
    int64_t tbs;         // full tables: elements between batch items
};

struct QKParams {
    QKDev q, k;
    int64_t dim, head_dim, half, slots, slots_per_head;
    int64_t q_groups;    // row groups of q (unpaired launches: blocks [0, q_groups) are q)
    float eps;
};

template <int S>
struct SlotPos {
    int64_t h[S], j8[S];
    bool ok[S];
};

// Compact tables: the table row of each axis for token `row` of t.
template <int AX>
struct TabIdx {
    int32_t r[AX > 0 ? AX : 1];
};

template <int AX>
__device__ __forceinline__ TabIdx<AX> index_fetch(const QKDev &t, int64_t row)
{
    TabIdx<AX> ti;
#pragma unroll
    for (int a = 0; a < AX; ++a) ti.r[a] = t.idx[row * AX + a];
    return ti;
}

// Table chunk offsets (elements) of this thread's slots for token `row` of t.
// AX = 0: full tables; AX >= 1: compact rows, one per axis.
template <int AX, int S>
struct TabRefs {
    int64_t off[AX > 0 ? AX : 1][S];
};

template <int AX, int S>
__device__ __forceinline__ void table_offsets(const QKDev &t, const QKParams &p, int64_t row, const SlotPos<S> &sp,
                                              const TabIdx<AX> &ti, TabRefs<AX, S> &tr)
{
    if constexpr (AX == 0) {
        const int64_t b = udiv32(row, t.tokens);
        const int64_t tok = row - b * t.tokens;
#pragma unroll
        for (int k = 0; k < S; ++k) tr.off[0][k] = b * t.tbs + (sp.h[k] * t.tokens + tok) * p.half + sp.j8[k];
    } else {
#pragma unroll
        for (int a = 0; a < AX; ++a)
#pragma unroll
            for (int k = 0; k < S; ++k)
                tr.off[a][k] = static_cast<int64_t>(ti.r[a]) * (p.dim / 2) + sp.h[k] * p.half + sp.j8[k];
    }
}

template <int AX>
struct TabRaw {
    uint4 c[AX > 0 ? AX : 1], s[AX > 0 ? AX : 1];
};

template <int AX, int S>
__device__ __forceinline__ void table_fetch(const QKDev &t, const TabRefs<AX, S> &tr, TabRaw<AX> raw[S])
{
    constexpr int NA = AX > 0 ? AX : 1;
#pragma unroll
    for (int k = 0; k < S; ++k)
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            raw[k].c[a] = ld16(t.cos + tr.off[a][k]);
            raw[k].s[a] = ld16(t.sin + tr.off[a][k]);
        }
}

// The compact rows of the other axes hold +0.0 (bits 0) at this thread's
// pairs, so OR-ing the raw bf16 words yields the one non-zero entry exactly:
// the full table's value, bit for bit.
template <int AX>
__device__ __forceinline__ void table_values(const TabRaw<AX> &raw, float c[8], float s[8])
{
    constexpr int NA = AX > 0 ? AX : 1;
    uint4 rc = raw.c[0], rs = raw.s[0];
#pragma unroll
    for (int a = 1; a < NA; ++a) {
        rc.x |= raw.c[a].x; rc.y |= raw.c[a].y; rc.z |= raw.c[a].z; rc.w |= raw.c[a].w;
        rs.x |= raw.s[a].x; rs.y |= raw.s[a].y; rs.z |= raw.s[a].z; rs.w |= raw.s[a].w;
    }
    unpack8(rc, c);
    unpack8(rs, s);
}

struct Pair8 {
    float a[8], b[8];
};

__device__ __forceinline__ void rotate(Pair8 &d, const float c[8], const float s[8])
{
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x1 = d.a[i], x2 = d.b[i];
        d.a[i] = x1 * c[i] - x2 * s[i];
        d.b[i] = x2 * c[i] + x1 * s[i];
    }
}

// One tensor's part of the work for one row: loads (x, weight), optional
// norm, rotation with the given table values, stores.
template <int TPR, int S>
struct RowWork {
    uint4 xa[S], xb[S], wa[S], wb[S];
    __device__ void load(const QKDev &t, const QKParams &p, int64_t row, const SlotPos<S> &sp)
    {
        const uint16_t *base = t.x + row * p.dim;
        const uint16_t *w = t.w ? t.w : g_ada_zeros;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            const int64_t off = sp.h[k] * p.head_dim + sp.j8[k];
            xa[k] = ld16_stream(base + off);
            xb[k] = ld16_stream(base + off + p.half);
            wa[k] = ld16(w + (t.w ? off : 0));
            wb[k] = ld16(w + (t.w ? off + p.half : 0));
        }
    }
    __device__ float sumsq(Pair8 d[S], const SlotPos<S> &sp)
    {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            unpack8(xa[k], d[k].a);
            unpack8(xb[k], d[k].b);
            if (!sp.ok[k])
#pragma unroll
                for (int i = 0; i < 8; ++i) d[k].a[i] = d[k].b[i] = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(d[k].b[i], d[k].b[i], __builtin_fmaf(d[k].a[i], d[k].a[i], ss));
        }
        return ss;
    }
    __device__ void weight(Pair8 &d, int k, float r)
    {
        float fa[8], fb[8];
        unpack8(wa[k], fa);
        unpack8(wb[k], fb);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            d.a[i] = (d.a[i] * r) * fa[i];
            d.b[i] = (d.b[i] * r) * fb[i];
        }
    }
};

template <int TPR, int S>
__device__ __forceinline__ SlotPos<S> slot_pos(const QKParams &p, int lane)
{
    SlotPos<S> sp;
#pragma unroll
    for (int k = 0; k < S; ++k) {
        int64_t s = lane + static_cast<int64_t>(k) * TPR;
        sp.ok[k] = s < p.slots;
        s = sp.ok[k] ? s : p.slots - 1;
        sp.h[k] = s / p.slots_per_head;
        sp.j8[k] = (s - sp.h[k] * p.slots_per_head) * 8;
    }
    return sp;
}

__device__ __forceinline__ void store_pair(uint16_t *base, int64_t off, int64_t half, const Pair8 &d)
{
    st16_stream(base + off, pack8(d.a));
    st16_stream(base + off + half, pack8(d.b));
}

// AX: -1 no rotation, 0 full tables, 1..3 compact tables with AX axes.
// PAIRED: q and k rows of the same token in one thread (shared tables).
template <int TPR, int S, int AX, bool PAIRED>
__global__ void __launch_bounds__(kBlock) qk_kernel(QKParams p)
{
    __shared__ float lds[kBlock / 64];
    constexpr int RPB = kBlock / TPR;
    const int lrow = threadIdx.x / TPR;
    const int lane = threadIdx.x % TPR;
    const bool is_q = PAIRED || static_cast<int64_t>(blockIdx.x) < p.q_groups;
    const QKDev t = is_q ? p.q : p.k;
    const int64_t grp = is_q ? blockIdx.x : blockIdx.x - p.q_groups;
    // One row per block: the row (and so the compact index) is block-uniform
    // and its index is fetched with a scalar load.
    int64_t row = RPB == 1 ? grp : grp * RPB + lrow;
    const bool active = row < t.rows;
    row = active ? row : t.rows - 1;
    const SlotPos<S> sp = slot_pos<TPR, S>(p, lane);
    constexpr int TA = AX > 0 ? AX : 0;

    // Order of the loads: the compact index, then the streamed rows, then the
    // table rows that depend on the index (cache hits), so the index latency
    // overlaps the row loads instead of preceding them.
    TabIdx<TA> ti{};
    if constexpr (AX > 0) ti = index_fetch<TA>(t, row);
    RowWork<TPR, S> wq, wk;
    wq.load(t, p, row, sp);
    if constexpr (PAIRED) wk.load(p.k, p, row, sp);
    __builtin_amdgcn_sched_barrier(0);  // keep every row load ahead of the wait for the index
    TabRefs<TA, S> tr;
    TabRaw<TA> traw[S];
    if constexpr (AX >= 0) {
        table_offsets<TA, S>(t, p, row, sp, ti, tr);
        table_fetch<TA, S>(t, tr, traw);
    }

    Pair8 dq[S], dk[S];
    const float ssq = wq.sumsq(dq, sp);
    float ssk = 0.f;
    if constexpr (PAIRED) ssk = wk.sumsq(dk, sp);
    float rq = 1.f, rk = 1.f;
    if (t.w) rq = rsqrtf(row_sum<TPR>(ssq, lds) / static_cast<float>(p.dim) + p.eps);
    if constexpr (PAIRED)
        if (p.k.w) rk = rsqrtf(row_sum<TPR>(ssk, lds) / static_cast<float>(p.dim) + p.eps);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < S; ++k) {
        if (!sp.ok[k]) continue;
        const int64_t off = sp.h[k] * p.head_dim + sp.j8[k];
        if (t.w) wq.weight(dq[k], k, rq);
        if constexpr (PAIRED)
            if (p.k.w) wk.weight(dk[k], k, rk);
        if constexpr (AX >= 0) {
            float c[8], s[8];
            table_values<TA>(traw[k], c, s);
            rotate(dq[k], c, s);
            if constexpr (PAIRED) rotate(dk[k], c, s);
        }
        store_pair(t.x + row * p.dim, off, p.half, dq[k]);
        if constexpr (PAIRED) store_pair(p.k.x + row * p.dim, off, p.half, dk[k]);
    }
}

QKDev make_dev(const ltxk_qk *t)
{
    QKDev d{};
    if (!t || !t->x) return d;
    d.x = static_cast<uint16_t *>(t->x);
    d.w = static_cast<const uint16_t *>(t->weight);
    d.cos = static_cast<const uint16_t *>(t->cos);
    d.sin = static_cast<const uint16_t *>(t->sin);
    d.idx = t->pos_index;
    d.rows = t->batch * t->tokens;
    d.tokens = t->tokens;
    d.tbs = t->table_bstride;
    return d;
}

// Table mode of an operand: -1 none, 0 full, n compact with n axes.
int table_mode(const ltxk_qk *t) { return t->cos == nullptr ? -1 : (t->pos_index ? static_cast<int>(t->n_axes) : 0); }

int check_operand(const ltxk_qk *t, const char *name)
{
    static const char *what = "qk_norm_rope";
    if (t->batch < 0 || t->tokens < 0) return fail(LTXK_E_ARG, "%s: %s has negative batch/tokens", what, name);
    if (t->batch * t->tokens > 0x7fffffff) return fail(LTXK_E_ARG, "%s: %s has too many rows", what, name);
    if (!aligned16(t->x) || !aligned16(t->weight) || !aligned16(t->cos) || !aligned16(t->sin))
        return fail(LTXK_E_ALIGN, "%s: %s buffers must be 16-byte aligned", what, name);
    if ((t->cos == nullptr) != (t->sin == nullptr))
        return fail(LTXK_E_ARG, "%s: %s needs both cos and sin or neither", what, name);
    if (t->cos && !t->pos_index && (t->table_bstride % 8))
        return fail(LTXK_E_ALIGN, "%s: %s table_bstride must be a multiple of 8", what, name);
    if (t->pos_index && (t->n_axes < 1 || t->n_axes > 3))
        return fail(LTXK_E_ARG, "%s: %s compact tables need 1..3 axes (got %lld)", what, name, (long long)t->n_axes);
    if (t->pos_index && !t->cos) return fail(LTXK_E_ARG, "%s: %s has a position index but no tables", what, name);
    return LTXK_OK;
}

template <int TPR, int S, int AX>
void launch_mode(const QKParams &p, bool paired, unsigned grid, hipStream_t s)
{
    if (paired)
        qk_kernel<TPR, S, AX, true><<<dim3(grid), dim3(kBlock), 0, s>>>(p);
    else
        qk_kernel<TPR, S, AX, false><<<dim3(grid), dim3(kBlock), 0, s>>>(p);
}

template <int TPR, int S>
int launch_geom(const QKParams &p, int mode, bool paired, unsigned grid, hipStream_t s)
{
    switch (mode) {
    case -1: launch_mode<TPR, S, -1>(p, paired, grid, s); return LTXK_OK;
    case 0: launch_mode<TPR, S, 0>(p, paired, grid, s); return LTXK_OK;
    case 1: launch_mode<TPR, S, 1>(p, paired, grid, s); return LTXK_OK;
    case 2: launch_mode<TPR, S, 2>(p, paired, grid, s); return LTXK_OK;
    case 3: launch_mode<TPR, S, 3>(p, paired, grid, s); return LTXK_OK;
    default: return fail(LTXK_E_ARG, "qk_norm_rope: bad table mode %d", mode);
    }
}

// One launch over q (and k): both operands must share the table mode.
int launch(QKParams p, int mode, bool paired, hipStream_t s)
{
    int tpr = 1;
    while (tpr < p.slots && tpr < kBlock) tpr <<= 1;
    const int64_t per = (p.slots + tpr - 1) / tpr;
    const int rpb = kBlock / tpr;
    const int64_t qg = (p.q.rows + rpb - 1) / rpb;
    const int64_t kg = p.k.x ? (p.k.rows + rpb - 1) / rpb : 0;
    p.q_groups = qg;
    const int64_t grid = paired ? qg : qg + kg;
    if (grid == 0) return LTXK_OK;
    if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "qk_norm_rope: too many rows");
    const unsigned g = static_cast<unsigned>(grid);
    int rc;
    if (tpr <= 1) rc = launch_geom<1, 1>(p, mode, paired, g, s);
    else if (tpr == 2) rc = launch_geom<2, 1>(p, mode, paired, g, s);
    else if (tpr == 4) rc = launch_geom<4, 1>(p, mode, paired, g, s);
    else if (tpr == 8) rc = launch_geom<8, 1>(p, mode, paired, g, s);
    else if (tpr == 16) rc = launch_geom<16, 1>(p, mode, paired, g, s);
    else if (tpr == 32) rc = launch_geom<32, 1>(p, mode, paired, g, s);
    else if (tpr == 64) rc = launch_geom<64, 1>(p, mode, paired, g, s);
    else if (tpr == 128) rc = launch_geom<128, 1>(p, mode, paired, g, s);
    else if (per <= 1) rc = launch_geom<256, 1>(p, mode, paired, g, s);
    else if (per <= 2) rc = launch_geom<256, 2>(p, mode, paired, g, s);
    else if (per <= 4) rc = launch_geom<256, 4>(p, mode, paired, g, s);
    else rc = launch_geom<256, 8>(p, mode, paired, g, s);
    if (rc) return rc;
    return check_launch("qk_norm_rope");
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int ltxk_qk_norm_rope(const ltxk_qk *q, const ltxk_qk *k, int64_t heads, int64_t head_dim, float eps,
                                 void *stream)
{
    static const char *what = "qk_norm_rope";
    clear_error();
    if (!q || !q->x) return fail(LTXK_E_ARG, "%s: q.x is required", what);
    if (heads <= 0 || head_dim <= 0 || head_dim % 16)
        return fail(LTXK_E_ARG, "%s: head_dim must be a positive multiple of 16 (got %lld)", what,
                    (long long)head_dim);
    const int64_t dim = heads * head_dim;
    if (dim > 16 * kBlock * 8) return fail(LTXK_E_ARG, "%s: heads*head_dim %lld above 32768", what, (long long)dim);
    int rc = check_operand(q, "q");
    if (rc) return rc;
    const bool has_k = k && k->x;
    if (has_k && (rc = check_operand(k, "k"))) return rc;

    QKParams p{};
    p.q = make_dev(q);
    p.dim = dim;
    p.head_dim = head_dim;
    p.half = head_dim / 2;
    p.slots = dim / 16;
    p.slots_per_head = head_dim / 16;
    p.eps = eps;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int qmode = table_mode(q);
    if (!has_k) return launch(p, qmode, false, s);
    const int kmode = table_mode(k);
    const bool same_tables = q->cos == k->cos && q->sin == k->sin && q->pos_index == k->pos_index &&
                             q->batch == k->batch && q->tokens == k->tokens &&
                             (q->cos == nullptr || q->pos_index || q->table_bstride == k->table_bstride);
    if (same_tables) {  // self-attention: one pass over both, tables fetched once
        p.k = make_dev(k);
        return launch(p, qmode, true, s);
    }
    if (qmode == kmode) {  // one launch, q rows then k rows
        p.k = make_dev(k);
        return launch(p, qmode, false, s);
    }
    if ((rc = launch(p, qmode, false, s))) return rc;
    QKParams pk = p;
    pk.q = make_dev(k);
    return launch(pk, kmode, false, s);
}
