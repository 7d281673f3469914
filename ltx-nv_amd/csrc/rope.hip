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
// Workgroups per CU of the persistent q/k kernels.  Measured on the
// [6144, 4096] video pair (buffers rotating past the MALL): the slot kernel
// 40.8 us at 3 per CU, 39.0 at 6, 37.9 at 6 with streaming stores; 43.7 at
// 4 and 45.1 at 24; with streaming stores 41.4 at 5, 38.0 at 7 and 40.5 at
// 8.  The contiguous-chunk kernel on the [6144, 2048] pair
// 21.1-21.4 us at 3 per CU, 23.4 at 2, 21.7 at 4, 22.9 at 6.
#ifndef LTXK_SLOT_PER_CU
#define LTXK_SLOT_PER_CU 6
#endif
#ifndef LTXK_CHUNK_PER_CU
#define LTXK_CHUNK_PER_CU 3
#endif

struct QKDev {
    uint16_t *x;
    const uint16_t *w;
    const uint16_t *cos;
    const uint16_t *sin;
    const int32_t *idx;  // compact tables: [rows, n_axes] table rows per token
    uint32_t tab_rows;   // compact tables: rows R of cos/sin; indexes are clamped into [0, R)
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
    for (int a = 0; a < AX; ++a) {
        // unsigned compare: a negative index clamps to the last row as well
        const uint32_t r = static_cast<uint32_t>(t.idx[row * AX + a]);
        ti.r[a] = static_cast<int32_t>(r < t.tab_rows ? r : t.tab_rows - 1);
    }
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
    // rx: buffer range over the workgroup's rows of t.x; rowoff: this thread's
    // row within it, in bytes (past the range for a missing row: zeros)
    __device__ void load(const QKDev &t, const QKParams &p, rsrc_t rx, uint32_t rowoff, const SlotPos<S> &sp)
    {
        const uint16_t *w = t.w ? t.w : g_ada_zeros;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            const int64_t off = sp.h[k] * p.head_dim + sp.j8[k];
            xa[k] = ldb4(rx, rowoff + static_cast<uint32_t>(off * 2));
            xb[k] = ldb4(rx, rowoff + static_cast<uint32_t>((off + p.half) * 2));
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

__device__ __forceinline__ void store_pair(rsrc_t rx, uint32_t rowoff, int64_t off, int64_t half, const Pair8 &d)
{
    stb(rx, rowoff + static_cast<uint32_t>(off * 2), pack8v(d.a));
    stb(rx, rowoff + static_cast<uint32_t>((off + half) * 2), pack8v(d.b));
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
    // the workgroup's rows [row0, row0 + nrows) of q (and k) as buffer ranges
    const int64_t row0 = grp * RPB;
    const int64_t nrows = t.rows - row0 < RPB ? t.rows - row0 : RPB;
    const uint32_t rowoff = static_cast<uint32_t>(lrow * p.dim * 2);
    const rsrc_t rxq = make_rsrc(t.x + row0 * p.dim, static_cast<uint32_t>(nrows * p.dim * 2));
    const rsrc_t rxk = make_rsrc((PAIRED ? p.k.x : t.x) + row0 * p.dim,
                                 PAIRED ? static_cast<uint32_t>(nrows * p.dim * 2) : 0u);

    // Order of the loads: the compact index, then the streamed rows, then the
    // table rows that depend on the index (cache hits), so the index latency
    // overlaps the row loads instead of preceding them.
    TabIdx<TA> ti{};
    if constexpr (AX > 0) ti = index_fetch<TA>(t, row);
    RowWork<TPR, S> wq, wk;
    wq.load(t, p, rxq, rowoff, sp);
    if constexpr (PAIRED) wk.load(p.k, p, rxk, rowoff, sp);
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
        store_pair(rxq, rowoff, off, p.half, dq[k]);
        if constexpr (PAIRED) store_pair(rxk, rowoff, off, p.half, dk[k]);
    }
}

// base + a 32-bit byte offset: with a workgroup-uniform base this is the
// scalar-base + vector-offset addressing form (one offset register for many
// loads and stores).
__device__ __forceinline__ const void *at(const void *base, uint32_t bytes)
{
    return static_cast<const char *>(base) + bytes;
}
__device__ __forceinline__ void *at(void *base, uint32_t bytes) { return static_cast<char *>(base) + bytes; }

// Hides v's value from the optimiser (no instruction): unpacking it again
// afterwards is not merged with an earlier unpack, so the raw words, not the
// floats, stay live across a barrier.
__device__ __forceinline__ void opaque(uint4 &v) { asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)); }

// Compact tables, rows of at most kBlock slots (inner dim <= 4096), R
// consecutive rows per workgroup: every load of the R rows is issued before
// the first use, the weights are loaded once for the R rows, and a table row
// that consecutive rows share (the same coordinate on that axis, as
// neighbouring tokens of a latent grid do on the slower axes) is loaded once.
// One barrier for the R rows' sums.
template <int R, int AX, bool PAIRED, bool NORM>
__global__ void __launch_bounds__(kBlock) qk_rows_kernel(QKParams p)
{
    static_assert(AX >= 1 && AX <= 3, "compact tables only");
    constexpr int W = kBlock / 64;
    constexpr int TA = AX;
    constexpr int NA = AX;
    __shared__ float lds[R * 2 * W];
    const int lane = threadIdx.x, wave = lane >> 6;
    const bool is_q = PAIRED || static_cast<int64_t>(blockIdx.x) < p.q_groups;
    const QKDev t = is_q ? p.q : p.k;
    const int64_t grp = is_q ? blockIdx.x : blockIdx.x - p.q_groups;
    const SlotPos<1> sp = slot_pos<kBlock, 1>(p, lane);
    // 32-bit byte offsets from workgroup-uniform row pointers: one offset
    // register for every load and store (scalar base + vector offset)
    const uint32_t off = static_cast<uint32_t>(sp.h[0] * p.head_dim + sp.j8[0]) * 2;  // bytes
    const uint32_t half = static_cast<uint32_t>(p.half) * 2;
    const uint32_t toff = static_cast<uint32_t>(sp.h[0] * p.half + sp.j8[0]) * 2;  // in a table row
    int64_t row[R];
    bool act[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        row[j] = grp * R + j;
        act[j] = row[j] < t.rows;
        row[j] = act[j] ? row[j] : t.rows - 1;
    }
    TabIdx<TA> ti[R];
#pragma unroll
    for (int j = 0; j < R; ++j) ti[j] = index_fetch<TA>(t, row[j]);
    // each row as a buffer range (empty for a missing row: zeros, stores dropped)
    rsrc_t rq[R], rk[R];
    uint4 qa[R], qb[R], ka[R], kb[R];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const uint32_t nb = act[j] ? static_cast<uint32_t>(p.dim * 2) : 0u;
        rq[j] = make_rsrc(t.x + row[j] * p.dim, nb);
        qa[j] = ldb4(rq[j], off);
        qb[j] = ldb4(rq[j], off + half);
        if constexpr (PAIRED) {
            rk[j] = make_rsrc(p.k.x + row[j] * p.dim, nb);
            ka[j] = ldb4(rk[j], off);
            kb[j] = ldb4(rk[j], off + half);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every row load ahead of the wait for the index
    TabRaw<TA> traw[R] = {};
    int src[R][NA];  // the row whose table registers serve row j on axis a
#pragma unroll
    for (int j = 0; j < R; ++j) {
#pragma unroll
        for (int a = 0; a < NA; ++a) {
            const bool reuse = j > 0 && ti[j].r[a] == ti[j - 1].r[a];  // workgroup-uniform
            src[j][a] = reuse ? src[j - 1][a] : j;
            if (!reuse) {
                const int64_t base = static_cast<int64_t>(ti[j].r[a]) * (p.dim / 2);
                traw[j].c[a] = ld16(at(t.cos + base, toff));
                traw[j].s[a] = ld16(at(t.sin + base, toff));
            }
        }
    }

    // sums of squares from the raw words; the values are unpacked again after
    // the barrier rather than held as floats across it.  Without a norm on
    // either operand (NORM false) there is nothing to reduce.
#pragma unroll
    for (int j = 0; j < (NORM ? R : 0); ++j) {
        float ssq = 0.f, ssk = 0.f;
        if (sp.ok[0]) {
            Pair8 d;
            unpack8(qa[j], d.a);
            unpack8(qb[j], d.b);
#pragma unroll
            for (int i = 0; i < 8; ++i) ssq = __builtin_fmaf(d.b[i], d.b[i], __builtin_fmaf(d.a[i], d.a[i], ssq));
            if constexpr (PAIRED) {
                unpack8(ka[j], d.a);
                unpack8(kb[j], d.b);
#pragma unroll
                for (int i = 0; i < 8; ++i) ssk = __builtin_fmaf(d.b[i], d.b[i], __builtin_fmaf(d.a[i], d.a[i], ssk));
            }
        }
        ssq = wave_sum64(ssq);
        if constexpr (PAIRED) ssk = wave_sum64(ssk);
        if ((lane & 63) == 0) {
            lds[(2 * j) * W + wave] = ssq;
            lds[(2 * j + 1) * W + wave] = ssk;
        }
    }
    // the weights (cache hits) are needed only after the barrier
    const uint4 wqa = t.w ? ld16(at(t.w, off)) : uint4{}, wqb = t.w ? ld16(at(t.w, off + half)) : uint4{};
    uint4 wka{}, wkb{};
    if constexpr (PAIRED) {
        if (p.k.w) {  // uniform
            wka = ld16(at(p.k.w, off));
            wkb = ld16(at(p.k.w, off + half));
        }
    }
    if constexpr (NORM) __syncthreads();
    if (!sp.ok[0]) return;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (!act[j]) continue;
        float tq = 0.f, tk = 0.f;
        if constexpr (NORM)
#pragma unroll
            for (int w = 0; w < W; ++w) {
                tq += lds[(2 * j) * W + w];
                tk += lds[(2 * j + 1) * W + w];
            }
        float c[8], sn[8];
        {
            TabRaw<TA> use;
#pragma unroll
            for (int a = 0; a < NA; ++a) {
                use.c[a] = traw[0].c[a];
                use.s[a] = traw[0].s[a];
#pragma unroll
                for (int jj = 1; jj <= j; ++jj)
                    if (src[j][a] == jj) {
                        use.c[a] = traw[jj].c[a];
                        use.s[a] = traw[jj].s[a];
                    }
            }
            table_values<TA>(use, c, sn);
        }
        // one tensor at a time (q, then k): bounds the live floats
        auto finish = [&](uint4 xa, uint4 xb, const uint4 &wa, const uint4 &wb, bool has_w, float tot, rsrc_t rx) {
            opaque(xa);
            opaque(xb);
            Pair8 d;
            unpack8(xa, d.a);
            unpack8(xb, d.b);
            if (has_w) {
                const float r = rsqrtf(tot / static_cast<float>(p.dim) + p.eps);
                float fa[8], fb[8];
                unpack8(wa, fa);
                unpack8(wb, fb);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    d.a[i] = (d.a[i] * r) * fa[i];
                    d.b[i] = (d.b[i] * r) * fb[i];
                }
            }
            rotate(d, c, sn);
            stb(rx, off, pack8v(d.a));
            stb(rx, off + half, pack8v(d.b));
        };
        finish(qa[j], qb[j], wqa, wqb, t.w != nullptr, tq, rq[j]);
        if constexpr (PAIRED) {
            __builtin_amdgcn_sched_barrier(0);
            finish(ka[j], kb[j], wka, wkb, p.k.w != nullptr, tk, rk[j]);
        }
        __builtin_amdgcn_sched_barrier(0);  // one row at a time: bounds the live floats
    }
}

// ---------------------------------------------------------------- streaming --
// Persistent form for self-attention q/k pairs (shared compact tables) with
// rows of 128 or 256 slots (inner dim 2048 or 4096).  A row group is RPI =
// 256/TPR consecutive rows of q and the same rows of k; workgroup w takes a
// contiguous run of groups.  The norm weights stay in registers (as floats)
// for the whole launch; while group g is reduced, rotated and written, the
// next group's q/k rows and table rows are already in flight in the other of
// two register stages (its index was fetched one group earlier), a stage keeps
// a table row it already holds, and the reduction
// takes one barrier per group (LDS partials double-buffered by parity).  Each
// thread owns one slot (8 rotation pairs of one head) of its row in q and in k.
template <int AX>
struct StreamStage {
    u32x4 qa, qb, ka, kb;    // the two halves of the slot in q and in k
    u32x4 c[AX], s[AX];      // table rows per axis
    int32_t tr[AX];          // which table row c/s hold (-1: none yet)
};

template <int TPR, int AX>
__global__ void __launch_bounds__(kBlock) qk_stream_kernel(QKParams p)
{
    static_assert(AX >= 1, "compact tables only");
    constexpr int RPI = kBlock / TPR;  // rows per group
    constexpr int W = kBlock / 64;
    __shared__ float lds[2][2][W];  // [parity][q, k][wave]
    const int tid = threadIdx.x, wave = tid >> 6;
    const int lrow = tid / TPR, lane = tid % TPR;
    // the operands by value: scalar registers for the whole launch (a
    // reference into the parameter block is re-read from memory every group)
    const QKDev Q = p.q, K = p.k;
    const int64_t groups = p.q_groups;
    // With two or more table axes workgroup w takes the contiguous groups
    // [w*per, (w+1)*per): neighbouring tokens share the slower axes' table
    // rows, which are then kept in registers.  With one axis every token has
    // its own row and the groups are dealt out w, w + grid, ...: the launch
    // then sweeps the tensors in address order (measured 17.1-17.2 against
    // 17.8-17.9 us for the A2V q + V2A k pair; 39.9 against 37.4 us for the
    // video self-attention pair on two axes).
    const int64_t per = (groups + gridDim.x - 1) / gridDim.x;
    const int64_t gbeg = AX == 1 ? blockIdx.x : blockIdx.x * per;
    const int64_t G = AX == 1 ? gridDim.x : 1;
    const int64_t gend = AX == 1 ? groups : (gbeg + per < groups ? gbeg + per : groups);
    const int64_t h = udiv32(lane, p.slots_per_head);
    const int64_t j8 = (lane - h * p.slots_per_head) * 8;
    const uint32_t off = static_cast<uint32_t>((lrow * p.dim + h * p.head_dim + j8) * 2);  // in a group's range
    const uint32_t half = static_cast<uint32_t>(p.half * 2);
    const int64_t toff = h * p.half + j8;  // in a table row
    const int64_t trow = p.dim / 2;        // elements per table row

    // norm weights of q and k as floats, once for the launch (zeros when absent)
    float wq[2][8], wk[2][8];
    {
        const uint16_t *pq = Q.w ? Q.w : g_ada_zeros, *pk = K.w ? K.w : g_ada_zeros;
        const int64_t wo = h * p.head_dim + j8;
        unpack8(ld16(pq + (Q.w ? wo : 0)), wq[0]);
        unpack8(ld16(pq + (Q.w ? wo + p.half : 0)), wq[1]);
        unpack8(ld16(pk + (K.w ? wo : 0)), wk[0]);
        unpack8(ld16(pk + (K.w ? wo + p.half : 0)), wk[1]);
    }
    // rows of 2048 or 4096: 1/dim is a power of two, so tot * inv_dim rounds
    // exactly as tot / dim
    const float inv_dim = 1.0f / static_cast<float>(p.dim);

    // first row and row count of group g (g past this workgroup's end: no rows)
    auto rows_of = [&](int64_t g, int64_t &row0) {
        row0 = g >= gend ? 0 : g * RPI;
        return g >= gend ? int64_t(0) : (Q.rows - row0 < RPI ? Q.rows - row0 : int64_t(RPI));
    };
    auto fetch_index = [&](int64_t g) {
        int64_t row0;
        rows_of(g, row0);
        const int64_t r = row0 + lrow < Q.rows ? row0 + lrow : Q.rows - 1;  // in range, for the index
        if constexpr (RPI == 1) {
            // one row per group: the index is the same for the whole workgroup;
            // read it through the scalar cache (constant address space), so
            // waiting for it does not wait for this workgroup's vector stores
            const int32_t ru = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(r));
            const __attribute__((address_space(4))) int32_t *ci =
                (const __attribute__((address_space(4))) int32_t *)(Q.idx);
            TabIdx<AX> ti;
#pragma unroll
            for (int a = 0; a < AX; ++a) {
                const uint32_t v = static_cast<uint32_t>(ci[static_cast<int64_t>(ru) * AX + a]);
                ti.r[a] = static_cast<int32_t>(v < Q.tab_rows ? v : Q.tab_rows - 1);
            }
            return ti;
        } else {
            return index_fetch<AX>(Q, r);
        }
    };
    // A stage keeps the table rows it last held: a row equal to it (the slow
    // axes change every few tokens) is not loaded again.  The check is against
    // the stage's own rows, not the other stage's, so no register is copied
    // from a stage whose loads may still be in flight (a copy would wait for
    // them, and for every store issued after them).
    auto load = [&](int64_t g, const TabIdx<AX> &ti, StreamStage<AX> &st) {
        int64_t row0;
        const uint32_t nb = static_cast<uint32_t>(rows_of(g, row0) * p.dim * 2);
        const rsrc_t rq = make_rsrc(Q.x + row0 * p.dim, nb), rk = make_rsrc(K.x + row0 * p.dim, nb);
        st.qa = ldb(rq, off);
        st.qb = ldb(rq, off + half);
        st.ka = ldb(rk, off);
        st.kb = ldb(rk, off + half);
#pragma unroll
        for (int a = 0; a < AX; ++a) {
            if (ti.r[a] == st.tr[a]) continue;
            const int64_t e = static_cast<int64_t>(ti.r[a]) * trow + toff;
            st.c[a] = *reinterpret_cast<const u32x4 *>(Q.cos + e);
            st.s[a] = *reinterpret_cast<const u32x4 *>(Q.sin + e);
            st.tr[a] = ti.r[a];
        }
    };
    // reduce, normalise, rotate and store group g from stage cur
    auto compute = [&](int64_t g, const StreamStage<AX> &cur, int par) {
        int64_t row0;
        const uint32_t nb = static_cast<uint32_t>(rows_of(g, row0) * p.dim * 2);
        Pair8 dq, dk;
        unpack8v(cur.qa, dq.a);
        unpack8v(cur.qb, dq.b);
        unpack8v(cur.ka, dk.a);
        unpack8v(cur.kb, dk.b);
        float ssq = 0.f, ssk = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ssq = __builtin_fmaf(dq.b[i], dq.b[i], __builtin_fmaf(dq.a[i], dq.a[i], ssq));
            ssk = __builtin_fmaf(dk.b[i], dk.b[i], __builtin_fmaf(dk.a[i], dk.a[i], ssk));
        }
        ssq = wave_sum64(ssq);
        ssk = wave_sum64(ssk);
        if ((tid & 63) == 0) {
            lds[par][0][wave] = ssq;
            lds[par][1][wave] = ssk;
        }
        __syncthreads();
        float tq = 0.f, tk = 0.f;
#pragma unroll
        for (int q = 0; q < W / RPI; ++q) {
            tq += lds[par][0][lrow * (W / RPI) + q];
            tk += lds[par][1][lrow * (W / RPI) + q];
        }
        u32x4 rc = cur.c[0], rs = cur.s[0];
#pragma unroll
        for (int a = 1; a < AX; ++a) {
            rc |= cur.c[a];
            rs |= cur.s[a];
        }
        float c[8], sn[8];
        unpack8v(rc, c);
        unpack8v(rs, sn);
        auto finish = [&](Pair8 &d, bool has_w, const float (&w)[2][8], float tot, uint16_t *x) {
            if (has_w) {
                const float r = rsqrtf(tot * inv_dim + p.eps);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    d.a[i] = (d.a[i] * r) * w[0][i];
                    d.b[i] = (d.b[i] * r) * w[1][i];
                }
            }
            rotate(d, c, sn);
            const rsrc_t rx = make_rsrc(x + row0 * p.dim, nb);
            // streaming stores (measured faster here than write-through);
            // rows past the group's end are dropped
            stb_stream(rx, off, pack8v(d.a));
            stb_stream(rx, off + half, pack8v(d.b));
        };
        finish(dq, Q.w != nullptr, wq, tq, Q.x);
        finish(dk, K.w != nullptr, wk, tk, K.x);
    };

    int64_t g = gbeg;
    if (g >= gend) return;  // uniform
    TabIdx<AX> ti_next = fetch_index(g + G);
    // two stages used in turn: group g computes from one while the next
    // group's loads land in the other (no register copies between groups)
    StreamStage<AX> sa, sb;
#pragma unroll
    for (int a = 0; a < AX; ++a) sa.tr[a] = sb.tr[a] = -1;
    load(g, fetch_index(g), sa);
    auto step = [&](const StreamStage<AX> &cur, StreamStage<AX> &nxt, int par) {
        const int64_t gn = g + G;
        const TabIdx<AX> ti_after = fetch_index(gn + G);
        load(gn, ti_next, nxt);  // past the end: empty ranges, cached table rows
        compute(g, cur, par);
        ti_next = ti_after;
        g = gn;
        return gn < gend;
    };
    while (step(sa, sb, 0) && step(sb, sa, 1)) {
    }
}

unsigned stream_grid(int64_t groups, int per_cu);

// ------------------------------------------------------- contiguous chunks --
// Persistent form with contiguous chunks, for self-attention pairs of rows of
// 256*CH chunks with heads of 16*PX elements (launched for rows of 2048 with
// heads of 64 on two- or three-axis tables: CH = 1, PX = 4; one-axis tables
// take the wave-token form below): thread t owns the 16-byte chunks t + c*256 of
// a row, so every load and store
// instruction of a wave covers one contiguous 1 KiB span.  The rotation
// partner of a chunk (same pair index, other half of the head) is chunk
// ^ PX with PX = head_dim/16; its raw words come from that lane through
// ds_swizzle (lane ^ PX inside a 32-lane group), and each lane writes only
// its own chunk:
//   first half   out = x*c - p*s
//   second half  out = x*c + p*s
// with x the lane's normalised, weighted value and p the partner's, the
// same operations as the reference's pair form (standalone/ltx_nn.py:99-115).
// With the slot form (a thread owns both halves of 8 pairs), a wave's load
// of 64-wide heads touches every 128-byte line twice, half each time: on the
// A2V q + V2A k pair ([6144, 2048] each) 25.5 us against 20.5 us for the
// contiguous access pattern.
template <int X>
__device__ __forceinline__ u32x4 swizzle_xor(const u32x4 &v)
{
    constexpr int pattern = (X << 10) | 0x1F;  // bitmask mode: and 0x1f, or 0, xor X
    return u32x4{static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v[0]), pattern)),
                 static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v[1]), pattern)),
                 static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v[2]), pattern)),
                 static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v[3]), pattern))};
}

template <int CH, int AX>
struct ChunkStage {
    u32x4 q[CH], k[CH];          // the lane's own chunks of the row in q and in k
    u32x4 c[CH][AX], s[CH][AX];  // table chunks per axis
    int32_t tr[AX];              // which table row c/s hold (-1: none yet)
};

template <int CH, int PX, int AX>
__global__ void __launch_bounds__(kBlock) qk_chunk_kernel(QKParams p)
{
    static_assert(AX >= 1, "compact tables only");
    constexpr int W = kBlock / 64;
    __shared__ float lds[2][2][W];  // [parity][q, k][wave]
    const int tid = threadIdx.x, wave = tid >> 6;
    const QKDev Q = p.q, K = p.k;
    const int64_t groups = p.q_groups;  // one row per group
    // each workgroup a contiguous run of rows, for every axis count: with the
    // time axis alone a run stays in one frame and fetches its table row once
    // (rows dealt 768 apart changed the row at every step: 21.4 against
    // 20.3 us on the [6144, 2048] A2V q + V2A k pair)
    const int64_t per = (groups + gridDim.x - 1) / gridDim.x;
    const int64_t gbeg = blockIdx.x * per;
    constexpr int64_t G = 1;
    const int64_t gend = gbeg + per < groups ? gbeg + per : groups;
    const uint32_t rbytes = static_cast<uint32_t>(p.dim * 2);
    const int64_t trow = p.dim / 2;  // elements per table row

    uint32_t off[CH];   // byte offset of the chunk in a row
    int64_t toff[CH];   // element offset of its pair index in a table row
    bool first[CH];     // the chunk is in the first half of its head
    u32x4 wqo[CH], wqp[CH], wko[CH], wkp[CH];  // norm weights: own and partner chunk, raw bf16
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t e = 8 * (static_cast<int64_t>(tid) + c * kBlock);
        const int64_t h = udiv32(e, p.head_dim);
        const int64_t pos = e - h * p.head_dim;
        first[c] = pos < p.half;
        toff[c] = h * p.half + (first[c] ? pos : pos - p.half);
        off[c] = static_cast<uint32_t>(e * 2);
        const int64_t ep = e ^ (8 * PX);
        const uint16_t *pq = Q.w ? Q.w : g_ada_zeros, *pk = K.w ? K.w : g_ada_zeros;
        wqo[c] = *reinterpret_cast<const u32x4 *>(pq + (Q.w ? e : 0));
        wqp[c] = *reinterpret_cast<const u32x4 *>(pq + (Q.w ? ep : 0));
        wko[c] = *reinterpret_cast<const u32x4 *>(pk + (K.w ? e : 0));
        wkp[c] = *reinterpret_cast<const u32x4 *>(pk + (K.w ? ep : 0));
    }
    // rows of 2048 or 4096: 1/dim is a power of two, so tot * inv_dim rounds
    // exactly as tot / dim
    const float inv_dim = 1.0f / static_cast<float>(p.dim);

    // the group's row index through the scalar cache (workgroup-uniform), so
    // waiting for it does not wait for this workgroup's vector stores
    auto fetch_index = [&](int64_t g) {
        const int64_t r = g < gend ? g : gend - 1;
        const int32_t ru = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(r));
        const __attribute__((address_space(4))) int32_t *ci =
            (const __attribute__((address_space(4))) int32_t *)(Q.idx);
        TabIdx<AX> ti;
#pragma unroll
        for (int a = 0; a < AX; ++a) {
            const uint32_t v = static_cast<uint32_t>(ci[static_cast<int64_t>(ru) * AX + a]);
            ti.r[a] = static_cast<int32_t>(v < Q.tab_rows ? v : Q.tab_rows - 1);
        }
        return ti;
    };
    auto load = [&](int64_t g, const TabIdx<AX> &ti, ChunkStage<CH, AX> &st) {
        const bool ok = g < gend;
        const int64_t row = ok ? g : 0;
        const rsrc_t rq = make_rsrc(Q.x + row * p.dim, ok ? rbytes : 0u);
        const rsrc_t rk = make_rsrc(K.x + row * p.dim, ok ? rbytes : 0u);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            st.q[c] = ldb(rq, off[c]);
            st.k[c] = ldb(rk, off[c]);
        }
#pragma unroll
        for (int a = 0; a < AX; ++a) {
            if (ti.r[a] == st.tr[a]) continue;  // workgroup-uniform
            const int64_t base = static_cast<int64_t>(ti.r[a]) * trow;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                st.c[c][a] = *reinterpret_cast<const u32x4 *>(Q.cos + base + toff[c]);
                st.s[c][a] = *reinterpret_cast<const u32x4 *>(Q.sin + base + toff[c]);
            }
            st.tr[a] = ti.r[a];
        }
    };
    auto compute = [&](int64_t g, const ChunkStage<CH, AX> &cur, int par) {
        const bool ok = g < gend;
        const int64_t row = ok ? g : 0;
        u32x4 pq[CH], pk[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            pq[c] = swizzle_xor<PX>(cur.q[c]);
            pk[c] = swizzle_xor<PX>(cur.k[c]);
        }
        float ssq = 0.f, ssk = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            float vq[8], vk[8];
            unpack8v(cur.q[c], vq);
            unpack8v(cur.k[c], vk);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ssq = __builtin_fmaf(vq[i], vq[i], ssq);
                ssk = __builtin_fmaf(vk[i], vk[i], ssk);
            }
        }
        ssq = wave_sum64(ssq);
        ssk = wave_sum64(ssk);
        if ((tid & 63) == 0) {
            lds[par][0][wave] = ssq;
            lds[par][1][wave] = ssk;
        }
        __syncthreads();
        float tq = 0.f, tk = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            tq += lds[par][0][w];
            tk += lds[par][1][w];
        }
        const rsrc_t rq = make_rsrc(Q.x + row * p.dim, ok ? rbytes : 0u);
        const rsrc_t rk = make_rsrc(K.x + row * p.dim, ok ? rbytes : 0u);
        auto finish = [&](const u32x4 &own, const u32x4 &par_raw, const u32x4 &wo, const u32x4 &wp, bool has_w,
                          float tot, const float cs[8], const float sn[8], bool fst, rsrc_t rx, uint32_t o) {
            float x[8], y[8];
            unpack8v(own, x);
            unpack8v(par_raw, y);
            if (has_w) {
                const float r = rsqrtf(tot * inv_dim + p.eps);
                float fo[8], fp[8];
                unpack8v(wo, fo);
                unpack8v(wp, fp);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    x[i] = (x[i] * r) * fo[i];
                    y[i] = (y[i] * r) * fp[i];
                }
            }
            float out[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float ps = y[i] * sn[i];
                out[i] = x[i] * cs[i] + (fst ? -ps : ps);  // a - b is a + (-b), bit for bit
            }
            stb(rx, o, pack8v(out));
        };
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            u32x4 rc = cur.c[c][0], rs = cur.s[c][0];
#pragma unroll
            for (int a = 1; a < AX; ++a) {
                rc |= cur.c[c][a];
                rs |= cur.s[c][a];
            }
            float cs[8], sn[8];
            unpack8v(rc, cs);
            unpack8v(rs, sn);
            finish(cur.q[c], pq[c], wqo[c], wqp[c], Q.w != nullptr, tq, cs, sn, first[c], rq, off[c]);
            finish(cur.k[c], pk[c], wko[c], wkp[c], K.w != nullptr, tk, cs, sn, first[c], rk, off[c]);
        }
    };

    int64_t g = gbeg;
    if (g >= gend) return;  // uniform
    TabIdx<AX> ti_next = fetch_index(g + G);
    ChunkStage<CH, AX> sa, sb;
#pragma unroll
    for (int a = 0; a < AX; ++a) sa.tr[a] = sb.tr[a] = -1;
    load(g, fetch_index(g), sa);
    auto step = [&](const ChunkStage<CH, AX> &cur, ChunkStage<CH, AX> &nxt, int par) {
        const int64_t gn = g + G;
        const TabIdx<AX> ti_after = fetch_index(gn + G);
        load(gn, ti_next, nxt);  // past the end: empty ranges, cached table rows
        compute(g, cur, par);
        ti_next = ti_after;
        g = gn;
        return gn < gend;
    };
    while (step(sa, sb, 0) && step(sb, sa, 1)) {
    }
}

// ------------------------------------------------------------ wave tokens --
// Persistent form with one wave per token, for self-attention pairs of rows
// of 2048 (4 chunks a lane) with heads of 16*PX elements and one-axis compact
// tables (the video-side A2V q + V2A k launch, the audio self-attention).
// Lane l owns the 16-byte chunks l + 64c of the token's q row and k row; a
// row's sum of squares is one wave reduction, so the token loop has no
// barrier.  Waves walk tokens w, w + NW, ... with the token's table chunks
// loaded with its rows: a lane in the first half of a head loads its pair
// index's cos chunk and its partner lane (l ^ PX, the same pair index) the
// sin chunk, and each takes the other's through ds_swizzle, so a token's
// tables cost 4 loads and 16 registers a lane.  As each output chunk is
// stored, its registers are refilled with the same chunk of the wave's next
// token.  The norm weights sit in LDS (the partner's at chunk ^ PX).  The
// arithmetic is the contiguous-chunk kernel's, operation for operation, with
// the row's sum in another order.
//
// Measured on the [6144, 2048] A2V q + V2A k pair (buffers rotating past the
// MALL, us): this form at four workgroups per CU and one token in registers
// 19.9-20.0, against 20.2-20.4 for the contiguous-chunk kernel; two tokens in
// registers (everything in flight from the start) 20.3 at three per CU and
// 21.8 at two (four per CU spills); loads issued back to back 20.2.  Timing
// copies of this form: loads and stores only 18.2, with the table loads 18.9,
// the arithmetic without the table loads 18.7; the 48-block chain is the same
// with it (17.20-17.21 ms, graph replay 17.01 against 17.05-17.06).  Streaming
// (nt) stores instead of write-through: 19.45 against 19.99 us, the chain
// 16.92-16.96 against 17.00-17.04 ms.
// Rows a one-wave-per-row launch takes: the kernels count rows in int and
// look up to a few wave strides (at most 4 x 1024 x 4 waves each) past a
// wave's row, so the count leaves 2^20 of headroom below 2^31.
constexpr int64_t kWaveRowsMax = 0x7fffffff - (int64_t{1} << 20);

constexpr int kPairPerCU = 4;
constexpr int kPairStages = 1;
constexpr int kPairLoadNops = 2;

template <int N>
__device__ __forceinline__ void pair_spacing()
{
#pragma unroll
    for (int q = 0; q < N; ++q) asm volatile("s_nop 7");
}

template <int PX>
__global__ void __launch_bounds__(kBlock, kPairPerCU) qk_pair_wave_kernel(QKParams p)
{
    // the head position must depend on the lane only, and the partner lane
    // (lane ^ PX) must be inside the 32-lane group ds_swizzle works on
    static_assert(PX >= 1 && PX <= 16 && (32 % PX) == 0, "PX must be a power of two up to 16");
    constexpr int CW = 4;           // 16-byte chunks a lane per row of 2048
    constexpr int kDim = 64 * 8 * CW;
    constexpr int kTrow = kDim / 2;  // elements per table row
    constexpr uint32_t kRowBytes = kDim * 2;
    __shared__ u32x4 lw[2][CW * 64];  // norm weights of q and k (raw bf16)
    const int lane = threadIdx.x & 63;
    const int NW = static_cast<int>(gridDim.x) * (kBlock / 64);
    // wave-uniform (lane 0's value), so token rows and resources stay scalar
    const int w = static_cast<int>(blockIdx.x) * (kBlock / 64) +
                  __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const QKDev Q = p.q, K = p.k;
    const int rows = static_cast<int>(Q.rows);
    const bool first = (lane & PX) == 0;  // the lane's chunks are in the first half of their heads
    // chunk lane + 64c starts at element 8*lane + 512c of the row: head
    // position 8*lane mod 16*PX; its pair index in the table row is toff +
    // 256c (a table row holds half a head per head: 512 elements of the row
    // are 256 of the table)
    const int hpos = (8 * lane) % (16 * PX);
    const int toff = ((8 * lane) / (16 * PX)) * (8 * PX) + (first ? hpos : hpos - 8 * PX);
    const uint16_t *tb = first ? Q.cos : Q.sin;
    const __attribute__((address_space(4))) int32_t *ci =
        (const __attribute__((address_space(4))) int32_t *)(Q.idx);
    auto table_row = [&](int r) {  // clamped into the tables; r past the end reads the last token's
        const uint32_t v = static_cast<uint32_t>(ci[r < rows ? r : rows - 1]);
        return static_cast<int64_t>(v < Q.tab_rows ? v : Q.tab_rows - 1) * kTrow;
    };
    auto rsrc_of = [&](uint16_t *base, int r) {
        const bool ok = r < rows;
        return make_rsrc(base + static_cast<int64_t>(ok ? r : 0) * kDim, ok ? kRowBytes : 0u);
    };

    int r = w;
    u32x4 sq[kPairStages][CW], sk[kPairStages][CW], st[kPairStages][CW];
#pragma unroll
    for (int j = 0; j < kPairStages; ++j) {
        const int rj = r + j * NW;
        const rsrc_t rq = rsrc_of(Q.x, rj), rk = rsrc_of(K.x, rj);
        const int64_t tr = table_row(rj);
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            sq[j][c] = ldb(rq, (lane + 64 * c) * 16u);
            pair_spacing<kPairLoadNops>();
        }
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            sk[j][c] = ldb(rk, (lane + 64 * c) * 16u);
            pair_spacing<kPairLoadNops>();
        }
#pragma unroll
        for (int c = 0; c < CW; ++c) st[j][c] = *reinterpret_cast<const u32x4 *>(tb + tr + toff + 256 * c);
    }
    // an absent weight: no normalisation, the raw values are rotated (scale
    // 1 and weights 1.0: (x * 1) * 1 is x, bit for bit)
    const bool has_wq = Q.w != nullptr, has_wk = K.w != nullptr;
    constexpr uint32_t kOnes = 0x3f803f80u;
    constexpr u32x4 ones = {kOnes, kOnes, kOnes, kOnes};
    for (int u = threadIdx.x; u < CW * 64; u += kBlock) {
        lw[0][u] = has_wq ? *reinterpret_cast<const u32x4 *>(Q.w + 8 * u) : ones;
        lw[1][u] = has_wk ? *reinterpret_cast<const u32x4 *>(K.w + 8 * u) : ones;
    }
    __syncthreads();
    // rows of 2048: 1/dim is a power of two, so tot * inv_dim rounds exactly as tot / dim
    constexpr float inv_dim = 1.0f / static_cast<float>(kDim);

    auto step = [&](u32x4 (&cq)[CW], u32x4 (&ck)[CW], u32x4 (&ct)[CW]) {
        // the weights are read from LDS per token, not hoisted out of the
        // token loop into registers (16 more chunks a lane)
        asm volatile("" ::: "memory");
        const int rn = r + kPairStages * NW;
        const int64_t trn = table_row(rn);
        float ssq = 0.f, ssk = 0.f;
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            float vq[8], vk[8];
            unpack8v(cq[c], vq);
            unpack8v(ck[c], vk);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ssq = __builtin_fmaf(vq[i], vq[i], ssq);
                ssk = __builtin_fmaf(vk[i], vk[i], ssk);
            }
        }
        const float rq_ = has_wq ? rsqrtf(wave_sum64(ssq) * inv_dim + p.eps) : 1.0f;
        const float rk_ = has_wk ? rsqrtf(wave_sum64(ssk) * inv_dim + p.eps) : 1.0f;
        const rsrc_t oq = rsrc_of(Q.x, r), ok = rsrc_of(K.x, r);
        const rsrc_t nq = rsrc_of(Q.x, rn), nk = rsrc_of(K.x, rn);
        auto finish = [&](const u32x4 &own, const u32x4 &par, int t, int c, float rs, const float (&cs)[8],
                          const float (&sn)[8]) -> u32x4 {
            float x[8], y[8], fo[8], fp[8];
            unpack8v(own, x);
            unpack8v(par, y);
            unpack8v(lw[t][lane + 64 * c], fo);
            unpack8v(lw[t][(lane ^ PX) + 64 * c], fp);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[i] = (x[i] * rs) * fo[i];
                y[i] = (y[i] * rs) * fp[i];
            }
            float out[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float ps = y[i] * sn[i];
                out[i] = x[i] * cs[i] + (first ? -ps : ps);  // a - b is a + (-b), bit for bit
            }
            return pack8v(out);
        };
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            // the rows stay packed between their two uses (unpacking them once
            // for both would hold 16 * CW more registers)
            asm volatile("" : "+v"(cq[c]), "+v"(ck[c]));
            const u32x4 other = swizzle_xor<PX>(ct[c]);
            float cs[8], sn[8];
            unpack8v(first ? ct[c] : other, cs);
            unpack8v(first ? other : ct[c], sn);
            const u32x4 pq = swizzle_xor<PX>(cq[c]), pk = swizzle_xor<PX>(ck[c]);
            stb_stream(oq, (lane + 64 * c) * 16u, finish(cq[c], pq, 0, c, rq_, cs, sn));
            cq[c] = ldb(nq, (lane + 64 * c) * 16u);
            pair_spacing<kPairLoadNops>();
            stb_stream(ok, (lane + 64 * c) * 16u, finish(ck[c], pk, 1, c, rk_, cs, sn));
            ck[c] = ldb(nk, (lane + 64 * c) * 16u);
            pair_spacing<kPairLoadNops>();
            ct[c] = *reinterpret_cast<const u32x4 *>(tb + trn + toff + 256 * c);
            // chunk by chunk: the next chunk's swizzles and weight reads are
            // not hoisted above this one (they would hold its registers)
            __builtin_amdgcn_sched_barrier(0);
        }
        r += NW;
        return r < rows;
    };
    bool more = r < rows;
    while (more) {
#pragma unroll
        for (int j = 0; j < kPairStages; ++j)
            if (more) more = step(sq[j], sk[j], st[j]);
    }
}

// -------------------------------------------------------------- wave rows --
// q/k norm + rotation on compact tables with AX axes (launched with one) when
// q and k have their own tables (a cross-attention launch, or q alone): rows of 64*8*CW elements
// with heads of 16*PX, in place, one wave per row of q or of k.  The launch's
// rows are q's then k's, each with its own index and tables, and waves walk
// them w, w + NW, ...  Lane l owns the 16-byte chunks l + 64c of its row; a
// row's sum of squares is one wave reduction (no barrier).  A lane in the
// first half of a head loads its pair index's cos chunk from each axis row,
// its partner lane (l ^ PX, the same pair index) the sin chunk; OR-ing the
// axis rows gives the full table's value (the other axes hold +0.0 there) and
// each lane takes the partner's through ds_swizzle.  Two rows of data and of
// table chunks are in registers; as each output chunk is stored, its registers
// are refilled with the same chunk of the wave's row two ahead.  The norm
// weights sit in LDS (the partner's at chunk ^ PX).  The arithmetic is the
// wave-token pair kernel's, operation for operation.
//
// Measured on q [6144, 2048] + k [126, 2048] with one-axis tables each (us):
// 12.1-12.2 against 14.7 for the two-rows-per-workgroup kernel; loads spaced
// by no, one or four s_nop 7 13.1, 12.8, 12.0-12.1; three rows in registers
// at three workgroups per CU 13.0.  Two- and three-axis tables would spill
// here.  (The same form for 4096-wide rows of 128-wide heads on two-axis
// tables needs twice the registers a lane and was slower than the slot
// kernel there, which the self-attention pair keeps.)
constexpr int kRopeWavePerCU = 4;
constexpr int kRopeWaveStages = 2;

template <int CW, int PX, int AX>
__global__ void __launch_bounds__(kBlock, kRopeWavePerCU) qk_rope_wave_kernel(QKParams p)
{
    static_assert(PX >= 1 && PX <= 16 && (32 % PX) == 0, "PX must be a power of two up to 16");
    static_assert(AX >= 1 && AX <= 3, "compact tables with one to three axes");
    constexpr int DS = kRopeWaveStages;
    constexpr int kDim = 64 * 8 * CW;
    constexpr int kTrow = kDim / 2;  // elements per table row
    constexpr uint32_t kRowBytes = kDim * 2;
    __shared__ u32x4 lw[2][CW * 64];  // norm weights of q and k (raw bf16)
    const int lane = threadIdx.x & 63;
    const int NW = static_cast<int>(gridDim.x) * (kBlock / 64);
    const int w = static_cast<int>(blockIdx.x) * (kBlock / 64) +
                  __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const QKDev Q = p.q, K = p.k;
    const int qrows = static_cast<int>(Q.rows);
    const int units = qrows + (K.x ? static_cast<int>(K.rows) : 0);
    const bool first = (lane & PX) == 0;
    // chunk lane + 64c starts at element 8*lane + 512c of the row; its pair
    // index in a table row is toff + 256c (as in the wave-token pair kernel)
    const int hpos = (8 * lane) % (16 * PX);
    const int toff = ((8 * lane) / (16 * PX)) * (8 * PX) + (first ? hpos : hpos - 8 * PX);
    const uint16_t *tq = (first ? Q.cos : Q.sin) + toff;
    const uint16_t *tk = K.x ? (first ? K.cos : K.sin) + toff : tq;
    // unit u: row u of q or row u - qrows of k; past the end an empty buffer
    // range, and the table rows of the last unit (always in the tables)
    auto rsrc_of = [&](int u) {
        const bool ok = u < units, isq = u < qrows;
        uint16_t *base = isq ? Q.x : K.x;
        const int r = ok ? (isq ? u : u - qrows) : 0;
        return make_rsrc(base + static_cast<int64_t>(r) * kDim, ok ? kRowBytes : 0u);
    };
    auto table_rows = [&](int u, int64_t (&e)[AX]) {
        const int uc = u < units ? u : units - 1;
        const bool isq = uc < qrows;
        const int32_t *idx = isq ? Q.idx : K.idx;
        const uint32_t nrows = isq ? Q.tab_rows : K.tab_rows;
        const __attribute__((address_space(4))) int32_t *ci =
            (const __attribute__((address_space(4))) int32_t *)(idx);
        const int64_t r = isq ? uc : uc - qrows;
#pragma unroll
        for (int a = 0; a < AX; ++a) {
            const uint32_t v = static_cast<uint32_t>(ci[r * AX + a]);
            e[a] = static_cast<int64_t>(v < nrows ? v : nrows - 1) * kTrow;
        }
        return isq ? tq : tk;
    };

    int u = w;
    u32x4 sd[DS][CW], st[DS][AX][CW];
#pragma unroll
    for (int j = 0; j < DS; ++j) {
        const rsrc_t rs = rsrc_of(u + j * NW);
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            sd[j][c] = ldb_s(rs, lane * 16u, c * 1024u);
            pair_spacing<kPairLoadNops>();
        }
        int64_t e[AX];
        const uint16_t *tb = table_rows(u + j * NW, e);
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int a = 0; a < AX; ++a) st[j][a][c] = *reinterpret_cast<const u32x4 *>(tb + e[a] + 256 * c);
    }
    // an absent weight: no normalisation, the raw values are rotated (scale
    // 1 and weights 1.0: (x * 1) * 1 is x, bit for bit)
    const bool has_wq = Q.w != nullptr, has_wk = K.w != nullptr;
    constexpr uint32_t kOnes = 0x3f803f80u;
    constexpr u32x4 ones = {kOnes, kOnes, kOnes, kOnes};
    for (int i = threadIdx.x; i < CW * 64; i += kBlock) {
        lw[0][i] = has_wq ? *reinterpret_cast<const u32x4 *>(Q.w + 8 * i) : ones;
        lw[1][i] = has_wk ? *reinterpret_cast<const u32x4 *>(K.w + 8 * i) : ones;
    }
    __syncthreads();
    // rows of 2048: 1/dim is a power of two, so tot * inv_dim rounds exactly as tot / dim
    constexpr float inv_dim = 1.0f / static_cast<float>(kDim);

    auto step = [&](u32x4 (&cd)[CW], u32x4 (&ct)[AX][CW]) {
        // the weights are read from LDS per row, not hoisted out of the loop
        asm volatile("" ::: "memory");
        const bool isq = u < qrows;
        const int t = isq ? 0 : 1;
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            float v[8];
            unpack8v(cd[c], v);
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[i], v[i], ss);
        }
        const float rs = (isq ? has_wq : has_wk) ? rsqrtf(wave_sum64(ss) * inv_dim + p.eps) : 1.0f;
        const rsrc_t o = rsrc_of(u), n = rsrc_of(u + DS * NW);
        int64_t e[AX];
        const uint16_t *tb = table_rows(u + DS * NW, e);
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            // the row stays packed between its two uses
            asm volatile("" : "+v"(cd[c]));
            u32x4 tc = ct[0][c];
#pragma unroll
            for (int a = 1; a < AX; ++a) tc |= ct[a][c];
            const u32x4 other = swizzle_xor<PX>(tc);
            float cs[8], sn[8], x[8], y[8], fo[8], fp[8];
            unpack8v(first ? tc : other, cs);
            unpack8v(first ? other : tc, sn);
            unpack8v(cd[c], x);
            unpack8v(swizzle_xor<PX>(cd[c]), y);
            unpack8v(lw[t][lane + 64 * c], fo);
            unpack8v(lw[t][(lane ^ PX) + 64 * c], fp);
            float out[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float xv = (x[i] * rs) * fo[i];
                const float ps = ((y[i] * rs) * fp[i]) * sn[i];
                out[i] = xv * cs[i] + (first ? -ps : ps);  // a - b is a + (-b), bit for bit
            }
            stb_s_stream(o, lane * 16u, c * 1024u, pack8v(out));
            cd[c] = ldb_s(n, lane * 16u, c * 1024u);
            pair_spacing<kPairLoadNops>();
#pragma unroll
            for (int a = 0; a < AX; ++a) ct[a][c] = *reinterpret_cast<const u32x4 *>(tb + e[a] + 256 * c);
            // chunk by chunk: the next chunk's swizzles and weight reads are
            // not hoisted above this one (they would hold its registers)
            __builtin_amdgcn_sched_barrier(0);
        }
        u += NW;
        return u < units;
    };
    bool more = u < units;
    while (more) {
#pragma unroll
        for (int j = 0; j < DS; ++j)
            if (more) more = step(sd[j], st[j]);
    }
}

template <int CW, int PX>
int launch_rope_wave(QKParams p, int mode, hipStream_t s)
{
    const int64_t units = p.q.rows + (p.k.x ? p.k.rows : 0);
    if (units == 0) return LTXK_OK;
    if (units > kWaveRowsMax) return fail(LTXK_E_ARG, "qk_norm_rope: too many rows");
    const dim3 grid(stream_grid((units + 3) / 4, kRopeWavePerCU)), block(kBlock);
    if (mode != 1) return fail(LTXK_E_ARG, "qk_norm_rope: the wave-row kernel takes one-axis tables (mode %d)", mode);
    qk_rope_wave_kernel<CW, PX, 1><<<grid, block, 0, s>>>(p);
    return check_launch("qk_norm_rope");
}

// -------------------------------------------------------------- wave norm --
// q/k RMSNorm with weights and no rotation (the text cross-attention's q and
// the block's context keys), rows of 64*8*CW elements, in place, one wave per
// row: lane l owns the 16-byte chunks l + 64c, a row's sum of squares is one
// wave reduction (no barrier in the row loop).  The launch's rows are q's
// rows then k's; waves walk them w, w + NW, ... with two rows in registers,
// and as each output chunk is stored its register is refilled with the same
// chunk of the wave's next row.  Both weights sit in LDS.  The arithmetic is
// qk_kernel's, (x * r) * w, with the row's sum in another order.  Streaming
// (nt) stores: 19.24 against 19.42 us with write-through ones on q [6144,
// 4096] + k [1024, 4096].
constexpr int kNormWavePerCU = 4;
constexpr int kNormWaveStages = 2;

template <int CW>
__global__ void __launch_bounds__(kBlock, kNormWavePerCU) qk_norm_wave_kernel(QKParams p)
{
    constexpr int kDim = 64 * 8 * CW;
    constexpr uint32_t kRowBytes = kDim * 2;
    __shared__ u32x4 lw[2][CW * 64];  // weights of q and k (raw bf16)
    const int lane = threadIdx.x & 63;
    const int NW = static_cast<int>(gridDim.x) * (kBlock / 64);
    const int w = static_cast<int>(blockIdx.x) * (kBlock / 64) +
                  __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const QKDev Q = p.q, K = p.k;
    const int qrows = static_cast<int>(Q.rows);
    const int units = qrows + (K.x ? static_cast<int>(K.rows) : 0);
    // unit u: row u of q, or row u - qrows of k (past the end: an empty range)
    auto rsrc_of = [&](int u) {
        const bool ok = u < units, isq = u < qrows;
        uint16_t *base = isq ? Q.x : K.x;
        const int r = ok ? (isq ? u : u - qrows) : 0;
        return make_rsrc(base + static_cast<int64_t>(r) * kDim, ok ? kRowBytes : 0u);
    };
    int u = w;
    u32x4 st[kNormWaveStages][CW];
#pragma unroll
    for (int j = 0; j < kNormWaveStages; ++j) {
        const rsrc_t rs = rsrc_of(u + j * NW);
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            st[j][c] = ldb_s(rs, lane * 16u, c * 1024u);
            pair_spacing<kPairLoadNops>();
        }
    }
    // an absent weight: no normalisation (scale 1, weights 1.0: (x * 1) * 1 is x)
    const bool has_wq = Q.w != nullptr, has_wk = K.w != nullptr;
    constexpr uint32_t kOnes = 0x3f803f80u;
    constexpr u32x4 ones = {kOnes, kOnes, kOnes, kOnes};
    for (int i = threadIdx.x; i < CW * 64; i += kBlock) {
        lw[0][i] = has_wq ? *reinterpret_cast<const u32x4 *>(Q.w + 8 * i) : ones;
        lw[1][i] = has_wk ? *reinterpret_cast<const u32x4 *>(K.w + 8 * i) : ones;
    }
    __syncthreads();
    // rows of 2048 or 4096: 1/dim is a power of two, so tot * inv_dim rounds exactly as tot / dim
    constexpr float inv_dim = 1.0f / static_cast<float>(kDim);

    auto step = [&](u32x4 (&cur)[CW]) {
        // the weights are read from LDS per row, not hoisted out of the loop
        asm volatile("" ::: "memory");
        const bool isq = u < qrows;
        float s2 = 0.f;
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            float v[8];
            unpack8v(cur[c], v);
#pragma unroll
            for (int i = 0; i < 8; ++i) s2 = __builtin_fmaf(v[i], v[i], s2);
        }
        // (the weight pointer itself, a scalar: a bool kept across the loop lands in a vector register)
        const float r = (isq ? Q.w : K.w) ? rsqrtf(wave_sum64(s2) * inv_dim + p.eps) : 1.0f;
        const int t = isq ? 0 : 1;
        const rsrc_t ro = rsrc_of(u);
        const rsrc_t rn = rsrc_of(u + kNormWaveStages * NW);
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            // the row stays packed between its two uses
            asm volatile("" : "+v"(cur[c]));
            float v[8], f[8], o[8];
            unpack8v(cur[c], v);
            unpack8v(lw[t][lane + 64 * c], f);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = (v[i] * r) * f[i];
            stb_s_stream(ro, lane * 16u, c * 1024u, pack8v(o));
            cur[c] = ldb_s(rn, lane * 16u, c * 1024u);
            pair_spacing<kPairLoadNops>();
        }
        u += NW;
        return u < units;
    };
    bool more = u < units;
    while (more) {
#pragma unroll
        for (int j = 0; j < kNormWaveStages; ++j)
            if (more) more = step(st[j]);
    }
}

template <int CW>
int launch_norm_wave(QKParams p, hipStream_t s)
{
    const int64_t units = p.q.rows + (p.k.x ? p.k.rows : 0);
    if (units == 0) return LTXK_OK;
    if (units > kWaveRowsMax) return fail(LTXK_E_ARG, "qk_norm_rope: too many rows");
    const dim3 grid(stream_grid((units + 3) / 4, kNormWavePerCU)), block(kBlock);
    qk_norm_wave_kernel<CW><<<grid, block, 0, s>>>(p);
    return check_launch("qk_norm_rope");
}

template <int PX>
int launch_pair_wave(QKParams p, hipStream_t s)
{
    const int64_t waves = p.q.rows;
    if (waves > kWaveRowsMax) return fail(LTXK_E_ARG, "qk_norm_rope: too many rows");
    const dim3 grid(stream_grid((waves + 3) / 4, kPairPerCU)), block(kBlock);
    qk_pair_wave_kernel<PX><<<grid, block, 0, s>>>(p);
    return check_launch("qk_norm_rope");
}

template <int CH, int PX>
int launch_chunk(QKParams p, int mode, hipStream_t s)
{
    p.q_groups = p.q.rows;
    if (p.q_groups == 0) return LTXK_OK;
    const dim3 grid(stream_grid(p.q_groups, LTXK_CHUNK_PER_CU)), block(kBlock);
    switch (mode) {
    case 1: qk_chunk_kernel<CH, PX, 1><<<grid, block, 0, s>>>(p); break;
    case 2: qk_chunk_kernel<CH, PX, 2><<<grid, block, 0, s>>>(p); break;
    case 3: qk_chunk_kernel<CH, PX, 3><<<grid, block, 0, s>>>(p); break;
    default: return fail(LTXK_E_ARG, "qk_norm_rope: bad table mode %d", mode);
    }
    return check_launch("qk_norm_rope");
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
    d.tab_rows = static_cast<uint32_t>(t->table_rows);
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
    if (t->pos_index && (t->table_rows <= 0 || t->table_rows > 0x7fffffff))
        return fail(LTXK_E_ARG, "%s: %s compact tables need table_rows in [1, 2^31) (got %lld)", what, name,
                    (long long)t->table_rows);
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
// Workgroups of a streaming launch: per_cu per compute unit, never more than groups.
unsigned stream_grid(int64_t groups, int per_cu)
{
    const int64_t blocks = static_cast<int64_t>(per_cu) * device_cus();
    return static_cast<unsigned>(groups < blocks ? groups : blocks);
}

template <int TPR>
int launch_stream(QKParams p, int mode, hipStream_t s)
{
    constexpr int RPI = kBlock / TPR;
    p.q_groups = (p.q.rows + RPI - 1) / RPI;
    if (p.q_groups == 0) return LTXK_OK;
    const dim3 grid(stream_grid(p.q_groups, LTXK_SLOT_PER_CU)), block(kBlock);
    switch (mode) {
    case 1: qk_stream_kernel<TPR, 1><<<grid, block, 0, s>>>(p); break;
    case 2: qk_stream_kernel<TPR, 2><<<grid, block, 0, s>>>(p); break;
    case 3: qk_stream_kernel<TPR, 3><<<grid, block, 0, s>>>(p); break;
    default: return fail(LTXK_E_ARG, "qk_norm_rope: bad table mode %d", mode);
    }
    return check_launch("qk_norm_rope");
}

int launch(QKParams p, int mode, bool paired, hipStream_t s)
{
    // paired q/k rows of 128 or 256 slots with compact tables: the streaming form.  Measured on
    // MI355X it is 5-8% faster there (video self q/k 40.0 vs 41.9 us, audio 3.4 vs 3.7 us) and
    // slower for unpaired or unrotated launches (text q/k 26.4 vs 18.1 us), which keep the
    // one-pass kernels below.
    // norm without rotation (the text cross-attention's q and context keys), rows of 2048 or 4096:
    // one wave per row (q [6144, 4096] + k [1024, 4096]: 20.1-20.2 against 21.8-22.0 us for the
    // one-pass kernel below; the 48-block chain 17.08 against 17.19 ms)
    if (mode == -1 && (p.dim == 4096 || p.dim == 2048))
        return p.dim == 4096 ? launch_norm_wave<8>(p, s) : launch_norm_wave<4>(p, s);
    // paired rows of 2048 with 64-wide heads: one table axis the wave-token form, more axes (whose
    // table rows do not repeat along a wave's tokens) the contiguous-chunk form
    if (paired && mode == 1 && p.q.rows > 0 && p.dim == 8 * kBlock && p.head_dim == 64)
        return launch_pair_wave<4>(p, s);
    if (paired && mode > 0 && p.q.rows > 0 && p.dim == 8 * kBlock && p.head_dim == 64)
        return launch_chunk<1, 4>(p, mode, s);
    // the same rows with one-axis tables when q and k have their own (or q alone): one wave per
    // row of q or of k (more axes would not fit its registers)
    if (!paired && mode == 1 && p.q.rows > 0 && p.dim == 8 * kBlock && p.head_dim == 64)
        return launch_rope_wave<4, 4>(p, mode, s);
    // (one wave per row of q or of k, no barrier or LDS, waves of a whole grid
    // instead of persistent workgroups: 21.7 against 21.4 us on the [6144, 2048]
    // pair, 21.6 with streaming stores; a flat GELU over the same bytes takes
    // 17.3 us in place and out of place alike)
    // (a persistent two-stage form for the unrotated text q/k norm, rows of 4096:
    // 21.7 against 21.8 us for q [6144] + k [1024], no faster, and the same in the chain)
    // (the same form for 4096-wide rows of 128-wide heads, two chunks per
    // thread, measured 50.2 against 40.8 us on the video pair: those heads
    // already load whole 128-byte lines in the slot form)
    if (paired && mode > 0 && p.q.rows > 0 && (p.slots == kBlock || p.slots == kBlock / 2))
        return p.slots == kBlock ? launch_stream<kBlock>(p, mode, s) : launch_stream<kBlock / 2>(p, mode, s);
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
    if (tpr == kBlock && per <= 1 && mode > 0) {  // compact tables: two rows per workgroup
        constexpr int R = 2;
        p.q_groups = (p.q.rows + R - 1) / R;
        const int64_t kg2 = p.k.x ? (p.k.rows + R - 1) / R : 0;
        const unsigned g2 = static_cast<unsigned>(paired ? p.q_groups : p.q_groups + kg2);
        const bool norm = p.q.w != nullptr || (p.k.x && p.k.w != nullptr);
        auto go = [&](auto k1, auto k2, auto k3) {
            if (mode == 1) k1<<<dim3(g2), dim3(kBlock), 0, s>>>(p);
            else if (mode == 2) k2<<<dim3(g2), dim3(kBlock), 0, s>>>(p);
            else k3<<<dim3(g2), dim3(kBlock), 0, s>>>(p);
        };
        if (paired && norm)
            go(qk_rows_kernel<R, 1, true, true>, qk_rows_kernel<R, 2, true, true>, qk_rows_kernel<R, 3, true, true>);
        else if (paired)
            go(qk_rows_kernel<R, 1, true, false>, qk_rows_kernel<R, 2, true, false>,
               qk_rows_kernel<R, 3, true, false>);
        else if (norm)
            go(qk_rows_kernel<R, 1, false, true>, qk_rows_kernel<R, 2, false, true>,
               qk_rows_kernel<R, 3, false, true>);
        else
            go(qk_rows_kernel<R, 1, false, false>, qk_rows_kernel<R, 2, false, false>,
               qk_rows_kernel<R, 3, false, false>);
        return check_launch("qk_norm_rope");
    }
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
                             (q->pos_index == nullptr || (q->n_axes == k->n_axes && q->table_rows == k->table_rows)) &&
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
