// q/k preparation: RMSNorm over the whole inner dim with a weight, then
// LTXRopeType.SPLIT rotation per head, in place, one HBM round trip.
//
// A row is one token of x [batch*tokens, heads*head_dim].  It is cut into
// "slots": slot s covers 8 rotation pairs of one head, i.e. the 8 elements at
// h*Dh + 8j (first half) and the 8 at h*Dh + Dh/2 + 8j (second half) for
// h = s / (Dh/16), j = s % (Dh/16).  A thread owns whole slots, so the pair
// partner of every element it rotates is already in its registers, and the
// matching cos/sin entries are 16 contiguous bytes of each table
// (tables are (batch, heads, tokens, Dh/2) as precompute_freqs_cis builds
// them, standalone/ltx_nn.py:63-96).
//
// When q and k share tables and token count (self-attention), one launch
// handles both for the same token and reads each table chunk once.
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;

struct QKDev {
    uint16_t *x;
    const uint16_t *w;
    const uint16_t *cos;
    const uint16_t *sin;
    int64_t rows;
    int64_t tokens;
    int64_t tbs;
};

struct QKParams {
    QKDev q, k;
    int64_t dim, head_dim, half, slots, slots_per_head;
    int tpr, rows_per_block;
    int64_t q_blocks;
    float eps;
};

struct SlotData {
    float a[8], b[8];
};

__device__ __forceinline__ void load_slot(const uint16_t *row, int64_t off_a, int64_t half, SlotData &d)
{
    unpack8(ld16_stream(row + off_a), d.a);
    unpack8(ld16_stream(row + off_a + half), d.b);
}

__device__ __forceinline__ float slot_sumsq(const SlotData &d)
{
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += d.a[i] * d.a[i] + d.b[i] * d.b[i];
    return s;
}

__device__ __forceinline__ void apply_weight(SlotData &d, const uint16_t *w, int64_t off_a, int64_t half, float r)
{
    float wa[8], wb[8];
    unpack8(ld16(w + off_a), wa);
    unpack8(ld16(w + off_a + half), wb);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        d.a[i] = (d.a[i] * r) * wa[i];
        d.b[i] = (d.b[i] * r) * wb[i];
    }
}

__device__ __forceinline__ void rotate(SlotData &d, const float c[8], const float s[8])
{
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x1 = d.a[i], x2 = d.b[i];
        d.a[i] = x1 * c[i] - x2 * s[i];
        d.b[i] = x2 * c[i] + x1 * s[i];
    }
}

__device__ __forceinline__ void store_slot(uint16_t *row, int64_t off_a, int64_t half, const SlotData &d)
{
    st16_stream(row + off_a, pack8(d.a));
    st16_stream(row + off_a + half, pack8(d.b));
}

__device__ __forceinline__ void load_tables(const QKDev &t, int64_t row, int64_t h, int64_t j8, int64_t half,
                                            float c[8], float s[8])
{
    const int64_t b = row / t.tokens;
    const int64_t tok = row - b * t.tokens;
    const int64_t off = b * t.tbs + (h * t.tokens + tok) * half + j8;
    unpack8(ld16(t.cos + off), c);
    unpack8(ld16(t.sin + off), s);
}

// One tensor per row (cross-attention q/k with different tables or lengths).
template <int MAXS>
__global__ void __launch_bounds__(kBlock) qk_single_kernel(QKParams p)
{
    __shared__ float lds[kBlock / 64];
    const bool is_q = blockIdx.x < p.q_blocks;
    const QKDev t = is_q ? p.q : p.k;
    const int64_t blk = is_q ? blockIdx.x : blockIdx.x - p.q_blocks;
    const int lrow = threadIdx.x / p.tpr;
    const int lane = threadIdx.x - lrow * p.tpr;
    const int64_t row = blk * p.rows_per_block + lrow;
    const bool active = row < t.rows;
    uint16_t *xrow = t.x + row * p.dim;
    SlotData d[MAXS];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
        const int64_t s = lane + static_cast<int64_t>(k) * p.tpr;
        if (active && s < p.slots) {
            const int64_t h = s / p.slots_per_head, j8 = (s - h * p.slots_per_head) * 8;
            load_slot(xrow, h * p.head_dim + j8, p.half, d[k]);
            ss += slot_sumsq(d[k]);
        }
    }
    float r = 1.f;
    if (t.w) r = rsqrtf(group_sum(ss, p.tpr, lds) / static_cast<float>(p.dim) + p.eps);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
        const int64_t s = lane + static_cast<int64_t>(k) * p.tpr;
        if (s >= p.slots) continue;
        const int64_t h = s / p.slots_per_head, j8 = (s - h * p.slots_per_head) * 8;
        const int64_t off_a = h * p.head_dim + j8;
        if (t.w) apply_weight(d[k], t.w, off_a, p.half, r);
        if (t.cos) {
            float c[8], sn[8];
            load_tables(t, row, h, j8, p.half, c, sn);
            rotate(d[k], c, sn);
        }
        store_slot(xrow, off_a, p.half, d[k]);
    }
}

// q and k of the same token with shared tables (self-attention).
template <int MAXS>
__global__ void __launch_bounds__(kBlock) qk_paired_kernel(QKParams p)
{
    __shared__ float lds[kBlock / 64];
    const int lrow = threadIdx.x / p.tpr;
    const int lane = threadIdx.x - lrow * p.tpr;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * p.rows_per_block + lrow;
    const bool active = row < p.q.rows;
    uint16_t *qrow = p.q.x + row * p.dim;
    uint16_t *krow = p.k.x + row * p.dim;
    SlotData dq[MAXS], dk[MAXS];
    float ssq = 0.f, ssk = 0.f;
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
        const int64_t s = lane + static_cast<int64_t>(k) * p.tpr;
        if (active && s < p.slots) {
            const int64_t h = s / p.slots_per_head, j8 = (s - h * p.slots_per_head) * 8;
            load_slot(qrow, h * p.head_dim + j8, p.half, dq[k]);
            load_slot(krow, h * p.head_dim + j8, p.half, dk[k]);
            ssq += slot_sumsq(dq[k]);
            ssk += slot_sumsq(dk[k]);
        }
    }
    float rq = 1.f, rk = 1.f;
    if (p.q.w) rq = rsqrtf(group_sum(ssq, p.tpr, lds) / static_cast<float>(p.dim) + p.eps);
    if (p.k.w) rk = rsqrtf(group_sum(ssk, p.tpr, lds) / static_cast<float>(p.dim) + p.eps);
    if (!active) return;
#pragma unroll
    for (int k = 0; k < MAXS; ++k) {
        const int64_t s = lane + static_cast<int64_t>(k) * p.tpr;
        if (s >= p.slots) continue;
        const int64_t h = s / p.slots_per_head, j8 = (s - h * p.slots_per_head) * 8;
        const int64_t off_a = h * p.head_dim + j8;
        if (p.q.w) apply_weight(dq[k], p.q.w, off_a, p.half, rq);
        if (p.k.w) apply_weight(dk[k], p.k.w, off_a, p.half, rk);
        if (p.q.cos) {
            float c[8], sn[8];
            load_tables(p.q, row, h, j8, p.half, c, sn);
            rotate(dq[k], c, sn);
            rotate(dk[k], c, sn);
        }
        store_slot(qrow, off_a, p.half, dq[k]);
        store_slot(krow, off_a, p.half, dk[k]);
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
    d.rows = t->batch * t->tokens;
    d.tokens = t->tokens;
    d.tbs = t->table_bstride;
    return d;
}

int check_operand(const ltxk_qk *t, const char *name, int64_t half)
{
    static const char *what = "qk_norm_rope";
    if (t->batch < 0 || t->tokens < 0) return fail(LTXK_E_ARG, "%s: %s has negative batch/tokens", what, name);
    if (!aligned16(t->x) || !aligned16(t->weight) || !aligned16(t->cos) || !aligned16(t->sin))
        return fail(LTXK_E_ALIGN, "%s: %s buffers must be 16-byte aligned", what, name);
    if ((t->cos == nullptr) != (t->sin == nullptr))
        return fail(LTXK_E_ARG, "%s: %s needs both cos and sin or neither", what, name);
    if (t->cos && (t->table_bstride % 8)) return fail(LTXK_E_ALIGN, "%s: %s table_bstride must be a multiple of 8",
                                                      what, name);
    (void)half;
    return LTXK_OK;
}

template <int MAXS>
void launch(const QKParams &p, bool paired, unsigned grid, hipStream_t s)
{
    if (paired)
        qk_paired_kernel<MAXS><<<dim3(grid), dim3(kBlock), 0, s>>>(p);
    else
        qk_single_kernel<MAXS><<<dim3(grid), dim3(kBlock), 0, s>>>(p);
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
    int rc = check_operand(q, "q", head_dim / 2);
    if (rc) return rc;
    const bool has_k = k && k->x;
    if (has_k && (rc = check_operand(k, "k", head_dim / 2))) return rc;

    QKParams p{};
    p.q = make_dev(q);
    p.k = has_k ? make_dev(k) : QKDev{};
    p.dim = dim;
    p.head_dim = head_dim;
    p.half = head_dim / 2;
    p.slots = dim / 16;
    p.slots_per_head = head_dim / 16;
    p.eps = eps;
    RowLayout l = row_layout(p.slots, kBlock);
    p.tpr = l.tpr;
    p.rows_per_block = l.rows_per_block;

    const bool paired = has_k && q->batch == k->batch && q->tokens == k->tokens && q->cos == k->cos &&
                        q->sin == k->sin && (q->cos == nullptr || q->table_bstride == k->table_bstride);
    const int64_t qb = (p.q.rows + p.rows_per_block - 1) / p.rows_per_block;
    const int64_t kb = has_k ? (p.k.rows + p.rows_per_block - 1) / p.rows_per_block : 0;
    p.q_blocks = qb;
    const int64_t grid = paired ? qb : qb + kb;
    if (grid == 0) return LTXK_OK;
    if (grid > 0x7fffffff) return fail(LTXK_E_ARG, "%s: too many rows", what);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int per = l.per_thread;
    if (per <= 1)
        launch<1>(p, paired, static_cast<unsigned>(grid), s);
    else if (per <= 2)
        launch<2>(p, paired, static_cast<unsigned>(grid), s);
    else if (per <= 4)
        launch<4>(p, paired, static_cast<unsigned>(grid), s);
    else
        launch<8>(p, paired, static_cast<unsigned>(grid), s);
    return check_launch(what);
}
