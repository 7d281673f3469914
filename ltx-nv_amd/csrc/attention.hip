// Combine of key-split attention: the V2A attention (a few hundred queries
// over thousands of keys) runs PyTorch's flash kernel over the keys cut into
// `parts` chunks (the chunks as extra batch items), which returns one output
// and one log-sum-exp per chunk; this kernel merges them and applies the
// per-head gate of the attention epilogue in the same pass:
//
//   w_c = exp(lse_c - max_c lse_c) / sum_c exp(lse_c - max_c lse_c)
//   o   = round_bf16(sum_c w_c * part_c)                (fp32, one rounding)
//   out[b, t, h*D + d] = round_bf16(o[d] * 2 * sigmoid(logit[b, t, h]))
//
// which is softmax(q k^T / sqrt(D)) v evaluated chunk by chunk, then the head
// merge and gate of standalone/ltx_nn.py:227-235.  One thread per 16-byte
// chunk of the merged output (8 elements of one head of one token): the
// threads of a workgroup write contiguous output rows; the partial outputs are
// read through their strides (any of the flash kernel's layouts).
#include "ltxk_common.h"

namespace ltxk {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxParts = 16;

struct CombineParams {
    uint16_t *out;
    const uint16_t *part;
    const float *lse;
    const uint16_t *logits;
    int64_t pbs, pcs, phs, pts;  // part strides (elements): batch, chunk, head, token
    int64_t lbs, lcs, lhs, lts;  // lse strides (elements)
    int64_t tokens, heads, head_dim, chunks_per_head;
    int64_t total;               // output chunks: batch * tokens * heads * chunks_per_head
};

template <int PARTS>
__global__ void __launch_bounds__(kBlock) attn_combine_kernel(CombineParams p)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= p.total) return;
    const int64_t c8 = i % p.chunks_per_head;
    const int64_t rest = i / p.chunks_per_head;
    const int64_t h = rest % p.heads;
    const int64_t bt = rest / p.heads;
    const int64_t t = bt % p.tokens;
    const int64_t b = bt / p.tokens;
    // issue every load first: the partial chunks, the log-sum-exps, the logit
    u32x4 raw[PARTS];
    float l[PARTS];
    const uint16_t *pp = p.part + b * p.pbs + h * p.phs + t * p.pts + c8 * 8;
    const float *lp = p.lse + b * p.lbs + h * p.lhs + t * p.lts;
#pragma unroll
    for (int c = 0; c < PARTS; ++c) {
        raw[c] = *reinterpret_cast<const u32x4 *>(pp + c * p.pcs);
        l[c] = lp[c * p.lcs];
    }
    const float lg = p.logits ? bf16_to_f32(p.logits[bt * p.heads + h]) : 0.f;
    float m = l[0];
#pragma unroll
    for (int c = 1; c < PARTS; ++c) m = fmaxf(m, l[c]);
    float e[PARTS], s = 0.f;
#pragma unroll
    for (int c = 0; c < PARTS; ++c) {
        e[c] = expf(l[c] - m);
        s += e[c];
    }
    float acc[8] = {};
#pragma unroll
    for (int c = 0; c < PARTS; ++c) {
        const float wc = e[c] / s;
        float v[8];
        unpack8v(raw[c], v);
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += v[k] * wc;
    }
    // the attention output in bf16 (as the unfused path hands it to the gate),
    // then the gate: 2*sigmoid(l) = 2 / (1 + e^-l); no logits: exactly 1
    float o[8];
    unpack8v(pack8v(acc), o);
    if (p.logits) {
        const float gate = 2.0f / (1.0f + expf(-lg));
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = o[k] * gate;
    }
    *reinterpret_cast<u32x4 *>(p.out + i * 8) = pack8v(o);
}

}  // namespace
}  // namespace ltxk

using namespace ltxk;

extern "C" int ltxk_attn_combine(void *out, const void *part, int64_t part_bstride, int64_t part_cstride,
                                 int64_t part_hstride, int64_t part_tstride, const float *lse, int64_t lse_bstride,
                                 int64_t lse_cstride, int64_t lse_hstride, int64_t lse_tstride, const void *logits,
                                 int64_t batch, int64_t parts, int64_t tokens, int64_t heads, int64_t head_dim,
                                 void *stream)
{
    static const char *what = "attn_combine";
    clear_error();
    if (batch < 0 || tokens < 0 || heads <= 0 || head_dim <= 0)
        return fail(LTXK_E_ARG, "%s: bad shape batch=%lld tokens=%lld heads=%lld head_dim=%lld", what,
                    (long long)batch, (long long)tokens, (long long)heads, (long long)head_dim);
    if (head_dim % 8) return fail(LTXK_E_ARG, "%s: head_dim must be a multiple of 8 (got %lld)", what,
                                  (long long)head_dim);
    if (parts < 1 || parts > kMaxParts || (parts & (parts - 1)))
        return fail(LTXK_E_ARG, "%s: parts must be a power of two in [1, %d] (got %lld)", what, kMaxParts,
                    (long long)parts);
    const int64_t total = batch * tokens * heads * (head_dim / 8);
    if (total == 0) return LTXK_OK;
    if (!out || !part || !lse) return fail(LTXK_E_ARG, "%s: null out, part or lse", what);
    if (!aligned16(out) || !aligned16(part) || (reinterpret_cast<uintptr_t>(lse) & 3u) ||
        (reinterpret_cast<uintptr_t>(logits) & 1u))
        return fail(LTXK_E_ALIGN, "%s: out and part must be 16-byte aligned, lse 4-byte, logits 2-byte", what);
    for (int64_t st : {part_bstride, part_cstride, part_hstride, part_tstride})
        if (st < 0 || st % 8) return fail(LTXK_E_ALIGN, "%s: part strides must be non-negative multiples of 8", what);
    for (int64_t st : {lse_bstride, lse_cstride, lse_hstride, lse_tstride})
        if (st < 0) return fail(LTXK_E_ARG, "%s: negative lse stride", what);
    if (total / kBlock + 1 > 0x7fffffff) return fail(LTXK_E_ARG, "%s: too many output chunks", what);
    CombineParams p{};
    p.out = static_cast<uint16_t *>(out);
    p.part = static_cast<const uint16_t *>(part);
    p.lse = lse;
    p.logits = static_cast<const uint16_t *>(logits);
    p.pbs = part_bstride;
    p.pcs = part_cstride;
    p.phs = part_hstride;
    p.pts = part_tstride;
    p.lbs = lse_bstride;
    p.lcs = lse_cstride;
    p.lhs = lse_hstride;
    p.lts = lse_tstride;
    p.tokens = tokens;
    p.heads = heads;
    p.head_dim = head_dim;
    p.chunks_per_head = head_dim / 8;
    p.total = total;
    const dim3 grid(static_cast<unsigned>((total + kBlock - 1) / kBlock)), block(kBlock);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (parts) {
    case 1: attn_combine_kernel<1><<<grid, block, 0, s>>>(p); break;
    case 2: attn_combine_kernel<2><<<grid, block, 0, s>>>(p); break;
    case 4: attn_combine_kernel<4><<<grid, block, 0, s>>>(p); break;
    case 8: attn_combine_kernel<8><<<grid, block, 0, s>>>(p); break;
    default: attn_combine_kernel<16><<<grid, block, 0, s>>>(p); break;
    }
    return check_launch(what);
}
