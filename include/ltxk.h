/*
 * ltxk: MI355X (gfx950) kernels for the memory-bound core of the LTX-2.5
 * audio-video DiT denoise step.  Plain C ABI: device pointers, sizes, strides
 * and a HIP stream handle (passed as void*; NULL = the default stream).
 *
 * Conventions (every entry point):
 *   - Buffers are owned by the caller; nothing here allocates or frees
 *     device memory, and nothing synchronises the host.  Work is enqueued on
 *     `stream` in order.
 *   - Activations are row-major [rows, dim], rows = batch * tokens, contiguous,
 *     16-byte aligned; dim must be a multiple of 8 (16 for the RoPE kernel).
 *   - Return 0 on success or an LTXK_E_* code; ltxk_last_error() returns a
 *     message for the calling thread's last failure.  Nothing here exits.
 *   - Floating-point kernels compute in fp32 and round each output once.
 *
 * The reference path has no native operator layer: its hot path is the
 * Python module API of standalone/ltx_nn.py and standalone/ltx_dit.py calling
 * torch eager ops, plus the native TorchRNG of
 * cuda_c_standalone/common/philox.h:6-18.  Each entry point below names the
 * reference function it stands in for.
 */
#ifndef LTXK_H
#define LTXK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTXK_OK 0
#define LTXK_E_ARG 1      /* null pointer, bad size or unsupported shape */
#define LTXK_E_ALIGN 2    /* pointer or row not 16-byte aligned */
#define LTXK_E_DTYPE 3    /* unsupported dtype code */
#define LTXK_E_HIP 4      /* the HIP runtime reported an error */

#define LTXK_DTYPE_F32 0
#define LTXK_DTYPE_BF16 1

/* ABI version of this header.  It changes whenever an entry point's
 * arguments or a struct's layout change (200: ltxk_ada gained emb_index and
 * emb_rows, ltxk_qk gained table_rows), so a caller built against another
 * header can refuse the library: check ltxk_version() == LTXK_VERSION. */
#define LTXK_VERSION 200

/* The ABI version the library was built with (LTXK_VERSION of its header). */
int ltxk_version(void);

/* Message describing the calling thread's most recent failure ("" if none). */
const char *ltxk_last_error(void);

/* ----------------------------------------------------------------------- */
/* Philox4x32-10 Gaussian noise                                            */
/* ----------------------------------------------------------------------- */

/* Thread count T of the reference's grid-stride launch policy:
 * 256 * min(ceil(n/256), multiprocessors * floor(max_threads_per_mp/256)).
 * Replaces calc_policy, cuda_c_standalone/common/philox.cu:6-17. */
int64_t ltxk_philox_policy_threads(int64_t n, int64_t multiprocessors, int64_t max_threads_per_mp);

/* Offset advance after drawing n values with T threads: 4*ceil(n/(4T)).
 * Replaces the bookkeeping of philox.cu:47-61 (TorchRNG::randn_* then
 * offset += policy_counter_offset(n)). */
int64_t ltxk_philox_offset_advance(int64_t n, int64_t total_threads);

/* out[e], e in [0,n): N(0,1) from Philox4x32-10 with key = seed and counter
 * (offset/4 + e/(4T), e%T), lane (e/T)%4, Box-Muller pairs (sin, cos).
 * dtype LTXK_DTYPE_F32 or LTXK_DTYPE_BF16 (RNE).  offset % 4 == 0.
 * Replaces TorchRNG::randn_fp32 / randn_bf16 (philox.h:15-17,
 * philox.cu:19-61) and torch.randn(..., generator) as called by
 * create_noised_states (standalone/ltx_dit.py:495-520). */
int ltxk_philox_normal(void *out, int dtype, int64_t n, uint64_t seed, uint64_t offset,
                       int64_t total_threads, void *stream);

/* Raw uint32 Philox stream in the same element order as ltxk_philox_normal:
 * out[e] = word (e/T)%4 of the block for thread e%T at iteration e/(4T).
 * The integer half of philox.cu:19-35 exposed for bit-exact checking. */
int ltxk_philox_u32(uint32_t *out, int64_t n, uint64_t seed, uint64_t offset, int64_t total_threads,
                    void *stream);

/* ----------------------------------------------------------------------- */
/* Flow-matching Euler                                                     */
/* ----------------------------------------------------------------------- */

/* x <- x + dt*v elementwise (product rounded before the add, as the two
 * tensor ops of the reference).  dtype F32 or BF16. */
int ltxk_euler_update(void *x, const void *v, int64_t n, int dtype, float dt, void *stream);

/* euler_step (standalone/ltx_dit.py:602-606):
 *   vel = round((sample - denoised) / sigma);  out = round(sample + vel*dt)
 * all in fp32 from the stored values, round() to dtype.  out may alias sample. */
int ltxk_euler_step(void *out, const void *sample, const void *denoised, int64_t n, int dtype, float sigma,
                    float dt, void *stream);

/* X0Model (standalone/ltx_dit.py:592-593): x0 = round(latent - v * ts[b,t])
 * for rows (b, t) of [rows, dim] bf16, ts fp32 at ts[b*ts_batch_stride +
 * t*ts_token_stride] (token stride 0: one timestep per batch item). */
int ltxk_x0(void *x0, const void *latent, const void *velocity, const float *ts, int64_t ts_batch_stride,
            int64_t ts_token_stride, int64_t rows, int64_t tokens, int64_t dim, void *stream);

/* ----------------------------------------------------------------------- */
/* Guidance tail of a denoising step                                       */
/* ----------------------------------------------------------------------- */

/* GuiderParams (standalone/ltx_dit.py:542-548) without the block list. */
typedef struct ltxk_guidance {
    double cfg_scale;
    double stg_scale;
    double modality_scale;
    double rescale_scale;  /* 0: no std rescale */
} ltxk_guidance;

/* Workspace bytes ltxk_guide needs for n = rows*dim elements when
 * rescale_scale != 0 (at most 8 KB). */
int64_t ltxk_guide_workspace_bytes(int64_t n);

/* x0 of the four guidance passes, guide() and euler_step in one pass over
 * the latent (standalone/ltx_dit.py:551-562 guide, :592-598 the x0/chunk
 * part of guided_denoise_step, :602-606 euler_step):
 *   latent    [rows, dim] bf16 (the state latent, shared by the passes)
 *   velocity  [4, rows, dim] bf16: model outputs of cond, uncond, ptb, mod
 *   timesteps fp32 ts[p*ts_pass_stride + row*ts_row_stride]
 *   x0_p      = round(latent - velocity_p * ts_p)
 *   pred      = c + (cfg-1)(c-u) + stg(c-p) + (mod-1)(c-m), c = x0_cond (fp32)
 *   if rescale_scale != 0: pred *= r*std(c)/std(pred) + (1-r) (unbiased std
 *                          over all rows*dim elements)
 *   denoised  = round(pred)                           -> denoised [rows, dim]
 *   next      = round(latent + round((latent - denoised)/sigma)*dt) -> next
 *   x0 (optional) receives the four x0_p, [4, rows, dim].
 * timesteps NULL: `velocity` holds the four x0_p themselves (guide() alone,
 * ltx_dit.py:551-562); latent is then needed only for the Euler step.
 * Outputs may be NULL (not written); next may alias latent (each element is
 * read before it is written, by the same thread).  dim % 8 == 0,
 * rows*dim <= 2^28, bf16 buffers 16-byte aligned.  With rescale_scale != 0,
 * `workspace` is 8-byte aligned device memory of ltxk_guide_workspace_bytes
 * bytes that holds partial sums between the two launches: concurrent calls
 * need separate workspaces. */
int ltxk_guide(void *denoised, void *x0, void *next, const void *latent, const void *velocity,
               const float *timesteps, int64_t ts_pass_stride, int64_t ts_row_stride, int64_t rows, int64_t dim,
               const ltxk_guidance *g, float sigma, float dt, void *workspace, int64_t workspace_bytes,
               void *stream);

/* ltxk_guide with no workspace argument and no allocation of any kind.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  The rescale's partial sums live in the library's own
 * device array (8 KB per GPU, held until the process ends; its address is
 * looked up once per device with hipGetSymbolAddress, with that device
 * current), which covers every size ltxk_guide accepts: rows*dim <= 2^28.
 * The stream must belong to the current device.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (concurrent streams or
 * threads) race and must be serialised by the caller.  Nothing needs to be
 * zero between calls: each call writes every partial it reads. */
int ltxk_guide_noalloc(void *denoised, void *x0, void *next, const void *latent, const void *velocity,
                       const float *timesteps, int64_t ts_pass_stride, int64_t ts_row_stride, int64_t rows,
                       int64_t dim, const ltxk_guidance *g, float sigma, float dt, void *stream);

/* ----------------------------------------------------------------------- */
/* Text-encoder connector: multi-layer feature normalisation               */
/* ----------------------------------------------------------------------- */

/* FeatureExtractorV2 up to its two projections (standalone/ltx_te.py:167-184):
 * for the n_layers (1..64) hidden states layers[l], each [rows, dim] bf16,
 *   n_l[r, d]         = round(x_l[r, d] * rsqrt(mean_d(x_l[r, :]^2) + eps))
 *   out0[r, d*L + l]  = keep[r] ? round(n_l[r, d] * scale0) : +0
 *   out1[r, d*L + l]  = keep[r] ? round(n_l[r, d] * scale1) : +0   (out1 may be NULL)
 * outputs [rows, dim*n_layers] bf16 (the reference's stack over a new last
 * axis, flattened); keep: [rows] bytes, non-zero = token kept, or NULL (all
 * kept).  The outputs of a masked token do not depend on its hidden states:
 * when the token's L rows fit in one workgroup's registers they are not
 * read.  `layers` is a host array of device pointers.  dim % 8 == 0.  One
 * launch, no workspace. */
int ltxk_feature_norm(void *out0, void *out1, const void *const *layers, int64_t n_layers, const uint8_t *keep,
                      int64_t rows, int64_t dim, float eps, float scale0, float scale1, void *stream);

/* ----------------------------------------------------------------------- */
/* AdaLN modulation operands                                               */
/* ----------------------------------------------------------------------- */

/* One modulation vector (shift, scale or gate) of get_ada_values
 * (standalone/ltx_dit.py:192-198): value[b,t,d] = round(tab[d] +
 * emb[b*emb_bstride + t*emb_tstride + d]).  tab or emb may be NULL (then the
 * other is used alone, unrounded); both NULL means "absent".  Element type is
 * bf16.  emb_tstride 0 means one row per batch item (broadcast over tokens).
 *
 * Indexed form (emb_index != NULL): the timestep embedding holds one row per
 * distinct timestep value instead of one per token (the reference computes
 * the AdaLN MLP per token, ltx_dit.py:146-150, although a keyframe-
 * conditioned step has only two values: 0 on the conditioning tokens and
 * sigma elsewhere).  Activation row r = b*tokens + t then reads embedding
 * row emb_index[r]: value = round(tab[d] + emb[emb_index[r]*emb_tstride + d]);
 * emb_bstride is unused and emb_rows (> 0) is the number of embedding rows:
 * the kernels clamp every index into [0, emb_rows). */
typedef struct ltxk_ada {
    const void *tab;
    const void *emb;
    int64_t emb_bstride;
    int64_t emb_tstride;
    const int32_t *emb_index;
    int64_t emb_rows;
} ltxk_ada;

/* ----------------------------------------------------------------------- */
/* Row normalisation + modulation                                          */
/* ----------------------------------------------------------------------- */

#define LTXK_NORM_RMS 0        /* x * rsqrt(mean(x^2) + eps)              */
#define LTXK_NORM_LAYER 1      /* (x - mean) * rsqrt(var + eps), no affine */

/* y = norm(x) * (1 + scale) + shift for every row, and optionally a second
 * output y2 = norm(x) * (1 + scale2) + shift2 from the same read of x.
 * scale/shift "absent" means 0.  bf16 in/out, fp32 math, one rounding.
 * Replaces `rms_norm(x) * (1 + scale) + shift` at standalone/ltx_dit.py:261,
 * 273,290,294,301,305,311,314 and norm_out + modulate in LTXModel._output
 * (ltx_dit.py:371-378; norm = LTXK_NORM_LAYER). */
int ltxk_norm_modulate(void *y, void *y2, const void *x, int64_t rows, int64_t tokens, int64_t dim, int norm,
                       float eps, const ltxk_ada *shift, const ltxk_ada *scale, const ltxk_ada *shift2,
                       const ltxk_ada *scale2, void *stream);

/* y = round(rmsnorm(x) * weight) over rows of [rows, dim]; weight may be NULL.
 * Replaces rms_norm (standalone/ltx_nn.py:18-19, common.py:134-135) and the
 * torch.nn.RMSNorm q_norm/k_norm when applied without RoPE (ltx_nn.py:214-215). */
int ltxk_rms_norm(void *y, const void *x, const void *weight, int64_t rows, int64_t dim, float eps, void *stream);

/* Gated residual fused with the next norm + modulation:
 *   x_out = round(x + f * gate * mask[b]);  y = rmsnorm(x_out)*(1+scale)+shift
 *   and optionally y2 = rmsnorm(x_out)*(1+scale2)+shift2 from the same pass.
 * gate absent = 1; mask NULL = 1 (mask is one bf16 per batch item, a 0/1 keep
 * mask).  y may be NULL (then only the residual is written); y2 needs y.
 * x_out may alias x.
 * Replaces `vx_fma = vx + out * vgate; rms_norm(vx_fma)` followed by the
 * text-cross query modulation (ltx_dit.py:245,265-266); the text-cross
 * residual followed by the two A2V/V2A modulations of the same row
 * (ltx_dit.py:267,290,305); the A2V/V2A residual followed by the FFN norm
 * (ltx_dit.py:295-296,306-307,311,314); the FFN residual followed by the
 * next block's first norm (ltx_dit.py:311 then 261). */
int ltxk_add_norm_modulate(void *x_out, void *y, void *y2, const void *x, const void *f, const ltxk_ada *gate,
                           const void *mask, int64_t rows, int64_t tokens, int64_t dim, float eps,
                           const ltxk_ada *shift, const ltxk_ada *scale, const ltxk_ada *shift2,
                           const ltxk_ada *scale2, void *stream);

/* y = round(x * (1 + scale) + shift) with no normalisation: the context
 * modulation `context * (1 + scale_kv) + shift_kv` (ltx_dit.py:246). */
int ltxk_modulate(void *y, const void *x, int64_t rows, int64_t tokens, int64_t dim, const ltxk_ada *shift,
                  const ltxk_ada *scale, void *stream);

/* The context modulation of `layers` blocks from one read of x:
 *   y[l] = round(x * (1 + scale_l) + shift_l),  l in [0, layers),
 * y [layers, rows, dim]; shift_l / scale_l are the operands shift / scale
 * with their tab pointers advanced by l * tab_layer_stride elements and their
 * emb pointers by l * emb_layer_stride (0: the same embedding row for every
 * layer).  Each y[l] equals ltxk_modulate with the layer-l operands.  Replaces
 * the once-per-block `context * (1 + scale_kv) + shift_kv` of the text
 * cross-attention (standalone/ltx_dit.py:240-246) for all blocks of a step:
 * the context, the blocks' prompt tables and the prompt timestep do not
 * change between blocks.  Strides are multiples of 8 elements;
 * layers*rows <= 2^31. */
int ltxk_modulate_layers(void *y, const void *x, int64_t layers, int64_t rows, int64_t tokens, int64_t dim,
                         const ltxk_ada *shift, const ltxk_ada *scale, int64_t tab_layer_stride,
                         int64_t emb_layer_stride, void *stream);

/* ----------------------------------------------------------------------- */
/* q/k preparation: RMSNorm with weight and split RoPE                     */
/* ----------------------------------------------------------------------- */

/* One tensor operand of ltxk_qk_norm_rope.  x is [batch*tokens, heads*head_dim]
 * bf16 (token-major, as the q/k projections produce it); updated in place.
 * weight: [heads*head_dim] bf16 RMSNorm weight, or NULL for no norm.
 * cos/sin: rotation tables, NULL for no rotation, in one of two forms:
 *   full     (pos_index NULL): bf16 (batch, heads, tokens, head_dim/2) as
 *            precompute_freqs_cis returns them, table_bstride elements between
 *            batch items (0 = shared);
 *   compact  (pos_index != NULL): bf16 rows [R, heads*head_dim/2]; row r holds
 *            cos (sin) of one coordinate value of one position axis at that
 *            axis' pairs and +0.0 (bits 0) elsewhere (axis 0's rows also carry
 *            the identity padding: cos 1, sin 0); pos_index [batch*tokens,
 *            n_axes] int32 gives each token's row for every axis, and
 *            table_rows = R (required, > 0): the kernel clamps every index
 *            into [0, R), so a bad index reads a wrong row, never outside the
 *            tables.  A pair's value is the one non-zero axis entry (the rows'
 *            bits are OR-ed), equal to the full table's entry. */
typedef struct ltxk_qk {
    void *x;
    const void *weight;
    const void *cos;
    const void *sin;
    int64_t batch;
    int64_t tokens;
    int64_t table_bstride;
    const int32_t *pos_index;
    int64_t n_axes;
    int64_t table_rows;
} ltxk_qk;

/* For q and (optionally, k.x != NULL) k:
 *   x = rope(rmsnorm(x) * weight) in place, one rounding per element.
 * rope is LTXRopeType.SPLIT per head: halves (x1, x2) ->
 *   (x1*c - x2*s, x2*c + x1*s).
 * Limits: heads*head_dim <= 32768, head_dim a multiple of 16, each operand's
 * batch*tokens < 2^31; launches that take one wavefront per row (rows of
 * 2048 or 4096 without tables, rows of 2048 with 64-wide heads on one-axis
 * compact tables) take at most 2^31 - 2^20 rows (q's plus k's; tokens when
 * q and k share tables) and return LTXK_E_ARG above that.
 * Replaces Attention.q_norm/k_norm + apply_split_rotary_emb
 * (standalone/ltx_nn.py:99-115,186-187,214-218). */
int ltxk_qk_norm_rope(const ltxk_qk *q, const ltxk_qk *k, int64_t heads, int64_t head_dim, float eps,
                      void *stream);

/* ----------------------------------------------------------------------- */
/* Elementwise                                                             */
/* ----------------------------------------------------------------------- */

/* y = round(0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))), bf16, y may alias x.
 * Replaces F.gelu(approximate="tanh") in FeedForward (ltx_nn.py:247-248). */
int ltxk_gelu_tanh(void *y, const void *x, int64_t n, void *stream);

/* out = round(x + f * gate * mask[b]); gate absent = 1, mask NULL = 1.
 * Replaces `x + out * gate` residuals (ltx_dit.py:247,265,277,311,314) and
 * `* gate * mask` (ltx_dit.py:295-296,306-307). */
int ltxk_gated_residual(void *out, const void *x, const void *f, const ltxk_ada *gate, const void *mask,
                        int64_t rows, int64_t tokens, int64_t dim, void *stream);

/* Attention epilogue between SDPA and to_out, one pass:
 *   a = x[b, t, h, :]                       (read through strides)
 *   a = a*m[b] + v[b*T + t, h, :]*(1 - m[b])  if v != NULL (perturbation blend)
 *   out[b*T + t, h, :] = round(a * 2*sigmoid(logits[b*T + t, h]))  (gate 1 if logits NULL)
 * x is read through strides (elements) for batch, token and head with the
 * head_dim axis contiguous, so the attention output is consumed in whatever
 * (batch, heads, tokens, head_dim) view SDPA returns; out, v are contiguous
 * token-major [batch*tokens, heads*head_dim]; logits contiguous
 * [batch*tokens, heads]; mask is one 0/1 bf16 keep value per batch item.
 * Replaces the head merge `out.transpose(1, 2).reshape(...)`, the perturbation
 * blend and the per-head gate of Attention.forward (ltx_nn.py:228-235). */
int ltxk_head_gate(void *out, const void *x, int64_t x_bstride, int64_t x_tstride, int64_t x_hstride,
                   const void *logits, const void *v, const void *mask, int64_t batch, int64_t tokens,
                   int64_t heads, int64_t head_dim, void *stream);

/* Combine of key-split attention partials + the attention epilogue's head
 * merge and per-head gate, one pass.  For each (b, t, h), with part_c the
 * attention output over key chunk c (c < parts) and lse_c its log-sum-exp:
 *   w_c = exp(lse_c - max lse) / sum_c' exp(lse_c' - max lse)
 *   o   = round(sum_c w_c * part_c)                          (fp32, bf16 once)
 *   out[b*T + t, h, :] = round(o * 2*sigmoid(logits[b*T + t, h]))  (gate 1 if logits NULL)
 * part element (b, c, h, t, d) at part + b*part_bstride + c*part_cstride +
 * h*part_hstride + t*part_tstride + d (bf16, strides in elements, multiples
 * of 8); lse element (b, c, h, t) likewise (fp32); out contiguous token-major
 * [batch*tokens, heads*head_dim]; parts a power of two up to 16.
 * Stands in for SDPA (ltx_nn.py:22-26,227) when the keys are split for few
 * queries over many keys (the V2A attention), and for the head merge and gate
 * after it (ltx_nn.py:228-235). */
int ltxk_attn_combine(void *out, const void *part, int64_t part_bstride, int64_t part_cstride,
                      int64_t part_hstride, int64_t part_tstride, const float *lse, int64_t lse_bstride,
                      int64_t lse_cstride, int64_t lse_hstride, int64_t lse_tstride, const void *logits,
                      int64_t batch, int64_t parts, int64_t tokens, int64_t heads, int64_t head_dim, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LTXK_H */
