// Shared device/host helpers for the ltxk kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ltxk.h"

namespace ltxk {

// ---------------------------------------------------------------- errors --
// Records a message for ltxk_last_error() and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's error message.
void clear_error();
// Checks the launch that was just enqueued.
int check_launch(const char *what);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device, looked up once per device per host
// thread (256 if the runtime cannot say): persistent launches size their grid
// with it.
inline int device_cus()
{
    static thread_local int cached_dev = -1, cached_cus = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (dev != cached_dev) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached_dev = dev;
        cached_cus = cus;
    }
    return cached_cus;
}

// a / b for 0 <= a, b < 2^32 (row, element and column counts; the entry points
// reject larger shapes).  A 64-bit division compiles to a software routine
// with a branch on the operands' high words, and a branch between a kernel's
// loads makes the compiler wait for the loads before it.
__host__ __device__ __forceinline__ int64_t udiv32(int64_t a, int64_t b)
{
    return static_cast<int64_t>(static_cast<uint32_t>(a) / static_cast<uint32_t>(b));
}

// ------------------------------------------------------------ bf16 <-> f32 --
// bf16 is carried as its 16-bit pattern.  Widening is a shift; narrowing is
// round-to-nearest-even through the compiler's __bf16 conversion (gfx950 has
// a native instruction for it).
__device__ __forceinline__ float bf16_to_f32(uint16_t h)
{
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two floats -> packed pair of bf16 (low half = a), RNE: one
// v_cvt_pk_bf16_f32 (two scalar conversions cost a shift and an OR more).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// 8 bf16 values in one 16-byte vector <-> 8 floats.
__device__ __forceinline__ void unpack8(const uint4 &v, float f[8])
{
    f[0] = __uint_as_float(v.x << 16);
    f[1] = __uint_as_float(v.x & 0xffff0000u);
    f[2] = __uint_as_float(v.y << 16);
    f[3] = __uint_as_float(v.y & 0xffff0000u);
    f[4] = __uint_as_float(v.z << 16);
    f[5] = __uint_as_float(v.z & 0xffff0000u);
    f[6] = __uint_as_float(v.w << 16);
    f[7] = __uint_as_float(v.w & 0xffff0000u);
}

__device__ __forceinline__ uint4 pack8(const float f[8])
{
    uint4 v;
    v.x = pack_bf16x2(f[0], f[1]);
    v.y = pack_bf16x2(f[2], f[3]);
    v.z = pack_bf16x2(f[4], f[5]);
    v.w = pack_bf16x2(f[6], f[7]);
    return v;
}

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ void st16(void *p, const uint4 &v) { *reinterpret_cast<uint4 *>(p) = v; }

// Streaming variants for data touched exactly once (no reuse in L2/MALL).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 8 bf16 in a native 4 x u32 vector <-> 8 floats.  Kernels that keep rows
// in this type from load to store (no uint4 struct copies) schedule their
// loads better: on [6144, 4096] the broadcast norm streams at 18.4-18.7 us in
// this form against 19.4-19.7 us over uint4.
__device__ __forceinline__ void unpack8v(const u32x4 &v, float f[8])
{
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(v[j] << 16);
        f[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
    }
}

__device__ __forceinline__ u32x4 pack8v(const float f[8])
{
    return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                 pack_bf16x2(f[6], f[7])};
}

// ------------------------------------------------- buffer loads and stores --
// The streaming kernels address their activations through buffer resources:
// a workgroup-uniform base (a row, a group of rows or a block's span) in
// scalar registers, a 32-bit per-lane byte offset, and a byte range checked
// by the hardware (a load outside it returns zeros and touches no memory, a
// store outside it is dropped).  The cache policy is part of each
// instruction: loads stream (`nt`), stores write through the XCD's L2 to the
// device scope (`sc1`), so a kernel ends with no dirty L2 lines to write back.
// Measured on the [6144, 4096] bf16 norm + modulate (persistent, 2 workgroups
// per CU): global nt loads and stores 19.0 us, buffer nt/nt 18.1 us, buffer
// nt/sc1 17.0 us; a row copy of the same bytes 17.4 -> 15.7 us with sc1
// stores.  At 4x the size the streaming rate is the same for all of them,
// so the store policy removes a fixed per-launch cost.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
#ifndef LTXK_LOAD_AUX
#define LTXK_LOAD_AUX 2
#endif
#ifndef LTXK_STORE_AUX
#define LTXK_STORE_AUX 16
#endif
constexpr int kLoadStream = LTXK_LOAD_AUX;     // aux cache-policy bits: nt
constexpr int kStoreThrough = LTXK_STORE_AUX;  // aux cache-policy bits: sc1
// A streaming store: nt with sc1 (written through to device scope as it
// streams).  Against nt alone: the one-wave-per-row headline 17.23 against
// 17.33 us, residual + norm 32.2 / 40.2 against 33.0 / 41.7 us (one / two
// modulated outputs), the 48-block chain 16.63 against 16.74 ms; nt with sc0
// measured as nt alone.
constexpr int kStoreStream = 18;   // aux cache-policy bits: nt | sc1
// A byte offset past every resource's range (ranges stay below 2^31).
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes)
{
    // dword 3 of a raw (unswizzled, untyped) gfx9 buffer descriptor
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4 ldb(rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kLoadStream);
}
__device__ __forceinline__ void stb(rsrc_t r, uint32_t off, const u32x4 &v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStoreThrough);
}
// A streaming (non-temporal) store: for kernels whose extra outputs are pure
// write streams next to in-place updates (measured per kernel; most kernels
// are faster with the write-through stb).
__device__ __forceinline__ void stb_stream(rsrc_t r, uint32_t off, const u32x4 &v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStoreStream);
}
// The same with a wave-uniform part of the offset in a scalar register (the
// hardware adds voff + soff): a row's chunks at voff + k*1 KiB need no vector
// register per chunk.  Only voff is range-checked against the resource, so
// callers keep voff + soff inside it themselves (whole rows); an empty range
// still drops every access.
__device__ __forceinline__ u32x4 ldb_s(rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, static_cast<int>(soff), kLoadStream);
}
__device__ __forceinline__ void stb_s(rsrc_t r, uint32_t voff, uint32_t soff, const u32x4 &v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, static_cast<int>(soff), kStoreThrough);
}
__device__ __forceinline__ void stb_s_stream(rsrc_t r, uint32_t voff, uint32_t soff, const u32x4 &v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, static_cast<int>(soff), kStoreStream);
}
__device__ __forceinline__ uint4 ldb4(rsrc_t r, uint32_t off)
{
    const u32x4 v = ldb(r, off);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void stb4(rsrc_t r, uint32_t off, const uint4 &v) { stb(r, off, u32x4{v.x, v.y, v.z, v.w}); }

__device__ __forceinline__ uint4 ld16_stream(const void *p)
{
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16_stream(void *p, const uint4 &v)
{
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
}
__device__ __forceinline__ void st16f_stream(void *p, float a, float b, float c, float d)
{
    const f32x4 w = {a, b, c, d};
    __builtin_nontemporal_store(w, reinterpret_cast<f32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld16f_stream(const void *p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}

// --------------------------------------------------------- AdaLN operand --
// Device view of an ltxk_ada: value(b, t, d) = round(tab[d] + emb[off + d]),
// off = b*bs + t*ts, or idx[row]*ts for an indexed operand (one embedding
// row per distinct timestep; the index is clamped into [0, idx_rows)).
struct Ada {
    const uint16_t *tab;
    const uint16_t *emb;
    int64_t bs;
    int64_t ts;
    const int32_t *idx;
    uint32_t idx_rows;
    int kind;  // 0 absent, 1 tab only, 2 emb only, 3 both
};

inline Ada make_ada(const ltxk_ada *a)
{
    Ada r{nullptr, nullptr, 0, 0, nullptr, 0, 0};
    if (!a) return r;
    r.tab = static_cast<const uint16_t *>(a->tab);
    r.emb = static_cast<const uint16_t *>(a->emb);
    r.bs = a->emb_bstride;
    r.ts = a->emb_tstride;
    r.idx = a->emb ? a->emb_index : nullptr;
    r.idx_rows = static_cast<uint32_t>(a->emb_rows);
    r.kind = (r.tab ? 1 : 0) | (r.emb ? 2 : 0);
    return r;
}

inline bool ada_aligned(const Ada &a)
{
    return aligned16(a.tab) && aligned16(a.emb) && (a.bs % 8) == 0 && (a.ts % 8) == 0;
}

// Offset (elements) of the embedding row that activation row `row` = (b, t) reads.
__device__ __forceinline__ int64_t ada_emb_off(const Ada &a, int64_t b, int64_t t, int64_t row)
{
    if (a.idx) {
        const uint32_t u = static_cast<uint32_t>(a.idx[row]);  // negative clamps high, like too large
        return static_cast<int64_t>(u < a.idx_rows ? u : a.idx_rows - 1) * a.ts;
    }
    return b * a.bs + t * a.ts;
}

// Zeros standing in for an absent table or embedding row, so that an AdaLN
// operand is always two unconditional loads (branches around loads would make
// the compiler wait for each load before the next one issues).  Read-only.
__device__ __align__(16) static uint16_t g_ada_zeros[16384];

// Raw 16-byte fetch of one AdaLN operand chunk (table part and embedding
// part), issued early and finished later so its latency overlaps other loads.
struct AdaRaw {
    uint4 tab, emb;
};

__device__ __forceinline__ AdaRaw ada_fetch(const Ada &a, int64_t b, int64_t t, int64_t row, int64_t d)
{
    const uint16_t *tab = a.tab ? a.tab : g_ada_zeros;
    const uint16_t *emb = a.emb ? a.emb + ada_emb_off(a, b, t, row) : g_ada_zeros;
    return AdaRaw{ld16(tab + d), ld16(emb + d)};
}

// The 8 modulation values of a fetched chunk.  The reference materialises
// table + timestep as a bf16 tensor; when one side is absent (zero) the
// rounding is exact and returns the other.  `absent_value` stands for an
// operand with neither part.
__device__ __forceinline__ void ada_finish(const Ada &a, const AdaRaw &r, float absent_value, float out[8])
{
    float tv[8], ev[8];
    unpack8(r.tab, tv);
    unpack8(r.emb, ev);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = a.kind ? bf16_to_f32(f32_to_bf16(tv[i] + ev[i])) : absent_value;
}

// p[i] as fp32 when p is set, else 0, with one unconditional load: the
// address selects p or the zero row, so no branch guards the load (a load
// under a branch makes the compiler wait for it, and for every load issued
// before it, right where it is issued).
__device__ __forceinline__ float ld_bf16_or_zero(const uint16_t *p, int64_t i)
{
    return bf16_to_f32(*(p ? p + i : g_ada_zeros));
}

__device__ __forceinline__ void ada_load8(const Ada &a, int64_t b, int64_t t, int64_t row, int64_t d,
                                          float absent_value, float out[8])
{
    ada_finish(a, ada_fetch(a, b, t, row, d), absent_value, out);
}

// ----------------------------------------------------------- reductions --
// Sums of squares for the norms accumulate with fused multiply-adds (one
// rounding per term instead of two; the summation order differs from any
// eager evaluation anyway).  Everything else keeps the reference's separate
// multiplies and adds: the build passes -ffp-contract=off.
__device__ __forceinline__ float dpp_add(float v, int ctrl_sel)
{
    // ctrl_sel picks one of the fixed DPP patterns below (must be constant).
    int iv = __builtin_bit_cast(int, v);
    int r;
    switch (ctrl_sel) {
    case 0: r = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    case 1: r = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false); break;   // quad_perm 2,3,0,1
    case 2: r = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
    default: r = __builtin_amdgcn_update_dpp(0, iv, 0x140, 0xF, 0xF, false); break; // row_mirror
    }
    return v + __builtin_bit_cast(float, r);
}

// Sum over all 64 lanes of the wave, result in every lane.
__device__ __forceinline__ float wave_sum64(float v)
{
    v = dpp_add(v, 0);
    v = dpp_add(v, 1);
    v = dpp_add(v, 2);
    v = dpp_add(v, 3);  // every lane: sum of its 16-lane DPP row
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Sum over the TPR threads that own one row.  Every thread of the block calls
// it (TPR == 256 uses a barrier).
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float *lds)
{
    if constexpr (TPR < 64) {
#pragma unroll
        for (int o = TPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        return v;
    } else if constexpr (TPR == 64) {
        return wave_sum64(v);
    } else {
        v = wave_sum64(v);
        const int wave = threadIdx.x >> 6;
        const int w0 = (threadIdx.x / TPR) * (TPR / 64);  // first wave of this row
        if ((threadIdx.x & 63) == 0) lds[wave] = v;
        __syncthreads();
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < TPR / 64; ++w) s += lds[w0 + w];
        __syncthreads();
        return s;
    }
}

}  // namespace ltxk
