// Shared device helpers for the HBA kernels (gfx950 only).
//
// Storage types: fp32 and bf16.  bf16 rounding is round-to-nearest-even,
// identical to the rounding the reference applies when it casts fp32 results
// back to bf16 tensors (e.g. _HeadRMSNorm's `.to(x.dtype)`,
// src/hba/attention.py:94).
//
// All code is compiled with -ffp-contract=off: every a*b+c below is two
// roundings unless written as fmaf().  The declared-order routines
// (qknorm_row, dot_decl, slot max) reproduce the oracle's operation order
// exactly so that block selection is bit-exact.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hba_amd.h"

namespace hba {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t bf16_t;  // raw bf16 bits in memory

__device__ __forceinline__ float bf2f(bf16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even; a NaN stays a (quiet) NaN.  Branch
// free: infinities pass through the rounding unchanged, finite values that
// round past the largest bf16 become infinities, as RNE requires.
__device__ __forceinline__ bf16_t f2bf(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t qnan = (u >> 16) | 0x40u;
    return (bf16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? qnan : r);
}

__device__ __forceinline__ float rnd_bf16(float x) { return bf2f(f2bf(x)); }

// Two values rounded to bf16 (nearest even) at once by v_cvt_pk_bf16_f32 and
// widened back: the same results as rnd_bf16 for every non-NaN input.
__device__ __forceinline__ void rnd_bf16_pair(float &a, float &b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
}

// Two values as packed bf16 (nearest even; a in the low half), the same bits
// as f2bf for every non-NaN input.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Storage-type traits: DT 0 = fp32, 1 = bf16.
template <int DT> struct St;
template <> struct St<0> {
    typedef float T;
    static __device__ __forceinline__ float ld(const T *p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(T *p, int64_t i, float v) { p[i] = v; }
    static __device__ __forceinline__ float rnd(float v) { return v; }
};
template <> struct St<1> {
    typedef bf16_t T;
    static __device__ __forceinline__ float ld(const T *p, int64_t i) { return bf2f(p[i]); }
    static __device__ __forceinline__ void st(T *p, int64_t i, float v) { p[i] = f2bf(v); }
    static __device__ __forceinline__ float rnd(float v) { return rnd_bf16(v); }
};

// Largest candidate block of query position i (0 = none):
// candidate(i, b) <=> b >= 1 and (b + 1) * Bk <= i - W + 1   (attention.py:250-256)
__device__ __host__ __forceinline__ int64_t cand_bmax(int64_t i, int64_t Bk, int64_t W) {
    int64_t lim = i - W + 1;
    if (lim < 2 * Bk) return 0;
    return lim / Bk - 1;
}

// Paged cache layouts (one page = 64 tokens of one KV head, D elements each),
// ordered so that every 16-byte operand load of the decode MFMA tiles is part
// of a contiguous 1 KB run across the wave's 64 lanes (lane L = l16 + 16*lg):
//   keys  (kc_pages, kr_pages): key j, element t at
//         ((mt * (D/32) + ks) * 64 + l16 + 16*lg) * 8 + e, where
//         mt = 2*(j/32) + (j/4)%2, l16 = 4*((j%32)/8) + j%4  (the S^T tile row
//         that holds key j), ks = t/32, lg = (t%32)/8, e = t%8;
//   values (v_pages): key j, element t at
//         ((dt * 2 + h) * 64 + l16 + 16*lg) * 8 + e, where
//         dt = t/16, l16 = t%16, h = j/32, lg = (j%32)/8, e = j%8.
__host__ __device__ __forceinline__ int64_t page_key_off(int j, int t, int D) {
    const int mt = 2 * (j >> 5) + ((j >> 2) & 1);
    const int l16 = 4 * ((j & 31) >> 3) + (j & 3);
    return ((int64_t)(mt * (D / 32) + (t >> 5)) * 64 + l16 + 16 * ((t >> 3) & 3)) * 8 + (t & 7);
}
__host__ __device__ __forceinline__ int64_t page_val_off(int j, int t) {
    return ((int64_t)((t >> 4) * 2 + (j >> 5)) * 64 + (t & 15) + 16 * ((j >> 3) & 3)) * 8 + (j & 7);
}
// Inverse for a chunk of 8 consecutive storage elements c*8 .. c*8+7: keys
// hold key j, elements t0 .. t0+7; values hold element t, keys j0 .. j0+7.
__host__ __device__ __forceinline__ void page_key_chunk(int c, int D, int &j, int &t0) {
    const int L = c & 63, r = c >> 6, ks = r % (D / 32), mt = r / (D / 32);
    const int l16 = L & 15, lg = L >> 4;
    j = 32 * (mt >> 1) + 8 * (l16 >> 2) + 4 * (mt & 1) + (l16 & 3);
    t0 = 32 * ks + 8 * lg;
}
__host__ __device__ __forceinline__ void page_val_chunk(int c, int &t, int &j0) {
    const int L = c & 63, r = c >> 6;
    t = 16 * (r >> 1) + (L & 15);
    j0 = 32 * (r & 1) + 8 * (L >> 4);
}

// QKNorm of one row held in registers, declared order (see oracle):
// ss = fma(x,x,ss) sequential, ms = ss/d, ms = max(ms, eps), r = sqrt(ms),
// y = (x / r) * gain, rounded to the storage dtype.
template <int DT, int D>
__device__ __forceinline__ void qknorm_row(float (&x)[D], float gain, float eps) {
    float ss = 0.0f;
#pragma unroll
    for (int t = 0; t < D; ++t) ss = fmaf(x[t], x[t], ss);
    float ms = ss / (float)D;
    if (ms < eps) ms = eps;
    float r = sqrtf(ms);
#pragma unroll
    for (int t = 0; t < D; ++t) x[t] = St<DT>::rnd((x[t] / r) * gain);
}

// RoPE of one row (rotate-half; cos/sin rounded to the storage dtype and each
// elementwise op rounded, as apply_rope does on x.dtype tensors).
template <int DT, int D>
__device__ __forceinline__ void rope_row(const float (&x)[D], float (&y)[D], const float *cs,
                                         const float *sn) {
    constexpr int H = D / 2;
#pragma unroll
    for (int t = 0; t < D; ++t) {
        float rot = (t < H) ? -x[t + H] : x[t - H];
        float c = St<DT>::rnd(cs[t]);
        float s = St<DT>::rnd(sn[t]);
        float t1 = St<DT>::rnd(x[t] * c);
        float t2 = St<DT>::rnd(rot * s);
        y[t] = St<DT>::rnd(t1 + t2);
    }
}

// x / r rounded to nearest even, bit-identical to the IEEE quotient, from
// inv = 1.0f / r (the correctly rounded reciprocal): q0 = x * inv is within
// one ulp of x / r, so e = fma(-q0, r, x) is exact, and q0 + e * inv rounds
// to x / r (Markstein's correction step).  Valid for 2^-30 <= r <= 2^30 and
// x zero or normal (div_rn_ok); e == 0 keeps q0, which keeps a zero's sign.
// Checked against the IEEE quotient on 4e8 random operand pairs in that
// range; subnormal x and out-of-range r take the IEEE division.
__device__ __forceinline__ bool div_rn_row_ok(float r) { return r >= 0x1p-30f && r <= 0x1p30f; }
__device__ __forceinline__ bool div_rn_subnormal(float x) {
    return __builtin_amdgcn_class(x, 0x010 | 0x080);   // negative or positive subnormal
}
__device__ __forceinline__ float div_rn_fast(float x, float r, float inv) {
    const float q0 = x * inv;
    const float e = fmaf(-q0, r, x);
    return (e == 0.0f) ? q0 : fmaf(e, inv, q0);
}

// ----------------------------------------------------------- wave helpers --
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace hba

// Host-side launch check.
#define HBA_LAUNCH_CHECK()                                      \
    do {                                                        \
        if (hipGetLastError() != hipSuccess) return HBA_ERR_LAUNCH; \
    } while (0)
