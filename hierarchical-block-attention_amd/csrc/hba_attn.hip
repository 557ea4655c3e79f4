// Union attention forward: one softmax per (query i, head h) over
//   sinks   j < min(S, i+1)               NoPE  (qc . kc)
//   window  max(S, i-W+1) <= j <= i        RoPE  (qr . kr)
//   routed  the Bk keys of each valid selected block      NoPE
// (hba_attention_dense src/hba/attention.py:342-356, hba_attention_eval
//  :676-711, hba_attention_fused's LSE merge :592-603).
//
// bf16: attn_bf16_kernel, MFMA v_mfma_f32_16x16x32_bf16, one workgroup per
//   (batch, KV head, tile of QT queries) with one wave per query head of the
//   group.  Two phases share one workgroup and merge on chip:
//   phase B (routed): each wave takes whole queries; the MFMA rows are the G
//     heads of that query (the only rows that share a routed block), keys of
//     each selected block stream from HBM/L2 straight into MFMA operands;
//     the partial (O, m, l) per (query, head) goes to LDS;
//   phase A (sinks + window): rows are the QT queries of the wave's head;
//     64-key tiles of RoPE'd keys and V^T are staged in LDS and shared by all
//     G waves (the sliding window is what consecutive queries share);
//   merge: LSE merge of the two partials, normalise, store.
//   Scores are computed as S^T = K . Q^T so that the probabilities come out
//   of the MFMA accumulators already in the B-operand layout of the P.V MFMA
//   (key rows of the K operand are permuted to make that exact).
// f32: attn_f32_kernel, one thread per (query, head), sequential fp32 dot
//   products and a two-pass softmax; the fp32 parity path.
#include "hba_common.h"
#include "hba_abi.h"

namespace hba {

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
constexpr float LOG2E_F = 1.4426950408889634f;

__device__ __forceinline__ bf16x8 ld_b8(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4v *>(p));
}

__device__ __forceinline__ bf16x8 pack_b8(const float (&x)[8]) {
    u32x4v u;
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = (uint32_t)f2bf(x[2 * e]) | ((uint32_t)f2bf(x[2 * e + 1]) << 16);
    return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------ fp32 path ----
template <int D>
__device__ __forceinline__ float dot_row(const float (&qv)[D], const float *k) {
    float a = 0.0f;
#pragma unroll
    for (int t = 0; t < D; t += 4) {
        float4 kv = *reinterpret_cast<const float4 *>(k + t);
        a = fmaf(qv[t], kv.x, a);
        a = fmaf(qv[t + 1], kv.y, a);
        a = fmaf(qv[t + 2], kv.z, a);
        a = fmaf(qv[t + 3], kv.w, a);
    }
    return a;
}

template <int D>
__global__ __launch_bounds__(64) void attn_f32_kernel(
    const float *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const float *__restrict__ kc, const float *__restrict__ kr, const float *__restrict__ vt,
    const float *__restrict__ cosT, const float *__restrict__ sinT, const int32_t *__restrict__ idx,
    const int32_t *__restrict__ cnt, int64_t n, int Hq, int Hkv, int S, int64_t W, int kk, float scale,
    float *__restrict__ out, int64_t osb, int64_t osn, int64_t osh) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (i >= n) return;
    const int G = Hq / Hkv;
    const int g = h / G;
    float qc[D], qr[D];
    const float *qrow = q + b * qsb + i * qsn + (int64_t)h * qsh;
#pragma unroll
    for (int t = 0; t < D; t += 4) {
        float4 u = *reinterpret_cast<const float4 *>(qrow + t);
        qc[t] = u.x;
        qc[t + 1] = u.y;
        qc[t + 2] = u.z;
        qc[t + 3] = u.w;
    }
    if (qgain) qknorm_row<0, D>(qc, qgain[h], eps);
    rope_row<0, D>(qc, qr, cosT + i * D, sinT + i * D);
    const int64_t bh = b * Hkv + g;
    const float *KC = kc + bh * n * D;
    const float *KR = kr + bh * n * D;
    const float *VT = vt + bh * D * n;
    const int64_t s_end = ((int64_t)S < i + 1) ? (int64_t)S : i + 1;
    const int64_t w_beg = ((int64_t)S > i - W + 1) ? (int64_t)S : i - W + 1;
    const int c = min(max(cnt[bh * n + i], 0), kk);
    const int32_t *ix = idx + (bh * n + i) * kk;
    const int64_t nb = n / 64;
    float mx = -INFINITY;
    for (int64_t j = 0; j < s_end; ++j) mx = fmaxf(mx, dot_row<D>(qc, KC + j * D) * scale);
    for (int64_t j = w_beg; j <= i; ++j) mx = fmaxf(mx, dot_row<D>(qr, KR + j * D) * scale);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 0 || ix[r] >= nb) continue;
        int64_t j0 = (int64_t)ix[r] * 64;
        for (int64_t j = j0; j < j0 + 64; ++j) mx = fmaxf(mx, dot_row<D>(qc, KC + j * D) * scale);
    }
    float acc[D];
#pragma unroll
    for (int t = 0; t < D; ++t) acc[t] = 0.0f;
    float l = 0.0f;
    for (int64_t j = 0; j < s_end; ++j) {
        float p = expf(dot_row<D>(qc, KC + j * D) * scale - mx);
        l += p;
#pragma unroll
        for (int t = 0; t < D; ++t) acc[t] = fmaf(p, VT[(int64_t)t * n + j], acc[t]);
    }
    for (int64_t j = w_beg; j <= i; ++j) {
        float p = expf(dot_row<D>(qr, KR + j * D) * scale - mx);
        l += p;
#pragma unroll
        for (int t = 0; t < D; ++t) acc[t] = fmaf(p, VT[(int64_t)t * n + j], acc[t]);
    }
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 0 || ix[r] >= nb) continue;
        int64_t j0 = (int64_t)ix[r] * 64;
        for (int64_t j = j0; j < j0 + 64; ++j) {
            float p = expf(dot_row<D>(qc, KC + j * D) * scale - mx);
            l += p;
#pragma unroll
            for (int t = 0; t < D; ++t) acc[t] = fmaf(p, VT[(int64_t)t * n + j], acc[t]);
        }
    }
    float *orow = out + b * osb + i * osn + (int64_t)h * osh;
    float inv = 1.0f / l;
#pragma unroll
    for (int t = 0; t < D; ++t) orow[t] = acc[t] * inv;
}

// ------------------------------------------------------------ bf16 path ----
//
// One workgroup = 8 waves = one (batch, KV head) and a tile of QT queries.
// MFMA rows are (query, head) pairs: a 16-row tile holds QPT = 16/G
// consecutive queries x the G heads of the group (14 of 16 rows at G = 7), so
// every key tile -- window, sinks or a routed block -- updates ONE
// online-softmax state per row and nothing is merged at the end.
//   1. selection lists: each query's picks sorted ascending in LDS, and their
//      union over the tile (bitmap + compaction), ascending;
//   2. window: 64-key tiles of RoPE'd keys and V^T staged in LDS, shared by
//      all 8 waves (register-prefetched one tile ahead);
//   3. sinks + routed: the sink tile, then the union blocks in ascending
//      order, staged in LDS; a tile is computed for a block only if one of its
//      queries picked it, with the other queries' rows masked.  Each block is
//      read from HBM/L2 once per workgroup instead of once per query, and
//      workgroups walk blocks in the same order, which keeps the set of blocks
//      in flight on an XCD small enough for its L2.
// Softmax: when QKNorm bounds the logits (|q.k| * scale <= d gq gk scale,
// attention.py:74-81) and that bound is small enough that exp(-2 bound)
// cannot underflow, the bound itself is the softmax shift: no running max,
// no rescaling, additive partial sums (mathematically the same softmax).
// Otherwise a standard online max is kept per row.
// Scores are S^T = K . Q^T: the probabilities come out of the accumulators in
// the B-operand layout of the P.V MFMA (key rows permuted, perm_key).
template <int D>
struct AC2 {
    static constexpr int NKS = D / 32;                 // 32-wide d steps of QK^T
    static constexpr int NDT = D / 16;                 // 16-row d tiles of O^T
    static constexpr int WAVES = 8;
    static constexpr int NTHR = WAVES * 64;
    static constexpr int PTW = (D == 64) ? 4 : 2;      // max 16-row tiles per wave
    static constexpr int KROW = D + 8;                 // bf16 per LDS K row (padded)
    static constexpr int VROW = 64 + 8;                // bf16 per LDS V^T row (padded)
    static constexpr int TILE = 64 * KROW + D * VROW;  // bf16 of one staged K + V^T tile
    static constexpr int KCH = 64 * D / 8;             // 16-byte chunks of a K tile
    static constexpr int VCH = D * 8;                  // 16-byte chunks of a V^T tile
    static constexpr int NCH = (KCH + VCH) / NTHR;     // chunks per thread per tile
    static constexpr int NBLK = (D == 64) ? 2 : 1;     // routed blocks per LDS stage
};

constexpr int16_t SEL_SENT = 0x7fff;

__device__ __forceinline__ int perm_key(int mt, int r) {
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3);
}

template <int D>
__device__ __forceinline__ void tile_load_regs(const bf16_t *K, const bf16_t *VT, int64_t n,
                                               int64_t kb, u32x4v (&r)[AC2<D>::NCH]) {
    using C = AC2<D>;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
        const int idx = threadIdx.x + c * C::NTHR;
        if (idx < C::KCH) {
            const int key = idx / (D / 8), ch = idx % (D / 8);
            r[c] = *reinterpret_cast<const u32x4v *>(K + (kb + key) * D + 8 * ch);
        } else {
            const int c2 = idx - C::KCH;
            r[c] = *reinterpret_cast<const u32x4v *>(VT + (int64_t)(c2 >> 3) * n + kb + 8 * (c2 & 7));
        }
    }
}

template <int D>
__device__ __forceinline__ void tile_store_regs(bf16_t *T, const u32x4v (&r)[AC2<D>::NCH]) {
    using C = AC2<D>;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) {
        const int idx = threadIdx.x + c * C::NTHR;
        if (idx < C::KCH) {
            const int key = idx / (D / 8), ch = idx % (D / 8);
            *reinterpret_cast<u32x4v *>(T + key * C::KROW + 8 * ch) = r[c];
        } else {
            const int c2 = idx - C::KCH;
            *reinterpret_cast<u32x4v *>(T + 64 * C::KROW + (c2 >> 3) * C::VROW + 8 * (c2 & 7)) = r[c];
        }
    }
}

// Query operand of one lane's column (query i, head h) for S^T = K . Q^T:
// d = 32*ks + 8*lg + 0..7.  QKNorm in fp32 rounded to bf16 (attention.py:
// 88-94); with rope, apply_rope's rotation and bf16 roundings (:40-44).  The
// rotation partner d +- D/2 is in the same lane at ks +- NKS/2.  Invalid
// columns read a valid row and are zeroed (no divergence around shuffles).
template <int D>
__device__ __forceinline__ void build_qop(const bf16_t *q, int64_t qsb, int64_t qsn, int64_t qsh,
                                          const float *qgain, float eps, const float *cosT,
                                          const float *sinT, int64_t b, int64_t i, int h, bool valid,
                                          bool rope, int lg, bf16x8 (&qop)[AC2<D>::NKS]) {
    using C = AC2<D>;
    const int64_t ii = valid ? i : 0;
    const bf16_t *row = q + b * qsb + ii * qsn + (int64_t)h * qsh;
    float x[C::NKS][8];
    float ss = 0.0f;
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
        u32x4v u = *reinterpret_cast<const u32x4v *>(row + 32 * ks + 8 * lg);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[ks][2 * e] = __uint_as_float(u[e] << 16);
            x[ks][2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[ks][e], x[ks][e], ss);
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (qgain) {
        float ms = ss / (float)D;
        if (ms < eps) ms = eps;
        const float r = sqrtf(ms);
        const float gn = qgain[h];
#pragma unroll
        for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) x[ks][e] = rnd_bf16((x[ks][e] / r) * gn);
    }
#pragma unroll
    for (int ks = 0; ks < C::NKS; ++ks) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = x[ks][e];
            if (rope) {
                const int d = 32 * ks + 8 * lg + e;
                const float rot = (ks < C::NKS / 2) ? -x[ks + C::NKS / 2][e] : x[ks - C::NKS / 2][e];
                const float t1 = rnd_bf16(v * rnd_bf16(cosT[ii * D + d]));
                const float t2 = rnd_bf16(rot * rnd_bf16(sinT[ii * D + d]));
                v = rnd_bf16(t1 + t2);
            }
            y[e] = valid ? v : 0.0f;
        }
        qop[ks] = pack_b8(y);
    }
}

enum { MASK_NONE = 0, MASK_WIN = 1, MASK_SINK = 2, MASK_COL = 3 };

// One 64-key tile (K rows and V^T in LDS) against one 16-row tile.
// Element (mt, e) of this lane is key kb + 32(mt>>1) + 8lg + 4(mt&1) + e and
// column (query icol).  nmt: M-tiles that can hold valid keys (sinks).
template <int D>
__device__ __forceinline__ void tile_update(const bf16_t *Kl, const bf16_t *Vl,
                                            const bf16x8 (&qop)[AC2<D>::NKS],
                                            f32x4 (&O)[AC2<D>::NDT], float &mrun, float &lsum,
                                            int mode, int kb, int icol, bool colok, int S,
                                            int W, int nmt, bool fixed, float sl2, float bl2,
                                            int l16, int lg) {
    using C = AC2<D>;
    f32x4 Sa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (mt < nmt) {
            const bf16_t *kr = Kl + perm_key(mt, l16) * C::KROW + 8 * lg;
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks) Sa[mt] = mfma16(ld_b8(kr + 32 * ks), qop[ks], Sa[mt]);
        }
    }
    float pk[2][8];
    float shift;
    float alpha = 1.0f;
    if (fixed) {
        shift = bl2;
    } else {
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = kb + 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                bool ok = mt < nmt;
                if (mode == MASK_WIN) ok = ok && j >= S && j <= icol && j > icol - W;
                else if (mode == MASK_SINK) ok = ok && j < S && j <= icol;
                else if (mode == MASK_COL) ok = ok && colok;
                if (ok) tmax = fmaxf(tmax, Sa[mt][e]);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrun, tmax * sl2);
        shift = (mnew == -INFINITY) ? 0.0f : mnew;
        alpha = fast_exp2(mrun - shift);
        mrun = mnew;
    }
    float psum = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float p = fast_exp2(fmaf(Sa[mt][e], sl2, -shift));
            if (mode != MASK_NONE || mt >= nmt) {
                const int j = kb + 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                bool ok = mt < nmt;
                if (mode == MASK_WIN) ok = ok && j >= S && j <= icol && j > icol - W;
                else if (mode == MASK_SINK) ok = ok && j < S && j <= icol;
                else if (mode == MASK_COL) ok = ok && colok;
                p = ok ? p : 0.0f;
            }
            pk[mt >> 1][(mt & 1) * 4 + e] = p;
            psum += p;
        }
    lsum = lsum * alpha + psum;
    bf16x8 pb0, pb1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        pb0[e] = (__bf16)pk[0][e];
        pb1[e] = (__bf16)pk[1][e];
    }
    const int nkp = (nmt > 2) ? 2 : 1;
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt) {
        if (!fixed) O[dt] *= alpha;
        const bf16_t *vr = Vl + (16 * dt + l16) * C::VROW + 8 * lg;
        O[dt] = mfma16(ld_b8(vr), pb0, O[dt]);
        if (nkp > 1) O[dt] = mfma16(ld_b8(vr + 32), pb1, O[dt]);
    }
}

template <int D>
__global__ __launch_bounds__(512) void attn_bf16_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    const float *__restrict__ kgain, float eps, const bf16_t *__restrict__ kc,
    const bf16_t *__restrict__ kr, const bf16_t *__restrict__ vt, const float *__restrict__ cosT,
    const float *__restrict__ sinT, const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt,
    int64_t n, int B, int Hq, int Hkv, int S, int64_t W, int kk, float scale, int ptw, int ntiles,
    int xmap, bf16_t *__restrict__ out, int64_t osb, int64_t osn, int64_t osh) {
    using C = AC2<D>;
    extern __shared__ __align__(16) char smem[];
    __shared__ int nuni;
    const int G = Hq / Hkv;
    const int QPT = 16 / G;
    const int ROWS = QPT * G;
    const int QT = C::WAVES * ptw * QPT;
    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;

    // workgroup -> (batch*KV head, query tile); XCD-aware (workgroup i runs on
    // XCD i % 8): every XCD works on one KV head's keys at a time
    const int Cn = B * Hkv;
    int combo, tile;
    {
        const int i = blockIdx.x;
        if (xmap == 1) {
            combo = (i & 7) % Cn;
            tile = (i >> 3) * (8 / Cn) + (i & 7) / Cn;
        } else if (xmap == 2) {
            combo = (i / (8 * ntiles)) * 8 + (i & 7);
            tile = (i >> 3) % ntiles;
        } else {
            combo = i / ntiles;
            tile = i % ntiles;
        }
    }
    if (tile >= ntiles || combo >= Cn) return;
    const int b = combo / Hkv, g = combo % Hkv;
    const int64_t i0 = (int64_t)tile * QT;
    const int64_t bh = (int64_t)b * Hkv + g;
    const int64_t nb = n / 64;
    const int nbw = (int)((nb + 31) / 32);
    const bf16_t *KC = kc + bh * n * D;
    const bf16_t *KR = kr + bh * n * D;
    const bf16_t *VT = vt + bh * D * n;

    bf16_t *tiles = reinterpret_cast<bf16_t *>(smem);
    int16_t *sel = reinterpret_cast<int16_t *>(smem + (size_t)C::NBLK * C::TILE * 2);
    uint32_t *bitmap = reinterpret_cast<uint32_t *>(sel + ((QT * kk + 1) & ~1));
    int16_t *uni = reinterpret_cast<int16_t *>(bitmap + nbw);

    // the logit bound d * gq * gk * scale (per group); fixed softmax shift when
    // 2 * bound stays clear of fp32 underflow
    bool fixed = false;
    float bl2 = 0.0f;
    if (qgain && kgain) {
        float gq = 0.0f;
        for (int hh = 0; hh < G; ++hh) gq = fmaxf(gq, fabsf(qgain[g * G + hh]));
        const float bound = (float)D * gq * fabsf(kgain[g]) * scale * LOG2E_F;
        fixed = bound <= 60.0f;
        bl2 = bound;
    }
    const float sl2 = scale * LOG2E_F;

    // ---------------------------------------- selection lists and their union
    for (int e = tid; e < nbw; e += C::NTHR) bitmap[e] = 0u;
    __syncthreads();
    for (int qq = tid; qq < QT; qq += C::NTHR) {
        int16_t *sl = sel + qq * kk;
        const int64_t i = i0 + qq;
        int m2 = 0;
        if (i < n) {
            const int c = min(max(cnt[bh * n + i], 0), kk);
            const int32_t *ix = idx + (bh * n + i) * kk;
            for (int r = 0; r < c; ++r) {
                const int v = ix[r];
                if (v < 0 || v >= nb) continue;
                int p = m2++;
                while (p > 0 && sl[p - 1] > v) {
                    sl[p] = sl[p - 1];
                    --p;
                }
                sl[p] = (int16_t)v;
                atomicOr(&bitmap[v >> 5], 1u << (v & 31));
            }
        }
        for (int r = m2; r < kk; ++r) sl[r] = SEL_SENT;
    }
    __syncthreads();
    if (w == 0) {
        int base = 0;
        for (int w0 = 0; w0 < nbw; w0 += 64) {
            uint32_t word = (w0 + lane < nbw) ? bitmap[w0 + lane] : 0u;
            const int pc = __popc(word);
            int incl = pc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            int off = base + incl - pc;
            while (word) {
                const int bit = __ffs(word) - 1;
                uni[off++] = (int16_t)((w0 + lane) * 32 + bit);
                word &= word - 1u;
            }
            base += __shfl(incl, 63, 64);
        }
        if (lane == 0) nuni = base;
    }

    // ---------------------------------------------------- per-row state ------
    const int qs = l16 / G;
    const int hh = l16 % G;
    const bool colv = l16 < ROWS;
    bf16x8 qop[C::PTW][C::NKS];
    f32x4 O[C::PTW][C::NDT];
    float mrun[C::PTW], lsum[C::PTW];
    int icol[C::PTW];
    bool cok[C::PTW];
#pragma unroll
    for (int t = 0; t < C::PTW; ++t) {
        icol[t] = (int)i0 + (w * ptw + t) * QPT + qs;
        cok[t] = colv && t < ptw && (int64_t)icol[t] < n;
        mrun[t] = -INFINITY;
        lsum[t] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) O[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (t < ptw)
            build_qop<D>(q, qsb, qsn, qsh, qgain, eps, cosT, sinT, b, icol[t], g * G + hh, cok[t], true,
                         lg, qop[t]);
    }

    // ------------------------------------------------------- RoPE window -----
    const int64_t qhi = ((i0 + QT < n) ? i0 + QT : n) - 1;
    const int64_t wfirst = ((int64_t)S > i0 - W + 1) ? (int64_t)S : i0 - W + 1;
    const int64_t kt0 = (wfirst / 64) * 64;
    const int nwin = (wfirst <= qhi) ? (int)((qhi / 64) * 64 - kt0) / 64 + 1 : 0;
    {
        u32x4v pre[C::NCH];
        if (nwin > 0) tile_load_regs<D>(KR, VT, n, kt0, pre);
        for (int t = 0; t < nwin; ++t) {
            const int64_t kb = kt0 + 64 * (int64_t)t;
            __syncthreads();
            tile_store_regs<D>(tiles, pre);
            __syncthreads();
            if (t + 1 < nwin) tile_load_regs<D>(KR, VT, n, kb + 64, pre);
#pragma unroll
            for (int tt = 0; tt < C::PTW; ++tt) {
                if (tt >= ptw) break;
                const int64_t lo = i0 + (int64_t)(w * ptw + tt) * QPT;
                if (lo >= n) break;
                const int64_t hi = (lo + QPT - 1 < n) ? lo + QPT - 1 : n - 1;
                const int64_t wlo = ((int64_t)S > lo - W + 1) ? (int64_t)S : lo - W + 1;
                if (kb > hi || kb + 63 < wlo) continue;
                const bool full = kb >= S && kb + 63 <= lo && kb > hi - W;
                tile_update<D>(tiles, tiles + 64 * C::KROW, qop[tt], O[tt], mrun[tt], lsum[tt],
                               full ? MASK_NONE : MASK_WIN, (int)kb, icol[tt], cok[tt], S, (int)W, 4, fixed,
                               sl2, bl2, l16, lg);
            }
        }
    }

    // ------------------------------------------------ sinks + routed blocks --
#pragma unroll
    for (int t = 0; t < C::PTW; ++t)
        if (t < ptw)
            build_qop<D>(q, qsb, qsn, qsh, qgain, eps, cosT, sinT, b, icol[t], g * G + hh, cok[t], false,
                         lg, qop[t]);
    if (S > 0) {
        __syncthreads();
        u32x4v pre[C::NCH];
        tile_load_regs<D>(KC, VT, n, 0, pre);
        tile_store_regs<D>(tiles, pre);
        __syncthreads();
        const int nmt = (S <= 4) ? 1 : (S <= 32 ? 2 : 4);
#pragma unroll
        for (int tt = 0; tt < C::PTW; ++tt) {
            if (tt >= ptw) break;
            const int64_t lo = i0 + (int64_t)(w * ptw + tt) * QPT;
            if (lo >= n) break;
            tile_update<D>(tiles, tiles + 64 * C::KROW, qop[tt], O[tt], mrun[tt], lsum[tt], MASK_SINK, 0,
                           icol[tt], cok[tt], S, (int)W, nmt, fixed, sl2, bl2, l16, lg);
        }
    }
    {
        // cursor into each row's ascending selection list
        int cur[C::PTW], nxt[C::PTW];
#pragma unroll
        for (int t = 0; t < C::PTW; ++t) {
            cur[t] = 0;
            const int ql = (w * ptw + t) * QPT + qs;
            nxt[t] = (cok[t]) ? (int)sel[ql * kk] : (int)SEL_SENT;
        }
        __syncthreads();
        const int nu = nuni;
        for (int c0 = 0; c0 < nu; c0 += C::NBLK) {
            const int nc = (nu - c0 < C::NBLK) ? nu - c0 : C::NBLK;
            __syncthreads();
            for (int k = 0; k < nc; ++k) {
                u32x4v pre[C::NCH];
                tile_load_regs<D>(KC, VT, n, (int64_t)uni[c0 + k] * 64, pre);
                tile_store_regs<D>(tiles + k * C::TILE, pre);
            }
            __syncthreads();
            for (int k = 0; k < nc; ++k) {
                const int blk = uni[c0 + k];
                const bf16_t *Tk = tiles + k * C::TILE;
#pragma unroll
                for (int tt = 0; tt < C::PTW; ++tt) {
                    if (tt >= ptw) break;
                    const bool hit = nxt[tt] == blk;
                    if (__ballot(hit) == 0) continue;
                    tile_update<D>(Tk, Tk + 64 * C::KROW, qop[tt], O[tt], mrun[tt], lsum[tt], MASK_COL,
                                   blk * 64, icol[tt], hit, S, (int)W, 4, fixed, sl2, bl2, l16, lg);
                    if (hit) {
                        ++cur[tt];
                        const int ql = (w * ptw + tt) * QPT + qs;
                        nxt[tt] = (cur[tt] < kk) ? (int)sel[ql * kk + cur[tt]] : (int)SEL_SENT;
                    }
                }
            }
        }
    }

    // ------------------------------------------------------- normalise, store
#pragma unroll
    for (int t = 0; t < C::PTW; ++t) {
        if (t >= ptw) break;
        float l = lsum[t];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (!cok[t]) continue;
        const float inv = 1.0f / l;
        bf16_t *orow = out + (int64_t)b * osb + (int64_t)icol[t] * osn + (int64_t)(g * G + hh) * osh;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
            const int d0 = 16 * dt + 4 * lg;
            u32x2v u;
            u[0] = (uint32_t)f2bf(O[t][dt][0] * inv) | ((uint32_t)f2bf(O[t][dt][1] * inv) << 16);
            u[1] = (uint32_t)f2bf(O[t][dt][2] * inv) | ((uint32_t)f2bf(O[t][dt][3] * inv) << 16);
            *reinterpret_cast<u32x2v *>(orow + d0) = u;
        }
    }
}

}  // namespace hba

using namespace hba;

namespace {
template <int D>
int launch_attn_bf16(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                     const void *kc, const void *kr, const void *vt, const float *cosT,
                     const float *sinT, const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n,
                     int64_t Hq, int64_t Hkv, int64_t S, int64_t W, int64_t k, float scale, void *out,
                     const int64_t *os, hipStream_t s) {
    using C = AC2<D>;
    const int G = (int)(Hq / Hkv);
    if (G > 16 || n / 64 >= SEL_SENT) return HBA_ERR_UNSUPPORTED;
    const int QPT = 16 / G;
    const int64_t nb = n / 64;
    const int64_t nbw = (nb + 31) / 32;
    int ptw = C::PTW;
    size_t lds = 0;
    for (; ptw >= 1; --ptw) {
        const int64_t QT = (int64_t)C::WAVES * ptw * QPT;
        lds = (size_t)C::NBLK * C::TILE * 2 + (size_t)((QT * k + 1) & ~1LL) * 2 + (size_t)nbw * 4 +
              (size_t)nb * 2 + 16;
        if (lds <= 160 * 1024 - 64) break;
    }
    if (ptw < 1) return HBA_ERR_UNSUPPORTED;
    const int64_t QT = (int64_t)C::WAVES * ptw * QPT;
    const int64_t ntiles = (n + QT - 1) / QT;
    const int64_t Cn = B * Hkv;
    int xmap;
    int64_t grid;
    if (8 % Cn == 0) {
        xmap = 1;   // 8 workgroups per round, 8/Cn tiles of each combo per round
        grid = 8 * ((ntiles + (8 / Cn) - 1) / (8 / Cn));
    } else if (Cn % 8 == 0) {
        xmap = 2;
        grid = Cn * ntiles;
    } else {
        xmap = 0;
        grid = Cn * ntiles;
    }
    if (grid > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_bf16_kernel<D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return HBA_ERR_LAUNCH;
    hipLaunchKernelGGL(attn_bf16_kernel<D>, dim3((unsigned)grid), dim3(C::NTHR), lds, s,
                       (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, kgain, eps, (const bf16_t *)kc,
                       (const bf16_t *)kr, (const bf16_t *)vt, cosT, sinT, idx, cnt, n, (int)B, (int)Hq,
                       (int)Hkv, (int)S, W, (int)k, scale, ptw, (int)ntiles, xmap, (bf16_t *)out, os[0],
                       os[1], os[2]);
    return HBA_OK;
}

template <int D>
int launch_attn_f32(const void *q, const int64_t *qs, const float *qgain, float eps, const void *kc,
                    const void *kr, const void *vt, const float *cosT, const float *sinT,
                    const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n, int64_t Hq,
                    int64_t Hkv, int64_t S, int64_t W, int64_t k, float scale, void *out,
                    const int64_t *os, hipStream_t s) {
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)Hq, (unsigned)B);
    hipLaunchKernelGGL(attn_f32_kernel<D>, grid, dim3(64), 0, s, (const float *)q, qs[0], qs[1], qs[2],
                       qgain, eps, (const float *)kc, (const float *)kr, (const float *)vt, cosT, sinT,
                       idx, cnt, n, (int)Hq, (int)Hkv, (int)S, W, (int)k, scale, (float *)out, os[0],
                       os[1], os[2]);
    return HBA_OK;
}
}  // namespace

extern "C" int hba_attn_fwd(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
                            const float *k_gain, float eps, const void *kc, const void *kr, const void *vt,
                            const float *cos_tab, const float *sin_tab, const int32_t *idx,
                            const int32_t *cnt, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                            int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t k, float scale,
                            void *out, const int64_t out_strides[3], void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !q_strides || !kc || !kr || !vt || !cos_tab || !sin_tab || !idx || !cnt || !out ||
        !out_strides)
        return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || W < 1 || S < 0 || k < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0 || S > Bk) return HBA_ERR_INVALID_ARG;
    if (!abi::rows_aligned(dtype, q, q_strides) || !abi::rows_aligned(dtype, out, out_strides) ||
        !abi::aligned16(kc) || !abi::aligned16(kr) || !abi::aligned16(vt))
        return HBA_ERR_UNSUPPORTED;
    if (B > 65535 || Hq > 65535) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    if (dtype == HBA_DTYPE_BF16)
        st = (d == 64) ? launch_attn_bf16<64>(q, q_strides, q_gain, k_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                              idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides, s)
                       : launch_attn_bf16<128>(q, q_strides, q_gain, k_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                               idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out,
                                               out_strides, s);
    else
        st = (d == 64) ? launch_attn_f32<64>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                             idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides, s)
                       : launch_attn_f32<128>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                              idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out,
                                              out_strides, s);
    if (st) return st;
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
