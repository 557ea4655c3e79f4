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
template <int D>
struct ACfg {
    static constexpr int QT = (D == 64) ? 64 : 32;  // queries per workgroup
    static constexpr int NQT = QT / 16;             // 16-query column tiles per wave (phase A)
    static constexpr int NKS = D / 32;              // 32-wide d steps of the QK^T MFMA
    static constexpr int NDT = D / 16;              // 16-row d tiles of O^T
    static constexpr int KROW = D + 8;              // LDS row of the K tile (bf16, padded)
    static constexpr int VROW = 64 + 8;             // LDS row of the V^T tile (bf16, padded)
    static constexpr int PROW = D + 2;              // LDS row of a phase-B partial (fp32)
    static size_t lds_bytes(int G) {
        return (size_t)QT * G * PROW * 4 + (size_t)64 * KROW * 2 + (size_t)D * VROW * 2;
    }
};

// Row r of M-tile mt (16 keys) of a 64-key tile holds key perm_key(mt, r):
// then the C-layout rows 4*lg..4*lg+3 of M-tiles 2kp and 2kp+1 are keys
// 32kp + 8lg + 0..7, exactly the k-slice lane group lg owns in the B operand
// of the P.V MFMA for k-step kp.
__device__ __forceinline__ int perm_key(int mt, int r) {
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3);
}

// Phase-A query operands of one head for the QT queries of the tile: lane
// (l16, lg) holds query 16*qt + l16, d = 32*ks + 8*lg + 0..7 (B operand of
// S^T = K . Q^T).  QKNorm in fp32, rounded to bf16 (attention.py:88-94); with
// rope, the NeoX rotation at the query's position with apply_rope's bf16
// roundings (attention.py:40-44).  The rotation partner d +- D/2 sits in the
// same lane at k-step ks +- NKS/2.
template <int D>
__device__ __forceinline__ void phaseA_query(const bf16_t *q, int64_t qsb, int64_t qsn, int64_t qsh,
                                             const float *qgain, float eps, const float *cosT,
                                             const float *sinT, int64_t b, int64_t i0, int h, int l16,
                                             int lg, bool rope,
                                             bf16x8 (&qa)[ACfg<D>::NQT][ACfg<D>::NKS]) {
    using C = ACfg<D>;
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt) {
        const int64_t i = i0 + 16 * qt + l16;
        const bf16_t *qrow = q + b * qsb + i * qsn + (int64_t)h * qsh;
        float x[C::NKS][8];
        float ss = 0.0f;
#pragma unroll
        for (int ks = 0; ks < C::NKS; ++ks) {
            u32x4v u = *reinterpret_cast<const u32x4v *>(qrow + 32 * ks + 8 * lg);
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
            float r = sqrtf(ms);
            float gn = qgain[h];
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) x[ks][e] = rnd_bf16((x[ks][e] / r) * gn);
        }
        if (rope) {
            const float *cs = cosT + i * D;
            const float *sn = sinT + i * D;
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks) {
                float y[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = 32 * ks + 8 * lg + e;
                    const float rot = (ks < C::NKS / 2) ? -x[ks + C::NKS / 2][e] : x[ks - C::NKS / 2][e];
                    const float t1 = rnd_bf16(x[ks][e] * rnd_bf16(cs[d]));
                    const float t2 = rnd_bf16(rot * rnd_bf16(sn[d]));
                    y[e] = rnd_bf16(t1 + t2);
                }
                qa[qt][ks] = pack_b8(y);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks) qa[qt][ks] = pack_b8(x[ks]);
        }
    }
}

template <int D>
__global__ __launch_bounds__(512) void attn_bf16_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const bf16_t *__restrict__ kc, const bf16_t *__restrict__ kr,
    const bf16_t *__restrict__ vt, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, int64_t n, int Hq, int Hkv, int S,
    int64_t W, int kk, float sl2, bf16_t *__restrict__ out, int64_t osb, int64_t osn, int64_t osh) {
    using C = ACfg<D>;
    extern __shared__ __align__(16) char smem[];
    const int G = Hq / Hkv;
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15;
    const int lg = lane >> 4;
    const int nthr = G * 64;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t i0 = (int64_t)blockIdx.x * C::QT;
    const int64_t bh = b * Hkv + g;
    float *P = reinterpret_cast<float *>(smem);
    bf16_t *Kt = reinterpret_cast<bf16_t *>(smem + (size_t)C::QT * G * C::PROW * 4);
    bf16_t *Vs = Kt + 64 * C::KROW;
    const bf16_t *KC = kc + bh * n * D;
    const bf16_t *KR = kr + bh * n * D;
    const bf16_t *VT = vt + bh * D * n;

    // ------------------------------------------------ phase B: routed keys --
    for (int qq = w; qq < C::QT; qq += G) {
        const int64_t i = i0 + qq;
        const int c = min(max(cnt[bh * n + i], 0), kk);
        float *Ph = P + ((size_t)qq * G + l16) * C::PROW;
        if (c == 0) {
            if (l16 < G) {
#pragma unroll
                for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) Ph[16 * dt + 4 * lg + e] = 0.0f;
                if (lg == 0) {
                    Ph[D] = -INFINITY;
                    Ph[D + 1] = 0.0f;
                }
            }
            continue;
        }
        bf16x8 qb[C::NKS];
        {
            const bool hv = l16 < G;
            const bf16_t *qrow = q + b * qsb + i * qsn + (int64_t)(g * G + (hv ? l16 : 0)) * qsh;
            float x[C::NKS][8];
            float ss = 0.0f;
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks) {
                u32x4v u = *reinterpret_cast<const u32x4v *>(qrow + 32 * ks + 8 * lg);
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
                float r = sqrtf(ms);
                float gn = qgain[g * G + (hv ? l16 : 0)];
#pragma unroll
                for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[ks][e] = rnd_bf16((x[ks][e] / r) * gn);
            }
#pragma unroll
            for (int ks = 0; ks < C::NKS; ++ks) {
                if (!hv)
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[ks][e] = 0.0f;
                qb[ks] = pack_b8(x[ks]);
            }
        }
        f32x4 O[C::NDT];
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        float mrun = -INFINITY, lrun = 0.0f;
        const int32_t *ix = idx + (bh * n + i) * kk;
        for (int r = 0; r < c; ++r) {
            const int32_t blk = ix[r];
            if (blk < 0 || (int64_t)blk >= n / 64) continue;   // never read outside the keys
            const int64_t base = (int64_t)blk * 64;
            f32x4 Sa[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int64_t key = base + perm_key(mt, l16);
                Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < C::NKS; ++ks)
                    Sa[mt] = mfma16(ld_b8(KC + key * D + 32 * ks + 8 * lg), qb[ks], Sa[mt]);
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    Sa[mt][e] *= sl2;
                    tmax = fmaxf(tmax, Sa[mt][e]);
                }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(mrun, tmax);
            const float alpha = fast_exp2(mrun - mnew);
            float pk[2][8];
            float psum = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float p = rnd_bf16(fast_exp2(Sa[mt][e] - mnew));
                    pk[mt >> 1][(mt & 1) * 4 + e] = p;
                    psum += p;
                }
            psum += __shfl_xor(psum, 16, 64);
            psum += __shfl_xor(psum, 32, 64);
            lrun = lrun * alpha + psum;
            mrun = mnew;
            bf16x8 pb0 = pack_b8(pk[0]);
            bf16x8 pb1 = pack_b8(pk[1]);
#pragma unroll
            for (int dt = 0; dt < C::NDT; ++dt) {
                O[dt] *= alpha;
                const bf16_t *vrow = VT + (int64_t)(16 * dt + l16) * n + base + 8 * lg;
                O[dt] = mfma16(ld_b8(vrow), pb0, O[dt]);
                O[dt] = mfma16(ld_b8(vrow + 32), pb1, O[dt]);
            }
        }
        if (l16 < G) {
#pragma unroll
            for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
                for (int e = 0; e < 4; ++e) Ph[16 * dt + 4 * lg + e] = O[dt][e];
            if (lg == 0) {
                Ph[D] = mrun;
                Ph[D + 1] = lrun;
            }
        }
    }

    // ----------------------------------------- phase A: sinks + RoPE window --
    const int hh = w;
    const int h = g * G + hh;
    bf16x8 qa[C::NQT][C::NKS];
    phaseA_query<D>(q, qsb, qsn, qsh, qgain, eps, cosT, sinT, b, i0, h, l16, lg, false, qa);
    f32x4 O[C::NDT][C::NQT];
    float mrun[C::NQT], lrun[C::NQT];
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt) {
        mrun[qt] = -INFINITY;
        lrun[qt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) O[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int64_t wfirst = ((int64_t)S > i0 - W + 1) ? (int64_t)S : i0 - W + 1;
    const int64_t qlast = i0 + C::QT - 1;
    const int64_t kt0 = (wfirst / 64) * 64;
    const int nwin = (wfirst <= qlast) ? (int)((qlast / 64) * 64 - kt0) / 64 + 1 : 0;
    constexpr int KCH = 64 * D / 8;   // 16-byte chunks of the K tile
    constexpr int VCH = D * 8;        // 16-byte chunks of the V^T tile
    for (int t = 0; t <= nwin; ++t) {
        const bool sink = (t == 0);
        const int64_t kbase = sink ? 0 : kt0 + (int64_t)(t - 1) * 64;
        const bf16_t *Ksrc = sink ? KC : KR;
        __syncthreads();
        for (int cidx = threadIdx.x; cidx < KCH + VCH; cidx += nthr) {
            if (cidx < KCH) {
                const int key = cidx / (D / 8), ch = cidx % (D / 8);
                *reinterpret_cast<u32x4v *>(Kt + key * C::KROW + 8 * ch) =
                    *reinterpret_cast<const u32x4v *>(Ksrc + (kbase + key) * D + 8 * ch);
            } else {
                const int c2 = cidx - KCH;
                const int dd = c2 >> 3, ch = c2 & 7;
                *reinterpret_cast<u32x4v *>(Vs + dd * C::VROW + 8 * ch) =
                    *reinterpret_cast<const u32x4v *>(VT + (int64_t)dd * n + kbase + 8 * ch);
            }
        }
        __syncthreads();
#pragma unroll
        for (int qt = 0; qt < C::NQT; ++qt) {
            const int64_t i = i0 + 16 * qt + l16;
            f32x4 Sa[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int krow = perm_key(mt, l16);
                Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < C::NKS; ++ks)
                    Sa[mt] = mfma16(ld_b8(Kt + krow * C::KROW + 32 * ks + 8 * lg), qa[qt][ks], Sa[mt]);
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t j = kbase + 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                    const bool ok = sink ? (j < S && j <= i) : (j >= S && j <= i && j > i - W);
                    Sa[mt][e] = ok ? Sa[mt][e] * sl2 : -INFINITY;
                    tmax = fmaxf(tmax, Sa[mt][e]);
                }
            tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(mrun[qt], tmax);
            const float muse = (mnew == -INFINITY) ? 0.0f : mnew;
            const float alpha = fast_exp2(mrun[qt] - muse);
            float pk[2][8];
            float psum = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float p = rnd_bf16(fast_exp2(Sa[mt][e] - muse));
                    pk[mt >> 1][(mt & 1) * 4 + e] = p;
                    psum += p;
                }
            psum += __shfl_xor(psum, 16, 64);
            psum += __shfl_xor(psum, 32, 64);
            lrun[qt] = lrun[qt] * alpha + psum;
            mrun[qt] = mnew;
            bf16x8 pb0 = pack_b8(pk[0]);
            bf16x8 pb1 = pack_b8(pk[1]);
#pragma unroll
            for (int dt = 0; dt < C::NDT; ++dt) {
                O[dt][qt] *= alpha;
                const bf16_t *vrow = Vs + (16 * dt + l16) * C::VROW + 8 * lg;
                O[dt][qt] = mfma16(ld_b8(vrow), pb0, O[dt][qt]);
                O[dt][qt] = mfma16(ld_b8(vrow + 32), pb1, O[dt][qt]);
            }
        }
        if (sink)  // switch the query operand to its RoPE rotation
            phaseA_query<D>(q, qsb, qsn, qsh, qgain, eps, cosT, sinT, b, i0, h, l16, lg, true, qa);
    }

    // ---------------------------------------------------- merge and store --
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt) {
        const int qq = 16 * qt + l16;
        const int64_t i = i0 + qq;
        const float *Ph = P + ((size_t)qq * G + hh) * C::PROW;
        const float mB = Ph[D], lB = Ph[D + 1];
        const float mA = mrun[qt], lA = lrun[qt];
        const float m = fmaxf(mA, mB);
        const float wA = fast_exp2(mA - m);
        const float wB = fast_exp2(mB - m);
        const float inv = 1.0f / (lA * wA + lB * wB);
        bf16_t *orow = out + b * osb + i * osn + (int64_t)h * osh;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
            const int d0 = 16 * dt + 4 * lg;
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (O[dt][qt][e] * wA + Ph[d0 + e] * wB) * inv;
            u32x2v u;
            u[0] = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
            u[1] = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
            *reinterpret_cast<u32x2v *>(orow + d0) = u;
        }
    }
}

}  // namespace hba

using namespace hba;

namespace {
template <int D>
int launch_attn_bf16(const void *q, const int64_t *qs, const float *qgain, float eps, const void *kc,
                     const void *kr, const void *vt, const float *cosT, const float *sinT,
                     const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n, int64_t Hq,
                     int64_t Hkv, int64_t S, int64_t W, int64_t k, float scale, void *out,
                     const int64_t *os, hipStream_t s) {
    using C = ACfg<D>;
    const int G = (int)(Hq / Hkv);
    if (G > 8) return HBA_ERR_UNSUPPORTED;
    size_t lds = C::lds_bytes(G);
    if (lds > 160 * 1024) return HBA_ERR_UNSUPPORTED;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_bf16_kernel<D>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return HBA_ERR_LAUNCH;
    dim3 grid((unsigned)(n / C::QT), (unsigned)Hkv, (unsigned)B);
    hipLaunchKernelGGL(attn_bf16_kernel<D>, grid, dim3(G * 64), lds, s, (const bf16_t *)q, qs[0], qs[1],
                       qs[2], qgain, eps, (const bf16_t *)kc, (const bf16_t *)kr, (const bf16_t *)vt,
                       cosT, sinT, idx, cnt, n, (int)Hq, (int)Hkv, (int)S, W, (int)k,
                       scale * LOG2E_F, (bf16_t *)out, os[0], os[1], os[2]);
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
                            float eps, const void *kc, const void *kr, const void *vt,
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
        st = (d == 64) ? launch_attn_bf16<64>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                              idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides, s)
                       : launch_attn_bf16<128>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
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
