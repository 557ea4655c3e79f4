// The summarizer auxiliary loss (aux-KL) and its gradient into the slot
// summarizer's probes and projection (hba_attention_dense
// src/hba/attention.py:366-389; the chunked teacher of the fused path
// :478-549).
//
//   aux = -mean over (batch, KV head g, query i with a candidate block) of
//         sum_b p*_b log softmax_b(bsc)      (terms with p*_b = 0 dropped)
//   bsc[i, b] = max over slots of (grouped query . S0[b, slot]) * scale_r
//   p*[i, b]  = mean over the G heads of g of softmax_b(LSE of head h's
//               content logits over the 64 keys of block b), renormalised;
//               both softmaxes run over the candidate blocks of i only.
//
// Gradients reach only probes and proj (routing runs on detached q/k, the
// teacher under no_grad): d aux / d bsc = (softmax(bsc) * sum p* - p*) / N,
// the slot max passes it evenly to tied slots, and the summariser is
// differentiated by hand.
//
// Launches, in order (one stream, no host synchronisation):
//   aux_qc      content queries qc = QKNorm(q) rounded to the storage type
//   aux_scores  grouped queries qg (fp32) and bsc with the tied-slot masks
//   aux_teacher per (query, head, candidate block) the block LSE of the
//               content logits, on MFMA (16 keys x 16 (query, head) columns;
//               bf16: 16 waves share each staged key block)
//   aux_rows    per (query, KV head): p*, the row's KL term, d aux / d bsc
//   aux_sum     aux = -(sum of row terms) / N, one workgroup, fixed order
//   aux_dsum    d aux / d S0 = sum over queries of d bsc * tie share * qg
//               (query segments, partials summed in order by aux_gsum)
//   aux_sbwd    per block: the summariser's backward into per-block partial
//               d probes / d proj
//   aux_gsum    partials summed over blocks in a fixed order
// Every reduction runs in a fixed order: the results are deterministic.
#include "hba_common.h"
#include "hba_abi.h"
#include "hba_generic.h"

namespace hba {
namespace aux {

constexpr int BK = 64;

constexpr int QS = 8;           // query segments of aux_dsum (partials summed in order)

struct Ws {
    size_t qc, qg, bsc, ties, L, rowt, dS0, pdS0, pproj, pprb, total;
};

inline size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

inline Ws layout(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m) {
    const int64_t nb = n / BK, G = Hq / Hkv;
    Ws w;
    size_t o = 0;
    w.qc = o;    o += up256((size_t)B * n * Hq * d * (dtype == HBA_DTYPE_BF16 ? 2 : 4));
    w.qg = o;    o += up256((size_t)B * Hkv * n * d * 4);
    w.bsc = o;   o += up256((size_t)B * Hkv * n * nb * 4);
    w.ties = o;  o += up256((size_t)B * Hkv * n * nb);
    w.L = o;     o += up256((size_t)B * Hkv * n * G * nb * 4);
    w.rowt = o;  o += up256((size_t)B * Hkv * n * 4);
    w.dS0 = o;   o += up256((size_t)B * Hkv * nb * m * d * 4);
    w.pdS0 = o;  o += up256((size_t)QS * B * Hkv * nb * m * d * 4);
    w.pproj = o; o += up256((size_t)B * nb * Hkv * d * d * 4);
    w.pprb = o;  o += up256((size_t)B * nb * Hkv * m * d * 4);
    w.total = o;
    return w;
}

// First query with a candidate block: cand_bmax(i) >= 1 <=> i >= 2*BK + W - 1.
__host__ __device__ inline int64_t first_valid(int64_t W) { return 2 * BK + W - 1; }

// ------------------------------------------------------------------ qc -----
template <int DT, int D>
__global__ __launch_bounds__(256) void aux_qc_kernel(const typename St<DT>::T *__restrict__ q, int64_t sb,
                                                     int64_t sn, int64_t sh, const float *__restrict__ qgain,
                                                     float eps, int64_t B, int64_t n, int64_t Hq,
                                                     typename St<DT>::T *__restrict__ qc) {
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= B * n * Hq) return;
    const int64_t h = r % Hq, i = (r / Hq) % n, b = r / (Hq * n);
    const typename St<DT>::T *src = q + b * sb + i * sn + h * sh;
    float x[D];
#pragma unroll
    for (int t = 0; t < D; ++t) x[t] = St<DT>::ld(src, t);
    if (qgain) qknorm_row<DT, D>(x, qgain[h], eps);
#pragma unroll
    for (int t = 0; t < D; ++t) St<DT>::st(qc, r * D + t, x[t]);
}

// -------------------------------------------------------------- scores -----
// Workgroup = (64 queries, KV head g, batch b).  qg rows (the G heads summed
// in head order, rounded to the storage type, as grouped_query) go to LDS and
// to the qg buffer; the summaries of CB blocks at a time are staged in LDS;
// thread (query, block) takes the slot max of the fp32 dot products and the
// mask of the slots that reach it.
template <int DT, int D>
__global__ __launch_bounds__(256) void aux_scores_kernel(const typename St<DT>::T *__restrict__ qc,
                                                         const typename St<DT>::T *__restrict__ S0, int64_t n,
                                                         int64_t Hq, int64_t Hkv, int m, int64_t W, float scale_r,
                                                         float *__restrict__ qg_out, float *__restrict__ bsc,
                                                         uint8_t *__restrict__ ties) {
    constexpr int CB = (D == 64) ? 8 : 4;   // summary blocks staged per step (LDS under 64 KB)
    __shared__ float qgs[64][D + 1];
    __shared__ float s0[CB][8][D];
    const int tid = threadIdx.x;
    const int64_t i0 = (int64_t)blockIdx.x * 64, g = blockIdx.y, b = blockIdx.z;
    const int64_t G = Hq / Hkv, nb = n / BK;
    for (int e = tid; e < 64 * D; e += 256) {
        const int qi = e / D, t = e % D;
        const int64_t i = i0 + qi;
        float s = 0.0f;
        if (i < n) {
            const typename St<DT>::T *row = qc + ((b * n + i) * Hq + g * G) * D + t;
            s = St<DT>::ld(row, 0);
            for (int64_t h = 1; h < G; ++h) s = s + St<DT>::ld(row, h * D);
            s = St<DT>::rnd(s);
            qg_out[((b * Hkv + g) * n + i) * D + t] = s;
        }
        qgs[qi][t] = s;
    }
    const int64_t ilast = (i0 + 63 < n) ? i0 + 63 : n - 1;
    const int64_t bmax = cand_bmax(ilast, BK, W);
    const typename St<DT>::T *sg = S0 + (b * Hkv + g) * nb * m * D;
    for (int64_t c0 = 1; c0 <= bmax; c0 += CB) {
        __syncthreads();   // qgs written / the previous chunk is used
        for (int e = tid; e < CB * m * D; e += 256) {
            const int cb = e / (m * D), rem = e % (m * D);
            const int64_t c = c0 + cb;
            s0[cb][rem / D][rem % D] = (c <= bmax) ? St<DT>::ld(sg, c * m * D + rem) : 0.0f;
        }
        __syncthreads();
        for (int e = tid; e < 64 * CB; e += 256) {
            const int qi = e % 64, cb = e / 64;
            const int64_t i = i0 + qi, c = c0 + cb;
            if (i >= n || c > cand_bmax(i, BK, W)) continue;
            float best = -INFINITY;
            uint32_t mask = 0;
            for (int sl = 0; sl < m; ++sl) {
                float acc = 0.0f;
#pragma unroll 16
                for (int t = 0; t < D; ++t) acc = fmaf(qgs[qi][t], s0[cb][sl][t], acc);
                if (acc > best) {
                    best = acc;
                    mask = 1u << sl;
                } else if (acc == best) {
                    mask |= 1u << sl;
                }
            }
            const int64_t o = ((b * Hkv + g) * n + i) * nb + c;
            bsc[o] = best * scale_r;
            ties[o] = (uint8_t)mask;
        }
    }
}

// The same block scores for bf16 storage and m = 4 on MFMA: per (batch, KV
// head, 64 queries) the GEMM C^T[summary rows x queries] = S0 . qg^T with
// v_mfma_f32_16x16x32_bf16.  qg and S0 are bf16-exact, so every product is
// exact in fp32 and only the order of the fp32 sums differs from the
// sequential chain (scores within a few fp32 ulps).  A 16-row M tile is 4
// blocks x 4 slots: lane (l16, lg) receives the 4 slot scores of one block
// for one query, so the slot max and the tie mask come from registers.  The
// four waves take 16-block stages w, w + 4, ... and load their A fragments
// from L2 a stage ahead (d = 64: two stages in flight; d = 128: one stage's
// buffers refilled M-tile by M-tile, for registers).
typedef __bf16 abf16x8 __attribute__((ext_vector_type(8)));
typedef float af32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int au32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ abf16x8 a_ldb8(const bf16_t *p) {
    return __builtin_bit_cast(abf16x8, *reinterpret_cast<const au32x4 *>(p));
}
template <int D>
__global__ __launch_bounds__(256, 2) void aux_scores_mfma_kernel(const bf16_t *__restrict__ qc,
                                                                 const bf16_t *__restrict__ S0, int64_t n,
                                                                 int64_t Hq, int64_t Hkv, int64_t W, float scale_r,
                                                                 float *__restrict__ qg_out,
                                                                 float *__restrict__ bsc,
                                                                 uint8_t *__restrict__ ties) {
    constexpr int NKS = D / 32, NCT = 4, CB = 16, ROWQ = D + 8;
    __shared__ __align__(16) bf16_t qgs[64 * ROWQ];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int64_t i0 = (int64_t)blockIdx.x * 64, g = blockIdx.y, b = blockIdx.z;
    const int64_t G = Hq / Hkv, nb = n / BK;
    const int64_t bh = b * Hkv + g;
    // the grouped queries: the head sum in head order, rounded (as aux_scores_kernel)
    for (int e = tid; e < 64 * D; e += 256) {
        const int qi = e / D, t = e % D;
        const int64_t i = i0 + qi;
        float s = 0.0f;
        if (i < n) {
            const bf16_t *row = qc + ((b * n + i) * Hq + g * G) * D + t;
            s = bf2f(row[0]);
            for (int64_t h = 1; h < G; ++h) s = s + bf2f(row[h * D]);
            s = rnd_bf16(s);
            qg_out[(bh * n + i) * D + t] = s;
        }
        qgs[qi * ROWQ + t] = f2bf(s);
    }
    __syncthreads();
    abf16x8 qb[NCT][NKS];
    int64_t bm[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qb[ct][ks] = a_ldb8(qgs + (16 * ct + l16) * ROWQ + 32 * ks + 8 * lg);
        const int64_t i = i0 + 16 * ct + l16;
        bm[ct] = (i < n) ? cand_bmax(i, BK, W) : 0;
    }
    const int64_t ilast = (i0 + 63 < n) ? i0 + 63 : n - 1;
    const int64_t tile_bmax = cand_bmax(ilast, BK, W);
    const int nst = (tile_bmax > 0) ? (int)((tile_bmax + CB - 1) / CB) : 0;
    const bf16_t *Sg = S0 + bh * nb * 4 * D;
    auto load_mt = [&](int st, int mt, abf16x8 (&af)[NKS]) {
        int64_t blk = 1 + (int64_t)st * CB + 4 * mt + (l16 >> 2);
        blk = (blk <= tile_bmax) ? blk : tile_bmax;
        const bf16_t *src = Sg + (blk * 4 + (l16 & 3)) * D + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) af[ks] = a_ldb8(src + 32 * ks);
    };
    auto stage = [&](int st, abf16x8 (&af)[4][NKS], int nxt) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            af32x4 acc[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) acc[ct] = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct)
                    acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][ks], qb[ct][ks], acc[ct], 0, 0, 0);
            if (D > 64 && nxt >= 0) load_mt(nxt, mt, af[mt]);   // wave-uniform
            const int64_t c = 1 + (int64_t)st * CB + 4 * mt + lg;
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const int64_t i = i0 + 16 * ct + l16;
                if (i >= n || c > bm[ct]) continue;
                float best = -INFINITY;
                uint32_t mask = 0;
#pragma unroll
                for (int sl = 0; sl < 4; ++sl) {
                    const float v = acc[ct][sl];
                    if (v > best) {
                        best = v;
                        mask = 1u << sl;
                    } else if (v == best) {
                        mask |= 1u << sl;
                    }
                }
                const int64_t o = (bh * n + i) * nb + c;
                bsc[o] = best * scale_r;
                ties[o] = (uint8_t)mask;
            }
        }
    };
    auto load = [&](int st, abf16x8 (&af)[4][NKS]) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) load_mt(st, mt, af[mt]);
    };
    if constexpr (D > 64) {
        abf16x8 a0[4][NKS];
        int st = w;
        if (st < nst) load(st, a0);
        while (st < nst) {
            stage(st, a0, (st + 4 < nst) ? st + 4 : -1);
            st += 4;
        }
    } else {
        abf16x8 a0[4][NKS], a1[4][NKS];
        int st = w;
        if (st < nst) load(st, a0);
        if (st + 4 < nst) load(st + 4, a1);
        while (st < nst) {
            stage(st, a0, -1);
            if (st + 8 < nst) load(st + 8, a0);
            st += 4;
            if (st >= nst) break;
            stage(st, a1, -1);
            if (st + 8 < nst) load(st + 8, a1);
            st += 4;
        }
    }
}

// ------------------------------------------------------------- teacher -----
// Each wave owns 16 columns: QPW = 16/G queries x the G heads of KV head g
// (column c -> query i0w + c/G, head g*G + c%G; columns past QPW*G idle).
// For every candidate block of its last query it forms S^T = K_blk . Q^T as
// four 16-key M-tiles, and per column the LSE over the block's 64 keys of the
// content logits (scale_u); it writes the LSE of each (query, head, block)
// that is a candidate.  Waves are independent (no LDS, no barriers).
__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int DT, int D>
__global__ __launch_bounds__(256) void aux_teacher_kernel(const typename St<DT>::T *__restrict__ qc,
                                                          const typename St<DT>::T *__restrict__ kc, int64_t n,
                                                          int64_t Hq, int64_t Hkv, int64_t W, float scale_u,
                                                          float *__restrict__ L) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t g = blockIdx.y, b = blockIdx.z;
    const int G = (int)(Hq / Hkv), QPW = 16 / G;
    const int64_t nb = n / BK;
    const int64_t i0w = ((int64_t)blockIdx.x * 4 + w) * QPW;
    if (i0w >= n) return;
    const int cq = l16 / G, ch = l16 % G;
    const int64_t iq = i0w + cq;
    const bool col_ok = l16 < QPW * G && iq < n;
    const int64_t ic = col_ok ? iq : i0w;
    const int64_t col_bmax = col_ok ? cand_bmax(iq, BK, W) : 0;
    const int64_t ilast = (i0w + QPW - 1 < n) ? i0w + QPW - 1 : n - 1;
    const int64_t bmax = cand_bmax(ilast, BK, W);
    const typename St<DT>::T *qrow = qc + ((b * n + ic) * Hq + g * G + ch) * D;
    const typename St<DT>::T *kg = kc + (b * Hkv + g) * n * D;
    float *Lrow = L + (((b * Hkv + g) * n + ic) * G + ch) * nb;
    if constexpr (DT == 1) {
        constexpr int NKS = D / 32;
        bf16x8 qop[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const uint4 u = col_ok ? *reinterpret_cast<const uint4 *>(qrow + 32 * ks + 8 * lg) : make_uint4(0, 0, 0, 0);
            qop[ks] = __builtin_bit_cast(bf16x8, u);
        }
        for (int64_t c = 1; c <= bmax; ++c) {
            f32x4 acc[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const typename St<DT>::T *krow = kg + (c * BK + mt * 16 + l16) * D + 8 * lg;
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    const uint4 u = *reinterpret_cast<const uint4 *>(krow + 32 * ks);
                    acc[mt] = mfma_bf16(__builtin_bit_cast(bf16x8, u), qop[ks], acc[mt]);
                }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, acc[mt][r] * scale_u);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            float se = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) se += expf(acc[mt][r] * scale_u - mx);
            se += __shfl_xor(se, 16, 64);
            se += __shfl_xor(se, 32, 64);
            if (lg == 0 && col_ok && c <= col_bmax) Lrow[c] = mx + logf(se);
        }
    } else {
        constexpr int NK4 = D / 4;
        float qop[NK4];
#pragma unroll
        for (int ks = 0; ks < NK4; ++ks) qop[ks] = col_ok ? St<DT>::ld(qrow, 4 * ks + lg) : 0.0f;
        for (int64_t c = 1; c <= bmax; ++c) {
            f32x4 acc[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const typename St<DT>::T *krow = kg + (c * BK + mt * 16 + l16) * D + lg;
#pragma unroll
                for (int ks = 0; ks < NK4; ++ks)
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(St<DT>::ld(krow, 4 * ks), qop[ks], acc[mt], 0,
                                                                   0, 0);
            }
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, acc[mt][r] * scale_u);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            float se = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) se += expf(acc[mt][r] * scale_u - mx);
            se += __shfl_xor(se, 16, 64);
            se += __shfl_xor(se, 32, 64);
            if (lg == 0 && col_ok && c <= col_bmax) Lrow[c] = mx + logf(se);
        }
    }
}

// bf16 teacher with the key blocks shared: a workgroup of 16 waves covers
// 16 * CT * QPW consecutive queries (each wave CT column tiles of 16 columns,
// QPW = 16/G queries x G heads each, so every A fragment read from LDS feeds
// CT MFMAs) and streams the candidate blocks of its last query once through
// a two-slot LDS buffer (rows padded to D + 8 bf16, so the 16 rows of an
// A-fragment read fall in distinct banks); the next block's 16-byte chunks
// are loaded into registers while the current one is used.  A wave skips the
// blocks past its own last query's candidates but meets every barrier.
// Logits go through exp2 with scale * log2(e) folded into one multiply.
constexpr int TCT = 2;   // column tiles per teacher wave

template <int D>
__global__ __launch_bounds__(1024) void aux_teacher_bf16_kernel(const bf16_t *__restrict__ qc,
                                                                const bf16_t *__restrict__ kc, int64_t n,
                                                                int64_t Hq, int64_t Hkv, int64_t W, float scale_u,
                                                                const float *__restrict__ qgain,
                                                                const float *__restrict__ kgain,
                                                                float *__restrict__ L) {
    constexpr int NW = 16, NKS = D / 32, ROW = D + 8, CH = BK * D / 8;   // CH 16-byte chunks per block
    static_assert(CH <= NW * 64, "one chunk per thread");
    __shared__ __align__(16) bf16_t kb[2][BK * ROW];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t g = blockIdx.y, b = blockIdx.z;
    const int G = (int)(Hq / Hkv), QPW = 16 / G;
    const int64_t nb = n / BK;
    const int64_t i0 = (int64_t)blockIdx.x * NW * TCT * QPW;
    const int64_t ilast = (i0 + NW * TCT * QPW - 1 < n) ? i0 + NW * TCT * QPW - 1 : n - 1;
    const int64_t bmax = cand_bmax(ilast, BK, W);          // uniform over the workgroup
    if (bmax < 1) return;
    const int64_t i0w = i0 + (int64_t)w * TCT * QPW;
    const int64_t wlast = (i0w + TCT * QPW - 1 < n) ? i0w + TCT * QPW - 1 : n - 1;
    const int64_t wmax = (i0w < n) ? cand_bmax(wlast, BK, W) : 0;
    const int cq = l16 / G, ch = l16 % G;
    const float s2 = scale_u * 1.4426950408889634f;       // logits in log2 units
    // QKNorm bounds a column's logits by D * |gq| * |gk| * scale (the rows'
    // norms are gain * sqrt(D)); when that bound is at most 60 in log2 units
    // for every column of the wave, it is the column's shift (exp2 of the
    // lowest logit stays a normal float) and no per-block max is needed
    const float bcol = (qgain && kgain) ? (float)D * fabsf(qgain[g * G + ch]) * fabsf(kgain[g]) * s2 : INFINITY;
    const bool fixed = __builtin_amdgcn_readfirstlane(
                           (int)(__builtin_amdgcn_ballot_w64(!(bcol <= 60.0f)) == 0ull)) != 0;
    bf16x8 qop[TCT][NKS];
    bool col_ok[TCT];
    int64_t col_bmax[TCT];
    float *Lrow[TCT];
#pragma unroll
    for (int t = 0; t < TCT; ++t) {
        const int64_t iq = i0w + t * QPW + cq;
        col_ok[t] = l16 < QPW * G && iq < n;
        const int64_t ic = col_ok[t] ? iq : i0;
        col_bmax[t] = col_ok[t] ? cand_bmax(iq, BK, W) : 0;
        const bf16_t *qrow = qc + ((b * n + ic) * Hq + g * G + ch) * D;
        Lrow[t] = L + (((b * Hkv + g) * n + ic) * G + ch) * nb;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const uint4 u =
                col_ok[t] ? *reinterpret_cast<const uint4 *>(qrow + 32 * ks + 8 * lg) : make_uint4(0, 0, 0, 0);
            qop[t][ks] = __builtin_bit_cast(bf16x8, u);
        }
    }
    const bf16_t *kg = kc + (b * Hkv + g) * n * D;
    const bool ld = tid < CH;
    const int r = tid / (D / 8), cc = tid % (D / 8);
    uint4 reg = ld ? *reinterpret_cast<const uint4 *>(kg + (BK + r) * D + 8 * cc) : make_uint4(0, 0, 0, 0);
    for (int64_t c = 1; c <= bmax; ++c) {
        bf16_t *slot = kb[c & 1];
        if (ld) *reinterpret_cast<uint4 *>(slot + r * ROW + 8 * cc) = reg;
        __syncthreads();   // this block staged; every wave is past block c - 2, which used this slot
        if (ld && c + 1 <= bmax) reg = *reinterpret_cast<const uint4 *>(kg + ((c + 1) * BK + r) * D + 8 * cc);
        if (c > wmax) continue;
        f32x4 acc[TCT][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int t = 0; t < TCT; ++t) acc[t][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const bf16_t *krow = slot + (mt * 16 + l16) * ROW + 8 * lg;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(krow + 32 * ks));
#pragma unroll
                for (int t = 0; t < TCT; ++t) acc[t][mt] = mfma_bf16(a, qop[t][ks], acc[t][mt]);
            }
        }
#pragma unroll
        for (int t = 0; t < TCT; ++t) {
            float off = bcol;
            if (!fixed) {
                float mx = -INFINITY;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) mx = fmaxf(mx, acc[t][mt][e]);
                mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                off = mx * s2;
            }
            float se = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) se += __builtin_amdgcn_exp2f(fmaf(acc[t][mt][e], s2, -off));
            se += __shfl_xor(se, 16, 64);
            se += __shfl_xor(se, 32, 64);
            if (lg == 0 && col_ok[t] && c <= col_bmax[t]) Lrow[t][c] = (off + __log2f(se)) * 0.6931471805599453f;
        }
    }
}

// ---------------------------------------------------------------- rows -----
// One wave per (b, g, i) with a candidate block: p* from the block LSEs, the
// row's KL term (rowt), and d aux / d bsc written over bsc.  Head h's max and
// sum of exponentials over the candidate blocks are kept by lane h.
__global__ __launch_bounds__(256) void aux_rows_kernel(float *__restrict__ L, int64_t B, int64_t n,
                                                       int64_t Hkv, int G, int64_t W, float invN,
                                                       float *__restrict__ bsc, float *__restrict__ rowt) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t r = (int64_t)blockIdx.x * 4 + w;
    if (r >= B * Hkv * n) return;
    const int64_t i = r % n;
    const int64_t nb = n / BK;
    const int64_t nbm = cand_bmax(i, BK, W);
    if (nbm < 1) {
        if (lane == 0) rowt[r] = 0.0f;
        return;
    }
    float *Lr = L + r * G * nb;
    float *br = bsc + r * nb;
    float myM = 0.0f, myZ = 1.0f;
    for (int h = 0; h < G; ++h) {   // one pass per head: running max and sum of exponentials
        float mx = -INFINITY, z = 0.0f;
        for (int64_t c = 1 + lane; c <= nbm; c += 64) {
            const float v = Lr[h * nb + c];
            if (v > mx) {
                z = z * expf(mx - v) + 1.0f;
                mx = v;
            } else {
                z += expf(v - mx);
            }
        }
        const float M = wave_max(mx);
        const float Z = wave_sum((mx == -INFINITY) ? 0.0f : z * expf(mx - M));
        if (lane == h) {
            myM = M;
            myZ = Z;
        }
    }
    // p(c), the group mean of the heads' block probabilities, replaces L[head 0][c]
    // (each lane reads and writes only its own blocks c)
    const int64_t cend = 1 + ((nbm + 63) / 64) * 64;   // uniform trip count for the shuffles
    float p0 = 0.0f, top = -INFINITY;
    for (int64_t c = 1 + lane; c < cend; c += 64) {
        float p = 0.0f;
        for (int h = 0; h < G; ++h) {
            const float Mh = __shfl(myM, h, 64), Zh = __shfl(myZ, h, 64);
            p += (c <= nbm) ? expf(Lr[h * nb + c] - Mh) / Zh : 0.0f;
        }
        if (c <= nbm) {
            p /= (float)G;
            Lr[c] = p;
            p0 += p;
            top = fmaxf(top, br[c]);
        }
    }
    p0 = fmaxf(wave_sum(p0), 1e-9f);
    top = wave_max(top);
    float zb = 0.0f;
    for (int64_t c = 1 + lane; c <= nbm; c += 64) zb += expf(br[c] - top);
    const float lse = top + logf(wave_sum(zb));
    float term = 0.0f, P = 0.0f;
    for (int64_t c = 1 + lane; c <= nbm; c += 64) {
        const float ps = Lr[c] / p0;
        if (ps > 0.0f) {
            term += ps * (br[c] - lse);
            P += ps;
        }
    }
    term = wave_sum(term);
    P = wave_sum(P);
    for (int64_t c = 1 + lane; c <= nbm; c += 64) {
        const float ps = Lr[c] / p0;
        const float soft = expf(br[c] - lse);
        br[c] = (soft * P - (ps > 0.0f ? ps : 0.0f)) * invN;
    }
    if (lane == 0) rowt[r] = term;
}

// aux = -(sum of the row terms) / N: one workgroup, double accumulation in a
// fixed order.
__global__ __launch_bounds__(256) void aux_sum_kernel(const float *__restrict__ rowt, int64_t rows, float invN,
                                                      float *__restrict__ aux) {
    __shared__ double part[256];
    double s = 0.0;
    for (int64_t r = threadIdx.x; r < rows; r += 256) s += (double)rowt[r];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int o = 128; o >= 1; o >>= 1) {
        if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) aux[0] = (float)(-part[0] * (double)invN);
}

// ---------------------------------------------------------------- dS0 ------
// d aux / d S0[c, slot, :] = sum over the candidate queries i of c of
// d bsc[i, c] * scale_r / (number of tied slots) * qg[i, :], over the slots
// that tie the max -- in practice one slot per (i, c).  Workgroup = (group
// of 16/m blocks, query segment qs of QS, KV head g, batch b), 16 waves: wave
// (bb, slot) owns that block's slot row, lane t its dims t and t + 64.  Per
// chunk of 64 queries the grouped queries and the (coefficient, tie mask)
// pairs are staged in LDS; a wave adds a query only when its slot is tied at
// the max (a wave-uniform branch), in ascending query order.  The segment's
// partial goes to pdS0[qs]; aux_gsum adds the QS partials in order.
template <int D>
__global__ __launch_bounds__(1024) void aux_dsum_kernel(const float *__restrict__ dbsc,
                                                        const uint8_t *__restrict__ ties,
                                                        const float *__restrict__ qg, int64_t n, int64_t Hkv, int m,
                                                        int64_t W, float scale_r, float *__restrict__ pdS0) {
    constexpr int DL = D / 64;                     // dims per lane
    __shared__ float qgs[64][D];
    __shared__ float coef[64][16];
    __shared__ uint8_t msk[64][16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int bt = 16 / m;                         // blocks per workgroup
    const int bb = w / m, sl = w % m;              // this wave's (block, slot); waves past bt*m idle
    const int64_t c0 = (int64_t)blockIdx.x * bt, qs = blockIdx.y % QS, g = blockIdx.y / QS, b = blockIdx.z;
    const int64_t nb = n / BK;
    const int64_t bg = b * Hkv + g;
    const int64_t c = c0 + bb;
    float acc[DL];
#pragma unroll
    for (int u = 0; u < DL; ++u) acc[u] = 0.0f;
    // this segment's 64-query chunks of the group's candidate queries
    const int64_t ilo = (c0 + 1) * BK + W - 1;
    const int64_t nch = (ilo < n) ? (n - ilo + 63) / 64 : 0;
    const int64_t per = (nch + QS - 1) / QS;
    const int64_t k0 = qs * per, k1 = (k0 + per < nch) ? k0 + per : nch;
    for (int64_t kc_ = k0; kc_ < k1; ++kc_) {
        const int64_t i0 = ilo + kc_ * 64;
        __syncthreads();   // the previous chunk is used
        for (int e = tid; e < 64 * D; e += 1024) {
            const int64_t i = i0 + e / D;
            qgs[e / D][e % D] = (i < n) ? qg[(bg * n + i) * D + e % D] : 0.0f;
        }
        for (int e = tid; e < 64 * bt; e += 1024) {
            const int qi = e / bt, j = e % bt;
            const int64_t i = i0 + qi, cj = c0 + j;
            float cf = 0.0f;
            uint32_t mk = 0;
            if (i < n && cj < nb && cj >= 1 && cj <= cand_bmax(i, BK, W)) {
                const int64_t o = (bg * n + i) * nb + cj;
                mk = ties[o];
                cf = dbsc[o] * scale_r / (float)__builtin_popcount(mk);
            }
            coef[qi][j] = cf;
            msk[qi][j] = (uint8_t)mk;
        }
        __syncthreads();
        if (bb < bt) {
            for (int qi = 0; qi < 64; ++qi) {
                if ((msk[qi][bb] >> sl) & 1u) {   // uniform over the wave
                    const float cf = coef[qi][bb];
#pragma unroll
                    for (int u = 0; u < DL; ++u) acc[u] = fmaf(cf, qgs[qi][lane + 64 * u], acc[u]);
                }
            }
        }
    }
    if (bb < bt && c < nb) {
        float *dst = pdS0 + ((qs * Hkv * gridDim.z + bg) * nb + c) * m * D + sl * D;
        // (pdS0 is [QS][B*Hkv][nb][m][D]; gridDim.z = B)
#pragma unroll
        for (int u = 0; u < DL; ++u) dst[lane + 64 * u] = acc[u];
    }
}

// The same partials on fp32 MFMA (v_mfma_f32_16x16x4_f32): per 64-query
// chunk, dS0 rows (block, slot) += A^T . qg with A[q][(block, slot)] = the
// query's d bsc * scale / tie count where the slot is one of its maxima, else
// 0.  A workgroup takes 64 / m blocks (64 rows, 4 M-tiles) and one query
// segment, so that each staged chunk of qg serves 16 blocks; wave w takes
// the 16-column tiles w, w + 4, ... of d.  fp32 operands: the products are
// those of the scalar chain, the sums run in the MFMA's fixed order.
// CE: (d bsc, tie mask) entries per thread and chunk, 64 * (64 / m) / 256 rounded up (4 for m >= 4)
template <int D, int CE>
__global__ __launch_bounds__(256) void aux_dsum_mfma_kernel(const float *__restrict__ dbsc,
                                                            const uint8_t *__restrict__ ties,
                                                            const float *__restrict__ qg, int64_t n, int64_t Hkv,
                                                            int m, int64_t W, float scale_r,
                                                            float *__restrict__ pdS0) {
    constexpr int NDT = D / 16, DTW = NDT / 4;      // 16-column tiles of d; per wave
    __shared__ float qgs[64][D + 4];
    __shared__ float ca[64][64 + 4];                 // [query][row = block * m + slot]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, lg = lane >> 4;
    const int bt = 64 / m;                           // blocks per workgroup
    const int64_t c0 = (int64_t)blockIdx.x * bt, qs = blockIdx.y % QS, g = blockIdx.y / QS, b = blockIdx.z;
    const int64_t nb = n / BK;
    const int64_t bg = b * Hkv + g;
    af32x4 acc[4][DTW];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int u = 0; u < DTW; ++u) acc[mt][u] = af32x4{0.f, 0.f, 0.f, 0.f};
    // this segment's 64-query chunks of the first block's candidate queries
    const int64_t ilo = (c0 + 1) * BK + W - 1;
    const int64_t nch = (ilo < n) ? (n - ilo + 63) / 64 : 0;
    const int64_t per = (nch + QS - 1) / QS;
    const int64_t k0 = qs * per, k1 = (k0 + per < nch) ? k0 + per : nch;
    // chunk staging through registers, one chunk ahead of the products:
    // qg rows (64 x D) and the 64 x bt (d bsc, tie mask) entries
    constexpr int QPT = 64 * D / 256;
    float rq[QPT];
    float rc[CE];
    uint32_t rm[CE];
    auto gload = [&](int64_t kc_) {
        const int64_t i0 = ilo + kc_ * 64;
#pragma unroll
        for (int r = 0; r < QPT; ++r) {
            const int e = tid + 256 * r;
            const int64_t i = i0 + e / D;
            rq[r] = (i < n) ? qg[(bg * n + i) * D + e % D] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < CE; ++r) {
            const int e = tid + 256 * r;
            const int qi = e / bt, j = e % bt;
            const int64_t i = i0 + qi, cj = c0 + j;
            rc[r] = 0.0f;
            rm[r] = 0u;
            if (e < 64 * bt && i < n && cj < nb && cj >= 1 && cj <= cand_bmax(i, BK, W)) {
                const int64_t o = (bg * n + i) * nb + cj;
                rm[r] = ties[o];
                rc[r] = dbsc[o];
            }
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int r = 0; r < QPT; ++r) {
            const int e = tid + 256 * r;
            qgs[e / D][e % D] = rq[r];
        }
#pragma unroll
        for (int r = 0; r < CE; ++r) {
            const int e = tid + 256 * r;
            if (e >= 64 * bt) continue;
            const int qi = e / bt, j = e % bt;
            const float cf = rm[r] ? rc[r] * scale_r / (float)__builtin_popcount(rm[r]) : 0.0f;
            for (int sl = 0; sl < m; ++sl) ca[qi][j * m + sl] = ((rm[r] >> sl) & 1u) ? cf : 0.0f;
        }
    };
    if (k0 < k1) gload(k0);
    for (int64_t kc_ = k0; kc_ < k1; ++kc_) {
        __syncthreads();   // the previous chunk is used
        lstore();
        __syncthreads();
        if (kc_ + 1 < k1) gload(kc_ + 1);   // in flight during this chunk's products
        // A: row l16 of M-tile mt, queries 4 ks + lg; B: query 4 ks + lg, column l16 of the d tile
#pragma unroll 4
        for (int ks = 0; ks < 16; ++ks) {
            const int qk = 4 * ks + lg;
            float a[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) a[mt] = ca[qk][16 * mt + l16];
#pragma unroll
            for (int u = 0; u < DTW; ++u) {
                const float bv = qgs[qk][16 * (w + 4 * u) + l16];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
                    acc[mt][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt], bv, acc[mt][u], 0, 0, 0);
            }
        }
    }
    // C row 4 lg + e of M-tile mt is dS0 row 16 mt + 4 lg + e = block * m + slot; column l16 of tile w + 4 u
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * mt + 4 * lg + e;
            const int64_t c = c0 + r / m;
            const int sl = r % m;
            if (r / m >= bt || c >= nb) continue;
            float *dst = pdS0 + ((qs * Hkv * gridDim.z + bg) * nb + c) * m * D + sl * D;
#pragma unroll
            for (int u = 0; u < DTW; ++u) dst[16 * (w + 4 * u) + l16] = acc[mt][u][e];
        }
}

// -------------------------------------------------- summariser backward ----
// Workgroup = (block c, g, b): recompute the block's slot attention (att) and
// pooled rows (Sp) from its keys, then with dO = d aux / d S0[c]:
//   d proj  += Sp^T dO                 (per-block partial)
//   dSp      = dO proj^T
//   datt     = dSp K^T,  dlogit = att * (datt - sum_k att * datt)
//   d probes += dlogit K / sqrt(d)     (per-block partial)
template <int DT, int D>
__global__ __launch_bounds__(256) void aux_sbwd_kernel(const typename St<DT>::T *__restrict__ kc,
                                                       const float *__restrict__ probes,
                                                       const float *__restrict__ proj,
                                                       const float *__restrict__ dS0, int64_t n, int64_t Hkv, int m,
                                                       float *__restrict__ pproj, float *__restrict__ pprb) {
    __shared__ float kb[BK][D + 1];
    __shared__ float pr[8][D];
    __shared__ float att[8][BK];
    __shared__ float sp[8][D];
    __shared__ float dO[8][D];
    __shared__ float dsp[8][D];
    const int tid = threadIdx.x;
    const int64_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int64_t nb = n / BK;
    const float isd = 1.0f / sqrtf((float)D);
    const typename St<DT>::T *src = kc + ((b * Hkv + g) * n + c * BK) * D;
    for (int e = tid; e < BK * D; e += 256) kb[e / D][e % D] = St<DT>::ld(src, e);
    for (int e = tid; e < m * D; e += 256) {
        pr[e / D][e % D] = probes[g * m * D + e];
        dO[e / D][e % D] = dS0[((b * Hkv + g) * nb + c) * m * D + e];
    }
    __syncthreads();
    for (int e = tid; e < m * BK; e += 256) {
        const int s = e / BK, k = e % BK;
        float a = 0.0f;
        for (int t = 0; t < D; ++t) a = fmaf(pr[s][t], kb[k][t], a);
        att[s][k] = a * isd;
    }
    __syncthreads();
    {   // softmax over the 64 keys of each slot, one wave per slot
        const int wv = tid / 64, l = tid % 64;
        for (int s = wv; s < m; s += 4) {
            const float x = att[s][l];
            const float mx = wave_max(x);
            const float ex = expf(x - mx);
            att[s][l] = ex / wave_sum(ex);
        }
    }
    __syncthreads();
    for (int e = tid; e < m * D; e += 256) {
        const int s = e / D, t = e % D;
        float a = 0.0f;
        for (int k = 0; k < BK; ++k) a = fmaf(att[s][k], kb[k][t], a);
        sp[s][t] = a;
    }
    __syncthreads();
    float *pp = pproj + ((b * nb + c) * Hkv + g) * D * D;
    for (int e = tid; e < D * D; e += 256) {
        const int t = e / D, ee = e % D;
        float a = 0.0f;
        for (int s = 0; s < m; ++s) a = fmaf(sp[s][t], dO[s][ee], a);
        pp[e] = a;
    }
    const float *pj = proj + g * D * D;
    for (int e = tid; e < m * D; e += 256) {
        const int s = e / D, t = e % D;
        float a = 0.0f;
        for (int ee = 0; ee < D; ++ee) a = fmaf(dO[s][ee], pj[t * D + ee], a);
        dsp[s][t] = a;
    }
    __syncthreads();
    {   // datt, then the softmax backward, one wave per slot (lane = key)
        const int wv = tid / 64, l = tid % 64;
        for (int s = wv; s < m; s += 4) {
            float a = 0.0f;
            for (int t = 0; t < D; ++t) a = fmaf(dsp[s][t], kb[l][t], a);
            const float at = att[s][l];
            const float dot = wave_sum(at * a);
            att[s][l] = at * (a - dot);   // dlogit, in place
        }
    }
    __syncthreads();
    float *pb = pprb + ((b * nb + c) * Hkv + g) * m * D;
    for (int e = tid; e < m * D; e += 256) {
        const int s = e / D, t = e % D;
        float a = 0.0f;
        for (int k = 0; k < BK; ++k) a = fmaf(att[s][k], kb[k][t], a);
        pb[e] = a * isd;
    }
}

// Sum of per-block partials (count of them, each `len` floats apart) in block
// order.
__global__ __launch_bounds__(256) void aux_gsum_kernel(const float *__restrict__ part, int64_t count,
                                                       int64_t len, float *__restrict__ out) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= len) return;
    float s = 0.0f;
    for (int64_t p = 0; p < count; ++p) s += part[p * len + e];
    out[e] = s;
}

__global__ void aux_zero_kernel(float *__restrict__ p, int64_t len) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < len) p[e] = 0.0f;
}

}  // namespace aux
}  // namespace hba

using namespace hba;

// fp32 off the tuned kernels' geometry (64-key blocks, d = 64 / 128, m <= 8,
// G <= 16): the generic kernels (hba_generic.hip)
static bool aux_generic(int dtype, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk) {
    return dtype == HBA_DTYPE_F32 && Hkv > 0 && Hq % Hkv == 0 &&
           !(Bk == aux::BK && (d == 64 || d == 128) && m <= 8 && Hq / Hkv <= 16);
}

extern "C" int hba_aux_kl_workspace_size(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                                         int64_t m, int64_t Bk, size_t *bytes) {
    if (aux_generic(dtype, Hq, Hkv, d, m, Bk)) {
        if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || m <= 0 || Bk <= 0) return HBA_ERR_INVALID_ARG;
        if (!gen_aux_ok(d, Bk, m, Hq / Hkv)) return HBA_ERR_UNSUPPORTED;
        if (n % Bk) return HBA_ERR_UNSUPPORTED;
        *bytes = gen_aux_ws_bytes(B, n, Hq, Hkv, d, m, Bk);
        return HBA_OK;
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || m <= 0) return HBA_ERR_INVALID_ARG;
    if (Hq % Hkv) return HBA_ERR_INVALID_ARG;
    if (Bk != aux::BK || n % aux::BK || m > 8 || Hq / Hkv > 16) return HBA_ERR_UNSUPPORTED;
    *bytes = aux::layout(dtype, B, n, Hq, Hkv, d, m).total;
    return HBA_OK;
}

extern "C" int hba_aux_kl(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
                          const float *k_gain, float eps,
                          const void *kc, const void *S0, const float *probes, const float *proj, int64_t B,
                          int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W,
                          float scale_u, float scale_r, void *ws, size_t ws_bytes, float *aux, float *dprobes,
                          float *dproj, void *stream) {
    size_t need = 0;
    int st = hba_aux_kl_workspace_size(dtype, B, n, Hq, Hkv, d, m, Bk, &need);
    if (st) return st;
    if (!q || !q_strides || !kc || !S0 || !probes || !proj || !ws || !aux || (!dprobes) != (!dproj) || W < 1)
        return HBA_ERR_INVALID_ARG;
    if (ws_bytes < need) return HBA_ERR_INVALID_ARG;
    if (!abi::aligned16(ws) || !abi::aligned16(kc)) return HBA_ERR_UNSUPPORTED;
    if (aux_generic(dtype, Hq, Hkv, d, m, Bk))
        return gen_aux_kl((const float *)q, q_strides, q_gain, eps, (const float *)kc, (const float *)S0, probes, proj,
                          B, n, Hq, Hkv, d, m, Bk, W, scale_u, scale_r, ws, aux, dprobes, dproj,
                          (hipStream_t)stream);
    if (n / aux::BK > 0x7fffffff || Hkv > 65535 || B > 65535) return HBA_ERR_UNSUPPORTED;
    const aux::Ws L = aux::layout(dtype, B, n, Hq, Hkv, d, m);
    char *w = (char *)ws;
    hipStream_t s = (hipStream_t)stream;
    const int64_t nb = n / aux::BK, G = Hq / Hkv;
    const int64_t nvalid = n > aux::first_valid(W) ? n - aux::first_valid(W) : 0;
    const int64_t N = B * Hkv * nvalid;
    const float invN = N ? (float)(1.0 / (double)N) : 0.0f;
    float *qg = (float *)(w + L.qg), *bsc = (float *)(w + L.bsc), *Lb = (float *)(w + L.L);
    float *rowt = (float *)(w + L.rowt), *dS0 = (float *)(w + L.dS0), *pdS0 = (float *)(w + L.pdS0);
    float *pproj = (float *)(w + L.pproj), *pprb = (float *)(w + L.pprb);
    uint8_t *ties = (uint8_t *)(w + L.ties);
    const int64_t rows = B * Hkv * n;
    if (N == 0) {   // no query has a candidate block: aux and its gradients are zero
        hipLaunchKernelGGL(aux::aux_zero_kernel, dim3(1), dim3(256), 0, s, aux, (int64_t)1);
        if (dprobes) {
            hipLaunchKernelGGL(aux::aux_zero_kernel, dim3((unsigned)((Hkv * m * d + 255) / 256)), dim3(256), 0, s,
                               dprobes, Hkv * m * d);
            hipLaunchKernelGGL(aux::aux_zero_kernel, dim3((unsigned)((Hkv * d * d + 255) / 256)), dim3(256), 0, s,
                               dproj, Hkv * d * d);
        }
        HBA_LAUNCH_CHECK();
        return HBA_OK;
    }
#define HBA_AUX_FWD(DT, D)                                                                               \
    do {                                                                                                 \
        typedef St<DT>::T T;                                                                             \
        T *qc = (T *)(w + L.qc);                                                                         \
        hipLaunchKernelGGL((aux::aux_qc_kernel<DT, D>), dim3((unsigned)((B * n * Hq + 255) / 256)),       \
                           dim3(256), 0, s, (const T *)q, q_strides[0], q_strides[1], q_strides[2], q_gain, \
                           eps, B, n, Hq, qc);                                                           \
        if (DT == 1 && m == 4)                                                                           \
            hipLaunchKernelGGL((aux::aux_scores_mfma_kernel<D>), dim3((unsigned)((n + 63) / 64),         \
                               (unsigned)Hkv, (unsigned)B), dim3(256), 0, s, (const bf16_t *)qc,          \
                               (const bf16_t *)S0, n, Hq, Hkv, W, scale_r, qg, bsc, ties);                \
        else                                                                                             \
            hipLaunchKernelGGL((aux::aux_scores_kernel<DT, D>), dim3((unsigned)((n + 63) / 64),          \
                               (unsigned)Hkv, (unsigned)B), dim3(256), 0, s, (const T *)qc, (const T *)S0, n, \
                               Hq, Hkv, (int)m, W, scale_r, qg, bsc, ties);                              \
        const int64_t qpw = 16 / G;                                                                      \
        if (DT == 1)                                                                                     \
            hipLaunchKernelGGL((aux::aux_teacher_bf16_kernel<D>),                                        \
                               dim3((unsigned)((n + 16 * aux::TCT * qpw - 1) / (16 * aux::TCT * qpw)),    \
                                    (unsigned)Hkv,                                                       \
                               (unsigned)B), dim3(1024), 0, s, (const bf16_t *)qc, (const bf16_t *)kc, n,  \
                               Hq, Hkv, W, scale_u, q_gain, k_gain, Lb);                                 \
        else                                                                                             \
            hipLaunchKernelGGL((aux::aux_teacher_kernel<DT, D>),                                         \
                               dim3((unsigned)((n + 4 * qpw - 1) / (4 * qpw)), (unsigned)Hkv,             \
                               (unsigned)B), dim3(256), 0, s, (const T *)qc, (const T *)kc, n, Hq, Hkv, W, \
                               scale_u, Lb);                                                             \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_AUX_FWD);
#undef HBA_AUX_FWD
    hipLaunchKernelGGL(aux::aux_rows_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, Lb, B, n, Hkv,
                       (int)G, W, invN, bsc, rowt);
    hipLaunchKernelGGL(aux::aux_sum_kernel, dim3(1), dim3(256), 0, s, rowt, rows, invN, aux);
    if (dprobes) {
#define HBA_AUX_BWD(DT, D)                                                                               \
    do {                                                                                                 \
        typedef St<DT>::T T;                                                                             \
        if (64 % m == 0 && m >= 4)                                                                       \
            hipLaunchKernelGGL((aux::aux_dsum_mfma_kernel<D, 4>), dim3((unsigned)((nb + 64 / m - 1) / (64 / m)), \
                               (unsigned)(Hkv * aux::QS), (unsigned)B), dim3(256), 0, s, bsc, ties, qg, n,  \
                               Hkv, (int)m, W, scale_r, pdS0);                                           \
        else if (64 % m == 0)                                                                            \
            hipLaunchKernelGGL((aux::aux_dsum_mfma_kernel<D, 16>), dim3((unsigned)((nb + 64 / m - 1) / (64 / m)), \
                               (unsigned)(Hkv * aux::QS), (unsigned)B), dim3(256), 0, s, bsc, ties, qg, n,  \
                               Hkv, (int)m, W, scale_r, pdS0);                                           \
        else                                                                                             \
            hipLaunchKernelGGL((aux::aux_dsum_kernel<D>), dim3((unsigned)((nb + 16 / m - 1) / (16 / m)), \
                               (unsigned)(Hkv * aux::QS), (unsigned)B), dim3(1024), 0, s, bsc, ties, qg, n, \
                               Hkv, (int)m, W, scale_r, pdS0);                                           \
        hipLaunchKernelGGL(aux::aux_gsum_kernel, dim3((unsigned)((B * Hkv * nb * m * d + 255) / 256)),   \
                           dim3(256), 0, s, pdS0, (int64_t)aux::QS, B * Hkv * nb * m * d, dS0);          \
        hipLaunchKernelGGL((aux::aux_sbwd_kernel<DT, D>), dim3((unsigned)nb, (unsigned)Hkv, (unsigned)B),  \
                           dim3(256), 0, s, (const T *)kc, probes, proj, dS0, n, Hkv, (int)m, pproj, pprb); \
    } while (0)
        HBA_DISPATCH_DT_D(dtype, d, HBA_AUX_BWD);
#undef HBA_AUX_BWD
        const int64_t lp = Hkv * d * d, lb = Hkv * m * d;
        hipLaunchKernelGGL(aux::aux_gsum_kernel, dim3((unsigned)((lp + 255) / 256)), dim3(256), 0, s, pproj, B * nb,
                           lp, dproj);
        hipLaunchKernelGGL(aux::aux_gsum_kernel, dim3((unsigned)((lb + 255) / 256)), dim3(256), 0, s, pprb, B * nb,
                           lb, dprobes);
    }
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
