// Decode step over a paged KV cache.  The reference has no decode path; the
// step is defined as row L-1 of hba_attention_eval (src/hba/attention.py:
// 610-713) for a sequence of length L: flat top-k over the full pages before
// the window (route_topk's rule, :272-303), then one softmax over sinks,
// the RoPE window and the selected pages.
//
// The step is HBM-bound (~0.7 MB of keys, values and summaries per (sequence,
// KV head) at 32K).  To spread it over all CUs it is split flash-decoding
// style into three launches:
//   D1  score chunks (64 candidate pages each: declared-order slot scores and
//       a chunk-local top-k) and, in the same grid, window chunks (64 keys
//       each, RoPE applied in the kernel; chunk 0 also takes the sinks) that
//       write partial softmax states;
//   D2  one workgroup per (sequence, KV head, pick rank): merges the chunk
//       top-k lists, takes its pick and writes that page's partial state;
//   D3  LSE merge of all partial states into the output.
#include "hba_common.h"
#include "hba_abi.h"

namespace hba {

constexpr int DEC_WG = 256;
constexpr int DEC_CP = 64;    // candidate pages per score chunk
constexpr int DEC_WCH = 64;   // window keys per chunk
constexpr int DEC_KMAX = 64;  // largest k

struct DecGeom {
    int nsc;   // score chunks
    int nwc;   // window chunks
    int npart; // partial states per (seq, KV head) = nwc + k
};

__host__ __device__ inline DecGeom dec_geom(int64_t W, int64_t k, int64_t max_len) {
    DecGeom gm;
    int64_t bm = cand_bmax(max_len - 1, 64, W);
    gm.nsc = (int)((bm + DEC_CP - 1) / DEC_CP);
    gm.nwc = (int)((W + DEC_WCH - 1) / DEC_WCH);
    gm.npart = gm.nwc + (int)k;
    return gm;
}

// QKNorm'd query rows of the G heads of (s, g) into LDS (fp32), declared order.
template <int DT, int D>
__device__ __forceinline__ void dec_query(const typename St<DT>::T *q, const float *qgain, float eps,
                                          int64_t s, int g, int G, int Hq, float *qc_lds) {
    const int tid = threadIdx.x;
    if (tid < G) {
        const int h = g * G + tid;
        const typename St<DT>::T *row = q + ((int64_t)s * Hq + h) * D;
        float x[D];
#pragma unroll
        for (int t = 0; t < D; ++t) x[t] = St<DT>::ld(row, t);
        if (qgain) qknorm_row<DT, D>(x, qgain[h], eps);
#pragma unroll
        for (int t = 0; t < D; ++t) qc_lds[tid * D + t] = x[t];
    }
}

template <int DT, int D, int M>
__global__ __launch_bounds__(DEC_WG) void decode_d1_kernel(
    const typename St<DT>::T *__restrict__ q, const float *__restrict__ qgain, float eps,
    const typename St<DT>::T *__restrict__ kcp, const typename St<DT>::T *__restrict__ vp,
    const typename St<DT>::T *__restrict__ sp, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const float *__restrict__ scales, int Hq, int Hkv, int S, int64_t W, int K, DecGeom gm,
    float *__restrict__ ws_val, int32_t *__restrict__ ws_idx, float *__restrict__ ws_part) {
    constexpr int BK = 64;
    __shared__ __align__(16) float qc[8 * D];
    __shared__ __align__(16) float qx[8 * D];
    __shared__ __align__(16) float kb[DEC_WCH][D + 1];
    __shared__ __align__(16) float sc[8][DEC_WCH + 64];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t L = min((int64_t)lens[s], maxp * 64);   // never index past the page table
    const float scale = scales[s];
    const int32_t *pt = ptab + s * maxp;
    dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc);
    __syncthreads();
    if (z < gm.nsc) {
        // ------------------------------------------------ score chunk --------
        // routing query: sequential head sum, rounded (summarizer.py:50-54)
        if (tid < D) {
            float a = qc[tid];
            for (int h = 1; h < G; ++h) a = a + qc[h * D + tid];
            qx[tid] = St<DT>::rnd(a);
        }
        __syncthreads();
        const int64_t bmax = (L >= 1) ? cand_bmax(L - 1, BK, W) : 0;
        const int p = tid % DEC_CP;
        const int64_t blk = 1 + (int64_t)z * DEC_CP + p;
        for (int sl = tid / DEC_CP; sl < M; sl += DEC_WG / DEC_CP) {
            float acc = 0.0f;
            if (blk <= bmax) {
                const int64_t phys = pt[blk];
                const typename St<DT>::T *srow = sp + ((phys * Hkv + g) * M + sl) * D;
#pragma unroll 8
                for (int t = 0; t < D; ++t) acc = fmaf(qx[t], St<DT>::ld(srow, t), acc);
            }
            sc[sl][p] = acc;
        }
        __syncthreads();
        if (tid < DEC_CP) {
            float best = sc[0][p];
#pragma unroll
            for (int sl = 1; sl < M; ++sl) best = (sc[sl][p] > best) ? sc[sl][p] : best;
            const float v = (blk <= bmax) ? best * scale : -INFINITY;
            const int id = (int)blk;
            // rank of (v, id) among the 64 entries under (value desc, id asc)
            int rank = 0;
            for (int o = 0; o < DEC_CP; ++o) {
                float vo = __shfl(v, o, 64);
                int io = __shfl(id, o, 64);
                rank += ((vo > v) || (vo == v && io < id)) ? 1 : 0;
            }
            if (rank < K) {
                const int64_t o = (((int64_t)s * Hkv + g) * gm.nsc + z) * K + rank;
                ws_val[o] = v;
                ws_idx[o] = (v == -INFINITY) ? -1 : id;
            }
        }
        return;
    }
    // ---------------------------------------------------- window chunk ------
    const int wc = z - gm.nsc;
    const int64_t i = L - 1;
    const int64_t wbeg = ((int64_t)S > i - W + 1) ? (int64_t)S : i - W + 1;
    const int64_t k0 = wbeg + (int64_t)wc * DEC_WCH;
    const int64_t k1 = (k0 + DEC_WCH - 1 < i) ? k0 + DEC_WCH - 1 : i;   // inclusive
    const int nw = (L >= 1 && k0 <= k1) ? (int)(k1 - k0 + 1) : 0;
    const int ns = (wc == 0 && L >= 1) ? (int)(((int64_t)S < L) ? S : L) : 0;
    // RoPE of the query at position i (rounded like apply_rope on x.dtype)
    for (int e = tid; e < G * D; e += DEC_WG) {
        const int h = e / D, t = e % D;
        if (L >= 1) {
            const float x = qc[h * D + t];
            const float rot = (t < D / 2) ? -qc[h * D + t + D / 2] : qc[h * D + t - D / 2];
            const float c = St<DT>::rnd(cosT[i * D + t]), sn = St<DT>::rnd(sinT[i * D + t]);
            qx[h * D + t] = St<DT>::rnd(St<DT>::rnd(x * c) + St<DT>::rnd(rot * sn));
        }
    }
    float *part = ws_part + (((int64_t)s * Hkv + g) * gm.npart + wc) * G * (D + 2);
    // sinks and window keys: rows 0..ns-1 = sinks (NoPE), ns..ns+nw-1 = window (RoPE)
    const int nk = ns + nw;
    // two passes of at most DEC_WCH keys held in LDS (pass 0: sinks, pass 1:
    // the window chunk); the per-head running state lives in LDS
    __shared__ float Oacc[8][D];
    __shared__ float Mh[8], Lh[8];
    for (int e = tid; e < G * D; e += DEC_WG) Oacc[e / D][e % D] = 0.0f;
    if (tid < G) {
        Mh[tid] = -INFINITY;
        Lh[tid] = 0.0f;
    }
    for (int pass = 0; pass < 2; ++pass) {
        const int cntk = pass == 0 ? ns : nw;
        if (cntk == 0) continue;
        __syncthreads();
        // load keys (kc; rotated for the window) into kb, one thread per (key, d)
        for (int e = tid; e < cntk * D; e += DEC_WG) {
            const int r = e / D, t = e % D;
            const int64_t j = pass == 0 ? r : k0 + r;
            const int64_t phys = pt[j / BK];
            const typename St<DT>::T *krow = kcp + ((phys * Hkv + g) * BK + j % BK) * D;
            float x = St<DT>::ld(krow, t);
            if (pass == 1) {
                const float rot = (t < D / 2) ? -St<DT>::ld(krow, t + D / 2) : St<DT>::ld(krow, t - D / 2);
                const float c = St<DT>::rnd(cosT[j * D + t]), sn = St<DT>::rnd(sinT[j * D + t]);
                x = St<DT>::rnd(St<DT>::rnd(x * c) + St<DT>::rnd(rot * sn));
            }
            kb[r][t] = x;
        }
        __syncthreads();
        const float *qv = pass == 0 ? qc : qx;
        for (int e = tid; e < G * cntk; e += DEC_WG) {
            const int h = e / cntk, r = e % cntk;
            float a = 0.0f;
#pragma unroll 8
            for (int t = 0; t < D; ++t) a = fmaf(qv[h * D + t], kb[r][t], a);
            sc[h][r] = a * scale;
        }
        __syncthreads();
        // per-head softmax update (one wave per head)
        {
            const int wv = tid / 64, ln = tid % 64;
            for (int h = wv; h < G; h += DEC_WG / 64) {
                float mx = -INFINITY;
                for (int r = ln; r < cntk; r += 64) mx = fmaxf(mx, sc[h][r]);
                mx = wave_max(mx);
                const float mnew = fmaxf(Mh[h], mx);
                float sm = 0.0f;
                for (int r = ln; r < cntk; r += 64) {
                    float p = expf(sc[h][r] - mnew);
                    sc[h][r] = p;
                    sm += p;
                }
                sm = wave_sum(sm);
                if (ln == 0) {
                    const float alpha = expf(Mh[h] - mnew);
                    Lh[h] = Lh[h] * alpha + sm;
                    Mh[h] = mnew;
                    sc[h][DEC_WCH + 63] = alpha;  // stash alpha for the O rescale
                }
            }
        }
        __syncthreads();
        // values into kb (reuse), then O = O*alpha + P.V
        for (int e = tid; e < cntk * D; e += DEC_WG) {
            const int r = e / D, t = e % D;
            const int64_t j = pass == 0 ? r : k0 + r;
            const int64_t phys = pt[j / BK];
            kb[r][t] = St<DT>::ld(vp + ((phys * Hkv + g) * BK + j % BK) * D, t);
        }
        __syncthreads();
        for (int e = tid; e < G * D; e += DEC_WG) {
            const int h = e / D, t = e % D;
            float a = Oacc[h][t] * sc[h][DEC_WCH + 63];
            for (int r = 0; r < cntk; ++r) a = fmaf(sc[h][r], kb[r][t], a);
            Oacc[h][t] = a;
        }
    }
    __syncthreads();
    for (int e = tid; e < G * (D + 2); e += DEC_WG) {
        const int h = e / (D + 2), t = e % (D + 2);
        float v;
        if (nk == 0) v = (t == D) ? -INFINITY : 0.0f;
        else v = (t < D) ? Oacc[h][t] : (t == D ? Mh[h] : Lh[h]);
        part[e] = v;
    }
}

template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d2_kernel(
    const typename St<DT>::T *__restrict__ q, const float *__restrict__ qgain, float eps,
    const typename St<DT>::T *__restrict__ kcp, const typename St<DT>::T *__restrict__ vp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ scales, int Hq, int Hkv, int K, DecGeom gm,
    const float *__restrict__ ws_val, const int32_t *__restrict__ ws_idx, float *__restrict__ ws_part,
    int32_t *__restrict__ sel_idx, int32_t *__restrict__ sel_cnt) {
    constexpr int BK = 64;
    __shared__ __align__(16) float qc[8 * D];
    __shared__ float ev[2048];
    __shared__ int ei[2048];
    __shared__ int pick;
    __shared__ int nvalid;
    __shared__ float kb[BK][D + 1];
    __shared__ float sc[8][BK];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int r = blockIdx.z;
    const int G = Hq / Hkv;
    const int E = gm.nsc * K;
    const float scale = scales[s];
    const int64_t base = ((int64_t)s * Hkv + g) * gm.nsc * K;
    if (tid == 0) {
        pick = -1;
        nvalid = 0;
    }
    for (int e = tid; e < E; e += DEC_WG) {
        ev[e] = ws_val[base + e];
        ei[e] = ws_idx[base + e];
    }
    __syncthreads();
    for (int e = tid; e < E; e += DEC_WG) {
        const float v = ev[e];
        const int id = ei[e];
        if (v == -INFINITY) continue;
        int rank = 0;
        for (int o = 0; o < E; ++o) {
            const float vo = ev[o];
            const int io = ei[o];
            rank += (vo != -INFINITY && ((vo > v) || (vo == v && io < id))) ? 1 : 0;
        }
        if (rank == r) pick = id;
        if (r == 0 && rank < K) {
            if (sel_idx) sel_idx[((int64_t)s * Hkv + g) * K + rank] = id;
            atomicAdd(&nvalid, 1);
        }
    }
    __syncthreads();
    if (r == 0) {
        const int nv = nvalid;
        if (sel_idx)
            for (int e = nv + tid; e < K; e += DEC_WG) sel_idx[((int64_t)s * Hkv + g) * K + e] = -1;
        if (sel_cnt && tid == 0) sel_cnt[(int64_t)s * Hkv + g] = nv < K ? nv : K;
    }
    float *part = ws_part + (((int64_t)s * Hkv + g) * gm.npart + gm.nwc + r) * G * (D + 2);
    const int blk = pick;
    if (blk < 0 || (int64_t)blk >= maxp) {
        for (int e = tid; e < G * (D + 2); e += DEC_WG) part[e] = ((e % (D + 2)) == D) ? -INFINITY : 0.0f;
        return;
    }
    dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc);
    const int64_t phys = ptab[s * maxp + blk];
    const typename St<DT>::T *kbase = kcp + (phys * Hkv + g) * BK * D;
    const typename St<DT>::T *vbase = vp + (phys * Hkv + g) * BK * D;
    for (int e = tid; e < BK * D; e += DEC_WG) kb[e / D][e % D] = St<DT>::ld(kbase, e);
    __syncthreads();
    for (int e = tid; e < G * BK; e += DEC_WG) {
        const int h = e / BK, j = e % BK;
        float a = 0.0f;
#pragma unroll 8
        for (int t = 0; t < D; ++t) a = fmaf(qc[h * D + t], kb[j][t], a);
        sc[h][j] = a * scale;
    }
    __syncthreads();
    __shared__ float Mh[8], Lh[8];
    {
        const int wv = tid / 64, ln = tid % 64;
        for (int h = wv; h < G; h += DEC_WG / 64) {
            const float x = sc[h][ln];
            const float mx = wave_max(x);
            const float p = expf(x - mx);
            sc[h][ln] = p;
            const float sm = wave_sum(p);
            if (ln == 0) {
                Mh[h] = mx;
                Lh[h] = sm;
            }
        }
    }
    for (int e = tid; e < BK * D; e += DEC_WG) kb[e / D][e % D] = St<DT>::ld(vbase, e);
    __syncthreads();
    for (int e = tid; e < G * (D + 2); e += DEC_WG) {
        const int h = e / (D + 2), t = e % (D + 2);
        float v;
        if (t < D) {
            float a = 0.0f;
            for (int j = 0; j < BK; ++j) a = fmaf(sc[h][j], kb[j][t], a);
            v = a;
        } else {
            v = (t == D) ? Mh[h] : Lh[h];
        }
        part[e] = v;
    }
}

template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d3_kernel(const float *__restrict__ ws_part, int Hq,
                                                           int Hkv, DecGeom gm,
                                                           typename St<DT>::T *__restrict__ out) {
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int G = Hq / Hkv;
    const float *part = ws_part + ((int64_t)s * Hkv + g) * gm.npart * G * (D + 2);
    for (int e = tid; e < G * D; e += DEC_WG) {
        const int h = e / D, t = e % D;
        float m = -INFINITY;
        for (int c = 0; c < gm.npart; ++c) m = fmaxf(m, part[((int64_t)c * G + h) * (D + 2) + D]);
        float num = 0.0f, den = 0.0f;
        for (int c = 0; c < gm.npart; ++c) {
            const float *ph = part + ((int64_t)c * G + h) * (D + 2);
            const float mc = ph[D];
            if (mc == -INFINITY) continue;
            const float wgt = expf(mc - m);
            num = fmaf(ph[t], wgt, num);
            den = fmaf(ph[D + 1], wgt, den);
        }
        St<DT>::st(out, ((int64_t)s * Hq + g * G + h) * D + t, den > 0.0f ? num / den : 0.0f);
    }
}

}  // namespace hba

using namespace hba;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static void ws_layout(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k, DecGeom gm,
                      size_t *off_val, size_t *off_idx, size_t *off_part, size_t *total) {
    size_t nsel = (size_t)Bd * Hkv * (gm.nsc > 0 ? gm.nsc : 1) * k;
    size_t G = (size_t)(Hq / Hkv);
    *off_val = 0;
    *off_idx = align256(nsel * 4);
    *off_part = *off_idx + align256(nsel * 4);
    *total = *off_part + align256((size_t)Bd * Hkv * gm.npart * G * (d + 2) * 4);
}

extern "C" int hba_decode_workspace_size(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k,
                                         int64_t Bk, int64_t W, int64_t max_len, size_t *bytes) {
    if (!bytes || Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || k < 1 || W < 1 || max_len < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || k > DEC_KMAX) return HBA_ERR_UNSUPPORTED;
    DecGeom gm = dec_geom(W, k, max_len);
    size_t a, b, c;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &a, &b, &c, bytes);
    return HBA_OK;
}

extern "C" int hba_decode_fwd(int dtype, const void *q, const float *q_gain, float eps,
                              const void *kc_pages, const void *v_pages, const void *summ_pages,
                              const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                              const float *cos_tab, const float *sin_tab, const float *scales,
                              int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t S,
                              int64_t W, int64_t Bk, int64_t k, int64_t max_len, void *workspace,
                              size_t ws_bytes, void *out, int32_t *sel_idx, int32_t *sel_cnt,
                              void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !kc_pages || !v_pages || !summ_pages || !page_table || !seq_lens || !cos_tab ||
        !sin_tab || !scales || !workspace || !out)
        return HBA_ERR_INVALID_ARG;
    if (Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || W < 1 || S < 0 || k < 1 || max_len < 1 ||
        max_pages < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || S > Bk) return HBA_ERR_UNSUPPORTED;
    if (Hq / Hkv > 8 || k > DEC_KMAX || !(m == 1 || m == 2 || m == 4 || m == 8)) return HBA_ERR_UNSUPPORTED;
    if ((max_len + Bk - 1) / Bk > max_pages) return HBA_ERR_INVALID_ARG;
    if (Bd > 65535 || Hkv > 65535) return HBA_ERR_UNSUPPORTED;
    DecGeom gm = dec_geom(W, k, max_len);
    if ((int64_t)gm.nsc * k > 2048) return HBA_ERR_UNSUPPORTED;
    size_t ov, oi, op, total;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &ov, &oi, &op, &total);
    if (ws_bytes < total) return HBA_ERR_INVALID_ARG;
    char *ws = (char *)workspace;
    float *wv = (float *)(ws + ov);
    int32_t *wi = (int32_t *)(ws + oi);
    float *wp = (float *)(ws + op);
    hipStream_t s = (hipStream_t)stream;
    dim3 g1((unsigned)Bd, (unsigned)Hkv, (unsigned)(gm.nsc + gm.nwc));
    dim3 g2((unsigned)Bd, (unsigned)Hkv, (unsigned)k);
    dim3 g3((unsigned)Bd, (unsigned)Hkv, 1);
#define HBA_D1(DT, D, M)                                                                          \
    hipLaunchKernelGGL((decode_d1_kernel<DT, D, M>), g1, dim3(DEC_WG), 0, s,                        \
                       (const St<DT>::T *)q, q_gain, eps, (const St<DT>::T *)kc_pages,              \
                       (const St<DT>::T *)v_pages, (const St<DT>::T *)summ_pages, page_table,       \
                       max_pages, seq_lens, cos_tab, sin_tab, scales, (int)Hq, (int)Hkv, (int)S, W, \
                       (int)k, gm, wv, wi, wp)
#define HBA_D1M(DT, D)                  \
    do {                                \
        if (m == 1) HBA_D1(DT, D, 1);   \
        else if (m == 2) HBA_D1(DT, D, 2); \
        else if (m == 4) HBA_D1(DT, D, 4); \
        else HBA_D1(DT, D, 8);          \
    } while (0)
#define HBA_D23(DT, D)                                                                            \
    do {                                                                                          \
        hipLaunchKernelGGL((decode_d2_kernel<DT, D>), g2, dim3(DEC_WG), 0, s,                       \
                           (const St<DT>::T *)q, q_gain, eps, (const St<DT>::T *)kc_pages,          \
                           (const St<DT>::T *)v_pages, page_table, max_pages, seq_lens, scales,    \
                           (int)Hq, (int)Hkv, (int)k, gm, wv, wi, wp, sel_idx, sel_cnt);            \
        hipLaunchKernelGGL((decode_d3_kernel<DT, D>), g3, dim3(DEC_WG), 0, s, wp, (int)Hq,          \
                           (int)Hkv, gm, (St<DT>::T *)out);                                         \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_D1M);
    HBA_DISPATCH_DT_D(dtype, d, HBA_D23);
#undef HBA_D1
#undef HBA_D1M
#undef HBA_D23
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
