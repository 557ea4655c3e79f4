// Decode step over a paged KV cache.  The reference has no decode path; the
// step is defined as row L-1 of hba_attention_eval (src/hba/attention.py:
// 610-713) for a sequence of length L: flat top-k over the full pages before
// the window (route_topk's rule, :272-303), then one softmax over sinks,
// the RoPE window and the selected pages.
//
// The step is HBM-bound (~0.7 MB of keys, values and summaries per (sequence,
// KV head) at 32K), so it is split flash-decoding style over the whole chip,
// every workgroup issuing all of its 16-byte loads before it computes:
//   D1  per (sequence, KV head): score chunks of 64 candidate pages
//       (declared-order slot scores, chunk-local top-k) and, in the same grid,
//       window chunks of 64 keys (RoPE applied to the keys in the kernel;
//       chunk 0 also takes the sinks) that write partial softmax states;
//   D2  one workgroup per (sequence, KV head, pick rank): merges the chunk
//       top-k lists, takes its pick and writes that page's partial state;
//   D3  LSE merge of all partial states of a (sequence, KV head).
#include "hba_common.h"
#include "hba_abi.h"

namespace hba {

constexpr int DEC_WG = 256;
constexpr int DEC_CP = 64;    // candidate pages per score chunk
constexpr int DEC_WCH = 64;   // window keys per chunk
constexpr int DEC_KMAX = 64;  // largest k
constexpr int DEC_GMAX = 8;   // largest group size
constexpr int DEC_PMAX = 128; // largest number of partial states

typedef unsigned int u32x4d __attribute__((ext_vector_type(4)));

struct DecGeom {
    int nsc;    // score chunks
    int nwc;    // window chunks
    int npart;  // partial states per (seq, KV head) = nwc + k
};

__host__ __device__ inline DecGeom dec_geom(int64_t W, int64_t k, int64_t max_len) {
    DecGeom gm;
    int64_t bm = cand_bmax(max_len - 1, 64, W);
    gm.nsc = (int)((bm + DEC_CP - 1) / DEC_CP);
    gm.nwc = (int)((W + DEC_WCH - 1) / DEC_WCH);
    gm.npart = gm.nwc + (int)k;
    return gm;
}

// 8 consecutive storage elements -> fp32 (16 bytes for bf16, 32 for fp32)
template <int DT>
__device__ __forceinline__ void ld8(const typename St<DT>::T *p, float (&x)[8]) {
    if constexpr (DT == 1) {
        u32x4d u = *reinterpret_cast<const u32x4d *>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(u[e] << 16);
            x[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        }
    } else {
        const float4 a = reinterpret_cast<const float4 *>(p)[0];
        const float4 c = reinterpret_cast<const float4 *>(p)[1];
        x[0] = a.x;
        x[1] = a.y;
        x[2] = a.z;
        x[3] = a.w;
        x[4] = c.x;
        x[5] = c.y;
        x[6] = c.z;
        x[7] = c.w;
    }
}

// QKNorm'd query rows of the G heads of (s, g) into LDS (fp32): the rows
// are staged cooperatively, then one thread per head normalises its row in
// the declared order (sequential FMA sum of squares, as qknorm_row); with
// qr_lds also their rotation at position `pos` (apply_rope's roundings).
// Ends with a barrier.
template <int DT, int D>
__device__ __forceinline__ void dec_query(const typename St<DT>::T *q, const float *qgain, float eps,
                                          int64_t s, int g, int G, int Hq, float *qc_lds, float *qr_lds,
                                          const float *cosT, const float *sinT, int64_t pos) {
    const int tid = threadIdx.x;
    const typename St<DT>::T *rows = q + ((int64_t)s * Hq + (int64_t)g * G) * D;
    for (int e = 8 * tid; e < G * D; e += 8 * DEC_WG) {   // 8-element vector loads
        float x[8];
        ld8<DT>(rows + e, x);
#pragma unroll
        for (int u = 0; u < 8; ++u) qc_lds[e + u] = x[u];
    }
    __syncthreads();
    if (qgain) {
        // sum of squares: sequential per head (declared order); the scaling
        // of the elements is independent and spread over the workgroup
        __shared__ float rinv[DEC_GMAX];
        if (tid < G) {
            const float *x = qc_lds + tid * D;
            float ss = 0.0f;
#pragma unroll
            for (int t = 0; t < D; ++t) ss = fmaf(x[t], x[t], ss);
            float ms = ss / (float)D;
            if (ms < eps) ms = eps;
            rinv[tid] = sqrtf(ms);
        }
        __syncthreads();
        for (int e = tid; e < G * D; e += DEC_WG) {
            const int h = e / D;
            qc_lds[e] = St<DT>::rnd((qc_lds[e] / rinv[h]) * qgain[g * G + h]);
        }
    }
    __syncthreads();
    if (qr_lds) {
        for (int e = tid; e < G * D; e += DEC_WG) {
            const int h = e / D, t = e % D;
            const float x = qc_lds[h * D + t];
            const float rot = (t < D / 2) ? -qc_lds[h * D + t + D / 2] : qc_lds[h * D + t - D / 2];
            const float c = St<DT>::rnd(cosT[pos * D + t]), sn = St<DT>::rnd(sinT[pos * D + t]);
            qr_lds[e] = St<DT>::rnd(St<DT>::rnd(x * c) + St<DT>::rnd(rot * sn));
        }
        __syncthreads();
    }
}

// Partial softmax state of G heads over the first nk keys held in LDS (kb,
// vb rows, fp32) for queries qv [G][D] in LDS; writes (O[G][D], m[G], l[G])
// rows of D + 2 floats to `part` (global or LDS).  Ends with a barrier.
template <int D>
__device__ __forceinline__ void dec_partial(const float *qv, float (*kb)[D + 1], float (*vb)[D + 1],
                                            float (*sc)[DEC_WCH], int G, int nk, float scale,
                                            float *part) {
    __shared__ float Mh[DEC_GMAX], Lh[DEC_GMAX];
    const int tid = threadIdx.x;
    for (int e = tid; e < G * DEC_WCH; e += DEC_WG) {
        const int h = e / DEC_WCH, r = e % DEC_WCH;
        float a = -INFINITY;
        if (r < nk) {
            a = 0.0f;
#pragma unroll 16
            for (int t = 0; t < D; ++t) a = fmaf(qv[h * D + t], kb[r][t], a);
            a *= scale;
        }
        sc[h][r] = a;
    }
    __syncthreads();
    {
        const int wv = tid / 64, ln = tid % 64;
        for (int h = wv; h < G; h += DEC_WG / 64) {
            const float x = sc[h][ln];
            const float mx = wave_max(x);
            const float p = (x == -INFINITY) ? 0.0f : expf(x - mx);
            sc[h][ln] = p;
            const float sm = wave_sum(p);
            if (ln == 0) {
                Mh[h] = mx;
                Lh[h] = sm;
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < G * (D + 2); e += DEC_WG) {
        const int h = e / (D + 2), t = e % (D + 2);
        float v;
        if (t < D) {
            float a = 0.0f;
#pragma unroll 16
            for (int r = 0; r < nk; ++r) a = fmaf(sc[h][r], vb[r][t], a);
            v = a;
        } else {
            v = (t == D) ? Mh[h] : Lh[h];
        }
        part[e] = v;
    }
    __syncthreads();
}

__device__ __forceinline__ void empty_partial(float *part, int G, int D2) {
    for (int e = threadIdx.x; e < G * D2; e += DEC_WG) part[e] = ((e % D2) == D2 - 2) ? -INFINITY : 0.0f;
}

template <int DT, int D, int M>
__global__ __launch_bounds__(DEC_WG) void decode_d1_kernel(
    const typename St<DT>::T *__restrict__ q, const float *__restrict__ qgain, float eps,
    const typename St<DT>::T *__restrict__ kcp, const typename St<DT>::T *__restrict__ vp,
    const typename St<DT>::T *__restrict__ sp, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const float *__restrict__ scales, int Hq, int Hkv, int S, int64_t W, int K, DecGeom gm,
    float *__restrict__ ws_val, int32_t *__restrict__ ws_idx, int32_t *__restrict__ ws_phys,
    float *__restrict__ ws_part) {
    constexpr int BK = 64;
    constexpr int SR = (M > 4) ? 2 : 1;   // slot rows per thread
    __shared__ int physs[DEC_CP];
    __shared__ __align__(16) float qc[DEC_GMAX * D];
    __shared__ __align__(16) float qx[DEC_GMAX * D];
    __shared__ float kb[DEC_WCH][D + 1];
    __shared__ float vb[DEC_WCH][D + 1];
    __shared__ float sc[DEC_GMAX][DEC_WCH];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t L = min((int64_t)lens[s], maxp * BK);   // never index past the page table
    const float scale = scales[s];
    const int32_t *pt = ptab + s * maxp;
    if (z < gm.nsc) {
        // ------------------------------------------------ score chunk --------
        // thread (page p = tid / 4, slot tid % 4 [+ 4]); the summary rows are
        // loaded before the routing query is built so the latencies overlap
        const int64_t bmax = (L >= 1) ? cand_bmax(L - 1, BK, W) : 0;
        const int p = tid >> 2, sl = tid & 3;
        const int64_t blk = 1 + (int64_t)z * DEC_CP + p;
        const bool live = blk <= bmax;
        float srow[SR][D];
        if (live) {
            const int64_t phys = pt[blk];
            if (sl == 0) physs[p] = (int)phys;
#pragma unroll
            for (int r = 0; r < SR; ++r) {
                const int slot = sl + 4 * r;
                if (slot < M) {
                    const typename St<DT>::T *src = sp + ((phys * Hkv + g) * M + slot) * D;
#pragma unroll
                    for (int c = 0; c < D / 8; ++c) {
                        float y[8];
                        ld8<DT>(src + 8 * c, y);
#pragma unroll
                        for (int e = 0; e < 8; ++e) srow[r][8 * c + e] = y[e];
                    }
                }
            }
        }
        dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc, nullptr, cosT, sinT, 0);
        if (tid < D) {   // routing query: sequential head sum, rounded (summarizer.py:50-54)
            float a = qc[tid];
            for (int h = 1; h < G; ++h) a = a + qc[h * D + tid];
            qx[tid] = St<DT>::rnd(a);
        }
        __syncthreads();
        float best = -INFINITY;
#pragma unroll
        for (int r = 0; r < SR; ++r) {
            const int slot = sl + 4 * r;
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < D; ++t) acc = fmaf(qx[t], srow[r][t], acc);
            if (slot < M) best = (acc > best) ? acc : best;
        }
        // max over the lanes of a page: the max is exact in any order
        const float o1 = __shfl_xor(best, 1, 64);
        best = (o1 > best) ? o1 : best;
        const float o2 = __shfl_xor(best, 2, 64);
        best = (o2 > best) ? o2 : best;
        if (sl == 0) sc[0][p] = live ? best * scale : -INFINITY;
        __syncthreads();
        if (tid < DEC_CP) {
            const float vv = sc[0][tid];
            const int id = (int)(1 + (int64_t)z * DEC_CP + tid);
            int rank = 0;
#pragma unroll 16
            for (int o = 0; o < DEC_CP; ++o) {
                const float vo = sc[0][o];
                const int io = (int)(1 + (int64_t)z * DEC_CP + o);
                rank += ((vo > vv) || (vo == vv && io < id)) ? 1 : 0;
            }
            if (rank < K) {
                const int64_t o = (((int64_t)s * Hkv + g) * gm.nsc + z) * K + rank;
                ws_val[o] = vv;
                ws_idx[o] = (vv == -INFINITY) ? -1 : id;
                ws_phys[o] = (vv == -INFINITY) ? -1 : physs[tid];
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
    float *part = ws_part + (((int64_t)s * Hkv + g) * gm.npart + wc) * G * (D + 2);
    if (nw == 0 && ns == 0) {
        empty_partial(part, G, D + 2);
        return;
    }
    // every global load of the chunk is issued before any compute: thread
    // (row r, pair-chunk hc) loads key chunks hc and hc + D/16 (the RoPE
    // partners), the same value chunks and the matching cos/sin entries
    constexpr int HC = D / 16;                        // pair-chunks per row
    constexpr int PER = (DEC_WCH * HC + DEC_WG - 1) / DEC_WG;
    const int64_t pg0 = pt[k0 / BK];
    const int64_t pg1 = pt[(k1 >= k0 ? k1 : k0) / BK];
    float kx[PER][2][8], vx[PER][2][8], cx[PER][2][8], sx[PER][2][8];
#pragma unroll
    for (int c = 0; c < PER; ++c) {
        const int e = tid + c * DEC_WG;
        const int r = e / HC, hc = e % HC;
        if (r < nw) {
            const int64_t j = k0 + r;
            const int64_t page = (j / BK == k0 / BK) ? pg0 : pg1;
            const int64_t off = (page * Hkv + g) * BK * D + (j % BK) * D;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int t0 = 8 * hc + u * (D / 2);
                ld8<DT>(kcp + off + t0, kx[c][u]);
                ld8<DT>(vp + off + t0, vx[c][u]);
                ld8<0>(cosT + j * D + t0, cx[c][u]);
                ld8<0>(sinT + j * D + t0, sx[c][u]);
            }
        }
    }
    dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc, qx, cosT, sinT, i);
    // RoPE of the window keys in registers (apply_rope's roundings), to LDS
#pragma unroll
    for (int c = 0; c < PER; ++c) {
        const int e = tid + c * DEC_WG;
        const int r = e / HC, hc = e % HC;
        if (r < nw) {
#pragma unroll
            for (int e2 = 0; e2 < 8; ++e2) {
                const float x0 = kx[c][0][e2], x1 = kx[c][1][e2];
                const float c0 = St<DT>::rnd(cx[c][0][e2]), s0 = St<DT>::rnd(sx[c][0][e2]);
                const float c1 = St<DT>::rnd(cx[c][1][e2]), s1 = St<DT>::rnd(sx[c][1][e2]);
                kb[r][8 * hc + e2] = St<DT>::rnd(St<DT>::rnd(x0 * c0) + St<DT>::rnd(-x1 * s0));
                kb[r][8 * hc + e2 + D / 2] = St<DT>::rnd(St<DT>::rnd(x1 * c1) + St<DT>::rnd(x0 * s1));
                vb[r][8 * hc + e2] = vx[c][0][e2];
                vb[r][8 * hc + e2 + D / 2] = vx[c][1][e2];
            }
        }
    }
    __syncthreads();
    if (ns == 0) {
        dec_partial<D>(qx, kb, vb, sc, G, nw, scale, part);
        return;
    }
    // chunk 0 with sinks: the window's and the sinks' partials, merged
    __shared__ float wpart[DEC_GMAX * (D + 2)];
    __shared__ float spart[DEC_GMAX * (D + 2)];
    if (nw > 0) dec_partial<D>(qx, kb, vb, sc, G, nw, scale, wpart);
    else {
        empty_partial(wpart, G, D + 2);
        __syncthreads();
    }
    for (int e = tid; e < ns * D; e += DEC_WG) {
        const int r = e / D, t = e % D;
        const int64_t off = ((int64_t)pt[0] * Hkv + g) * BK * D + (int64_t)r * D + t;
        kb[r][t] = St<DT>::ld(kcp, off);
        vb[r][t] = St<DT>::ld(vp, off);
    }
    __syncthreads();
    dec_partial<D>(qc, kb, vb, sc, G, ns, scale, spart);
    for (int e = tid; e < G * (D + 2); e += DEC_WG) {
        const int h = e / (D + 2), t = e % (D + 2);
        const float *pw = wpart + h * (D + 2);
        const float *ps = spart + h * (D + 2);
        const float m1 = pw[D], m2 = ps[D];
        const float m = fmaxf(m1, m2);
        const float w1 = (m1 == -INFINITY) ? 0.0f : expf(m1 - m);
        const float w2 = (m2 == -INFINITY) ? 0.0f : expf(m2 - m);
        float v;
        if (t < D) v = pw[t] * w1 + ps[t] * w2;
        else if (t == D) v = m;
        else v = pw[D + 1] * w1 + ps[D + 1] * w2;
        part[e] = v;
    }
}

template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d2_kernel(
    const typename St<DT>::T *__restrict__ q, const float *__restrict__ qgain, float eps,
    const typename St<DT>::T *__restrict__ kcp, const typename St<DT>::T *__restrict__ vp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ scales, int Hq, int Hkv, int K, DecGeom gm,
    const float *__restrict__ ws_val, const int32_t *__restrict__ ws_idx,
    const int32_t *__restrict__ ws_phys, float *__restrict__ ws_part, int32_t *__restrict__ sel_idx,
    int32_t *__restrict__ sel_cnt) {
    constexpr int BK = 64;
    __shared__ __align__(16) float qc[DEC_GMAX * D];
    __shared__ float ev[2048];
    __shared__ int ei[2048];
    __shared__ int pick, pickphys;
    __shared__ int nvalid;
    __shared__ float kb[BK][D + 1];
    __shared__ float vb[BK][D + 1];
    __shared__ float sc[DEC_GMAX][DEC_WCH];
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
    dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc, nullptr, nullptr, nullptr, 0);
    __syncthreads();
    // global rank of each valid entry: its position in its own (sorted) chunk
    // list plus, for every other chunk, the number of entries ordered before
    // it under (score desc, block asc) -- a binary search per chunk
    for (int e = tid; e < E; e += DEC_WG) {
        const float v = ev[e];
        const int id = ei[e];
        if (v == -INFINITY) continue;
        const int ce = e / K;
        int rank = e % K;
        for (int c = 0; c < gm.nsc; ++c) {
            if (c == ce) continue;
            int lo = 0, hi = K;               // first position not ordered before (v, id)
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                const float vo = ev[c * K + mid];
                const int io = ei[c * K + mid];
                const bool before = vo != -INFINITY && ((vo > v) || (vo == v && io < id));
                if (before) lo = mid + 1;
                else hi = mid;
            }
            rank += lo;
        }
        if (rank == r) {
            pick = id;
            pickphys = ws_phys[base + e];
        }
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
        empty_partial(part, G, D + 2);
        return;
    }
    const int64_t phys = pickphys;
    const typename St<DT>::T *kbase = kcp + (phys * Hkv + g) * BK * D;
    const typename St<DT>::T *vbase = vp + (phys * Hkv + g) * BK * D;
    constexpr int CH = D / 8;
    constexpr int PER = (BK * CH + DEC_WG - 1) / DEC_WG;
    float kx[PER][8], vx[PER][8];
#pragma unroll
    for (int c = 0; c < PER; ++c) {
        const int e = tid + c * DEC_WG;
        if (e < BK * CH) {
            ld8<DT>(kbase + (int64_t)e * 8, kx[c]);
            ld8<DT>(vbase + (int64_t)e * 8, vx[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < PER; ++c) {
        const int e = tid + c * DEC_WG;
        if (e < BK * CH) {
            const int row = e / CH, ch = e % CH;
#pragma unroll
            for (int e2 = 0; e2 < 8; ++e2) {
                kb[row][8 * ch + e2] = kx[c][e2];
                vb[row][8 * ch + e2] = vx[c][e2];
            }
        }
    }
    __syncthreads();
    dec_partial<D>(qc, kb, vb, sc, G, BK, scale, part);
}

// LSE merge of the npart partial states of one (sequence, KV head): every
// partial maximum is loaded at once (one lane per partial), the weights go
// through LDS, then one thread per (head, d) sums the weighted numerators.
template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d3_kernel(const float *__restrict__ ws_part, int Hq,
                                                           int Hkv, DecGeom gm,
                                                           typename St<DT>::T *__restrict__ out) {
    __shared__ float wgt[DEC_GMAX][DEC_PMAX];
    __shared__ float den[DEC_GMAX];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int G = Hq / Hkv;
    const int np = gm.npart;
    const float *part = ws_part + ((int64_t)s * Hkv + g) * np * G * (D + 2);
    const int wv = tid / 64, ln = tid % 64;
    for (int h = wv; h < G; h += DEC_WG / 64) {
        float mloc = -INFINITY;
        float mc[2], lc[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = ln + 64 * u;
            mc[u] = (c < np) ? part[((int64_t)c * G + h) * (D + 2) + D] : -INFINITY;
            lc[u] = (c < np) ? part[((int64_t)c * G + h) * (D + 2) + D + 1] : 0.0f;
            mloc = fmaxf(mloc, mc[u]);
        }
        const float m = wave_max(mloc);
        float dsum = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = ln + 64 * u;
            const float w = (mc[u] == -INFINITY) ? 0.0f : expf(mc[u] - m);
            if (c < np) wgt[h][c] = w;
            dsum += w * lc[u];
        }
        dsum = wave_sum(dsum);
        if (ln == 0) den[h] = dsum;
    }
    __syncthreads();
    for (int e = tid; e < G * D; e += DEC_WG) {
        const int h = e / D, t = e % D;
        float num = 0.0f;
#pragma unroll 8
        for (int c = 0; c < np; ++c) num = fmaf(part[((int64_t)c * G + h) * (D + 2) + t], wgt[h][c], num);
        const float dd = den[h];
        St<DT>::st(out, ((int64_t)s * Hq + g * G + h) * D + t, dd > 0.0f ? num / dd : 0.0f);
    }
}

}  // namespace hba

using namespace hba;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static void ws_layout(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k, DecGeom gm,
                      size_t *off_val, size_t *off_idx, size_t *off_phys, size_t *off_part,
                      size_t *total) {
    size_t nsel = (size_t)Bd * Hkv * (gm.nsc > 0 ? gm.nsc : 1) * k;
    size_t G = (size_t)(Hq / Hkv);
    *off_val = 0;
    *off_idx = align256(nsel * 4);
    *off_phys = *off_idx + align256(nsel * 4);
    *off_part = *off_phys + align256(nsel * 4);
    *total = *off_part + align256((size_t)Bd * Hkv * gm.npart * G * (d + 2) * 4);
}

extern "C" int hba_decode_workspace_size(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k,
                                         int64_t Bk, int64_t W, int64_t max_len, size_t *bytes) {
    if (!bytes || Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || k < 1 || W < 1 || max_len < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || k > DEC_KMAX) return HBA_ERR_UNSUPPORTED;
    DecGeom gm = dec_geom(W, k, max_len);
    size_t a, b, c, e;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &a, &b, &c, &e, bytes);
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
    if (Hq / Hkv > DEC_GMAX || k > DEC_KMAX || !(m == 1 || m == 2 || m == 4 || m == 8))
        return HBA_ERR_UNSUPPORTED;
    if ((max_len + Bk - 1) / Bk > max_pages) return HBA_ERR_INVALID_ARG;
    if (Bd > 65535 || Hkv > 65535) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(q) || !abi::aligned16(kc_pages) || !abi::aligned16(v_pages) ||
        !abi::aligned16(summ_pages) || !abi::aligned16(cos_tab) || !abi::aligned16(sin_tab))
        return HBA_ERR_UNSUPPORTED;
    DecGeom gm = dec_geom(W, k, max_len);
    if ((int64_t)gm.nsc * k > 2048 || gm.npart > DEC_PMAX) return HBA_ERR_UNSUPPORTED;
    size_t ov, oi, oph, op, total;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &ov, &oi, &oph, &op, &total);
    if (ws_bytes < total) return HBA_ERR_INVALID_ARG;
    char *ws = (char *)workspace;
    float *wv = (float *)(ws + ov);
    int32_t *wi = (int32_t *)(ws + oi);
    int32_t *wph = (int32_t *)(ws + oph);
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
                       (int)k, gm, wv, wi, wph, wp)
#define HBA_D1M(DT, D)                     \
    do {                                   \
        if (m == 1) HBA_D1(DT, D, 1);      \
        else if (m == 2) HBA_D1(DT, D, 2); \
        else if (m == 4) HBA_D1(DT, D, 4); \
        else HBA_D1(DT, D, 8);             \
    } while (0)
#define HBA_D23(DT, D)                                                                            \
    do {                                                                                          \
        hipLaunchKernelGGL((decode_d2_kernel<DT, D>), g2, dim3(DEC_WG), 0, s,                       \
                           (const St<DT>::T *)q, q_gain, eps, (const St<DT>::T *)kc_pages,          \
                           (const St<DT>::T *)v_pages, page_table, max_pages, seq_lens, scales,    \
                           (int)Hq, (int)Hkv, (int)k, gm, wv, wi, wph, wp, sel_idx, sel_cnt);            \
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
