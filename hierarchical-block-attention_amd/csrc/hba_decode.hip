// Decode step over a paged KV cache.  The reference has no decode path; the
// step is defined as row L-1 of hba_attention_eval (src/hba/attention.py:
// 610-713) for a sequence of length L: flat top-k over the full pages before
// the window (route_topk's rule, :272-303), then one softmax over sinks,
// the RoPE window and the selected pages.
//
// Cache layout (page = 64 tokens of one sequence): kc_pages [P, Hkv, 64, d]
// (QKNorm'd NoPE keys), kr_pages [P, Hkv, 64, d] (the same keys rotated at
// their own positions, written once on append: a key's rotation does not
// depend on the query), v_pages [P, Hkv, d, 64] (values, d-major, so that the
// A operand of the P.V MFMA is one 16-byte load per lane), summ_pages
// [P, Hkv, m, d].
//
// The attended keys of a (sequence, KV head) are cut into page units: the
// window pages (page-aligned, masked to [max(S, L-W), L-1], rotated keys),
// one sink unit (page 0, keys < S) and the k routed pages.  Every unit yields
// a partial softmax state (O, m, l) per head.  Three launches:
//   D1  score chunks of 64 candidate pages: declared-order slot scores and
//       the chunk-local top-k; chunk 0 also writes the attention query
//       operands (QKNorm'd, and rotated at L-1) of (s, g) to the workspace;
//   D2  every attention unit: window and sink units directly; routed units
//       first merge the chunk top-k lists and take their pick;
//   D3  LSE merge of the partial states, one wave per (sequence, head).
// bf16 units run one per wave on MFMA (the G heads are the columns of a
// 16-wide tile: S^T = K.Q^T, softmax in registers, O^T = V^T.P^T, operands
// loaded straight from the cache into registers); fp32 units run one per
// workgroup with fp32 dot products through LDS.
#include <mutex>

#include "hba_common.h"
#include "hba_abi.h"

namespace hba {

constexpr int DEC_WG = 256;
constexpr int DEC_CP = 64;    // candidate pages per score chunk
constexpr int DEC_KMAX = 64;  // largest k
constexpr int DEC_GMAX = 8;   // largest group size
constexpr int DEC_PMAX = 128; // largest number of partial states
constexpr int DEC_QROWS = 16; // query operand rows per (seq, KV head) and kind
constexpr float DEC_LOG2E = 1.4426950408889634f;

typedef unsigned int u32x4d __attribute__((ext_vector_type(4)));

struct DecGeom {
    int nsc;       // score chunks
    int nwp;       // window page units; the sink unit is unit nwp
    int npart;     // partial states per (seq, KV head) = nwp + 1 + k
    int uwg;       // D2 workgroups (per seq, KV head) running window/sink units
    int upw;       // units per D2 workgroup: 4 (one per wave, MFMA) or 1
    int64_t lmax;  // longest sequence the geometry (and the RoPE tables) cover
};

__host__ __device__ inline DecGeom dec_geom(int64_t W, int64_t k, int64_t max_len, bool mfma) {
    DecGeom gm;
    int64_t bm = cand_bmax(max_len - 1, 64, W);
    gm.nsc = (int)((bm + DEC_CP - 1) / DEC_CP);
    gm.nwp = (int)((W + 63) / 64) + 1;   // W keys span at most ceil(W/64) + 1 pages
    gm.npart = gm.nwp + 1 + (int)k;
    gm.upw = mfma ? 4 : 1;
    gm.uwg = (gm.nwp + 1 + gm.upw - 1) / gm.upw;
    gm.lmax = max_len;
    return gm;
}

// Key range [lo, hi] and logical page of unit u (u < nwp: window page u;
// u == nwp: the sinks) of a sequence of length L; false if the unit is empty.
__device__ __forceinline__ bool dec_unit_range(int u, int64_t L, int S, int64_t W, int nwp,
                                               int64_t &lo, int64_t &hi, int64_t &page) {
    if (L < 1) return false;
    const int64_t i = L - 1;
    if (u == nwp) {
        page = 0;
        lo = 0;
        hi = (((int64_t)S < L) ? (int64_t)S : L) - 1;
        return hi >= 0;
    }
    const int64_t wbeg = ((int64_t)S > i - W + 1) ? (int64_t)S : i - W + 1;
    page = wbeg / 64 + u;
    lo = (wbeg > 64 * page) ? wbeg : 64 * page;
    hi = (i < 64 * page + 63) ? i : 64 * page + 63;
    return lo <= hi;
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

// A partial softmax state is one row of dec_prow(D) floats per head:
// O[0..D-1], m at D (natural-log logit units), l at D + 1, 2 pad floats
// (the row stride is a multiple of 16 bytes).
__host__ __device__ constexpr int dec_prow(int D) { return D + 4; }

// Partial state of a unit with no key: m = -inf, O = l = 0.
__device__ __forceinline__ void empty_partial(float *part, int G, int D, int tid, int nthr) {
    const int PR = dec_prow(D);
    for (int e = tid; e < G * PR; e += nthr) part[e] = ((e % PR) == D) ? -INFINITY : 0.0f;
}

// QKNorm'd query rows of the G heads of (s, g) into LDS (fp32): the rows
// are staged cooperatively, then one thread per head takes the sum of
// squares in the declared order (sequential FMA, as qknorm_row) and the
// scaling of the elements is spread over the workgroup; with qr_lds also
// their rotation at position `pos` (apply_rope's roundings).  Ends with a
// barrier.
template <int DT, int D>
__device__ __forceinline__ void dec_query(const typename St<DT>::T *q, const float *qgain, float eps,
                                          int64_t s, int g, int G, int Hq, float *qc_lds, float *qr_lds,
                                          const float *cosT, const float *sinT, int64_t pos) {
    __shared__ float rinv[DEC_GMAX];
    const int tid = threadIdx.x;
    const typename St<DT>::T *rows = q + ((int64_t)s * Hq + (int64_t)g * G) * D;
    for (int e = 8 * tid; e < G * D; e += 8 * DEC_WG) {
        float x[8];
        ld8<DT>(rows + e, x);
#pragma unroll
        for (int u = 0; u < 8; ++u) qc_lds[e + u] = x[u];
    }
    __syncthreads();
    if (qgain) {
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

// ---------------------------------------------------------- bf16 units ----
__device__ __forceinline__ bf16x8 dld_b8(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4d *>(p));
}

__device__ __forceinline__ bf16x8 dpack_b8(const float (&x)[8]) {
    u32x4d u;
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = (uint32_t)f2bf(x[2 * e]) | ((uint32_t)f2bf(x[2 * e + 1]) << 16);
    return __builtin_bit_cast(bf16x8, u);
}

// 8 values of keys k0..k0+7 with the keys outside [lo, hi] zeroed (cache rows
// past the sequence end may hold anything, and 0 * NaN would poison P.V).
__device__ __forceinline__ bf16x8 dld_b8_masked(const bf16_t *p, int64_t k0, int64_t lo, int64_t hi) {
    u32x4d u = *reinterpret_cast<const u32x4d *>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t a = k0 + 2 * e;
        const uint32_t m = ((a >= lo && a <= hi) ? 0x0000ffffu : 0u) |
                           ((a + 1 >= lo && a + 1 <= hi) ? 0xffff0000u : 0u);
        u[e] &= m;
    }
    return __builtin_bit_cast(bf16x8, u);
}

// Row r of M-tile mt of S^T holds key slot dperm_key(mt, r): the C layout of
// the score MFMA then equals the B layout of the P.V MFMA (keys 8*lg..8*lg+7
// of each 32-key half in one lane).
__device__ __forceinline__ int dperm_key(int mt, int r) {
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3);
}

// Cache operands of one page unit: K rows in the permuted S^T row order,
// V^T slices with the keys outside [lo, hi] zeroed when the unit is partial.
template <int D>
__device__ __forceinline__ void dec_unit_load(const bf16_t *kpage, const bf16_t *vpage, int64_t kbase,
                                              int64_t lo, int64_t hi, bf16x8 (&ka)[4][D / 32],
                                              bf16x8 (&va)[D / 16][2]) {
    const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
    const bool partial = lo > kbase || hi < kbase + 63;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int slot = dperm_key(mt, l16);
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) ka[mt][ks] = dld_b8(kpage + slot * D + 32 * ks + 8 * lg);
    }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
        const bf16_t *vr = vpage + (16 * dt + l16) * 64 + 8 * lg;
        if (partial) {
            va[dt][0] = dld_b8_masked(vr, kbase + 8 * lg, lo, hi);
            va[dt][1] = dld_b8_masked(vr + 32, kbase + 32 + 8 * lg, lo, hi);
        } else {
            va[dt][0] = dld_b8(vr);
            va[dt][1] = dld_b8(vr + 32);
        }
    }
}

// One page unit on MFMA (one wave): keys kbase..kbase+63, valid positions
// [lo, hi]; writes the partial state (O[G][D], m, l; m in natural-log logit
// units) to part.
template <int D>
__device__ __forceinline__ void dec_unit_mfma(const bf16x8 (&ka)[4][D / 32], const bf16x8 (&va)[D / 16][2],
                                              const bf16x8 (&qop)[D / 32], int64_t kbase, int64_t lo,
                                              int64_t hi, float scale, int G, float *part) {
    constexpr int NKS = D / 32;
    constexpr int NDT = D / 16;
    const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
    f32x4 Sa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
            Sa[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[mt][ks], qop[ks], Sa[mt], 0, 0, 0);
    }
    // Sa[mt][e] of lane (l16, lg): head l16, key kbase + 32*(mt>>1) + 8*lg + 4*(mt&1) + e
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t jj = kbase + 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
            if (jj >= lo && jj <= hi) tmax = fmaxf(tmax, Sa[mt][e]);
        }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnat = tmax * scale;                 // finite: the unit holds a valid key
    const float sl2 = scale * DEC_LOG2E, ml2 = mnat * DEC_LOG2E;
    float pk[2][8];
    float psum = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t jj = kbase + 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
            float p = (jj >= lo && jj <= hi) ? __builtin_amdgcn_exp2f(fmaf(Sa[mt][e], sl2, -ml2)) : 0.0f;
            p = rnd_bf16(p);                           // the weight P.V uses
            pk[mt >> 1][(mt & 1) * 4 + e] = p;
            psum += p;
        }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    const bf16x8 pb0 = dpack_b8(pk[0]), pb1 = dpack_b8(pk[1]);
    f32x4 O[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][0], pb0, O[dt], 0, 0, 0);
        O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][1], pb1, O[dt], 0, 0, 0);
    }
    // O[dt][e] of lane (l16, lg): head l16, d = 16*dt + 4*lg + e
    if (l16 < G) {
        float *ph = part + l16 * dec_prow(D);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            *reinterpret_cast<float4 *>(ph + 16 * dt + 4 * lg) = float4{O[dt][0], O[dt][1], O[dt][2], O[dt][3]};
        if (lg == 0) {
            ph[D] = mnat;
            ph[D + 1] = psum;
        }
    }
}

// ----------------------------------------------------------- fp32 units ----
// Stage one page into LDS (fp32): keys as rows, values transposed back to
// rows; rows outside [rlo, rhi] are zeroed.
template <int DT, int D>
__device__ __forceinline__ void dec_stage_page(const typename St<DT>::T *kpage,
                                               const typename St<DT>::T *vpage, float (*kb)[D + 1],
                                               float (*vb)[D + 1], int rlo, int rhi) {
    const int tid = threadIdx.x;
    for (int e = 8 * tid; e < 64 * D; e += 8 * DEC_WG) {
        const int r = e / D, t = e % D;
        float x[8];
        ld8<DT>(kpage + e, x);
        const bool ok = r >= rlo && r <= rhi;
#pragma unroll
        for (int u = 0; u < 8; ++u) kb[r][t + u] = ok ? x[u] : 0.0f;
    }
    for (int e = 8 * tid; e < 64 * D; e += 8 * DEC_WG) {   // vpage is [D][64]
        const int t = e / 64, r0 = e % 64;
        float x[8];
        ld8<DT>(vpage + e, x);
#pragma unroll
        for (int u = 0; u < 8; ++u) vb[r0 + u][t] = (r0 + u >= rlo && r0 + u <= rhi) ? x[u] : 0.0f;
    }
}

// Partial softmax state of G heads over rows [rlo, rhi] of a page held in
// LDS (kb, vb, fp32) for queries qv [G][D] in LDS; writes (O[G][D], m[G],
// l[G]) rows of dec_prow(D) floats to `part`.  Ends with a barrier.
template <int D>
__device__ __forceinline__ void dec_partial(const float *qv, float (*kb)[D + 1], float (*vb)[D + 1],
                                            float (*sc)[64], int G, int rlo, int rhi, float scale,
                                            float *part) {
    __shared__ float Mh[DEC_GMAX], Lh[DEC_GMAX];
    const int tid = threadIdx.x;
    for (int e = tid; e < G * 64; e += DEC_WG) {
        const int h = e / 64, r = e % 64;
        float a = -INFINITY;
        if (r >= rlo && r <= rhi) {
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
            for (int r = 0; r < 64; ++r) a = fmaf(sc[h][r], vb[r][t], a);
            v = a;
        } else {
            v = (t == D) ? Mh[h] : Lh[h];
        }
        part[h * dec_prow(D) + t] = v;
    }
    __syncthreads();
}

// ------------------------------------------------------------------ D1 ----
// Score chunk z of (s, g): thread (page p = tid / 4, slot tid % 4 [+ 4]); the
// summary rows are loaded before the routing query is built so that the
// latencies overlap.  Writes the chunk's top-K (score desc, page asc).
template <int DT, int D, int M>
__global__ __launch_bounds__(DEC_WG) void decode_d1_kernel(
    const typename St<DT>::T *__restrict__ q, const float *__restrict__ qgain, float eps,
    const typename St<DT>::T *__restrict__ sp, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const float *__restrict__ scales, int Hq, int Hkv, int64_t W, int K, DecGeom gm,
    float *__restrict__ ws_val, int32_t *__restrict__ ws_idx, int32_t *__restrict__ ws_phys,
    typename St<DT>::T *__restrict__ ws_q) {
    constexpr int BK = 64;
    constexpr int SR = (M > 4) ? 2 : 1;   // slot rows per thread
    __shared__ __align__(16) float qc[DEC_GMAX * D];
    __shared__ __align__(16) float qr[DEC_GMAX * D];
    __shared__ float qx[D];
    __shared__ float sc[DEC_CP];
    __shared__ int physs[DEC_CP];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    // never index past the page table or the RoPE tables
    const int64_t L = min(min((int64_t)lens[s], maxp * BK), gm.lmax);
    const float scale = scales[s];
    const int32_t *pt = ptab + s * maxp;
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
    // chunk 0 also leaves the attention query operands of (s, g) in the
    // workspace: QKNorm'd rows and their rotation at L-1, 16 rows per kind
    // (rows >= G zero), in the storage type
    const bool qout = z == 0 && L >= 1;
    dec_query<DT, D>(q, qgain, eps, s, g, G, Hq, qc, qout ? qr : nullptr, cosT, sinT, L - 1);
    if (qout) {
        typename St<DT>::T *dst = ws_q + ((int64_t)s * Hkv + g) * 2 * DEC_QROWS * D;
        for (int e = tid; e < DEC_QROWS * D; e += DEC_WG) {
            const bool hv = e < G * D;
            St<DT>::st(dst, e, hv ? qc[e] : 0.0f);
            St<DT>::st(dst, DEC_QROWS * D + e, hv ? qr[e] : 0.0f);
        }
    }
    if (gm.nsc == 0) return;   // launched for the query operands only
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
    if (sl == 0) sc[p] = live ? best * scale : -INFINITY;
    __syncthreads();
    if (tid < DEC_CP) {
        const float vv = sc[tid];
        const int id = (int)(1 + (int64_t)z * DEC_CP + tid);
        int rank = 0;
#pragma unroll 16
        for (int o = 0; o < DEC_CP; ++o) {
            const float vo = sc[o];
            rank += ((vo > vv) || (vo == vv && o < tid)) ? 1 : 0;
        }
        if (rank < K) {
            const int64_t o = (((int64_t)s * Hkv + g) * gm.nsc + z) * K + rank;
            ws_val[o] = vv;
            ws_idx[o] = (vv == -INFINITY) ? -1 : id;
            ws_phys[o] = (vv == -INFINITY) ? -1 : physs[tid];
        }
    }
}

// ------------------------------------------------------------------ D2 ----
// Workgroups z < uwg of (s, g) run the window and sink units; the others run
// the routed units (ranks r0 .. r0 + upw - 1), after merging the chunk top-K
// lists: an entry's global rank is its position in its own sorted list plus,
// for every other chunk, the number of entries ordered before it (binary
// search).  Rank 0's workgroup also writes sel_idx / sel_cnt.
template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d2_kernel(
    const typename St<DT>::T *__restrict__ ws_q, const typename St<DT>::T *__restrict__ kcp,
    const typename St<DT>::T *__restrict__ krp, const typename St<DT>::T *__restrict__ vp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ scales, int Hq, int Hkv, int S, int64_t W, int K, DecGeom gm,
    const float *__restrict__ ws_val, const int32_t *__restrict__ ws_idx,
    const int32_t *__restrict__ ws_phys, float *__restrict__ ws_part, int32_t *__restrict__ sel_idx,
    int32_t *__restrict__ sel_cnt) {
    constexpr int BK = 64;
    constexpr bool MF = DT == 1;
    constexpr int FR = MF ? 1 : 64;         // fp32 staging (unused on MFMA)
    constexpr int FQ = MF ? 1 : DEC_GMAX * D;
    __shared__ float ev[2048];
    __shared__ int ei[2048];
    __shared__ int pick[4], pickphys[4];
    __shared__ int nvalid;
    __shared__ __align__(16) float qc[FQ];
    __shared__ float kb[FR][D + 1];
    __shared__ float vb[FR][D + 1];
    __shared__ float sc[MF ? 1 : DEC_GMAX][64];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t L = min(min((int64_t)lens[s], maxp * BK), gm.lmax);
    const float scale = scales[s];
    const int32_t *pt = ptab + s * maxp;
    float *partsg = ws_part + ((int64_t)s * Hkv + g) * gm.npart * G * dec_prow(D);
    const int w = MF ? (tid >> 6) : 0;
    // query operands written by D1: [2][DEC_QROWS][D], NoPE rows then rotated rows
    const typename St<DT>::T *qsg = ws_q + ((int64_t)s * Hkv + g) * 2 * DEC_QROWS * D;
    const int lane = tid & 63, l16 = lane & 15, lg = lane >> 4;

    if (z < gm.uwg) {
        // ------------------------------------------ window / sink units -----
        const int u = z * gm.upw + w;
        if (u > gm.nwp) return;                        // past the sink unit (wave-uniform)
        float *part = partsg + (int64_t)u * G * dec_prow(D);
        int64_t lo, hi, page;
        const bool any = dec_unit_range(u, L, S, W, gm.nwp, lo, hi, page);
        const bool rope = u < gm.nwp;
        if constexpr (MF) {
            if (!any) {
                empty_partial(part, G, D, tid & 63, 64);
                return;
            }
            const int64_t phys = pt[page];
            bf16x8 ka[4][D / 32], va[D / 16][2], qop[D / 32];
            dec_unit_load<D>((const bf16_t *)(rope ? krp : kcp) + (phys * Hkv + g) * BK * D,
                             (const bf16_t *)vp + (phys * Hkv + g) * D * BK, 64 * page, lo, hi, ka, va);
            const bf16_t *qrow = (const bf16_t *)qsg + ((rope ? DEC_QROWS : 0) + l16) * D + 8 * lg;
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) qop[ks] = dld_b8(qrow + 32 * ks);
            dec_unit_mfma<D>(ka, va, qop, 64 * page, lo, hi, scale, G, part);
        } else {
            if (!any) {
                empty_partial(part, G, D, tid, DEC_WG);
                return;
            }
            const int rlo = (int)(lo - 64 * page), rhi = (int)(hi - 64 * page);
            const int64_t phys = pt[page];
            dec_stage_page<DT, D>((rope ? krp : kcp) + (phys * Hkv + g) * BK * D,
                                  vp + (phys * Hkv + g) * D * BK, kb, vb, rlo, rhi);
            for (int e = tid; e < G * D; e += DEC_WG) qc[e] = St<DT>::ld(qsg, (rope ? DEC_QROWS * D : 0) + e);
            __syncthreads();
            dec_partial<D>(qc, kb, vb, sc, G, rlo, rhi, scale, part);
        }
        return;
    }
    // ------------------------------------------------------ routed units ----
    const int r0 = (z - gm.uwg) * gm.upw;
    const int E = gm.nsc * K;
    const int64_t base = ((int64_t)s * Hkv + g) * gm.nsc * K;
    bf16x8 qop[D / 32];
    if constexpr (MF) {   // the query operand is independent of the pick: loaded first
        const bf16_t *qrow = (const bf16_t *)qsg + l16 * D + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) qop[ks] = dld_b8(qrow + 32 * ks);
    }
    if (tid < 4) {
        pick[tid] = -1;
        pickphys[tid] = -1;
    }
    if (tid == 0) nvalid = 0;
    for (int e = tid; e < E; e += DEC_WG) {
        ev[e] = ws_val[base + e];
        ei[e] = ws_idx[base + e];
    }
    __syncthreads();
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
        if (rank >= r0 && rank < r0 + gm.upw) {
            pick[rank - r0] = id;
            pickphys[rank - r0] = ws_phys[base + e];
        }
        if (r0 == 0 && rank < K) {
            if (sel_idx) sel_idx[((int64_t)s * Hkv + g) * K + rank] = id;
            atomicAdd(&nvalid, 1);
        }
    }
    __syncthreads();
    if (r0 == 0) {
        const int nv = nvalid;
        if (sel_idx)
            for (int e = nv + tid; e < K; e += DEC_WG) sel_idx[((int64_t)s * Hkv + g) * K + e] = -1;
        if (sel_cnt && tid == 0) sel_cnt[(int64_t)s * Hkv + g] = nv < K ? nv : K;
    }
    const int r = r0 + w;
    if (r >= K) return;                                // wave-uniform (MFMA) / uniform
    float *part = partsg + (int64_t)(gm.nwp + 1 + r) * G * dec_prow(D);
    const int blk = pick[w];
    const int64_t phys = pickphys[w];
    const bool ok = blk >= 1 && (int64_t)blk < maxp && phys >= 0;
    const int64_t kb0 = 64 * (int64_t)blk;
    if constexpr (MF) {
        if (!ok) {
            empty_partial(part, G, D, tid & 63, 64);
            return;
        }
        bf16x8 ka[4][D / 32], va[D / 16][2];
        dec_unit_load<D>((const bf16_t *)kcp + (phys * Hkv + g) * BK * D,
                         (const bf16_t *)vp + (phys * Hkv + g) * D * BK, kb0, kb0, kb0 + 63, ka, va);
        dec_unit_mfma<D>(ka, va, qop, kb0, kb0, kb0 + 63, scale, G, part);
    } else {
        if (!ok) {
            empty_partial(part, G, D, tid, DEC_WG);
            return;
        }
        dec_stage_page<DT, D>(kcp + (phys * Hkv + g) * BK * D, vp + (phys * Hkv + g) * D * BK, kb, vb, 0, 63);
        for (int e = tid; e < G * D; e += DEC_WG) qc[e] = St<DT>::ld(qsg, e);
        __syncthreads();
        dec_partial<D>(qc, kb, vb, sc, G, 0, 63, scale, part);
    }
}

// ------------------------------------------------------------------ D3 ----
// LSE merge of the npart partial states of one (sequence, head): one wave;
// lane c holds partials c and c + 64 for the maxima and weights, then lane t
// sums the weighted numerators of elements t (and t + 64), every load of the
// sum issued independently.
template <int DT, int D>
__global__ __launch_bounds__(64) void decode_d3_kernel(const float *__restrict__ ws_part, int Hq,
                                                       int Hkv, DecGeom gm,
                                                       typename St<DT>::T *__restrict__ out) {
    __shared__ float wgt[DEC_PMAX];
    const int ln = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int h = blockIdx.z;
    const int G = Hq / Hkv;
    const int np = gm.npart;
    constexpr int PR = dec_prow(D);
    const float *part = ws_part + ((int64_t)s * Hkv + g) * np * G * PR + (int64_t)h * PR;
    const int64_t cs = (int64_t)G * PR;               // stride between partials
    constexpr int TPL = D / 64;                       // elements per lane
    // up to NPR partials' numerators are loaded with the maxima, so that the
    // merge costs one memory round trip
    constexpr int NPR = 48;
    float pv[NPR][TPL];
    if (np <= NPR) {
#pragma unroll
        for (int c = 0; c < NPR; ++c)
#pragma unroll
            for (int e = 0; e < TPL; ++e) pv[c][e] = (c < np) ? part[c * cs + ln + 64 * e] : 0.0f;
    }
    float mc[2], lc[2];
    float mloc = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int c = ln + 64 * u;
        mc[u] = (c < np) ? part[c * cs + D] : -INFINITY;
        lc[u] = (c < np) ? part[c * cs + D + 1] : 0.0f;
        mloc = fmaxf(mloc, mc[u]);
    }
    const float m = wave_max(mloc);
    float dsum = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int c = ln + 64 * u;
        const float wv = (mc[u] == -INFINITY) ? 0.0f : expf(mc[u] - m);
        if (c < np) wgt[c] = wv;
        dsum += wv * lc[u];
    }
    dsum = wave_sum(dsum);
    __syncthreads();
    float num[TPL];
#pragma unroll
    for (int e = 0; e < TPL; ++e) num[e] = 0.0f;
    if (np <= NPR) {
#pragma unroll
        for (int c = 0; c < NPR; ++c) {
            if (c < np) {
                const float wv = wgt[c];
#pragma unroll
                for (int e = 0; e < TPL; ++e) num[e] = fmaf(pv[c][e], wv, num[e]);
            }
        }
    } else {
#pragma unroll 8
        for (int c = 0; c < np; ++c) {
            const float wv = wgt[c];
#pragma unroll
            for (int e = 0; e < TPL; ++e) num[e] = fmaf(part[c * cs + ln + 64 * e], wv, num[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < TPL; ++e)
        St<DT>::st(out, ((int64_t)s * Hq + g * G + h) * D + ln + 64 * e, dsum > 0.0f ? num[e] / dsum : 0.0f);
}

}  // namespace hba

using namespace hba;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace: chunk top-k (values, pages, physical pages), query operands
// (fp32-sized so that one layout serves both dtypes), partial states.
static void ws_layout(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k, DecGeom gm,
                      size_t *off_val, size_t *off_idx, size_t *off_phys, size_t *off_q,
                      size_t *off_part, size_t *total) {
    size_t nsel = (size_t)Bd * Hkv * (gm.nsc > 0 ? gm.nsc : 1) * k;
    size_t G = (size_t)(Hq / Hkv);
    *off_val = 0;
    *off_idx = align256(nsel * 4);
    *off_phys = *off_idx + align256(nsel * 4);
    *off_q = *off_phys + align256(nsel * 4);
    *off_part = *off_q + align256((size_t)Bd * Hkv * 2 * DEC_QROWS * d * 4);
    *total = *off_part + align256((size_t)Bd * Hkv * gm.npart * G * dec_prow((int)d) * 4);
}

extern "C" int hba_decode_workspace_size(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k,
                                         int64_t Bk, int64_t W, int64_t max_len, size_t *bytes) {
    if (!bytes || Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || k < 1 || W < 1 || max_len < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || k > DEC_KMAX) return HBA_ERR_UNSUPPORTED;
    DecGeom gm = dec_geom(W, k, max_len, false);   // the layout does not depend on the unit mapping
    size_t a, b, c, e, f;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &a, &b, &c, &e, &f, bytes);
    return HBA_OK;
}

// The decode step on a given workspace; scratch_max > 0 marks the
// no-allocation entry point, whose workspace is the fixed scratch array
// (a request that does not fit it is HBA_ERR_SCRATCH).
static int decode_fwd_ws(int dtype, const void *q, const float *q_gain, float eps, const void *kc_pages,
                         const void *kr_pages, const void *v_pages, const void *summ_pages,
                         const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                         const float *cos_tab, const float *sin_tab, const float *scales, int64_t Bd,
                         int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t S, int64_t W, int64_t Bk,
                         int64_t k, int64_t max_len, void *workspace, size_t ws_bytes, size_t scratch_max,
                         void *out, int32_t *sel_idx, int32_t *sel_cnt, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !kc_pages || !kr_pages || !v_pages || !summ_pages || !page_table || !seq_lens ||
        !cos_tab || !sin_tab || !scales || !workspace || !out)
        return HBA_ERR_INVALID_ARG;
    if (Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || W < 1 || S < 0 || k < 1 || max_len < 1 ||
        max_pages < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || S > Bk) return HBA_ERR_UNSUPPORTED;
    if (Hq / Hkv > DEC_GMAX || k > DEC_KMAX || !(m == 1 || m == 2 || m == 4 || m == 8))
        return HBA_ERR_UNSUPPORTED;
    if ((max_len + Bk - 1) / Bk > max_pages) return HBA_ERR_INVALID_ARG;
    if (Bd > 65535 || Hkv > 65535) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(q) || !abi::aligned16(kc_pages) || !abi::aligned16(kr_pages) ||
        !abi::aligned16(v_pages) || !abi::aligned16(summ_pages) || !abi::aligned16(cos_tab) ||
        !abi::aligned16(sin_tab))
        return HBA_ERR_UNSUPPORTED;
    const bool mf = dtype == HBA_DTYPE_BF16;   // bf16: one unit per wave on MFMA
    DecGeom gm = dec_geom(W, k, max_len, mf);
    if ((int64_t)gm.nsc * k > 2048 || gm.npart > DEC_PMAX) return HBA_ERR_UNSUPPORTED;
    size_t ov, oi, oph, oq, op, total;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &ov, &oi, &oph, &oq, &op, &total);
    if (scratch_max && total > scratch_max) return HBA_ERR_SCRATCH;
    if (ws_bytes < total) return HBA_ERR_INVALID_ARG;
    char *ws = (char *)workspace;
    float *wv = (float *)(ws + ov);
    int32_t *wi = (int32_t *)(ws + oi);
    int32_t *wph = (int32_t *)(ws + oph);
    void *wq = (void *)(ws + oq);
    float *wp = (float *)(ws + op);
    hipStream_t s = (hipStream_t)stream;
    const int G = (int)(Hq / Hkv);
    dim3 g1((unsigned)Bd, (unsigned)Hkv, (unsigned)(gm.nsc > 0 ? gm.nsc : 1));
    dim3 g2((unsigned)Bd, (unsigned)Hkv, (unsigned)(gm.uwg + (k + gm.upw - 1) / gm.upw));
    dim3 g3((unsigned)Bd, (unsigned)Hkv, (unsigned)G);
#define HBA_D1(DT, D, M)                                                                          \
    hipLaunchKernelGGL((decode_d1_kernel<DT, D, M>), g1, dim3(DEC_WG), 0, s,                        \
                       (const St<DT>::T *)q, q_gain, eps, (const St<DT>::T *)summ_pages,            \
                       page_table, max_pages, seq_lens, cos_tab, sin_tab, scales, (int)Hq,         \
                       (int)Hkv, W, (int)k, gm, wv, wi, wph, (St<DT>::T *)wq)
#define HBA_D1M(DT, D)                                   \
    do {                                                 \
        if (m == 1) HBA_D1(DT, D, 1);                    \
        else if (m == 2) HBA_D1(DT, D, 2);               \
        else if (m == 4) HBA_D1(DT, D, 4);               \
        else HBA_D1(DT, D, 8);                           \
    } while (0)
#define HBA_D23(DT, D)                                                                            \
    do {                                                                                          \
        hipLaunchKernelGGL((decode_d2_kernel<DT, D>), g2, dim3(DEC_WG), 0, s,                       \
                           (const St<DT>::T *)wq, (const St<DT>::T *)kc_pages,                      \
                           (const St<DT>::T *)kr_pages, (const St<DT>::T *)v_pages, page_table,     \
                           max_pages, seq_lens, scales, (int)Hq, (int)Hkv, (int)S, W, (int)k, gm,  \
                           wv, wi, wph, wp, sel_idx, sel_cnt);                                      \
        hipLaunchKernelGGL((decode_d3_kernel<DT, D>), g3, dim3(64), 0, s, wp, (int)Hq, (int)Hkv,    \
                           gm, (St<DT>::T *)out);                                                   \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_D1M);
    HBA_DISPATCH_DT_D(dtype, d, HBA_D23);
#undef HBA_D1
#undef HBA_D1M
#undef HBA_D23
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_decode_fwd(int dtype, const void *q, const float *q_gain, float eps,
                              const void *kc_pages, const void *kr_pages, const void *v_pages,
                              const void *summ_pages, const int32_t *page_table, int64_t max_pages,
                              const int32_t *seq_lens, const float *cos_tab, const float *sin_tab,
                              const float *scales, int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d,
                              int64_t m, int64_t S, int64_t W, int64_t Bk, int64_t k, int64_t max_len,
                              void *workspace, size_t ws_bytes, void *out, int32_t *sel_idx,
                              int32_t *sel_cnt, void *stream) {
    return decode_fwd_ws(dtype, q, q_gain, eps, kc_pages, kr_pages, v_pages, summ_pages, page_table, max_pages,
                         seq_lens, cos_tab, sin_tab, scales, Bd, Hq, Hkv, d, m, S, W, Bk, k, max_len, workspace,
                         ws_bytes, 0, out, sel_idx, sel_cnt, stream);
}

// ------------------------------------------------ no-allocation variant ----
// The decode workspace as a fixed device array, one copy per GPU the library
// runs on, held until the process ends.  In host code `scratch` names a
// host-side stand-in, never device memory: its device address on the current
// device comes from hipGetSymbolAddress, looked up once per device and kept
// in scratch_ptr.  Every call on a GPU shares that GPU's copy; the kernels
// write every workspace entry they read within the same call, so nothing is
// cleared between calls.  Calls that overlap on one GPU (different streams)
// race on it.
static __device__ __align__(256) char scratch[HBA_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void *scratch_ptr[kMaxDevices];   // device address of `scratch` per device, or null

int scratch_on_current_device(void **ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return HBA_ERR_DEVICE;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return HBA_ERR_DEVICE;
        scratch_ptr[dev] = p;
    }
    *ptr = scratch_ptr[dev];
    return HBA_OK;
}
}  // namespace

extern "C" int hba_decode_fwd_noalloc(int dtype, const void *q, const float *q_gain, float eps,
                                      const void *kc_pages, const void *kr_pages, const void *v_pages,
                                      const void *summ_pages, const int32_t *page_table, int64_t max_pages,
                                      const int32_t *seq_lens, const float *cos_tab, const float *sin_tab,
                                      const float *scales, int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d,
                                      int64_t m, int64_t S, int64_t W, int64_t Bk, int64_t k, int64_t max_len,
                                      void *out, int32_t *sel_idx, int32_t *sel_cnt, void *stream) {
    void *ws = nullptr;
    const int st = scratch_on_current_device(&ws);
    if (st) return st;
    return decode_fwd_ws(dtype, q, q_gain, eps, kc_pages, kr_pages, v_pages, summ_pages, page_table, max_pages,
                         seq_lens, cos_tab, sin_tab, scales, Bd, Hq, Hkv, d, m, S, W, Bk, k, max_len, ws,
                         (size_t)HBA_DECODE_SCRATCH_BYTES, (size_t)HBA_DECODE_SCRATCH_BYTES, out, sel_idx,
                         sel_cnt, stream);
}
