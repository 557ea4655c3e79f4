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
// a partial softmax state (O, m, l) per head.
//
// bf16: one launch (decode_fused_kernel).  Per (s, g), score workgroups take
// chunks of candidate pages (declared-order slot scores, chunk-local top-k);
// the last of them to finish merges the chunk lists and runs the k routed
// pages, while window workgroups run the window and sink pages.  Units run
// one per wave on MFMA (the G heads are the columns of a 16-wide tile:
// S^T = K.Q^T, softmax in registers, O^T = V^T.P^T, operands loaded straight
// from the cache into registers); the last workgroup to finish merges the
// partial states into out.
//
// fp32: three launches, one unit per workgroup with fp32 dot products
// through LDS:
//   D1  score chunks of 64 candidate pages and the chunk-local top-k; chunk
//       0 also writes the attention query operands (QKNorm'd, and rotated at
//       L-1) of (s, g) to the workspace;
//   D2  every attention unit: window and sink units directly; routed units
//       first merge the chunk top-k lists and take their pick;
//   D3  LSE merge of the partial states, one wave per (sequence, head).
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "hba_common.h"
#include "hba_abi.h"

namespace hba {

constexpr int DEC_WG = 256;
constexpr int DEC_CP = 64;    // candidate pages per score chunk
constexpr int DEC_KMAX = 64;  // largest k
constexpr int DEC_GMAX = 16;  // largest group size (fp32 three-launch path)
constexpr int DEC_PMAX = 128; // largest number of partial states
constexpr int DEC_QROWS = 16; // query operand rows per (seq, KV head) and kind
constexpr float DEC_LOG2E = 1.4426950408889634f;

typedef unsigned int u32x4d __attribute__((ext_vector_type(4)));

// Geometry of the fp32 step (three launches, one unit per D2 workgroup).
struct DecGeom {
    int nsc;       // score chunks
    int nwp;       // window page units; the sink unit is unit nwp
    int npart;     // partial states per (seq, KV head) = nwp + 1 + k
    int uwg;       // D2 workgroups (per seq, KV head) running window/sink units: nwp + 1
    int64_t lmax;  // longest sequence the geometry (and the RoPE tables) cover
};

__host__ __device__ inline DecGeom dec_geom(int64_t W, int64_t k, int64_t max_len) {
    DecGeom gm;
    int64_t bm = cand_bmax(max_len - 1, 64, W);
    gm.nsc = (int)((bm + DEC_CP - 1) / DEC_CP);
    gm.nwp = (int)((W + 63) / 64) + 1;   // W keys span at most ceil(W/64) + 1 pages
    gm.npart = gm.nwp + 1 + (int)k;
    gm.uwg = gm.nwp + 1;
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

// 1 if entry (u, iu) ranks before (v, iv) under score desc, index asc; 0
// otherwise.  Bitwise, so that it compiles to selects (the short-circuit form
// becomes a branch per comparison).
__device__ __forceinline__ int rank_before(float u, int iu, float v, int iv) {
    return (int)(u > v) | ((int)(u == v) & (int)(iu < iv));
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

// Row r of M-tile mt of S^T holds key slot dperm_key(mt, r): the C layout of
// the score MFMA then equals the B layout of the P.V MFMA (keys 8*lg..8*lg+7
// of each 32-key half in one lane).
__device__ __forceinline__ int dperm_key(int mt, int r) {
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3);
}

// Cache operands of one page unit in the MFMA layouts (ka[mt][ks]: keys
// dperm_key(mt, l16), elements 32*ks + 8*lg ..; va[dt][h]: elements
// 16*dt + l16 of keys 32*h + 8*lg ..): the page layouts (page_key_off,
// page_val_off) put each operand of the wave in one contiguous 1 KB run.
// Plain loads only (no branch between them, so that all are in flight at
// once); dec_unit_core masks the keys outside the unit's range.
template <int D>
__device__ __forceinline__ void dec_unit_load(const bf16_t *kpage, const bf16_t *vpage,
                                              bf16x8 (&ka)[4][D / 32], bf16x8 (&va)[D / 16][2]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) ka[mt][ks] = dld_b8(kpage + ((mt * (D / 32) + ks) * 64 + lane) * 8);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int h = 0; h < 2; ++h) va[dt][h] = dld_b8(vpage + ((dt * 2 + h) * 64 + lane) * 8);
}

// Zero the V^T values of the keys outside page offsets [rlo, rhi] (cache
// rows past the sequence end may hold anything, and 0 * NaN would poison
// P.V).  Lane (l16, lg) holds page offsets 32*h + 8*lg .. +7 in va[dt][h].
template <int D>
__device__ __forceinline__ void dec_mask_v(bf16x8 (&va)[D / 16][2], int rlo, int rhi) {
    const int lg = (threadIdx.x & 63) >> 4;
    uint32_t m[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int a = 32 * h + 8 * lg + 2 * e;   // key offset within the page
            m[h][e] = ((a >= rlo && a <= rhi) ? 0x0000ffffu : 0u) | ((a + 1 >= rlo && a + 1 <= rhi) ? 0xffff0000u : 0u);
        }
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            u32x4d u = __builtin_bit_cast(u32x4d, va[dt][h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) u[e] &= m[h][e];
            va[dt][h] = __builtin_bit_cast(bf16x8, u);
        }
}

// One page unit on MFMA (one wave): keys kbase..kbase+63, valid positions
// [lo, hi] (at least one; the V values of the other keys are zeroed in va
// when the unit is partial).  Leaves the partial state in registers: O[dt][e]
// of lane (l16, lg) is head l16, element 16*dt + 4*lg + e; mnat (the
// maximum logit, natural-log units) and psum are that head's, in every lg.
template <int D>
__device__ __forceinline__ void dec_unit_core(const bf16x8 (&ka)[4][D / 32], bf16x8 (&va)[D / 16][2],
                                              const bf16x8 (&qop)[D / 32], int64_t kbase, int64_t lo,
                                              int64_t hi, float scale, f32x4 (&O)[D / 16], float &mnat,
                                              float &psum) {
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
    // Sa[mt][e] of lane (l16, lg): head l16, key kbase + 32*(mt>>1) + 8*lg + 4*(mt&1) + e;
    // the valid keys are page offsets rlo..rhi (a unit lies within one page)
    const int rlo = (int)(lo - kbase), rhi = (int)(hi - kbase);
    float tmax = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int jj = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
            if (jj >= rlo && jj <= rhi) tmax = fmaxf(tmax, Sa[mt][e]);
        }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    mnat = tmax * scale;                             // finite: the unit holds a valid key
    const float sl2 = scale * DEC_LOG2E, ml2 = mnat * DEC_LOG2E;
    float pk[2][8];
    psum = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int jj = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
            float p = (jj >= rlo && jj <= rhi) ? __builtin_amdgcn_exp2f(fmaf(Sa[mt][e], sl2, -ml2)) : 0.0f;
            p = rnd_bf16(p);                           // the weight P.V uses
            pk[mt >> 1][(mt & 1) * 4 + e] = p;
            psum += p;
        }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    const bf16x8 pb0 = dpack_b8(pk[0]), pb1 = dpack_b8(pk[1]);
    if (rlo > 0 || rhi < 63) dec_mask_v<D>(va, rlo, rhi);   // wave-uniform
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][0], pb0, O[dt], 0, 0, 0);
        O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[dt][1], pb1, O[dt], 0, 0, 0);
    }
}

// Fold one unit's partial state (O, m, l), m finite, into a running one
// (Oa, ma, la; ma = -inf while empty): the LSE merge, lane-local (every lane
// holds its own head's m and l).
template <int NDT>
__device__ __forceinline__ void dec_fold(f32x4 (&Oa)[NDT], float &ma, float &la, const f32x4 (&O)[NDT], float m,
                                         float l) {
    const float mn = fmaxf(ma, m);
    const float a = (ma == -INFINITY) ? 0.0f : exp2f((ma - mn) * DEC_LOG2E);
    const float b = exp2f((m - mn) * DEC_LOG2E);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) Oa[dt][e] = fmaf(O[dt][e], b, Oa[dt][e] * a);
    la = fmaf(l, b, la * a);
    ma = mn;
}

// ----------------------------------------------------------- fp32 units ----
// Stage one page into LDS (fp32): keys and values as token rows, rows
// outside [rlo, rhi] zeroed.  Each thread moves chunks of 8 consecutive
// storage elements (page_key_chunk / page_val_chunk name their place).
template <int DT, int D>
__device__ __forceinline__ void dec_stage_page(const typename St<DT>::T *kpage,
                                               const typename St<DT>::T *vpage, float (*kb)[D + 1],
                                               float (*vb)[D + 1], int rlo, int rhi) {
    const int tid = threadIdx.x;
    for (int c = tid; c < 8 * D; c += DEC_WG) {
        int j, t0;
        page_key_chunk(c, D, j, t0);
        float x[8];
        ld8<DT>(kpage + 8 * c, x);
        const bool ok = j >= rlo && j <= rhi;
#pragma unroll
        for (int u = 0; u < 8; ++u) kb[j][t0 + u] = ok ? x[u] : 0.0f;
    }
    for (int c = tid; c < 8 * D; c += DEC_WG) {
        int t, j0;
        page_val_chunk(c, t, j0);
        float x[8];
        ld8<DT>(vpage + 8 * c, x);
#pragma unroll
        for (int u = 0; u < 8; ++u) vb[j0 + u][t] = (j0 + u >= rlo && j0 + u <= rhi) ? x[u] : 0.0f;
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
            rank += rank_before(vo, o, vv, tid);
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
// fp32, one unit per workgroup.  Workgroups z < uwg of (s, g) run the window
// and sink units; workgroup uwg + r runs routed rank r, after merging the
// chunk top-K lists: an entry's global rank is its position in its own sorted
// list plus, for every other chunk, the number of entries ordered before it
// (binary search).  Rank 0's workgroup also writes sel_idx / sel_cnt.
template <int DT, int D>
__global__ __launch_bounds__(DEC_WG) void decode_d2_kernel(
    const typename St<DT>::T *__restrict__ ws_q, const typename St<DT>::T *__restrict__ kcp,
    const typename St<DT>::T *__restrict__ krp, const typename St<DT>::T *__restrict__ vp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ scales, int Hq, int Hkv, int S, int64_t W, int K, DecGeom gm,
    const float *__restrict__ ws_val, const int32_t *__restrict__ ws_idx,
    const int32_t *__restrict__ ws_phys, float *__restrict__ ws_part, int32_t *__restrict__ sel_idx,
    int32_t *__restrict__ sel_cnt) {
    static_assert(DT == 0, "bf16 decode runs in decode_fused_kernel");
    constexpr int BK = 64;
    __shared__ float ev[2048];
    __shared__ int ei[2048];
    __shared__ int pick[1], pickphys[1];
    __shared__ int nvalid;
    __shared__ __align__(16) float qc[DEC_GMAX * D];
    __shared__ float kb[64][D + 1];
    __shared__ float vb[64][D + 1];
    __shared__ float sc[DEC_GMAX][64];
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t L = min(min((int64_t)lens[s], maxp * BK), gm.lmax);
    const float scale = scales[s];
    const int32_t *pt = ptab + s * maxp;
    float *partsg = ws_part + ((int64_t)s * Hkv + g) * gm.npart * G * dec_prow(D);
    // query operands written by D1: [2][DEC_QROWS][D], NoPE rows then rotated rows
    const typename St<DT>::T *qsg = ws_q + ((int64_t)s * Hkv + g) * 2 * DEC_QROWS * D;

    if (z < gm.uwg) {
        // ------------------------------------------ window / sink units -----
        const int u = z;
        if (u > gm.nwp) return;                        // past the sink unit
        float *part = partsg + (int64_t)u * G * dec_prow(D);
        int64_t lo, hi, page;
        const bool any = dec_unit_range(u, L, S, W, gm.nwp, lo, hi, page);
        const bool rope = u < gm.nwp;
        if (!any) {
            empty_partial(part, G, D, tid, DEC_WG);
            return;
        }
        const int rlo = (int)(lo - 64 * page), rhi = (int)(hi - 64 * page);
        const int64_t phys = pt[page];
        dec_stage_page<DT, D>((rope ? krp : kcp) + (phys * Hkv + g) * BK * D, vp + (phys * Hkv + g) * D * BK,
                              kb, vb, rlo, rhi);
        for (int e = tid; e < G * D; e += DEC_WG) qc[e] = St<DT>::ld(qsg, (rope ? DEC_QROWS * D : 0) + e);
        __syncthreads();
        dec_partial<D>(qc, kb, vb, sc, G, rlo, rhi, scale, part);
        return;
    }
    // ------------------------------------------------------ routed units ----
    const int r0 = z - gm.uwg;
    const int E = gm.nsc * K;
    const int64_t base = ((int64_t)s * Hkv + g) * gm.nsc * K;
    if (tid == 0) {
        pick[0] = -1;
        pickphys[0] = -1;
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
        const int ce = e / K;
        int rank = e % K;
        for (int c = 0; c < gm.nsc; ++c) {
            if (c == ce) continue;
            int lo = 0, hi = K;               // first position not ordered before (v, id)
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                const float vo = ev[c * K + mid];
                const int io = ei[c * K + mid];
                const bool before = (int)(vo != -INFINITY) & rank_before(vo, io, v, id);
                if (before) lo = mid + 1;
                else hi = mid;
            }
            rank += lo;
        }
        if (rank == r0) {
            pick[0] = id;
            pickphys[0] = ws_phys[base + e];
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
    const int r = r0;
    if (r >= K) return;
    float *part = partsg + (int64_t)(gm.nwp + 1 + r) * G * dec_prow(D);
    const int blk = pick[0];
    const int64_t phys = pickphys[0];
    const bool ok = blk >= 1 && (int64_t)blk < maxp && phys >= 0;
    if (!ok) {
        empty_partial(part, G, D, tid, DEC_WG);
        return;
    }
    dec_stage_page<DT, D>(kcp + (phys * Hkv + g) * BK * D, vp + (phys * Hkv + g) * D * BK, kb, vb, 0, 63);
    for (int e = tid; e < G * D; e += DEC_WG) qc[e] = St<DT>::ld(qsg, e);
    __syncthreads();
    dec_partial<D>(qc, kb, vb, sc, G, 0, 63, scale, part);
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


// ============================================================================
// bf16: the step in one launch.
//
// Grid (Bd, Hkv, nz), DF_NT threads.  Workgroups z < nsg score chunk z of
// cpb = DF_NT / m candidate pages (one slot row per thread) and publish the
// chunk's top-K; the last of them to arrive at the (s, g) score counter
// merges the lists (and writes sel_idx / sel_cnt), then runs the K routed
// pages, ceil(K / 8) per wave.  Wave w of workgroup z >= nsg runs window /
// sink unit 8*(z - nsg) + w (if there is one): the score workgroups load only
// what the selection needs, so that their summaries do not queue behind the
// window pages, and the routing workgroup has no unit of its own between its
// merge and the routed pages.  Workgroup z folds its window units into one
// partial state per head (an LSE merge over its waves; none for a score
// workgroup) in workspace slot z, the
// routing workgroup its routed pages in slot nz (a slot of their own, so
// that the merge order does not depend on which workgroup routes: the step
// is deterministic); the last of the nz workgroups to arrive at the (s, g)
// merge counter merges the nz + 1 slots, in slot order, into out.  No
// workgroup waits for another (the last arrival does the dependent work), so
// any dispatch order completes.  The counters are zero on entry and the last
// arrival leaves them zero.  At 32 sequences of 16-32K tokens, 2 KV heads and
// m = 4 the grid is 448 workgroups (4 score + 3 unit workgroups per pair).
// ============================================================================
constexpr int DF_NT = 512;
constexpr int DF_NW = DF_NT / 64;
constexpr int DF_GMAX = 16;     // heads per KV head: the 16 columns of the MFMA tile
constexpr int DF_EMAX = 2048;   // chunk-list entries merged per (s, g)
constexpr int DF_HB = 8;        // heads per pass of the cross-wave merge

struct DecFGeom {
    int nsc;       // score chunks (0: no length up to lmax has a candidate page)
    int nsg;       // score workgroups per (s, g): max(nsc, 1)
    int cpb;       // candidate pages per chunk: DF_NT / m
    int nwp;       // window page units; unit nwp is the sinks
    int nz;        // workgroups per (s, g): nsg score workgroups, then ceil((nwp + 1) / DF_NW) unit workgroups
    int64_t bmax;  // largest candidate page of any length up to lmax
    int64_t lmax;  // longest sequence the geometry (and the RoPE tables) cover
};

__host__ __device__ inline DecFGeom dec_fgeom(int64_t W, int64_t m, int64_t max_len) {
    DecFGeom gm;
    gm.cpb = DF_NT / (int)m;
    gm.bmax = cand_bmax(max_len - 1, 64, W);
    gm.nsc = (int)((gm.bmax + gm.cpb - 1) / gm.cpb);
    gm.nsg = gm.nsc > 0 ? gm.nsc : 1;
    gm.nwp = (int)((W + 63) / 64) + 1;
    const int uwg = (gm.nwp + 1 + DF_NW - 1) / DF_NW;
    gm.nz = gm.nsg + uwg;
    gm.lmax = max_len;
    return gm;
}

// LDS of decode_fused_kernel: the query rows, then either the merge's chunk
// lists or the per-wave partial states (never live together).
template <int D>
struct DfSmem {
    static constexpr int LISTS = DF_EMAX * 3 * 4;
    static constexpr int PBUF = DF_NW * DF_HB * dec_prow(D) * 4;
    float qc[DF_GMAX * D];
    float qr[DF_GMAX * D];
    float qx[D];
    float sc[DF_NT];
    int physs[DF_NT];
    int pick[DEC_KMAX], pickp[DEC_KMAX];
    int nvalid, flag;
    alignas(16) char un[LISTS > PBUF ? LISTS : PBUF];
};

// Workspace entries that one workgroup writes and another reads in the same
// launch go through device-scope atomic stores and loads (relaxed): these
// are coherent across the XCDs' L2 caches by themselves (write-through
// stores, loads that do not hit a stale L2 line), so that no L2-wide
// write-back or invalidation (a device-scope fence) is needed.
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_dev(const int *p) {
    return __hip_atomic_load(const_cast<int *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One arrival of this workgroup at *ctr, which counts `target` arrivals per
// launch: true in the last one, which then reads (ld_dev) what every other
// arrival wrote (st_dev) before arriving, and resets the counter.  Each
// thread waits for its own stores to complete before the workgroup barrier
// that precedes the count; the readers' loads follow the count.
__device__ __forceinline__ bool dec_arrive(int *ctr, int target, int *flag) {
    __builtin_amdgcn_s_waitcnt(0);   // vmcnt = expcnt = lgkmcnt = 0: this thread's stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        const int last = atomicAdd(ctr, 1) == target - 1;
        if (last) atomicExch(ctr, 0);
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

// Query operands of the G heads of (s, g) in LDS, fp32 values of bf16
// precision: qc = the QKNorm'd rows (QKNorm only with qk), and if qr is not
// null their rotation at the query position.  Thread tid holds elements
// 8*tid .. 8*tid+7 of the [G][D] rows in x (hx), its head's gain in gn and,
// to rotate, the cos/sin values of those elements in cs/sn: all loaded by
// the caller, early.  The sum of squares runs in the declared order
// (sequential FMA over the row, as qknorm_row) as a chain through the D/8
// lanes that hold a row: lane j of a row continues the sum of lane j-1
// (row_shr:1 DPP move) over its 8 elements.  The rotation rounds as
// rope_row.  Ends with a barrier.
template <int D>
__device__ __forceinline__ void df_query(float (&x)[8], bool hx, bool qk, float gn, float eps, float *qc,
                                         float *qr, const float (&cs)[8], const float (&sn)[8]) {
    constexpr int TPH = D / 8;   // lanes per row: 8 or 16, inside one 16-lane DPP row
    const int tid = threadIdx.x;
    const int e0 = 8 * tid;
    if (qk) {
        const int j = tid % TPH;
        float run = 0.0f;
#pragma unroll
        for (int step = 0; step < TPH; ++step) {
            const float in = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, run), 0x111, 0xf, 0xf, false));
            if (j == step) {
                float a = (j == 0) ? 0.0f : in;
#pragma unroll
                for (int u = 0; u < 8; ++u) a = fmaf(x[u], x[u], a);
                run = a;
            }
        }
        const float ss = __shfl(run, (tid & 63) | (TPH - 1), 64);   // the row's last lane
        float ms = ss / (float)D;
        if (ms < eps) ms = eps;
        const float r = sqrtf(ms);
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = rnd_bf16((x[u] / r) * gn);
    }
    if (hx)
#pragma unroll
        for (int u = 0; u < 8; ++u) qc[e0 + u] = x[u];
    __syncthreads();
    if (qr) {
        if (hx) {   // the 8 partner elements (rotate-half) lie in the other half of the row
            const int h = e0 / D, t0 = e0 % D;
            const bool lo_half = t0 < D / 2;
            const float *pr = qc + h * D + (lo_half ? t0 + D / 2 : t0 - D / 2);
            const float4 pa = *reinterpret_cast<const float4 *>(pr);
            const float4 pb = *reinterpret_cast<const float4 *>(pr + 4);
            const float part[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float rot = lo_half ? -part[u] : part[u];
                qr[e0 + u] = rnd_bf16(rnd_bf16(x[u] * rnd_bf16(cs[u])) + rnd_bf16(rot * rnd_bf16(sn[u])));
            }
        }
        __syncthreads();
    }
}

// This lane's MFMA query operand (B of S^T = K.Q^T: head l16, elements
// 32*ks + 8*lg .. +7) from rows [G][D] in LDS; heads >= G are zero.
template <int D>
__device__ __forceinline__ void df_qop(const float *rows, int G, bf16x8 (&qop)[D / 32]) {
    const int lane = threadIdx.x & 63, l16 = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (l16 < G) ? rows[l16 * D + 32 * ks + 8 * lg + e] : 0.0f;
        qop[ks] = dpack_b8(v);
    }
}

// Fold the waves' running partial states (Oa, ma, la: lane (l16, lg) holds
// head l16's elements 16*dt + 4*lg ..) into one state per head (an LSE merge
// in wave order, through LDS pbuf) and write it to slot [G][dec_prow(D)]
// with device-scope stores.  Called by the whole workgroup.
template <int D>
__device__ __forceinline__ void df_fold_slot(const f32x4 (&Oa)[D / 16], float ma, float la, float *pbuf, int G,
                                             float *slot) {
    constexpr int NDT = D / 16, PR = dec_prow(D);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    for (int hc = 0; hc < G; hc += DF_HB) {
        __syncthreads();   // the region's earlier readers are done
        const int hh = l16 - hc;
        if (l16 < G && hh >= 0 && hh < DF_HB) {
            float *dst = pbuf + (w * DF_HB + hh) * PR;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                *reinterpret_cast<float4 *>(dst + 16 * dt + 4 * lg) = float4{Oa[dt][0], Oa[dt][1], Oa[dt][2], Oa[dt][3]};
            if (lg == 0) {
                dst[D] = ma;
                dst[D + 1] = la;
            }
        }
        __syncthreads();
        for (int e = tid; e < DF_HB * D; e += DF_NT) {
            const int hb = e / D, t = e % D, h = hc + hb;
            if (h >= G) continue;
            float mx = -INFINITY;
#pragma unroll
            for (int ww = 0; ww < DF_NW; ++ww) mx = fmaxf(mx, pbuf[(ww * DF_HB + hb) * PR + D]);
            float o = 0.0f, l = 0.0f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int ww = 0; ww < DF_NW; ++ww) {
                    const float *src = pbuf + (ww * DF_HB + hb) * PR;
                    const float mw = src[D];
                    if (mw == -INFINITY) continue;
                    const float a = exp2f((mw - mx) * DEC_LOG2E);
                    o = fmaf(src[t], a, o);
                    l = fmaf(src[D + 1], a, l);
                }
            }
            float *dst = slot + (int64_t)h * PR;
            st_dev(dst + t, o);
            if (t == 0) {
                st_dev(dst + D, mx);
                st_dev(dst + D + 1, l);
            }
        }
    }
}

template <int D, int M>
__global__ __launch_bounds__(DF_NT) void decode_fused_kernel(
    const bf16_t *__restrict__ q, const float *__restrict__ qgain, float eps, const bf16_t *__restrict__ kcp,
    const bf16_t *__restrict__ krp, const bf16_t *__restrict__ vp, const bf16_t *__restrict__ sp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ cosT, const float *__restrict__ sinT, const float *__restrict__ scales, int Hq,
    int Hkv, int S, int64_t W, int K, DecFGeom gm, int *__restrict__ ctr, float *__restrict__ ws_val,
    int32_t *__restrict__ ws_idx, int32_t *__restrict__ ws_phys, float *__restrict__ ws_part,
    bf16_t *__restrict__ out, int32_t *__restrict__ sel_idx, int32_t *__restrict__ sel_cnt) {
    constexpr int BK = 64;
    constexpr int NKS = D / 32, NDT = D / 16;
    constexpr int PR = dec_prow(D);
    constexpr int CPB = DF_NT / M;   // candidate pages per chunk (gm.cpb)
    __shared__ DfSmem<D> sm;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int z = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t sg = s * Hkv + g;
    const int32_t *pt = ptab + s * maxp;
    float *slots = ws_part + sg * (gm.nz + 1) * G * PR;   // window slots 0..nz-1, routed slot nz
    const bool scorer = z < gm.nsg;

    // The prologue's loads are unconditional and in the order of their use,
    // so that each wait leaves the later ones in flight (after a load under a
    // branch the compiler's wait before a later use is a full one).  A lane
    // with nothing to load reads a fixed valid location instead (the pool's
    // first page: cache hits after the first read).
    // 1. this thread's query elements 8*tid .. of the G rows of (s, g) (past
    //    the rows: the last 8 again) and their head's gain
    const int e0 = 8 * tid;
    const bool hx = e0 < G * D;
    const int ec = hx ? e0 : G * D - 8;
    const u32x4d xr = *reinterpret_cast<const u32x4d *>(q + (s * Hq + (int64_t)g * G) * D + ec);
    const float graw = *(qgain ? qgain + g * G + ec / D : scales + s);
    const float gn = qgain ? graw : 1.0f;
    // 2. the page-table entry of this thread's candidate page (any length's:
    //    inside the table whatever L is)
    const int p = tid / M, sl = tid % M;
    const int64_t blk = 1 + (int64_t)z * CPB + p;
    const int phys = pt[(scorer && blk <= gm.bmax) ? blk : 0];
    // never index past the page table or the RoPE tables
    const int64_t L = min(min((int64_t)lens[s], maxp * BK), gm.lmax);
    const float scale = scales[s];
    const int64_t bmax = (L >= 1) ? cand_bmax(L - 1, BK, W) : 0;
    const int nsc_s = (int)((bmax + CPB - 1) / CPB);   // this sequence's chunks
    // this wave's window / sink unit (unit workgroups z >= nsg only: the
    // score workgroups load just what the selection needs, and the routing
    // one goes from its merge straight to the routed pages)
    const int u = scorer ? gm.nwp + 1 : (z - gm.nsg) * DF_NW + w;
    int64_t lo = 0, hi = -1, page = 0;
    const bool any = u <= gm.nwp && dec_unit_range(u, L, S, W, gm.nwp, lo, hi, page);   // wave-uniform
    const bool rope = u < gm.nwp;
    // 3. the page-table entry of the wave's window page; cos/sin at L-1 of the
    //    query elements
    const bool live = scorer && blk <= bmax;
    const int64_t wph = pt[any ? page : 0];
    const int64_t crow = ((L >= 1) ? L - 1 : 0) * D + ec % D;
    float cs[8], sn[8];
    ld8<0>(cosT + crow, cs);
    ld8<0>(sinT + crow, sn);
    // 4. the summary row of the candidate page (the window page's keys and
    //    values are loaded after the scores)
    u32x4d srow[D / 8];
    const bf16_t *src = live ? sp + (((int64_t)phys * Hkv + g) * M + sl) * D : sp;
#pragma unroll
    for (int c = 0; c < D / 8; ++c) srow[c] = *reinterpret_cast<const u32x4d *>(src + 8 * c);
    const bf16_t *wk = any ? (rope ? krp : kcp) + (wph * Hkv + g) * BK * D : kcp;
    const bf16_t *wv = any ? vp + (wph * Hkv + g) * D * BK : vp;
    // the window page's operands, in flight during the scoring (ready when
    // the routing workgroup computes its window unit while its chunk-list
    // loads are in flight)
    bf16x8 ka[4][NKS], va[NDT][2];
    dec_unit_load<D>(wk, wv, ka, va);
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = hx ? __uint_as_float(xr[e] << 16) : 0.0f;
        x[2 * e + 1] = hx ? __uint_as_float(xr[e] & 0xffff0000u) : 0.0f;
    }
    df_query<D>(x, hx, qgain != nullptr, gn, eps, sm.qc, sm.qr, cs, sn);

    // The chunk list's stores complete at the arrival below; until then their
    // operands stay in registers (a register they read may not be reused
    // before the store completes, which would make the compiler wait for it
    // at the reuse).
    float *pub_v = ws_val;
    int32_t *pub_i = ws_idx, *pub_p = ws_phys;
    int pub_iv = 0, pub_pv = 0;
    float pub_vv = 0.0f;
    if (scorer) {
        // ------------------------------------------------ score chunk z ----
        if (tid < D) {   // routing query: sequential head sum, rounded (summarizer.py:50-54)
            float a = sm.qc[tid];
            for (int h = 1; h < G; ++h) a = a + sm.qc[h * D + tid];
            sm.qx[tid] = rnd_bf16(a);
        }
        __syncthreads();
        if (z < nsc_s) {
            float acc = 0.0f;   // declared order: sequential FMA over the elements
#pragma unroll
            for (int c0 = 0; c0 < D / 8; c0 += 4) {   // 32 query elements per LDS batch
                float4 qv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) qv[i] = *reinterpret_cast<const float4 *>(&sm.qx[8 * c0 + 4 * i]);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const uint32_t *sr = reinterpret_cast<const uint32_t *>(&srow[c0 + c]);
                    const float4 a = qv[2 * c], b = qv[2 * c + 1];
                    acc = fmaf(a.x, __uint_as_float(sr[0] << 16), acc);
                    acc = fmaf(a.y, __uint_as_float(sr[0] & 0xffff0000u), acc);
                    acc = fmaf(a.z, __uint_as_float(sr[1] << 16), acc);
                    acc = fmaf(a.w, __uint_as_float(sr[1] & 0xffff0000u), acc);
                    acc = fmaf(b.x, __uint_as_float(sr[2] << 16), acc);
                    acc = fmaf(b.y, __uint_as_float(sr[2] & 0xffff0000u), acc);
                    acc = fmaf(b.z, __uint_as_float(sr[3] << 16), acc);
                    acc = fmaf(b.w, __uint_as_float(sr[3] & 0xffff0000u), acc);
                }
            }
            float best = (acc > -INFINITY) ? acc : -INFINITY;
#pragma unroll
            for (int o = 1; o < M; o <<= 1) {   // max over a page's slots: exact in any order
                const float ot = __shfl_xor(best, o, 64);
                best = (ot > best) ? ot : best;
            }
            if (sl == 0) {
                sm.sc[p] = live ? best * scale : -INFINITY;
                sm.physs[p] = phys;
            }
            __syncthreads();
            if (tid < CPB) {   // rank in the chunk: score desc, page asc
                const float vv = sm.sc[tid];
                int rank = 0;
#pragma unroll
                for (int o0 = 0; o0 < CPB; o0 += 32) {   // 8 LDS reads in flight per batch
                    float4 v4[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v4[i] = *reinterpret_cast<const float4 *>(&sm.sc[o0 + 4 * i]);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int o = o0 + 4 * i;
                        rank += rank_before(v4[i].x, o, vv, tid);
                        rank += rank_before(v4[i].y, o + 1, vv, tid);
                        rank += rank_before(v4[i].z, o + 2, vv, tid);
                        rank += rank_before(v4[i].w, o + 3, vv, tid);
                    }
                }
                if (rank < K) {
                    const int64_t o = (sg * gm.nsc + z) * K + rank;
                    const bool dead = vv == -INFINITY;
                    pub_v = ws_val + o;
                    pub_i = ws_idx + o;
                    pub_p = ws_phys + o;
                    pub_iv = dead ? -1 : (int)(1 + (int64_t)z * CPB + tid);
                    pub_pv = dead ? -1 : sm.physs[tid];
                    pub_vv = vv;
                    st_dev(pub_v, pub_vv);
                    st_dev(pub_i, pub_iv);
                    st_dev(pub_p, pub_pv);
                }
            }
        }
    }

    // ------------------------------------------- the score counter ------
    asm volatile("" ::"v"(pub_v), "v"(pub_i), "v"(pub_p), "v"(pub_iv), "v"(pub_pv), "v"(pub_vv));
    const bool router = scorer && dec_arrive(ctr + sg, gm.nsg, &sm.flag);   // workgroup-uniform
    // The routing workgroup's chunk-list loads go out first; the window unit
    // computes while they are in flight.
    const int E = router ? nsc_s * K : 0;
    const int64_t lb = sg * gm.nsc * K;
    float lv[4];
    int li[4], lp[4];
    if (router) {   // E <= DF_EMAX = 4 * DF_NT
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = tid + r * DF_NT;
            const int64_t o = lb + (e < E ? e : 0);   // an entry of this (s, g) whatever e
            lv[r] = ld_dev(ws_val + o);
            li[r] = ld_dev(ws_idx + o);
            lp[r] = ld_dev(ws_phys + o);
        }
    }
    // --------------------------------------------- window / sink unit ------
    f32x4 Oa[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) Oa[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ma = -INFINITY, la = 0.0f;
    if (any) {
        bf16x8 qop[NKS];
        df_qop<D>(rope ? sm.qr : sm.qc, G, qop);
        f32x4 O[NDT];
        float mu, lu;
        dec_unit_core<D>(ka, va, qop, 64 * page, lo, hi, scale, O, mu, lu);
        dec_fold<NDT>(Oa, ma, la, O, mu, lu);
    }
    df_fold_slot<D>(Oa, ma, la, reinterpret_cast<float *>(sm.un), G, slots + (int64_t)z * G * PR);
    __syncthreads();   // the fold's LDS readers are done before the lists are staged there
    if (router) {
        // ---------------------------- merge of the chunk lists of (s, g) -----
        // The lists (sorted; ties by page) hold distinct pages, so an entry's
        // global rank is the number of live entries of all lists ordered
        // before it: 8 threads count an eighth of the entries each.
        float *ev = reinterpret_cast<float *>(sm.un);
        int *ei = reinterpret_cast<int *>(sm.un) + DF_EMAX;
        int *ep = reinterpret_cast<int *>(sm.un) + 2 * DF_EMAX;
        if (tid < K) {
            sm.pick[tid] = -1;
            sm.pickp[tid] = -1;
        }
        if (tid == 0) sm.nvalid = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = tid + r * DF_NT;
            if (e < E) {
                ev[e] = lv[r];
                ei[e] = li[r];
                ep[e] = lp[r];
            }
        }
        __syncthreads();
        for (int e0 = 0; e0 < E; e0 += DF_NT / 8) {
            const int e = e0 + tid / 8, part = tid % 8;
            const float v = (e < E) ? ev[e] : -INFINITY;
            const int id = (e < E) ? ei[e] : 0;
            int cnt = 0;
#pragma unroll 4
            for (int o = part; o < E; o += 8) {
                const float vo = ev[o];
                const int io = ei[o];
                cnt += (int)(vo != -INFINITY) & rank_before(vo, io, v, id);
            }
            cnt += __shfl_xor(cnt, 1, 64);
            cnt += __shfl_xor(cnt, 2, 64);
            cnt += __shfl_xor(cnt, 4, 64);
            if (part == 0 && v != -INFINITY && cnt < K) {
                sm.pick[cnt] = id;
                sm.pickp[cnt] = ep[e];
                atomicAdd(&sm.nvalid, 1);
            }
        }
        __syncthreads();
    }


    if (router) {
        // ------------------------------------ routed pages of (s, g) ---------
        bf16x8 qop[NKS];
        df_qop<D>(sm.qc, G, qop);
        // routed pages r = w, w + 8, ...: UB at a time, every load first (a
        // missing pick reads the pool's first page instead and is skipped).
        // One page at a time: two in flight per wave at d = 64 held 180
        // VGPRs against 152 and measured 35.2 against 34.8 us per cold step.
        constexpr int UB = 1;
        const int KU = (K + DF_NW - 1) / DF_NW;
        f32x4 Ra[NDT];   // the routed pages' state: a slot of its own, whichever workgroup routes
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) Ra[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        float mr = -INFINITY, lr = 0.0f;
        for (int j0 = 0; j0 < KU; j0 += UB) {
            bf16x8 rka[UB][4][NKS], rva[UB][NDT][2];
            int64_t kb0[UB];
            bool ok[UB];
#pragma unroll
            for (int ub = 0; ub < UB; ++ub) {
                const int r = w + DF_NW * (j0 + ub);
                const int pb = (r < K) ? sm.pick[r] : -1;
                const int64_t ph = (r < K) ? sm.pickp[r] : -1;
                ok[ub] = pb >= 1 && (int64_t)pb < maxp && ph >= 0;   // wave-uniform
                kb0[ub] = 64 * (int64_t)pb;
                const int64_t off = ok[ub] ? (ph * Hkv + g) * BK * D : 0;
                dec_unit_load<D>(kcp + off, vp + off, rka[ub], rva[ub]);
            }
#pragma unroll
            for (int ub = 0; ub < UB; ++ub) {
                if (!ok[ub]) continue;
                f32x4 O[NDT];
                float mu, lu;
                dec_unit_core<D>(rka[ub], rva[ub], qop, kb0[ub], kb0[ub], kb0[ub] + 63, scale, O, mu, lu);
                dec_fold<NDT>(Ra, mr, lr, O, mu, lu);
            }
        }
        df_fold_slot<D>(Ra, mr, lr, reinterpret_cast<float *>(sm.un), G, slots + (int64_t)gm.nz * G * PR);
        const int nv = sm.nvalid;   // the selection (its stores complete with the arrival below)
        if (sel_idx && tid < K) sel_idx[sg * K + tid] = (tid < nv) ? sm.pick[tid] : -1;
        if (sel_cnt && tid == 0) sel_cnt[sg] = nv < K ? nv : K;
    }

    // ---------------------- the last workgroup of (s, g) merges the slots ---
    if (!dec_arrive(ctr + (int64_t)gridDim.x * gridDim.y + sg, gm.nz, &sm.flag)) return;
    for (int e = tid; e < G * D; e += DF_NT) {
        const int h = e / D, t = e % D;
        float mx = -INFINITY, o = 0.0f, l = 0.0f;
        const int nslot = gm.nz + 1;
        for (int j0 = 0; j0 < nslot; j0 += 4) {   // 4 slots' loads in flight at a time
            float mj[4], lj[4], oj[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float *src = slots + ((int64_t)(j0 + v < nslot ? j0 + v : 0) * G + h) * PR;
                mj[v] = ld_dev(src + D);
                lj[v] = ld_dev(src + D + 1);
                oj[v] = ld_dev(src + t);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (j0 + v >= nslot || mj[v] == -INFINITY) continue;
                const float mn = fmaxf(mx, mj[v]);
                const float a = (mx == -INFINITY) ? 0.0f : exp2f((mx - mn) * DEC_LOG2E);
                const float b = exp2f((mj[v] - mn) * DEC_LOG2E);
                o = fmaf(oj[v], b, o * a);
                l = fmaf(lj[v], b, l * a);
                mx = mn;
            }
        }
        out[(s * Hq + (int64_t)g * G + h) * D + t] = f2bf(l > 0.0f ? o / l : 0.0f);
    }
}

// ============================================================================
// bf16: one workgroup per (sequence, KV head).
//
// Grid (Bd, Hkv), DP_NT threads, no workspace.  The workgroup scores every
// candidate page of its (s, g) (the declared-order slot scores of
// decode_fused_kernel), ranks them in LDS (64-page chunks, one wave each,
// then the chunk lists: an entry's rank is the number of live entries ordered
// before it), and runs the window, sink and routed page units on MFMA: wave w
// takes units w, w + DP_NW, ... of the list (window pages, the sinks, the k
// routed pages), loading the next unit while it computes one, and folds them
// into one partial state per head; the waves' states merge by LSE, in wave
// order, into out.  Every dependent step stays inside the workgroup, so the
// step needs no cross-workgroup hand-off: page table; summaries (and, at
// d = 64, the first window page); routed pages; out.
// ============================================================================
constexpr int DP_NT = 512;
constexpr int DP_NW = DP_NT / 64;
constexpr int DP_PMAX = 2048;                      // candidate pages ranked in LDS
constexpr int DP_LMAX = DP_PMAX / 64 * DEC_KMAX;   // chunk-list entries
constexpr int DP_WMAX = 256;                       // window + sink units

template <int D>
struct DpSmem {
    float qc[DF_GMAX * D];
    float qr[DF_GMAX * D];
    float qx[D];
    float sc[DP_PMAX];
    int phys[DP_PMAX];
    int wph[DP_WMAX];
    int pick[DEC_KMAX], pickp[DEC_KMAX];
    int nvalid;
    union {
        struct {
            float v[DP_LMAX];
            int p[DP_LMAX];
        } ls;
        float pbuf[DP_NW * DF_HB * dec_prow(D)];
    } un;
};

// A page unit of the pair kernel: its key and value pages, first key,
// valid key range and operand (rotated or not); ok false if it has no key.
struct DpUnit {
    const bf16_t *kp, *vp;
    int64_t kbase, lo, hi;
    bool ok, rope;
};

template <int D, int M>
__global__ __launch_bounds__(DP_NT) void decode_pair_kernel(
    const bf16_t *__restrict__ q, const float *__restrict__ qgain, float eps, const bf16_t *__restrict__ kcp,
    const bf16_t *__restrict__ krp, const bf16_t *__restrict__ vp, const bf16_t *__restrict__ sp,
    const int32_t *__restrict__ ptab, int64_t maxp, const int32_t *__restrict__ lens,
    const float *__restrict__ cosT, const float *__restrict__ sinT, const float *__restrict__ scales, int Hq,
    int Hkv, int S, int64_t W, int K, int nwp, int64_t gbmax, int64_t lmax, bf16_t *__restrict__ out,
    int32_t *__restrict__ sel_idx, int32_t *__restrict__ sel_cnt) {
    constexpr int BK = 64;
    constexpr int NKS = D / 32, NDT = D / 16, PR = dec_prow(D);
    constexpr int CPP = DP_NT / M;        // candidate pages per scoring pass
    constexpr bool PREF = D == 64;        // the first window unit loads during the scoring
    constexpr bool DBUF = D == 64;        // the next unit loads while one computes
    __shared__ DpSmem<D> sm;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int64_t s = blockIdx.x;
    const int g = blockIdx.y;
    const int G = Hq / Hkv;
    const int64_t sg = s * Hkv + g;
    const int32_t *pt = ptab + s * maxp;

    // Loads in the order of their use (see decode_fused_kernel): query
    // elements and gain, length and scale, page-table entries of every page
    // that can be a candidate at any length up to lmax (gbmax < maxp).
    const int e0 = 8 * tid;
    const bool hx = e0 < G * D;
    const int ec = hx ? e0 : G * D - 8;
    const u32x4d xr = *reinterpret_cast<const u32x4d *>(q + (s * Hq + (int64_t)g * G) * D + ec);
    const float graw = *(qgain ? qgain + g * G + ec / D : scales + s);
    const float gn = qgain ? graw : 1.0f;
    int ph[DP_PMAX / DP_NT];
#pragma unroll
    for (int r = 0; r < DP_PMAX / DP_NT; ++r) {
        const int64_t blk = 1 + tid + r * DP_NT;
        ph[r] = pt[blk <= gbmax ? blk : 0];
    }
    const int64_t L = min(min((int64_t)lens[s], maxp * BK), lmax);
    const float scale = scales[s];
    const int64_t bmax = (L >= 1) ? cand_bmax(L - 1, BK, W) : 0;   // candidate pages 1..bmax
    const int npass = (int)((bmax + CPP - 1) / CPP);
    // window and sink units: their pages' table entries; cos/sin at L-1
    int64_t ulo = 0, uhi = -1, upage = 0;
    const bool uany = tid <= nwp && dec_unit_range(tid, L, S, W, nwp, ulo, uhi, upage);
    const int uph = pt[uany ? upage : 0];
    const int64_t crow = ((L >= 1) ? L - 1 : 0) * D + ec % D;
    float cs[8], sn[8];
    ld8<0>(cosT + crow, cs);
    ld8<0>(sinT + crow, sn);
#pragma unroll
    for (int r = 0; r < DP_PMAX / DP_NT; ++r) sm.phys[tid + r * DP_NT] = ph[r];
    if (tid <= nwp) sm.wph[tid] = uph;
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[2 * e] = hx ? __uint_as_float(xr[e] << 16) : 0.0f;
        x[2 * e + 1] = hx ? __uint_as_float(xr[e] & 0xffff0000u) : 0.0f;
    }
    df_query<D>(x, hx, qgain != nullptr, gn, eps, sm.qc, sm.qr, cs, sn);   // ends with a barrier
    if (tid < D) {   // routing query: sequential head sum, rounded (summarizer.py:50-54)
        float a = sm.qc[tid];
        for (int h = 1; h < G; ++h) a = a + sm.qc[h * D + tid];
        sm.qx[tid] = rnd_bf16(a);
    }
    if (tid == 0) sm.nvalid = 0;
    if (tid < K) {
        sm.pick[tid] = -1;
        sm.pickp[tid] = -1;
    }
    __syncthreads();

    // ------------------------------------------------ unit list of wave w --
    const int nwin = (w <= nwp) ? (nwp - w) / DP_NW + 1 : 0;   // window and sink units
    const int nrt = (w < K) ? (K - 1 - w) / DP_NW + 1 : 0;      // routed pages
    const int nj = nwin + nrt;
    auto unit = [&](int j) {
        DpUnit U{kcp, vp, 0, 0, -1, false, false};
        if (j < nwin) {
            const int u = w + DP_NW * j;
            int64_t lo, hi, page;
            if (dec_unit_range(u, L, S, W, nwp, lo, hi, page)) {
                const int64_t phy = sm.wph[u];
                U.ok = true;
                U.rope = u < nwp;
                U.kbase = 64 * page;
                U.lo = lo;
                U.hi = hi;
                U.kp = (U.rope ? krp : kcp) + (phy * Hkv + g) * BK * D;
                U.vp = vp + (phy * Hkv + g) * D * BK;
            }
        } else if (j < nj) {
            const int r = w + DP_NW * (j - nwin);
            const int pb = sm.pick[r];
            const int64_t phy = sm.pickp[r];
            if (pb >= 1 && (int64_t)pb < maxp && phy >= 0) {
                U.ok = true;
                U.kbase = 64 * (int64_t)pb;
                U.lo = U.kbase;
                U.hi = U.kbase + 63;
                U.kp = kcp + (phy * Hkv + g) * BK * D;
                U.vp = vp + (phy * Hkv + g) * D * BK;
            }
        }
        return U;
    };
    bf16x8 ka0[4][NKS], va0[NDT][2];
    DpUnit cur{kcp, vp, 0, 0, -1, false, false};
    const bool pre = PREF && nwin > 0;   // wave-uniform
    if (pre) {
        cur = unit(0);
        dec_unit_load<D>(cur.kp, cur.vp, ka0, va0);
    }

    // ------------------------------------------------ candidate scores ----
    const int p = tid / M, sl = tid % M;
    auto srow_load = [&](int ps, u32x4d (&sr)[D / 8]) {
        const int64_t blk = 1 + (int64_t)ps * CPP + p;
        const bf16_t *src = (blk <= bmax) ? sp + (((int64_t)sm.phys[blk - 1] * Hkv + g) * M + sl) * D : sp;
#pragma unroll
        for (int c = 0; c < D / 8; ++c) sr[c] = *reinterpret_cast<const u32x4d *>(src + 8 * c);
    };
    auto score = [&](int ps, const u32x4d (&sr)[D / 8]) {
        const int64_t blk = 1 + (int64_t)ps * CPP + p;
        float acc = 0.0f;   // declared order: sequential FMA over the elements
#pragma unroll
        for (int c0 = 0; c0 < D / 8; c0 += 4) {
            float4 qv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) qv[i] = *reinterpret_cast<const float4 *>(&sm.qx[8 * c0 + 4 * i]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t *r32 = reinterpret_cast<const uint32_t *>(&sr[c0 + c]);
                const float4 a = qv[2 * c], b = qv[2 * c + 1];
                acc = fmaf(a.x, __uint_as_float(r32[0] << 16), acc);
                acc = fmaf(a.y, __uint_as_float(r32[0] & 0xffff0000u), acc);
                acc = fmaf(a.z, __uint_as_float(r32[1] << 16), acc);
                acc = fmaf(a.w, __uint_as_float(r32[1] & 0xffff0000u), acc);
                acc = fmaf(b.x, __uint_as_float(r32[2] << 16), acc);
                acc = fmaf(b.y, __uint_as_float(r32[2] & 0xffff0000u), acc);
                acc = fmaf(b.z, __uint_as_float(r32[3] << 16), acc);
                acc = fmaf(b.w, __uint_as_float(r32[3] & 0xffff0000u), acc);
            }
        }
        float best = (acc > -INFINITY) ? acc : -INFINITY;
#pragma unroll
        for (int o = 1; o < M; o <<= 1) {   // max over a page's slots: exact in any order
            const float ot = __shfl_xor(best, o, 64);
            best = (ot > best) ? ot : best;
        }
        if (sl == 0 && blk <= bmax) sm.sc[blk - 1] = best * scale;
    };
    {
        u32x4d sa[D / 8], sb[D / 8];
        srow_load(0, sa);
        srow_load(1, sb);
        for (int ps = 0; ps < npass; ps += 2) {
            score(ps, sa);
            srow_load(ps + 2, sa);
            score(ps + 1, sb);
            srow_load(ps + 3, sb);
        }
    }
    __syncthreads();

    // -------------------------------------- top-K: 64-page chunk lists ----
    // (rolled loops in this single-pass code: every workgroup runs it once,
    // so its length is instruction fetch time)
    const int nb = (int)bmax;   // <= DP_PMAX
    const int nch = (nb + 63) / 64;
    float *lv = sm.un.ls.v;
    int *lp = sm.un.ls.p;
#pragma unroll 1
    for (int c = w; c < nch; c += DP_NW) {
        const int cb = 64 * c;
        const int pg = cb + lane;
        const float vr = sm.sc[pg];   // inside sc (pg < DP_PMAX); masked below
        const float v = (pg < nb) ? vr : -INFINITY;
        const int lim = nb - cb;   // valid entries of the chunk
        int rank = 0;   // score desc, page asc
#pragma unroll 1
        for (int o = 0; o < 64; o += 8) {
            const float4 va4 = *reinterpret_cast<const float4 *>(&sm.sc[cb + o]);
            const float4 vb4 = *reinterpret_cast<const float4 *>(&sm.sc[cb + o + 4]);
            const float vo[8] = {va4.x, va4.y, va4.z, va4.w, vb4.x, vb4.y, vb4.z, vb4.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float u = (o + e < lim) ? vo[e] : -INFINITY;
                rank += rank_before(u, o + e, v, lane);
            }
        }
        if (rank < K) {   // the ranks are a permutation: every list entry is written
            lv[c * K + rank] = v;
            lp[c * K + rank] = pg + 1;
        }
    }
    __syncthreads();
    // merge: an entry's global rank is the number of live entries of all
    // lists ordered before it (the lists hold distinct pages); 8 threads
    // count an eighth of the entries each
    const int E = nch * K;
#pragma unroll 1
    for (int f0 = 0; f0 < E; f0 += DP_NT / 8) {
        const int e = f0 + tid / 8, part = tid % 8;
        const float v = (e < E) ? lv[e] : -INFINITY;
        const int id = (e < E) ? lp[e] : 0;
        int cnt = 0;
#pragma unroll 4
        for (int o = part; o < E; o += 8) {
            const float vo = lv[o];
            const int io = lp[o];
            cnt += (int)(vo != -INFINITY) & rank_before(vo, io, v, id);
        }
        cnt += __shfl_xor(cnt, 1, 64);
        cnt += __shfl_xor(cnt, 2, 64);
        cnt += __shfl_xor(cnt, 4, 64);
        if (part == 0 && v != -INFINITY && cnt < K) {
            sm.pick[cnt] = id;
            sm.pickp[cnt] = sm.phys[id - 1];
            atomicAdd(&sm.nvalid, 1);
        }
    }
    __syncthreads();

    // ------------------------------------------------------- page units ----
    bf16x8 qr_op[NKS], qc_op[NKS];
    df_qop<D>(sm.qr, G, qr_op);
    df_qop<D>(sm.qc, G, qc_op);
    f32x4 Oa[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) Oa[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ma = -INFINITY, la = 0.0f;
    auto run = [&](const DpUnit &U, const bf16x8 (&ka)[4][NKS], bf16x8 (&va)[NDT][2]) {
        if (!U.ok) return;
        f32x4 O[NDT];
        float mu, lu;
        dec_unit_core<D>(ka, va, U.rope ? qr_op : qc_op, U.kbase, U.lo, U.hi, scale, O, mu, lu);
        dec_fold<NDT>(Oa, ma, la, O, mu, lu);
    };
    if (!pre && nj > 0) {
        cur = unit(0);
        dec_unit_load<D>(cur.kp, cur.vp, ka0, va0);
    }
    if constexpr (DBUF) {
        // the next unit's loads are in flight while this one computes; one
        // copy of the unit code (the operands move between the buffers)
#pragma unroll 1
        for (int j = 0; j < nj; ++j) {
            const DpUnit nx = unit(j + 1);
            bf16x8 ka1[4][NKS], va1[NDT][2];
            dec_unit_load<D>(nx.kp, nx.vp, ka1, va1);
            run(cur, ka0, va0);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) ka0[mt][ks] = ka1[mt][ks];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                va0[dt][0] = va1[dt][0];
                va0[dt][1] = va1[dt][1];
            }
            cur = nx;
        }
    } else {
#pragma unroll 1
        for (int j = 0; j < nj; ++j) {
            if (j > 0) {
                cur = unit(j);
                dec_unit_load<D>(cur.kp, cur.vp, ka0, va0);
            }
            run(cur, ka0, va0);
        }
    }

    // --------------------------- the waves' states, merged by LSE, to out ---
    float *pbuf = sm.un.pbuf;
#pragma unroll 1
    for (int hc = 0; hc < G; hc += DF_HB) {
        __syncthreads();   // the region's earlier readers (the lists, the last pass) are done
        const int hh = l16 - hc;
        if (l16 < G && hh >= 0 && hh < DF_HB) {
            float *dst = pbuf + (w * DF_HB + hh) * PR;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                *reinterpret_cast<float4 *>(dst + 16 * dt + 4 * lg) = float4{Oa[dt][0], Oa[dt][1], Oa[dt][2], Oa[dt][3]};
            if (lg == 0) {
                dst[D] = ma;
                dst[D + 1] = la;
            }
        }
        __syncthreads();
        for (int e = tid; e < DF_HB * D; e += DP_NT) {
            const int hb = e / D, t = e % D, h = hc + hb;
            if (h >= G) continue;
            float mx = -INFINITY;
#pragma unroll
            for (int ww = 0; ww < DP_NW; ++ww) mx = fmaxf(mx, pbuf[(ww * DF_HB + hb) * PR + D]);
            float o = 0.0f, l = 0.0f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int ww = 0; ww < DP_NW; ++ww) {
                    const float *src = pbuf + (ww * DF_HB + hb) * PR;
                    const float mw = src[D];
                    if (mw == -INFINITY) continue;
                    const float a = exp2f((mw - mx) * DEC_LOG2E);
                    o = fmaf(src[t], a, o);
                    l = fmaf(src[D + 1], a, l);
                }
            }
            out[(s * Hq + (int64_t)g * G + h) * D + t] = f2bf(l > 0.0f ? o / l : 0.0f);
        }
    }
    const int nv = sm.nvalid;
    if (sel_idx && tid < K) sel_idx[sg * K + tid] = (tid < nv) ? sm.pick[tid] : -1;
    if (sel_cnt && tid == 0) sel_cnt[sg] = nv < K ? nv : K;
}

// Clears n 16-byte words (the no-allocation scratch, once per device).
__global__ void dec_zero_kernel(uint4 *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = uint4{0u, 0u, 0u, 0u};
}

}  // namespace hba

using namespace hba;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace.  Both layouts start with the counters of the one-launch bf16
// step, two per (s, g) of one launch: zero before the first call on a
// workspace, and left zero by every call.  The counter region has one fixed
// size whatever the call's batch, so that the other regions of an earlier
// call on the same workspace (fp32, or a smaller or larger batch) never lie
// under a later call's counters; a bf16 step of more than DEC_CTR_PAIRS
// (sequence, KV head) pairs runs as several launches over slices of the
// batch, one after another on the stream.
constexpr int64_t DEC_CTR_PAIRS = 4096;
static size_t ws_ctr_bytes() { return align256((size_t)2 * DEC_CTR_PAIRS * 4); }
// Sequences per bf16 fused launch.
static int64_t dec_fused_chunk(int64_t Bd, int64_t Hkv) {
    const int64_t c = DEC_CTR_PAIRS / Hkv;
    return Bd < c ? Bd : c;
}

// fp32 (three launches): chunk top-k (values, pages, physical pages), query
// operands, partial states.
static void ws_layout(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k, DecGeom gm,
                      size_t *off_val, size_t *off_idx, size_t *off_phys, size_t *off_q,
                      size_t *off_part, size_t *total) {
    size_t nsel = (size_t)Bd * Hkv * (gm.nsc > 0 ? gm.nsc : 1) * k;
    size_t G = (size_t)(Hq / Hkv);
    *off_val = ws_ctr_bytes();
    *off_idx = *off_val + align256(nsel * 4);
    *off_phys = *off_idx + align256(nsel * 4);
    *off_q = *off_phys + align256(nsel * 4);
    *off_part = *off_q + align256((size_t)Bd * Hkv * 2 * DEC_QROWS * d * 4);
    *total = *off_part + align256((size_t)Bd * Hkv * gm.npart * G * dec_prow((int)d) * 4);
}

// bf16 (one launch per slice of dec_fused_chunk sequences): chunk top-k
// (values, pages, physical pages), one partial-state slot per contributing
// workgroup, for one slice (the slices run in turn and reuse them).
static void ws_layout_fused(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k, const DecFGeom &gm,
                            size_t *off_val, size_t *off_idx, size_t *off_phys, size_t *off_part,
                            size_t *total) {
    const int64_t Bc = dec_fused_chunk(Bd, Hkv);
    size_t nsel = (size_t)Bc * Hkv * (gm.nsc > 0 ? gm.nsc : 1) * k;
    size_t G = (size_t)(Hq / Hkv);
    *off_val = ws_ctr_bytes();
    *off_idx = *off_val + align256(nsel * 4);
    *off_phys = *off_idx + align256(nsel * 4);
    *off_part = *off_phys + align256(nsel * 4);
    *total = *off_part + align256((size_t)Bc * Hkv * (gm.nz + 1) * G * dec_prow((int)d) * 4);
}

extern "C" int hba_decode_workspace_size(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k,
                                         int64_t Bk, int64_t W, int64_t max_len, size_t *bytes) {
    if (!bytes || Bd <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || k < 1 || W < 1 || max_len < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || k > DEC_KMAX || Hkv > DEC_CTR_PAIRS) return HBA_ERR_UNSUPPORTED;
    size_t a, b, c, e, f, t32, t16;
    ws_layout(Bd, Hq, Hkv, d, k, dec_geom(W, k, max_len), &a, &b, &c, &e, &f, &t32);
    // the bf16 layout at m = 8, which has the most score chunks
    ws_layout_fused(Bd, Hq, Hkv, d, k, dec_fgeom(W, 8, max_len), &a, &b, &c, &e, &t16);
    *bytes = t32 > t16 ? t32 : t16;
    return HBA_OK;
}

// The bf16 step's kernel.  decode_pair_kernel (one workgroup per (sequence,
// KV head), no hand-off between workgroups) when there are at least
// DP_MIN_PAIRS pairs and its LDS holds the candidate and window pages of the
// longest sequence; decode_fused_kernel (the scoring split over workgroups)
// otherwise.  Measured at 16-32K tokens, 14/2 heads, d = 64 (graph replay):
// 32 sequences fused 30.7 / pair 38.1 us, 128 sequences 69.2 / 47.8 us, 256
// sequences 143.5 / 95.7 us.  HBA_DECODE_KERNEL=pair or =fused in the
// environment overrides the pair count (the LDS bounds still hold).
constexpr int64_t DP_MIN_PAIRS = 128;
static bool dec_use_pair(int64_t Bd, int64_t Hkv, int64_t gbmax, int nwp) {
    if (gbmax > DP_PMAX || nwp + 1 > DP_WMAX) return false;
    const char *e = getenv("HBA_DECODE_KERNEL");
    if (e && !strcmp(e, "fused")) return false;
    if (e && !strcmp(e, "pair")) return true;
    return Bd * Hkv >= DP_MIN_PAIRS;
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
    const bool mf = dtype == HBA_DTYPE_BF16;   // bf16: one launch, units on MFMA
    if (Hq / Hkv > (mf ? DF_GMAX : DEC_GMAX) || k > DEC_KMAX || !(m == 1 || m == 2 || m == 4 || m == 8))
        return HBA_ERR_UNSUPPORTED;
    if ((max_len + Bk - 1) / Bk > max_pages) return HBA_ERR_INVALID_ARG;
    if (Bd > 65535 || Hkv > DEC_CTR_PAIRS) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(q) || !abi::aligned16(kc_pages) || !abi::aligned16(kr_pages) ||
        !abi::aligned16(v_pages) || !abi::aligned16(summ_pages) || !abi::aligned16(cos_tab) ||
        !abi::aligned16(sin_tab))
        return HBA_ERR_UNSUPPORTED;
    char *ws = (char *)workspace;
    hipStream_t s = (hipStream_t)stream;
    const int G = (int)(Hq / Hkv);
    if (mf) {
        const DecFGeom fg = dec_fgeom(W, m, max_len);
        if ((int64_t)fg.nsc * k > DF_EMAX) return HBA_ERR_UNSUPPORTED;
        size_t ov, oi, oph, op, total;
        ws_layout_fused(Bd, Hq, Hkv, d, k, fg, &ov, &oi, &oph, &op, &total);
        if (scratch_max && total > scratch_max) return HBA_ERR_SCRATCH;
        if (ws_bytes < total) return HBA_ERR_INVALID_ARG;
        const int64_t gbmax = cand_bmax(max_len - 1, 64, W);
        if (dec_use_pair(Bd, Hkv, gbmax, fg.nwp)) {
#define HBA_DP(D, M)                                                                                          \
    hipLaunchKernelGGL((decode_pair_kernel<D, M>), dim3((unsigned)Bd, (unsigned)Hkv), dim3(DP_NT), 0, s,        \
                       (const bf16_t *)q, q_gain, eps, (const bf16_t *)kc_pages, (const bf16_t *)kr_pages,     \
                       (const bf16_t *)v_pages, (const bf16_t *)summ_pages, page_table, max_pages, seq_lens,   \
                       cos_tab, sin_tab, scales, (int)Hq, (int)Hkv, (int)S, W, (int)k, fg.nwp, gbmax, max_len, \
                       (bf16_t *)out, sel_idx, sel_cnt)
#define HBA_DPM(D)                     \
    do {                               \
        if (m == 1) HBA_DP(D, 1);      \
        else if (m == 2) HBA_DP(D, 2); \
        else if (m == 4) HBA_DP(D, 4); \
        else HBA_DP(D, 8);             \
    } while (0)
            if (d == 64) HBA_DPM(64);
            else HBA_DPM(128);
#undef HBA_DP
#undef HBA_DPM
            HBA_LAUNCH_CHECK();
            return HBA_OK;
        }
        // slices of Bc sequences, so that one launch's counters fit their region
        const int64_t Bc = dec_fused_chunk(Bd, Hkv);
        for (int64_t c0 = 0; c0 < Bd; c0 += Bc) {
            const int64_t nc = (Bd - c0 < Bc) ? Bd - c0 : Bc;
            dim3 grid((unsigned)nc, (unsigned)Hkv, (unsigned)fg.nz);
            const bf16_t *qc0 = (const bf16_t *)q + c0 * Hq * d;
            bf16_t *oc0 = (bf16_t *)out + c0 * Hq * d;
            int32_t *si0 = sel_idx ? sel_idx + c0 * Hkv * k : nullptr;
            int32_t *sc0 = sel_cnt ? sel_cnt + c0 * Hkv : nullptr;
#define HBA_DF(D, M)                                                                                            \
    hipLaunchKernelGGL((decode_fused_kernel<D, M>), grid, dim3(DF_NT), 0, s, qc0, q_gain, eps,                  \
                       (const bf16_t *)kc_pages, (const bf16_t *)kr_pages, (const bf16_t *)v_pages,             \
                       (const bf16_t *)summ_pages, page_table + c0 * max_pages, max_pages, seq_lens + c0,       \
                       cos_tab, sin_tab, scales + c0, (int)Hq, (int)Hkv, (int)S, W, (int)k, fg, (int *)ws,      \
                       (float *)(ws + ov), (int32_t *)(ws + oi), (int32_t *)(ws + oph), (float *)(ws + op), oc0, \
                       si0, sc0)
#define HBA_DFM(D)                     \
    do {                               \
        if (m == 1) HBA_DF(D, 1);      \
        else if (m == 2) HBA_DF(D, 2); \
        else if (m == 4) HBA_DF(D, 4); \
        else HBA_DF(D, 8);             \
    } while (0)
            if (d == 64) HBA_DFM(64);
            else HBA_DFM(128);
#undef HBA_DF
#undef HBA_DFM
            HBA_LAUNCH_CHECK();
        }
        return HBA_OK;
    }
    DecGeom gm = dec_geom(W, k, max_len);
    if ((int64_t)gm.nsc * k > 2048 || gm.npart > DEC_PMAX) return HBA_ERR_UNSUPPORTED;
    size_t ov, oi, oph, oq, op, total;
    ws_layout(Bd, Hq, Hkv, d, k, gm, &ov, &oi, &oph, &oq, &op, &total);
    if (scratch_max && total > scratch_max) return HBA_ERR_SCRATCH;
    if (ws_bytes < total) return HBA_ERR_INVALID_ARG;
    float *wv = (float *)(ws + ov);
    int32_t *wi = (int32_t *)(ws + oi);
    int32_t *wph = (int32_t *)(ws + oph);
    void *wq = (void *)(ws + oq);
    float *wp = (float *)(ws + op);
    dim3 g1((unsigned)Bd, (unsigned)Hkv, (unsigned)(gm.nsc > 0 ? gm.nsc : 1));
    dim3 g2((unsigned)Bd, (unsigned)Hkv, (unsigned)(gm.uwg + k));
    dim3 g3((unsigned)Bd, (unsigned)Hkv, (unsigned)G);
#define HBA_D1(DT, D, M)                                                                          \
    hipLaunchKernelGGL((decode_d1_kernel<DT, D, M>), g1, dim3(DEC_WG), 0, s,                        \
                       (const St<DT>::T *)q, q_gain, eps, (const St<DT>::T *)summ_pages,            \
                       page_table, max_pages, seq_lens, cos_tab, sin_tab, scales, (int)Hq,         \
                       (int)Hkv, W, (int)k, gm, wv, wi, wph, (St<DT>::T *)wq)
#define HBA_D1M(D)                                       \
    do {                                                 \
        if (m == 1) HBA_D1(0, D, 1);                     \
        else if (m == 2) HBA_D1(0, D, 2);                \
        else if (m == 4) HBA_D1(0, D, 4);                \
        else HBA_D1(0, D, 8);                            \
    } while (0)
#define HBA_D23(D)                                                                                \
    do {                                                                                          \
        hipLaunchKernelGGL((decode_d2_kernel<0, D>), g2, dim3(DEC_WG), 0, s, (const float *)wq,     \
                           (const float *)kc_pages, (const float *)kr_pages, (const float *)v_pages, \
                           page_table, max_pages, seq_lens, scales, (int)Hq, (int)Hkv, (int)S, W,  \
                           (int)k, gm, wv, wi, wph, wp, sel_idx, sel_cnt);                          \
        hipLaunchKernelGGL((decode_d3_kernel<0, D>), g3, dim3(64), 0, s, wp, (int)Hq, (int)Hkv, gm, \
                           (float *)out);                                                           \
    } while (0)
    if (d == 64) {
        HBA_D1M(64);
        HBA_D23(64);
    } else {
        HBA_D1M(128);
        HBA_D23(128);
    }
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
// in scratch_ptr.  Every call on a GPU shares that GPU's copy.  Set-up (the
// first call on a device) clears it with a kernel on the call's stream, so
// that the counters at its start are zero; every call leaves them zero and
// writes every other entry it reads, so nothing is cleared between calls.
// A set-up under stream capture is repeated by the next call.  Calls that
// overlap on one GPU (different streams) race on it.
static __device__ __align__(256) char scratch[HBA_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void *scratch_ptr[kMaxDevices];   // device address of `scratch` per device, or null
bool scratch_clear[kMaxDevices];  // a clearing of that copy has run (not only been captured)

int scratch_on_current_device(hipStream_t stream, void **ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return HBA_ERR_DEVICE;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return HBA_ERR_DEVICE;
        scratch_ptr[dev] = p;
    }
    if (!scratch_clear[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return HBA_ERR_DEVICE;
        hipLaunchKernelGGL(dec_zero_kernel, dim3(256), dim3(256), 0, stream, (uint4 *)scratch_ptr[dev],
                           (size_t)HBA_DECODE_SCRATCH_BYTES / 16);
        if (hipGetLastError() != hipSuccess) return HBA_ERR_LAUNCH;
        scratch_clear[dev] = cs == hipStreamCaptureStatusNone;
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
    const int st = scratch_on_current_device((hipStream_t)stream, &ws);
    if (st) return st;
    return decode_fwd_ws(dtype, q, q_gain, eps, kc_pages, kr_pages, v_pages, summ_pages, page_table, max_pages,
                         seq_lens, cos_tab, sin_tab, scales, Bd, Hq, Hkv, d, m, S, W, Bk, k, max_len, ws,
                         (size_t)HBA_DECODE_SCRATCH_BYTES, (size_t)HBA_DECODE_SCRATCH_BYTES, out, sel_idx,
                         sel_cnt, stream);
}
