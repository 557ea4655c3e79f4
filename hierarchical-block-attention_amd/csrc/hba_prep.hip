// Key preparation, slot summaries, super-summaries and the paged-cache append.
//
//   prep_keys        QKNorm(k) -> kc, RoPE(kc) -> kr, V^T -> vt
//                    (_HeadRMSNorm.forward src/hba/attention.py:88-94,
//                     apply_rope src/hba/attention.py:40-44)
//   summarize        SlotSummarizer.summarize src/hba/summarizer.py:34-42
//   build_super      build_super src/hba/attention.py:202-214
//   kv_append        decode-cache append (no reference counterpart)
//   kv_append_advance  the decode loop's append: token, page summary when it
//                    fills a page, seq_lens += 1 and the new length's scale
//
// All of these are HBM-bound elementwise / tiny-GEMM work: one thread per key
// row (prep), d/8 lanes per key row (append), one workgroup per 64-key block
// (summaries).
#include "hba_common.h"
#include "hba_abi.h"
#include "hba_generic.h"

namespace hba {

// ------------------------------------------------------------- row I/O ----
// Rows are d-contiguous and 16-byte aligned (checked by the host entry points).
template <int DT, int D>
__device__ __forceinline__ void load_row(const typename St<DT>::T *p, float (&x)[D]) {
    if constexpr (DT == 1) {
        const uint4 *q = reinterpret_cast<const uint4 *>(p);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            uint4 u = q[c];
            uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[8 * c + 2 * e] = __uint_as_float(w[e] << 16);
                x[8 * c + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            }
        }
    } else {
        const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
        for (int c = 0; c < D / 4; ++c) {
            float4 u = q[c];
            x[4 * c] = u.x;
            x[4 * c + 1] = u.y;
            x[4 * c + 2] = u.z;
            x[4 * c + 3] = u.w;
        }
    }
}

template <int DT, int D>
__device__ __forceinline__ void store_row(typename St<DT>::T *p, const float (&x)[D]) {
    if constexpr (DT == 1) {
        uint4 *q = reinterpret_cast<uint4 *>(p);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = (uint32_t)f2bf(x[8 * c + 2 * e]) | ((uint32_t)f2bf(x[8 * c + 2 * e + 1]) << 16);
            q[c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    } else {
        float4 *q = reinterpret_cast<float4 *>(p);
#pragma unroll
        for (int c = 0; c < D / 4; ++c) q[c] = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]);
    }
}

// 8 consecutive elements (16 bytes of bf16, 32 of fp32; 16-byte aligned)
template <int DT>
__device__ __forceinline__ void load8(const typename St<DT>::T *p, float (&x)[8]) {
    if constexpr (DT == 1) {
        const uint4 u = *reinterpret_cast<const uint4 *>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[2 * e] = __uint_as_float(w[e] << 16);
            x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        }
    } else {
        const float4 a = reinterpret_cast<const float4 *>(p)[0], c = reinterpret_cast<const float4 *>(p)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
    }
}

template <int DT>
__device__ __forceinline__ void store8(typename St<DT>::T *p, const float (&x)[8]) {
    if constexpr (DT == 1) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (uint32_t)f2bf(x[2 * e]) | ((uint32_t)f2bf(x[2 * e + 1]) << 16);
        *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        float4 *q = reinterpret_cast<float4 *>(p);
        q[0] = make_float4(x[0], x[1], x[2], x[3]);
        q[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
}

// --------------------------------------------------------------- kernels ----
// One workgroup per (batch, KV head, 64-key tile); D/8 lanes per key row, 8
// elements each, so that every row load and store is one coalesced 16-byte
// access per lane.  QKNorm's sum of squares runs in the declared order
// (sequential FMA over the row, as qknorm_row) as a chain through the row's
// lanes: lane c continues the sum of lane c-1 (row_shr:1 DPP move); the
// rotation's partner elements (rotate-half) come from lane c ^ (D/16).  The
// values are transposed through LDS, so that vt rows are written as 8
// consecutive keys per lane.
// kb (optional): the tile's kc rows as floats, row stride D + 1, for a
// summary of the block in the same workgroup.  256 threads.
template <int DT, int D>
__device__ __forceinline__ void prep_tile(
    const typename St<DT>::T *__restrict__ k, int64_t ksb, int64_t ksn, int64_t ksh,
    const typename St<DT>::T *__restrict__ v, int64_t vsb, int64_t vsn, int64_t vsh,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t n, int64_t Hkv, int64_t tile, int64_t bg,
    typename St<DT>::T *__restrict__ kc, typename St<DT>::T *__restrict__ kr,
    typename St<DT>::T *__restrict__ vt, float *__restrict__ kb) {
    using T = typename St<DT>::T;
    constexpr int TPH = D / 8;          // lanes per key row
    constexpr int RPP = 256 / TPH;      // rows per pass
    __shared__ float vs[D][65];         // the tile's values (exact in fp32), key-minor
    const int tid = threadIdx.x;
    const int64_t b = bg / Hkv, g = bg % Hkv;
    const int jl = tid % TPH, t0 = 8 * jl;
    const bool lo = t0 < D / 2;
    const float gn = kgain ? kgain[g] : 0.0f;
#pragma unroll 1
    for (int pass = 0; pass < 64 / RPP; ++pass) {
        const int r = pass * RPP + tid / TPH;
        const int64_t j = tile * 64 + r;
        const bool act = j < n;
        const int64_t jj = act ? j : 0;
        float x[8];
        load8<DT>(k + b * ksb + jj * ksn + g * ksh + t0, x);
        if (kgain) {
            float run = 0.0f;
#pragma unroll
            for (int step = 0; step < TPH; ++step) {
                const float in = __builtin_bit_cast(
                    float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, run), 0x111, 0xf, 0xf, false));
                if (jl == step) {
                    float a = (jl == 0) ? 0.0f : in;
#pragma unroll
                    for (int u = 0; u < 8; ++u) a = fmaf(x[u], x[u], a);
                    run = a;
                }
            }
            const float ss = __shfl(run, (tid & 63) | (TPH - 1), 64);   // the row's last lane
            float ms = ss / (float)D;
            if (ms < eps) ms = eps;
            const float rr = sqrtf(ms);
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = St<DT>::rnd((x[u] / rr) * gn);
        }
        const int64_t row = (bg * n + jj) * D + t0;
        if (act) store8<DT>(kc + row, x);
        if (kb) {
#pragma unroll
            for (int u = 0; u < 8; ++u) kb[r * (D + 1) + t0 + u] = x[u];
        }
        if (kr) {
            float cs[8], sn[8], y[8];
            load8<0>(cosT + jj * D + t0, cs);
            load8<0>(sinT + jj * D + t0, sn);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float part = __shfl_xor(x[u], TPH / 2, 64);
                const float rot = lo ? -part : part;
                y[u] = St<DT>::rnd(St<DT>::rnd(x[u] * St<DT>::rnd(cs[u])) + St<DT>::rnd(rot * St<DT>::rnd(sn[u])));
            }
            if (act) store8<DT>(kr + row, y);
        }
        if (vt) {
            float vv[8];
            load8<DT>(v + b * vsb + jj * vsn + g * vsh + t0, vv);
#pragma unroll
            for (int u = 0; u < 8; ++u) vs[t0 + u][r] = vv[u];
        }
    }
    if (!vt) return;
    __syncthreads();
    // vt[bg][t][tile*64 + 8c' .. +7]: 8 consecutive keys of one row per thread
    T *vrow = vt + bg * D * n;
    const int64_t k0 = tile * 64;
    const bool vec = ((reinterpret_cast<uintptr_t>(vt) & 15) == 0) && (n % 8 == 0);   // uniform
#pragma unroll 1
    for (int c = tid; c < D * 8; c += 256) {
        const int t = c / 8, j8 = 8 * (c % 8);
        float o[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) o[u] = vs[t][j8 + u];
        const int64_t jo = k0 + j8;
        if (vec && jo + 8 <= n) {
            store8<DT>(vrow + (int64_t)t * n + jo, o);
        } else {
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (jo + u < n) St<DT>::st(vrow, (int64_t)t * n + jo + u, o[u]);
        }
    }
}

template <int DT, int D>
__global__ __launch_bounds__(256) void prep_keys_kernel(
    const typename St<DT>::T *__restrict__ k, int64_t ksb, int64_t ksn, int64_t ksh,
    const typename St<DT>::T *__restrict__ v, int64_t vsb, int64_t vsn, int64_t vsh,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t n, int64_t Hkv, int64_t ntile,
    typename St<DT>::T *__restrict__ kc, typename St<DT>::T *__restrict__ kr,
    typename St<DT>::T *__restrict__ vt) {
    prep_tile<DT, D>(k, ksb, ksn, ksh, v, vsb, vsn, vsh, kgain, eps, cosT, sinT, n, Hkv, blockIdx.x % ntile,
                     blockIdx.x / ntile, kc, kr, vt, nullptr);
}

// LDS of one block summary: the block's 64 key rows (reused, once the pooled
// rows are done, for chunks of the projection), slot scores, pooled rows,
// and for LONE the probes.
template <int D, bool LONE> struct SummSmem {
    float kb[64][D + 1];
    float att[8][64];
    float pooled[8][D];
    float prl[LONE ? 8 : 1][D];
};

// Slot summaries of one block whose 64 key rows are staged in sm.kb: slot
// scores, softmax over the 64 keys of each slot, pooling, projection.  Every
// output is one sequential fma chain in the index order of the sums
// (probes . key, att . keys, pooled . proj), so both forms below give the
// same bits.  256 threads; starts after the staging barrier; its callers
// barrier before restaging sm.kb.
//   LONE = false (many workgroups, prefill and page lists): probes and the
//     projection are read from global memory inside the chains; other
//     workgroups hide the load latency.
//   LONE = true (a workgroup or two, the decode loop's page fill): probes and
//     the projection are staged through LDS in coalesced bulk loads (the
//     projection in chunks over sm.kb's space), so the workgroup waits on a
//     few load round trips instead of one per chain step.
template <int DT, int D, bool LONE>
__device__ __forceinline__ void summarize_staged(SummSmem<D, LONE> &sm, const float *__restrict__ pr,
                                                 const float *__restrict__ pj, int m, float att_scale,
                                                 typename St<DT>::T *__restrict__ dst, int tid) {
    constexpr int BK = 64;
    if constexpr (LONE) {
        for (int e = tid; e < m * D; e += 256) sm.prl[e / D][e % D] = pr[e];
        __syncthreads();
    }
    for (int e = tid; e < m * BK; e += 256) {
        int s = e / BK, t = e % BK;
        float acc = 0.0f;
        if constexpr (LONE) {
#pragma unroll 16
            for (int dd = 0; dd < D; ++dd) acc = fmaf(sm.prl[s][dd], sm.kb[t][dd], acc);
        } else {
            for (int dd = 0; dd < D; ++dd) acc = fmaf(pr[s * D + dd], sm.kb[t][dd], acc);
        }
        sm.att[s][t] = acc * att_scale;
    }
    __syncthreads();
    {   // softmax over the 64 keys of each slot: one wave per slot
        int w = tid / 64, l = tid % 64;
        for (int s = w; s < m; s += 4) {
            float x = sm.att[s][l];
            float mx = wave_max(x);
            float e = expf(x - mx);
            float sm_ = wave_sum(e);
            sm.att[s][l] = e / sm_;
        }
    }
    __syncthreads();
    for (int e = tid; e < m * D; e += 256) {
        int s = e / D, dd = e % D;
        float acc = 0.0f;
        for (int t = 0; t < BK; ++t) acc = fmaf(sm.att[s][t], sm.kb[t][dd], acc);
        sm.pooled[s][dd] = acc;
    }
    __syncthreads();
    if constexpr (!LONE) {
        for (int e = tid; e < m * D; e += 256) {
            int s = e / D, ee = e % D;
            float acc = 0.0f;
            for (int dd = 0; dd < D; ++dd) acc = fmaf(sm.pooled[s][dd], pj[dd * D + ee], acc);
            St<DT>::st(dst, (int64_t)s * D + ee, acc);
        }
    } else {
        // up to 4 outputs per thread (m * D <= 1024); pj rows staged CHR at a
        // time into the key tile's space (65 or 64 rows fit; CHR divides D)
        constexpr int CH = (BK * (D + 1)) / D;
        constexpr int CHR = (CH < D) ? CH : D;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float *pjl = &sm.kb[0][0];
        for (int c0 = 0; c0 < D; c0 += CHR) {
            if (c0) __syncthreads();   // the previous chunk is used
#pragma unroll 8
            for (int i = tid; i < CHR * D; i += 256) pjl[i] = pj[(int64_t)c0 * D + i];
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = tid + 256 * q;
                if (e < m * D) {
                    const int s = e / D, ee = e % D;
                    float a = acc[q];
#pragma unroll 16
                    for (int dd = 0; dd < CHR; ++dd) a = fmaf(sm.pooled[s][c0 + dd], pjl[dd * D + ee], a);
                    acc[q] = a;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = tid + 256 * q;
            if (e < m * D) St<DT>::st(dst, e, acc[q]);
        }
    }
}

// Stage the rows of one cache page (page_key_chunk order) into kb, all but
// row `skip` (-1: none).
template <int DT, int D>
__device__ __forceinline__ void stage_page(const typename St<DT>::T *__restrict__ src, float (&kb)[64][D + 1],
                                           int skip, int tid) {
    for (int c = tid; c < 8 * D; c += 256) {
        int j, t0;
        page_key_chunk(c, D, j, t0);
        if (j == skip) continue;
#pragma unroll
        for (int u = 0; u < 8; ++u) kb[j][t0 + u] = St<DT>::ld(src, 8 * c + u);
    }
}

// One workgroup (256 threads) per 64-key block.  Block base pointers come
// from the contiguous head-major layout, from a list of pages, or (ptab set)
// from a page table: workgroup c takes sequence c's page that its last append
// filled (seq_lens[c] a positive multiple of 64) and exits otherwise (LONE:
// few workgroups run).
template <int DT, int D, bool LONE>
__global__ __launch_bounds__(256) void summarize_kernel(
    const typename St<DT>::T *__restrict__ kc, int64_t n, int64_t nb, int64_t Hkv,
    const int32_t *__restrict__ pages, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, const float *__restrict__ probes,
    const float *__restrict__ proj, int m, float att_scale, typename St<DT>::T *__restrict__ out) {
    constexpr int BK = 64;
    __shared__ SummSmem<D, LONE> sm;
    auto &kb = sm.kb;
    const int tid = threadIdx.x;
    const int64_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const typename St<DT>::T *src;
    typename St<DT>::T *dst;
    int64_t filled = -1;
    if (ptab) {   // uniform per workgroup: the exit comes before any barrier
        const int64_t L = lens[c];
        if (L <= 0 || L % BK != 0 || L / BK > maxp) return;
        filled = ptab[c * maxp + L / BK - 1];
    }
    if (pages || ptab) {   // a cache page: chunks of 8 elements in the page layout (page_key_chunk)
        int64_t p = ptab ? filled : (int64_t)pages[c];
        src = kc + (p * Hkv + g) * BK * D;
        dst = out + (p * Hkv + g) * m * D;
        stage_page<DT, D>(src, kb, -1, tid);
    } else {
        src = kc + ((b * Hkv + g) * n + c * BK) * D;
        dst = out + ((b * Hkv + g) * nb + c) * m * D;
        for (int c8 = tid; c8 < BK * D / 8; c8 += 256) {   // 16-byte loads, 8 elements of one row
            float x[8];
            load8<DT>(src + 8 * c8, x);
            const int r = (8 * c8) / D, t0 = (8 * c8) % D;
#pragma unroll
            for (int u = 0; u < 8; ++u) kb[r][t0 + u] = x[u];
        }
    }
    __syncthreads();
    summarize_staged<DT, D, LONE>(sm, probes + g * m * D, proj + g * D * D, m, att_scale, dst, tid);
}

// prep_keys and the slot summaries of every full block in one launch: the
// workgroup of a 64-key tile keeps its kc rows (as the floats it stores) in
// LDS and runs summarize_staged on them, so that S0 has the bits of
// summarize_kernel over the stored kc, without its launch and its re-read.
template <int DT, int D>
__global__ __launch_bounds__(256) void prep_summ_kernel(
    const typename St<DT>::T *__restrict__ k, int64_t ksb, int64_t ksn, int64_t ksh,
    const typename St<DT>::T *__restrict__ v, int64_t vsb, int64_t vsn, int64_t vsh,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t n, int64_t Hkv, int64_t ntile,
    typename St<DT>::T *__restrict__ kc, typename St<DT>::T *__restrict__ kr,
    typename St<DT>::T *__restrict__ vt, const float *__restrict__ probes, const float *__restrict__ proj,
    int m, float att_scale, typename St<DT>::T *__restrict__ S0) {
    __shared__ SummSmem<D, false> sm;
    const int64_t tile = blockIdx.x % ntile, bg = blockIdx.x / ntile;
    prep_tile<DT, D>(k, ksb, ksn, ksh, v, vsb, vsn, vsh, kgain, eps, cosT, sinT, n, Hkv, tile, bg, kc, kr, vt,
                     &sm.kb[0][0]);
    const int64_t nb = n / 64;
    if (tile >= nb) return;   // a partial last tile has no summary (workgroup-uniform)
    __syncthreads();          // every kb row is written
    const int64_t g = bg % Hkv;
    summarize_staged<DT, D, false>(sm, probes + g * m * D, proj + g * D * D, m, att_scale,
                                   S0 + (bg * nb + tile) * m * D, threadIdx.x);
}

// Super-summaries: sequential child sum, rounded, divided by the child count,
// rounded (the reference's bf16 sum-then-divide, attention.py:210-214).
template <int DT>
__global__ __launch_bounds__(256) void build_super_kernel(const typename St<DT>::T *__restrict__ S0,
                                                           int64_t BH, int64_t nb, int64_t m,
                                                           int64_t d, int64_t F,
                                                           typename St<DT>::T *__restrict__ S1) {
    int64_t ns = (nb + F - 1) / F;
    int64_t total = BH * ns * m * d;
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    int64_t t = gid % d;
    int64_t s = (gid / d) % m;
    int64_t p = (gid / (d * m)) % ns;
    int64_t bh = gid / (d * m * ns);
    int64_t c0 = p * F;
    int64_t cn = (c0 + F <= nb) ? F : nb - c0;
    const typename St<DT>::T *base = S0 + bh * nb * m * d;
    float acc = St<DT>::ld(base, (c0 * m + s) * d + t);
    for (int64_t c = 1; c < cn; ++c) acc = acc + St<DT>::ld(base, ((c0 + c) * m + s) * d + t);
    acc = St<DT>::rnd(acc);
    St<DT>::st(S1, gid, acc / (float)cn);
}

// One appended token row (one sequence, one KV head) spread over TPH = D/8
// lanes of a wave, lane jl holding elements t0 = 8*jl .. t0+7: QKNorm with
// the sum of squares chained across the row's lanes in element order (DPP
// row_shr:1, so the fma order is qknorm_row's), the rotation with the
// partner half from lane jl ^ TPH/2 (rope_row's roundings), the key and its
// rotation stored as one 8-element chunk each at page_key_off(j, t0), the
// value elements at page_val_off(j, t).  Every lane of the wave calls it
// (the chain needs them all); act = false lanes load nothing and store
// nothing.  x returns the lane's 8 key elements.
template <int DT, int D>
__device__ __forceinline__ void append_row8(bool act, const typename St<DT>::T *__restrict__ krow,
                                            const typename St<DT>::T *__restrict__ vrow, const float *kgain,
                                            int64_t g, float eps, const float *cs, const float *sn, int64_t base,
                                            int j, typename St<DT>::T *__restrict__ kcp,
                                            typename St<DT>::T *__restrict__ krp,
                                            typename St<DT>::T *__restrict__ vp, float (&x)[8]) {
    constexpr int TPH = D / 8;
    const int jl = (int)(threadIdx.x % TPH), t0 = 8 * jl;
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = act ? St<DT>::ld(krow, t0 + u) : 0.0f;
    if (kgain) {
        float run = 0.0f;
#pragma unroll
        for (int step = 0; step < TPH; ++step) {
            const float in = __builtin_bit_cast(
                float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, run), 0x111, 0xf, 0xf, false));
            if (jl == step) {
                float a = (jl == 0) ? 0.0f : in;
#pragma unroll
                for (int u = 0; u < 8; ++u) a = fmaf(x[u], x[u], a);
                run = a;
            }
        }
        const float ss = __shfl(run, (int)(threadIdx.x & 63) | (TPH - 1), 64);   // the row's last lane
        float ms = ss / (float)D;
        if (ms < eps) ms = eps;
        const float r = sqrtf(ms);
        const float gn = act ? kgain[g] : 0.0f;
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = St<DT>::rnd((x[u] / r) * gn);
    }
    const bool lo = t0 < D / 2;
    float y[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const float part = __shfl_xor(x[u], TPH / 2, 64);
        const float rot = lo ? -part : part;
        const float c = act ? St<DT>::rnd(cs[t0 + u]) : 0.0f;
        const float sv = act ? St<DT>::rnd(sn[t0 + u]) : 0.0f;
        y[u] = St<DT>::rnd(St<DT>::rnd(x[u] * c) + St<DT>::rnd(rot * sv));
    }
    if (!act) return;
    const int64_t o = base + page_key_off(j, t0, D);   // 8 consecutive elements, 16-byte aligned
    if constexpr (DT == 1) {
        uint32_t wk[4], wr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            wk[e] = (uint32_t)f2bf(x[2 * e]) | ((uint32_t)f2bf(x[2 * e + 1]) << 16);
            wr[e] = (uint32_t)f2bf(y[2 * e]) | ((uint32_t)f2bf(y[2 * e + 1]) << 16);
        }
        *reinterpret_cast<uint4 *>(kcp + o) = make_uint4(wk[0], wk[1], wk[2], wk[3]);
        *reinterpret_cast<uint4 *>(krp + o) = make_uint4(wr[0], wr[1], wr[2], wr[3]);
    } else {
        float4 *pk = reinterpret_cast<float4 *>(kcp + o), *pq = reinterpret_cast<float4 *>(krp + o);
        pk[0] = make_float4(x[0], x[1], x[2], x[3]);
        pk[1] = make_float4(x[4], x[5], x[6], x[7]);
        pq[0] = make_float4(y[0], y[1], y[2], y[3]);
        pq[1] = make_float4(y[4], y[5], y[6], y[7]);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) St<DT>::st(vp, base + page_val_off(j, t0 + u), St<DT>::ld(vrow, t0 + u));
}

// kv_append: rows (s, g) = blockIdx.x * RPP + threadIdx.x / TPH, one token
// each at position seq_lens[s] - 1.
template <int DT, int D>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const typename St<DT>::T *__restrict__ knew, const typename St<DT>::T *__restrict__ vnew,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, int64_t lmax, int64_t Bd, int64_t Hkv,
    typename St<DT>::T *__restrict__ kcp, typename St<DT>::T *__restrict__ krp,
    typename St<DT>::T *__restrict__ vp) {
    constexpr int BK = 64, TPH = D / 8, RPP = 256 / TPH;
    const int64_t row = (int64_t)blockIdx.x * RPP + threadIdx.x / TPH;
    const int64_t s = row / Hkv, g = row % Hkv;
    const int64_t pos = (row < Bd * Hkv) ? (int64_t)lens[s] - 1 : -1;
    // nothing to append, outside the page table or past the RoPE tables
    const bool act = pos >= 0 && pos / BK < maxp && pos < lmax;
    const int64_t page = act ? (int64_t)ptab[s * maxp + pos / BK] : 0;
    const int64_t pc = act ? pos : 0;
    const int64_t rr = act ? row : 0;
    float x[8];
    append_row8<DT, D>(act, knew + rr * D, vnew + rr * D, kgain, g, eps, cosT + pc * D, sinT + pc * D,
                       (page * Hkv + g) * BK * D, (int)(pc % BK), kcp, krp, vp, x);
}

// The decode loop's append: one workgroup per sequence s.  The token goes to
// position pos = seq_lens[s] (KV head g on lanes g*TPH ..); when it fills its
// page, the page's summaries are computed from the page staged in LDS (the
// new row from the writers' registers through LDS, so no global
// read-after-write inside the launch); then seq_lens[s] = pos + 1 and
// scales[s] = scale_tab[pos + 1].  A position outside the page table or the
// RoPE tables appends nothing and leaves seq_lens[s] as it is.  Only thread
// 0 reads and writes seq_lens[s].
template <int DT, int D>
__global__ __launch_bounds__(256) void kv_append_advance_kernel(
    const typename St<DT>::T *__restrict__ knew, const typename St<DT>::T *__restrict__ vnew,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t lmax, const int32_t *__restrict__ ptab, int64_t maxp,
    int32_t *__restrict__ lens, int64_t Hkv, typename St<DT>::T *__restrict__ kcp,
    typename St<DT>::T *__restrict__ krp, typename St<DT>::T *__restrict__ vp,
    const float *__restrict__ probes, const float *__restrict__ proj, int m, float att_scale,
    typename St<DT>::T *__restrict__ summ, const float *__restrict__ scale_tab, int64_t n_scale,
    float *__restrict__ scales) {
    constexpr int BK = 64, TPH = D / 8, RPP = 256 / TPH;
    __shared__ SummSmem<D, true> sm;
    __shared__ float newk[RPP][D];
    __shared__ int32_t pos_lds;
    const int tid = threadIdx.x;
    const int64_t s = blockIdx.x;
    if (tid == 0) pos_lds = lens[s];
    __syncthreads();
    const int64_t pos = pos_lds;
    const bool ok = pos >= 0 && pos / BK < maxp && pos < lmax;
    const int64_t pc = ok ? pos : 0;
    const int j = (int)(pc % BK);
    const bool filled = ok && j == BK - 1;
    const int64_t page = ok ? (int64_t)ptab[s * maxp + pos / BK] : 0;
    const int r = tid / TPH, t0 = 8 * (tid % TPH);
    for (int64_t g0 = 0; g0 < Hkv; g0 += RPP) {
        const int64_t g = g0 + r;
        const bool act = ok && g < Hkv;
        const int64_t row = s * Hkv + (act ? g : 0);
        float x[8];
        append_row8<DT, D>(act, knew + row * D, vnew + row * D, kgain, g, eps, cosT + pc * D, sinT + pc * D,
                           (page * Hkv + g) * BK * D, j, kcp, krp, vp, x);
        if (!filled) continue;
#pragma unroll
        for (int u = 0; u < 8; ++u) newk[r][t0 + u] = x[u];
        __syncthreads();   // newk rows come from other waves
        const int64_t gend = (Hkv < g0 + RPP) ? Hkv : g0 + RPP;
        for (int64_t gg = g0; gg < gend; ++gg) {
            const int64_t hp = page * Hkv + gg;
            stage_page<DT, D>(kcp + hp * BK * D, sm.kb, BK - 1, tid);
            for (int t = tid; t < D; t += 256) sm.kb[BK - 1][t] = newk[gg - g0][t];
            __syncthreads();
            summarize_staged<DT, D, true>(sm, probes + gg * m * D, proj + gg * D * D, m, att_scale,
                                          summ + hp * m * D, tid);
            __syncthreads();
        }
    }
    if (tid == 0) {
        const int64_t L = ok ? pos + 1 : pos;
        if (scales) scales[s] = scale_tab[(L < n_scale) ? (L > 0 ? L : 0) : n_scale - 1];
        if (ok) lens[s] = (int32_t)L;
    }
}

}  // namespace hba

using namespace hba;

// ------------------------------------------------------------ entry points --
extern "C" int hba_abi_version(void) { return HBA_ABI_VERSION; }

extern "C" const char *hba_status_string(int status) {
    switch (status) {
        case HBA_OK: return "ok";
        case HBA_ERR_INVALID_ARG: return "invalid argument";
        case HBA_ERR_UNSUPPORTED: return "unsupported shape or dtype";
        case HBA_ERR_DEVICE: return "no gfx950 device";
        case HBA_ERR_LAUNCH: return "kernel launch failed";
        case HBA_ERR_SCRATCH: return "request exceeds the fixed scratch of the no-allocation entry point";
        default: return "unknown status";
    }
}

extern "C" int hba_device_check(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return HBA_ERR_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return HBA_ERR_DEVICE;
    const char *a = prop.gcnArchName;
    if (!(a[0] == 'g' && a[1] == 'f' && a[2] == 'x' && a[3] == '9' && a[4] == '5' && a[5] == '0'))
        return HBA_ERR_DEVICE;
    return HBA_OK;
}

extern "C" int hba_prep_keys(int dtype, const void *k, const int64_t k_strides[3], const void *v,
                             const int64_t v_strides[3], const float *k_gain, float eps,
                             const float *cos_tab, const float *sin_tab, int64_t B, int64_t n,
                             int64_t Hkv, int64_t d, void *kc, void *kr, void *vt, void *stream) {
    if (dtype == HBA_DTYPE_F32 && d != 64 && d != 128) {   // fp32, another head dim: the generic kernel
        if (!gen_shape_ok(d, 1)) return HBA_ERR_UNSUPPORTED;
        if (!k || !k_strides || !kc || B <= 0 || n <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
        if ((kr && (!cos_tab || !sin_tab)) || (vt && (!v || !v_strides))) return HBA_ERR_INVALID_ARG;
        return gen_prep_keys((const float *)k, k_strides, (const float *)v, v_strides ? v_strides : k_strides,
                             k_gain, eps, cos_tab, sin_tab, B, n, Hkv, d, (float *)kc, (float *)kr, (float *)vt,
                             (hipStream_t)stream);
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!k || !k_strides || !kc || B <= 0 || n <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
    if (kr && (!cos_tab || !sin_tab)) return HBA_ERR_INVALID_ARG;
    if (vt && (!v || !v_strides)) return HBA_ERR_INVALID_ARG;
    if (kr && (!abi::aligned16(cos_tab) || !abi::aligned16(sin_tab))) return HBA_ERR_UNSUPPORTED;
    if (!abi::rows_aligned(dtype, k, k_strides) || (vt && !abi::rows_aligned(dtype, v, v_strides)) ||
        !abi::aligned16(kc) || (kr && !abi::aligned16(kr)))
        return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    const int64_t ntile = (n + 63) / 64;
    if (B * Hkv * ntile > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)(B * Hkv * ntile));
    const int64_t *vs = v_strides ? v_strides : k_strides;
#define HBA_PREP(DT, D)                                                                            \
    hipLaunchKernelGGL((prep_keys_kernel<DT, D>), grid, dim3(256), 0, s,                           \
                       (const St<DT>::T *)k, k_strides[0], k_strides[1], k_strides[2],             \
                       (const St<DT>::T *)v, vs[0], vs[1], vs[2], k_gain, eps, cos_tab, sin_tab, n, \
                       Hkv, ntile, (St<DT>::T *)kc, (St<DT>::T *)kr, (St<DT>::T *)vt)
    HBA_DISPATCH_DT_D(dtype, d, HBA_PREP);
#undef HBA_PREP
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_prep_keys_summarize(int dtype, const void *k, const int64_t k_strides[3], const void *v,
                                       const int64_t v_strides[3], const float *k_gain, float eps,
                                       const float *cos_tab, const float *sin_tab, int64_t B, int64_t n,
                                       int64_t Hkv, int64_t d, void *kc, void *kr, void *vt, const float *probes,
                                       const float *proj, int64_t m, void *S0, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!k || !k_strides || !kc || !probes || !proj || !S0 || B <= 0 || n <= 0 || Hkv <= 0)
        return HBA_ERR_INVALID_ARG;
    if (kr && (!cos_tab || !sin_tab)) return HBA_ERR_INVALID_ARG;
    if (vt && (!v || !v_strides)) return HBA_ERR_INVALID_ARG;
    if (m < 1 || m > 8) return HBA_ERR_UNSUPPORTED;
    if (kr && (!abi::aligned16(cos_tab) || !abi::aligned16(sin_tab))) return HBA_ERR_UNSUPPORTED;
    if (!abi::rows_aligned(dtype, k, k_strides) || (vt && !abi::rows_aligned(dtype, v, v_strides)) ||
        !abi::aligned16(kc) || (kr && !abi::aligned16(kr)))
        return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    const int64_t ntile = (n + 63) / 64;
    if (B * Hkv * ntile > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)(B * Hkv * ntile));
    const int64_t *vs = v_strides ? v_strides : k_strides;
    const float att_scale = (float)(1.0 / __builtin_sqrt((double)d));
#define HBA_PREP_SUMM(DT, D)                                                                       \
    hipLaunchKernelGGL((prep_summ_kernel<DT, D>), grid, dim3(256), 0, s,                           \
                       (const St<DT>::T *)k, k_strides[0], k_strides[1], k_strides[2],             \
                       (const St<DT>::T *)v, vs[0], vs[1], vs[2], k_gain, eps, cos_tab, sin_tab, n, \
                       Hkv, ntile, (St<DT>::T *)kc, (St<DT>::T *)kr, (St<DT>::T *)vt, probes, proj, \
                       (int)m, att_scale, (St<DT>::T *)S0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_PREP_SUMM);
#undef HBA_PREP_SUMM
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

static int summarize_common(int dtype, const void *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                            int64_t Bk, const int32_t *pages, const int32_t *ptab, int64_t maxp,
                            const int32_t *lens, int64_t nblocks, const float *probes,
                            const float *proj, int64_t m, void *out, void *stream) {
    if (dtype == HBA_DTYPE_F32 && !pages && !ptab && !tuned_shape(d, Bk)) {   // fp32 prefill, other geometry
        if (!kc || !probes || !proj || !out || B <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
        if (!gen_shape_ok(d, Bk) || m < 1 || m > 8) return HBA_ERR_UNSUPPORTED;
        if (nblocks <= 0) return HBA_OK;
        if (nblocks > 0x7fffffff || Hkv > 65535 || B > 65535) return HBA_ERR_UNSUPPORTED;
        return gen_summarize((const float *)kc, B, Hkv, n, d, Bk, nblocks, probes, proj, m, (float *)out,
                             (hipStream_t)stream);
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!kc || !probes || !proj || !out || B <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (m < 1 || m > 8) return HBA_ERR_UNSUPPORTED;
    if (nblocks <= 0) return HBA_OK;
    if (nblocks > 0x7fffffff || Hkv > 65535 || B > 65535) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(kc)) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)nblocks, (unsigned)Hkv, (unsigned)B);
    float att_scale = (float)(1.0 / __builtin_sqrt((double)d));
#define HBA_SUMM(DT, D)                                                                            \
    do {                                                                                           \
        if (ptab)                                                                                  \
            hipLaunchKernelGGL((summarize_kernel<DT, D, true>), grid, dim3(256), 0, s,             \
                               (const St<DT>::T *)kc, n, nblocks, Hkv, pages, ptab, maxp, lens,    \
                               probes, proj, (int)m, att_scale, (St<DT>::T *)out);                 \
        else                                                                                       \
            hipLaunchKernelGGL((summarize_kernel<DT, D, false>), grid, dim3(256), 0, s,            \
                               (const St<DT>::T *)kc, n, nblocks, Hkv, pages, ptab, maxp, lens,    \
                               probes, proj, (int)m, att_scale, (St<DT>::T *)out);                 \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_SUMM);
#undef HBA_SUMM
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_summarize(int dtype, const void *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                             int64_t Bk, const float *probes, const float *proj, int64_t m, void *S0,
                             void *stream) {
    if (Bk <= 0 || n <= 0) return HBA_ERR_INVALID_ARG;
    return summarize_common(dtype, kc, B, Hkv, n, d, Bk, nullptr, nullptr, 0, nullptr, n / Bk, probes,
                            proj, m, S0, stream);
}

extern "C" int hba_summarize_pages(int dtype, const void *kc_pages, const int32_t *pages,
                                   int64_t npages, int64_t Hkv, int64_t d, int64_t Bk,
                                   const float *probes, const float *proj, int64_t m,
                                   void *summ_pages, void *stream) {
    if (!pages || npages < 0) return HBA_ERR_INVALID_ARG;
    return summarize_common(dtype, kc_pages, 1, Hkv, Bk, d, Bk, pages, nullptr, 0, nullptr, npages,
                            probes, proj, m, summ_pages, stream);
}

extern "C" int hba_summarize_filled(int dtype, const void *kc_pages, const int32_t *page_table,
                                    int64_t max_pages, const int32_t *seq_lens, int64_t Bd,
                                    int64_t Hkv, int64_t d, int64_t Bk, const float *probes,
                                    const float *proj, int64_t m, void *summ_pages, void *stream) {
    if (!page_table || !seq_lens || max_pages <= 0 || Bd < 0) return HBA_ERR_INVALID_ARG;
    return summarize_common(dtype, kc_pages, 1, Hkv, Bk, d, Bk, nullptr, page_table, max_pages,
                            seq_lens, Bd, probes, proj, m, summ_pages, stream);
}

extern "C" int hba_build_super(int dtype, const void *S0, int64_t B, int64_t Hkv, int64_t nb,
                               int64_t m, int64_t d, int64_t fanout, void *S1, void *stream) {
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    if (!S0 || !S1 || B <= 0 || Hkv <= 0 || nb <= 0 || m <= 0 || d <= 0 || fanout <= 0)
        return HBA_ERR_INVALID_ARG;
    int64_t ns = (nb + fanout - 1) / fanout;
    int64_t total = B * Hkv * ns * m * d;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == HBA_DTYPE_F32)
        hipLaunchKernelGGL(build_super_kernel<0>, grid, dim3(256), 0, s, (const float *)S0, B * Hkv,
                           nb, m, d, fanout, (float *)S1);
    else
        hipLaunchKernelGGL(build_super_kernel<1>, grid, dim3(256), 0, s, (const bf16_t *)S0, B * Hkv,
                           nb, m, d, fanout, (bf16_t *)S1);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_kv_append_advance(int dtype, const void *k_new, const void *v_new,
                                     const float *k_gain, float eps, const float *cos_tab,
                                     const float *sin_tab, int64_t n_tab, const int32_t *page_table,
                                     int64_t max_pages, int32_t *seq_lens, int64_t Bd, int64_t Hkv,
                                     int64_t d, int64_t Bk, void *kc_pages, void *kr_pages,
                                     void *v_pages, const float *probes, const float *proj, int64_t m,
                                     void *summ_pages, const float *scale_tab, int64_t n_scale,
                                     float *scales, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!k_new || !v_new || !cos_tab || !sin_tab || !page_table || !seq_lens || !kc_pages ||
        !kr_pages || !v_pages || !probes || !proj || !summ_pages || Bd <= 0 || Hkv <= 0 ||
        max_pages <= 0 || n_tab <= 0 || (scales && (!scale_tab || n_scale <= 0)))
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64 || m < 1 || m > 8) return HBA_ERR_UNSUPPORTED;
    if (Bd > 0x7fffffff || Hkv > 65535) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(k_new) || !abi::aligned16(v_new) || !abi::aligned16(kc_pages) ||
        !abi::aligned16(kr_pages) || !abi::aligned16(v_pages))
        return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    const float att_scale = (float)(1.0 / __builtin_sqrt((double)d));
#define HBA_APPA(DT, D)                                                                            \
    hipLaunchKernelGGL((kv_append_advance_kernel<DT, D>), dim3((unsigned)Bd), dim3(256), 0, s,      \
                       (const St<DT>::T *)k_new, (const St<DT>::T *)v_new, k_gain, eps, cos_tab,    \
                       sin_tab, n_tab, page_table, max_pages, seq_lens, Hkv,                       \
                       (St<DT>::T *)kc_pages, (St<DT>::T *)kr_pages, (St<DT>::T *)v_pages, probes, \
                       proj, (int)m, att_scale, (St<DT>::T *)summ_pages, scale_tab, n_scale, scales)
    HBA_DISPATCH_DT_D(dtype, d, HBA_APPA);
#undef HBA_APPA
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_kv_append(int dtype, const void *k_new, const void *v_new, const float *k_gain,
                             float eps, const float *cos_tab, const float *sin_tab, int64_t n_tab,
                             const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                             int64_t Bd, int64_t Hkv, int64_t d, int64_t Bk, void *kc_pages,
                             void *kr_pages, void *v_pages, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!k_new || !v_new || !cos_tab || !sin_tab || !page_table || !seq_lens || !kc_pages ||
        !kr_pages || !v_pages || Bd <= 0 || Hkv <= 0 || max_pages <= 0 || n_tab <= 0)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (!abi::aligned16(k_new) || !abi::aligned16(v_new) || !abi::aligned16(kc_pages) ||
        !abi::aligned16(kr_pages) || !abi::aligned16(v_pages))
        return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    const int64_t rpp = 256 / (d / 8);   // token rows per workgroup
    if ((Bd * Hkv + rpp - 1) / rpp > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)((Bd * Hkv + rpp - 1) / rpp));
#define HBA_APP(DT, D)                                                                             \
    hipLaunchKernelGGL((kv_append_kernel<DT, D>), grid, dim3(256), 0, s, (const St<DT>::T *)k_new,   \
                       (const St<DT>::T *)v_new, k_gain, eps, cos_tab, sin_tab, page_table,        \
                       max_pages, seq_lens, n_tab, Bd, Hkv, (St<DT>::T *)kc_pages,                  \
                       (St<DT>::T *)kr_pages, (St<DT>::T *)v_pages)
    HBA_DISPATCH_DT_D(dtype, d, HBA_APP);
#undef HBA_APP
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
