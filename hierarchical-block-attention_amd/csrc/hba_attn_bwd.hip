// Backward of the union attention (the training path of hba_attention_dense /
// hba_attention_fused, src/hba/attention.py:306-356 and :552-607): gradients
// of the output with respect to the raw q, k, v and the QKNorm gains, with
// the block selection held fixed (the reference routes on detached q/k,
// attention.py:288-303, so no gradient reaches the selection).
//
// Per query row (b, i, h) the forward is one softmax over the disjoint union
// U_i = sinks (NoPE) + window (RoPE) + routed blocks (NoPE):
//   s_j = scale * <x_i, y_j>   (x, y = QKNorm'd q, k; rotated for window keys)
//   p = softmax(s), O_i = sum_j p_j v_j.
// With dO the output cotangent and D_i = <dO_i, O_i>:
//   ds_j = p_j (<dO_i, v_j> - D_i)
//   dx_i += scale ds_j y_j,  dy_j += scale ds_j x_i,  dv_j += p_j dO_i
// then the rotation's transpose (rope^T(z) = z cos + rot^T(z sin), rot^T(z) =
// [z2, -z1]) and the QKNorm backward
//   dx = g/r dy - [ms >= eps] x g <dy, x> / (d r^3),   dg += <dy, x> / r
// with r = sqrt(max(mean(x^2), eps)) (attention.py:88-94).  Arithmetic is
// fp32 throughout; storage roundings of the forward are treated as identity,
// as autograd treats the reference's casts.
//
// Two kernels:
//   bwd_dq:  one wave per (b, i, KV head g), lanes over d, the G heads of the
//            group in registers.  Pass 1 recomputes the union LSE, pass 2
//            accumulates dq; it also leaves the QKNorm'd and rotated query
//            rows, the LSE and D in the workspace for bwd_dkv.
//   bwd_dkv: one workgroup per (b, g, 64-key block); a lane holds 16 elements
//            of one key (keys x 16-element chunks per wave) and walks the
//            query rows that attend its keys: the window rows, the sink rows
//            (block 0), and the rows whose selection holds the block (found by
//            scanning the selection lists into LDS).
#include "hba_abi.h"
#include "hba_common.h"

namespace hba {
namespace bw {

constexpr int BW_GMAX = 16;

template <int D>
__device__ __forceinline__ float wsum(float v) {
    return wave_sum(v);
}

// element e of lane l is t = l + 64 e; GM = the largest group size held
template <int DT, int D, int GM>
__global__ __launch_bounds__(256) void bwd_dq_kernel(
    const typename St<DT>::T *__restrict__ q, const typename St<DT>::T *__restrict__ kc,
    const typename St<DT>::T *__restrict__ kr, const typename St<DT>::T *__restrict__ v,
    const float *__restrict__ qgain, float eps, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const typename St<DT>::T *__restrict__ out,
    const typename St<DT>::T *__restrict__ dout, int B, int64_t n, int Hq, int Hkv, int S, int64_t W, int kk,
    float scale, float *__restrict__ qc_ws, float *__restrict__ qr_ws, float *__restrict__ lse_ws,
    float *__restrict__ dd_ws, typename St<DT>::T *__restrict__ dq, float *__restrict__ dq_gain) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (int64_t)B * Hkv * n) return;                      // wave-uniform
    const int64_t i = wid % n;
    const int g = (int)((wid / n) % Hkv);
    const int b = (int)(wid / (n * Hkv));
    const int G = Hq / Hkv;
    const int64_t nb = n / 64;

    float xr[GM][E], qcv[GM][E], qrv[GM][E], dov[GM][E];
    float rr[GM], msr[GM], dd[GM];
    float cs[E], sn[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int t = lane + 64 * e;
        cs[e] = St<DT>::rnd(cosT[i * D + t]);
        sn[e] = St<DT>::rnd(sinT[i * D + t]);
    }
#pragma unroll
    for (int hh = 0; hh < GM; ++hh) {
        if (hh >= G) break;
        const int h = g * G + hh;
        const int64_t row = (((int64_t)b * n + i) * Hq + h) * D;
        float ss = 0.0f, od = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int t = lane + 64 * e;
            xr[hh][e] = St<DT>::ld(q, row + t);
            dov[hh][e] = St<DT>::ld(dout, row + t);
            ss = fmaf(xr[hh][e], xr[hh][e], ss);
            od = fmaf(dov[hh][e], St<DT>::ld(out, row + t), od);
        }
        dd[hh] = wsum<D>(od);
        msr[hh] = wsum<D>(ss) / (float)D;
        const float r = sqrtf(fmaxf(msr[hh], eps));
        rr[hh] = r;
#pragma unroll
        for (int e = 0; e < E; ++e)
            qcv[hh][e] = qgain ? St<DT>::rnd((xr[hh][e] / r) * qgain[h]) : xr[hh][e];
        // rotation: the partner of element t is t ^ (D/2)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int t = lane + 64 * e;
            const float pv = (D == 64) ? __shfl_xor(qcv[hh][0], 32, 64) : qcv[hh][e ^ 1];
            const float rot = (t < D / 2) ? -pv : pv;
            qrv[hh][e] = St<DT>::rnd(St<DT>::rnd(qcv[hh][e] * cs[e]) + St<DT>::rnd(rot * sn[e]));
            qc_ws[row + t] = qcv[hh][e];
            qr_ws[row + t] = qrv[hh][e];
        }
    }
    const int64_t bg = (int64_t)b * Hkv + g;
    const int64_t wlo = (S > i - W + 1) ? (int64_t)S : i - W + 1;   // window [wlo, i]
    const int64_t nsink = ((int64_t)S < i + 1) ? (int64_t)S : i + 1;
    const int ncnt = min(max(cnt[bg * n + i], 0), kk);
    const int32_t *sel = idx + (bg * n + i) * kk;
    // the keys of the union in a fixed order: sinks, window, routed picks
    const int64_t nwin = (i >= wlo) ? i - wlo + 1 : 0;                 // empty for i < S
    const int64_t nkeys = nsink + nwin + (int64_t)ncnt * 64;
    auto key_of = [&](int64_t u, bool &rope, bool &ok) -> int64_t {
        rope = false;
        ok = true;
        if (u < nsink) return u;
        u -= nsink;
        if (u < nwin) {
            rope = true;
            return wlo + u;
        }
        u -= nwin;
        const int blk = sel[u >> 6];
        ok = blk >= 1 && (int64_t)blk < nb;
        return ok ? 64 * (int64_t)blk + (u & 63) : 0;
    };
    const typename St<DT>::T *KC = kc + bg * n * D, *KR = kr + bg * n * D;

    // pass 1: the union LSE of each head
    float m[GM], l[GM];
#pragma unroll
    for (int hh = 0; hh < GM; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.0f;
    }
    for (int64_t u = 0; u < nkeys; ++u) {
        bool rope, ok;
        const int64_t j = key_of(u, rope, ok);
        if (!ok) continue;
        float kv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) kv[e] = St<DT>::ld(rope ? KR : KC, j * D + lane + 64 * e);
#pragma unroll
        for (int hh = 0; hh < GM; ++hh) {
            if (hh >= G) break;
            float pr = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) pr = fmaf(rope ? qrv[hh][e] : qcv[hh][e], kv[e], pr);
            const float s = wsum<D>(pr) * scale;
            const float mn = fmaxf(m[hh], s);
            l[hh] = l[hh] * __expf(m[hh] - mn) + __expf(s - mn);
            m[hh] = mn;
        }
    }
    float lse[GM];
#pragma unroll
    for (int hh = 0; hh < GM; ++hh) {
        if (hh >= G) break;
        lse[hh] = (l[hh] > 0.0f) ? m[hh] + __logf(l[hh]) : INFINITY;   // no key: every p is 0
        if (lane == 0) {
            const int64_t o = ((int64_t)b * Hq + g * G + hh) * n + i;
            lse_ws[o] = lse[hh];
            dd_ws[o] = dd[hh];
        }
    }

    // pass 2: dq (NoPE and rotated parts)
    float gc[GM][E], gr[GM][E];
#pragma unroll
    for (int hh = 0; hh < GM; ++hh)
#pragma unroll
        for (int e = 0; e < E; ++e) gc[hh][e] = gr[hh][e] = 0.0f;
    const typename St<DT>::T *V = v + ((int64_t)b * n * Hkv + g) * D;   // v[b, j, g, :] at j * Hkv * D
    for (int64_t u = 0; u < nkeys; ++u) {
        bool rope, ok;
        const int64_t j = key_of(u, rope, ok);
        if (!ok) continue;
        float kv[E], vv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            kv[e] = St<DT>::ld(rope ? KR : KC, j * D + lane + 64 * e);
            vv[e] = St<DT>::ld(V, j * Hkv * D + lane + 64 * e);
        }
#pragma unroll
        for (int hh = 0; hh < GM; ++hh) {
            if (hh >= G) break;
            float pr = 0.0f, pd = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                pr = fmaf(rope ? qrv[hh][e] : qcv[hh][e], kv[e], pr);
                pd = fmaf(dov[hh][e], vv[e], pd);
            }
            const float s = wsum<D>(pr) * scale;
            const float dp = wsum<D>(pd);
            const float p = __expf(s - lse[hh]);
            const float ds = p * (dp - dd[hh]) * scale;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (rope) gr[hh][e] = fmaf(ds, kv[e], gr[hh][e]);
                else gc[hh][e] = fmaf(ds, kv[e], gc[hh][e]);
            }
        }
    }

    // rope^T, then the QKNorm backward, per head
#pragma unroll
    for (int hh = 0; hh < GM; ++hh) {
        if (hh >= G) break;
        const int h = g * G + hh;
        const int64_t row = (((int64_t)b * n + i) * Hq + h) * D;
        float y[E], zs[E];
#pragma unroll
        for (int e = 0; e < E; ++e) zs[e] = gr[hh][e] * sn[e];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int t = lane + 64 * e;
            const float pv = (D == 64) ? __shfl_xor(zs[0], 32, 64) : zs[e ^ 1];
            y[e] = gc[hh][e] + gr[hh][e] * cs[e] + ((t < D / 2) ? pv : -pv);
        }
        if (qgain) {
            const float gn = qgain[h];
            const float r = rr[hh];
            float yx = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) yx = fmaf(y[e], xr[hh][e], yx);
            yx = wsum<D>(yx);
            const float corr = (msr[hh] >= eps) ? gn * yx / ((float)D * r * r * r) : 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) y[e] = (gn / r) * y[e] - xr[hh][e] * corr;
            if (lane == 0 && dq_gain) atomicAdd(&dq_gain[h], yx / r);
        }
#pragma unroll
        for (int e = 0; e < E; ++e) St<DT>::st(dq, row + lane + 64 * e, y[e]);
    }
}

// ------------------------------------------------------------- bwd_dkv ----
// Lane (kl, c) of wave w: key j = 64 blk + KW w + kl, elements 16c .. 16c+15.
template <int D>
struct DkvCfg {
    static constexpr int NC = D / 16;          // 16-element chunks per key
    static constexpr int KW = 64 / NC;         // keys per wave
    static constexpr int WAVES = 64 / KW;      // waves per 64-key block
    static constexpr int NT = WAVES * 64;
};

template <int D>
__device__ __forceinline__ float chunk_sum(float v) {
    constexpr int KW = DkvCfg<D>::KW;
#pragma unroll
    for (int o = KW; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int DT>
__device__ __forceinline__ void ld16(const typename St<DT>::T *p, float (&x)[16]) {
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = St<DT>::ld(p, e);
}

template <int DT, int D>
__global__ __launch_bounds__(DkvCfg<D>::NT) void bwd_dkv_kernel(
    const typename St<DT>::T *__restrict__ k, const typename St<DT>::T *__restrict__ kc,
    const typename St<DT>::T *__restrict__ kr, const typename St<DT>::T *__restrict__ v,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const typename St<DT>::T *__restrict__ dout,
    int64_t n, int Hq, int Hkv, int S, int64_t W, int kk, float scale, const float *__restrict__ qc_ws,
    const float *__restrict__ qr_ws, const float *__restrict__ lse_ws, const float *__restrict__ dd_ws,
    typename St<DT>::T *__restrict__ dk, typename St<DT>::T *__restrict__ dv, float *__restrict__ dk_gain) {
    using C = DkvCfg<D>;
    __shared__ int rows[C::NT];
    __shared__ int wcount[C::WAVES];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int kl = lane % C::KW, c = lane / C::KW;
    const int64_t nb = n / 64;
    const int blk = (int)(blockIdx.x % nb);
    const int g = (int)((blockIdx.x / nb) % Hkv);
    const int b = (int)(blockIdx.x / (nb * Hkv));
    const int G = Hq / Hkv;
    const int64_t j = 64 * (int64_t)blk + C::KW * w + kl;       // this lane's key
    const int64_t bg = (int64_t)b * Hkv + g;
    const int64_t kro = (bg * n + j) * D + 16 * c;              // kc / kr row chunk
    const int64_t rro = (((int64_t)b * n + j) * Hkv + g) * D + 16 * c;   // k / v / dk / dv row chunk
    float kcv[16], krv[16], vv[16], gkc[16], gkr[16], gv[16];
    ld16<DT>(kc + kro, kcv);
    ld16<DT>(kr + kro, krv);
    ld16<DT>(v + rro, vv);
#pragma unroll
    for (int e = 0; e < 16; ++e) gkc[e] = gkr[e] = gv[e] = 0.0f;

    // one query row (i, all G heads) against this lane's key; rope selects
    // the rotated operands; valid is the lane's own mask
    auto row_update = [&](int64_t i, bool rope, bool valid) {
        for (int hh = 0; hh < G; ++hh) {
            const int h = g * G + hh;
            const int64_t ro = (((int64_t)b * n + i) * Hq + h) * D + 16 * c;
            float x[16], dov[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) x[e] = (rope ? qr_ws : qc_ws)[ro + e];
            ld16<DT>(dout + ro, dov);
            const int64_t so = ((int64_t)b * Hq + h) * n + i;
            const float lse = lse_ws[so], ddv = dd_ws[so];
            float pr = 0.0f, pd = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                pr = fmaf(x[e], rope ? krv[e] : kcv[e], pr);
                pd = fmaf(dov[e], vv[e], pd);
            }
            const float s = chunk_sum<D>(pr) * scale;
            const float dp = chunk_sum<D>(pd);
            const float p = valid ? __expf(s - lse) : 0.0f;
            const float ds = p * (dp - ddv) * scale;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                gv[e] = fmaf(p, dov[e], gv[e]);
                if (rope) gkr[e] = fmaf(ds, x[e], gkr[e]);
                else gkc[e] = fmaf(ds, x[e], gkc[e]);
            }
        }
    };

    // window rows: key j >= S is in the window of queries j .. j + W - 1
    {
        const int64_t j0 = 64 * (int64_t)blk + C::KW * w;           // the wave's first key
        const int64_t ihi = min(n - 1, j0 + C::KW - 1 + W - 1);
        for (int64_t i = j0; i <= ihi; ++i) row_update(i, true, j >= S && i >= j && i <= j + W - 1);
    }
    // sink rows (NoPE): key j < S is attended by every query i >= j
    if (blk == 0 && C::KW * w < S) {
        for (int64_t i = C::KW * w; i < n; ++i) row_update(i, false, j < S && i >= j);
    }
    // routed rows (NoPE): the queries whose selection holds this block
    if (blk >= 1) {
        for (int64_t i0 = 0; i0 < n; i0 += C::NT) {
            const int64_t i = i0 + tid;
            bool picked = false;
            if (i < n) {
                const int nc = min(max(cnt[bg * n + i], 0), kk);
                const int32_t *sl = idx + (bg * n + i) * kk;
                for (int r = 0; r < nc; ++r) picked |= sl[r] == blk;
            }
            const uint64_t bal = __ballot(picked);
            if (lane == 0) wcount[w] = __popcll(bal);
            __syncthreads();
            int base = 0, tot = 0;
            for (int u = 0; u < C::WAVES; ++u) {
                if (u < w) base += wcount[u];
                tot += wcount[u];
            }
            if (picked) rows[base + __popcll(bal & ((1ull << lane) - 1ull))] = (int)i;
            __syncthreads();
            for (int e = 0; e < tot; ++e) row_update(rows[e], false, true);
            __syncthreads();                                     // rows[] and wcount[] reused
        }
    }

    // rope^T at position j, then the QKNorm backward of k row (b, j, g)
    float y[16];
    {
        float zs[16];
        const float *cp = cosT + j * D + 16 * c, *sp = sinT + j * D + 16 * c;
#pragma unroll
        for (int e = 0; e < 16; ++e) zs[e] = gkr[e] * St<DT>::rnd(sp[e]);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float pv = __shfl_xor(zs[e], 32, 64);             // chunk c ^ (NC/2): element t ^ (D/2)
            y[e] = gkc[e] + gkr[e] * St<DT>::rnd(cp[e]) + ((c < C::NC / 2) ? pv : -pv);
        }
    }
    if (kgain) {
        float x[16];
        ld16<DT>(k + rro, x);
        float ss = 0.0f, yx = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            ss = fmaf(x[e], x[e], ss);
            yx = fmaf(y[e], x[e], yx);
        }
        const float ms = chunk_sum<D>(ss) / (float)D;
        yx = chunk_sum<D>(yx);
        const float r = sqrtf(fmaxf(ms, eps));
        const float gn = kgain[g];
        const float corr = (ms >= eps) ? gn * yx / ((float)D * r * r * r) : 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) y[e] = (gn / r) * y[e] - x[e] * corr;
        if (c == 0 && dk_gain) atomicAdd(&dk_gain[g], yx / r);
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        St<DT>::st(dk, rro + e, y[e]);
        St<DT>::st(dv, rro + e, gv[e]);
    }
}

}  // namespace bw
}  // namespace hba

using namespace hba;

extern "C" int hba_attn_bwd_workspace_size(int64_t B, int64_t n, int64_t Hq, int64_t d, size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || d <= 0) return HBA_ERR_INVALID_ARG;
    *bytes = (size_t)(2 * B * n * Hq * d + 2 * B * Hq * n) * 4;
    return HBA_OK;
}

extern "C" int hba_attn_bwd(int dtype, const void *q, const void *k, const void *v, const void *kc, const void *kr,
                            const float *q_gain, const float *k_gain, float eps, const float *cos_tab,
                            const float *sin_tab, const int32_t *idx, const int32_t *cnt, const void *out,
                            const void *dout, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t S,
                            int64_t W, int64_t Bk, int64_t k_blocks, float scale, void *workspace, size_t ws_bytes,
                            void *dq, void *dk, void *dv, float *dq_gain, float *dk_gain, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !k || !v || !kc || !kr || !cos_tab || !sin_tab || !idx || !cnt || !out || !dout || !workspace ||
        !dq || !dk || !dv)
        return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || S < 0 || W < 1 || k_blocks < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0 || S > Bk) return HBA_ERR_INVALID_ARG;
    if (Hq / Hkv > bw::BW_GMAX) return HBA_ERR_UNSUPPORTED;
    if (B * Hkv * n > 0x7fffffffLL * 4 || B * Hkv * (n / 64) > 0x7fffffffLL || n > 0x7fffffffLL)
        return HBA_ERR_UNSUPPORTED;
    size_t need = 0;
    hba_attn_bwd_workspace_size(B, n, Hq, d, &need);
    if (ws_bytes < need || !abi::aligned16(workspace)) return HBA_ERR_INVALID_ARG;
    float *qc_ws = (float *)workspace;
    float *qr_ws = qc_ws + B * n * Hq * d;
    float *lse_ws = qr_ws + B * n * Hq * d;
    float *dd_ws = lse_ws + B * Hq * n;
    hipStream_t s = (hipStream_t)stream;
    const int64_t nwaves = B * Hkv * n;
    const int64_t g1 = (nwaves + 3) / 4;
    const int64_t g2 = B * Hkv * (n / 64);
#define HBA_BWD(DT, D)                                                                                          \
    do {                                                                                                        \
        using T = St<DT>::T;                                                                                    \
        if (Hq / Hkv <= 8)                                                                                      \
            hipLaunchKernelGGL((bw::bwd_dq_kernel<DT, D, 8>), dim3((unsigned)g1), dim3(256), 0, s,               \
                               (const T *)q, (const T *)kc, (const T *)kr, (const T *)v, q_gain, eps, cos_tab,   \
                               sin_tab, idx, cnt, (const T *)out, (const T *)dout, (int)B, n, (int)Hq, (int)Hkv, \
                               (int)S, W, (int)k_blocks, scale, qc_ws, qr_ws, lse_ws, dd_ws, (T *)dq, dq_gain);  \
        else                                                                                                    \
            hipLaunchKernelGGL((bw::bwd_dq_kernel<DT, D, bw::BW_GMAX>), dim3((unsigned)g1), dim3(256), 0, s,     \
                               (const T *)q, (const T *)kc, (const T *)kr, (const T *)v, q_gain, eps, cos_tab,   \
                               sin_tab, idx, cnt, (const T *)out, (const T *)dout, (int)B, n, (int)Hq, (int)Hkv, \
                               (int)S, W, (int)k_blocks, scale, qc_ws, qr_ws, lse_ws, dd_ws, (T *)dq, dq_gain);  \
        hipLaunchKernelGGL((bw::bwd_dkv_kernel<DT, D>), dim3((unsigned)g2), dim3(bw::DkvCfg<D>::NT), 0, s,       \
                           (const T *)k, (const T *)kc, (const T *)kr, (const T *)v, k_gain, eps, cos_tab,       \
                           sin_tab, idx, cnt, (const T *)dout, n, (int)Hq, (int)Hkv, (int)S, W, (int)k_blocks,   \
                           scale, qc_ws, qr_ws, lse_ws, dd_ws, (T *)dk, (T *)dv, dk_gain);                       \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_BWD);
#undef HBA_BWD
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
