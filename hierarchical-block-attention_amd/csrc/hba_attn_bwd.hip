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
// fp32 inputs take two VALU kernels:
//   bwd_dq:  one wave per (b, i, KV head g), lanes over d, the G heads of the
//            group in registers.  Pass 1 recomputes the union LSE, pass 2
//            accumulates dq; it also leaves the QKNorm'd and rotated query
//            rows, the LSE and D in the workspace for bwd_dkv.
//   bwd_dkv: one workgroup per (b, g, 64-key block); a lane holds 16 elements
//            of one key (keys x 16-element chunks per wave) and walks the
//            query rows that attend its keys: the window rows, the sink rows
//            (block 0), and the rows whose selection holds the block (found by
//            scanning the selection lists into LDS).
// bf16 inputs take the same gradients on MFMA: bwd_kt (transposed keys),
// bwd_dq_mfma (16/G queries per wave, their heads the columns of 16-wide
// tiles, one online pass), bwd_dkv_mfma (64 (row, head) pairs per tile, one
// workgroup per key block and row range)
// and bwd_dkv_fin (rope^T and the QKNorm backward of the key rows); a second
// bwd_dkv_mfma launch takes the sink keys.  The fp32 path takes the sink keys
// in bwd_sink.  Both split the sink keys' query rows over workgroups.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "hba_abi.h"
#include "hba_attn_bf16.h"
#include "hba_generic.h"
#include "hba_common.h"

namespace hba {
namespace bw {

constexpr int BW_GMAX = 16;

// Cross-lane sums on DPP (no LDS round trip): quad xor 1, quad xor 2,
// half-row mirror, row mirror leave every lane of a 16-lane row with the
// row's sum; the four rows are then added from their first lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_mov<0xb1>(v);    // quad_perm [1,0,3,2]
    v += dpp_mov<0x4e>(v);    // quad_perm [2,3,0,1]
    return v;
}
__device__ __forceinline__ float oct_sum(float v) {
    v = quad_sum(v);
    return v + dpp_mov<0x141>(v);   // row_half_mirror: the other quad of the 8
}
__device__ __forceinline__ float row16_sum(float v) {
    v = oct_sum(v);
    return v + dpp_mov<0x140>(v);   // row_mirror: the other 8 of the 16
}
template <int D>
__device__ __forceinline__ float wsum(float v) {
    v = row16_sum(v);
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (a + b) + (c + d);
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
    float *__restrict__ dd_ws, float *__restrict__ sink_acc, typename St<DT>::T *__restrict__ dq,
    float *__restrict__ dq_gain) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= (int64_t)B * Hkv * n) return;                      // wave-uniform
    const int64_t i = wid % n;
    const int g = (int)((wid / n) % Hkv);
    const int b = (int)(wid / (n * Hkv));
    const int G = Hq / Hkv;
    const int64_t nb = n / 64;
    if (i < 64) {   // clear key row i of the sink accumulators (bwd_sink adds into them next)
        float *acc = sink_acc + (((int64_t)b * Hkv + g) * 2 * 64 + i) * D;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[lane + 64 * e] = 0.0f;
            acc[64 * D + lane + 64 * e] = 0.0f;
        }
    }

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

// -------------------------------------------------- bwd_dq on MFMA (bf16) ----
// The same gradient as bwd_dq_kernel with every product on
// v_mfma_f32_16x16x32_bf16.  A wave takes qpw = 16 / G consecutive queries
// (at most 4) of one (b, g); the 16 tile columns are its (query, head) pairs
// (l16 = column).  The keys come in 64-key units (the sink unit, the window
// pages, the routed blocks):
//   S^T  = K . Q^T     (A: K rows in the permuted slot order kslot)
//   dP^T = V . dO^T    (A: V rows, same order)
//   dQ^T += K^T . dS^T (A: the transposed keys kct / krt; B: dS^T straight
//                       from the accumulators, which the slot order puts in
//                       the B-operand layout)
// One pass, online in the union softmax (running maximum, rescaled
// accumulators), since dS needs only D = <dO, O> besides p.  The window
// pages of a workgroup's four waves are staged once in LDS; the sink unit and
// the routed blocks are read per wave.
// Lane (l16, lg) holds, per M-tile mt, keys 32(mt>>1) + 8lg + 4(mt&1) + e of
// column l16, and of dQ^T the elements d = 16 dt + 4 lg + e.
typedef unsigned int u32x4b __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 ld_b8(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4b *>(p));
}
__device__ __forceinline__ bf16x8 pack_b8(const float (&x)[8]) {
    u32x4b u;
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = (uint32_t)f2bf(x[2 * e]) | ((uint32_t)f2bf(x[2 * e + 1]) << 16);
    return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int kslot(int mt, int r) { return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3); }
__device__ __forceinline__ int kkey(int mt, int lg, int e) { return 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e; }
__device__ __forceinline__ float col_max(float v) {   // over the 4 lanes of a column (lg)
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float col_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// Query rows per bwd_dkv_mfma workgroup (its row range), and the routed rows
// of each (range, key block) as bits: pbits [B, Hkv, nsplit, n / 64,
// PB_WORDS], bit i % DKV_ROWS of range i / DKV_ROWS set when row i's
// selection holds the block.
constexpr int DKV_ROWS = 4096;
constexpr int PB_WORDS = DKV_ROWS / 32;

// transposed prepared keys, kct / krt [B, Hkv, d, n]: one workgroup per 64-key
// tile; it also clears the tile's rows of the dk / dv accumulator dkv_acc
// [B, Hkv, n, 3, d] (bwd_dkv_mfma adds into it next) and the tile's routed-row
// bits of every range (bwd_pick_bits sets them next)
template <int D>
__global__ __launch_bounds__(256) void bwd_kt_kernel(const bf16_t *__restrict__ kc, const bf16_t *__restrict__ kr,
                                                     bf16_t *__restrict__ kct, bf16_t *__restrict__ krt, int64_t n,
                                                     float *__restrict__ dkv_acc, uint32_t *__restrict__ pbits,
                                                     int nsplit) {
    __shared__ bf16_t tile[64][D + 2];
    const int64_t nt = n / 64;
    const int64_t bg = blockIdx.x / nt, kb = (blockIdx.x % nt) * 64;
    {
        f32x4 *acc = reinterpret_cast<f32x4 *>(dkv_acc + (bg * n + kb) * 3 * D);
        for (int e = threadIdx.x; e < 64 * 3 * D / 4; e += 256) acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int64_t blk = blockIdx.x % nt;
        for (int e = threadIdx.x; e < nsplit * PB_WORDS; e += 256)
            pbits[((bg * nsplit + e / PB_WORDS) * nt + blk) * PB_WORDS + e % PB_WORDS] = 0u;
    }
    for (int pass = 0; pass < 2; ++pass) {
        const bf16_t *src = (pass ? kr : kc) + (bg * n + kb) * D;
        bf16_t *dst = (pass ? krt : kct) + bg * D * n + kb;
        for (int e = threadIdx.x; e < 64 * D; e += 256) tile[e / D][e % D] = src[e];
        __syncthreads();
        for (int e = threadIdx.x; e < 64 * D; e += 256) dst[(int64_t)(e / 64) * n + (e % 64)] = tile[e % 64][e / 64];
        __syncthreads();
    }
}

// The routed rows of every key block as bits (layout above): one thread per
// (b, g, row, pick); atomic ORs, so the bits are the same in any order.  A
// block picked twice by a row sets one bit, as the row attends it once.
__global__ __launch_bounds__(256) void bwd_pick_bits_kernel(const int32_t *__restrict__ idx,
                                                            const int32_t *__restrict__ cnt, int64_t n, int64_t nb,
                                                            int kk, int64_t total, int nsplit,
                                                            uint32_t *__restrict__ pbits) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= total) return;                                       // total = B Hkv n kk
    const int64_t row = t / kk;                                   // bg n + i
    const int r = (int)(t - row * kk);
    if (r >= min(max(cnt[row], 0), kk)) return;
    const int v = idx[t];
    if (v < 1 || v >= nb) return;                                 // block 0 is never routed
    const int64_t bg = row / n, i = row - bg * n;
    const int li = (int)(i % DKV_ROWS);
    atomicOr(&pbits[((bg * nsplit + i / DKV_ROWS) * nb + v) * PB_WORDS + (li >> 5)], 1u << (li & 31));
}

template <int D>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void bwd_dq_mfma_kernel(
    const bf16_t *__restrict__ q, const bf16_t *__restrict__ kc, const bf16_t *__restrict__ kr,
    const bf16_t *__restrict__ kct, const bf16_t *__restrict__ krt, const bf16_t *__restrict__ v,
    const float *__restrict__ qgain, float eps, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const bf16_t *__restrict__ out,
    const bf16_t *__restrict__ dout, int B, int64_t n, int Hq, int Hkv, int S, int64_t W, int kk, float scale,
    int qpw, bf16_t *__restrict__ qc_ws, bf16_t *__restrict__ qr_ws, float *__restrict__ lse_ws,
    float *__restrict__ dd_ws, float *__restrict__ sink_acc, bf16_t *__restrict__ dq, float *__restrict__ dq_gain) {
    constexpr int NKS = D / 32, NDT = D / 16, E = D / 64;
    // the window pages of the workgroup's queries, staged once for its four
    // waves: K and V rows [64][D + 8], K^T rows [D][64 + 8]
    constexpr int KS = D + 8, TS = 64 + 8, NCK = D / 8, CPK = D / 32;
    __shared__ __align__(16) bf16_t wk[2][64 * KS];
    __shared__ __align__(16) bf16_t wv[2][64 * KS];
    __shared__ __align__(16) bf16_t wkt[2][D * TS];
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int G = Hq / Hkv;
    const int64_t nw = (n + qpw - 1) / qpw;                       // query waves per (b, g)
    const int64_t nwg = (nw + 3) / 4;                             // workgroups per (b, g)
    const int64_t wgi = blockIdx.x % nwg;
    const int64_t wq = 4 * wgi + (tid >> 6);
    const bool act = wq < nw;              // wave-uniform; an idle wave still stages and meets every barrier
    const int64_t i0 = act ? wq * qpw : 0;                        // the wave's first query row
    const int g = (int)((blockIdx.x / nwg) % Hkv);
    const int b = (int)(blockIdx.x / (nwg * Hkv));
    const int64_t nb = n / 64;
    const int64_t bg = (int64_t)b * Hkv + g;
    for (int qq = 0; act && qq < qpw; ++qq) {   // clear key row i of the sink accumulators (bwd_sink adds into them next)
        const int64_t ic = i0 + qq;
        if (ic >= 64 || ic >= n) break;
        float *acc = sink_acc + (bg * 2 * 64 + ic) * D;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[lane + 64 * e] = 0.0f;
            acc[64 * D + lane + 64 * e] = 0.0f;
        }
    }
    // column l16 = (query qs of the wave, head l16 - qs G)
    const int qs = l16 / G;
    const int64_t iq = i0 + qs;
    const bool hv = act && qs < qpw && iq < n;
    const int64_t i = hv ? iq : i0;                               // a row in range for every column
    const int h = g * G + (hv ? l16 - qs * G : 0);
    const int64_t row = (((int64_t)b * n + i) * Hq + h) * D;

    // query row elements t = 32 ks + 8 lg + e of this column: raw, dO, O
    float x[NKS][8], dov[NKS][8];
    float ss = 0.0f, od = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t o = row + 32 * ks + 8 * lg + e;
            x[ks][e] = hv ? bf2f(q[o]) : 0.0f;
            dov[ks][e] = hv ? bf2f(dout[o]) : 0.0f;
            ss = fmaf(x[ks][e], x[ks][e], ss);
            od = fmaf(dov[ks][e], hv ? bf2f(out[o]) : 0.0f, od);
        }
    const float ms = col_sum(ss) / (float)D;
    const float rq = sqrtf(fmaxf(ms, eps));
    const float Dh = col_sum(od);
    const float gn = (qgain && hv) ? qgain[h] : 1.0f;
    float qcv[NKS][8];
    bf16x8 qopc[NKS], qopr[NKS], dop[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qcv[ks][e] = qgain ? rnd_bf16((x[ks][e] / rq) * gn) : x[ks][e];
        qopc[ks] = pack_b8(qcv[ks]);
        dop[ks] = pack_b8(dov[ks]);
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        float qrv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int t = 32 * ks + 8 * lg + e;
            const float pv = qcv[ks ^ (NKS / 2)][e];                    // element t ^ (D/2)
            const float rot = (t < D / 2) ? -pv : pv;
            const float c = rnd_bf16(cosT[i * D + t]), sn = rnd_bf16(sinT[i * D + t]);
            qrv[e] = rnd_bf16(rnd_bf16(qcv[ks][e] * c) + rnd_bf16(rot * sn));
            if (hv) {
                qc_ws[row + t] = f2bf(qcv[ks][e]);                      // bf16-exact values
                qr_ws[row + t] = f2bf(qrv[e]);
            }
        }
        qopr[ks] = pack_b8(qrv);
    }

    // the units of each wave, shared by its queries: the sink unit, then the
    // routed picks of each query in turn; a block an earlier query of the wave
    // also picked is skipped (it was taken then, for every query that holds
    // it).  The window pages, from the workgroup's first query's window start
    // to its last query, are taken by the whole workgroup from LDS.
    const int64_t nsink = hv ? (((int64_t)S < i + 1) ? (int64_t)S : i + 1) : 0;
    const int64_t wlo = (S > i - W + 1) ? (int64_t)S : i - W + 1;
    const int64_t iw0 = 4 * wgi * qpw, iw1 = min(n - 1, 4 * (wgi + 1) * qpw - 1);
    const int64_t wlo0 = (S > iw0 - W + 1) ? (int64_t)S : iw0 - W + 1;
    const int64_t npg = (iw1 >= wlo0) ? iw1 / 64 - wlo0 / 64 + 1 : 0;
    const int64_t nwu = 0;
    const int hs = (act && S > 0) ? 1 : 0;
    int ncq[4];                                                    // picks per query of the wave (qpw <= 4)
    int nrt = 0;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        ncq[qq] = (act && qq < qpw && i0 + qq < n) ? min(max(cnt[bg * n + i0 + qq], 0), kk) : 0;
        nrt += ncq[qq];
    }
    // the picks of the wave, one per lane (entry lane + 64 t = query x kk + r)
    int ent[2], entq[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int en = lane + 64 * t, qe = en / kk, r = en % kk;
        const bool ok = act && qe < qpw && i0 + qe < n && r < min(max(cnt[bg * n + min(i0 + qe, n - 1)], 0), kk);
        ent[t] = ok ? idx[(bg * n + i0 + qe) * kk + r] : -1;
        entq[t] = qe;
    }
    const int64_t nunits = hs + nwu + nrt;
    auto unit = [&](int64_t u, int64_t &kb, int64_t &lo, int64_t &hi, bool &rope) -> bool {
        rope = false;
        if (u < hs) {
            kb = 0;
            lo = 0;
            hi = nsink - 1;
            return true;
        }
        u -= hs;
        if (u < nwu) {
            rope = true;
            kb = 64 * (wlo0 / 64 + u);
            lo = (wlo > kb) ? wlo : kb;
            hi = !hv ? kb - 1 : (i < kb + 63) ? i : kb + 63;
            return true;
        }
        int e = (int)(u - nwu), qp = 0;
#pragma unroll
        for (int qq = 0; qq < 3; ++qq)
            if (qp == qq && e >= ncq[qq]) {
                e -= ncq[qq];
                qp = qq + 1;
            }
        const int blk = idx[(bg * n + i0 + qp) * kk + e];
        if (blk < 1 || (int64_t)blk >= nb) return false;
        unsigned has = 1u << qp;                                   // its own query, whatever kk
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const bool m0 = ent[0] == blk && entq[0] == qq, m1 = ent[1] == blk && entq[1] == qq;
            if (__ballot(m0) | __ballot(m1)) has |= 1u << qq;
        }
        if (has & ((1u << qp) - 1u)) return false;                // an earlier query of the wave took it
        kb = 64 * (int64_t)blk;
        lo = kb;
        hi = (hv && ((has >> qs) & 1u)) ? kb + 63 : kb - 1;
        return true;
    };
    auto scores = [&](int64_t kb, bool rope, f32x4 (&Sa)[4]) {
        const bf16_t *K = (rope ? kr : kc) + (bg * n + kb) * D;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const bf16_t *kp = K + (int64_t)kslot(mt, l16) * D + 8 * lg;
            Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) Sa[mt] = mfma16(ld_b8(kp + 32 * ks), rope ? qopr[ks] : qopc[ks], Sa[mt]);
        }
    };

    // staging of window page kb: K rows (both passes), V and K^T rows (pass 2)
    u32x4b rk[CPK], rv[CPK], rt[CPK];
    auto wload = [&](int64_t kb, bool full) {
#pragma unroll
        for (int c = 0; c < CPK; ++c) {
            const int qc = tid + 256 * c, kr_ = qc / NCK, kc_ = (qc % NCK) * 8, dr = qc / 8, kcol = (qc % 8) * 8;
            rk[c] = *reinterpret_cast<const u32x4b *>(kr + (bg * n + kb + kr_) * D + kc_);
            if (full) {
                rv[c] = *reinterpret_cast<const u32x4b *>(v + (((int64_t)b * n + kb + kr_) * Hkv + g) * D + kc_);
                rt[c] = *reinterpret_cast<const u32x4b *>(krt + (bg * D + dr) * n + kb + kcol);
            }
        }
    };
    auto wstore = [&](int bf, bool full) {
#pragma unroll
        for (int c = 0; c < CPK; ++c) {
            const int qc = tid + 256 * c, kr_ = qc / NCK, kc_ = (qc % NCK) * 8, dr = qc / 8, kcol = (qc % 8) * 8;
            *reinterpret_cast<u32x4b *>(&wk[bf][kr_ * KS + kc_]) = rk[c];
            if (full) {
                *reinterpret_cast<u32x4b *>(&wv[bf][kr_ * KS + kc_]) = rv[c];
                *reinterpret_cast<u32x4b *>(&wkt[bf][dr * TS + kcol]) = rt[c];
            }
        }
    };
    // this column's keys of window page kb
    auto wrange = [&](int64_t kb, int64_t &lo, int64_t &hi) {
        lo = (wlo > kb) ? wlo : kb;
        hi = !hv ? kb - 1 : (i < kb + 63) ? i : kb + 63;
    };

    // one pass, online in the union softmax of column l16: with m the running
    // maximum of its scaled scores and l = sum exp(s - m), the accumulators
    // hold sum_j exp(s_j - m) (dP_j - D) scale k_j and are rescaled when m
    // grows; dq = acc / l and the LSE m + log l at the end (D = <dO, O> needs
    // no LSE).  A unit may hold no key of a column.
    f32x4 gc[NDT], gr[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) gc[dt] = gr[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    // Sa, Pa of a unit at keys kb..; KT = the unit's K^T rows (row stride kts)
    // from this lane's key offset 8 lg
    auto grad_acc = [&](const f32x4 (&Sa)[4], const f32x4 (&Pa)[4], int64_t kb, int64_t lo, int64_t hi,
                        const bf16_t *KT, int64_t kts, bool rope) {
        float mu = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t key = kb + kkey(mt, lg, e);
                if (key >= lo && key <= hi) mu = fmaxf(mu, Sa[mt][e] * scale);
            }
        mu = col_max(mu);
        const float mn = fmaxf(m, mu);
        const float alpha = (m == -INFINITY) ? 0.0f : __expf(m - mn);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            gc[dt] *= alpha;
            gr[dt] *= alpha;
        }
        float dsv[2][8], ps = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t key = kb + kkey(mt, lg, e);
                const float p = (key >= lo && key <= hi) ? __expf(Sa[mt][e] * scale - mn) : 0.0f;
                ps += p;
                dsv[mt >> 1][(mt & 1) * 4 + e] = p * (Pa[mt][e] - Dh) * scale;
            }
        l = l * alpha + col_sum(ps);
        m = mn;
        const bf16x8 db0 = pack_b8(dsv[0]), db1 = pack_b8(dsv[1]);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const bf16_t *ktp = KT + (int64_t)(16 * dt + l16) * kts;
            f32x4 a = rope ? gr[dt] : gc[dt];
            a = mfma16(ld_b8(ktp), db0, a);
            a = mfma16(ld_b8(ktp + 32), db1, a);
            if (rope) gr[dt] = a;
            else gc[dt] = a;
        }
    };
    for (int64_t u = 0; u < nunits; ++u) {
        int64_t kb, lo, hi;
        bool rope;
        if (!unit(u, kb, lo, hi, rope)) continue;
        f32x4 Sa[4], Pa[4];
        scores(kb, rope, Sa);
        const bf16_t *V = v + (((int64_t)b * n + kb) * Hkv + g) * D;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const bf16_t *vp = V + (int64_t)kslot(mt, l16) * Hkv * D + 8 * lg;
            Pa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) Pa[mt] = mfma16(ld_b8(vp + 32 * ks), dop[ks], Pa[mt]);
        }
        grad_acc(Sa, Pa, kb, lo, hi, (rope ? krt : kct) + bg * D * n + kb + 8 * lg, n, rope);
    }
    if (npg > 0) {                                                // workgroup-uniform
        wload(64 * (wlo0 / 64), true);
        wstore(0, true);
        __syncthreads();
        for (int64_t pg = 0; pg < npg; ++pg) {
            const int64_t kb = 64 * (wlo0 / 64 + pg);
            if (pg + 1 < npg) wload(kb + 64, true);
            if (act) {
                const bf16_t *Kp = wk[pg & 1], *Vp = wv[pg & 1];
                f32x4 Sa[4], Pa[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    Sa[mt] = Pa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) {
                        Sa[mt] = mfma16(ld_b8(Kp + kslot(mt, l16) * KS + 8 * lg + 32 * ks), qopr[ks], Sa[mt]);
                        Pa[mt] = mfma16(ld_b8(Vp + kslot(mt, l16) * KS + 8 * lg + 32 * ks), dop[ks], Pa[mt]);
                    }
                }
                int64_t lo, hi;
                wrange(kb, lo, hi);
                grad_acc(Sa, Pa, kb, lo, hi, wkt[pg & 1] + 8 * lg, TS, true);
            }
            if (pg + 1 < npg) wstore((pg + 1) & 1, true);
            __syncthreads();
        }
    }
    const float lse = (l > 0.0f) ? m + __logf(l) : INFINITY;
    if (hv && lg == 0) {
        lse_ws[((int64_t)b * Hq + h) * n + i] = lse;
        dd_ws[((int64_t)b * Hq + h) * n + i] = Dh;
    }
    {
        const float il = (l > 0.0f) ? 1.0f / l : 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            gc[dt] *= il;
            gr[dt] *= il;
        }
    }

    // rope^T and the QKNorm backward on elements d = 16 dt + 4 lg + e
    float y[NDT][4], xr[NDT][4];
    float yx = 0.0f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = 16 * dt + 4 * lg + e;
            const float zp = gr[dt ^ (NDT / 2)][e] * rnd_bf16(sinT[i * D + (d ^ (D / 2))]);   // (z sin) at d ^ D/2
            y[dt][e] = gc[dt][e] + gr[dt][e] * rnd_bf16(cosT[i * D + d]) + ((d < D / 2) ? zp : -zp);
            xr[dt][e] = hv ? bf2f(q[row + d]) : 0.0f;
            yx = fmaf(y[dt][e], xr[dt][e], yx);
        }
    yx = col_sum(yx);
    if (qgain) {
        const float corr = (ms >= eps) ? gn * yx / ((float)D * rq * rq * rq) : 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) y[dt][e] = (gn / rq) * y[dt][e] - xr[dt][e] * corr;
    }
    if (hv) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) dq[row + 16 * dt + 4 * lg + e] = f2bf(y[dt][e]);
    }
    // the gain gradient: summed over the workgroup's queries per head before
    // one atomic add per head (the adds of all workgroups meet on Hq floats)
    if (qgain && dq_gain) {                                       // workgroup-uniform
        __shared__ float gqs[4][16];
        if (lg == 0) gqs[tid >> 6][l16] = hv ? yx / rq : 0.0f;
        __syncthreads();
        if (tid < G) {
            float t = 0.0f;
            for (int w4 = 0; w4 < 4; ++w4)
                for (int qq = 0; qq < qpw; ++qq) t += gqs[w4][qq * G + tid];
            unsafeAtomicAdd(&dq_gain[g * G + tid], t);
        }
    }
}

// ------------------------------------------------------------- bwd_dkv ----
// Lane (kl, c) = (lane / NC, lane % NC) of wave w: key j = 64 blk + KW w + kl,
// elements 16c .. 16c+15; a key's chunks sit on NC adjacent lanes, so its
// sums are DPP steps within a quad (NC = 4) or an 8-lane group (NC = 8).
template <int D>
struct DkvCfg {
    static constexpr int NC = D / 16;          // 16-element chunks per key
    static constexpr int KW = 64 / NC;         // keys per wave
    static constexpr int WAVES = 64 / KW;      // waves per 64-key block
    static constexpr int NT = WAVES * 64;
};

template <int D>
__device__ __forceinline__ float chunk_sum(float v) {
    if constexpr (DkvCfg<D>::NC == 4) return quad_sum(v);
    else return oct_sum(v);
}

template <int DT>
__device__ __forceinline__ void ld16(const typename St<DT>::T *p, float (&x)[16]) {
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = St<DT>::ld(p, e);
}

// nrows query rows (row_of(r)), all G heads of KV head g, against this lane's
// key j: accumulates gk += ds * x (x = the stored query rows qx_ws: NoPE or
// rotated) and gv += p * dO.  mode 0: window rows (j >= S, j <= i <= j+W-1),
// 1: sink rows (j < S, i >= j), 2: routed rows (every key of the block).  The
// next row's operands are loaded while the current one is computed.
template <int DT, int D, typename RowOf>
__device__ __forceinline__ void dkv_rows(RowOf row_of, int64_t nrows, int mode, int64_t j, int S, int64_t W,
                                         const float *qx_ws, const typename St<DT>::T *dout,
                                         const float *lse_ws, const float *dd_ws, int b, int64_t n, int Hq,
                                         int g, int G, int c, float scale, const float (&ky)[16],
                                         const float (&vv)[16], float (&gk)[16], float (&gv)[16]) {
    const int64_t total = nrows * G;
    if (total <= 0) return;
    auto load = [&](int64_t u, float (&x)[16], float (&dv)[16], float &lse, float &dd, int64_t &i) {
        i = row_of(u / G);
        const int h = g * G + (int)(u % G);
        const int64_t ro = (((int64_t)b * n + i) * Hq + h) * D + 16 * c;
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = qx_ws[ro + e];
        ld16<DT>(dout + ro, dv);
        const int64_t so = ((int64_t)b * Hq + h) * n + i;
        lse = lse_ws[so];
        dd = dd_ws[so];
    };
    auto compute = [&](const float (&x)[16], const float (&dov)[16], float lse, float dd, int64_t i) {
        const bool valid = (mode == 0) ? (j >= S && i >= j && i <= j + W - 1) : (mode == 1) ? (j < S && i >= j)
                                                                                           : true;
        float pr = 0.0f, pd = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            pr = fmaf(x[e], ky[e], pr);
            pd = fmaf(dov[e], vv[e], pd);
        }
        const float sc = chunk_sum<D>(pr) * scale;
        const float dp = chunk_sum<D>(pd);
        const float p = valid ? __expf(sc - lse) : 0.0f;
        const float ds = p * (dp - dd) * scale;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            gv[e] = fmaf(p, dov[e], gv[e]);
            gk[e] = fmaf(ds, x[e], gk[e]);
        }
    };
    float xa[16], da[16], xb[16], db[16], la, ldd, lb, ldb;
    int64_t ia, ib;
    load(0, xa, da, la, ldd, ia);
    for (int64_t u = 0; u < total; u += 2) {
        if (u + 1 < total) load(u + 1, xb, db, lb, ldb, ib);
        compute(xa, da, la, ldd, ia);
        if (u + 1 >= total) break;
        if (u + 2 < total) load(u + 2, xa, da, la, ldd, ia);
        compute(xb, db, lb, ldb, ib);
    }
}

// Sink keys (block 0, j < S) against query rows [r0, r0 + SINK_ROWS): one
// workgroup per (b, g, row range), the lanes laid out as in bwd_dkv; the
// partial gradients are added (fp32 atomics) into sink_acc [B, Hkv, 2, 64, D]
// (dk then dv), which bwd_dkv's block-0 workgroup reads.
constexpr int SINK_ROWS = 256;

template <int DT, int D>
__global__ __launch_bounds__(DkvCfg<D>::NT) void bwd_sink_kernel(
    const typename St<DT>::T *__restrict__ kc, const typename St<DT>::T *__restrict__ v,
    const typename St<DT>::T *__restrict__ dout, int64_t n, int Hq, int Hkv, int S, int nsplit, float scale,
    const float *__restrict__ qc_ws, const float *__restrict__ lse_ws, const float *__restrict__ dd_ws,
    float *__restrict__ sink_acc) {
    using C = DkvCfg<D>;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int kl = lane / C::NC, c = lane % C::NC;
    const int split = (int)(blockIdx.x % nsplit);
    const int g = (int)((blockIdx.x / nsplit) % Hkv);
    const int b = (int)(blockIdx.x / ((int64_t)nsplit * Hkv));
    const int G = Hq / Hkv;
    if (C::KW * w >= S) return;                                   // wave-uniform; no barrier follows
    const int64_t j = C::KW * w + kl;
    const int64_t bg = (int64_t)b * Hkv + g;
    float kcv[16], vv[16], gkc[16], gv[16];
    ld16<DT>(kc + (bg * n + j) * D + 16 * c, kcv);
    ld16<DT>(v + (((int64_t)b * n + j) * Hkv + g) * D + 16 * c, vv);
#pragma unroll
    for (int e = 0; e < 16; ++e) gkc[e] = gv[e] = 0.0f;
    const int64_t r0 = (int64_t)split * SINK_ROWS;
    const int64_t r1 = min(n, r0 + SINK_ROWS);
    dkv_rows<DT, D>([&](int64_t r) { return r0 + r; }, r1 - r0, 1, j, S, 0, qc_ws, dout, lse_ws, dd_ws, b, n, Hq, g,
                    G, c, scale, kcv, vv, gkc, gv);
    if (j < S) {
        float *acc = sink_acc + (bg * 2 * 64 + j) * D + 16 * c;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            atomicAdd(acc + e, gkc[e]);
            atomicAdd(acc + 64 * D + e, gv[e]);
        }
    }
}

template <int DT, int D>
__global__ __launch_bounds__(DkvCfg<D>::NT) void bwd_dkv_kernel(
    const typename St<DT>::T *__restrict__ k, const typename St<DT>::T *__restrict__ kc,
    const typename St<DT>::T *__restrict__ kr, const typename St<DT>::T *__restrict__ v,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const typename St<DT>::T *__restrict__ dout,
    int64_t n, int Hq, int Hkv, int S, int64_t W, int kk, float scale, const float *__restrict__ qc_ws,
    const float *__restrict__ qr_ws, const float *__restrict__ lse_ws, const float *__restrict__ dd_ws,
    const float *__restrict__ sink_acc, typename St<DT>::T *__restrict__ dk, typename St<DT>::T *__restrict__ dv,
    float *__restrict__ dk_gain) {
    using C = DkvCfg<D>;
    __shared__ int rows[C::NT];
    __shared__ int wcount[C::WAVES];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int kl = lane / C::NC, c = lane % C::NC;
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

    // window rows (rotated): key j >= S is in the window of queries j .. j + W - 1
    {
        const int64_t j0 = 64 * (int64_t)blk + C::KW * w;           // the wave's first key
        const int64_t ihi = min(n - 1, j0 + C::KW - 1 + W - 1);
        dkv_rows<DT, D>([&](int64_t r) { return j0 + r; }, ihi - j0 + 1, 0, j, S, W, qr_ws, dout, lse_ws, dd_ws, b,
                        n, Hq, g, G, c, scale, krv, vv, gkr, gv);
    }
    // sink keys (NoPE): every query i >= j; their rows were split over the
    // bwd_sink workgroups, whose sums are added here
    if (blk == 0 && j < S) {
        const float *acc = sink_acc + (bg * 2 * 64 + j) * D + 16 * c;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            gkc[e] += acc[e];
            gv[e] += acc[64 * D + e];
        }
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
            dkv_rows<DT, D>([&](int64_t r) { return (int64_t)rows[r]; }, tot, 2, j, S, W, qc_ws, dout, lse_ws, dd_ws,
                            b, n, Hq, g, G, c, scale, kcv, vv, gkc, gv);
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
            const float pv = __shfl_xor(zs[e], C::NC / 2, 64);      // chunk c ^ (NC/2): element t ^ (D/2)
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

// ------------------------------------------------ bwd_dkv on MFMA (bf16) ----
// dK and dV of one 64-key block from the (query row, head) pairs that attend
// it, 64 pairs per tile staged in LDS twice (row-major and transposed), taken
// as two halves of 32 (the contraction of one product); wave w
// owns keys kb + 16 w .. kb + 16 w + 15:
//   S   = X . K^T    (A: staged query rows X, pairs in the slot order pslot;
//                     B: the wave's key rows, held in registers)
//   dP  = dO . V^T   (A: staged dO rows; B: the wave's V rows)
//   dV += P^T . dO   (A: P^T straight from the accumulators, which the slot
//                     order puts in the A-operand layout; B: dO^T from the
//                     transposed copy)
//   dK += dS^T . X   (A: dS^T the same way; B: X^T)
// Lane (l16, lg) holds S and dP of key l16 and pairs 8 lg + 4 mt + e, and of
// dV / dK the element d = 16 dt + l16 of keys 16 w + 4 lg + e.
// One workgroup per (b, g, 64-key block, range of DKV_ROWS query rows): the
// window rows (rotated, X = qr) and the routed rows (NoPE, X = qc; found by
// scanning the range's selection lists) of its range.  Its sums are added
// (fp32 atomics) into dkv_acc [B, Hkv, n, 3, d] (NoPE dk, rotated dk, dv),
// which bwd_dkv_fin turns into dk and dv.  The split over row ranges keeps a
// block that nearly every query selects from becoming the tail.
// With sink_rows > 0 the launch takes the sink keys instead: one workgroup
// per (b, g, range of sink_rows rows) against block 0, every row of the range
// attending the keys j < S with j <= i (NoPE); waves whose 16 keys hold no
// sink skip the products.
constexpr int DKV_RL = 1024;   // routed rows run as one series of tiles at most
constexpr int DKV_TP = 64;   // pairs per tile: two halves of 32, the pair count of one product

__device__ __forceinline__ int pslot(int mt, int r) { return 8 * (r >> 2) + 4 * mt + (r & 3); }

template <int D>
struct DkvTile {
    static constexpr int XP = D + 8;        // padded row of the row-major copies
    static constexpr int TP = DKV_TP + 8;   // padded row of the transposed copies
    alignas(16) bf16_t xs[DKV_TP * XP];
    alignas(16) bf16_t os[DKV_TP * XP];
    alignas(16) bf16_t xt[D * TP];
    alignas(16) bf16_t ot[D * TP];
    alignas(16) float lse[DKV_TP];
    alignas(16) float dd[DKV_TP];
    alignas(16) int row[DKV_TP];
};

// 512 threads: wave w takes keys 16 (w & 3) .. + 15 of the block and pairs
// 32 (w >> 2) .. + 31 of each 64-pair tile (4 waves per SIMD at d = 64, so
// that one wave's LDS -> MFMA -> exp -> MFMA chain overlaps the others'); the
// two halves add their sums into the same accumulator rows.
constexpr int DKV_NT = 512;
template <int D>
__global__ __launch_bounds__(DKV_NT, D == 64 ? 4 : 2) void bwd_dkv_mfma_kernel(
    const bf16_t *__restrict__ kc, const bf16_t *__restrict__ kr, const bf16_t *__restrict__ v,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const bf16_t *__restrict__ dout, int64_t n,
    int Hq, int Hkv, int S, int64_t W, int kk, float scale, int nsplit, const bf16_t *__restrict__ qc_ws,
    const bf16_t *__restrict__ qr_ws, const float *__restrict__ lse_ws, const float *__restrict__ dd_ws,
    const float *__restrict__ cosT, const float *__restrict__ sinT, const uint32_t *__restrict__ pbits,
    float *__restrict__ dkv_acc, int sink_rows) {
    constexpr int NKS = D / 32, NDT = D / 16, NCH = D / 8, CPT = DKV_TP * NCH / DKV_NT;
    static_assert(CPT * DKV_NT == DKV_TP * NCH, "a tile's 16-byte chunks split evenly over the threads");
    using Tl = DkvTile<D>;
    constexpr int XP = Tl::XP, TP = Tl::TP;
    __shared__ Tl tl[2];
    __shared__ int rows[DKV_RL];
    __shared__ int wcount[DKV_NT / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, lg = lane >> 4;
    const int kg = w & 3, hw = w >> 2;   // this wave's 16 keys and 32-pair half of each tile
    const bool sinks = sink_rows > 0;
    const int64_t nb = sinks ? 1 : n / 64;
    const int split = (int)(blockIdx.x % nsplit);
    const int64_t blk = (blockIdx.x / nsplit) % nb;
    const int64_t bg = blockIdx.x / ((int64_t)nsplit * nb);
    const int g = (int)(bg % Hkv), b = (int)(bg / Hkv);
    const int G = Hq / Hkv;
    const int64_t kb = 64 * blk;
    const int64_t rows_per = sinks ? (int64_t)sink_rows : (int64_t)DKV_ROWS;
    const int64_t r0 = (int64_t)split * rows_per, r1 = min(n, r0 + rows_per);
    const int64_t jl = kb + 16 * kg + l16;   // the key of this lane's S / dP column

    // the key operand of the current rows (kr rows for the window, kc rows
    // for the sinks and routed rows) and the value rows
    bf16x8 kop[NKS], vb[NKS];
    auto load_k = [&](const bf16_t *kt) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kop[ks] = ld_b8(kt + (bg * n + jl) * D + 32 * ks + 8 * lg);
    };
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) vb[ks] = ld_b8(v + (((int64_t)b * n + jl) * Hkv + g) * D + 32 * ks + 8 * lg);
    // dk in the NoPE frame (the window rows' sums, taken in the rotated frame,
    // are mapped back by rope^T before the routed rows add theirs) and dv;
    // lane (l16, lg) holds keys kb + 16 kg + 4 lg + e, elements 16 dt + l16
    f32x4 gk[NDT], gv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) gk[dt] = gv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // rope^T(z) = z cos + rot^T(z sin) at each key's position, with the
    // tables rounded to bf16 as apply_rope's; an element's rotation partner
    // d ^ D/2 is element dt ^ NDT/2 of the same lane
    auto rope_t = [&]() {
        float cs[NDT][4], sn[NDT][4];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t j = kb + 16 * kg + 4 * lg + e;
                cs[dt][e] = rnd_bf16(cosT[j * D + 16 * dt + l16]);
                sn[dt][e] = rnd_bf16(sinT[j * D + 16 * dt + l16]);
            }
        f32x4 y[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pd = dt ^ (NDT / 2);
                const float zp = gk[pd][e] * sn[pd][e];
                y[dt][e] = gk[dt][e] * cs[dt][e] + ((dt < NDT / 2) ? zp : -zp);
            }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) gk[dt] = y[dt];
    };

    // pairs gp = 0 .. total-1: query row row_of(gp / G), head g G + gp % G;
    // mode 0: window rows (rotated), 1: routed rows, 2: sink rows (NoPE)
    auto run = [&](int64_t total, auto row_of, int mode) {
        const bool rope = mode == 0;
        const bf16_t *qx = rope ? qr_ws : qc_ws;
        const int64_t ntl = (total + DKV_TP - 1) / DKV_TP;
        u32x4b xr[CPT], orr[CPT];
        float plse[CPT], pdd[CPT];
        int prow[CPT];
        auto load = [&](int64_t t) {
#pragma unroll
            for (int r = 0; r < CPT; ++r) {
                const int q = tid + DKV_NT * r, p = q / NCH, c = q % NCH;
                const int64_t gp = t * DKV_TP + p;
                plse[r] = INFINITY;
                pdd[r] = 0.0f;
                prow[r] = -1;
                if (gp < total) {
                    const int64_t i = row_of(gp / G);
                    const int h = g * G + (int)(gp % G);
                    const int64_t ro = (((int64_t)b * n + i) * Hq + h) * D + 8 * c;
                    xr[r] = *reinterpret_cast<const u32x4b *>(qx + ro);
                    orr[r] = *reinterpret_cast<const u32x4b *>(dout + ro);
                    if (c == 0) {
                        const int64_t so = ((int64_t)b * Hq + h) * n + i;
                        plse[r] = lse_ws[so];
                        pdd[r] = dd_ws[so];
                        prow[r] = (int)i;
                    }
                } else {
                    xr[r] = orr[r] = u32x4b{0u, 0u, 0u, 0u};
                }
            }
        };
        auto store = [&](Tl &T) {
#pragma unroll
            for (int r = 0; r < CPT; ++r) {
                const int q = tid + DKV_NT * r, p = q / NCH, c = q % NCH;
                *reinterpret_cast<u32x4b *>(&T.xs[p * XP + 8 * c]) = xr[r];
                *reinterpret_cast<u32x4b *>(&T.os[p * XP + 8 * c]) = orr[r];
                // transposed rows d = 8 c + e, this pair in 8-pair group (p >> 3) ^ (c & 7)
                const int tc = ((((p >> 3) ^ c) & 7) << 3) | (p & 7);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    T.xt[(8 * c + e) * TP + tc] = (bf16_t)(xr[r][e >> 1] >> (16 * (e & 1)));
                    T.ot[(8 * c + e) * TP + tc] = (bf16_t)(orr[r][e >> 1] >> (16 * (e & 1)));
                }
                if (c == 0) {
                    T.lse[p] = plse[r];
                    T.dd[p] = pdd[r];
                    T.row[p] = prow[r];
                }
            }
        };
        auto compute = [&](const Tl &T) {
            if (mode == 2 && 16 * kg >= S) return;                 // no sink among the wave's keys
          {
            const int hp = hw;
            if (T.row[32 * hp] < 0) return;                        // padding (pairs fill in order)
            f32x4 Sa[2], Pa[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const bf16_t *xa = &T.xs[(32 * hp + pslot(mt, l16)) * XP + 8 * lg];
                const bf16_t *oa = &T.os[(32 * hp + pslot(mt, l16)) * XP + 8 * lg];
                Sa[mt] = Pa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    Sa[mt] = mfma16(ld_b8(xa + 32 * ks), kop[ks], Sa[mt]);
                    Pa[mt] = mfma16(ld_b8(oa + 32 * ks), vb[ks], Pa[mt]);
                }
            }
            float pk[8], dk[8];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const int pp = 32 * hp + 8 * lg + 4 * mt;
                const f32x4 ls = *reinterpret_cast<const f32x4 *>(&T.lse[pp]);
                const f32x4 ds = *reinterpret_cast<const f32x4 *>(&T.dd[pp]);
                const int4 rw = *reinterpret_cast<const int4 *>(&T.row[pp]);
                const int ri[4] = {rw.x, rw.y, rw.z, rw.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t i = ri[e];
                    const bool valid = (mode == 0) ? (jl >= S && i >= jl && i <= jl + W - 1)
                                     : (mode == 1) ? (i >= 0)
                                                   : (jl < S && i >= jl);
                    const float p = valid ? __expf(Sa[mt][e] * scale - ls[e]) : 0.0f;
                    pk[4 * mt + e] = p;
                    dk[4 * mt + e] = p * (Pa[mt][e] - ds[e]) * scale;
                }
            }
            const bf16x8 pa = pack_b8(pk), da = pack_b8(dk);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const int dr = 16 * dt + l16;                      // pairs 32 hp + 8 lg .. + 7 of row dr
                const int to = dr * TP + ((((4 * hp + lg) ^ (dr >> 3)) & 7) << 3);
                gv[dt] = mfma16(pa, ld_b8(&T.ot[to]), gv[dt]);
                gk[dt] = mfma16(da, ld_b8(&T.xt[to]), gk[dt]);
            }
          }
        };
        if (ntl <= 0) return;
        load(0);
        store(tl[0]);
        __syncthreads();
        for (int64_t t = 0; t < ntl; ++t) {
            if (t + 1 < ntl) load(t + 1);
            compute(tl[t & 1]);
            if (t + 1 < ntl) store(tl[(t + 1) & 1]);
            __syncthreads();
        }
    };

    bool had_win = false, had_rt = false;
    if (sinks) {
        had_rt = true;
        load_k(kc);
        run((r1 - r0) * G, [&](int64_t r) { return r0 + r; }, 2);
    }
    // window rows: key j >= S is in the window of queries j .. j + W - 1
    if (!sinks) {
        const int64_t wa = max(kb, r0);
        const int64_t wb = min(min(n - 1, kb + 63 + W - 1), r1 - 1);
        if (wb >= wa) {
            had_win = true;
            load_k(kr);
            run((wb - wa + 1) * G, [&](int64_t r) { return wa + r; }, 0);
            rope_t();
        }
    }
    // routed rows: the queries of the range whose selection holds this block,
    // read from its bits (ascending), run in series of at most DKV_RL rows
    if (!sinks && blk >= 1) {
        load_k(kc);
        const uint32_t *bits = pbits + ((bg * nsplit + split) * nb + blk) * PB_WORDS;
        const uint32_t word = (tid < PB_WORDS) ? bits[tid] : 0u;   // rows r0 + 32 tid ..
        const int c = __popc(word);
        int incl = c;   // prefix over the words (threads 0 .. PB_WORDS - 1: two waves)
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        static_assert(PB_WORDS == 128, "the words' prefix spans two waves");
        if (lane == 63 && w < 2) wcount[w] = incl;
        __syncthreads();
        const int pos = incl - c + ((w == 1) ? wcount[0] : 0);     // the word's first row's position
        const int total = wcount[0] + wcount[1];
        for (int run0 = 0; run0 < total; run0 += DKV_RL) {
            __syncthreads();                                      // rows[] consumed (and wcount[] read)
            if (word) {
                uint32_t wd = word;
                int p = pos;
                while (wd) {
                    const int bit = __ffs(wd) - 1;
                    wd &= wd - 1u;
                    if (p >= run0 && p < run0 + DKV_RL) rows[p - run0] = (int)(r0 + 32 * tid + bit);
                    ++p;
                }
            }
            __syncthreads();                                      // rows[] complete
            had_rt = true;
            const int tot = min(DKV_RL, total - run0);
            run((int64_t)tot * G, [&](int64_t r) { return (int64_t)rows[r]; }, 1);
        }
    }

    if (sinks && 16 * kg >= S) return;                             // after the last barrier
    float *acc = dkv_acc + (bg * n + kb + 16 * kg + 4 * lg) * 3 * D + l16;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (sinks && 16 * kg + 4 * lg + e >= S) continue;
            float *a = acc + e * 3 * D + 16 * dt;
            if (had_rt || had_win) {   // dk in the NoPE slot; the rotated slot stays zero
                unsafeAtomicAdd(a, gk[dt][e]);
                unsafeAtomicAdd(a + 2 * D, gv[dt][e]);
            }
        }
}

// dk / dv of key rows (b, j, g), lane = element d (and d + 64); a wave takes
// FIN_RPW consecutive rows, a workgroup one 64-key block: the summed NoPE /
// rotated dk and dv (plus the sink accumulators for j < S), rope^T at
// position j, then the QKNorm backward of k row (b, j, g).  The gain gradient
// is summed over the workgroup's 64 rows before its one atomic add (the adds
// of all workgroups meet on Hkv addresses).
constexpr int FIN_RPW = 16;
template <int D>
__global__ __launch_bounds__(256) void bwd_dkv_fin_kernel(
    const bf16_t *__restrict__ k, const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t n, int Hkv, int S, const float *__restrict__ dkv_acc,
    const float *__restrict__ sink_acc, bf16_t *__restrict__ dk, bf16_t *__restrict__ dv,
    float *__restrict__ dk_gain) {
    constexpr int E = D / 64;
    __shared__ float gsum[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t bg = blockIdx.x / (n / 64);                     // a workgroup never spans two (b, g)
    const int g = (int)(bg % Hkv), b = (int)(bg / Hkv);
    float gsv = 0.0f;
    for (int rr = 0; rr < FIN_RPW; ++rr) {
        const int64_t wid = (int64_t)blockIdx.x * 64 + w * FIN_RPW + rr;   // bg n + j
        const int64_t j = wid % n;
        const float *a = dkv_acc + wid * 3 * D;
        float gkc[E], gkr[E], gv[E], zs[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = lane + 64 * e;
            gkc[e] = a[d];
            gkr[e] = a[D + d];
            gv[e] = a[2 * D + d];
            if (j < S && sink_acc) {
                const float *sa = sink_acc + (bg * 2 * 64 + j) * D;
                gkc[e] += sa[d];
                gv[e] += sa[64 * D + d];
            }
            zs[e] = gkr[e] * rnd_bf16(sinT[j * D + d]);
        }
        float y[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int d = lane + 64 * e;
            const float pv = (E == 1) ? __shfl_xor(zs[0], 32, 64) : zs[e ^ 1];   // element d ^ (D/2)
            y[e] = gkc[e] + gkr[e] * rnd_bf16(cosT[j * D + d]) + ((d < D / 2) ? pv : -pv);
        }
        const int64_t rro = (((int64_t)b * n + j) * Hkv + g) * D;
        if (kgain) {
            float x[E], ss = 0.0f, yx = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[e] = bf2f(k[rro + lane + 64 * e]);
                ss = fmaf(x[e], x[e], ss);
                yx = fmaf(y[e], x[e], yx);
            }
            const float ms = wsum<D>(ss) / (float)D;
            yx = wsum<D>(yx);
            const float r = sqrtf(fmaxf(ms, eps));
            const float gn = kgain[g];
            const float corr = (ms >= eps) ? gn * yx / ((float)D * r * r * r) : 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) y[e] = (gn / r) * y[e] - x[e] * corr;
            gsv += yx / r;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            dk[rro + lane + 64 * e] = f2bf(y[e]);
            dv[rro + lane + 64 * e] = f2bf(gv[e]);
        }
    }
    if (kgain && dk_gain) {
        if (lane == 0) gsum[w] = gsv;
        __syncthreads();
        if (threadIdx.x == 0) unsafeAtomicAdd(&dk_gain[g], (gsum[0] + gsum[1]) + (gsum[2] + gsum[3]));
    }
}

}  // namespace bw
}  // namespace hba

using namespace hba;

// The bf16 query gradient: the union kernel (launch_attn_bf16_dq: 64 queries
// per workgroup sharing each staged block) where it takes the geometry, else
// bwd_dq_mfma.  HBA_BWD_DQ_KERNEL=pair in the environment selects
// bwd_dq_mfma (16/G queries per wave) everywhere.
static bool bwd_dq_union_on() {
    const char *e = getenv("HBA_BWD_DQ_KERNEL");
    return !(e && !strcmp(e, "pair"));
}

// Workspace of hba_attn_bwd: the query rows in the storage type (QKNorm'd,
// rotated), LSE and D per (head, row), the fp32 sink accumulators
// [B, Hkv, 2, 64, d]; on the bf16 path also the transposed keys kct, krt
// [B, Hkv, d, n] and the fp32 dk / dv accumulators [B, Hkv, n, 3, d].
namespace {
struct BwdWs {
    size_t qc, qr, lse, dd, sink, kct, krt, dkv, pbits, total;
};
size_t bw_align(size_t x) { return (x + 255) & ~(size_t)255; }
BwdWs bwd_ws_layout(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d) {
    BwdWs L{};
    size_t o = 0;
    auto take = [&](size_t bytes) {
        const size_t r = o;
        o = bw_align(o + bytes);
        return r;
    };
    const size_t qe = dtype == HBA_DTYPE_BF16 ? 2 : 4;
    L.qc = take((size_t)(B * n * Hq * d) * qe);
    L.qr = take((size_t)(B * n * Hq * d) * qe);
    L.lse = take((size_t)(B * Hq * n) * 4);
    L.dd = take((size_t)(B * Hq * n) * 4);
    L.sink = take((size_t)(B * Hkv * 2 * 64 * d) * 4);
    if (dtype == HBA_DTYPE_BF16) {
        L.kct = take((size_t)(B * Hkv * d * n) * 2);
        L.krt = take((size_t)(B * Hkv * d * n) * 2);
        L.dkv = take((size_t)(B * Hkv * n * 3 * d) * 4);
        const int64_t nsplit = (n + bw::DKV_ROWS - 1) / bw::DKV_ROWS;
        L.pbits = take((size_t)(B * Hkv * nsplit * (n / 64) * bw::PB_WORDS) * 4);
    }
    L.total = o;
    return L;
}
}  // namespace

extern "C" int hba_attn_bwd_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                                            size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || d <= 0) return HBA_ERR_INVALID_ARG;
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    *bytes = bwd_ws_layout(dtype, B, n, Hq, Hkv, d).total;
    if (dtype == HBA_DTYPE_F32) *bytes = std::max(*bytes, gen_bwd_ws_bytes(B, n, Hkv, d));   // the generic path
    return HBA_OK;
}

extern "C" int hba_attn_bwd_workspace_size(int64_t B, int64_t n, int64_t Hq, int64_t d, size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || d <= 0) return HBA_ERR_INVALID_ARG;
    // an upper bound for either dtype and any Hkv <= Hq
    *bytes = bwd_ws_layout(HBA_DTYPE_BF16, B, n, Hq, Hq, d).total + (size_t)(2 * B * n * Hq * d) * 2;
    *bytes = std::max(*bytes, gen_bwd_ws_bytes(B, n, Hq, d));   // the fp32 generic path
    return HBA_OK;
}

extern "C" int hba_attn_bwd(int dtype, const void *q, const void *k, const void *v, const void *kc, const void *kr,
                            const float *q_gain, const float *k_gain, float eps, const float *cos_tab,
                            const float *sin_tab, const int32_t *idx, const int32_t *cnt, const void *out,
                            const void *dout, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t S,
                            int64_t W, int64_t Bk, int64_t k_blocks, float scale, void *workspace, size_t ws_bytes,
                            void *dq, void *dk, void *dv, float *dq_gain, float *dk_gain, void *stream) {
    // fp32 off the tuned kernels' geometry (block != 64, head dim not 64 /
    // 128, more sinks than one block, k > 64, more query heads per KV head
    // than they take): the generic kernels
    const bool gen_geo = !tuned_shape(d, Bk) || S > Bk || k_blocks > 64 ||
                         (Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv > bw::BW_GMAX);
    if (dtype == HBA_DTYPE_F32 && gen_geo) {
        if (!q || !k || !v || !kc || !kr || !cos_tab || !sin_tab || !idx || !cnt || !out || !dout || !workspace ||
            !dq || !dk || !dv)
            return HBA_ERR_INVALID_ARG;
        if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || S < 0 || W < 1 || k_blocks < 1 || Bk < 1)
            return HBA_ERR_INVALID_ARG;
        if (!gen_shape_ok(d, Bk)) return HBA_ERR_UNSUPPORTED;
        if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
        if (ws_bytes < gen_bwd_ws_bytes(B, n, Hkv, d) || !abi::aligned16(workspace)) return HBA_ERR_INVALID_ARG;
        return gen_attn_bwd((const float *)q, (const float *)k, (const float *)v, (const float *)kc,
                            (const float *)kr, q_gain, k_gain, eps, cos_tab, sin_tab, idx, cnt, (const float *)out,
                            (const float *)dout, B, n, Hq, Hkv, d, S, W, Bk, k_blocks, scale, (float *)workspace,
                            (float *)dq, (float *)dk, (float *)dv, dq_gain, dk_gain, (hipStream_t)stream);
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !k || !v || !kc || !kr || !cos_tab || !sin_tab || !idx || !cnt || !out || !dout || !workspace ||
        !dq || !dk || !dv)
        return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || S < 0 || W < 1 || k_blocks < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
    // (bf16 reaches here with these; fp32 took the generic path above)
    if (S > Bk || k_blocks > 64 || Hq / Hkv > bw::BW_GMAX) return HBA_ERR_UNSUPPORTED;
    if (B * Hkv * n > 0x7fffffffLL * 4 || B * Hkv * (n / 64) > 0x7fffffffLL || n > 0x7fffffffLL)
        return HBA_ERR_UNSUPPORTED;
    const BwdWs L = bwd_ws_layout(dtype, B, n, Hq, Hkv, d);
    if (ws_bytes < L.total || !abi::aligned16(workspace)) return HBA_ERR_INVALID_ARG;
    char *wsb = (char *)workspace;
    float *qc_ws = (float *)(wsb + L.qc);                          // fp32 path's query rows
    float *qr_ws = (float *)(wsb + L.qr);
    bf16_t *qcb_ws = (bf16_t *)(wsb + L.qc);                       // bf16 path's query rows
    bf16_t *qrb_ws = (bf16_t *)(wsb + L.qr);
    float *lse_ws = (float *)(wsb + L.lse);
    float *dd_ws = (float *)(wsb + L.dd);
    float *sink_acc = (float *)(wsb + L.sink);                     // [B, Hkv, 2, 64, d]
    bf16_t *kct = (bf16_t *)(wsb + L.kct);                         // [B, Hkv, d, n] (bf16 path)
    bf16_t *krt = (bf16_t *)(wsb + L.krt);
    float *dkv_acc = (float *)(wsb + L.dkv);                       // [B, Hkv, n, 3, d] (bf16 path)
    uint32_t *pbits = (uint32_t *)(wsb + L.pbits);                 // routed-row bits (bf16 path)
    hipStream_t s = (hipStream_t)stream;
    const int64_t nwaves = B * Hkv * n;
    const int64_t g1 = (nwaves + 3) / 4;
    const int64_t g2 = B * Hkv * (n / 64);
    const int nsplit = (int)((n + bw::SINK_ROWS - 1) / bw::SINK_ROWS);
    const int64_t gs = B * Hkv * nsplit;
    // queries per bwd_dq_mfma wave: 16 / G tile columns, at most 4, with
    // every pick of the wave's queries held one per lane in two registers
    int qpw = (int)std::min<int64_t>(4, 16 / (Hq / Hkv));
    while (qpw > 1 && qpw * k_blocks > 128) --qpw;
    const int64_t g1q = B * Hkv * (((n + qpw - 1) / qpw + 3) / 4);   // whole workgroups per (b, g)
    const int nsplit_kv = (int)((n + bw::DKV_ROWS - 1) / bw::DKV_ROWS);
    const int64_t g3 = B * Hkv * (n / 64) * nsplit_kv;
    const int64_t g4 = B * Hkv * (n / 64);                        // bwd_dkv_fin: one workgroup per 64-key block
    const int64_t gpb = (B * Hkv * n * k_blocks + 255) / 256;     // bwd_pick_bits: a thread per pick
    if (gpb > 0x7fffffffLL) return HBA_ERR_UNSUPPORTED;
    if (g3 > 0x7fffffffLL) return HBA_ERR_UNSUPPORTED;
#define HBA_BWD(DT, D)                                                                                          \
    do {                                                                                                        \
        using T = St<DT>::T;                                                                                    \
        if constexpr (DT == 1) {                                                                                \
            hipLaunchKernelGGL((bw::bwd_kt_kernel<D>), dim3((unsigned)g2), dim3(256), 0, s, (const bf16_t *)kc,  \
                               (const bf16_t *)kr, kct, krt, n, dkv_acc, pbits, nsplit_kv);                      \
            hipLaunchKernelGGL(bw::bwd_pick_bits_kernel, dim3((unsigned)gpb), dim3(256), 0, s, idx, cnt, n,      \
                               n / 64, (int)k_blocks, B * Hkv * n * k_blocks, nsplit_kv, pbits);                 \
            int dqs = HBA_ERR_UNSUPPORTED;                                                                      \
            if constexpr (D == 64)                                                                              \
                if (bwd_dq_union_on())                                                                              \
                    dqs = launch_attn_bf16_dq<D>(q, q_gain, k_gain, eps, kc, kr, kct, krt, v, cos_tab, sin_tab,  \
                                                 idx, cnt, out, dout, B, n, Hq, Hkv, S, W, k_blocks, scale,      \
                                                 qcb_ws, qrb_ws, lse_ws, dd_ws, dq, dq_gain, s);                 \
            if (dqs == HBA_ERR_UNSUPPORTED)                                                                     \
                hipLaunchKernelGGL((bw::bwd_dq_mfma_kernel<D>), dim3((unsigned)g1q), dim3(256), 0, s,            \
                                   (const bf16_t *)q, (const bf16_t *)kc, (const bf16_t *)kr, kct, krt,         \
                                   (const bf16_t *)v, q_gain, eps, cos_tab, sin_tab, idx, cnt,                  \
                                   (const bf16_t *)out, (const bf16_t *)dout, (int)B, n, (int)Hq, (int)Hkv,     \
                                   (int)S, W, (int)k_blocks, scale, qpw, qcb_ws, qrb_ws, lse_ws, dd_ws,         \
                                   sink_acc, (bf16_t *)dq, dq_gain);                                            \
            else if (dqs != HBA_OK)                                                                             \
                return dqs;                                                                                     \
        } else if (Hq / Hkv <= 8)                                                                               \
            hipLaunchKernelGGL((bw::bwd_dq_kernel<DT, D, 8>), dim3((unsigned)g1), dim3(256), 0, s,               \
                               (const T *)q, (const T *)kc, (const T *)kr, (const T *)v, q_gain, eps, cos_tab,   \
                               sin_tab, idx, cnt, (const T *)out, (const T *)dout, (int)B, n, (int)Hq, (int)Hkv, \
                               (int)S, W, (int)k_blocks, scale, qc_ws, qr_ws, lse_ws, dd_ws, sink_acc, (T *)dq,   \
                               dq_gain);                                                                        \
        else                                                                                                    \
            hipLaunchKernelGGL((bw::bwd_dq_kernel<DT, D, bw::BW_GMAX>), dim3((unsigned)g1), dim3(256), 0, s,     \
                               (const T *)q, (const T *)kc, (const T *)kr, (const T *)v, q_gain, eps, cos_tab,   \
                               sin_tab, idx, cnt, (const T *)out, (const T *)dout, (int)B, n, (int)Hq, (int)Hkv, \
                               (int)S, W, (int)k_blocks, scale, qc_ws, qr_ws, lse_ws, dd_ws, sink_acc, (T *)dq,   \
                               dq_gain);                                                                        \
        if (S > 0 && DT == 0)                                                                                   \
            hipLaunchKernelGGL((bw::bwd_sink_kernel<DT, D>), dim3((unsigned)gs), dim3(bw::DkvCfg<D>::NT), 0, s,  \
                               (const T *)kc, (const T *)v, (const T *)dout, n, (int)Hq, (int)Hkv, (int)S,       \
                               nsplit, scale, qc_ws, lse_ws, dd_ws, sink_acc);                                   \
        if constexpr (DT == 1) {                                                                                \
            if (S > 0)                                                                                          \
                hipLaunchKernelGGL((bw::bwd_dkv_mfma_kernel<D>), dim3((unsigned)gs), dim3(bw::DKV_NT), 0, s,     \
                                   (const bf16_t *)kc, (const bf16_t *)kr, (const bf16_t *)v, idx, cnt,          \
                                   (const bf16_t *)dout, n, (int)Hq, (int)Hkv, (int)S, W, (int)k_blocks, scale,  \
                                   nsplit, qcb_ws, qrb_ws, lse_ws, dd_ws, cos_tab, sin_tab, pbits, dkv_acc,     \
                                   bw::SINK_ROWS);                                                              \
            hipLaunchKernelGGL((bw::bwd_dkv_mfma_kernel<D>), dim3((unsigned)g3), dim3(bw::DKV_NT), 0, s,         \
                               (const bf16_t *)kc, (const bf16_t *)kr, (const bf16_t *)v, idx, cnt,              \
                               (const bf16_t *)dout, n, (int)Hq, (int)Hkv, (int)S, W, (int)k_blocks, scale,      \
                               nsplit_kv, qcb_ws, qrb_ws, lse_ws, dd_ws, cos_tab, sin_tab, pbits, dkv_acc, 0);   \
            hipLaunchKernelGGL((bw::bwd_dkv_fin_kernel<D>), dim3((unsigned)g4), dim3(256), 0, s,                 \
                               (const bf16_t *)k, k_gain, eps, cos_tab, sin_tab, n, (int)Hkv, (int)S, dkv_acc,    \
                               (const float *)nullptr, (bf16_t *)dk, (bf16_t *)dv, dk_gain);                     \
        } else                                                                                                  \
            hipLaunchKernelGGL((bw::bwd_dkv_kernel<DT, D>), dim3((unsigned)g2), dim3(bw::DkvCfg<D>::NT), 0, s,   \
                               (const T *)k, (const T *)kc, (const T *)kr, (const T *)v, k_gain, eps, cos_tab,   \
                               sin_tab, idx, cnt, (const T *)dout, n, (int)Hq, (int)Hkv, (int)S, W,              \
                               (int)k_blocks, scale, qc_ws, qr_ws, lse_ws, dd_ws, sink_acc, (T *)dk, (T *)dv,    \
                               dk_gain);                                                                        \
    } while (0)
    HBA_DISPATCH_DT_D(dtype, d, HBA_BWD);
#undef HBA_BWD
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
