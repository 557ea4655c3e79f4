// Union attention forward: one softmax per (query i, head h) over
//   sinks   j < min(S, i+1)               NoPE  (qc . kc)
//   window  max(S, i-W+1) <= j <= i        RoPE  (qr . kr)
//   routed  the Bk keys of each valid selected block      NoPE
// (hba_attention_dense src/hba/attention.py:342-356, hba_attention_eval
//  :676-711, hba_attention_fused's LSE merge :592-603).
//
// bf16: hba_attn_bf16.hip (MFMA: one launch streams each query tile's
//   window tiles, sink blocks and routed blocks in one softmax state; the
//   split entry points below run the window and the rest as two launches
//   merged by LSE).
// f32: attn_f32_kernel, one thread per (query, head), sequential fp32 dot
//   products and a two-pass softmax; the fp32 parity path.
#include "hba_common.h"
#include "hba_abi.h"
#include "hba_generic.h"
#include "hba_attn_bf16.h"

namespace hba {

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
    // a routed block's keys below S are sinks, counted once (the union mask
    // of attention.py:351-352; with S <= 64 no routed block holds one)
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;   // block 0 is never routed (sinks, window)
        const int64_t j0 = (int64_t)ix[r] * 64;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + 64; ++j) mx = fmaxf(mx, dot_row<D>(qc, KC + j * D) * scale);
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
        if (ix[r] < 1 || ix[r] >= nb) continue;   // block 0 is never routed (sinks, window)
        const int64_t j0 = (int64_t)ix[r] * 64;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + 64; ++j) {
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

}  // namespace hba

using namespace hba;

namespace {
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

extern "C" int hba_attn_fwd_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t d,
                                            size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || d <= 0) return HBA_ERR_INVALID_ARG;
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    // bf16: the RoPE query operand of the window tiles, [B, n, Hq, d] bf16
    *bytes = (dtype == HBA_DTYPE_BF16) ? (((size_t)B * n * Hq * d * 2 + 255) & ~(size_t)255) : 0;
    return HBA_OK;
}

extern "C" int hba_attn_workspace_size(int dtype, int64_t B, int64_t n, int64_t Hq, size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0) return HBA_ERR_INVALID_ARG;
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    // bf16 split launches: the window's LSE per (batch, head, query), fp32
    *bytes = (dtype == HBA_DTYPE_BF16) ? (size_t)B * Hq * n * sizeof(float) : 0;
    return HBA_OK;
}

extern "C" int hba_attn_fwd(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
                            const float *k_gain, float eps, const void *kc, const void *kr, const void *vt,
                            const float *cos_tab, const float *sin_tab, const int32_t *idx,
                            const int32_t *cnt, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                            int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t k, float scale,
                            void *workspace, size_t ws_bytes, void *out, const int64_t out_strides[3],
                            void *stream) {
    if (dtype == HBA_DTYPE_F32 && !tuned_shape(d, Bk)) {   // fp32, other geometry: the generic kernel
        if (!q || !q_strides || !kc || !kr || !vt || !cos_tab || !sin_tab || !idx || !cnt || !out ||
            !out_strides)
            return HBA_ERR_INVALID_ARG;
        if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || W < 1 || S < 0 || k < 1)
            return HBA_ERR_INVALID_ARG;
        if (!gen_shape_ok(d, Bk)) return HBA_ERR_UNSUPPORTED;
        if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
        if (B > 65535 || Hq > 65535) return HBA_ERR_UNSUPPORTED;
        return gen_attn((const float *)q, q_strides, q_gain, eps, (const float *)kc, (const float *)kr,
                        (const float *)vt, cos_tab, sin_tab, idx, cnt, B, n, Hq, Hkv, d, S, W, Bk, k, scale,
                        (float *)out, out_strides, (hipStream_t)stream);
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !q_strides || !kc || !kr || !vt || !cos_tab || !sin_tab || !idx || !cnt || !out ||
        !out_strides)
        return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || W < 1 || S < 0 || k < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
    if (dtype == HBA_DTYPE_BF16 && S > 2 * Bk) return HBA_ERR_UNSUPPORTED;   // the MFMA path stages 2 sink blocks
    if (!abi::rows_aligned(dtype, q, q_strides) || !abi::rows_aligned(dtype, out, out_strides) ||
        !abi::aligned16(kc) || !abi::aligned16(kr) || !abi::aligned16(vt))
        return HBA_ERR_UNSUPPORTED;
    if (B > 65535 || Hq > 65535) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    if (dtype == HBA_DTYPE_BF16) {
        size_t need = 0;
        hba_attn_fwd_workspace_bytes(dtype, B, n, Hq, d, &need);
        if (!workspace || ws_bytes < need || !abi::aligned16(workspace)) return HBA_ERR_INVALID_ARG;
        st = (d == 64) ? launch_attn_bf16<64>(q, q_strides, q_gain, k_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                              idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides, workspace,
                                              s)
                       : launch_attn_bf16<128>(q, q_strides, q_gain, k_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                               idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides,
                                               workspace, s);
    } else
        st = (d == 64) ? launch_attn_f32<64>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                             idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out, out_strides, s)
                       : launch_attn_f32<128>(q, q_strides, q_gain, eps, kc, kr, vt, cos_tab, sin_tab,
                                              idx, cnt, B, n, Hq, Hkv, S, W, k, scale, out,
                                              out_strides, s);
    if (st) return st;
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

// The bf16 union attention's two launches as separate calls, so that a caller
// can run the window (which needs no selection) concurrently with the
// selection on another stream.  Same arguments and checks as hba_attn_fwd.
static int attn_split_checks(const void *q, const int64_t *q_strides, int64_t B, int64_t n, int64_t Hq,
                             int64_t Hkv, int64_t d, int64_t S, int64_t Bk, void *workspace, size_t ws_bytes,
                             void *out, const int64_t *out_strides) {
    int st = abi::check_dtype_dim(HBA_DTYPE_BF16, d);
    if (st) return st;
    if (!q || !q_strides || !out || !out_strides) return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || S < 0) return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
    if (S > 2 * Bk) return HBA_ERR_UNSUPPORTED;   // the MFMA path stages 2 sink blocks
    if (!abi::rows_aligned(HBA_DTYPE_BF16, q, q_strides) || !abi::rows_aligned(HBA_DTYPE_BF16, out, out_strides))
        return HBA_ERR_UNSUPPORTED;
    if (B > 65535 || Hq > 65535) return HBA_ERR_UNSUPPORTED;
    size_t need = 0;
    hba_attn_workspace_size(HBA_DTYPE_BF16, B, n, Hq, &need);
    if (!workspace || ws_bytes < need || !abi::aligned16(workspace)) return HBA_ERR_INVALID_ARG;
    return HBA_OK;
}

extern "C" int hba_attn_window_fwd(const void *q, const int64_t q_strides[3], const float *q_gain,
                                   const float *k_gain, float eps, const void *kr, const void *vt,
                                   const float *cos_tab, const float *sin_tab, int64_t B, int64_t n, int64_t Hq,
                                   int64_t Hkv, int64_t d, int64_t S, int64_t W, int64_t Bk, float scale,
                                   void *workspace, size_t ws_bytes, void *out, const int64_t out_strides[3],
                                   void *stream) {
    int st = attn_split_checks(q, q_strides, B, n, Hq, Hkv, d, S, Bk, workspace, ws_bytes, out, out_strides);
    if (st) return st;
    if (!kr || !vt || !cos_tab || !sin_tab || W < 1) return HBA_ERR_INVALID_ARG;
    if (!abi::aligned16(kr) || !abi::aligned16(vt)) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    float *lse = (float *)workspace;
    st = (d == 64) ? launch_attn_bf16_window<64>(q, q_strides, q_gain, k_gain, eps, kr, vt, cos_tab, sin_tab, B, n,
                                                 Hq, Hkv, S, W, scale, out, out_strides, lse, s)
                   : launch_attn_bf16_window<128>(q, q_strides, q_gain, k_gain, eps, kr, vt, cos_tab, sin_tab, B, n,
                                                  Hq, Hkv, S, W, scale, out, out_strides, lse, s);
    if (st) return st;
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_attn_routed_fwd(const void *q, const int64_t q_strides[3], const float *q_gain,
                                   const float *k_gain, float eps, const void *kc, const void *vt,
                                   const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n, int64_t Hq,
                                   int64_t Hkv, int64_t d, int64_t S, int64_t Bk, int64_t k, float scale,
                                   void *workspace, size_t ws_bytes, void *out, const int64_t out_strides[3],
                                   void *stream) {
    int st = attn_split_checks(q, q_strides, B, n, Hq, Hkv, d, S, Bk, workspace, ws_bytes, out, out_strides);
    if (st) return st;
    if (!kc || !vt || !idx || !cnt || k < 1) return HBA_ERR_INVALID_ARG;
    if (!abi::aligned16(kc) || !abi::aligned16(vt)) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    const float *lse = (const float *)workspace;
    st = (d == 64) ? launch_attn_bf16_routed<64>(q, q_strides, q_gain, k_gain, eps, kc, vt, idx, cnt, B, n, Hq,
                                                 Hkv, S, k, scale, out, out_strides, lse, s)
                   : launch_attn_bf16_routed<128>(q, q_strides, q_gain, k_gain, eps, kc, vt, idx, cnt, B, n, Hq,
                                                  Hkv, S, k, scale, out, out_strides, lse, s);
    if (st) return st;
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
