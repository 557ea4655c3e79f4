// Launchers of the bf16 union attention: one launch over the whole union
// (launch_attn_bf16; qrw: bf16 [B, n, Hq, D] scratch for the RoPE query
// operand), or the window and the sinks + routed blocks as two launches
// merged by the window's LSE (lse: fp32 [B, Hq, n] scratch).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hba {

template <int D>
int launch_attn_bf16(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                     const void *kc, const void *kr, const void *vt, const float *cosT, const float *sinT,
                     const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                     int64_t S, int64_t W, int64_t k, float scale, void *out, const int64_t *os, void *qrw,
                     hipStream_t s);

// The two launches separately (window; then sinks + routed, ordered after it).
template <int D>
int launch_attn_bf16_window(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                            const void *kr, const void *vt, const float *cosT, const float *sinT, int64_t B,
                            int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t W, float scale, void *out,
                            const int64_t *os, float *lse, hipStream_t s);
template <int D>
int launch_attn_bf16_routed(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                            const void *kc, const void *vt, const int32_t *idx, const int32_t *cnt, int64_t B,
                            int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t k, float scale, void *out,
                            const int64_t *os, const float *lse, hipStream_t s);

// The query gradient of the union attention (bf16, d = 64, G <= 16, S <= 64;
// HBA_ERR_UNSUPPORTED otherwise): dq (raw q) and the gain gradient added into
// dq_gain, and for the key gradients the QKNorm'd and rotated rows (qc_ws,
// qr_ws: bf16 [B, n, Hq, D]), the LSE and D (lse_ws, dd_ws: fp32 [B, Hq, n]).
// kct, krt: kc and kr transposed, [B, Hkv, D, n]; v, out, dout as the
// forward's inputs and output.
template <int D>
int launch_attn_bf16_dq(const void *q, const float *qgain, const float *kgain, float eps, const void *kc,
                        const void *kr, const void *kct, const void *krt, const void *v, const float *cosT,
                        const float *sinT, const int32_t *idx, const int32_t *cnt, const void *out,
                        const void *dout, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t W,
                        int64_t k, float scale, void *qc_ws, void *qr_ws, float *lse_ws, float *dd_ws, void *dq,
                        float *dq_gain, hipStream_t s);

}  // namespace hba
