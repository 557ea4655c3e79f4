// fp32 forward for geometry outside the tuned kernels (hba_generic.hip): the
// entry points call these when an fp32 call's head dim is not 64 / 128, its
// block size is not 64, (selection) k > 64 or the slot count is not 1, 2, 4
// or 8, or (routing queries) more than 16 query heads share a KV head.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace hba {

// an even head dim <= 256 and a block size 1..256
bool gen_shape_ok(int64_t d, int64_t Bk);
// the tuned kernels' geometry (they refuse anything else)
inline bool tuned_shape(int64_t d, int64_t Bk) { return (d == 64 || d == 128) && Bk == 64; }

int gen_prep_keys(const float *k, const int64_t *ks, const float *v, const int64_t *vs, const float *kgain,
                  float eps, const float *cosT, const float *sinT, int64_t B, int64_t n, int64_t Hkv, int64_t d,
                  float *kc, float *kr, float *vt, hipStream_t s);
int gen_summarize(const float *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d, int64_t Bk, int64_t nblocks,
                  const float *probes, const float *proj, int64_t m, float *out, hipStream_t s);
int gen_score_select(const float *q, const int64_t *qs, const float *qgain, float eps, const float *S0, int64_t B,
                     int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W, int64_t k,
                     float scale, int32_t *idx, float *val, int32_t *cnt, float *scores, hipStream_t s);
int gen_route_queries(const float *q, const int64_t *qs, const float *qgain, float eps, int64_t B, int64_t n,
                      int64_t Hq, int64_t Hkv, int64_t d, float *qg, hipStream_t s);
int gen_attn(const float *q, const int64_t *qs, const float *qgain, float eps, const float *kc, const float *kr,
             const float *vt, const float *cosT, const float *sinT, const int32_t *idx, const int32_t *cnt, int64_t B,
             int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t k, float scale,
             float *out, const int64_t *os, hipStream_t s);

// the generic backward's workspace: dk (NoPE and rotated frames) and dv
// accumulators, fp32 [B, Hkv, n, d] each
size_t gen_bwd_ws_bytes(int64_t B, int64_t n, int64_t Hkv, int64_t d);
// fp32 gradients of gen_attn's output: q, k, v, dq, dk, dv contiguous
// [B, n, H, d]; kc, kr [B, Hkv, n, d]; dq_gain / dk_gain accumulated into
// (the caller zeroes them)
int gen_attn_bwd(const float *q, const float *k, const float *v, const float *kc, const float *kr,
                 const float *qgain, const float *kgain, float eps, const float *cosT, const float *sinT,
                 const int32_t *idx, const int32_t *cnt, const float *out, const float *dout, int64_t B, int64_t n,
                 int64_t Hq, int64_t Hkv, int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t kk, float scale,
                 float *ws, float *dq, float *dk, float *dv, float *dq_gain, float *dk_gain, hipStream_t s);

// the generic aux-KL (fp32): even d <= 256, Bk 1..256, m <= 32 slots,
// G <= 64 query heads per KV head
bool gen_aux_ok(int64_t d, int64_t Bk, int64_t m, int64_t G);
size_t gen_aux_ws_bytes(int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk);
// aux (1 float) and, if dprobes is set, dprobes [Hkv, m, d] and dproj
// [Hkv, d, d]; q raw with strides qs, kc [B, Hkv, n, d] content keys, S0
// [B, Hkv, n/Bk, m, d] summaries
int gen_aux_kl(const float *q, const int64_t *qs, const float *qgain, float eps, const float *kc, const float *S0,
               const float *probes, const float *proj, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
               int64_t m, int64_t Bk, int64_t W, float scale_u, float scale_r, void *ws, float *aux, float *dprobes,
               float *dproj, hipStream_t s);

}  // namespace hba
