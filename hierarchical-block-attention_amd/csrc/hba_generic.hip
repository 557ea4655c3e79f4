// fp32 forward kernels for geometry outside the tuned paths: any even head
// dim d <= 256, any block size Bk (1..256), any k.  They serve the entry
// points hba_prep_keys, hba_summarize, hba_score_select and hba_attn_fwd when
// those are called in fp32 with such a shape -- the reference's own test
// geometry is block 16, head_dim 8 (tests/test_qknorm.py:28-35), and its
// select-all gate sets k = n / block (gates.py:211).  Plain one-thread-per-
// row / one-workgroup-per-block-or-query kernels in the declared fp32 orders
// of the tuned fp32 kernels (QKNorm: sequential FMA sum of squares; RoPE:
// rotate-half; routing query: sequential head sum; slot scores: sequential
// FMA dots, slot max, times scale; top-k: score desc, block asc).  A
// correctness path, not a tuned one.
//   prep    src/hba/attention.py:40-44, 88-94
//   summary src/hba/summarizer.py:34-42
//   select  src/hba/attention.py:272-303 (eval :695-698), summarizer.py:45-54
//   attend  src/hba/attention.py:342-356, 676-711
#include "hba_common.h"
#include "hba_abi.h"
#include "hba_generic.h"

namespace hba {
namespace gen {

constexpr int DMAX = 256;
constexpr int NT = 256;

__device__ __forceinline__ void qknorm_n(float *x, int d, float gain, float eps) {
    float ss = 0.0f;
    for (int t = 0; t < d; ++t) ss = fmaf(x[t], x[t], ss);
    float ms = ss / (float)d;
    if (ms < eps) ms = eps;
    const float r = sqrtf(ms);
    for (int t = 0; t < d; ++t) x[t] = (x[t] / r) * gain;
}

__device__ __forceinline__ void rope_n(const float *x, float *y, int d, const float *cs, const float *sn) {
    const int H = d / 2;
    for (int t = 0; t < d; ++t) {
        const float rot = (t < H) ? -x[t + H] : x[t - H];
        const float t1 = x[t] * cs[t];
        const float t2 = rot * sn[t];
        y[t] = t1 + t2;
    }
}

__device__ __forceinline__ float dot_n(const float *a, const float *b, int d) {
    float acc = 0.0f;
    for (int t = 0; t < d; ++t) acc = fmaf(a[t], b[t], acc);
    return acc;
}

// ---------------------------------------------------------------- prep ----
__global__ __launch_bounds__(NT) void prep_kernel(const float *__restrict__ k, int64_t ksb, int64_t ksn,
                                                  int64_t ksh, const float *__restrict__ v, int64_t vsb,
                                                  int64_t vsn, int64_t vsh, const float *__restrict__ kgain,
                                                  float eps, const float *__restrict__ cosT,
                                                  const float *__restrict__ sinT, int64_t B, int64_t n,
                                                  int64_t Hkv, int d, float *__restrict__ kc,
                                                  float *__restrict__ kr, float *__restrict__ vt) {
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (gid >= B * Hkv * n) return;
    const int64_t j = gid % n, g = (gid / n) % Hkv, b = gid / (n * Hkv);
    float x[DMAX], y[DMAX];
    const float *src = k + b * ksb + j * ksn + g * ksh;
    for (int t = 0; t < d; ++t) x[t] = src[t];
    if (kgain) qknorm_n(x, d, kgain[g], eps);
    const int64_t row = ((b * Hkv + g) * n + j) * d;
    for (int t = 0; t < d; ++t) kc[row + t] = x[t];
    if (kr) {
        rope_n(x, y, d, cosT + j * d, sinT + j * d);
        for (int t = 0; t < d; ++t) kr[row + t] = y[t];
    }
    if (vt) {
        const float *vs = v + b * vsb + j * vsn + g * vsh;
        float *o = vt + (b * Hkv + g) * d * n + j;
        for (int t = 0; t < d; ++t) o[(int64_t)t * n] = vs[t];
    }
}

// ------------------------------------------------------------ summaries ----
// One workgroup per (block c, KV head g, batch b): the block's Bk keys in
// LDS, slot logits probes . key * d^-0.5, softmax over the keys, pooled rows,
// then @ proj.
__global__ __launch_bounds__(NT) void summ_kernel(const float *__restrict__ kc, int64_t n, int64_t nb,
                                                  int64_t Hkv, int Bk, int d, const float *__restrict__ probes,
                                                  const float *__restrict__ proj, int m, float att_scale,
                                                  float *__restrict__ out) {
    extern __shared__ float sm[];
    float *kb = sm;                      // [Bk][d]
    float *att = kb + Bk * d;            // [m][Bk]
    float *pooled = att + m * Bk;        // [m][d]
    const int tid = threadIdx.x;
    const int64_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const float *src = kc + ((b * Hkv + g) * n + c * Bk) * d;
    for (int e = tid; e < Bk * d; e += NT) kb[e] = src[e];
    __syncthreads();
    const float *pr = probes + g * m * d;
    for (int e = tid; e < m * Bk; e += NT) {
        const int s = e / Bk, t = e % Bk;
        att[e] = dot_n(pr + s * d, kb + t * d, d) * att_scale;
    }
    __syncthreads();
    for (int s = tid; s < m; s += NT) {   // softmax over the block's keys, one thread per slot
        float *a = att + s * Bk;
        float mx = -INFINITY;
        for (int t = 0; t < Bk; ++t) mx = fmaxf(mx, a[t]);
        float sum = 0.0f;
        for (int t = 0; t < Bk; ++t) {
            a[t] = expf(a[t] - mx);
            sum += a[t];
        }
        for (int t = 0; t < Bk; ++t) a[t] = a[t] / sum;
    }
    __syncthreads();
    for (int e = tid; e < m * d; e += NT) {
        const int s = e / d, dd = e % d;
        float acc = 0.0f;
        for (int t = 0; t < Bk; ++t) acc = fmaf(att[s * Bk + t], kb[t * d + dd], acc);
        pooled[e] = acc;
    }
    __syncthreads();
    const float *pj = proj + g * d * d;
    float *dst = out + ((b * Hkv + g) * nb + c) * m * d;
    for (int e = tid; e < m * d; e += NT) {
        const int s = e / d, ee = e % d;
        float acc = 0.0f;
        for (int dd = 0; dd < d; ++dd) acc = fmaf(pooled[s * d + dd], pj[dd * d + ee], acc);
        dst[e] = acc;
    }
}

// ------------------------------------------------------------ selection ----
// Best finite entry of sc[0..len) under (score desc, position asc) as a
// position, -1 if none; the same in every thread.  Ends with a barrier.
__device__ int block_argmax(const float *sc, int len, float *wv, int *wj) {
    float bv = -INFINITY;
    int bj = -1;
    for (int j = threadIdx.x; j < len; j += NT) {
        const float v = sc[j];
        if (v != -INFINITY && v == v && (bj < 0 || v > bv)) {   // ascending j: ties keep the first
            bv = v;
            bj = j;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oj = __shfl_xor(bj, o, 64);
        if (oj >= 0 && (bj < 0 || ov > bv || (ov == bv && oj < bj))) {
            bv = ov;
            bj = oj;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        wv[threadIdx.x >> 6] = bv;
        wj[threadIdx.x >> 6] = bj;
    }
    __syncthreads();
    float rv = wv[0];
    int rj = wj[0];
    for (int x = 1; x < NT / 64; ++x)
        if (wj[x] >= 0 && (rj < 0 || wv[x] > rv || (wv[x] == rv && wj[x] < rj))) {
            rv = wv[x];
            rj = wj[x];
        }
    __syncthreads();
    return rj;
}

// One workgroup per (query i, KV head g, batch b): the routing query (QKNorm
// of the G heads, sequential head sum), every candidate block's score into
// LDS, then k argmax rounds.
__global__ __launch_bounds__(NT) void select_kernel(const float *__restrict__ q, int64_t qsb, int64_t qsn,
                                                    int64_t qsh, const float *__restrict__ qgain, float eps,
                                                    const float *__restrict__ S0, int64_t n, int Hq, int Hkv,
                                                    int64_t nb, int m, int d, int Bk, int64_t W, int kk,
                                                    float scale, int32_t *__restrict__ idx,
                                                    float *__restrict__ val, int32_t *__restrict__ cnt,
                                                    float *__restrict__ scores) {
    extern __shared__ float sm[];
    float *qg = sm;          // [d]
    float *sc = qg + DMAX;   // [nb]
    __shared__ float wv[NT / 64];
    __shared__ int wj[NT / 64];
    const int tid = threadIdx.x;
    const int64_t i = blockIdx.x;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int G = Hq / Hkv;
    if (tid == 0) {   // the routing query: one thread, the declared order
        float x[DMAX], a[DMAX];
        for (int h = 0; h < G; ++h) {
            const float *row = q + b * qsb + i * qsn + (int64_t)(g * G + h) * qsh;
            for (int t = 0; t < d; ++t) x[t] = row[t];
            if (qgain) qknorm_n(x, d, qgain[g * G + h], eps);
            for (int t = 0; t < d; ++t) a[t] = (h == 0) ? x[t] : a[t] + x[t];
        }
        for (int t = 0; t < d; ++t) qg[t] = a[t];
    }
    __syncthreads();
    const int64_t bmax = cand_bmax(i, Bk, W);
    const float *Sg = S0 + (b * Hkv + g) * nb * m * d;
    const int64_t o = (b * Hkv + g) * n + i;
    for (int64_t blk = tid; blk < nb; blk += NT) {
        float v = -INFINITY;
        if (blk >= 1 && blk <= bmax) {
            const float *S = Sg + blk * m * d;
            float best = dot_n(qg, S, d);
            for (int s = 1; s < m; ++s) {
                const float t = dot_n(qg, S + (int64_t)s * d, d);
                best = (t > best) ? t : best;
            }
            v = best * scale;
            if (scores) scores[o * nb + blk] = v;
        }
        sc[blk] = v;
    }
    __syncthreads();
    int c = 0;
    for (int r = 0; r < kk; ++r) {
        const int j = block_argmax(sc, (int)nb, wv, wj);
        if (j < 0) break;   // uniform
        if (tid == 0) {
            idx[o * kk + r] = j;
            val[o * kk + r] = sc[j];
            sc[j] = -INFINITY;
        }
        c = r + 1;
        __syncthreads();
    }
    for (int r = c + tid; r < kk; r += NT) {
        idx[o * kk + r] = -1;
        val[o * kk + r] = -INFINITY;
    }
    if (tid == 0) cnt[o] = c;
}

// ------------------------------------------------------------ attention ----
// One thread per (query i, head h): the tuned fp32 kernel's two-pass
// softmax with a runtime head dim and block size.
__global__ __launch_bounds__(64) void attn_kernel(const float *__restrict__ q, int64_t qsb, int64_t qsn,
                                                  int64_t qsh, const float *__restrict__ qgain, float eps,
                                                  const float *__restrict__ kc, const float *__restrict__ kr,
                                                  const float *__restrict__ vt, const float *__restrict__ cosT,
                                                  const float *__restrict__ sinT, const int32_t *__restrict__ idx,
                                                  const int32_t *__restrict__ cnt, int64_t n, int Hq, int Hkv,
                                                  int S, int64_t W, int Bk, int kk, int d, float scale,
                                                  float *__restrict__ out, int64_t osb, int64_t osn, int64_t osh) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (i >= n) return;
    const int G = Hq / Hkv, g = h / G;
    float qc[DMAX], qr[DMAX], acc[DMAX];
    const float *qrow = q + b * qsb + i * qsn + (int64_t)h * qsh;
    for (int t = 0; t < d; ++t) qc[t] = qrow[t];
    if (qgain) qknorm_n(qc, d, qgain[h], eps);
    rope_n(qc, qr, d, cosT + i * d, sinT + i * d);
    const int64_t bh = b * Hkv + g;
    const float *KC = kc + bh * n * d;
    const float *KR = kr + bh * n * d;
    const float *VT = vt + bh * d * n;
    const int64_t s_end = ((int64_t)S < i + 1) ? (int64_t)S : i + 1;
    const int64_t w_beg = ((int64_t)S > i - W + 1) ? (int64_t)S : i - W + 1;
    const int c = min(max(cnt[bh * n + i], 0), kk);
    const int32_t *ix = idx + (bh * n + i) * kk;
    const int64_t nb = n / Bk;
    float mx = -INFINITY;
    for (int64_t j = 0; j < s_end; ++j) mx = fmaxf(mx, dot_n(qc, KC + j * d, d) * scale);
    for (int64_t j = w_beg; j <= i; ++j) mx = fmaxf(mx, dot_n(qr, KR + j * d, d) * scale);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;   // block 0 is never routed (sinks, window)
        const int64_t j0 = (int64_t)ix[r] * Bk;   // keys below S are sinks, counted once
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + Bk; ++j) mx = fmaxf(mx, dot_n(qc, KC + j * d, d) * scale);
    }
    for (int t = 0; t < d; ++t) acc[t] = 0.0f;
    float l = 0.0f;
    auto add = [&](const float *qv, const float *K, int64_t j) {
        const float p = expf(dot_n(qv, K + j * d, d) * scale - mx);
        l += p;
        for (int t = 0; t < d; ++t) acc[t] = fmaf(p, VT[(int64_t)t * n + j], acc[t]);
    };
    for (int64_t j = 0; j < s_end; ++j) add(qc, KC, j);
    for (int64_t j = w_beg; j <= i; ++j) add(qr, KR, j);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;
        const int64_t j0 = (int64_t)ix[r] * Bk;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + Bk; ++j) add(qc, KC, j);
    }
    float *orow = out + b * osb + i * osn + (int64_t)h * osh;
    const float inv = 1.0f / l;
    for (int t = 0; t < d; ++t) orow[t] = acc[t] * inv;
}

// ------------------------------------------------------- routing query ----
// One thread per (query, KV head): the QKNorm'd rows of the group's G heads
// summed in head order (grouped_query, summarizer.py:50-54), any G.
__global__ __launch_bounds__(NT) void route_queries_kernel(const float *__restrict__ q, int64_t qsb, int64_t qsn,
                                                           int64_t qsh, const float *__restrict__ qgain, float eps,
                                                           int64_t B, int64_t n, int Hq, int Hkv, int d,
                                                           float *__restrict__ qg) {
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (gid >= B * n * Hkv) return;
    const int g = (int)(gid % Hkv);
    const int64_t i = (gid / Hkv) % n, b = gid / (Hkv * n);
    const int G = Hq / Hkv;
    float acc[DMAX], x[DMAX];
    for (int h = 0; h < G; ++h) {
        const float *row = q + b * qsb + i * qsn + (int64_t)(g * G + h) * qsh;
        for (int t = 0; t < d; ++t) x[t] = row[t];
        if (qgain) qknorm_n(x, d, qgain[g * G + h], eps);
        for (int t = 0; t < d; ++t) acc[t] = (h == 0) ? x[t] : acc[t] + x[t];
    }
    float *dst = qg + ((b * n + i) * Hkv + g) * d;
    for (int t = 0; t < d; ++t) dst[t] = acc[t];
}

// ------------------------------------------------------------ backward ----
// Gradients of attn_kernel's output (the autograd of attention.py:306-356
// with the selection held fixed, routing on detached q/k :288-303), any
// geometry gen_shape_ok takes.  With p the union softmax of row (i, h) and
// D = <dO, O>: ds_j = p_j (<dO, v_j> - D) * scale; the query side gains
// ds_j y_j, key j's side ds_j x and dv_j p_j dO (x, y: the NoPE rows for the
// sinks and routed keys, the rotated rows for the window).  Then rope^T
// (x_u = y_u cos_u + (u < H ? y_{u+H} sin_{u+H} : -y_{u-H} sin_{u-H})) and the
// QKNorm backward dx = g/r y - [ms >= eps] x g <y, x> / (d r^3), dg = <y, x> / r.
//   bwd_q: one thread per (query, head): dq and dq_gain, and the key sides
//          into fp32 accumulators by atomics (dkc, dkr: NoPE and rotated
//          frames; dv), zeroed first by bwd_zero.
//   bwd_k: one thread per (key row, KV head): dk, dv and dk_gain.
__global__ __launch_bounds__(NT) void bwd_zero_kernel(float *__restrict__ p, int64_t nel) {
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (gid < nel) p[gid] = 0.0f;
}

__device__ __forceinline__ void rope_t_n(const float *y, float *x, int d, const float *cs, const float *sn) {
    const int H = d / 2;
    for (int u = 0; u < d; ++u) x[u] = y[u] * cs[u] + ((u < H) ? y[u + H] * sn[u + H] : -y[u - H] * sn[u - H]);
}

// y (the gradient with respect to the normalised row) -> the raw row's, in
// place; returns <y, x> / r (the gain's gradient).  x is the raw row.
__device__ __forceinline__ float qknorm_bwd_n(const float *x, float *y, int d, float gain, float eps) {
    float ss = 0.0f, yx = 0.0f;
    for (int t = 0; t < d; ++t) {
        ss = fmaf(x[t], x[t], ss);
        yx = fmaf(y[t], x[t], yx);
    }
    const float ms = ss / (float)d;
    const float r = sqrtf(ms < eps ? eps : ms);
    const float corr = (ms >= eps) ? gain * yx / ((float)d * r * r * r) : 0.0f;
    for (int t = 0; t < d; ++t) y[t] = (gain / r) * y[t] - x[t] * corr;
    return yx / r;
}

__global__ __launch_bounds__(64) void bwd_q_kernel(const float *__restrict__ q, const float *__restrict__ qgain,
                                                   float eps, const float *__restrict__ kc,
                                                   const float *__restrict__ kr, const float *__restrict__ v,
                                                   const float *__restrict__ cosT, const float *__restrict__ sinT,
                                                   const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt,
                                                   const float *__restrict__ out, const float *__restrict__ dout,
                                                   int64_t n, int Hq, int Hkv, int S, int64_t W, int Bk, int kk,
                                                   int d, float scale, float *__restrict__ dq,
                                                   float *__restrict__ dq_gain, float *__restrict__ dkc,
                                                   float *__restrict__ dkr, float *__restrict__ dv) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (i >= n) return;
    const int G = Hq / Hkv, g = h / G;
    float x[DMAX], qc[DMAX], qr[DMAX], go[DMAX], gc[DMAX], gr[DMAX];
    const int64_t qrow = ((b * n + i) * Hq + h) * d;   // q, out, dout, dq: [B, n, Hq, d]
    for (int t = 0; t < d; ++t) {
        x[t] = q[qrow + t];
        qc[t] = x[t];
        go[t] = dout[qrow + t];
        gc[t] = gr[t] = 0.0f;
    }
    if (qgain) qknorm_n(qc, d, qgain[h], eps);
    rope_n(qc, qr, d, cosT + i * d, sinT + i * d);
    float D = 0.0f;
    for (int t = 0; t < d; ++t) D = fmaf(go[t], out[qrow + t], D);
    const int64_t bh = b * Hkv + g;
    const float *KC = kc + bh * n * d;   // kc, kr: [B, Hkv, n, d]
    const float *KR = kr + bh * n * d;
    const int64_t s_end = ((int64_t)S < i + 1) ? (int64_t)S : i + 1;
    const int64_t w_beg = ((int64_t)S > i - W + 1) ? (int64_t)S : i - W + 1;
    const int c = min(max(cnt[bh * n + i], 0), kk);
    const int32_t *ix = idx + (bh * n + i) * kk;
    const int64_t nb = n / Bk;
    // the forward's softmax statistics, in its order
    float mx = -INFINITY;
    for (int64_t j = 0; j < s_end; ++j) mx = fmaxf(mx, dot_n(qc, KC + j * d, d) * scale);
    for (int64_t j = w_beg; j <= i; ++j) mx = fmaxf(mx, dot_n(qr, KR + j * d, d) * scale);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;
        const int64_t j0 = (int64_t)ix[r] * Bk;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + Bk; ++j) mx = fmaxf(mx, dot_n(qc, KC + j * d, d) * scale);
    }
    float l = 0.0f;
    for (int64_t j = 0; j < s_end; ++j) l += expf(dot_n(qc, KC + j * d, d) * scale - mx);
    for (int64_t j = w_beg; j <= i; ++j) l += expf(dot_n(qr, KR + j * d, d) * scale - mx);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;
        const int64_t j0 = (int64_t)ix[r] * Bk;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + Bk; ++j) l += expf(dot_n(qc, KC + j * d, d) * scale - mx);
    }
    const float inv = 1.0f / l;
    // key j against the row xv (qc or qr): the query side into acc, the key
    // side (frame buffer kacc) and dv by atomics
    auto key = [&](const float *xv, const float *K, float *acc, float *kacc, int64_t j) {
        const float *kj = K + j * d;
        const float p = expf(dot_n(xv, kj, d) * scale - mx) * inv;
        const int64_t vrow = ((b * n + j) * Hkv + g) * d;   // v: [B, n, Hkv, d]
        float dp = 0.0f;
        for (int t = 0; t < d; ++t) dp = fmaf(go[t], v[vrow + t], dp);
        const float ds = p * (dp - D) * scale;
        const int64_t krow = (bh * n + j) * d;
        for (int t = 0; t < d; ++t) {
            acc[t] = fmaf(ds, kj[t], acc[t]);
            atomicAdd(kacc + krow + t, ds * xv[t]);
            atomicAdd(dv + krow + t, p * go[t]);
        }
    };
    for (int64_t j = 0; j < s_end; ++j) key(qc, KC, gc, dkc, j);
    for (int64_t j = w_beg; j <= i; ++j) key(qr, KR, gr, dkr, j);
    for (int r = 0; r < c; ++r) {
        if (ix[r] < 1 || ix[r] >= nb) continue;
        const int64_t j0 = (int64_t)ix[r] * Bk;
        for (int64_t j = (j0 > S ? j0 : S); j < j0 + Bk; ++j) key(qc, KC, gc, dkc, j);
    }
    // d(qc) = gc + rope^T(gr) at position i, then the QKNorm backward
    float y[DMAX];
    rope_t_n(gr, y, d, cosT + i * d, sinT + i * d);
    for (int t = 0; t < d; ++t) y[t] += gc[t];
    if (qgain) {
        const float dg = qknorm_bwd_n(x, y, d, qgain[h], eps);
        atomicAdd(dq_gain + h, dg);
    }
    for (int t = 0; t < d; ++t) dq[qrow + t] = y[t];
}

__global__ __launch_bounds__(NT) void bwd_k_kernel(const float *__restrict__ k, const float *__restrict__ kgain,
                                                   float eps, const float *__restrict__ cosT,
                                                   const float *__restrict__ sinT, const float *__restrict__ dkc,
                                                   const float *__restrict__ dkr, const float *__restrict__ dva,
                                                   int64_t B, int64_t n, int Hkv, int d, float *__restrict__ dk,
                                                   float *__restrict__ dv, float *__restrict__ dk_gain) {
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (gid >= B * Hkv * n) return;
    const int64_t j = gid % n, g = (gid / n) % Hkv, b = gid / (n * Hkv);
    const int64_t arow = ((b * Hkv + g) * n + j) * d;   // accumulators: [B, Hkv, n, d]
    const int64_t row = ((b * n + j) * Hkv + g) * d;    // k, dk, dv: [B, n, Hkv, d]
    float x[DMAX], y[DMAX], zr[DMAX];
    for (int t = 0; t < d; ++t) {
        x[t] = k[row + t];
        zr[t] = dkr[arow + t];
    }
    rope_t_n(zr, y, d, cosT + j * d, sinT + j * d);
    for (int t = 0; t < d; ++t) y[t] += dkc[arow + t];
    if (kgain) {
        const float dg = qknorm_bwd_n(x, y, d, kgain[g], eps);
        atomicAdd(dk_gain + g, dg);
    }
    for (int t = 0; t < d; ++t) {
        dk[row + t] = y[t];
        dv[row + t] = dva[arow + t];
    }
}

// --------------------------------------------------------------- aux-KL ----
// The summarizer's auxiliary loss (attention.py:366-389) and its gradient
// into probes and proj at any geometry gen_shape_ok takes, in the oracle's
// arithmetic: the teacher's block LSEs per (query, head), then per (query, KV
// head) p* (each head's softmax over the candidate blocks' LSEs, averaged
// over the G heads and renormalised), the block scores bsc = slot max x
// scale_r with their tie masks, the row's KL term and d aux / d bsc = (softmax
// (bsc) sum p* - p*) / N; dS0 from the tie-shared d bsc, the summariser's
// backward per block, and sums in fixed orders.
constexpr int AUX_GMAX = 64;   // query heads per KV head
constexpr int AUX_MMAX = 32;   // slots (the tie mask is a 32-bit word)

__global__ __launch_bounds__(64) void aux_teacher_kernel(const float *__restrict__ q, int64_t qsb, int64_t qsn,
                                                         int64_t qsh, const float *__restrict__ qgain,
                                                         float eps, const float *__restrict__ kc, int64_t n, int Hq,
                                                         int Hkv, int Bk, int d, int64_t W, float scale_u,
                                                         float *__restrict__ L) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int h = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (i >= n) return;
    const int G = Hq / Hkv, g = h / G, hh = h % G;
    const int64_t bm = cand_bmax(i, Bk, W), nb = n / Bk;
    if (bm < 1) return;
    float qc[DMAX];
    const float *row = q + b * qsb + i * qsn + (int64_t)h * qsh;
    for (int t = 0; t < d; ++t) qc[t] = row[t];
    if (qgain) qknorm_n(qc, d, qgain[h], eps);
    const float *K = kc + (b * Hkv + g) * n * d;
    float *dst = L + (((b * Hkv + g) * n + i) * G + hh) * nb;
    for (int64_t c = 1; c <= bm; ++c) {
        float mx = -INFINITY;
        for (int64_t j = c * Bk; j < (c + 1) * Bk; ++j) mx = fmaxf(mx, dot_n(qc, K + j * d, d) * scale_u);
        float z = 0.0f;
        for (int64_t j = c * Bk; j < (c + 1) * Bk; ++j) z += expf(dot_n(qc, K + j * d, d) * scale_u - mx);
        dst[c] = mx + logf(z);
    }
}

// One thread per (b, g, i): p*, bsc and its tie mask, the KL term (rowt) and
// d aux / d bsc (written over bsc).
__global__ __launch_bounds__(NT) void aux_rows_kernel(const float *__restrict__ L, const float *__restrict__ qg,
                                                      const float *__restrict__ S0, int64_t B, int64_t n, int Hkv,
                                                      int G, int Bk, int m, int d, int64_t W, float scale_r,
                                                      float invN, float *__restrict__ bsc,
                                                      uint32_t *__restrict__ ties, float *__restrict__ rowt) {
    const int64_t r = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (r >= B * Hkv * n) return;
    const int64_t i = r % n, g = (r / n) % Hkv, b = r / (n * Hkv);
    const int64_t bm = cand_bmax(i, Bk, W), nb = n / Bk;
    if (bm < 1) {
        rowt[r] = 0.0f;
        return;
    }
    const float *Lr = L + r * G * nb;   // r = (b Hkv + g) n + i
    float M[AUX_GMAX], Z[AUX_GMAX];
    for (int h = 0; h < G; ++h) {
        float mx = -INFINITY;
        for (int64_t c = 1; c <= bm; ++c) mx = fmaxf(mx, Lr[h * nb + c]);
        float z = 0.0f;
        for (int64_t c = 1; c <= bm; ++c) z += expf(Lr[h * nb + c] - mx);
        M[h] = mx;
        Z[h] = z;
    }
    auto pstar_raw = [&](int64_t c) {
        float a = 0.0f;
        for (int h = 0; h < G; ++h) a += expf(Lr[h * nb + c] - M[h]) / Z[h];
        return a / (float)G;
    };
    float ptot = 0.0f;
    for (int64_t c = 1; c <= bm; ++c) ptot += pstar_raw(c);
    const float pnorm = 1.0f / fmaxf(ptot, 1e-9f);
    // block scores: slot max of qg . S0 times scale_r, and the slots at the max
    const float *qv = qg + ((b * n + i) * Hkv + g) * d;   // qg: [B, n, Hkv, d]
    float *br = bsc + r * nb;
    uint32_t *tr = ties + r * nb;
    float bmx = -INFINITY;
    for (int64_t c = 1; c <= bm; ++c) {
        const float *Sc = S0 + ((b * Hkv + g) * nb + c) * m * d;
        float best = -INFINITY;
        uint32_t mask = 0u;
        for (int sl = 0; sl < m; ++sl) {
            const float v = dot_n(qv, Sc + sl * d, d);
            if (v > best) {
                best = v;
                mask = 1u << sl;
            } else if (v == best) {
                mask |= 1u << sl;
            }
        }
        br[c] = best * scale_r;
        tr[c] = mask;
        bmx = fmaxf(bmx, br[c]);
    }
    float zb = 0.0f;
    for (int64_t c = 1; c <= bm; ++c) zb += expf(br[c] - bmx);
    const float lse = bmx + logf(zb);
    float term = 0.0f, P = 0.0f;
    for (int64_t c = 1; c <= bm; ++c) {
        const float ps = pstar_raw(c) * pnorm;
        if (ps > 0.0f) {
            term += ps * (br[c] - lse);
            P += ps;
        }
    }
    for (int64_t c = 1; c <= bm; ++c) {
        const float ps = pstar_raw(c) * pnorm;
        const float soft = expf(br[c] - lse);
        br[c] = (soft * P - (ps > 0.0f ? ps : 0.0f)) * invN;
    }
    rowt[r] = term;
}

// aux = -(sum of the row terms) / N, one workgroup, a fixed order.
__global__ __launch_bounds__(NT) void aux_sum_kernel(const float *__restrict__ rowt, int64_t rows, float invN,
                                                     float *__restrict__ aux) {
    __shared__ double part[NT];
    double a = 0.0;
    for (int64_t e = threadIdx.x; e < rows; e += NT) a += (double)rowt[e];
    part[threadIdx.x] = a;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int e = 0; e < NT; ++e) t += part[e];
        aux[0] = (float)(-t * (double)invN);
    }
}

// dS0 [b, g, c, slot, t] = sum over the queries with block c as a candidate,
// ascending, of d bsc x scale_r / (tie count) x qg[t] where the slot is at
// the max.
__global__ __launch_bounds__(NT) void aux_dS0_kernel(const float *__restrict__ dbsc, const uint32_t *__restrict__ ties,
                                                     const float *__restrict__ qg, int64_t B, int64_t n, int Hkv,
                                                     int Bk, int m, int d, int64_t W, float scale_r,
                                                     float *__restrict__ dS0) {
    const int64_t nb = n / Bk;
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (gid >= B * Hkv * nb * m * d) return;
    const int t = (int)(gid % d), sl = (int)((gid / d) % m);
    const int64_t c = (gid / ((int64_t)d * m)) % nb, bg = gid / ((int64_t)d * m * nb);
    const int64_t b = bg / Hkv, g = bg % Hkv;
    float acc = 0.0f;
    if (c >= 1) {
        for (int64_t i = 0; i < n; ++i) {
            if (cand_bmax(i, Bk, W) < c) continue;
            const int64_t o = (bg * n + i) * nb + c;
            const uint32_t mk = ties[o];
            if ((mk >> sl) & 1u)
                acc = fmaf(dbsc[o] * scale_r / (float)__popc(mk), qg[((b * n + i) * Hkv + g) * d + t], acc);
        }
    }
    dS0[gid] = acc;
}

// One thread per (b, g, block c, slot): the summariser's forward for the
// slot (att over the block's keys, pooled row Sp) and its backward given
// dS0: Sp (for d proj) and the slot's d probes partial.
__global__ __launch_bounds__(64) void aux_sbwd_kernel(const float *__restrict__ kc, const float *__restrict__ probes,
                                                      const float *__restrict__ proj, const float *__restrict__ dS0,
                                                      int64_t B, int64_t n, int Hkv, int Bk, int m, int d,
                                                      float *__restrict__ Sp_out, float *__restrict__ pprb) {
    const int64_t nb = n / Bk;
    const int64_t gid = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (gid >= B * Hkv * nb * m) return;
    const int sl = (int)(gid % m);
    const int64_t c = (gid / m) % nb, bg = gid / (m * nb);
    const int64_t g = bg % Hkv;
    const float *K = kc + (bg * n + c * Bk) * d;   // the block's keys
    const float *pr = probes + (g * m + sl) * d;
    const float *pj = proj + g * d * d;
    const float isd = 1.0f / sqrtf((float)d);
    float att[256], sp[DMAX], dsp[DMAX];
    float mx = -INFINITY;
    for (int k = 0; k < Bk; ++k) {
        att[k] = dot_n(pr, K + k * d, d) * isd;
        mx = fmaxf(mx, att[k]);
    }
    float z = 0.0f;
    for (int k = 0; k < Bk; ++k) {
        att[k] = expf(att[k] - mx);
        z += att[k];
    }
    for (int k = 0; k < Bk; ++k) att[k] /= z;
    for (int t = 0; t < d; ++t) {
        float a = 0.0f;
        for (int k = 0; k < Bk; ++k) a = fmaf(att[k], K[k * d + t], a);
        sp[t] = a;
    }
    const float *dS = dS0 + gid * d;   // gid = ((bg nb + c) m + sl)
    for (int t = 0; t < d; ++t) {
        float a = 0.0f;
        for (int e = 0; e < d; ++e) a = fmaf(dS[e], pj[t * d + e], a);
        dsp[t] = a;
    }
    float dat[256];
    float sad = 0.0f;   // sum over the keys of att * datt
    for (int k = 0; k < Bk; ++k) {
        dat[k] = dot_n(dsp, K + k * d, d);
        sad = fmaf(att[k], dat[k], sad);
    }
    float *dp = pprb + gid * d;
    for (int t = 0; t < d; ++t) dp[t] = 0.0f;
    for (int k = 0; k < Bk; ++k) {
        const float dl = att[k] * (dat[k] - sad) * isd;   // d logit, times the logit's scale
        for (int t = 0; t < d; ++t) dp[t] = fmaf(dl, K[k * d + t], dp[t]);
    }
    float *so = Sp_out + gid * d;
    for (int t = 0; t < d; ++t) so[t] = sp[t];
}

// d probes [g, slot, t] = sum over (b, c) of the partials; d proj [g, t, e] =
// sum over (b, c, slot) of Sp[t] dS0[e]; fixed orders.
__global__ __launch_bounds__(NT) void aux_grad_kernel(const float *__restrict__ pprb, const float *__restrict__ Sp,
                                                      const float *__restrict__ dS0, int64_t B, int64_t nb, int Hkv,
                                                      int m, int d, float *__restrict__ dprobes,
                                                      float *__restrict__ dproj) {
    const int64_t gid = (int64_t)blockIdx.x * NT + threadIdx.x;
    const int64_t np = (int64_t)Hkv * m * d, nj = (int64_t)Hkv * d * d;
    if (gid < np) {
        const int t = (int)(gid % d), sl = (int)((gid / d) % m);
        const int64_t g = gid / ((int64_t)d * m);
        float a = 0.0f;
        for (int64_t b = 0; b < B; ++b)
            for (int64_t c = 0; c < nb; ++c) a += pprb[(((b * Hkv + g) * nb + c) * m + sl) * d + t];
        dprobes[gid] = a;
    } else if (gid < np + nj) {
        const int64_t e2 = gid - np;
        const int e = (int)(e2 % d), t = (int)((e2 / d) % d);
        const int64_t g = e2 / ((int64_t)d * d);
        float a = 0.0f;
        for (int64_t b = 0; b < B; ++b)
            for (int64_t c = 0; c < nb; ++c)
                for (int sl = 0; sl < m; ++sl) {
                    const int64_t o = (((b * Hkv + g) * nb + c) * m + sl) * d;
                    a = fmaf(Sp[o + t], dS0[o + e], a);
                }
        dproj[e2] = a;
    }
}

}  // namespace gen

// ------------------------------------------------------------ launchers ----
bool gen_shape_ok(int64_t d, int64_t Bk) { return d >= 2 && d <= gen::DMAX && d % 2 == 0 && Bk >= 1 && Bk <= 256; }

int gen_prep_keys(const float *k, const int64_t *ks, const float *v, const int64_t *vs, const float *kgain,
                  float eps, const float *cosT, const float *sinT, int64_t B, int64_t n, int64_t Hkv, int64_t d,
                  float *kc, float *kr, float *vt, hipStream_t s) {
    const int64_t total = B * Hkv * n;
    if ((total + gen::NT - 1) / gen::NT > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(gen::prep_kernel, dim3((unsigned)((total + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s, k,
                       ks[0], ks[1], ks[2], v, vs[0], vs[1], vs[2], kgain, eps, cosT, sinT, B, n, Hkv, (int)d, kc, kr,
                       vt);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

int gen_summarize(const float *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d, int64_t Bk, int64_t nblocks,
                  const float *probes, const float *proj, int64_t m, float *out, hipStream_t s) {
    const size_t lds = (size_t)(Bk * d + m * Bk + m * d) * 4;
    if (lds > 64 * 1024) return HBA_ERR_UNSUPPORTED;
    const float att_scale = (float)(1.0 / __builtin_sqrt((double)d));
    hipLaunchKernelGGL(gen::summ_kernel, dim3((unsigned)nblocks, (unsigned)Hkv, (unsigned)B), dim3(gen::NT), lds, s,
                       kc, n, nblocks, Hkv, (int)Bk, (int)d, probes, proj, (int)m, att_scale, out);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

int gen_score_select(const float *q, const int64_t *qs, const float *qgain, float eps, const float *S0, int64_t B,
                     int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W, int64_t k,
                     float scale, int32_t *idx, float *val, int32_t *cnt, float *scores, hipStream_t s) {
    const int64_t nb = n / Bk;
    const size_t lds = (size_t)(gen::DMAX + nb) * 4;
    if (lds > 64 * 1024 || n > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(gen::select_kernel, dim3((unsigned)n, (unsigned)Hkv, (unsigned)B), dim3(gen::NT), lds, s, q,
                       qs[0], qs[1], qs[2], qgain, eps, S0, n, (int)Hq, (int)Hkv, nb, (int)m, (int)d, (int)Bk, W,
                       (int)k, scale, idx, val, cnt, scores);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

int gen_attn(const float *q, const int64_t *qs, const float *qgain, float eps, const float *kc, const float *kr,
             const float *vt, const float *cosT, const float *sinT, const int32_t *idx, const int32_t *cnt, int64_t B,
             int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t k, float scale,
             float *out, const int64_t *os, hipStream_t s) {
    hipLaunchKernelGGL(gen::attn_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)Hq, (unsigned)B), dim3(64), 0, s, q,
                       qs[0], qs[1], qs[2], qgain, eps, kc, kr, vt, cosT, sinT, idx, cnt, n, (int)Hq, (int)Hkv,
                       (int)S, W, (int)Bk, (int)k, (int)d, scale, out, os[0], os[1], os[2]);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

// the generic aux-KL's workspace: qg [B, n, Hkv, d], L [B, Hkv, n, G, nb],
// bsc and ties [B, Hkv, n, nb], row terms [B, Hkv, n], dS0, Sp and the d
// probes partials [B, Hkv, nb, m, d]
struct GenAuxWs {
    size_t qg, L, bsc, ties, rowt, dS0, Sp, pprb, total;
};
static GenAuxWs gen_aux_layout(int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const int64_t nb = n / Bk, G = Hq / Hkv;
    GenAuxWs w;
    size_t o = 0;
    w.qg = o;   o += up((size_t)B * n * Hkv * d * 4);
    w.L = o;    o += up((size_t)B * Hkv * n * G * nb * 4);
    w.bsc = o;  o += up((size_t)B * Hkv * n * nb * 4);
    w.ties = o; o += up((size_t)B * Hkv * n * nb * 4);
    w.rowt = o; o += up((size_t)B * Hkv * n * 4);
    w.dS0 = o;  o += up((size_t)B * Hkv * nb * m * d * 4);
    w.Sp = o;   o += up((size_t)B * Hkv * nb * m * d * 4);
    w.pprb = o; o += up((size_t)B * Hkv * nb * m * d * 4);
    w.total = o;
    return w;
}

bool gen_aux_ok(int64_t d, int64_t Bk, int64_t m, int64_t G) {
    return gen_shape_ok(d, Bk) && m >= 1 && m <= gen::AUX_MMAX && G >= 1 && G <= gen::AUX_GMAX;
}

size_t gen_aux_ws_bytes(int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk) {
    return gen_aux_layout(B, n, Hq, Hkv, d, m, Bk).total;
}

int gen_aux_kl(const float *q, const int64_t *qs, const float *qgain, float eps, const float *kc, const float *S0,
               const float *probes, const float *proj, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
               int64_t m, int64_t Bk, int64_t W, float scale_u, float scale_r, void *ws, float *aux, float *dprobes,
               float *dproj, hipStream_t s) {
    const GenAuxWs L = gen_aux_layout(B, n, Hq, Hkv, d, m, Bk);
    char *w = (char *)ws;
    float *qg = (float *)(w + L.qg), *Lb = (float *)(w + L.L), *bsc = (float *)(w + L.bsc);
    uint32_t *ties = (uint32_t *)(w + L.ties);
    float *rowt = (float *)(w + L.rowt), *dS0 = (float *)(w + L.dS0), *Sp = (float *)(w + L.Sp);
    float *pprb = (float *)(w + L.pprb);
    const int64_t nb = n / Bk, G = Hq / Hkv, rows = B * Hkv * n;
    // queries with a candidate block: cand_bmax(i) >= 1 <=> i >= 2 Bk + W - 1
    const int64_t f0 = 2 * Bk + W - 1;
    const int64_t N = B * Hkv * (n > f0 ? n - f0 : 0);
    const float invN = N ? (float)(1.0 / (double)N) : 0.0f;
    const int64_t ng = Hkv * m * d + Hkv * d * d;
    if ((rows + gen::NT - 1) / gen::NT > 0x7fffffff || (B * Hkv * nb * m * d + gen::NT - 1) / gen::NT > 0x7fffffff ||
        Hq > 65535 || B > 65535)
        return HBA_ERR_UNSUPPORTED;
    if (N == 0) {   // no query has a candidate block: aux and its gradients are zero
        hipLaunchKernelGGL(gen::bwd_zero_kernel, dim3(1), dim3(gen::NT), 0, s, aux, (int64_t)1);
        if (dprobes) {
            hipLaunchKernelGGL(gen::bwd_zero_kernel, dim3((unsigned)((Hkv * m * d + gen::NT - 1) / gen::NT)),
                               dim3(gen::NT), 0, s, dprobes, Hkv * m * d);
            hipLaunchKernelGGL(gen::bwd_zero_kernel, dim3((unsigned)((Hkv * d * d + gen::NT - 1) / gen::NT)),
                               dim3(gen::NT), 0, s, dproj, Hkv * d * d);
        }
        HBA_LAUNCH_CHECK();
        return HBA_OK;
    }
    int st = gen_route_queries(q, qs, qgain, eps, B, n, Hq, Hkv, d, qg, s);
    if (st) return st;
    hipLaunchKernelGGL(gen::aux_teacher_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)Hq, (unsigned)B), dim3(64), 0,
                       s, q, qs[0], qs[1], qs[2], qgain, eps, kc, n, (int)Hq, (int)Hkv, (int)Bk, (int)d, W, scale_u,
                       Lb);
    hipLaunchKernelGGL(gen::aux_rows_kernel, dim3((unsigned)((rows + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s,
                       Lb, qg, S0, B, n, (int)Hkv, (int)G, (int)Bk, (int)m, (int)d, W, scale_r, invN, bsc, ties, rowt);
    hipLaunchKernelGGL(gen::aux_sum_kernel, dim3(1), dim3(gen::NT), 0, s, rowt, rows, invN, aux);
    if (dprobes) {
        const int64_t nd = B * Hkv * nb * m * d, ns = B * Hkv * nb * m;
        hipLaunchKernelGGL(gen::aux_dS0_kernel, dim3((unsigned)((nd + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s,
                           bsc, ties, qg, B, n, (int)Hkv, (int)Bk, (int)m, (int)d, W, scale_r, dS0);
        hipLaunchKernelGGL(gen::aux_sbwd_kernel, dim3((unsigned)((ns + 63) / 64)), dim3(64), 0, s, kc, probes, proj,
                           dS0, B, n, (int)Hkv, (int)Bk, (int)m, (int)d, Sp, pprb);
        hipLaunchKernelGGL(gen::aux_grad_kernel, dim3((unsigned)((ng + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s,
                           pprb, Sp, dS0, B, nb, (int)Hkv, (int)m, (int)d, dprobes, dproj);
    }
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

size_t gen_bwd_ws_bytes(int64_t B, int64_t n, int64_t Hkv, int64_t d) {
    return (size_t)3 * B * Hkv * n * d * sizeof(float);
}

int gen_attn_bwd(const float *q, const float *k, const float *v, const float *kc, const float *kr,
                 const float *qgain, const float *kgain, float eps, const float *cosT, const float *sinT,
                 const int32_t *idx, const int32_t *cnt, const float *out, const float *dout, int64_t B, int64_t n,
                 int64_t Hq, int64_t Hkv, int64_t d, int64_t S, int64_t W, int64_t Bk, int64_t kk, float scale,
                 float *ws, float *dq, float *dk, float *dv, float *dq_gain, float *dk_gain, hipStream_t s) {
    const int64_t per = B * Hkv * n * d;   // one accumulator
    float *dkc = ws, *dkr = ws + per, *dva = ws + 2 * per;
    const int64_t nel = 3 * per, rows = B * Hkv * n;
    if ((nel + gen::NT - 1) / gen::NT > 0x7fffffff || (rows + gen::NT - 1) / gen::NT > 0x7fffffff ||
        (n + 63) / 64 > 0x7fffffff || Hq > 65535 || B > 65535)
        return HBA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(gen::bwd_zero_kernel, dim3((unsigned)((nel + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s, ws,
                       nel);
    hipLaunchKernelGGL(gen::bwd_q_kernel, dim3((unsigned)((n + 63) / 64), (unsigned)Hq, (unsigned)B), dim3(64), 0, s,
                       q, qgain, eps, kc, kr, v, cosT, sinT, idx, cnt, out, dout, n, (int)Hq, (int)Hkv, (int)S, W,
                       (int)Bk, (int)kk, (int)d, scale, dq, dq_gain, dkc, dkr, dva);
    hipLaunchKernelGGL(gen::bwd_k_kernel, dim3((unsigned)((rows + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0, s, k,
                       kgain, eps, cosT, sinT, dkc, dkr, dva, B, n, (int)Hkv, (int)d, dk, dv, dk_gain);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

int gen_route_queries(const float *q, const int64_t *qs, const float *qgain, float eps, int64_t B, int64_t n,
                      int64_t Hq, int64_t Hkv, int64_t d, float *qg, hipStream_t s) {
    const int64_t total = B * n * Hkv;
    hipLaunchKernelGGL(gen::route_queries_kernel, dim3((unsigned)((total + gen::NT - 1) / gen::NT)), dim3(gen::NT), 0,
                       s, q, qs[0], qs[1], qs[2], qgain, eps, B, n, (int)Hq, (int)Hkv, (int)d, qg);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

}  // namespace hba
