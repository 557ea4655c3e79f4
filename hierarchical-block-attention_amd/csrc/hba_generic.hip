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
