// Key preparation, slot summaries, super-summaries and the paged-cache append.
//
//   prep_keys        QKNorm(k) -> kc, RoPE(kc) -> kr, V^T -> vt
//                    (_HeadRMSNorm.forward src/hba/attention.py:88-94,
//                     apply_rope src/hba/attention.py:40-44)
//   summarize        SlotSummarizer.summarize src/hba/summarizer.py:34-42
//   build_super      build_super src/hba/attention.py:202-214
//   kv_append        decode-cache append (no reference counterpart)
//
// All of these are HBM-bound elementwise / tiny-GEMM work: one thread per key
// row (prep, append), one workgroup per 64-key block (summaries).
#include "hba_common.h"
#include "hba_abi.h"

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

// --------------------------------------------------------------- kernels ----
template <int DT, int D>
__global__ __launch_bounds__(256) void prep_keys_kernel(
    const typename St<DT>::T *__restrict__ k, int64_t ksb, int64_t ksn, int64_t ksh,
    const typename St<DT>::T *__restrict__ v, int64_t vsb, int64_t vsn, int64_t vsh,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, int64_t B, int64_t n, int64_t Hkv,
    typename St<DT>::T *__restrict__ kc, typename St<DT>::T *__restrict__ kr,
    typename St<DT>::T *__restrict__ vt) {
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= B * Hkv * n) return;
    int64_t j = gid % n;
    int64_t g = (gid / n) % Hkv;
    int64_t b = gid / (n * Hkv);
    float x[D];
    load_row<DT, D>(k + b * ksb + j * ksn + g * ksh, x);
    if (kgain) qknorm_row<DT, D>(x, kgain[g], eps);
    int64_t row = ((b * Hkv + g) * n + j) * D;
    store_row<DT, D>(kc + row, x);
    if (kr) {
        float y[D];
        rope_row<DT, D>(x, y, cosT + j * D, sinT + j * D);
        store_row<DT, D>(kr + row, y);
    }
    if (vt) {
        load_row<DT, D>(v + b * vsb + j * vsn + g * vsh, x);
        typename St<DT>::T *o = vt + (b * Hkv + g) * D * n + j;
#pragma unroll
        for (int t = 0; t < D; ++t) St<DT>::st(o, (int64_t)t * n, x[t]);
    }
}

// One workgroup (256 threads) per 64-key block.  Block base pointers come
// either from the contiguous head-major layout or from a list of pages.
template <int DT, int D>
__global__ __launch_bounds__(256) void summarize_kernel(
    const typename St<DT>::T *__restrict__ kc, int64_t n, int64_t nb, int64_t Hkv,
    const int32_t *__restrict__ pages, const float *__restrict__ probes,
    const float *__restrict__ proj, int m, float att_scale, typename St<DT>::T *__restrict__ out) {
    constexpr int BK = 64;
    __shared__ float kb[BK][D + 1];
    __shared__ float att[8][BK];
    __shared__ float pooled[8][D];
    const int tid = threadIdx.x;
    const int64_t c = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const typename St<DT>::T *src;
    typename St<DT>::T *dst;
    if (pages) {
        int64_t p = pages[c];
        src = kc + (p * Hkv + g) * BK * D;
        dst = out + (p * Hkv + g) * m * D;
    } else {
        src = kc + ((b * Hkv + g) * n + c * BK) * D;
        dst = out + ((b * Hkv + g) * nb + c) * m * D;
    }
    if (pages) {   // a cache page: chunks of 8 elements in the page layout (page_key_chunk)
        for (int c = tid; c < 8 * D; c += 256) {
            int j, t0;
            page_key_chunk(c, D, j, t0);
#pragma unroll
            for (int u = 0; u < 8; ++u) kb[j][t0 + u] = St<DT>::ld(src, 8 * c + u);
        }
    } else {
        for (int e = tid; e < BK * D; e += 256) kb[e / D][e % D] = St<DT>::ld(src, e);
    }
    __syncthreads();
    const float *pr = probes + g * m * D;
    for (int e = tid; e < m * BK; e += 256) {
        int s = e / BK, t = e % BK;
        float acc = 0.0f;
        for (int dd = 0; dd < D; ++dd) acc = fmaf(pr[s * D + dd], kb[t][dd], acc);
        att[s][t] = acc * att_scale;
    }
    __syncthreads();
    {   // softmax over the 64 keys of each slot: one wave per slot
        int w = tid / 64, l = tid % 64;
        for (int s = w; s < m; s += 4) {
            float x = att[s][l];
            float mx = wave_max(x);
            float e = expf(x - mx);
            float sm = wave_sum(e);
            att[s][l] = e / sm;
        }
    }
    __syncthreads();
    for (int e = tid; e < m * D; e += 256) {
        int s = e / D, dd = e % D;
        float acc = 0.0f;
        for (int t = 0; t < BK; ++t) acc = fmaf(att[s][t], kb[t][dd], acc);
        pooled[s][dd] = acc;
    }
    __syncthreads();
    const float *pj = proj + g * D * D;
    for (int e = tid; e < m * D; e += 256) {
        int s = e / D, ee = e % D;
        float acc = 0.0f;
        for (int dd = 0; dd < D; ++dd) acc = fmaf(pooled[s][dd], pj[dd * D + ee], acc);
        St<DT>::st(dst, (int64_t)s * D + ee, acc);
    }
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

template <int DT, int D>
__global__ __launch_bounds__(256) void kv_append_kernel(
    const typename St<DT>::T *__restrict__ knew, const typename St<DT>::T *__restrict__ vnew,
    const float *__restrict__ kgain, float eps, const float *__restrict__ cosT,
    const float *__restrict__ sinT, const int32_t *__restrict__ ptab, int64_t maxp,
    const int32_t *__restrict__ lens, int64_t lmax, int64_t Bd, int64_t Hkv,
    typename St<DT>::T *__restrict__ kcp, typename St<DT>::T *__restrict__ krp,
    typename St<DT>::T *__restrict__ vp) {
    constexpr int BK = 64;
    int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= Bd * Hkv) return;
    int64_t s = gid / Hkv, g = gid % Hkv;
    int64_t pos = (int64_t)lens[s] - 1;
    // nothing to append, outside the page table or past the RoPE tables
    if (pos < 0 || pos / BK >= maxp || pos >= lmax) return;
    int64_t page = ptab[s * maxp + pos / BK];
    const int64_t base = (page * Hkv + g) * BK * D;
    const int j = (int)(pos % BK);
    float x[D], y[D];
    load_row<DT, D>(knew + gid * D, x);
    if (kgain) qknorm_row<DT, D>(x, kgain[g], eps);
    rope_row<DT, D>(x, y, cosT + pos * D, sinT + pos * D);
    // keys: 8 consecutive elements per chunk of the page layout (page_key_off)
#pragma unroll
    for (int t0 = 0; t0 < D; t0 += 8) {
        const int64_t o = base + page_key_off(j, t0, D);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            St<DT>::st(kcp, o + u, x[t0 + u]);
            St<DT>::st(krp, o + u, y[t0 + u]);
        }
    }
    load_row<DT, D>(vnew + gid * D, x);
#pragma unroll
    for (int t = 0; t < D; ++t) St<DT>::st(vp, base + page_val_off(j, t), x[t]);
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
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!k || !k_strides || !kc || B <= 0 || n <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
    if (kr && (!cos_tab || !sin_tab)) return HBA_ERR_INVALID_ARG;
    if (vt && (!v || !v_strides)) return HBA_ERR_INVALID_ARG;
    if (!abi::rows_aligned(dtype, k, k_strides) || (vt && !abi::rows_aligned(dtype, v, v_strides)) ||
        !abi::aligned16(kc) || (kr && !abi::aligned16(kr)))
        return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    int64_t total = B * Hkv * n;
    dim3 grid((unsigned)((total + 255) / 256));
    const int64_t *vs = v_strides ? v_strides : k_strides;
#define HBA_PREP(DT, D)                                                                            \
    hipLaunchKernelGGL((prep_keys_kernel<DT, D>), grid, dim3(256), 0, s,                           \
                       (const St<DT>::T *)k, k_strides[0], k_strides[1], k_strides[2],             \
                       (const St<DT>::T *)v, vs[0], vs[1], vs[2], k_gain, eps, cos_tab, sin_tab, B, n, \
                       Hkv, (St<DT>::T *)kc, (St<DT>::T *)kr, (St<DT>::T *)vt)
    HBA_DISPATCH_DT_D(dtype, d, HBA_PREP);
#undef HBA_PREP
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

static int summarize_common(int dtype, const void *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                            int64_t Bk, const int32_t *pages, int64_t nblocks, const float *probes,
                            const float *proj, int64_t m, void *out, void *stream) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!kc || !probes || !proj || !out || B <= 0 || Hkv <= 0) return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (m < 1 || m > 8) return HBA_ERR_UNSUPPORTED;
    if (nblocks <= 0) return HBA_OK;
    if (nblocks > 0x7fffffff || Hkv > 65535 || B > 65535) return HBA_ERR_UNSUPPORTED;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid((unsigned)nblocks, (unsigned)Hkv, (unsigned)B);
    float att_scale = (float)(1.0 / __builtin_sqrt((double)d));
#define HBA_SUMM(DT, D)                                                                            \
    hipLaunchKernelGGL((summarize_kernel<DT, D>), grid, dim3(256), 0, s, (const St<DT>::T *)kc, n,   \
                       nblocks, Hkv, pages, probes, proj, (int)m, att_scale, (St<DT>::T *)out)
    HBA_DISPATCH_DT_D(dtype, d, HBA_SUMM);
#undef HBA_SUMM
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_summarize(int dtype, const void *kc, int64_t B, int64_t Hkv, int64_t n, int64_t d,
                             int64_t Bk, const float *probes, const float *proj, int64_t m, void *S0,
                             void *stream) {
    if (Bk <= 0 || n <= 0) return HBA_ERR_INVALID_ARG;
    return summarize_common(dtype, kc, B, Hkv, n, d, Bk, nullptr, n / Bk, probes, proj, m, S0, stream);
}

extern "C" int hba_summarize_pages(int dtype, const void *kc_pages, const int32_t *pages,
                                   int64_t npages, int64_t Hkv, int64_t d, int64_t Bk,
                                   const float *probes, const float *proj, int64_t m,
                                   void *summ_pages, void *stream) {
    if (!pages || npages < 0) return HBA_ERR_INVALID_ARG;
    return summarize_common(dtype, kc_pages, 1, Hkv, Bk, d, Bk, pages, npages, probes, proj, m,
                            summ_pages, stream);
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
    dim3 grid((unsigned)((Bd * Hkv + 255) / 256));
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
