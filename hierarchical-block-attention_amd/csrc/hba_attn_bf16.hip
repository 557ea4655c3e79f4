// Union attention forward for bf16 inputs on MFMA (gfx950).  Two launches
// together compute one softmax per (query i, head h) over
//   sinks   j < min(S, i+1)                 NoPE  (qc . kc)
//   window  max(S, i-W+1) <= j <= i          RoPE  (qr . kr)
//   routed  the 64 keys of each selected block    NoPE
// (hba_attention_dense src/hba/attention.py:342-356, hba_attention_eval
//  :676-711); the two partial softmaxes merge by LSE, as hba_attention_fused
// merges its two regions (:592-603).
//
// attn_win_kernel -- the RoPE window.  Workgroup = (batch, KV head, QT
//   consecutive queries); one wave per (head, 16*RT consecutive queries).  The
//   MFMA rows of a 16-row tile are 16 consecutive queries of one head, so no
//   row of a tile is idle.  64-key tiles of kr and vt go through a two-slot
//   LDS ring by direct-to-LDS DMA (the next tile lands during this one),
//   shared by every wave, and each K / V^T fragment read from LDS feeds the
//   wave's RT row tiles.  Only tiles on a window's edges are masked.  Output:
//   the window's normalised rows (bf16, into out) and their LSE (fp32
//   workspace).
// attn_routed_kernel -- sinks and routed blocks.  Workgroup = (batch, KV head,
//   QT queries); the rows of a 16-row tile are the G heads of 16/G queries
//   (the rows that share a routed block).  The sorted union of the tile's
//   selections, preceded by block 0 for the sinks, streams through an LDS
//   ring by direct-to-LDS DMA one phase of PH blocks ahead, one barrier per
//   phase; a wave updates a tile only if one of its queries picked the
//   block.  The partial then merges with the window's (out, LSE) and the row
//   is stored.
//
// Scores are S^T = K . Q^T with v_mfma_f32_16x16x32_bf16: key rows of the A
// operand are permuted (permk) so that the probabilities leave the
// accumulators in the B-operand layout of O^T = V^T . P^T.  Softmax: when
// QKNorm bounds every logit of a KV-head group by d*max|gq|*|gk|*scale
// (attention.py:74-81) and bound*log2(e) <= 60 (so exp2 of the lowest
// possible logit, 2*bound below the shift, is >= 2^-120, a normal fp32),
// the bound is the shift: no running max, no rescaling (the same softmax).
// Otherwise a running max per row is kept.  Each kernel decides per group.
#include "hba_common.h"
#include "hba_abi.h"
#include "hba_attn_bf16.h"
#include "hba_dma.h"

namespace hba {
namespace ab {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
constexpr float LOG2E = 1.4426950408889634f;
constexpr int16_t SENT = 0x7fff;     // list terminator (block ids are < 0x7fff)

__device__ __forceinline__ bf16x8 ldb8(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ f32x4 mma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Logit bound of KV-head group g in log2 units, and whether it can serve as
// the softmax shift.
__device__ __forceinline__ bool group_bound(const float *qgain, const float *kgain, int g, int G, float scale_l2,
                                            int D, float &bl2) {
    bl2 = 0.0f;
    if (!qgain || !kgain) return false;
    float gq = 0.0f;
    for (int hh = 0; hh < G; ++hh) gq = fmaxf(gq, fabsf(qgain[g * G + hh]));
    bl2 = (float)D * gq * fabsf(kgain[g]) * scale_l2;
    return bl2 <= 60.0f;
}

// Key held by row r of M-tile mt of S^T: lane (l16, lg) then receives keys
// 32*(mt>>1) + 8*lg + 4*(mt&1) + e -- keys 8*lg..8*lg+7 of each 32-key half
// over the two M-tiles of a half, which is the B layout of the P.V MFMA.
__device__ __forceinline__ int permk(int mt, int r) {
    return 32 * (mt >> 1) + 8 * (r >> 2) + 4 * (mt & 1) + (r & 3);
}

__device__ __forceinline__ bf16x8 pack8(const float (&x)[8]) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)x[e];   // v_cvt_pk_bf16_f32, round to nearest even
    return r;
}

// Sum over a 64-key block of one column's probabilities (P^T halves p0 =
// keys 0..31, p1 = keys 32..63 in the B layout), on the MFMA: a ones A
// operand makes every row of the product the column sum.  Each lane receives
// its column's full sum.
__device__ __forceinline__ float colsum(bf16x8 p0, bf16x8 p1) {
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (__bf16)1.0f;
    f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, p0, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, p1, t, 0, 0, 0);
    return t[0];
}

// Query operand of one lane's column (query i, head h) for S^T = K . Q^T:
// d = 32*ks + 8*lg + 0..7.  qrow: the row's elements this lane holds,
// QKNorm'd in fp32 and rounded to bf16 (attention.py:88-94; the sum of
// squares is reduced across the column's four lanes).  qpack: the NoPE
// operand; qpack_rope: apply_rope's rotation and bf16 roundings (:40-44) at
// position i (the rotation partner d +- D/2 sits in the same lane at ks +-
// NKS/2).  Invalid columns read row 0 and are zeroed (no divergence around
// the shuffles).  qscale multiplies the operand before its bf16 rounding:
// the fixed-shift softmax passes scale*log2(e), so that S^T comes out in
// log2 units.
template <int D>
__device__ __forceinline__ void qrow(const bf16_t *q, int64_t qsb, int64_t qsn, int64_t qsh, const float *qgain,
                                     float eps, int64_t b, int64_t i, int h, bool valid, int lg,
                                     float (&x)[D / 32][8]) {
    constexpr int NKS = D / 32;
    const int64_t ii = valid ? i : 0;
    const bf16_t *row = q + b * qsb + ii * qsn + (int64_t)h * qsh;
    float ss = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        const u32x4 u = *reinterpret_cast<const u32x4 *>(row + 32 * ks + 8 * lg);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[ks][2 * e] = __uint_as_float(u[e] << 16);
            x[ks][2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[ks][e], x[ks][e], ss);
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    if (qgain) {
        float ms = ss / (float)D;
        if (ms < eps) ms = eps;
        const float r = sqrtf(ms);
        const float gn = qgain[h];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                x[ks][e] = (x[ks][e] / r) * gn;
                x[ks][e + 1] = (x[ks][e + 1] / r) * gn;
                rnd_bf16_pair(x[ks][e], x[ks][e + 1]);   // v_cvt_pk_bf16_f32: two roundings per instruction
            }
    }
}

template <int D>
__device__ __forceinline__ void qpack(const float (&x)[D / 32][8], bool valid, float qscale,
                                      bf16x8 (&qop)[D / 32]) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = valid ? x[ks][e] * qscale : 0.0f;
        qop[ks] = pack8(y);
    }
}

template <int D>
__device__ __forceinline__ void qpack_rope(const float (&x)[D / 32][8], const float *cosT, const float *sinT,
                                           int64_t i, bool valid, int lg, float qscale, bf16x8 (&qop)[D / 32]) {
    constexpr int NKS = D / 32;
    const int64_t ii = valid ? i : 0;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
        // the lane's 8 consecutive table entries, two 16-byte loads per table
        float ct[8], st[8];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const float4 c = *reinterpret_cast<const float4 *>(cosT + ii * D + 32 * ks + 8 * lg + 4 * hf);
            const float4 sn = *reinterpret_cast<const float4 *>(sinT + ii * D + 32 * ks + 8 * lg + 4 * hf);
            ct[4 * hf] = c.x, ct[4 * hf + 1] = c.y, ct[4 * hf + 2] = c.z, ct[4 * hf + 3] = c.w;
            st[4 * hf] = sn.x, st[4 * hf + 1] = sn.y, st[4 * hf + 2] = sn.z, st[4 * hf + 3] = sn.w;
        }
        // the roundings in pairs (v_cvt_pk_bf16_f32)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            rnd_bf16_pair(ct[e], ct[e + 1]);
            rnd_bf16_pair(st[e], st[e + 1]);
        }
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float t1a = x[ks][e] * ct[e], t1b = x[ks][e + 1] * ct[e + 1];
            float t2a = ((ks < NKS / 2) ? -x[ks + NKS / 2][e] : x[ks - NKS / 2][e]) * st[e];
            float t2b = ((ks < NKS / 2) ? -x[ks + NKS / 2][e + 1] : x[ks - NKS / 2][e + 1]) * st[e + 1];
            rnd_bf16_pair(t1a, t1b);
            rnd_bf16_pair(t2a, t2b);
            float va = t1a + t2a, vb = t1b + t2b;
            rnd_bf16_pair(va, vb);
            y[e] = valid ? va * qscale : 0.0f;
            y[e + 1] = valid ? vb * qscale : 0.0f;
        }
        qop[ks] = pack8(y);
    }
}

template <int D>
__device__ __forceinline__ void qoperand(const bf16_t *q, int64_t qsb, int64_t qsn, int64_t qsh,
                                         const float *qgain, float eps, const float *cosT,
                                         const float *sinT, int64_t b, int64_t i, int h, bool valid,
                                         bool rope, int lg, float qscale, bf16x8 (&qop)[D / 32]) {
    float x[D / 32][8];
    qrow<D>(q, qsb, qsn, qsh, qgain, eps, b, i, h, valid, lg, x);
    if (rope)
        qpack_rope<D>(x, cosT, sinT, i, valid, lg, qscale, qop);
    else
        qpack<D>(x, valid, qscale, qop);
}

// Workgroup -> (batch*KV head combo, query tile).  Workgroup i runs on XCD
// i % 8; xmap 1 (8 % Cn == 0) and 2 (Cn % 8 == 0) give each XCD one combo's
// keys at a time, so the blocks it gathers share that XCD's L2.  Tiles go
// deepest first: a tile's union of routed blocks grows with its candidate
// count, and starting the longest workgroups first leaves the short ones to
// fill the end.
__device__ __forceinline__ void xcd_map(int i, int Cn, int ntiles, int xmap, int &combo, int &tile) {
    if (xmap == 1) {
        combo = (i & 7) % Cn;
        tile = (i >> 3) * (8 / Cn) + (i & 7) / Cn;
    } else if (xmap == 2) {
        combo = (i / (8 * ntiles)) * 8 + (i & 7);
        tile = (i >> 3) % ntiles;
    } else {
        combo = i / ntiles;
        tile = i % ntiles;
    }
    if (tile < ntiles) tile = ntiles - 1 - tile;   // padding workgroups (xmap 1) keep tile >= ntiles
}

// ======================================================== tile staging ====
// LDS ring slot: K tile [64 keys][D] then V^T tile [D][64 keys], rows
// unpadded; 16-byte chunk c of row r is stored at chunk c ^ f(r) (f < 8) so
// that the MFMA fragment reads hit distinct banks: the K rows one read
// instruction touches are permk(mt, 0..15), the V^T rows 16*dt + 0..15.
__device__ __forceinline__ int swzK(int r) { return (r & 3) | ((r >> 1) & 4); }
__device__ __forceinline__ int swzV(int r) { return r & 7; }

template <int D>
struct RtCfg {
    static constexpr int NKS = D / 32;
    static constexpr int NDT = D / 16;
    // 16 waves (4 per SIMD) within 128 VGPRs: 2 row tiles each at d = 64, 1
    // at d = 128 (32 queries per workgroup).  At d = 128, 8 waves (2 per SIMD)
    // of 3 row tiles within 256 VGPRs cover 48 queries, so that each staged
    // block serves more of them, but leave the update's LDS and MFMA
    // latencies exposed: the 64K donor-shaped attention took 13.62 ms that
    // way against 13.35 ms.
    static constexpr int WAVES = 16;
    static constexpr int NTHR = WAVES * 64;
    static constexpr int PTW = (D == 64) ? 2 : 1;      // max 16-row tiles per wave
    static constexpr int SLOT = 2 * 64 * D;            // bf16 per ring slot (K + V^T)
    static constexpr int NS = (D == 64) ? 8 : 4;       // ring depth (blocks, 128 KB)
    static constexpr int PH = NS / 2;                  // blocks per barrier phase
    static_assert(NS % PH == 0, "the ring holds whole phases");
    static constexpr int KPARTS = 64 * D * 2 / 1024;   // 1 KB parts of a K (and of a V^T) tile
    static constexpr int DPW = 2 * KPARTS / WAVES;     // DMA instructions per wave per block
    static_assert(DPW * WAVES == 2 * KPARTS, "parts split evenly over the waves");
};

// ======================================================= window kernel ====
template <int D, int RT>
struct WinCfg {
    static constexpr int NKS = D / 32;                 // 32-wide d steps of S^T
    static constexpr int NDT = D / 16;                 // 16-row d tiles of O^T
    static constexpr int SLOT = 2 * 64 * D;            // bf16 per staged tile (K + V^T)
    static constexpr int NS = 2;                       // ring slots: 2 or 3 workgroups share a CU
    static constexpr int PH = NS / 2;                  // tiles per barrier phase
};

// DMA of one 64-key tile (kr rows, vt columns) into a ring slot by the
// workgroup's waves: 2*D/64 KB split over nw waves (parts w, w + nw, ...).
template <int D>
__device__ __forceinline__ void win_fill(const bf16_t *KR, const bf16_t *VT, int n, int kb, uint32_t slot_lds,
                                         int w, int nw, int lane) {
    constexpr int CPR = D / 8;
    constexpr int KPARTS = 64 * D * 2 / 1024;
    for (int part = w; part < 2 * KPARTS; part += nw) {
        const int p = (part % KPARTS) * 64 + lane;
        if (part < KPARTS) {
            const int r = p / CPR, c = (p % CPR) ^ swzK(p / CPR);
            dma16(KR + (int64_t)(kb + r) * D + 8 * c, slot_lds + (uint32_t)part * 1024u);
        } else {
            const int r = p >> 3, c = (p & 7) ^ swzV(p >> 3);
            dma16(VT + (int64_t)r * n + kb + 8 * c, slot_lds + (uint32_t)part * 1024u);
        }
    }
}

template <int D, int RT, bool FIXED>
__device__ __forceinline__ void win_body(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const bf16_t *__restrict__ kr, const bf16_t *__restrict__ vt,
    const float *__restrict__ cosT, const float *__restrict__ sinT, int n, int Hq, int Hkv, int S,
    int W, float sl2, float bl2, int gw, int wsplit, int combo, int hs, int tile, bf16_t *__restrict__ out,
    int64_t osb, int64_t osn, int64_t osh, float *__restrict__ lse, bf16_t *ring) {
    using C = WinCfg<D, RT>;
    const int G = Hq / Hkv;
    const int nw = blockDim.x >> 6;
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index: uniform, kept in SGPRs
    const int hh = hs * gw + w % gw, rg = w / gw;     // head within the group, query range
    const bool hv = hh < G;                            // waves past the group's last head only stage
    constexpr int QW = 16 * RT;                        // queries per wave
    const int QT = QW * wsplit;                        // queries per workgroup
    const int b = combo / Hkv, g = combo % Hkv;
    const int64_t bh = (int64_t)b * Hkv + g;
    const int h = g * G + (hv ? hh : 0);
    const int i0 = tile * QT;
    const int q0 = i0 + QW * rg;
    const bf16_t *KR = kr + bh * n * D;
    const bf16_t *VT = vt + bh * D * n;
    const uint32_t ring_lds = lds_offset(ring);

    bf16x8 qop[RT][C::NKS];
    f32x4 O[RT][C::NDT];
    float ls[RT], mr[RT];
    const float es = FIXED ? 1.0f : sl2;   // log2 units per S^T unit (FIXED: folded into the query operand)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const int i = q0 + 16 * rt + l16;
        qoperand<D>(q, qsb, qsn, qsh, qgain, eps, cosT, sinT, b, i, h, i < n, true, lg, FIXED ? sl2 : 1.0f,
                    qop[rt]);
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) O[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        ls[rt] = 0.0f;
        mr[rt] = -INFINITY;
    }
    // this lane's key offset within a tile for accumulator element (mt, e)
    const int kl = 8 * lg;

    // the 64-key tiles covering every window of the workgroup's queries
    const int ilast = ((i0 + QT < n) ? i0 + QT : n) - 1;
    const int kfirst = (S > i0 - W + 1) ? S : i0 - W + 1;
    if (kfirst <= ilast) {
        const int t0 = kfirst / 64, t1 = ilast / 64, nt = t1 - t0 + 1;
        // one barrier per phase of PH tiles; the ring holds NPH phases
        constexpr int P = C::PH, NPH = C::NS / C::PH;
        constexpr int PARTS = 2 * (64 * D * 2 / 1024);   // 1 KB parts of a tile
        const int mine = (PARTS - w + nw - 1) / nw;       // this wave's parts per tile
        for (int e = 0; e < (NPH - 1) * P && e < nt; ++e)
            win_fill<D>(KR, VT, n, 64 * (t0 + e), ring_lds + (uint32_t)(e * C::SLOT * 2), w, nw, lane);
        for (int e0 = 0; e0 < nt; e0 += P) {
            // this wave's parts of the phase's tiles have landed once at most
            // those of the tiles issued after them are in flight
            const int issued = min(nt, e0 + (NPH - 1) * P);
            wait_vm_n(max(0, issued - (e0 + P)) * mine);
            __syncthreads();   // all parts of this phase landed; the previous phase is consumed
            const int nf = min(nt, e0 + NPH * P);
            for (int e = issued; e < nf; ++e)
                win_fill<D>(KR, VT, n, 64 * (t0 + e), ring_lds + (uint32_t)((e % C::NS) * C::SLOT * 2), w, nw,
                            lane);
            const int e1 = min(nt, e0 + P);
            for (int e = e0; e < e1; ++e) {
                const bf16_t *Ks = ring + (e % C::NS) * C::SLOT;
                const bf16_t *Vs = Ks + 64 * D;
                const int kb = 64 * (t0 + e);
                bool act[RT], full[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int qa = q0 + 16 * rt;
                    const int qb = (qa + 15 < n) ? qa + 15 : n - 1;
                    const int lo = (S > qa - W + 1) ? S : qa - W + 1;
                    const int lob = (S > qb - W + 1) ? S : qb - W + 1;
                    act[rt] = hv && qa < n && kb <= qb && kb + 63 >= lo;
                    full[rt] = kb >= lob && kb + 63 <= qa;
                }
                // the tile's K fragments, read from LDS once for all row tiles
                bf16x8 kf[4][C::NKS];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    const int r = permk(mt, l16);
                    const bf16_t *kp = Ks + r * D;
                    const int sw = swzK(r);
#pragma unroll
                    for (int ks = 0; ks < C::NKS; ++ks) kf[mt][ks] = ldb8(kp + 8 * ((4 * ks + lg) ^ sw));
                }
                bool allfull = true;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) allfull = allfull && act[rt] && full[rt];
                if (FIXED && RT > 1 && allfull) {
                    // interior tile (every key valid for every row tile), fixed
                    // shift: straight-line code over the row tiles, so that one
                    // row tile's exponentials overlap another's MFMAs
                    f32x4 Sa[RT][4];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) {
                            Sa[rt][mt] = f32x4{-bl2, -bl2, -bl2, -bl2};   // operand carries scale*log2(e)
#pragma unroll
                            for (int ks = 0; ks < C::NKS; ++ks) Sa[rt][mt] = mma(kf[mt][ks], qop[rt][ks], Sa[rt][mt]);
                        }
                    bf16x8 pf[RT][2];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        float p[2][8];
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                            for (int e = 0; e < 4; ++e) p[mt >> 1][(mt & 1) * 4 + e] = ex2(Sa[rt][mt][e]);
                        pf[rt][0] = pack8(p[0]);
                        pf[rt][1] = pack8(p[1]);
                        ls[rt] += colsum(pf[rt][0], pf[rt][1]);
                    }
#pragma unroll
                    for (int dt = 0; dt < C::NDT; ++dt) {
                        const int r = 16 * dt + l16;
                        const bf16_t *vp = Vs + r * 64;
                        const int sw = swzV(r);
                        const bf16x8 v0 = ldb8(vp + 8 * (lg ^ sw)), v1 = ldb8(vp + 8 * ((lg + 4) ^ sw));
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) {
                            O[rt][dt] = mma(v0, pf[rt][0], O[rt][dt]);
                            O[rt][dt] = mma(v1, pf[rt][1], O[rt][dt]);
                        }
                    }
                    continue;
                }
                bool allact = true;
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) allact = allact && act[rt];
                if (FIXED && RT > 1 && allact) {
                    // edge tile needed by every row tile: as the interior
                    // path (every row tile's S^T first, so that one row
                    // tile's exponentials overlap another's MFMAs), with the
                    // keys outside a column's window masked in the exponent
                    f32x4 Sa[RT][4];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt) {
                            Sa[rt][mt] = f32x4{-bl2, -bl2, -bl2, -bl2};
#pragma unroll
                            for (int ks = 0; ks < C::NKS; ++ks) Sa[rt][mt] = mma(kf[mt][ks], qop[rt][ks], Sa[rt][mt]);
                        }
                    bf16x8 pf[RT][2];
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        const int i = q0 + 16 * rt + l16;
                        // this lane's valid key offsets, relative to its own kl
                        const int rlo = ((S > i - W + 1) ? S : i - W + 1) - kb - kl;
                        const int rhi = full[rt] ? 63 : i - kb - kl;
                        const int rl = full[rt] ? -64 : rlo;
                        float p[2][8];
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = 32 * (mt >> 1) + 4 * (mt & 1) + e;
                                const bool ok = (j >= rl) & (j <= rhi);
                                p[mt >> 1][(mt & 1) * 4 + e] = ex2(ok ? Sa[rt][mt][e] : -INFINITY);
                            }
                        pf[rt][0] = pack8(p[0]);
                        pf[rt][1] = pack8(p[1]);
                        ls[rt] += colsum(pf[rt][0], pf[rt][1]);
                    }
#pragma unroll
                    for (int dt = 0; dt < C::NDT; ++dt) {
                        const int r = 16 * dt + l16;
                        const bf16_t *vp = Vs + r * 64;
                        const int sw = swzV(r);
                        const bf16x8 v0 = ldb8(vp + 8 * (lg ^ sw)), v1 = ldb8(vp + 8 * ((lg + 4) ^ sw));
#pragma unroll
                        for (int rt = 0; rt < RT; ++rt) {
                            O[rt][dt] = mma(v0, pf[rt][0], O[rt][dt]);
                            O[rt][dt] = mma(v1, pf[rt][1], O[rt][dt]);
                        }
                    }
                    continue;
                }
                // per row tile: S^T, probabilities, packed P^T
                bf16x8 pb[RT][2];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    if (!act[rt]) continue;
                    f32x4 Sa[4];
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        Sa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int ks = 0; ks < C::NKS; ++ks) Sa[mt] = mma(kf[mt][ks], qop[rt][ks], Sa[mt]);
                    }
                    const int i = q0 + 16 * rt + l16;      // this lane's column
                    const int jlo = ((S > i - W + 1) ? S : i - W + 1) - kb;   // valid key offsets [jlo, jhi]
                    const int jhi = i - kb;
                    const bool fullt = full[rt];           // wave-uniform: no mask at all
                    float p[2][8];
                    float shift = bl2;
                    if constexpr (!FIXED) {
                        float tmax = -INFINITY;
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = kl + 32 * (mt >> 1) + 4 * (mt & 1) + e;
                                const bool ok = fullt | ((j >= jlo) & (j <= jhi));
                                tmax = fmaxf(tmax, ok ? Sa[mt][e] : -INFINITY);
                            }
                        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
                        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
                        const float mnew = fmaxf(mr[rt], tmax * sl2);
                        shift = (mnew == -INFINITY) ? 0.0f : mnew;
                        const float alpha = ex2(mr[rt] - shift);
                        mr[rt] = mnew;
                        ls[rt] *= alpha;
#pragma unroll
                        for (int dt = 0; dt < C::NDT; ++dt) O[rt][dt] *= alpha;
                    }
                    if (fullt) {
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                            for (int e = 0; e < 4; ++e) p[mt >> 1][(mt & 1) * 4 + e] = ex2(fmaf(Sa[mt][e], es, -shift));
                    } else {
                        // masked keys: the exp2 argument is selected to -inf (no branch per element)
#pragma unroll
                        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = kl + 32 * (mt >> 1) + 4 * (mt & 1) + e;
                                const bool ok = (j >= jlo) & (j <= jhi);
                                const float a = fmaf(Sa[mt][e], es, -shift);
                                p[mt >> 1][(mt & 1) * 4 + e] = ex2(ok ? a : -INFINITY);
                            }
                    }
                    pb[rt][0] = pack8(p[0]);
                    pb[rt][1] = pack8(p[1]);
                    ls[rt] += colsum(pb[rt][0], pb[rt][1]);
                }
                // O^T += V^T . P^T; each V^T fragment read once
#pragma unroll
                for (int dt = 0; dt < C::NDT; ++dt) {
                    const int r = 16 * dt + l16;
                    const bf16_t *vp = Vs + r * 64;
                    const int sw = swzV(r);
                    const bf16x8 v0 = ldb8(vp + 8 * (lg ^ sw)), v1 = ldb8(vp + 8 * ((lg + 4) ^ sw));
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        if (!act[rt]) continue;
                        O[rt][dt] = mma(v0, pb[rt][0], O[rt][dt]);
                        O[rt][dt] = mma(v1, pb[rt][1], O[rt][dt]);
                    }
                }
            }
        }
    }

    // normalise and store the window's rows and their LSE
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        const float l = ls[rt];   // the column's full sum in every lane
        const int i = q0 + 16 * rt + l16;
        if (i >= n || !hv) continue;
        const float inv = (l > 0.0f) ? 1.0f / l : 0.0f;
        bf16_t *orow = out + (int64_t)b * osb + (int64_t)i * osn + (int64_t)h * osh;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
            u32x2 u;
            u[0] = (uint32_t)f2bf(O[rt][dt][0] * inv) | ((uint32_t)f2bf(O[rt][dt][1] * inv) << 16);
            u[1] = (uint32_t)f2bf(O[rt][dt][2] * inv) | ((uint32_t)f2bf(O[rt][dt][3] * inv) << 16);
            *reinterpret_cast<u32x2 *>(orow + 16 * dt + 4 * lg) = u;
        }
        if (lg == 0) {
            const float sh = FIXED ? bl2 : mr[rt];
            lse[((int64_t)b * Hq + h) * n + i] = (l > 0.0f) ? (__log2f(l) + sh) / LOG2E : -INFINITY;
        }
    }
}

// Grid: Cn = B*Hkv*hsplit combos (the heads of a group split over hsplit
// workgroups of gw heads when G > 8) times the query tiles.
template <int D, int RT>
__global__ __launch_bounds__(256, 3) void attn_win_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    const float *__restrict__ kgain, float eps, const bf16_t *__restrict__ kr, const bf16_t *__restrict__ vt,
    const float *__restrict__ cosT, const float *__restrict__ sinT, int n, int Hq, int Hkv, int S,
    int W, float scale, int gw, int hsplit, int wsplit, int ntiles, int Cn,
    bf16_t *__restrict__ out, int64_t osb, int64_t osn, int64_t osh, float *__restrict__ lse) {
    extern __shared__ __align__(16) char smem[];
    // Work unit u = ((combo * ntiles + tile) * hsplit + hs), hs fastest.  XCD
    // x (workgroup i runs on XCD i % 8) takes the x-th contiguous eighth of
    // the units, so the heads and neighbouring tiles that read the same
    // keys share that XCD's L2.
    const int U = Cn * ntiles;
    const int chunk = (U + 7) / 8;
    const int u = (int)(blockIdx.x & 7) * chunk + (int)(blockIdx.x >> 3);
    if (u >= U) return;
    const int hs = u % hsplit;
    const int tile = (u / hsplit) % ntiles;
    const int combo = u / (hsplit * ntiles);
    const int G = Hq / Hkv;
    const float sl2 = scale * LOG2E;
    float bl2;
    if (group_bound(qgain, kgain, combo % Hkv, G, sl2, D, bl2))
        win_body<D, RT, true>(q, qsb, qsn, qsh, qgain, eps, kr, vt, cosT, sinT, n, Hq, Hkv, S, W, sl2, bl2, gw,
                              wsplit, combo, hs, tile, out, osb, osn, osh, lse, reinterpret_cast<bf16_t *>(smem));
    else
        win_body<D, RT, false>(q, qsb, qsn, qsh, qgain, eps, kr, vt, cosT, sinT, n, Hq, Hkv, S, W, sl2, bl2, gw,
                               wsplit, combo, hs, tile, out, osb, osn, osh, lse, reinterpret_cast<bf16_t *>(smem));
}

// ======================================================= routed kernel ====
enum { RM_SINK = 0, RM_COL = 1 };

// One staged block against one 16-row tile.  mode RM_SINK: keys j < S and
// j <= i are valid (nmt M-tiles can hold them); RM_COL: the block's keys j >=
// kfloor are valid for the columns whose query picked it (colok) -- kfloor is
// 0 except for routed block 1 when S > 64, whose keys below S are sinks.  S,
// kfloor and icol count from the block's first key.
template <int D, bool FIXED>
__device__ __forceinline__ void rt_update(const bf16_t *Ks, const bf16_t *Vs, const bf16x8 (&qop)[D / 32],
                                          f32x4 (&O)[D / 16], float &mrun, float &lsum, int mode,
                                          int64_t icol, bool colok, int S, int nmt, float sl2, float bl2,
                                          int l16, int lg, int kfloor = 0) {
    constexpr int NKS = D / 32, NDT = D / 16;
    // fixed shift, block columns: the query operand carries scale*log2(e), so
    // S^T starts at -shift (a column whose query did not pick the block at
    // -inf) and its exp2 needs no other operation
    const bool cinit = FIXED && mode == RM_COL;
    const float c0 = cinit ? (colok ? -bl2 : -INFINITY) : 0.0f;
    f32x4 Sa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Sa[mt] = f32x4{c0, c0, c0, c0};
        if (mt < nmt) {
            const int r = permk(mt, l16);
            const bf16_t *kp = Ks + r * D;
            const int sw = swzK(r);
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) Sa[mt] = mma(ldb8(kp + 8 * ((4 * ks + lg) ^ sw)), qop[ks], Sa[mt]);
        }
    }
    if (kfloor > 0) {   // wave-uniform and rare: keys below the floor out
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e < kfloor) Sa[mt][e] = -INFINITY;
    }
    float p[2][8];
    float shift = bl2;
    if constexpr (!FIXED) {
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const bool ok = (mode == RM_SINK) ? ((mt < nmt) & (j < S) & ((int64_t)j <= icol)) : colok;
                tmax = fmaxf(tmax, ok ? Sa[mt][e] : -INFINITY);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrun, tmax * sl2);
        shift = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = ex2(mrun - shift);
        mrun = mnew;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) O[dt] *= alpha;
    }
    if (cinit) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) p[mt >> 1][(mt & 1) * 4 + e] = ex2(Sa[mt][e]);
    } else if (mode == RM_COL) {
        // a column whose query did not pick the block: shift +inf, so every
        // exp2 argument is -inf (no select per element)
        const float sh = colok ? shift : INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) p[mt >> 1][(mt & 1) * 4 + e] = ex2(fmaf(Sa[mt][e], sl2, -sh));
    } else {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const bool ok = (mt < nmt) & (j < S) & ((int64_t)j <= icol);
                const float a = fmaf(Sa[mt][e], sl2, -shift);
                p[mt >> 1][(mt & 1) * 4 + e] = ex2(ok ? a : -INFINITY);
            }
    }
    const bf16x8 pb0 = pack8(p[0]), pb1 = pack8(p[1]);
    lsum += colsum(pb0, pb1);
    const bool two = mode != RM_SINK || nmt > 2;        // keys 32..63 can be valid
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        const int r = 16 * dt + l16;
        const bf16_t *vp = Vs + r * 64;
        const int sw = swzV(r);
        O[dt] = mma(ldb8(vp + 8 * (lg ^ sw)), pb0, O[dt]);
        if (two) O[dt] = mma(ldb8(vp + 8 * ((lg + 4) ^ sw)), pb1, O[dt]);
    }
}

// One staged window tile (RoPE keys) against one 16-row tile of the routed
// layout: keys jlo..jhi (from the tile's first key) of the column's window
// are valid, every key when full (wave-uniform).  qop is the RoPE operand.
template <int D, bool FIXED>
__device__ __forceinline__ void win_update(const bf16_t *Ks, const bf16_t *Vs, const bf16x8 (&qop)[D / 32],
                                           f32x4 (&O)[D / 16], float &mrun, float &lsum, bool full, int jlo,
                                           int jhi, float sl2, float bl2, int l16, int lg) {
    constexpr int NKS = D / 32, NDT = D / 16;
    // the row tiles of a wave read the same fragments: keep the compiler from
    // holding one tile's fragments in registers for the next (the routed
    // layout has no registers to spare for them)
    asm volatile("" ::: "memory");
    const float c0 = FIXED ? -bl2 : 0.0f;   // fixed shift: S^T starts at -shift, exp2 takes it directly
    f32x4 Sa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Sa[mt] = f32x4{c0, c0, c0, c0};
        const int r = permk(mt, l16);
        const bf16_t *kp = Ks + r * D;
        const int sw = swzK(r);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) Sa[mt] = mma(ldb8(kp + 8 * ((4 * ks + lg) ^ sw)), qop[ks], Sa[mt]);
    }
    float p[2][8];
    if constexpr (FIXED) {
        if (full) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) p[mt >> 1][(mt & 1) * 4 + e] = ex2(Sa[mt][e]);
        } else {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                    p[mt >> 1][(mt & 1) * 4 + e] = ex2(((j >= jlo) & (j <= jhi)) ? Sa[mt][e] : -INFINITY);
                }
        }
    } else {
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                tmax = fmaxf(tmax, (full | ((j >= jlo) & (j <= jhi))) ? Sa[mt][e] : -INFINITY);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrun, tmax * sl2);
        const float shift = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = ex2(mrun - shift);
        mrun = mnew;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) O[dt] *= alpha;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const float a = fmaf(Sa[mt][e], sl2, -shift);
                p[mt >> 1][(mt & 1) * 4 + e] = ex2((full | ((j >= jlo) & (j <= jhi))) ? a : -INFINITY);
            }
    }
    const bf16x8 pb0 = pack8(p[0]), pb1 = pack8(p[1]);
    lsum += colsum(pb0, pb1);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        const int r = 16 * dt + l16;
        const bf16_t *vp = Vs + r * 64;
        const int sw = swzV(r);
        O[dt] = mma(ldb8(vp + 8 * (lg ^ sw)), pb0, O[dt]);
        O[dt] = mma(ldb8(vp + 8 * ((lg + 4) ^ sw)), pb1, O[dt]);
    }
}

// P bits of a bit row starting at bit r0 (r0 > -32; bits before the row's
// start or past its nw words read as 0).
template <int P>
__device__ __forceinline__ uint32_t bits_at(const uint32_t *row, int r0, int nw) {
    const int a = r0 >> 5, sh = r0 & 31;   // arithmetic shift: word -1 for r0 < 0
    uint32_t v = (a >= 0 && a < nw) ? row[a] >> sh : 0u;
    if (sh != 0 && a + 1 < nw) v |= row[a + 1] << (32 - sh);
    return v & ((1u << P) - 1u);
}

// The union of the picks of a tile's QT queries (from i0, kk picks each) as
// an ascending list of routed blocks (sel: the picks, invalid ones SENT;
// bitmap and pre: the union as bits and the entries before each word), and
// each pick as bits over the list's entries: per query (qbits) and per row
// tile of QPT queries (wbits, nrt rows).  Returns the entry count (also in
// nlist).  Called by the whole workgroup of NTHR threads; ends with a barrier.
// pk: this thread's first pick (t = threadIdx.x) as pick_load left it, so
// that its loads can go out before the caller's other set-up.
struct Pick {
    int v, c;   // idx and cnt entries (SENT, 0 past the tile or the sequence)
};
__device__ __forceinline__ Pick pick_load(const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, int64_t bh,
                                          int64_t n, int64_t i0, int QT, int kk) {
    const int t = threadIdx.x, qq = t / kk, r = t - qq * kk;
    const int64_t i = i0 + qq;
    Pick pk{SENT, 0};
    if (t < QT * kk && i < n) {   // two independent loads
        pk.c = cnt[bh * n + i];
        pk.v = idx[(bh * n + i) * kk + r];
    }
    return pk;
}
template <int NTHR>
__device__ __forceinline__ int union_of_picks(const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt,
                                              int64_t bh, int64_t n, int64_t i0, int QT, int QPT, int nrt, int kk,
                                              int64_t nb, int nbw, int16_t *sel, uint32_t *bitmap, int *pre,
                                              int16_t *list, uint32_t *qbits, uint32_t *wbits, int &nlist, Pick pk) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int e = tid; e < nbw; e += NTHR) bitmap[e] = 0u;
    for (int e = tid; e < (QT + nrt) * nbw; e += NTHR) qbits[e] = 0u;   // wbits follow qbits
    __syncthreads();
    // one thread per (query, pick); invalid picks become SENT in place
    for (int t = tid; t < QT * kk; t += NTHR) {
        const int qq = t / kk, r = t - qq * kk;
        const int64_t i = i0 + qq;
        int v = pk.v, c = pk.c;
        if (t != tid) {
            c = (i < n) ? cnt[bh * n + i] : 0;
            v = (i < n) ? idx[(bh * n + i) * kk + r] : SENT;
        }
        if (i < n && r < min(max(c, 0), kk) && v >= 1 && v < nb)   // block 0 is never routed
            atomicOr(&bitmap[v >> 5], 1u << (v & 31));
        else
            v = SENT;
        sel[t] = (int16_t)v;
    }
    __syncthreads();
    if (w == 0) {
        int base = 0;
        for (int w0 = 0; w0 < nbw; w0 += 64) {
            uint32_t word = (w0 + lane < nbw) ? bitmap[w0 + lane] : 0u;
            const int pc = __popc(word);
            int incl = pc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            int off = base + incl - pc;
            if (w0 + lane < nbw) pre[w0 + lane] = off;
            while (word) {
                const int bit = __ffs(word) - 1;
                list[off++] = (int16_t)((w0 + lane) * 32 + bit);
                word &= word - 1u;
            }
            base += __shfl(incl, 63, 64);
        }
        if (lane == 0) nlist = base;
    }
    __syncthreads();
    const int ne = nlist;
    auto entry_of = [&](int v) { return pre[v >> 5] + __popc(bitmap[v >> 5] & ((1u << (v & 31)) - 1u)); };
    // each pick as a union entry index: its query's bits, and its row tile's
    for (int t = tid; t < QT * kk; t += NTHR) {
        const int v = sel[t];
        if (v == SENT) continue;
        const int qq = t / kk;
        const int e = entry_of(v);
        atomicOr(&qbits[qq * nbw + (e >> 5)], 1u << (e & 31));
        atomicOr(&wbits[(qq / QPT) * nbw + (e >> 5)], 1u << (e & 31));   // row tile qq / QPT
    }
    __syncthreads();
    return ne;
}

template <int D, int PTW, bool FIXED, bool S2, bool WIN>
__device__ __forceinline__ void routed_body(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const bf16_t *__restrict__ kc, const bf16_t *__restrict__ vt,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, int64_t n, int Hq, int Hkv, int S,
    int kk, float sl2, float bl2, int combo, int tile, bf16_t *__restrict__ out,
    int64_t osb, int64_t osn, int64_t osh, const float *__restrict__ lse, char *smem, int &nlist,
    const bf16_t *__restrict__ kr, const float *__restrict__ cosT, const float *__restrict__ sinT, int W,
    bf16_t *__restrict__ qrw) {
    using C = RtCfg<D>;
    const int G = Hq / Hkv;
    const int QPT = 16 / G;
    const int QT = C::WAVES * PTW * QPT;
    const int tid = threadIdx.x;
    const int lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index: uniform, kept in SGPRs
    const int b = combo / Hkv, g = combo % Hkv;
    const int64_t i0 = (int64_t)tile * QT;
    const int64_t bh = (int64_t)b * Hkv + g;
    const int64_t nb = n / 64;
    const int nbw = (int)((nb + 31) / 32);
    const bf16_t *KC = kc + bh * n * D;
    const bf16_t *VT = vt + bh * D * n;
    // WIN: the workgroup first streams the window tiles of its queries (kr
    // rows, RoPE operand) through the ring, then the sinks and routed blocks.
    const int64_t dkr = WIN ? (kr - kc) : 0;   // kc row -> the same kr row, in elements
    int wt0 = 0, nwin = 0;
    int woff = 0, wpre = 0;   // WIN: the window tiles' first ring slot; how many the routed loop issued
    if constexpr (WIN) {
        const int64_t ilast = ((i0 + QT < n) ? i0 + QT : n) - 1;
        const int64_t kfirst = ((int64_t)S > i0 - W + 1) ? (int64_t)S : i0 - W + 1;
        if (kfirst <= ilast) {
            wt0 = (int)(kfirst / 64);
            nwin = (int)(ilast / 64) - wt0 + 1;
        }
    }

    // LDS: ring | sel [QT][kk] | bitmap [nbw] | pre [nbw] | list [nb] |
    //      qbits [QT][nbw] | wbits [WAVES*PTW][nbw]
    bf16_t *ring = reinterpret_cast<bf16_t *>(smem);
    const uint32_t ring_lds = lds_offset(ring);            // LDS byte address of the ring
    int16_t *sel = reinterpret_cast<int16_t *>(smem + (size_t)C::NS * C::SLOT * 2);
    uint32_t *bitmap = reinterpret_cast<uint32_t *>(sel + ((QT * kk + 1) & ~1));   // union over blocks
    int *pre = reinterpret_cast<int *>(bitmap + nbw);        // union entries before each bitmap word
    int16_t *list = reinterpret_cast<int16_t *>(pre + nbw);   // union of the routed blocks, ascending
    uint32_t *qbits = reinterpret_cast<uint32_t *>(list + ((nb + 1) & ~1LL));   // per query, over entries
    uint32_t *wbits = qbits + QT * nbw;                      // per row tile: OR of its queries' qbits

    // A ring slot holds a block's K tile (kc rows blk*64..+63) and V^T tile
    // (vt columns blk*64..+63) in 1 KB parts, swizzled; part w + WAVES*pp is
    // this wave's.  Each lane's source at block 0 and the wave-uniform stride
    // per block are set once, so a fill is one address add per part.
    const bf16_t *dsrc[C::DPW];
    int64_t dstr[C::DPW];
#pragma unroll
    for (int pp = 0; pp < C::DPW; ++pp) {
        const int part = w + C::WAVES * pp;
        const int pc = (part % C::KPARTS) * 64 + lane;
        if (part < C::KPARTS) {
            const int r = pc / (D / 8), c = (pc % (D / 8)) ^ swzK(pc / (D / 8));
            dsrc[pp] = KC + r * D + 8 * c;
            dstr[pp] = 64 * D;
        } else {
            const int r = pc >> 3, c = (pc & 7) ^ swzV(pc >> 3);
            dsrc[pp] = VT + (int64_t)r * n + 8 * c;
            dstr[pp] = 64;
        }
    }
    auto fill = [&](int blk, int slot, bool rope) {
#pragma unroll
        for (int pp = 0; pp < C::DPW; ++pp) {
            const bool kpart = w + C::WAVES * pp < C::KPARTS;   // wave-uniform
            dma16(dsrc[pp] + (int64_t)blk * dstr[pp] + ((WIN && rope && kpart) ? dkr : 0),
                  ring_lds + (uint32_t)(slot * C::SLOT * 2) + (uint32_t)(w + C::WAVES * pp) * 1024u);
        }
    };
    constexpr int NPRO = (C::NS / C::PH - 1) * C::PH;   // entries staged ahead of the first phase
    // sinks: block 0 into the last ring slot and (S > 64) block 1 into the
    // one before (both free until the first refill), landing during the set-up
    if (S > 0) fill(0, C::NS - 1, false);
    if (S2) fill(1, C::NS - 2, false);

    // this thread's first pick, loaded before the query rows
    const Pick pk = pick_load(idx, cnt, bh, n, i0, QT, kk);

    // ----------------------------------------------------- per-row state --
    // (first, so that the query loads overlap the selection set-up)
    const int qs = l16 / G;
    const int hh = l16 % G;
    const bool colv = l16 < QPT * G;
    bf16x8 qop[PTW][C::NKS];
    f32x4 O[PTW][C::NDT];
    float mrun[PTW], lsum[PTW];
    int64_t icol[PTW];
    bool cok[PTW];
#pragma unroll
    for (int t = 0; t < PTW; ++t) {
        icol[t] = i0 + (int64_t)(w * PTW + t) * QPT + qs;
        cok[t] = colv && icol[t] < n;
        mrun[t] = -INFINITY;
        lsum[t] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) O[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (WIN && nwin > 0) {
            // the RoPE operand of the window tiles, parked in the workspace
            // ([B, n, Hq, D], the row of this column) until the routed blocks
            // are done; its loads overlap the selection set-up
            float x[C::NKS][8];
            qrow<D>(q, qsb, qsn, qsh, qgain, eps, b, icol[t], g * G + hh, cok[t], lg, x);
            qpack<D>(x, cok[t], FIXED ? sl2 : 1.0f, qop[t]);
            bf16x8 qr[C::NKS];
            qpack_rope<D>(x, cosT, sinT, icol[t], cok[t], lg, FIXED ? sl2 : 1.0f, qr);
            if (cok[t]) {
                bf16_t *dst = qrw + (((int64_t)b * n + icol[t]) * Hq + g * G + hh) * D + 8 * lg;
#pragma unroll
                for (int ks = 0; ks < C::NKS; ++ks)
                    *reinterpret_cast<u32x4 *>(dst + 32 * ks) = __builtin_bit_cast(u32x4, qr[ks]);
            }
        } else {
            qoperand<D>(q, qsb, qsn, qsh, qgain, eps, nullptr, nullptr, b, icol[t], g * G + hh, cok[t], false, lg,
                        FIXED ? sl2 : 1.0f, qop[t]);
        }
    }

    // ------------------------------------- selection lists and their union
    const int ne = union_of_picks<C::NTHR>(idx, cnt, bh, n, i0, QT, QPT, C::WAVES * PTW, kk, nb, nbw, sel, bitmap, pre,
                                           list, qbits, wbits, nlist, pk);

    // The ring holds NPH phases of PH blocks, with one barrier per phase: a
    // block's hits fall on few of the waves, and a phase of several blocks
    // evens the waves' work out before they meet again.
    constexpr int P = C::PH, NPH = C::NS / C::PH;
    static_assert(32 % P == 0, "a phase's entries lie in one bitmap word");
    static_assert(NPRO == (NPH - 1) * P, "prologue depth");
    {
        const int npro = min(ne, NPRO);
        for (int e = 0; e < npro; ++e) fill(list[e], e, false);
        if (S > 0) {
            wait_vm_n(npro * C::DPW);
            __syncthreads();   // every share of the sink blocks landed
            for (int sb = 0; sb < (S2 ? 2 : 1); ++sb) {
                const bf16_t *Ks = ring + (C::NS - 1 - sb) * C::SLOT;
                const int Sb = min(S - 64 * sb, 64);            // sink keys of this block
                const int nmt = (Sb <= 4) ? 1 : (Sb <= 32 ? 2 : 4);   // M-tiles holding keys 0..Sb-1
#pragma unroll
                for (int tt = 0; tt < PTW; ++tt) {
                    if (i0 + (int64_t)(w * PTW + tt) * QPT >= n) break;
                    rt_update<D, FIXED>(Ks, Ks + 64 * D, qop[tt], O[tt], mrun[tt], lsum[tt], RM_SINK, icol[tt] - 64 * sb,
                                        cok[tt], Sb, nmt, FIXED ? 1.0f : sl2, bl2, l16, lg);
                }
            }
        }
        // with S > 64 the keys 64..S-1 are sinks: routed block 1 (union entry 0
        // if picked) counts only its keys from S on
        const bool b1 = S2 && ne > 0 && list[0] == 1;
        // WIN: the last routed phase also issues the first window tiles, into
        // the slots after its own (those of the phase before it, consumed
        // before its barrier), so that they land during its updates; the
        // window tiles then run through the ring from slot woff
        woff = 0;
        wpre = 0;
        uint32_t qw[PTW], ww[PTW];   // this lane's query's / this row tile's bits of the current word
        for (int e0 = 0; e0 < ne; e0 += P) {
            // this wave's shares of entries e0..e0+P-1 have landed once at most
            // the shares of the entries issued after them are in flight
            const int issued = min(ne, e0 + (NPH - 1) * P);
            wait_vm_n(max(0, issued - (e0 + P)) * C::DPW);
            __syncthreads();   // every share of this phase landed; the previous phase (and the sinks) consumed
            const int nf = min(ne, e0 + NPH * P);
            int nxt[P];   // the refill's block ids, read before the first DMA is issued
#pragma unroll
            for (int j = 0; j < P; ++j) nxt[j] = (issued + j < nf) ? list[issued + j] : 0;
#pragma unroll
            for (int j = 0; j < P; ++j)
                if (issued + j < nf) fill(nxt[j], (issued + j) % C::NS, false);
            if constexpr (WIN) {
                if (e0 + P >= ne && nwin > 0) {   // the last phase (wave-uniform)
                    woff = (e0 + P) % C::NS;
                    wpre = min(nwin, NPRO);
                    for (int e = 0; e < wpre; ++e) fill(wt0 + e, (woff + e) % C::NS, true);
                }
            }
            const int sh = e0 & 31;
            if (sh == 0) {
#pragma unroll
                for (int tt = 0; tt < PTW; ++tt) {
                    const int rt = w * PTW + tt;
                    qw[tt] = cok[tt] ? qbits[(rt * QPT + qs) * nbw + (e0 >> 5)] : 0u;
                    ww[tt] = __builtin_amdgcn_readfirstlane(wbits[rt * nbw + (e0 >> 5)]);
                }
            }
#pragma unroll
            for (int tt = 0; tt < PTW; ++tt) {
                uint32_t hits = (ww[tt] >> sh) & ((1u << P) - 1u);   // this phase's entries the row tile needs
                while (hits) {
                    const int j = __builtin_ctz(hits);
                    hits &= hits - 1u;
                    const int e = e0 + j;
                    const bf16_t *Ks = ring + (e % C::NS) * C::SLOT;
                    const bool hit = (qw[tt] >> (sh + j)) & 1u;
                    rt_update<D, FIXED>(Ks, Ks + 64 * D, qop[tt], O[tt], mrun[tt], lsum[tt], RM_COL, icol[tt], hit, S,
                                        4, FIXED ? 1.0f : sl2, bl2, l16, lg, (S2 && b1 && e == 0) ? S - 64 : 0);
                }
            }
        }
    }

    if constexpr (WIN) {
        // ---- then the window tiles (kr rows) with the RoPE operand, every
        // row tile whose columns have keys in them
        if (nwin > 0) {
            __syncthreads();   // every wave is done with the ring
            // the RoPE operand back from the workspace (this lane's own rows)
#pragma unroll
            for (int t = 0; t < PTW; ++t) {
                const bf16_t *src = qrw + (((int64_t)b * n + (cok[t] ? icol[t] : 0)) * Hq + g * G + hh) * D + 8 * lg;
#pragma unroll
                for (int ks = 0; ks < C::NKS; ++ks) {
                    const bf16x8 v = ldb8(src + 32 * ks);
                    qop[t][ks] = cok[t] ? v : bf16x8{};
                }
            }
            for (int e = wpre; e < nwin && e < NPRO; ++e) fill(wt0 + e, (woff + e) % C::NS, true);
        }
        for (int e0 = 0; e0 < nwin; e0 += P) {
            const int issued = min(nwin, e0 + (NPH - 1) * P);
            wait_vm_n(max(0, issued - (e0 + P)) * C::DPW);
            __syncthreads();   // every share of this phase landed; the previous phase consumed
            const int nf = min(nwin, e0 + NPH * P);
            for (int e = issued; e < nf; ++e) fill(wt0 + e, (woff + e) % C::NS, true);
            const int e1 = min(nwin, e0 + P);
#pragma nounroll
            for (int e = e0; e < e1; ++e) {
                const bf16_t *Ks = ring + ((woff + e) % C::NS) * C::SLOT;
                const int64_t kb = (int64_t)(wt0 + e) * 64;
#pragma unroll
                for (int tt = 0; tt < PTW; ++tt) {
                    const int64_t qa = i0 + (int64_t)(w * PTW + tt) * QPT;
                    if (qa >= n) break;
                    const int64_t qb = (qa + QPT - 1 < n) ? qa + QPT - 1 : n - 1;
                    const int64_t loa = ((int64_t)S > qa - W + 1) ? (int64_t)S : qa - W + 1;
                    const int64_t lob = ((int64_t)S > qb - W + 1) ? (int64_t)S : qb - W + 1;
                    if (kb > qb || kb + 63 < loa) continue;   // no column has a window key here
                    const bool full = kb >= lob && kb + 63 <= qa;
                    const int64_t lo = ((int64_t)S > icol[tt] - W + 1) ? (int64_t)S : icol[tt] - W + 1;
                    const int64_t jlo = lo - kb, jhi = icol[tt] - kb;
                    win_update<D, FIXED>(Ks, Ks + 64 * D, qop[tt], O[tt], mrun[tt], lsum[tt], full,
                                         (int)(jlo < 0 ? 0 : (jlo > 64 ? 64 : jlo)),
                                         (int)(jhi < -1 ? -1 : (jhi > 63 ? 63 : jhi)), FIXED ? 1.0f : sl2, bl2,
                                         l16, lg);
                }
            }
        }
        // ------------------------------------------- normalise and store
#pragma unroll
        for (int t = 0; t < PTW; ++t) {
            const float l = lsum[t];   // the column's full sum in every lane
            if (!cok[t]) continue;
            const float inv = (l > 0.0f) ? 1.0f / l : 0.0f;
            bf16_t *orow = out + (int64_t)b * osb + icol[t] * osn + (int64_t)(g * G + hh) * osh;
#pragma unroll
            for (int dt = 0; dt < C::NDT; ++dt) {
                u32x2 u;
                u[0] = (uint32_t)f2bf(O[t][dt][0] * inv) | ((uint32_t)f2bf(O[t][dt][1] * inv) << 16);
                u[1] = (uint32_t)f2bf(O[t][dt][2] * inv) | ((uint32_t)f2bf(O[t][dt][3] * inv) << 16);
                *reinterpret_cast<u32x2 *>(orow + 16 * dt + 4 * lg) = u;
            }
        }
        return;
    }
    // ------------------- merge with the window's (out, LSE), normalise, store
#pragma unroll
    for (int t = 0; t < PTW; ++t) {
        const float l = lsum[t];   // the column's full sum in every lane
        if (!cok[t]) continue;
        const int h = g * G + hh;
        const int64_t i = icol[t];
        const float lw = lse[((int64_t)b * Hq + h) * n + i];           // natural log
        const float sh = FIXED ? bl2 : mrun[t];
        const float lr = (l > 0.0f) ? (__log2f(l) + sh) / LOG2E : -INFINITY;
        const float m = fmaxf(lw, lr);
        const float ww = (lw == -INFINITY) ? 0.0f : __expf(lw - m);
        const float wr = (lr == -INFINITY) ? 0.0f : __expf(lr - m);
        const float den = ww + wr;
        const float fw = den > 0.0f ? ww / den : 0.0f;
        const float fr = (den > 0.0f && l > 0.0f) ? wr / (den * l) : 0.0f;
        bf16_t *orow = out + (int64_t)b * osb + i * osn + (int64_t)h * osh;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
            u32x2 u = *reinterpret_cast<const u32x2 *>(orow + 16 * dt + 4 * lg);
            float o[4];
            o[0] = __uint_as_float(u[0] << 16) * fw + O[t][dt][0] * fr;
            o[1] = __uint_as_float(u[0] & 0xffff0000u) * fw + O[t][dt][1] * fr;
            o[2] = __uint_as_float(u[1] << 16) * fw + O[t][dt][2] * fr;
            o[3] = __uint_as_float(u[1] & 0xffff0000u) * fw + O[t][dt][3] * fr;
            u[0] = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
            u[1] = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
            *reinterpret_cast<u32x2 *>(orow + 16 * dt + 4 * lg) = u;
        }
    }
}

// S2: sinks beyond the first block (64 < S <= 128), a separate instantiation
// so that the common case carries none of its code.  WIN: the whole union in
// one launch (window tiles from kr first, then the sinks and routed blocks,
// one softmax state, rows normalised and stored); otherwise the sinks and
// routed blocks merged into the window launch's rows by their LSE.
template <int D, int PTW, bool S2, bool WIN>
__global__ __launch_bounds__(RtCfg<D>::NTHR, RtCfg<D>::NTHR / 256) void attn_routed_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    const float *__restrict__ kgain, float eps, const bf16_t *__restrict__ kc, const bf16_t *__restrict__ vt,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, int64_t n, int Hq, int Hkv, int S,
    int kk, float scale, int ntiles, int Cn, int xmap, bf16_t *__restrict__ out,
    int64_t osb, int64_t osn, int64_t osh, const float *__restrict__ lse, const bf16_t *__restrict__ kr,
    const float *__restrict__ cosT, const float *__restrict__ sinT, int W, bf16_t *__restrict__ qrw) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int nlist;
    int combo, tile;
    xcd_map(blockIdx.x, Cn, ntiles, xmap, combo, tile);
    if (tile >= ntiles || combo >= Cn) return;
    const int G = Hq / Hkv;
    const float sl2 = scale * LOG2E;
    float bl2;
    if (group_bound(qgain, kgain, combo % Hkv, G, sl2, D, bl2))
        routed_body<D, PTW, true, S2, WIN>(q, qsb, qsn, qsh, qgain, eps, kc, vt, idx, cnt, n, Hq, Hkv, S, kk, sl2,
                                           bl2, combo, tile, out, osb, osn, osh, lse, smem, nlist, kr, cosT, sinT,
                                           W, qrw);
    else
        routed_body<D, PTW, false, S2, WIN>(q, qsb, qsn, qsh, qgain, eps, kc, vt, idx, cnt, n, Hq, Hkv, S, kk,
                                            sl2, bl2, combo, tile, out, osb, osn, osh, lse, smem, nlist, kr, cosT,
                                            sinT, W, qrw);
}


// ========================================== query gradient (backward) ====
// bwd_dq_union_kernel: the query gradient of the union attention for bf16
// inputs, on the forward's layout -- workgroup = (batch, KV head, QT
// queries), 16-row tiles of the G heads of 16/G queries, PTW tiles per wave
// -- so that each staged block serves every query of the tile that picked
// it.  Per column (query i, head h) over its union U_i, with p the softmax,
// D = <dO, O> and k the key the score was taken against:
//   dP_j = <dO, v_j>,  ds_j = p_j (dP_j - D),  dq^ += scale sum_j ds_j k_j
// (the gradient with respect to the QKNorm'd row; window keys give it in the
// rotated frame).  Per 64-key block: S^T = K.Q^T and dP^T = V.dO^T (K and V
// tiles, key rows in permk order, so that both accumulators come out in the
// B-operand layout), then dq^T += K^T.dS^T (K^T tile).  A ring slot holds
// the three tiles.  The window tiles (kr, krt; the RoPE operand) stream
// first; rope^T then maps the column's partial sum back to the unrotated
// frame in registers (a row element and its rotation partner sit in the same
// lane) and the sinks and routed blocks (kc, kct; the NoPE operand, read back
// from the rows this workgroup wrote at set-up) follow in the same softmax
// state.  Softmax as the forward: the QKNorm bound as a fixed shift when it
// holds, else a running max.  Outputs: dq (rope^T and the QKNorm backward
// applied), the gain gradient (one atomic per head per workgroup), and for
// the key-gradient kernels the QKNorm'd and rotated rows (bf16), the LSE
// (natural log) and D.
template <int D, int WAVES>
struct DqCfg {
    static constexpr int NKS = D / 32;
    static constexpr int NDT = D / 16;
    static constexpr int NTHR = WAVES * 64;
    static constexpr int TILE = 64 * D;                   // bf16 elements of a K, V or K^T tile
    static constexpr int SLOT = 3 * TILE;
    static constexpr int KPARTS = TILE * 2 / 1024;        // 1 KB parts of a tile
    static constexpr int NPARTS = 3 * KPARTS;
    static constexpr int PPW = (NPARTS + WAVES - 1) / WAVES;   // DMA parts per wave per block, at most
};

enum { DQ_ALL = 0, DQ_COL = 1, DQ_RANGE = 2 };

// The MFMA operand x * f, rounded to bf16 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 scale8(bf16x8 x, float f) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (float)x[e] * f;
    return pack8(y);
}

// One staged block (K tile Ks, V tile Vk, K^T tile KT) against one 16-row
// tile.  MODE DQ_ALL: every key of every column; DQ_COL: every key of the
// columns whose query picked the block (colok); DQ_RANGE: keys jlo..jhi
// (from the block's first key) of each column.  acc accumulates
// sum_j p~_j (dP_j - D) k_j with p~ = exp2 of the score less the shift;
// lsum (per lane: the lane's keys only) sum_j p~_j.  The V fragments are read
// after the scores' exponentials, so that the K and V fragments are not live
// together.
template <int D, bool FIXED, int MODE>
__device__ __forceinline__ void dq_update(const bf16_t *Ks, const bf16_t *Vk, const bf16_t *KT,
                                          const bf16x8 (&qop)[D / 32], const bf16x8 (&dop)[D / 32], float Dh,
                                          f32x4 (&acc)[D / 16], float &mrun, float &lsum, bool colok, int jlo,
                                          int jhi, float sl2, float bl2, int l16, int lg) {
    constexpr int NKS = D / 32, NDT = D / 16;
    asm volatile("" ::: "memory");   // no fragment held over from the previous row tile
    const bool cdead = MODE == DQ_COL && !colok;
    const float c0 = FIXED ? (cdead ? -INFINITY : -bl2) : 0.0f;
    const int sw = swzK(permk(0, l16));   // the same for every mt
    f32x4 Sa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Sa[mt] = f32x4{c0, c0, c0, c0};
        const int r = permk(mt, l16);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) Sa[mt] = mma(ldb8(Ks + r * D + 8 * ((4 * ks + lg) ^ sw)), qop[ks], Sa[mt]);
    }
    float p[4][4];
    if constexpr (FIXED) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const bool ok = (MODE != DQ_RANGE) || ((j >= jlo) & (j <= jhi));
                p[mt][e] = ex2(ok ? Sa[mt][e] : -INFINITY);
            }
    } else {
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const bool ok = (MODE == DQ_RANGE) ? ((j >= jlo) & (j <= jhi)) : !cdead;
                tmax = fmaxf(tmax, ok ? Sa[mt][e] : -INFINITY);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(mrun, tmax * sl2);
        const float shift = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = ex2(mrun - shift);
        mrun = mnew;
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[dt] *= alpha;
        const float sh = cdead ? INFINITY : shift;   // a dead column: every argument -inf
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 32 * (mt >> 1) + 8 * lg + 4 * (mt & 1) + e;
                const bool ok = (MODE != DQ_RANGE) || ((j >= jlo) & (j <= jhi));
                p[mt][e] = ex2(ok ? fmaf(Sa[mt][e], sl2, -sh) : -INFINITY);
            }
    }
    f32x4 Pa[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        Pa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int r = permk(mt, l16);
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) Pa[mt] = mma(ldb8(Vk + r * D + 8 * ((4 * ks + lg) ^ sw)), dop[ks], Pa[mt]);
    }
    float ds[2][8];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lsum += p[mt][e];
            ds[mt >> 1][(mt & 1) * 4 + e] = p[mt][e] * (Pa[mt][e] - Dh);
        }
    const bf16x8 db0 = pack8(ds[0]), db1 = pack8(ds[1]);
    const int swt = swzV(l16);   // swzV(16 dt + l16) for every dt
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        const bf16_t *kp = KT + (16 * dt + l16) * 64;
        acc[dt] = mma(ldb8(kp + 8 * (lg ^ swt)), db0, acc[dt]);
        acc[dt] = mma(ldb8(kp + 8 * ((lg + 4) ^ swt)), db1, acc[dt]);
    }
}

template <int D, int WAVES, int PTW, int NS, int PH, bool FIXED>
__device__ __forceinline__ void dq_body(
    const bf16_t *__restrict__ q, const float *__restrict__ qgain, float eps, const bf16_t *__restrict__ kc,
    const bf16_t *__restrict__ kr, const bf16_t *__restrict__ kct, const bf16_t *__restrict__ krt,
    const bf16_t *__restrict__ v, const float *__restrict__ cosT, const float *__restrict__ sinT,
    const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt, const bf16_t *__restrict__ out,
    const bf16_t *__restrict__ dout, int64_t n, int Hq, int Hkv, int S, int W, int kk, float scale, float sl2,
    float bl2, int combo, int tile, bf16_t *__restrict__ qc_ws, bf16_t *__restrict__ qr_ws,
    float *__restrict__ lse_ws, float *__restrict__ dd_ws, bf16_t *__restrict__ dq, float *__restrict__ dq_gain,
    char *smem, int &nlist) {
    using C = DqCfg<D, WAVES>;
    constexpr int NKS = C::NKS, NDT = C::NDT;
    constexpr int P = PH, NPH = NS / PH, NPRO = (NPH - 1) * PH;
    static_assert(NS % PH == 0 && NPH >= 2, "the ring holds whole phases, one of them ahead");
    const int G = Hq / Hkv;
    const int QPT = 16 / G;
    const int QT = WAVES * PTW * QPT;
    const int tid = threadIdx.x;
    const int lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = combo / Hkv, g = combo % Hkv;
    const int64_t i0 = (int64_t)tile * QT;
    const int64_t bh = (int64_t)b * Hkv + g;
    const int64_t nb = n / 64;
    const int nbw = (int)((nb + 31) / 32);
    int wt0 = 0, nwin = 0;   // the window tiles of the workgroup's queries
    {
        const int64_t ilast = ((i0 + QT < n) ? i0 + QT : n) - 1;
        const int64_t kfirst = ((int64_t)S > i0 - W + 1) ? (int64_t)S : i0 - W + 1;
        if (kfirst <= ilast) {
            wt0 = (int)(kfirst / 64);
            nwin = (int)(ilast / 64) - wt0 + 1;
        }
    }

    // LDS: ring | sel [QT][kk] | bitmap [nbw] | pre [nbw] | list [nb] |
    //      qbits [QT][nbw] | wbits [WAVES*PTW][nbw]
    bf16_t *ring = reinterpret_cast<bf16_t *>(smem);
    const uint32_t ring_lds = lds_offset(ring);
    int16_t *sel = reinterpret_cast<int16_t *>(smem + (size_t)NS * C::SLOT * 2);
    uint32_t *bitmap = reinterpret_cast<uint32_t *>(sel + ((QT * kk + 1) & ~1));
    int *pre = reinterpret_cast<int *>(bitmap + nbw);
    int16_t *list = reinterpret_cast<int16_t *>(pre + nbw);
    uint32_t *qbits = reinterpret_cast<uint32_t *>(list + ((nb + 1) & ~1LL));
    uint32_t *wbits = qbits + QT * nbw;

    // A ring slot: K tile [64][D] (swzK), V tile [64][D] (swzK), K^T tile
    // [D][64] (swzV), in 1 KB parts; part w + WAVES*pp is this wave's.  The
    // sources at block 0 and the stride per block are set once; a window tile
    // reads kr / krt (the same rows of the other tensor) instead of kc / kct.
    const bf16_t *KC = kc + bh * n * D;
    const bf16_t *KCT = kct + bh * D * n;
    const bf16_t *VB = v + ((int64_t)b * n * Hkv + g) * D;   // v [B, n, Hkv, D]
    const int64_t dkr = kr - kc, dkrt = krt - kct;
    const bf16_t *dsrc[C::PPW];
    int64_t dstr[C::PPW], drot[C::PPW];
#pragma unroll
    for (int pp = 0; pp < C::PPW; ++pp) {
        const int part = w + WAVES * pp;
        const int tl = part / C::KPARTS;            // 0: K, 1: V, 2: K^T, 3: none
        const int pc = (part % C::KPARTS) * 64 + lane;
        dsrc[pp] = KC;
        dstr[pp] = 0;
        drot[pp] = 0;
        if (tl == 0) {
            const int r = pc / (D / 8), c = (pc % (D / 8)) ^ swzK(pc / (D / 8));
            dsrc[pp] = KC + r * D + 8 * c;
            dstr[pp] = 64 * D;
            drot[pp] = dkr;
        } else if (tl == 1) {
            const int r = pc / (D / 8), c = (pc % (D / 8)) ^ swzK(pc / (D / 8));
            dsrc[pp] = VB + (int64_t)r * Hkv * D + 8 * c;
            dstr[pp] = 64 * (int64_t)Hkv * D;
        } else if (tl == 2) {
            const int r = pc >> 3, c = (pc & 7) ^ swzV(pc >> 3);
            dsrc[pp] = KCT + (int64_t)r * n + 8 * c;
            dstr[pp] = 64;
            drot[pp] = dkrt;
        }
    }
    const int dpw = (C::NPARTS - w + WAVES - 1) / WAVES;   // this wave's DMA instructions per block
    auto fill = [&](int blk, int slot, bool rope) {
#pragma unroll
        for (int pp = 0; pp < C::PPW; ++pp)
            if (w + WAVES * pp < C::NPARTS)   // wave-uniform
                dma16(dsrc[pp] + (int64_t)blk * dstr[pp] + (rope ? drot[pp] : 0),
                      ring_lds + (uint32_t)(slot * C::SLOT * 2) + (uint32_t)(w + WAVES * pp) * 1024u);
    };
    // the first window tiles land during the set-up
    for (int e = 0; e < nwin && e < NPRO; ++e) fill(wt0 + e, e, true);
    const Pick pk = pick_load(idx, cnt, bh, n, i0, QT, kk);   // this thread's first pick

    // ----------------------------------------------------- per-row state --
    const int qs = l16 / G;
    const int hh = l16 % G;
    const int h = g * G + hh;
    const bool colv = l16 < QPT * G;
    bf16x8 qop[PTW][NKS], dop[PTW][NKS];
    f32x4 acc[PTW][NDT];
    float mrun[PTW], lsum[PTW], Dh[PTW];
    int64_t icol[PTW];
    bool cok[PTW];
#pragma unroll
    for (int t = 0; t < PTW; ++t) {
        icol[t] = i0 + (int64_t)(w * PTW + t) * QPT + qs;
        cok[t] = colv && icol[t] < n;
        mrun[t] = -INFINITY;
        lsum[t] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[t][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int64_t row = (((int64_t)b * n + (cok[t] ? icol[t] : 0)) * Hq + h) * D + 8 * lg;
        float x[NKS][8];
        qrow<D>(q, n * Hq * D, (int64_t)Hq * D, D, qgain, eps, b, icol[t], h, cok[t], lg, x);
        bf16x8 qn[NKS], qr[NKS];   // the QKNorm'd row and its rotation (bf16-exact)
        qpack<D>(x, cok[t], 1.0f, qn);
        qpack_rope<D>(x, cosT, sinT, icol[t], cok[t], lg, 1.0f, qr);
        float od = 0.0f;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            if (cok[t]) {
                *reinterpret_cast<u32x4 *>(qc_ws + row + 32 * ks) = __builtin_bit_cast(u32x4, qn[ks]);
                *reinterpret_cast<u32x4 *>(qr_ws + row + 32 * ks) = __builtin_bit_cast(u32x4, qr[ks]);
            }
            qop[t][ks] = FIXED ? scale8(qr[ks], sl2) : qr[ks];
            const u32x4 du = *reinterpret_cast<const u32x4 *>(dout + row + 32 * ks);
            const u32x4 uo = *reinterpret_cast<const u32x4 *>(out + row + 32 * ks);
            dop[t][ks] = cok[t] ? __builtin_bit_cast(bf16x8, du) : bf16x8{};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                od = fmaf(__uint_as_float(du[e] << 16), __uint_as_float(uo[e] << 16), od);
                od = fmaf(__uint_as_float(du[e] & 0xffff0000u), __uint_as_float(uo[e] & 0xffff0000u), od);
            }
        }
        od += __shfl_xor(od, 16, 64);
        od += __shfl_xor(od, 32, 64);
        Dh[t] = cok[t] ? od : 0.0f;
        if (cok[t] && lg == 0) dd_ws[((int64_t)b * Hq + h) * n + icol[t]] = od;
    }

    // ------------------------------------- selection lists and their union
    const int ne = union_of_picks<C::NTHR>(idx, cnt, bh, n, i0, QT, QPT, WAVES * PTW, kk, nb, nbw, sel, bitmap, pre,
                                           list, qbits, wbits, nlist, pk);

    // ----------------------------------------- window tiles (RoPE operand)
    for (int e0 = 0; e0 < nwin; e0 += P) {
        const int issued = min(nwin, e0 + NPRO);
        wait_vm_n(max(0, issued - (e0 + P)) * dpw);
        __syncthreads();   // every share of this phase landed; the previous phase consumed
        const int nf = min(nwin, e0 + NPH * P);
        for (int e = issued; e < nf; ++e) fill(wt0 + e, e % NS, true);
        const int e1 = min(nwin, e0 + P);
#pragma nounroll
        for (int e = e0; e < e1; ++e) {
            const bf16_t *Ks = ring + (e % NS) * C::SLOT;
            const int64_t kb = (int64_t)(wt0 + e) * 64;
#pragma unroll
            for (int tt = 0; tt < PTW; ++tt) {
                const int64_t qa = i0 + (int64_t)(w * PTW + tt) * QPT;
                if (qa >= n) break;
                const int64_t qb = (qa + QPT - 1 < n) ? qa + QPT - 1 : n - 1;
                const int64_t loa = ((int64_t)S > qa - W + 1) ? (int64_t)S : qa - W + 1;
                const int64_t lob = ((int64_t)S > qb - W + 1) ? (int64_t)S : qb - W + 1;
                if (kb > qb || kb + 63 < loa) continue;   // no column has a window key here
                const bool full = kb >= lob && kb + 63 <= qa;
                const int64_t lo = ((int64_t)S > icol[tt] - W + 1) ? (int64_t)S : icol[tt] - W + 1;
                const int64_t jlo = lo - kb, jhi = cok[tt] ? icol[tt] - kb : -1;
                // a full tile as the range 0..63 (one inlined copy of the update)
                dq_update<D, FIXED, DQ_RANGE>(Ks, Ks + C::TILE, Ks + 2 * C::TILE, qop[tt], dop[tt], Dh[tt], acc[tt],
                                              mrun[tt], lsum[tt], true,
                                              full ? 0 : (int)(jlo < 0 ? 0 : (jlo > 64 ? 64 : jlo)),
                                              full ? 63 : (int)(jhi < -1 ? -1 : (jhi > 63 ? 63 : jhi)), sl2, bl2,
                                              l16, lg);
            }
        }
    }

    // ------------------- back to the unrotated frame; the NoPE operand
    __syncthreads();   // every wave is done with the ring
    const int hs = (S > 0) ? 1 : 0;   // stream entry 0 is the sink block when there are sinks
    const int ntot = hs + ne;
    auto sblk = [&](int c) { return (c < hs) ? 0 : (int)list[c - hs]; };
    for (int c = 0; c < ntot && c < NPRO; ++c) fill(sblk(c), c, false);
#pragma unroll
    for (int t = 0; t < PTW; ++t) {
        const int64_t ii = cok[t] ? icol[t] : 0;
        // rope^T(z) = z cos + rot^T(z sin), rot^T([z1, z2]) = [z2, -z1]: element
        // d = 16 dt + 4 lg + e and its partner d ^ D/2 (dt ^ NDT/2) in this lane
        float cs[NDT][4], sn[NDT][4];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const float4 c4 = *reinterpret_cast<const float4 *>(cosT + ii * D + 16 * dt + 4 * lg);
            const float4 s4 = *reinterpret_cast<const float4 *>(sinT + ii * D + 16 * dt + 4 * lg);
            cs[dt][0] = c4.x, cs[dt][1] = c4.y, cs[dt][2] = c4.z, cs[dt][3] = c4.w;
            sn[dt][0] = s4.x, sn[dt][1] = s4.y, sn[dt][2] = s4.z, sn[dt][3] = s4.w;
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                rnd_bf16_pair(cs[dt][e], cs[dt][e + 1]);
                rnd_bf16_pair(sn[dt][e], sn[dt][e + 1]);
            }
        }
        f32x4 y[NDT];
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int pd = dt ^ (NDT / 2);
                const float zp = acc[t][pd][e] * sn[pd][e];
                y[dt][e] = acc[t][dt][e] * cs[dt][e] + ((dt < NDT / 2) ? zp : -zp);
            }
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) acc[t][dt] = y[dt];
        const bf16_t *src = qc_ws + (((int64_t)b * n + ii) * Hq + h) * D + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const bf16x8 qv = ldb8(src + 32 * ks);
            qop[t][ks] = cok[t] ? (FIXED ? scale8(qv, sl2) : qv) : bf16x8{};
        }
    }

    // ------------------------------ sinks and routed blocks (NoPE operand)
    for (int c0 = 0; c0 < ntot; c0 += P) {
        const int issued = min(ntot, c0 + NPRO);
        wait_vm_n(max(0, issued - (c0 + P)) * dpw);
        __syncthreads();
        const int nf = min(ntot, c0 + NPH * P);
        int nxt[P];   // the refill's block ids, read before the first DMA is issued
#pragma unroll
        for (int j = 0; j < P; ++j) nxt[j] = (issued + j < nf) ? sblk(issued + j) : 0;
#pragma unroll
        for (int j = 0; j < P; ++j)
            if (issued + j < nf) fill(nxt[j], (issued + j) % NS, false);
#pragma unroll
        for (int tt = 0; tt < PTW; ++tt) {
            const int rt = w * PTW + tt;
            if (i0 + (int64_t)rt * QPT >= n) break;
            uint32_t hits = __builtin_amdgcn_readfirstlane(bits_at<P>(wbits + rt * nbw, c0 - hs, nbw));
            if (c0 < hs) hits |= 1u;   // the sink block: every row tile
            const uint32_t qw = cok[tt] ? bits_at<P>(qbits + (rt * QPT + qs) * nbw, c0 - hs, nbw) : 0u;
            while (hits) {
                const int j = __builtin_ctz(hits);
                hits &= hits - 1u;
                const int c = c0 + j;
                const bf16_t *Ks = ring + (c % NS) * C::SLOT;
                if (c < hs) {   // keys j < S and j <= i
                    const int64_t jh = (icol[tt] < (int64_t)S - 1) ? icol[tt] : (int64_t)S - 1;
                    dq_update<D, FIXED, DQ_RANGE>(Ks, Ks + C::TILE, Ks + 2 * C::TILE, qop[tt], dop[tt], Dh[tt],
                                                  acc[tt], mrun[tt], lsum[tt], true, 0, cok[tt] ? (int)jh : -1, sl2,
                                                  bl2, l16, lg);
                } else {
                    dq_update<D, FIXED, DQ_COL>(Ks, Ks + C::TILE, Ks + 2 * C::TILE, qop[tt], dop[tt], Dh[tt],
                                                acc[tt], mrun[tt], lsum[tt], (qw >> j) & 1u, 0, 63, sl2, bl2, l16, lg);
                }
            }
        }
    }

    // ------------- LSE, dq = QKNorm backward of scale * acc / l, gain sums
    float gq[PTW];
#pragma unroll
    for (int t = 0; t < PTW; ++t) {
        float l = lsum[t];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float sh = FIXED ? bl2 : mrun[t];
        if (cok[t] && lg == 0)
            lse_ws[((int64_t)b * Hq + h) * n + icol[t]] = (l > 0.0f) ? (sh + __log2f(l)) / LOG2E : INFINITY;
        const float f = (l > 0.0f) ? scale / l : 0.0f;
        const int64_t row = (((int64_t)b * n + (cok[t] ? icol[t] : 0)) * Hq + h) * D;
        float xr[NDT][4], yv[NDT][4];
        float ss = 0.0f, yx = 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const u32x2 u = *reinterpret_cast<const u32x2 *>(q + row + 16 * dt + 4 * lg);
            xr[dt][0] = __uint_as_float(u[0] << 16);
            xr[dt][1] = __uint_as_float(u[0] & 0xffff0000u);
            xr[dt][2] = __uint_as_float(u[1] << 16);
            xr[dt][3] = __uint_as_float(u[1] & 0xffff0000u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                yv[dt][e] = acc[t][dt][e] * f;
                ss = fmaf(xr[dt][e], xr[dt][e], ss);
                yx = fmaf(yv[dt][e], xr[dt][e], yx);
            }
        }
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        yx += __shfl_xor(yx, 16, 64);
        yx += __shfl_xor(yx, 32, 64);
        const float ms = ss / (float)D;
        const float rq = sqrtf(fmaxf(ms, eps));
        if (qgain) {
            const float gn = qgain[h];
            const float corr = (ms >= eps) ? gn * yx / ((float)D * rq * rq * rq) : 0.0f;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int e = 0; e < 4; ++e) yv[dt][e] = (gn / rq) * yv[dt][e] - xr[dt][e] * corr;
        }
        gq[t] = cok[t] ? yx / rq : 0.0f;
        if (cok[t]) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                u32x2 u;
                u[0] = (uint32_t)f2bf(yv[dt][0]) | ((uint32_t)f2bf(yv[dt][1]) << 16);
                u[1] = (uint32_t)f2bf(yv[dt][2]) | ((uint32_t)f2bf(yv[dt][3]) << 16);
                *reinterpret_cast<u32x2 *>(dq + row + 16 * dt + 4 * lg) = u;
            }
        }
    }
    if (qgain && dq_gain) {   // workgroup-uniform: per head over the workgroup's columns, one atomic each
        float *gs = reinterpret_cast<float *>(smem);   // the ring, once every wave is done with it: [WAVES * PTW][16]
        __syncthreads();
#pragma unroll
        for (int t = 0; t < PTW; ++t)
            if (lg == 0) gs[(w * PTW + t) * 16 + l16] = gq[t];
        __syncthreads();
        if (tid < G) {
            float sum = 0.0f;
            for (int r = 0; r < WAVES * PTW; ++r)
                for (int qq = 0; qq < QPT; ++qq) sum += gs[r * 16 + qq * G + tid];
            unsafeAtomicAdd(&dq_gain[g * G + tid], sum);
        }
    }
}

template <int D, int WAVES, int PTW, int NS, int PH>
__global__ __launch_bounds__(WAVES * 64, WAVES / 4) void bwd_dq_union_kernel(
    const bf16_t *__restrict__ q, const float *__restrict__ qgain, const float *__restrict__ kgain, float eps,
    const bf16_t *__restrict__ kc, const bf16_t *__restrict__ kr, const bf16_t *__restrict__ kct,
    const bf16_t *__restrict__ krt, const bf16_t *__restrict__ v, const float *__restrict__ cosT,
    const float *__restrict__ sinT, const int32_t *__restrict__ idx, const int32_t *__restrict__ cnt,
    const bf16_t *__restrict__ out, const bf16_t *__restrict__ dout, int64_t n, int Hq, int Hkv, int S, int W,
    int kk, float scale, int ntiles, int Cn, int xmap, bf16_t *__restrict__ qc_ws, bf16_t *__restrict__ qr_ws,
    float *__restrict__ lse_ws, float *__restrict__ dd_ws, bf16_t *__restrict__ dq, float *__restrict__ dq_gain) {
    extern __shared__ __align__(16) char smem[];
    __shared__ int nlist;
    int combo, tile;
    xcd_map(blockIdx.x, Cn, ntiles, xmap, combo, tile);
    if (tile >= ntiles || combo >= Cn) return;
    const int G = Hq / Hkv;
    const float sl2 = scale * LOG2E;
    float bl2;
    if (group_bound(qgain, kgain, combo % Hkv, G, sl2, D, bl2))
        dq_body<D, WAVES, PTW, NS, PH, true>(q, qgain, eps, kc, kr, kct, krt, v, cosT, sinT, idx, cnt, out, dout, n,
                                             Hq, Hkv, S, W, kk, scale, sl2, bl2, combo, tile, qc_ws, qr_ws, lse_ws,
                                             dd_ws, dq, dq_gain, smem, nlist);
    else
        dq_body<D, WAVES, PTW, NS, PH, false>(q, qgain, eps, kc, kr, kct, krt, v, cosT, sinT, idx, cnt, out, dout,
                                              n, Hq, Hkv, S, W, kk, scale, sl2, bl2, combo, tile, qc_ws, qr_ws,
                                              lse_ws, dd_ws, dq, dq_gain, smem, nlist);
}

// ============================================================ launchers ====
static void grid_map(int64_t Cn, int64_t ntiles, int &xmap, int64_t &grid) {
    if (8 % Cn == 0) {
        xmap = 1;   // 8 workgroups per round, 8/Cn tiles of each combo per round
        grid = 8 * ((ntiles + (8 / Cn) - 1) / (8 / Cn));
    } else if (Cn % 8 == 0) {
        xmap = 2;
        grid = Cn * ntiles;
    } else {
        xmap = 0;
        grid = Cn * ntiles;
    }
}

template <int D, int RT>
static int launch_win(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                      const void *kr, const void *vt, const float *cosT, const float *sinT, int64_t B, int64_t n,
                      int64_t Hq, int64_t Hkv, int64_t S, int64_t W, float scale, void *out, const int64_t *os,
                      float *lse, hipStream_t s) {
    using C = WinCfg<D, RT>;
    const int G = (int)(Hq / Hkv);
    // one head per workgroup, 4 waves over consecutive 16*RT-query ranges:
    // a small ring and <= 168 VGPRs let 2-3 workgroups share a CU, so one
    // workgroup's set-up and tail overlap another's tiles
    const int hsplit = G;
    const int gw = 1;
    const int wsplit = 4;
    const int nthr = 64 * gw * wsplit;
    const int64_t QT = 16 * RT * wsplit;
    const int64_t ntiles = (n + QT - 1) / QT;
    const int64_t Cn = B * Hkv * hsplit;
    const int64_t U = Cn * ntiles;
    const int64_t grid = 8 * ((U + 7) / 8);
    if (grid > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    const size_t lds = (size_t)C::NS * C::SLOT * 2;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&attn_win_kernel<D, RT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return HBA_ERR_LAUNCH;
    const int Wc = (int)((W < n + 1) ? W : n + 1);     // a window longer than the sequence is the sequence
    hipLaunchKernelGGL((attn_win_kernel<D, RT>), dim3((unsigned)grid), dim3(nthr), lds, s, (const bf16_t *)q, qs[0],
                       qs[1], qs[2], qgain, kgain, eps, (const bf16_t *)kr, (const bf16_t *)vt, cosT, sinT, (int)n,
                       (int)Hq, (int)Hkv, (int)S, Wc, scale, gw, hsplit, wsplit, (int)ntiles, (int)Cn,
                       (bf16_t *)out, os[0], os[1], os[2], lse);
    return HBA_OK;
}

template <int D, int PTW>
static size_t routed_lds(int64_t n, int64_t G, int64_t k) {
    using C = RtCfg<D>;
    const int64_t QT = (int64_t)C::WAVES * PTW * (16 / G);
    const int64_t nb = n / 64;
    const int64_t nbw = (nb + 31) / 32;
    return (size_t)C::NS * C::SLOT * 2 + (size_t)((QT * k + 1) & ~1LL) * 2 + (size_t)nbw * 8 +
           (size_t)((nb + 1) & ~1LL) * 2 + (size_t)(QT + C::WAVES * PTW) * nbw * 4 + 16;
}

template <int D, int PTW, bool WIN>
static int launch_routed_t(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                           const void *kc, const void *vt, const int32_t *idx, const int32_t *cnt, int64_t B,
                           int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t k, float scale, void *out,
                           const int64_t *os, const float *lse, const void *kr, const float *cosT,
                           const float *sinT, int64_t W, void *qrw, hipStream_t s) {
    using C = RtCfg<D>;
    const int G = (int)(Hq / Hkv);
    const size_t lds = routed_lds<D, PTW>(n, G, k);
    const int64_t QT = (int64_t)C::WAVES * PTW * (16 / G);
    const int64_t ntiles = (n + QT - 1) / QT;
    int xmap;
    int64_t grid;
    grid_map(B * Hkv, ntiles, xmap, grid);
    if (grid > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    const int Wc = (int)((W < n + 1) ? W : n + 1);     // a window longer than the sequence is the sequence
    auto go = [&](auto kern) -> int {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return HBA_ERR_LAUNCH;
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NTHR), lds, s, (const bf16_t *)q, qs[0], qs[1],
                           qs[2], qgain, kgain, eps, (const bf16_t *)kc, (const bf16_t *)vt, idx, cnt, n, (int)Hq,
                           (int)Hkv, (int)S, (int)k, scale, (int)ntiles, (int)(B * Hkv), xmap, (bf16_t *)out,
                           os[0], os[1], os[2], lse, (const bf16_t *)kr, cosT, sinT, Wc, (bf16_t *)qrw);
        return HBA_OK;
    };
    return (S > 64) ? go(&attn_routed_kernel<D, PTW, true, WIN>) : go(&attn_routed_kernel<D, PTW, false, WIN>);
}

// PTW row tiles per wave when the selection lists fit LDS beside the ring, else one
template <int D, bool WIN>
static int launch_routed(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                         const void *kc, const void *vt, const int32_t *idx, const int32_t *cnt, int64_t B,
                         int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t k, float scale, void *out,
                         const int64_t *os, const float *lse, const void *kr, const float *cosT, const float *sinT,
                         int64_t W, void *qrw, hipStream_t s) {
    constexpr size_t LDS_MAX = 160 * 1024 - 64;   // 64 bytes for the static nlist
    const int64_t G = Hq / Hkv;
    if (routed_lds<D, RtCfg<D>::PTW>(n, G, k) <= LDS_MAX)
        return launch_routed_t<D, RtCfg<D>::PTW, WIN>(q, qs, qgain, kgain, eps, kc, vt, idx, cnt, B, n, Hq, Hkv, S,
                                                       k, scale, out, os, lse, kr, cosT, sinT, W, qrw, s);
    if (RtCfg<D>::PTW > 1 && routed_lds<D, 1>(n, G, k) <= LDS_MAX)
        return launch_routed_t<D, 1, WIN>(q, qs, qgain, kgain, eps, kc, vt, idx, cnt, B, n, Hq, Hkv, S, k, scale,
                                          out, os, lse, kr, cosT, sinT, W, qrw, s);
    return HBA_ERR_UNSUPPORTED;
}

template <int D, int WAVES, int PTW, int NS>
static size_t dq_lds(int64_t n, int64_t G, int64_t k) {
    using C = DqCfg<D, WAVES>;
    const int64_t QT = (int64_t)WAVES * PTW * (16 / G);
    const int64_t nb = n / 64;
    const int64_t nbw = (nb + 31) / 32;
    return (size_t)NS * C::SLOT * 2 + (size_t)((QT * k + 1) & ~1LL) * 2 + (size_t)nbw * 8 +
           (size_t)((nb + 1) & ~1LL) * 2 + (size_t)(QT + WAVES * PTW) * nbw * 4 + 16;
}

template <int D, int WAVES, int PTW, int NS, int PH>
static int launch_dq_t(const void *q, const float *qgain, const float *kgain, float eps, const void *kc,
                       const void *kr, const void *kct, const void *krt, const void *v, const float *cosT,
                       const float *sinT, const int32_t *idx, const int32_t *cnt, const void *out, const void *dout,
                       int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t W, int64_t k, float scale,
                       void *qc_ws, void *qr_ws, float *lse_ws, float *dd_ws, void *dq, float *dq_gain,
                       hipStream_t s) {
    const int64_t G = Hq / Hkv;
    const size_t lds = dq_lds<D, WAVES, PTW, NS>(n, G, k);
    const int64_t QT = (int64_t)WAVES * PTW * (16 / G);
    const int64_t ntiles = (n + QT - 1) / QT;
    int xmap;
    int64_t grid;
    grid_map(B * Hkv, ntiles, xmap, grid);
    if (grid > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    const int Wc = (int)((W < n + 1) ? W : n + 1);     // a window longer than the sequence is the sequence
    auto kern = &bwd_dq_union_kernel<D, WAVES, PTW, NS, PH>;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return HBA_ERR_LAUNCH;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(WAVES * 64), lds, s, (const bf16_t *)q, qgain, kgain, eps,
                       (const bf16_t *)kc, (const bf16_t *)kr, (const bf16_t *)kct, (const bf16_t *)krt,
                       (const bf16_t *)v, cosT, sinT, idx, cnt, (const bf16_t *)out, (const bf16_t *)dout, n,
                       (int)Hq, (int)Hkv, (int)S, Wc, (int)k, scale, (int)ntiles, (int)(B * Hkv), xmap,
                       (bf16_t *)qc_ws, (bf16_t *)qr_ws, lse_ws, dd_ws, (bf16_t *)dq, dq_gain);
    return HBA_OK;
}

}  // namespace ab

template <int D>
int launch_attn_bf16_window(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                            const void *kr, const void *vt, const float *cosT, const float *sinT, int64_t B,
                            int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t W, float scale, void *out,
                            const int64_t *os, float *lse, hipStream_t s) {
    using namespace ab;
    const int G = (int)(Hq / Hkv);
    if (G > 16 || n / 64 >= SENT) return HBA_ERR_UNSUPPORTED;
    constexpr int RT = (D == 64) ? 2 : 1;      // row tiles per wave within 168 VGPRs (3 waves per SIMD)
    return launch_win<D, RT>(q, qs, qgain, kgain, eps, kr, vt, cosT, sinT, B, n, Hq, Hkv, S, W, scale, out, os,
                             lse, s);
}

template <int D>
int launch_attn_bf16_routed(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                            const void *kc, const void *vt, const int32_t *idx, const int32_t *cnt, int64_t B,
                            int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t k, float scale, void *out,
                            const int64_t *os, const float *lse, hipStream_t s) {
    using namespace ab;
    const int G = (int)(Hq / Hkv);
    if (G > 16 || n / 64 >= SENT) return HBA_ERR_UNSUPPORTED;
    return launch_routed<D, false>(q, qs, qgain, kgain, eps, kc, vt, idx, cnt, B, n, Hq, Hkv, S, k, scale, out, os,
                                   lse, nullptr, nullptr, nullptr, 1, nullptr, s);
}

template <int D>
int launch_attn_bf16(const void *q, const int64_t *qs, const float *qgain, const float *kgain, float eps,
                     const void *kc, const void *kr, const void *vt, const float *cosT, const float *sinT,
                     const int32_t *idx, const int32_t *cnt, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                     int64_t S, int64_t W, int64_t k, float scale, void *out, const int64_t *os, void *qrw,
                     hipStream_t s) {
    using namespace ab;
    const int G = (int)(Hq / Hkv);
    if (G > 16 || n / 64 >= SENT) return HBA_ERR_UNSUPPORTED;
    return launch_routed<D, true>(q, qs, qgain, kgain, eps, kc, vt, idx, cnt, B, n, Hq, Hkv, S, k, scale, out, os,
                                  nullptr, kr, cosT, sinT, W, qrw, s);
}

template <int D>
int launch_attn_bf16_dq(const void *q, const float *qgain, const float *kgain, float eps, const void *kc,
                        const void *kr, const void *kct, const void *krt, const void *v, const float *cosT,
                        const float *sinT, const int32_t *idx, const int32_t *cnt, const void *out,
                        const void *dout, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t S, int64_t W,
                        int64_t k, float scale, void *qc_ws, void *qr_ws, float *lse_ws, float *dd_ws, void *dq,
                        float *dq_gain, hipStream_t s) {
    using namespace ab;
    const int64_t G = Hq / Hkv;
    if (D != 64 || G > 16 || S > 64 || n % 64 || n / 64 >= SENT) return HBA_ERR_UNSUPPORTED;
    constexpr size_t LDS_MAX = 160 * 1024 - 64;   // 64 bytes for the static nlist
    // d = 64: 16 waves (4 per SIMD, within 128 VGPRs) of one row tile, 32
    // queries at G = 7; a 6-slot ring (3 blocks per phase) when the selection
    // lists fit beside it, else 4 slots.  Measured at 32K (whole backward):
    // 16 x 1 3.74 ms, 12 waves x 2 tiles 4.11, 8 x 3 4.09 (2 waves per SIMD
    // leave the update's LDS and MFMA latencies exposed); 16 x 1 with 2-block
    // phases 4.00, with a 4-slot ring 3.90
    if (dq_lds<64, 16, 1, 6>(n, G, k) <= LDS_MAX)
        return launch_dq_t<64, 16, 1, 6, 3>(q, qgain, kgain, eps, kc, kr, kct, krt, v, cosT, sinT, idx, cnt, out,
                                           dout, B, n, Hq, Hkv, S, W, k, scale, qc_ws, qr_ws, lse_ws, dd_ws, dq,
                                           dq_gain, s);
    if (dq_lds<64, 16, 1, 4>(n, G, k) <= LDS_MAX)
        return launch_dq_t<64, 16, 1, 4, 2>(q, qgain, kgain, eps, kc, kr, kct, krt, v, cosT, sinT, idx, cnt, out,
                                           dout, B, n, Hq, Hkv, S, W, k, scale, qc_ws, qr_ws, lse_ws, dd_ws, dq,
                                           dq_gain, s);
    return HBA_ERR_UNSUPPORTED;
}
template int launch_attn_bf16_dq<64>(const void *, const float *, const float *, float, const void *, const void *,
                                     const void *, const void *, const void *, const float *, const float *,
                                     const int32_t *, const int32_t *, const void *, const void *, int64_t, int64_t,
                                     int64_t, int64_t, int64_t, int64_t, int64_t, float, void *, void *, float *,
                                     float *, void *, float *, hipStream_t);

#define HBA_INST_WIN(D)                                                                                       \
    template int launch_attn_bf16_window<D>(const void *, const int64_t *, const float *, const float *, float, \
                                            const void *, const void *, const float *, const float *, int64_t,  \
                                            int64_t, int64_t, int64_t, int64_t, int64_t, float, void *,        \
                                            const int64_t *, float *, hipStream_t);                             \
    template int launch_attn_bf16_routed<D>(const void *, const int64_t *, const float *, const float *, float, \
                                            const void *, const void *, const int32_t *, const int32_t *,      \
                                            int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, float,       \
                                            void *, const int64_t *, const float *, hipStream_t);
HBA_INST_WIN(64)
HBA_INST_WIN(128)
#undef HBA_INST_WIN

template int launch_attn_bf16<64>(const void *, const int64_t *, const float *, const float *, float,
                                  const void *, const void *, const void *, const float *, const float *,
                                  const int32_t *, const int32_t *, int64_t, int64_t, int64_t, int64_t, int64_t,
                                  int64_t, int64_t, float, void *, const int64_t *, void *, hipStream_t);
template int launch_attn_bf16<128>(const void *, const int64_t *, const float *, const float *, float,
                                   const void *, const void *, const void *, const float *, const float *,
                                   const int32_t *, const int32_t *, int64_t, int64_t, int64_t, int64_t, int64_t,
                                   int64_t, int64_t, float, void *, const int64_t *, void *, hipStream_t);

}  // namespace hba
