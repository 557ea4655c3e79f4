// Block selection: flat top-k (route_topk, src/hba/attention.py:272-303; eval
// :695-698) and two-level beam descent (hier_select, src/hba/attention.py:217-246).
//
// One thread per (query, KV head); 64 queries per workgroup.  The routing
// query (QKNorm of the G heads, summed) is built in registers in the declared
// order, the block summaries are staged through LDS as fp32 and read as
// broadcasts, and every slot dot product is a sequential fp32 FMA chain over
// d -- the same operation order as the oracle, so scores and the selected
// indices are bit-exact.  The top-k list is a register-resident sorted array
// (score descending, block index ascending).
#include <type_traits>

#include "hba_common.h"
#include "hba_abi.h"
#include "hba_generic.h"
#include "hba_dma.h"

namespace hba {

constexpr int SEL_WG = 64;
constexpr int SEL_LDS_FLOATS = 4096;  // 16 KiB of staged summaries

__device__ __forceinline__ bool better(float v, int id, float w, int iw) {
    return (v > w) || (v == w && id < iw);
}

// Insert (v, id) into a list sorted by (value desc, id asc).  Entries arrive
// in increasing id order, so an equal value never displaces an earlier one.
// Once the new entry has taken a position, every later entry moves down one
// place (an entry displaced from position j precedes, in the order, the
// equal-valued entries after it).
template <int K>
__device__ __forceinline__ void insert_inorder(float (&vals)[K], int (&ids)[K], float v, int id) {
    if (v > vals[K - 1]) {
        bool moving = false;
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const bool sw = moving || v > vals[j];
            moving = sw;
            float tv = sw ? vals[j] : v;
            int ti = sw ? ids[j] : id;
            vals[j] = sw ? v : vals[j];
            ids[j] = sw ? id : ids[j];
            v = tv;
            id = ti;
        }
    }
}

// Same with the full (value desc, id asc) comparator, for out-of-order ids.
template <int K>
__device__ __forceinline__ void insert_any(float (&vals)[K], int (&ids)[K], float v, int id) {
    if (better(v, id, vals[K - 1], ids[K - 1])) {
#pragma unroll
        for (int j = 0; j < K; ++j) {
            bool sw = better(v, id, vals[j], ids[j]);
            float tv = sw ? vals[j] : v;
            int ti = sw ? ids[j] : id;
            vals[j] = sw ? v : vals[j];
            ids[j] = sw ? id : ids[j];
            v = tv;
            id = ti;
        }
    }
}

// Routing query of (b, i, g): QKNorm each of the G heads (declared order),
// sequential fp32 head sum, rounded to the storage dtype (summarizer.py:50-54).
template <int DT, int D>
__device__ __forceinline__ void routing_query(const typename St<DT>::T *q, int64_t qsb, int64_t qsn,
                                              int64_t qsh, const float *qgain, float eps, int64_t b,
                                              int64_t i, int g, int G, float (&qg)[D]) {
    for (int h = 0; h < G; ++h) {
        float x[D];
        const typename St<DT>::T *row = q + b * qsb + i * qsn + (int64_t)(g * G + h) * qsh;
        if constexpr (DT == 1) {
            const uint4 *p = reinterpret_cast<const uint4 *>(row);
#pragma unroll
            for (int c = 0; c < D / 8; ++c) {
                uint4 u = p[c];
                uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[8 * c + 2 * e] = __uint_as_float(w[e] << 16);
                    x[8 * c + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
                }
            }
        } else {
            const float4 *p = reinterpret_cast<const float4 *>(row);
#pragma unroll
            for (int c = 0; c < D / 4; ++c) {
                float4 u = p[c];
                x[4 * c] = u.x;
                x[4 * c + 1] = u.y;
                x[4 * c + 2] = u.z;
                x[4 * c + 3] = u.w;
            }
        }
        if (qgain) qknorm_row<DT, D>(x, qgain[g * G + h], eps);
        if (h == 0) {
#pragma unroll
            for (int t = 0; t < D; ++t) qg[t] = x[t];
        } else {
#pragma unroll
            for (int t = 0; t < D; ++t) qg[t] = qg[t] + x[t];
        }
    }
#pragma unroll
    for (int t = 0; t < D; ++t) qg[t] = St<DT>::rnd(qg[t]);
}

// max over slots of the sequential-FMA dot products, times scale.
template <int D, int M>
__device__ __forceinline__ float slot_score_lds(const float (&qg)[D], const float *S, float scale) {
    float acc[M];
#pragma unroll
    for (int s = 0; s < M; ++s) acc[s] = 0.0f;
#pragma unroll
    for (int t = 0; t < D; t += 4) {
#pragma unroll
        for (int s = 0; s < M; ++s) {
            float4 sv = *reinterpret_cast<const float4 *>(S + s * D + t);
            acc[s] = fmaf(qg[t], sv.x, acc[s]);
            acc[s] = fmaf(qg[t + 1], sv.y, acc[s]);
            acc[s] = fmaf(qg[t + 2], sv.z, acc[s]);
            acc[s] = fmaf(qg[t + 3], sv.w, acc[s]);
        }
    }
    float best = acc[0];
#pragma unroll
    for (int s = 1; s < M; ++s) best = (acc[s] > best) ? acc[s] : best;
    return best * scale;
}

template <int DT, int D, int M>
__device__ __forceinline__ float slot_score_gmem(const float (&qg)[D], const typename St<DT>::T *S,
                                                 float scale) {
    float acc[M];
#pragma unroll
    for (int s = 0; s < M; ++s) acc[s] = 0.0f;
#pragma unroll
    for (int s = 0; s < M; ++s) {
#pragma unroll 4
        for (int t = 0; t < D; ++t) acc[s] = fmaf(qg[t], St<DT>::ld(S, s * D + t), acc[s]);
    }
    float best = acc[0];
#pragma unroll
    for (int s = 1; s < M; ++s) best = (acc[s] > best) ? acc[s] : best;
    return best * scale;
}

// Stage summaries [first, first+cnt) of one (b, g) into LDS as fp32.
template <int DT, int D, int M>
__device__ __forceinline__ void stage_blocks(float *lds, const typename St<DT>::T *S, int64_t first,
                                             int cnt) {
    const int total = cnt * M * D;
    const typename St<DT>::T *src = S + first * M * D;
    for (int e = threadIdx.x; e < total; e += SEL_WG) lds[e] = St<DT>::ld(src, e);
}

template <int DT, int D, int M, int KMAX>
__global__ __launch_bounds__(SEL_WG) void score_select_kernel(
    const typename St<DT>::T *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh,
    const float *__restrict__ qgain, float eps, const typename St<DT>::T *__restrict__ S0, int64_t n,
    int Hq, int Hkv, int64_t nb, int64_t W, int kk, float scale, int32_t *__restrict__ idx,
    float *__restrict__ val, int32_t *__restrict__ cnt, float *__restrict__ scores) {
    constexpr int CB = SEL_LDS_FLOATS / (M * D);
    __shared__ __align__(16) float lds[SEL_LDS_FLOATS];
    const int lane = threadIdx.x;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t i0 = (int64_t)blockIdx.x * SEL_WG;
    const int64_t i = i0 + lane;
    const bool active = i < n;
    float qg[D];
    if (active) routing_query<DT, D>(q, qsb, qsn, qsh, qgain, eps, b, i, g, G, qg);
    const int64_t bmax = active ? cand_bmax(i, 64, W) : 0;
    const int64_t last = (i0 + SEL_WG - 1 < n) ? i0 + SEL_WG - 1 : n - 1;
    const int64_t tile_bmax = cand_bmax(last, 64, W);
    float vals[KMAX];
    int ids[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        vals[j] = -INFINITY;
        ids[j] = -1;
    }
    const typename St<DT>::T *Sg = S0 + (b * Hkv + g) * nb * M * D;
    for (int64_t b0 = 1; b0 <= tile_bmax; b0 += CB) {
        int cb = (int)((tile_bmax - b0 + 1 < CB) ? tile_bmax - b0 + 1 : CB);
        __syncthreads();
        stage_blocks<DT, D, M>(lds, Sg, b0, cb);
        __syncthreads();
        for (int c = 0; c < cb; ++c) {
            int64_t blk = b0 + c;
            if (blk <= bmax) {
                float v = slot_score_lds<D, M>(qg, lds + c * M * D, scale);
                if (scores) scores[((b * Hkv + g) * n + i) * nb + blk] = v;
                insert_inorder<KMAX>(vals, ids, v, (int)blk);
            }
        }
    }
    if (!active) return;
    int64_t o = ((b * Hkv + g) * n + i) * kk;
    int c = 0;
    for (int j = 0; j < kk; ++j) {
        idx[o + j] = ids[j];
        val[o + j] = vals[j];
        c += (vals[j] != -INFINITY) ? 1 : 0;
    }
    cnt[(b * Hkv + g) * n + i] = c;
}


// ----------------------------------------------------- bf16 MFMA scoring ----
typedef unsigned int u32x4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 ldb8(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4s *>(p));
}

// Scores as one bf16 GEMM per (batch, KV head, 64 queries):
// C^T[summary rows x queries] = S0 . qg^T with v_mfma_f32_16x16x32_bf16 (fp32
// accumulation).  A 16-row M tile is 4 blocks x 4 slots, so lane (l16, lg)
// receives the 4 slot scores of block 4*mt + lg for query column l16 and takes
// their max.  The summaries stream through a 3-stage direct-to-LDS ring of
// 16 blocks per stage.  Each lane keeps a top-KMAX of the blocks it sees (in
// ascending block order); the four lane lists of a query are then merged
// under the same order.  The routing query is built in the declared fp32 order
// and is exactly representable in bf16.
namespace sel {
constexpr int CB = 16;       // blocks per stage
constexpr int NSS = 3;       // stages in the ring
// chunk swizzle of stage row r: the 16 rows an A-fragment read touches land in
// distinct 16-byte bank groups
template <int D>
__device__ __forceinline__ int sw(int r) {
    return (D == 64) ? ((r >> 1) & 7) : (r & 15);
}
}  // namespace sel

// Lane l's copy of lane l ^ 16 / l ^ 32 (wave64), from v_permlane16_swap /
// v_permlane32_swap with the same register as both operands: the swap leaves
// the partner row's value in the first result on odd rows (upper half) and in
// the second on even rows (lower half).
__device__ __forceinline__ uint32_t lane_xor16(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t lane_xor32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ float lane_xor(float x, int o) {
    const uint32_t u = __float_as_uint(x);
    return __uint_as_float(o == 16 ? lane_xor16(u) : lane_xor32(u));
}
__device__ __forceinline__ int lane_xor(int x, int o) {
    return (int)(o == 16 ? lane_xor16((uint32_t)x) : lane_xor32((uint32_t)x));
}

// The four sorted lane lists of a query (lanes l16, l16+16, l16+32, l16+48)
// merged under (score desc, id asc) in registers: each step takes the best
// head over the four lanes (their ids are disjoint) and its lane pops it.
// take(j, v, id) runs in all four lanes for each of the best `want`; the
// count taken is returned.  Empty heads are (-inf, -1).
template <int K, class Take>
__device__ __forceinline__ int merge_lanes(float (&v)[K], int (&id)[K], int want, Take &&take) {
    int c = 0;
    for (int j = 0; j < want; ++j) {
        float bv = v[0];
        int bi = id[0];
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            const float ov = lane_xor(bv, o);
            const int oi = lane_xor(bi, o);
            if (oi >= 0 && (bi < 0 || better(ov, oi, bv, bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if (bi < 0) break;   // every list of the query is empty (the same in its four lanes)
        if (id[0] == bi) {
#pragma unroll
            for (int k = 0; k + 1 < K; ++k) {
                v[k] = v[k + 1];
                id[k] = id[k + 1];
            }
            v[K - 1] = -INFINITY;
            id[K - 1] = -1;
        }
        take(j, bv, bi);
        c = j + 1;
    }
    return c;
}

// The bf16 routing queries of the 64 queries i0 .. i0+63 (clamped to n-1)
// of KV head g into qgs[64][ROWQ], in routing_query's operation order.
// Thread (query tid / 4, part tid % 4):
//   1. the QKNorm sum of squares of heads part, part+4, ... (< G) over the
//      whole row: the declared sequential FMA chain; a thread's chains are
//      independent and interleave;
//   2. every head's r = sqrt(max(ss / D, eps)), broadcast within the query's
//      four threads;
//   3. its D/4 dims of every head: x / r (the IEEE quotient, through
//      div_rn_fast where that applies), times the gain, rounded to bf16, and
//      summed in head order.
// Needs 256 threads; G <= 16.
template <int D, int ROWQ>
__device__ __forceinline__ void routing_queries_tile(const bf16_t *q, int64_t qsb, int64_t qsn, int64_t qsh,
                                                     const float *qgain, float eps, int64_t b, int64_t i0,
                                                     int64_t n, int g, int G, bf16_t *qgs, int tid) {
    constexpr int DP = D / 4, NC = DP / 8;   // dims and 16-byte chunks per thread
    constexpr int GMAX = 16;
    const int qq = tid >> 2, part = tid & 3, lane = tid & 63;
    const int64_t i = (i0 + qq < n) ? i0 + qq : n - 1;
    const bf16_t *row0 = q + b * qsb + i * qsn + (int64_t)g * G * qsh;
    auto unpack = [](const uint4 &u, int e) {   // element e (0..7) of 8 packed bf16
        const uint32_t wd = (e >> 1) == 0 ? u.x : (e >> 1) == 1 ? u.y : (e >> 1) == 2 ? u.z : u.w;
        return (e & 1) ? __uint_as_float(wd & 0xffff0000u) : __uint_as_float(wd << 16);
    };
    float rr[GMAX / 4];
#pragma unroll
    for (int j = 0; j < GMAX / 4; ++j) rr[j] = 1.0f;
    auto chains = [&](auto nj_const) {
        constexpr int NJ = decltype(nj_const)::value;
        float ss[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) ss[j] = 0.0f;
        if constexpr (D <= 64) {   // every full row in flight at once
            uint4 rw[NJ][D / 8];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int h = (part + 4 * j < G) ? part + 4 * j : G - 1;   // past G: a duplicate, unused
#pragma unroll
                for (int c = 0; c < D / 8; ++c) rw[j][c] = reinterpret_cast<const uint4 *>(row0 + (int64_t)h * qsh)[c];
            }
#pragma unroll
            for (int t = 0; t < D; ++t)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const float x = unpack(rw[j][t >> 3], t & 7);
                    ss[j] = fmaf(x, x, ss[j]);
                }
        } else {   // one full row at a time: beside the quarter rows, two would not fit the registers
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int h = (part + 4 * j < G) ? part + 4 * j : G - 1;
                uint4 rw[D / 8];
#pragma unroll
                for (int c = 0; c < D / 8; ++c) rw[c] = reinterpret_cast<const uint4 *>(row0 + (int64_t)h * qsh)[c];
#pragma unroll
                for (int t = 0; t < D; ++t) {
                    const float x = unpack(rw[t >> 3], t & 7);
                    ss[j] = fmaf(x, x, ss[j]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            float ms = ss[j] / (float)D;
            if (ms < eps) ms = eps;
            rr[j] = sqrtf(ms);
        }
    };
    const bf16_t *base = row0 + part * DP;
    float acc[DP];
    auto head = [&](int h, const uint4 (&raw)[NC]) {
        float x[DP];
#pragma unroll
        for (int e = 0; e < DP; ++e) x[e] = unpack(raw[e >> 3], e & 7);
        if (qgain) {
            const float r = __shfl(rr[h >> 2], (lane & ~3) | (h & 3), 64);
            const float gn = qgain[g * G + h];
            bool slow = !div_rn_row_ok(r);
#pragma unroll
            for (int e = 0; e < DP; ++e) slow = slow || div_rn_subnormal(x[e]);
            if (!__any(slow)) {
                const float inv = 1.0f / r;
#pragma unroll
                for (int e = 0; e < DP; ++e) x[e] = div_rn_fast(x[e], r, inv) * gn;
#pragma unroll
                for (int e = 0; e < DP; e += 2) rnd_bf16_pair(x[e], x[e + 1]);
            } else {
#pragma unroll
                for (int e = 0; e < DP; ++e) x[e] = rnd_bf16((x[e] / r) * gn);
            }
        }
#pragma unroll
        for (int e = 0; e < DP; ++e) acc[e] = (h == 0) ? x[e] : acc[e] + x[e];
    };
    if (G <= 8) {
        // every load first: the quarter rows of all heads (past G: head G-1
        // again, unused), then the full rows of the sums of squares
        uint4 rq[8][NC];
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const int hc = h < G ? h : G - 1;
#pragma unroll
            for (int c = 0; c < NC; ++c) rq[h][c] = reinterpret_cast<const uint4 *>(base + (int64_t)hc * qsh)[c];
        }
        if (qgain) chains(std::integral_constant<int, 2>());
#pragma unroll
        for (int h = 0; h < 8; ++h)
            if (h < G) head(h, rq[h]);
    } else {
        if (qgain) chains(std::integral_constant<int, 4>());
#pragma unroll
        for (int h = 0; h < GMAX; ++h) {
            if (h >= G) break;   // uniform
            uint4 raw[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) raw[c] = reinterpret_cast<const uint4 *>(base + (int64_t)h * qsh)[c];
            head(h, raw);
        }
    }
#pragma unroll
    for (int e = 0; e < DP; e += 2)
        *reinterpret_cast<uint32_t *>(qgs + qq * ROWQ + part * DP + e) = pk_bf16(acc[e], acc[e + 1]);
}

// HIER: the two-level beam descent (hier_select) on the same machinery.  A
// scan over the super-summaries S1 keeps, per query, the top-min(beam, ns)
// supers holding a candidate child (score desc, super asc); the block scan
// then inserts only children of those supers.  On a GPU tile of 64 queries
// the kept supers cover nearly every super, so the children are scored as the
// flat GEMM and filtered, not gathered.
// (score, block) as one unsigned key ordered like (score desc, block asc):
// the score's bits mapped to an order-preserving unsigned (a zero score
// taken as +0, which the float comparison treats as equal to -0), then the
// complement of the block.
__device__ __forceinline__ uint64_t sel_key(float v, int blk) {
    const uint32_t u = __float_as_uint(v + 0.0f);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)blk);
}
__device__ __forceinline__ float sel_key_score(uint64_t key) {
    const uint32_t ord = (uint32_t)(key >> 32);
    return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}
__device__ __forceinline__ int sel_key_block(uint64_t key) { return (int)(0xffffffffu - (uint32_t)key); }

// Position of the r-th (0-based) set bit of m; m must hold more than r.
__device__ __forceinline__ int nth_set_bit64(uint64_t m, int r) {
    int pos = 0;
#pragma unroll
    for (int wdt = 32; wdt >= 1; wdt >>= 1) {
        const uint64_t low = m & ((1ull << wdt) - 1ull);
        const int c = __popcll(low);
        if (r >= c) {
            r -= c;
            m >>= wdt;
            pos += wdt;
        } else {
            m = low;
        }
    }
    return pos;
}

// Orders one wave's LDS writes before its later reads of them (other lanes'
// included): LDS operations of a wave are performed in issue order, so only
// the compiler needs holding back.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int o) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, o, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), o, 64);
    return ((uint64_t)hi << 32) | lo;
}

// Workgroup -> (64-query tile, KV head, batch) of a 1-D grid, the deepest
// tiles first: a tile's work grows with its candidate count, and starting the
// longest workgroups first leaves the short ones to fill the end (longest-
// first list scheduling).  The KV heads and batches of one depth are adjacent.
__device__ __forceinline__ void sel_deep_first(int ntiles, int Hkv, int &tile, int &g, int64_t &b) {
    const int64_t i = blockIdx.x;
    const int64_t per = (int64_t)Hkv * (gridDim.x / ((int64_t)ntiles * Hkv));   // Hkv * B
    const int64_t j = i / per, r = i % per;
    tile = ntiles - 1 - (int)j;
    g = (int)(r % Hkv);
    b = r / Hkv;
}

constexpr int SEL_PMW = 64;   // most words of the per-query super bitmask: ns <= 2048
constexpr int32_t SEL_OVERFLOW = -2;   // cnt marker: the threshold kernel left this query to the exact pass
constexpr int SEL_GMAXE = 256;   // gather path: most child positions per query (beam * F)
constexpr int SEL_GCAP = 64;     // gather path: most children at or above the threshold per query
// Dynamic LDS of the HIER kernel: the parent bitmask [64][nwp] (nwp = nw | 1,
// an odd row stride: the per-super ballot reads one word of every query
// without bank conflicts); for the gather path also the kept supers' prefix
// counts [64][nwp] (bytes), the kept supers ascending [64][16] and the
// children's scores [64][beam * F].
__host__ __device__ inline int sel_nwp(int64_t ns) { return (int)(((ns + 31) / 32) | 1); }
__host__ __device__ inline size_t sel_pre_off(int nwp) { return (size_t)64 * nwp * 4; }
__host__ __device__ inline size_t sel_ksup_off(int nwp) { return (sel_pre_off(nwp) + (size_t)64 * nwp + 15) & ~(size_t)15; }
__host__ __device__ inline size_t sel_cs_off(int nwp) { return sel_ksup_off(nwp) + (size_t)64 * 16 * 2; }
// marked_only: run only for a 64-query tile holding a query whose cnt is
// SEL_OVERFLOW (the threshold kernel's overflow), and recompute the tile.
// gather (HIER): 0 the block scan filtered by parent; 1 level 2 by super in
// this kernel; 2 level 1 only: each query's kept supers (ascending, -1 past
// them) into ks_out [B, Hkv, n, 16] and its routing query into rq_out
// [B, Hkv, n, D], for hier_l2_kernel.  L1 (with HIER and gather 2): an
// instantiation holding only that level-1 code, whose registers let three
// workgroups share a CU.
template <int D, int KMAX, bool HIER, int BEAMMAX = 16, bool L1 = false>
__global__ __launch_bounds__(256, L1 ? 3 : ((D == 64) ? 2 : 1)) void score_select_mfma_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const bf16_t *__restrict__ S0, int64_t n, int Hq, int Hkv, int64_t nb, int64_t W, int kk,
    float scale, int32_t *__restrict__ idx, float *__restrict__ val, int32_t *__restrict__ cnt,
    float *__restrict__ scores, const bf16_t *__restrict__ S1, int F, int beam, float *__restrict__ sup_scores,
    int marked_only, int gather, bf16_t *__restrict__ rq_out, int16_t *__restrict__ ks_out) {
    int tile_, g_;
    int64_t b_;
    sel_deep_first((int)((n + 63) / 64), Hkv, tile_, g_, b_);
    if (marked_only) {
        __shared__ int marked;
        const int64_t ib = (int64_t)tile_ * 64 + threadIdx.x;
        if (threadIdx.x == 0) marked = 0;
        __syncthreads();
        if (threadIdx.x < 64 && ib < n && cnt[(b_ * Hkv + g_) * n + ib] == SEL_OVERFLOW) marked = 1;
        __syncthreads();
        if (!marked) return;   // workgroup-uniform
    }
    using namespace sel;
    constexpr int NKS = D / 32;
    constexpr int CPR = D / 8;                         // 16-byte chunks per summary row
    constexpr int ROWQ = D + 8;                        // padded LDS row of the routing queries
    constexpr int SROWS = CB * 4;                      // rows per stage
    constexpr int PPW = SROWS * D * 2 / 1024 / 4;      // 1 KB DMA parts per wave per stage
    // LDS: the routing queries; the stage ring
    constexpr int RING_BYTES = NSS * SROWS * D * 2;
    __shared__ __align__(16) bf16_t qgs[64 * ROWQ];
    __shared__ __align__(16) char pool[RING_BYTES];
    extern __shared__ uint32_t pmask[];                // HIER: [64][ceil(ns / 32)], sized at launch
    bf16_t *ring = reinterpret_cast<bf16_t *>(pool);

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int g = g_;
    const int64_t b = b_;
    const int G = Hq / Hkv;
    const int64_t i0 = (int64_t)tile_ * 64;
    routing_queries_tile<D, ROWQ>(q, qsb, qsn, qsh, qgain, eps, b, i0, n, g, G, qgs, tid);
    __syncthreads();
    const int qcol = 16 * w + l16;
    const int64_t iq = i0 + qcol;
    bf16x8 qb[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qb[ks] = ldb8(qgs + qcol * ROWQ + 32 * ks + 8 * lg);
    const int64_t bmax = (iq < n) ? cand_bmax(iq, 64, W) : 0;
    const int64_t last = (i0 + 63 < n) ? i0 + 63 : n - 1;
    const int64_t tile_bmax = cand_bmax(last, 64, W);
    const uint32_t ring_lds = lds_offset(ring);

    // Stream rows [first, first + count) of a [*, 4, D] summary array through
    // the ring; visit(row index, slot-max score) per lane for each.
    auto scan = [&](const bf16_t *Src, int64_t first, int64_t count, auto &&visit, auto &&refresh) {
        const int nst = (count > 0) ? (int)((count + CB - 1) / CB) : 0;
        const int64_t lastr = first + count - 1;
        auto fill = [&](int st) {
            const uint32_t slot = ring_lds + (uint32_t)((st % NSS) * SROWS * D * 2);
#pragma unroll
            for (int pp = 0; pp < PPW; ++pp) {
                const int part = w * PPW + pp;
                const int p = part * 64 + lane;          // physical chunk index in the stage
                const int r = p / CPR, c = (p % CPR) ^ sw<D>(r & 15);
                int64_t blk = first + (int64_t)st * CB + r / 4;
                blk = (blk <= lastr) ? blk : lastr;      // rows past the end: never visited
                dma16(Src + (blk * 4 + (r & 3)) * D + 8 * c, slot + (uint32_t)part * 1024u);
            }
        };
        for (int st = 0; st < NSS - 1 && st < nst; ++st) fill(st);
        for (int st = 0; st < nst; ++st) {
            const int ahead = (nst - 1 - st < NSS - 2) ? nst - 1 - st : NSS - 2;
            wait_vm_n(ahead * PPW);
            __syncthreads();   // stage st landed everywhere; stage st-1 is consumed
            if (st + NSS - 1 < nst) fill(st + NSS - 1);
            const bf16_t *Ss = ring + (st % NSS) * SROWS * D;
            const int64_t b0 = first + (int64_t)st * CB;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int r = mt * 16 + l16;
                const bf16_t *ar = Ss + r * D;
                f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ldb8(ar + 8 * ((4 * ks + lg) ^ sw<D>(r & 15))),
                                                                 qb[ks], acc, 0, 0, 0);
                const int64_t blk = b0 + 4 * mt + lg;
                float best = acc[0];
                best = (acc[1] > best) ? acc[1] : best;
                best = (acc[2] > best) ? acc[2] : best;
                best = (acc[3] > best) ? acc[3] : best;
                if (blk <= lastr) visit((int)blk, best * scale);
            }
            refresh();
        }
        __syncthreads();   // the ring is free again
    };
    // Max over a query's four lanes of their lists' last entries: every
    // lane of the query holds LEN entries >= it, so the query's final picks
    // are all >= it and a lower score can be skipped without changing them.
    auto qfloor = [&](float last) {
        last = fmaxf(last, lane_xor(last, 16));
        return fmaxf(last, lane_xor(last, 32));
    };
    const int nw = HIER ? sel_nwp((nb + F - 1) / F) : 0;   // row stride of pmask
    int kout = kk;
    if constexpr (HIER) {
        // ---- level 1: supers holding at least one candidate child
        const int64_t ns = (nb + F - 1) / F;
        const int beff = (int)((beam < ns) ? beam : ns);
        kout = (kk < beff * F) ? kk : beff * F;
        const int64_t nsup = (tile_bmax >= 1) ? tile_bmax / F + 1 : 0;   // supers any query of the tile may keep
        float pv[BEAMMAX];
        int pid[BEAMMAX];
#pragma unroll
        for (int j = 0; j < BEAMMAX; ++j) {
            pv[j] = -INFINITY;
            pid[j] = -1;
        }
        const bf16_t *S1g = S1 + (b * Hkv + g) * ns * 4 * D;
        float pfloor = -INFINITY;
        scan(S1g, 0, nsup, [&](int p, float v) {
            const int64_t lo = (int64_t)p * F;
            const int64_t hi = (lo + F - 1 < nb - 1) ? lo + F - 1 : nb - 1;
            if (bmax >= 1 && lo <= bmax && hi >= 1) {
                if (sup_scores) sup_scores[((b * Hkv + g) * n + iq) * ns + p] = v;
                if (v >= pfloor) insert_inorder<BEAMMAX>(pv, pid, v, p);
            }
        }, [&]() { pfloor = qfloor(pv[BEAMMAX - 1]); });
        for (int e = tid; e < 64 * nw; e += 256) pmask[e] = 0u;
        __syncthreads();
        merge_lanes<BEAMMAX>(pv, pid, beff, [&](int, float, int p) {
            if (lg == 0) pmask[qcol * nw + (p >> 5)] |= 1u << (p & 31);
        });
        __syncthreads();
        if (L1 || gather == 2) {
            // ---- level 1 only: the kept supers ascending and the routing query
            const int nwu = (int)((ns + 31) / 32);
            if (tid < 64 && i0 + tid < n) {
                int16_t *dst = ks_out + ((b * Hkv + g) * n + i0 + tid) * 16;
                int c = 0;
                for (int wd = 0; wd < nwu && c < 16; ++wd) {
                    uint32_t msk = pmask[tid * nw + wd];
                    while (msk && c < 16) {
                        dst[c++] = (int16_t)(wd * 32 + __ffs(msk) - 1);
                        msk &= msk - 1u;
                    }
                }
                for (; c < 16; ++c) dst[c] = -1;
            }
            for (int e = tid; e < 64 * (D / 8); e += 256) {   // 16-byte chunks of the 64 rows
                const int qq = e / (D / 8), c = e % (D / 8);
                if (i0 + qq < n)
                    *reinterpret_cast<u32x4s *>(rq_out + ((b * Hkv + g) * n + i0 + qq) * D + 8 * c) =
                        *reinterpret_cast<const u32x4s *>(qgs + qq * ROWQ + 8 * c);
            }
            return;
        }
        if (gather) {
            // ---- level 2 by super (F = 4, 8 or 16; beff * F <= SEL_GMAXE):
            // each kept super's F children are scored against only the
            // queries of the tile that kept it, 16 to an MFMA column group,
            // with the operands and order of the flat scan (the same scores).
            // Child c of the query's r-th kept super (ascending) has list
            // position r * F + c; a position no child fills stays -inf.
            const int E = beff * F;
            const int NMT = F / 4;
            uint8_t *pre = reinterpret_cast<uint8_t *>(reinterpret_cast<char *>(pmask) + sel_pre_off(nw));
            uint16_t *ksup = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(pmask) + sel_ksup_off(nw));
            float *cs = reinterpret_cast<float *>(reinterpret_cast<char *>(pmask) + sel_cs_off(nw));
            const int nwu = (int)((ns + 31) / 32);        // words in use
            for (int e = tid; e < 64 * E; e += 256) cs[e] = -INFINITY;
            if (tid < 64) {   // per query: kept supers before each word, and the kept supers ascending
                int c = 0;
                for (int wd = 0; wd < nwu; ++wd) {
                    pre[tid * nw + wd] = (uint8_t)c;
                    uint32_t m = pmask[tid * nw + wd];
                    while (m) {
                        const int bit = __ffs(m) - 1;
                        if (c < 16) ksup[tid * 16 + c] = (uint16_t)(wd * 32 + bit);
                        ++c;
                        m &= m - 1u;
                    }
                }
            }
            __syncthreads();
            const bf16_t *Sg = S0 + (b * Hkv + g) * nb * 4 * D;
            auto loadA = [&](int64_t sp, bf16x8 (&af)[4][NKS]) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    if (mt >= NMT) break;   // uniform
                    int64_t blk = sp * F + 4 * mt + (l16 >> 2);
                    blk = (blk < nb) ? blk : nb - 1;   // rows past the last block: never stored
                    const bf16_t *src = Sg + (blk * 4 + (l16 & 3)) * D + 8 * lg;
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) af[mt][ks] = ldb8(src + 32 * ks);
                }
            };
            auto unit = [&](int64_t sp, const bf16x8 (&af)[4][NKS]) {
                const int wd = (int)(sp >> 5);
                const uint32_t bit = 1u << (sp & 31);
                const uint64_t qm = __ballot((pmask[lane * nw + wd] & bit) != 0u);   // lane = query
                const int nq = __popcll(qm);
                for (int j0 = 0; j0 < nq; j0 += 16) {
                    const int r = j0 + l16;
                    const bool cv = r < nq;
                    const int qc = cv ? nth_set_bit64(qm, r) : 0;
                    bf16x8 qv[NKS];
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) qv[ks] = ldb8(qgs + qc * ROWQ + 32 * ks + 8 * lg);
                    f32x4 acc[4];
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        if (mt >= NMT) break;
                        acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int ks = 0; ks < NKS; ++ks)
                            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][ks], qv[ks], acc[mt], 0, 0, 0);
                    }
                    const int rk = pre[qc * nw + wd] + __popc(pmask[qc * nw + wd] & (bit - 1u));
                    const int64_t qi = i0 + qc;
                    const int64_t bm = (qi < n) ? cand_bmax(qi, 64, W) : 0;
                    float *dst = cs + qc * E + rk * F;
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) {
                        if (mt >= NMT) break;
                        const int ch = 4 * mt + lg;
                        const int64_t blk = sp * F + ch;
                        float best = acc[mt][0];
                        best = (acc[mt][1] > best) ? acc[mt][1] : best;
                        best = (acc[mt][2] > best) ? acc[mt][2] : best;
                        best = (acc[mt][3] > best) ? acc[mt][3] : best;
                        const float v = best * scale;
                        const bool ok = cv && blk >= 1 && blk <= bm;
                        if (cv) dst[ch] = ok ? v : -INFINITY;
                        if (ok && scores) scores[((b * Hkv + g) * n + qi) * nb + blk] = v;
                    }
                }
            };
            // Two supers at a time, so that the two dependent chains (ballot,
            // column queries, operand loads, MFMAs, stores) overlap; the
            // general unit where either has more than 16 queries.
            auto pair = [&](int64_t sa, const bf16x8 (&fa)[4][NKS], int64_t sb, const bf16x8 (&fb)[4][NKS]) {
                if (sb >= nsup) {
                    unit(sa, fa);
                    return;
                }
                const int wa = (int)(sa >> 5), wb = (int)(sb >> 5);
                const uint32_t ba = 1u << (sa & 31), bb = 1u << (sb & 31);
                const uint32_t ma = pmask[lane * nw + wa], mb = pmask[lane * nw + wb];
                const uint64_t qa = __ballot((ma & ba) != 0u), qb2 = __ballot((mb & bb) != 0u);
                const int na = __popcll(qa), nb2 = __popcll(qb2);
                if (na > 16 || nb2 > 16) {   // uniform
                    unit(sa, fa);
                    unit(sb, fb);
                    return;
                }
                const bool ca = l16 < na, cb = l16 < nb2;
                const int qca = ca ? nth_set_bit64(qa, l16) : 0;
                const int qcb = cb ? nth_set_bit64(qb2, l16) : 0;
                bf16x8 va[NKS], vb[NKS];
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) {
                    va[ks] = ldb8(qgs + qca * ROWQ + 32 * ks + 8 * lg);
                    vb[ks] = ldb8(qgs + qcb * ROWQ + 32 * ks + 8 * lg);
                }
                const int rka = pre[qca * nw + wa] + __popc(pmask[qca * nw + wa] & (ba - 1u));
                const int rkb = pre[qcb * nw + wb] + __popc(pmask[qcb * nw + wb] & (bb - 1u));
                f32x4 xa[4], xb[4];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    if (mt >= NMT) break;
                    xa[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    xb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) {
                        xa[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[mt][ks], va[ks], xa[mt], 0, 0, 0);
                        xb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[mt][ks], vb[ks], xb[mt], 0, 0, 0);
                    }
                }
                const int64_t qia = i0 + qca, qib = i0 + qcb;
                const int64_t bma = (qia < n) ? cand_bmax(qia, 64, W) : 0;
                const int64_t bmb = (qib < n) ? cand_bmax(qib, 64, W) : 0;
                float *da = cs + qca * E + rka * F;
                float *db = cs + qcb * E + rkb * F;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    if (mt >= NMT) break;
                    const int ch = 4 * mt + lg;
                    const int64_t blka = sa * F + ch, blkb = sb * F + ch;
                    float ma4 = xa[mt][0], mb4 = xb[mt][0];   // as in unit: the same result, zeros included
#pragma unroll
                    for (int e = 1; e < 4; ++e) {
                        ma4 = (xa[mt][e] > ma4) ? xa[mt][e] : ma4;
                        mb4 = (xb[mt][e] > mb4) ? xb[mt][e] : mb4;
                    }
                    const float va4 = ma4 * scale, vb4 = mb4 * scale;
                    const bool oka = ca && blka >= 1 && blka <= bma;
                    const bool okb = cb && blkb >= 1 && blkb <= bmb;
                    if (ca) da[ch] = oka ? va4 : -INFINITY;
                    if (cb) db[ch] = okb ? vb4 : -INFINITY;
                    if (scores) {
                        if (oka) scores[((b * Hkv + g) * n + qia) * nb + blka] = va4;
                        if (okb) scores[((b * Hkv + g) * n + qib) * nb + blkb] = vb4;
                    }
                }
            };
            {   // this wave's supers w, w + 4, ... in pairs, their A fragments one pair ahead
                bf16x8 a0[4][NKS], a1[4][NKS], a2[4][NKS], a3[4][NKS];
                int64_t sp = w;
                if (sp < nsup) loadA(sp, a0);
                if (sp + 4 < nsup) loadA(sp + 4, a1);
                if (sp + 8 < nsup) loadA(sp + 8, a2);
                if (sp + 12 < nsup) loadA(sp + 12, a3);
                while (sp < nsup) {
                    pair(sp, a0, sp + 4, a1);
                    if (sp + 16 < nsup) loadA(sp + 16, a0);
                    if (sp + 20 < nsup) loadA(sp + 20, a1);
                    sp += 8;
                    if (sp >= nsup) break;
                    pair(sp, a2, sp + 4, a3);
                    if (sp + 16 < nsup) loadA(sp + 16, a2);
                    if (sp + 20 < nsup) loadA(sp + 20, a3);
                    sp += 8;
                }
            }
            __syncthreads();
            // ---- per query, 16 lanes: the kout best listed children.  Each
            // lane keeps its 2 best keys; the kout-th best key tau of the 32 is
            // a lower bound of the query's kout-th (or 0: every valid key
            // qualifies); the keys >= tau are listed and ranked by count.
            // the wave's own LDS (no other wave touches it: wave-level syncs)
            uint64_t *tk = reinterpret_cast<uint64_t *>(pool) + w * (4 * 32 + 4 * SEL_GCAP);
            uint64_t *lst = tk + 4 * 32;
            const int qq = lane >> 4, sl = lane & 15;
            constexpr int EL = SEL_GMAXE / 16;   // positions per lane
            const int j0 = sl / F, jstep = 16 / F, ch0 = sl % F;
            for (int r4 = 0; r4 < 4; ++r4) {
                const int qc = 16 * w + 4 * r4 + qq;
                const int64_t qi = i0 + qc;
                const float *cq = cs + qc * E;
                const uint16_t *kq = ksup + qc * 16;
                // this lane's keys: positions sl + 16 t, child sl % F of the
                // query's (sl / F + t * 16 / F)-th kept super (0 where no child)
                float cv[EL];
                int kb[EL];
#pragma unroll
                for (int t = 0; t < EL; ++t) {
                    const int p = sl + 16 * t;
                    const int jr = j0 + t * jstep;
                    cv[t] = (p < E) ? cq[p] : -INFINITY;
                    kb[t] = kq[jr < 16 ? jr : 15];
                }
                uint64_t ky[EL];
#pragma unroll
                for (int t = 0; t < EL; ++t) ky[t] = (cv[t] == -INFINITY) ? 0ull : sel_key(cv[t], kb[t] * F + ch0);
                uint64_t t0 = 0ull, t1 = 0ull;
#pragma unroll
                for (int t = 0; t < EL; ++t) {
                    const uint64_t key = ky[t];
                    t1 = (key > t0) ? t0 : ((key > t1) ? key : t1);
                    t0 = (key > t0) ? key : t0;
                }
                tk[qq * 32 + 2 * sl] = t0;
                tk[qq * 32 + 2 * sl + 1] = t1;
                wave_lds_sync();
                int g0 = 0, g1 = 0;
                for (int j = 0; j < 32; ++j) {
                    const uint64_t x = tk[qq * 32 + j];
                    g0 += (x > t0) ? 1 : 0;
                    g1 += (x > t1) ? 1 : 0;
                }
                uint64_t tau = ~0ull;
                if (g0 < kout) tau = t0;
                if (g1 < kout && t1 < tau) tau = t1;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    const uint64_t ot = shfl_xor_u64(tau, o);
                    tau = (ot < tau) ? ot : tau;
                }
                int mine = 0;
#pragma unroll
                for (int t = 0; t < EL; ++t) mine += (ky[t] != 0ull && ky[t] >= tau) ? 1 : 0;
                int incl = mine;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    const int t = __shfl_up(incl, o, 16);
                    if (sl >= o) incl += t;
                }
                const int total = __shfl(incl, 15, 16);
                if (total <= SEL_GCAP) {
                    int pos = incl - mine;
#pragma unroll
                    for (int t = 0; t < EL; ++t)
                        if (ky[t] != 0ull && ky[t] >= tau) lst[qq * SEL_GCAP + pos++] = ky[t];
                }
                wave_lds_sync();
                if (qi < n) {
                    const int64_t o = ((b * Hkv + g) * n + qi) * kk;
                    if (total > SEL_GCAP) {   // too many ties at tau: the exact pass recomputes the tile
                        if (sl == 0) cnt[(b * Hkv + g) * n + qi] = SEL_OVERFLOW;
                    } else {
                        const uint64_t *lq = lst + qq * SEL_GCAP;
                        for (int j = sl; j < total; j += 16) {
                            const uint64_t key = lq[j];
                            int rank = 0;
#pragma unroll 8
                            for (int j2 = 0; j2 < total; ++j2) rank += (lq[j2] > key) ? 1 : 0;
                            if (rank < kout) {
                                idx[o + rank] = sel_key_block(key);
                                val[o + rank] = sel_key_score(key);
                            }
                        }
                        const int taken = (total < kout) ? total : kout;
                        for (int j = taken + sl; j < kk; j += 16) {
                            idx[o + j] = -1;
                            val[o + j] = -INFINITY;
                        }
                        if (sl == 0) cnt[(b * Hkv + g) * n + qi] = taken;
                    }
                }
                wave_lds_sync();   // tk and lst are reused by the next four queries
            }
            return;
        }
    }
    // ---- blocks (children of the kept supers, for HIER)
    float vals[KMAX];
    int ids[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        vals[j] = -INFINITY;
        ids[j] = -1;
    }
    const bf16_t *Sg = S0 + (b * Hkv + g) * nb * 4 * D;
    float floor_ = -INFINITY;
    scan(Sg, 1, tile_bmax, [&](int blk, float v) {
        bool ok = blk <= bmax;
        if constexpr (HIER) {
            const int p = blk / F;
            ok = ok && ((pmask[qcol * nw + (p >> 5)] >> (p & 31)) & 1u);
        }
        if (ok) {
            if (scores) scores[((b * Hkv + g) * n + iq) * nb + blk] = v;
            if (v >= floor_) insert_inorder<KMAX>(vals, ids, v, blk);
        }
    }, [&]() { floor_ = qfloor(vals[KMAX - 1]); });
    // the query's picks, element j stored by lane group j % 4
    const int64_t o = ((b * Hkv + g) * n + iq) * kk;
    const bool live = iq < n;
    const int c = merge_lanes<KMAX>(vals, ids, kout, [&](int j, float v, int id) {
        if (live && (j & 3) == lg) {
            idx[o + j] = id;
            val[o + j] = v;
        }
    });
    if (live) {
        for (int j = c + ((lg - c) & 3); j < kk; j += 4) {
            idx[o + j] = -1;
            val[o + j] = -INFINITY;
        }
        if (lg == 0) cnt[(b * Hkv + g) * n + iq] = c;
    }
}

// ------------------------------------- bf16 level 2 over query groups ----
// Level 2 of the two-level descent for a group of QG queries (a multiple of
// 64) of one KV head, after score_select_mfma_kernel (gather 2) wrote each
// query's kept supers ks (ascending) and routing query rq.  The group's
// (query, kept super) pairs are bucketed by super in LDS; each super's F
// children are loaded once, as the A operand of the flat scan's MFMA tile,
// and scored against 16 of its queries per tile: the flat scan's operands and
// order, so its fp32 scores bit for bit.  Child c of a query's r-th kept
// super goes to its list position r*F + c in LDS (positions no child fills
// stay -inf); the kout best positions of each query are then ranked as in
// score_select_mfma_kernel's level 2 (threshold, list, rank by count), and a
// query whose list overflows is marked for the exact pass.  Against a 64-query
// tile, a group of a few hundred queries loads each super's children once for
// ~QG*beam/ns queries instead of ~64*beam/ns.
namespace hl2 {
constexpr int NT = 1024;   // 16 waves: the latency-bound phases overlap across waves
constexpr int NW = NT / 64;
constexpr int KSW = 16;   // kept-super slots per query in ks
constexpr int TKW = 4 * 32 + 4 * SEL_GCAP;   // top-k scratch per wave (8-byte keys)
// LDS layout: cs [QG][E] f32 | ksl [QG][16] i16 | lists [QG*beff] u16 |
// cntS, offS [nsp] i32 | one region holding the group's routing queries
// [QG][D + 8] bf16 (padded rows: a tile's 16 rows fall in distinct banks)
// while the supers are scored, then the top-k scratch [NW][TKW] u64
__host__ __device__ inline size_t off_ksl(int QG, int E) { return (size_t)QG * E * 4; }
__host__ __device__ inline size_t off_list(int QG, int E) { return off_ksl(QG, E) + (size_t)QG * KSW * 2; }
__host__ __device__ inline size_t off_cnt(int QG, int E, int beff) {
    return (off_list(QG, E) + (size_t)QG * beff * 2 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t off_tk(int QG, int E, int beff, int nsp) {
    return (off_cnt(QG, E, beff) + (size_t)nsp * 8 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t region(int QG, int D) {
    const size_t rq = (size_t)QG * (D + 8) * 2, tk = (size_t)NW * TKW * 8;
    return rq > tk ? rq : tk;
}
__host__ __device__ inline size_t bytes(int QG, int E, int beff, int nsp, int D) {
    return off_tk(QG, E, beff, nsp) + region(QG, D) + 16;
}
}  // namespace hl2

// EL: list positions per ranking lane (16 lanes per query), at least
// beff * F / 16: 4 at beam * fanout <= 64 (beam 4 of fanout 16), 8 at <= 128
// (the 128K geometry), else 16.
template <int D, int EL>
__global__ __launch_bounds__(hl2::NT) void hier_l2_kernel(
    const bf16_t *__restrict__ S0, const bf16_t *__restrict__ rq, const int16_t *__restrict__ ks, int64_t n,
    int Hkv, int64_t nb, int64_t W, int kk, int F, int beff, int QG, int ngroups, float scale,
    int32_t *__restrict__ idx, float *__restrict__ val, int32_t *__restrict__ cnt, float *__restrict__ scores) {
    using namespace hl2;
    constexpr int NKS = D / 32;
    extern __shared__ __align__(16) char hsm[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    // workgroup -> (group, KV head, batch), the deepest groups first
    const int64_t per = (int64_t)gridDim.x / ngroups;   // Hkv * B
    const int group = ngroups - 1 - (int)(blockIdx.x / per);
    const int g = (int)((blockIdx.x % per) % Hkv);
    const int64_t b = (blockIdx.x % per) / Hkv;
    const int64_t q0 = (int64_t)group * QG;
    const int nq = (int)((n - q0 < QG) ? n - q0 : QG);
    const int E = beff * F;
    const int kout = (kk < E) ? kk : E;
    const int64_t bh = b * Hkv + g;
    const int64_t last_bm = cand_bmax(q0 + nq - 1, 64, W);
    const int nsp = (last_bm >= 1) ? (int)(last_bm / F) + 1 : 0;   // supers a query of the group can keep
    float *cs = reinterpret_cast<float *>(hsm);
    int16_t *ksl = reinterpret_cast<int16_t *>(hsm + off_ksl(QG, E));
    uint16_t *lists = reinterpret_cast<uint16_t *>(hsm + off_list(QG, E));
    int *cntS = reinterpret_cast<int *>(hsm + off_cnt(QG, E, beff));
    int *offS = cntS + nsp;
    uint64_t *tkall = reinterpret_cast<uint64_t *>(hsm + off_tk(QG, E, beff, nsp));
    constexpr int RQS = D + 8;   // padded row of the routing queries in LDS
    bf16_t *rqs = reinterpret_cast<bf16_t *>(tkall);   // the same region, before the top-k

    // ---- the group's kept supers, the scores' -inf, zero counts
    for (int e = tid; e < QG * 2; e += NT) {   // 2 x 16 bytes per query
        const int qq = e >> 1;
        u32x4s v = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu};   // -1 pairs past the group
        if (qq < nq) v = *reinterpret_cast<const u32x4s *>(ks + (bh * n + q0 + qq) * KSW + 8 * (e & 1));
        *reinterpret_cast<u32x4s *>(ksl + qq * KSW + 8 * (e & 1)) = v;
    }
    for (int e = tid; e < QG * E; e += NT) cs[e] = -INFINITY;
    for (int e = tid; e < QG * (D / 8); e += NT) {   // the group's routing queries, 16 bytes at a time
        const int qq = e / (D / 8), c = e % (D / 8);
        u32x4s v = {0u, 0u, 0u, 0u};
        if (qq < nq) v = *reinterpret_cast<const u32x4s *>(rq + (bh * n + q0 + qq) * D + 8 * c);
        *reinterpret_cast<u32x4s *>(rqs + qq * RQS + 8 * c) = v;
    }
    for (int e = tid; e < nsp; e += NT) cntS[e] = 0;
    __syncthreads();
    // ---- bucket the (query, kept super) pairs by super: count, offsets, fill
    for (int qq = tid; qq < nq; qq += NT)
        for (int r = 0; r < beff; ++r) {
            const int sp = ksl[qq * KSW + r];
            if (sp >= 0 && sp < nsp) atomicAdd(&cntS[sp], 1);
        }
    __syncthreads();
    if (w == 0) {
        int base = 0;
        for (int s0 = 0; s0 < nsp; s0 += 64) {
            const int c = (s0 + lane < nsp) ? cntS[s0 + lane] : 0;
            int incl = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (s0 + lane < nsp) offS[s0 + lane] = base + incl - c;
            base += __shfl(incl, 63, 64);
        }
    }
    __syncthreads();
    for (int qq = tid; qq < nq; qq += NT)
        for (int r = 0; r < beff; ++r) {
            const int sp = ksl[qq * KSW + r];
            if (sp >= 0 && sp < nsp) {
                const int pos = atomicAdd(&offS[sp], 1);   // offS ends as the end of each bucket
                lists[pos] = (uint16_t)((qq << 4) | r);
            }
        }
    __syncthreads();
    // ---- per super: its children once, 16 of its queries per MFMA tile.
    // Wave w takes the non-empty supers w, w + NW, ...; the next one's
    // children and first tile of routing queries load while this one computes.
    const bf16_t *Sg = S0 + bh * nb * 4 * D;
    const int NMT = F / 4;
    auto loadA = [&](int sp, bf16x8 (&af)[4][NKS]) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            if (mt >= NMT) break;   // uniform
            int64_t blk = (int64_t)sp * F + 4 * mt + (l16 >> 2);
            blk = (blk < nb) ? blk : nb - 1;   // rows past the last block: never stored
            const bf16_t *src = Sg + (blk * 4 + (l16 & 3)) * D + 8 * lg;
#pragma unroll
            for (int ks2 = 0; ks2 < NKS; ++ks2) af[mt][ks2] = ldb8(src + 32 * ks2);
        }
    };
    // tile j0 of super sp: this lane's column entry and its routing query
    auto loadQ = [&](int sp, int j0, bf16x8 (&qv)[NKS], int &ent, bool &cv) {
        const int c = cntS[sp];
        cv = j0 + l16 < c;
        ent = cv ? lists[offS[sp] - c + j0 + l16] : 0;
        const bf16_t *row = rqs + (ent >> 4) * RQS + 8 * lg;
#pragma unroll
        for (int ks2 = 0; ks2 < NKS; ++ks2) qv[ks2] = ldb8(row + 32 * ks2);
    };
    auto tile = [&](int sp, const bf16x8 (&af)[4][NKS], const bf16x8 (&qv)[NKS], int ent, bool cv) {
        const int qq = ent >> 4, r = ent & 15;
        const int64_t qi = q0 + qq;
        f32x4 acc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            if (mt >= NMT) break;
            acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks2 = 0; ks2 < NKS; ++ks2)
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][ks2], qv[ks2], acc[mt], 0, 0, 0);
        }
        const int64_t bm = cand_bmax(qi, 64, W);
        float *dst = cs + qq * E + r * F;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            if (mt >= NMT) break;
            const int ch = 4 * mt + lg;
            const int64_t blk = (int64_t)sp * F + ch;
            float best = acc[mt][0];
            best = (acc[mt][1] > best) ? acc[mt][1] : best;
            best = (acc[mt][2] > best) ? acc[mt][2] : best;
            best = (acc[mt][3] > best) ? acc[mt][3] : best;
            const float v = best * scale;
            const bool ok = cv && blk >= 1 && blk <= bm;
            if (cv) dst[ch] = ok ? v : -INFINITY;
            if (ok && scores) scores[(bh * n + qi) * nb + blk] = v;
        }
    };
    auto next_super = [&](int sp) {   // the wave's next non-empty super at or after sp (uniform)
        while (sp < nsp && cntS[sp] == 0) sp += NW;
        return sp;
    };
    {
        bf16x8 afA[4][NKS], afB[4][NKS], qA[NKS], qB[NKS];
        int eA = 0, eB = 0;
        bool cA = false, cB = false;
        int sp = next_super(w);
        if (sp < nsp) {
            loadA(sp, afA);
            loadQ(sp, 0, qA, eA, cA);
        }
        while (sp < nsp) {
            const int sn = next_super(sp + NW);
            if (sn < nsp) {
                loadA(sn, afB);
                loadQ(sn, 0, qB, eB, cB);
            }
            tile(sp, afA, qA, eA, cA);
            const int c = cntS[sp];
            for (int j0 = 16; j0 < c; j0 += 16) {
                bf16x8 qv[NKS];
                int e;
                bool cv;
                loadQ(sp, j0, qv, e, cv);
                tile(sp, afA, qv, e, cv);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int ks2 = 0; ks2 < NKS; ++ks2) afA[mt][ks2] = afB[mt][ks2];
#pragma unroll
            for (int ks2 = 0; ks2 < NKS; ++ks2) qA[ks2] = qB[ks2];
            eA = eB;
            cA = cB;
            sp = sn;
        }
    }
    __syncthreads();
    // ---- per query, 16 lanes: the kout best listed children (as
    // score_select_mfma_kernel's level 2)
    uint64_t *tk = tkall + w * TKW;
    uint64_t *lst = tk + 4 * 32;
    const int qq4 = lane >> 4, sl = lane & 15;
    static_assert(16 * EL <= SEL_GMAXE, "positions per lane");
    const int j0l = sl / F, jstep = 16 / F, ch0 = sl % F;
    for (int base = 16 * w; base < nq; base += 16 * NW) {   // 16 queries per wave and pass
        for (int r4 = 0; r4 < 4; ++r4) {
            const int qc = base + 4 * r4 + qq4;
            const bool qv_ = qc < nq;
            const int qcc = qv_ ? qc : 0;
            const int64_t qi = q0 + qc;
            const float *cq = cs + qcc * E;
            const int16_t *kq = ksl + qcc * KSW;
            float cvv[EL];
            int kb[EL];
#pragma unroll
            for (int t = 0; t < EL; ++t) {
                const int p = sl + 16 * t;
                const int jr = j0l + t * jstep;
                cvv[t] = (qv_ && p < E) ? cq[p] : -INFINITY;
                kb[t] = kq[jr < 16 ? jr : 15];
            }
            uint64_t ky[EL];
#pragma unroll
            for (int t = 0; t < EL; ++t) ky[t] = (cvv[t] == -INFINITY) ? 0ull : sel_key(cvv[t], kb[t] * F + ch0);
            uint64_t t0 = 0ull, t1 = 0ull;
#pragma unroll
            for (int t = 0; t < EL; ++t) {
                const uint64_t key = ky[t];
                t1 = (key > t0) ? t0 : ((key > t1) ? key : t1);
                t0 = (key > t0) ? key : t0;
            }
            tk[qq4 * 32 + 2 * sl] = t0;
            tk[qq4 * 32 + 2 * sl + 1] = t1;
            wave_lds_sync();
            int g0 = 0, g1 = 0;
            for (int j = 0; j < 32; ++j) {
                const uint64_t x = tk[qq4 * 32 + j];
                g0 += (x > t0) ? 1 : 0;
                g1 += (x > t1) ? 1 : 0;
            }
            uint64_t tau = ~0ull;
            if (g0 < kout) tau = t0;
            if (g1 < kout && t1 < tau) tau = t1;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const uint64_t ot = shfl_xor_u64(tau, o);
                tau = (ot < tau) ? ot : tau;
            }
            int mine = 0;
#pragma unroll
            for (int t = 0; t < EL; ++t) mine += (ky[t] != 0ull && ky[t] >= tau) ? 1 : 0;
            int incl = mine;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const int t = __shfl_up(incl, o, 16);
                if (sl >= o) incl += t;
            }
            const int total = __shfl(incl, 15, 16);
            if (total <= SEL_GCAP) {
                int pos = incl - mine;
#pragma unroll
                for (int t = 0; t < EL; ++t)
                    if (ky[t] != 0ull && ky[t] >= tau) lst[qq4 * SEL_GCAP + pos++] = ky[t];
            }
            wave_lds_sync();
            if (qv_) {
                const int64_t o = (bh * n + qi) * kk;
                if (total > SEL_GCAP) {   // too many ties at tau: the exact pass recomputes the tile
                    if (sl == 0) cnt[bh * n + qi] = SEL_OVERFLOW;
                } else {
                    const uint64_t *lq = lst + qq4 * SEL_GCAP;
                    for (int j = sl; j < total; j += 16) {
                        const uint64_t key = lq[j];
                        int rank = 0;
#pragma unroll 8
                        for (int j2 = 0; j2 < total; ++j2) rank += (lq[j2] > key) ? 1 : 0;
                        if (rank < kout) {
                            idx[o + rank] = sel_key_block(key);
                            val[o + rank] = sel_key_score(key);
                        }
                    }
                    const int taken = (total < kout) ? total : kout;
                    for (int j = taken + sl; j < kk; j += 16) {
                        idx[o + j] = -1;
                        val[o + j] = -INFINITY;
                    }
                    if (sl == 0) cnt[bh * n + qi] = taken;
                }
            }
            wave_lds_sync();   // tk and lst are reused by the next four queries
        }
    }
}

// ---------------------------------------------- bf16 flat top-k, threshold ----
// The same scores as score_select_mfma_kernel (the same MFMA operands in the
// same order, so bit-identical), ranked without sorted lists.  Workgroup = 64
// queries of one KV head (four 16-column MFMA tiles); the four waves split the
// block stages (16 blocks each; wave w takes stages w, w+4, ...) and load
// their A fragments straight from L2 into registers two stages ahead: no LDS
// ring and no barrier in the scans.  A query's blocks are then spread over 16
// lanes (4 waves x 4 lane groups).
//   pass A  each lane keeps the 2 largest candidate scores it sees (values
//           only, a max/min network).  The k-th largest tau of the query's 32
//           values is a lower bound of its k-th score: at least k scores are
//           >= tau, so the top-k is among the scores >= tau.
//   pass B  the same scan appends every candidate scoring >= tau to the
//           query's list in LDS (about k + 2 entries on random scores).
//   rank    an entry's rank is the number of entries ordered before it under
//           (score desc, block asc); ranks < k are the picks.
// A query whose list overflows (many scores tied at tau) gets cnt =
// SEL_OVERFLOW, and score_select_mfma_kernel (marked_only) recomputes its
// 64-query tile exactly.
namespace thr {
constexpr int QW = 64;            // queries per workgroup
constexpr int NCT = QW / 16;      // 16-column MFMA tiles
constexpr int CB = 16;            // blocks per stage: 4 M-tiles of 4 blocks x 4 slots
constexpr int LPQ = 16;           // lanes holding a query's blocks
constexpr int TV = 2;             // values kept per lane
template <int KMAX>
struct Cfg {
    static constexpr int CAP = (5 * KMAX) / 2;   // list entries per query
};
}  // namespace thr


template <int D, int KMAX>
__global__ __launch_bounds__(256, 2) void score_select_thr_kernel(
    const bf16_t *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh, const float *__restrict__ qgain,
    float eps, const bf16_t *__restrict__ S0, int64_t n, int Hq, int Hkv, int64_t nb, int64_t W, int kk,
    float scale, int32_t *__restrict__ idx, float *__restrict__ val, int32_t *__restrict__ cnt,
    float *__restrict__ scores, int ntiles) {
    using namespace thr;
    constexpr int CAP = Cfg<KMAX>::CAP;
    constexpr int NKS = D / 32;
    constexpr int ROWQ = D + 8;                        // padded LDS row of the routing queries
    // LDS: phase 1 the routing queries and the kept values; phase 2 the lists
    constexpr size_t P1 = (size_t)QW * ROWQ * 2 + (size_t)QW * LPQ * TV * 4;
    constexpr size_t P2 = (size_t)QW * CAP * 8;
    constexpr size_t UB = P1 > P2 ? P1 : P2;
    __shared__ __align__(16) char pool[UB];
    __shared__ float taus[QW];
    __shared__ int qcnt[QW];
    bf16_t *qgs = reinterpret_cast<bf16_t *>(pool);
    float *tvs = reinterpret_cast<float *>(pool + (size_t)QW * ROWQ * 2);   // [query][lane][TV]
    uint64_t *lk = reinterpret_cast<uint64_t *>(pool);                     // [query][CAP] keys

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    int tile, g;
    int64_t b;
    sel_deep_first(ntiles, Hkv, tile, g, b);
    const int G = Hq / Hkv;
    const int64_t i0 = (int64_t)tile * QW;
    routing_queries_tile<D, ROWQ>(q, qsb, qsn, qsh, qgain, eps, b, i0, n, g, G, qgs, tid);
    __syncthreads();
    bf16x8 qb[NCT][NKS];
    int bmax[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        const int qc = 16 * ct + l16;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) qb[ct][ks] = ldb8(qgs + qc * ROWQ + 32 * ks + 8 * lg);
        const int64_t iq = i0 + qc;
        bmax[ct] = (iq < n) ? (int)cand_bmax(iq, 64, W) : 0;
    }
    const int64_t last = (i0 + QW - 1 < n) ? i0 + QW - 1 : n - 1;
    const int tile_bmax = (int)cand_bmax(last, 64, W);
    // every query of the tile has the candidates 1 .. bmin (bmax grows with i)
    const int bmin = (i0 + QW - 1 < n) ? (int)cand_bmax(i0, 64, W) : 0;
    const int nst = (tile_bmax > 0) ? (tile_bmax + CB - 1) / CB : 0;
    const bf16_t *Sg = S0 + (b * Hkv + g) * nb * 4 * D;

    // This wave's stages w, w+4, ...: A row l16 of M-tile mt is slot l16 & 3
    // of block 1 + 16 st + 4 mt + l16 / 4 (clamped to tile_bmax: rows past it
    // are never visited); visit(ct, block, score, candidate) per lane and
    // column tile.  Stages wholly within 1 .. bmin need no candidate mask.
    auto load_mt = [&](int st, int mt, bf16x8 (&af)[NKS]) {
        int blk = 1 + st * CB + 4 * mt + (l16 >> 2);
        blk = (blk <= tile_bmax) ? blk : tile_bmax;
        const bf16_t *src = Sg + ((int64_t)blk * 4 + (l16 & 3)) * D + 8 * lg;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) af[ks] = ldb8(src + 32 * ks);
    };
    auto load = [&](int st, bf16x8 (&af)[4][NKS]) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) load_mt(st, mt, af[mt]);
    };
    // d = 64: two stages of A fragments in flight (a0, a1).  d = 128: their
    // 128 VGPRs do not fit beside the B operand (1 KB per lane went to
    // scratch), so one stage's buffers roll: M-tile mt of stage st + 4 is
    // loaded into af[mt] as soon as stage st's MFMAs have read it.
    constexpr bool ROLL = D > 64;
    auto scan = [&](auto &&visit) {
        auto stage = [&](int st, bf16x8 (&af)[4][NKS], auto mask_c, int nxt) {
            constexpr bool MASK = decltype(mask_c)::value;
            const int b0 = 1 + st * CB;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int blk = b0 + 4 * mt + lg;
                // the column tiles' MFMA chains first (independent, so they
                // pipeline), then the scores
                f32x4 acc[NCT];
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) acc[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                    for (int ct = 0; ct < NCT; ++ct)
                        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt][ks], qb[ct][ks], acc[ct], 0, 0, 0);
                if (ROLL && nxt >= 0) load_mt(nxt, mt, af[mt]);   // wave-uniform
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    // the max is exact in any order (no NaN)
                    const float best = fmaxf(fmaxf(acc[ct][0], acc[ct][1]), fmaxf(acc[ct][2], acc[ct][3]));
                    visit(ct, blk, best * scale, !MASK || blk <= bmax[ct]);
                }
            }
        };
        auto run = [&](int st, bf16x8 (&af)[4][NKS], int nxt) {
            if (st * CB + CB <= bmin) stage(st, af, std::false_type(), nxt);   // uniform
            else stage(st, af, std::true_type(), nxt);
        };
        if constexpr (ROLL) {
            bf16x8 a0[4][NKS];
            int st = w;
            if (st < nst) load(st, a0);
            while (st < nst) {
                run(st, a0, (st + 4 < nst) ? st + 4 : -1);
                st += 4;
            }
        } else {
            bf16x8 a0[4][NKS], a1[4][NKS];
            int st = w;
            if (st < nst) load(st, a0);
            if (st + 4 < nst) load(st + 4, a1);
            while (st < nst) {
                run(st, a0, -1);
                if (st + 8 < nst) load(st + 8, a0);
                st += 4;
                if (st >= nst) break;
                run(st, a1, -1);
                if (st + 8 < nst) load(st + 8, a1);
                st += 4;
            }
        }
    };

    // ---- pass A: the 2 largest candidate scores per lane and column tile
    float t0[NCT], t1[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) t0[ct] = t1[ct] = -INFINITY;
    auto keep2 = [&](int ct, float x) {
        t1[ct] = fmaxf(t1[ct], fminf(t0[ct], x));
        t0[ct] = fmaxf(t0[ct], x);
    };
    if (scores) {   // the verification dump: a separate scan keeps the other branch-free
        scan([&](int ct, int blk, float v, bool ok) {
            if (ok) scores[((b * Hkv + g) * n + i0 + 16 * ct + l16) * nb + blk] = v;
            keep2(ct, ok ? v : -INFINITY);
        });
    } else {
        scan([&](int ct, int, float v, bool ok) { keep2(ct, ok ? v : -INFINITY); });
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        float *dst = tvs + ((16 * ct + l16) * LPQ + 4 * w + lg) * TV;
        dst[0] = t0[ct];
        dst[1] = t1[ct];
    }
    __syncthreads();
    // tau of query tid / 4: the kk-th largest of its 32 values (the smallest
    // value with fewer than kk values strictly above it), 8 values per thread
    {
        const int qc = tid >> 2, part = tid & 3;
        const float4 *tq4 = reinterpret_cast<const float4 *>(tvs + qc * LPQ * TV);
        float tq[LPQ * TV];
#pragma unroll
        for (int j = 0; j < LPQ * TV / 4; ++j) {
            const float4 t4 = tq4[j];
            tq[4 * j] = t4.x;
            tq[4 * j + 1] = t4.y;
            tq[4 * j + 2] = t4.z;
            tq[4 * j + 3] = t4.w;
        }
        float best = INFINITY;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = tq[8 * part + j];
            int gt = 0;
#pragma unroll
            for (int j2 = 0; j2 < LPQ * TV; ++j2) gt += (tq[j2] > v) ? 1 : 0;
            best = (gt < kk) ? fminf(best, v) : best;
        }
        best = fminf(best, __shfl_xor(best, 1, 64));
        best = fminf(best, __shfl_xor(best, 2, 64));
        if (part == 0) taus[qc] = best;
    }
    __syncthreads();   // every tau is set; the values' LDS now holds the lists
    float tau[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) tau[ct] = taus[16 * ct + l16];

    // ---- pass B: every candidate scoring >= tau into its query's list
    if (tid < QW) qcnt[tid] = 0;
    __syncthreads();
    scan([&](int ct, int blk, float v, bool ok) {
        if (ok && v >= tau[ct]) {
            const int qc = 16 * ct + l16;
            const int pos = atomicAdd(&qcnt[qc], 1);
            if (pos < CAP) lk[qc * CAP + pos] = sel_key(v, blk);
        }
    });
    __syncthreads();

    // ---- rank the listed entries of query tid / 4: an entry's rank is the
    // number of keys above it; ranks < kk are the picks
    {
        const int qc = tid >> 2, part = tid & 3;
        const int64_t iq = i0 + qc;
        if (iq < n) {
            const int64_t o = ((b * Hkv + g) * n + iq) * kk;
            const int c = qcnt[qc];
            if (c > CAP) {                             // overflow: the exact pass recomputes the tile
                if (part == 0) cnt[(b * Hkv + g) * n + iq] = SEL_OVERFLOW;
            } else {
                const uint64_t *kl = lk + qc * CAP;
                for (int j = part; j < c; j += 4) {
                    const uint64_t key = kl[j];
                    int rank = 0;
                    for (int j2 = 0; j2 < c; j2 += 2) {   // CAP is even: the pair stays in the list
                        const ulonglong2 k2 = *reinterpret_cast<const ulonglong2 *>(kl + j2);
                        rank += (k2.x > key) ? 1 : 0;
                        rank += (j2 + 1 < c && k2.y > key) ? 1 : 0;
                    }
                    if (rank < kk) {
                        idx[o + rank] = sel_key_block(key);
                        val[o + rank] = sel_key_score(key);
                    }
                }
                const int taken = (c < kk) ? c : kk;
                for (int j = taken + ((part - taken) & 3); j < kk; j += 4) {
                    idx[o + j] = -1;
                    val[o + j] = -INFINITY;
                }
                if (part == 0) cnt[(b * Hkv + g) * n + iq] = taken;
            }
        }
    }
}

template <int DT, int D, int M, int KMAX>
__global__ __launch_bounds__(SEL_WG) void hier_select_kernel(
    const typename St<DT>::T *__restrict__ q, int64_t qsb, int64_t qsn, int64_t qsh,
    const float *__restrict__ qgain, float eps, const typename St<DT>::T *__restrict__ S0,
    const typename St<DT>::T *__restrict__ S1, int64_t n, int Hq, int Hkv, int64_t nb, int64_t W,
    int kk, int F, int beam, float scale, int32_t *__restrict__ idx, float *__restrict__ val,
    int32_t *__restrict__ cnt) {
    constexpr int CB = SEL_LDS_FLOATS / (M * D);
    constexpr int BEAMMAX = 16;
    __shared__ __align__(16) float lds[SEL_LDS_FLOATS];
    const int lane = threadIdx.x;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int G = Hq / Hkv;
    const int64_t i = (int64_t)blockIdx.x * SEL_WG + lane;
    const bool active = i < n;
    const int64_t ns = (nb + F - 1) / F;
    const int beff = (int)((beam < ns) ? beam : ns);
    float qg[D];
    if (active) routing_query<DT, D>(q, qsb, qsn, qsh, qgain, eps, b, i, g, G, qg);
    const int64_t bmax = active ? cand_bmax(i, 64, W) : 0;
    // level 1: supers holding at least one candidate child
    float pv[BEAMMAX];
    int pid[BEAMMAX];
#pragma unroll
    for (int j = 0; j < BEAMMAX; ++j) {
        pv[j] = -INFINITY;
        pid[j] = -1;
    }
    const typename St<DT>::T *S1g = S1 + (b * Hkv + g) * ns * M * D;
    for (int64_t p0 = 0; p0 < ns; p0 += CB) {
        int cb = (int)((ns - p0 < CB) ? ns - p0 : CB);
        __syncthreads();
        stage_blocks<DT, D, M>(lds, S1g, p0, cb);
        __syncthreads();
        for (int c = 0; c < cb; ++c) {
            int64_t p = p0 + c;
            int64_t lo = p * F, hi = lo + F - 1;
            if (hi > nb - 1) hi = nb - 1;
            bool has = (bmax >= 1) && (lo <= bmax) && (hi >= 1);
            if (has) {
                float v = slot_score_lds<D, M>(qg, lds + c * M * D, scale);
                insert_inorder<BEAMMAX>(pv, pid, v, (int)p);
            }
        }
    }
    if (!active) return;
    // level 2: children of the kept parents, in parent-rank order
    float vals[KMAX];
    int ids[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        vals[j] = -INFINITY;
        ids[j] = -1;
    }
    const typename St<DT>::T *S0g = S0 + (b * Hkv + g) * nb * M * D;
    for (int a = 0; a < beff; ++a) {
        if (pv[a] == -INFINITY) break;
        int64_t base = (int64_t)pid[a] * F;
        for (int c = 0; c < F; ++c) {
            int64_t blk = base + c;
            if (blk >= nb) break;
            if (blk < 1 || blk > bmax) continue;
            float v = slot_score_gmem<DT, D, M>(qg, S0g + blk * M * D, scale);
            insert_any<KMAX>(vals, ids, v, (int)blk);
        }
    }
    int kke = (kk < beff * F) ? kk : beff * F;
    int64_t o = ((b * Hkv + g) * n + i) * kk;
    int c = 0;
    for (int j = 0; j < kk; ++j) {
        bool ok = j < kke && vals[j] != -INFINITY;
        idx[o + j] = ok ? ids[j] : -1;
        val[o + j] = ok ? vals[j] : -INFINITY;
        c += ok ? 1 : 0;
    }
    cnt[(b * Hkv + g) * n + i] = c;
}

}  // namespace hba

using namespace hba;

namespace {

int select_checks(int dtype, const void *q, const int64_t *qs, const void *S0, int64_t B, int64_t n,
                  int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W, int64_t k,
                  const int32_t *idx, const float *val, const int32_t *cnt) {
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !qs || !S0 || !idx || !val || !cnt) return HBA_ERR_INVALID_ARG;
    if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || W < 1 || k < 1)
        return HBA_ERR_INVALID_ARG;
    if (Bk != 64) return HBA_ERR_UNSUPPORTED;
    if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
    if (k > 64 || !(m == 1 || m == 2 || m == 4 || m == 8)) return HBA_ERR_UNSUPPORTED;
    if (m * d > SEL_LDS_FLOATS) return HBA_ERR_UNSUPPORTED;
    if (!abi::rows_aligned(dtype, q, qs)) return HBA_ERR_UNSUPPORTED;
    if (B > 65535 || Hkv > 65535 || (n + SEL_WG - 1) / SEL_WG * Hkv * B > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    return HBA_OK;
}

template <int DT, int D, int M, int KMAX>
void launch_flat(const void *q, const int64_t *qs, const float *qgain, float eps, const void *S0,
                 int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t W, int64_t k, float scale,
                 int32_t *idx, float *val, int32_t *cnt, float *scores, hipStream_t s) {
    dim3 grid((unsigned)((n + SEL_WG - 1) / SEL_WG), (unsigned)Hkv, (unsigned)B);
    if constexpr (DT == 1 && M == 4 && KMAX <= 32) {
        if (Hq / Hkv <= 16) {   // the routing-query tile takes up to 16 heads per KV head
            // threshold top-k, then the exact kernel on the tiles it marked
            const int ntiles = (int)((n + thr::QW - 1) / thr::QW);
            const dim3 g1((unsigned)(ntiles * Hkv * B));
            hipLaunchKernelGGL((score_select_thr_kernel<D, KMAX>), g1, dim3(256), 0, s,
                               (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, eps, (const bf16_t *)S0, n, (int)Hq,
                               (int)Hkv, n / 64, W, (int)k, scale, idx, val, cnt, scores, ntiles);
            hipLaunchKernelGGL((score_select_mfma_kernel<D, KMAX, false>), g1, dim3(256), 0, s,
                               (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, eps, (const bf16_t *)S0, n, (int)Hq,
                               (int)Hkv, n / 64, W, (int)k, scale, idx, val, cnt, scores, nullptr, 1, 1, nullptr, 1, 0,
                               nullptr, nullptr);
            return;
        }
    }
    hipLaunchKernelGGL((score_select_kernel<DT, D, M, KMAX>), grid, dim3(SEL_WG), 0, s,
                       (const typename St<DT>::T *)q, qs[0], qs[1], qs[2], qgain, eps,
                       (const typename St<DT>::T *)S0, n, (int)Hq, (int)Hkv, n / 64, W, (int)k,
                       scale, idx, val, cnt, scores);
}

// Workspace of the grouped level 2 (hier_l2_kernel): the routing queries
// [B, Hkv, n, D] bf16, then the kept supers [B, Hkv, n, 16] int16.
inline size_t hier_ws_rq(int64_t B, int64_t n, int64_t Hkv, int64_t D) {
    return ((size_t)B * Hkv * n * D * 2 + 255) & ~(size_t)255;
}
inline size_t hier_ws_bytes(int64_t B, int64_t n, int64_t Hkv, int64_t D) {
    return hier_ws_rq(B, n, Hkv, D) + (((size_t)B * Hkv * n * hl2::KSW * 2 + 255) & ~(size_t)255);
}
// Queries per group: the largest multiple of 64 (up to 1024) whose lists fit LDS.
inline int hier_qg(int E, int beff, int64_t ns, int64_t D) {
    for (int QG = 1024; QG >= 64; QG -= 64)
        if (hl2::bytes(QG, E, beff, (int)ns, (int)D) <= (size_t)160 * 1024 - 64) return QG;
    return 0;
}
// The grouped level 2 applies: bf16, 4 slots, k <= 32, G <= 16, F in {4, 8,
// 16}, beam * F <= 256 (and the geometry of score_select_mfma_kernel's HIER).
inline bool hier_grouped_ok(int64_t d, int64_t m, int64_t n, int64_t Hq, int64_t Hkv, int64_t k, int64_t F,
                            int64_t beam) {
    const int64_t ns = (n / 64 + F - 1) / F;
    const int64_t beff = (beam < ns) ? beam : ns;
    return (d == 64 || d == 128) && m == 4 && k <= 32 && ns <= 32 * SEL_PMW && Hq / Hkv <= 16 && F >= 4 &&
           16 % F == 0 && beff * F <= SEL_GMAXE && beff <= hl2::KSW && hier_qg((int)(beff * F), (int)beff, ns, d) > 0;
}

template <int DT, int D, int M, int KMAX>
void launch_hier(const void *q, const int64_t *qs, const float *qgain, float eps, const void *S0,
                 const void *S1, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t W, int64_t k,
                 int64_t F, int64_t beam, float scale, int32_t *idx, float *val, int32_t *cnt,
                 float *scores, float *sup_scores, void *ws, hipStream_t s) {
    const int64_t ns = (n / 64 + F - 1) / F;
    if constexpr (DT == 1 && M == 4 && KMAX <= 32) {
        if (ns <= 32 * SEL_PMW && Hq / Hkv <= 16) {
            const dim3 grid((unsigned)(((n + 63) / 64) * Hkv * B));
            const int nwp = sel_nwp(ns);
            const int64_t beff = (beam < ns) ? beam : ns;
            // level 2 by super where its lists fit; the exact kernel then
            // recomputes any tile holding a query whose list overflowed
            const bool gather = F >= 4 && 16 % F == 0 && beff * F <= SEL_GMAXE;
            const size_t pm = (size_t)64 * nwp * sizeof(uint32_t);
            const size_t pmg = sel_cs_off(nwp) + (size_t)64 * beff * F * sizeof(float);
            // level 1 keeps beam-sized lists per lane (insertion cost grows with the length)
            auto kfn = (beam <= 8) ? score_select_mfma_kernel<D, KMAX, true, 8>
                                   : score_select_mfma_kernel<D, KMAX, true, 16>;
            if (ws) {
                // level 1 per 64-query tile into the workspace, then level 2
                // and the ranking per group of QG queries
                const int E = (int)(beff * F);
                const int QG = hier_qg(E, (int)beff, ns, D);
                const int ngroups = (int)((n + QG - 1) / QG);
                bf16_t *rq = reinterpret_cast<bf16_t *>(ws);
                int16_t *ksp = reinterpret_cast<int16_t *>(reinterpret_cast<char *>(ws) + hier_ws_rq(B, n, Hkv, D));
                auto k1 = (beam <= 4)   ? score_select_mfma_kernel<D, KMAX, true, 4, true>
                          : (beam <= 8) ? score_select_mfma_kernel<D, KMAX, true, 8, true>
                                        : score_select_mfma_kernel<D, KMAX, true, 16, true>;
                hipLaunchKernelGGL(k1, grid, dim3(256), pm, s, (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, eps,
                                   (const bf16_t *)S0, n, (int)Hq, (int)Hkv, n / 64, W, (int)k, scale, idx, val,
                                   cnt, scores, (const bf16_t *)S1, (int)F, (int)beam, sup_scores, 0, 2, rq, ksp);
                const size_t lds = hl2::bytes(QG, E, (int)beff, (int)ns, D);
                auto l2 = (E <= 64)    ? hier_l2_kernel<D, 4>
                          : (E <= 128) ? hier_l2_kernel<D, 8>
                                       : hier_l2_kernel<D, SEL_GMAXE / 16>;
                if (hipFuncSetAttribute(reinterpret_cast<const void *>(l2),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
                    return;   // the error stays as hipGetLastError's, which the entry point reports
                hipLaunchKernelGGL(l2, dim3((unsigned)(ngroups * Hkv * B)), dim3(hl2::NT), lds, s,
                                   (const bf16_t *)S0, (const bf16_t *)rq, (const int16_t *)ksp, n, (int)Hkv, n / 64,
                                   W, (int)k, (int)F, (int)beff, QG, ngroups, scale, idx, val, cnt, scores);
                hipLaunchKernelGGL(kfn, grid, dim3(256), pm, s, (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, eps,
                                   (const bf16_t *)S0, n, (int)Hq, (int)Hkv, n / 64, W, (int)k, scale, idx, val,
                                   cnt, scores, (const bf16_t *)S1, (int)F, (int)beam, sup_scores, 1, 0, nullptr,
                                   nullptr);
                return;
            }
            if (gather && pmg > 65536 &&
                hipFuncSetAttribute(reinterpret_cast<const void *>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)pmg) != hipSuccess)
                return;   // the error stays as hipGetLastError's, which the entry point reports
            hipLaunchKernelGGL(kfn, grid, dim3(256), gather ? pmg : pm, s, (const bf16_t *)q, qs[0], qs[1], qs[2],
                               qgain, eps, (const bf16_t *)S0, n, (int)Hq, (int)Hkv, n / 64, W, (int)k, scale, idx,
                               val, cnt, scores, (const bf16_t *)S1, (int)F, (int)beam, sup_scores, 0,
                               gather ? 1 : 0, nullptr, nullptr);
            if (gather)
                hipLaunchKernelGGL(kfn, grid, dim3(256), pm, s, (const bf16_t *)q, qs[0], qs[1], qs[2], qgain, eps,
                                   (const bf16_t *)S0, n, (int)Hq, (int)Hkv, n / 64, W, (int)k, scale, idx, val,
                                   cnt, scores, (const bf16_t *)S1, (int)F, (int)beam, sup_scores, 1, 0, nullptr,
                                   nullptr);
            return;
        }
    }
    dim3 grid((unsigned)((n + SEL_WG - 1) / SEL_WG), (unsigned)Hkv, (unsigned)B);
    hipLaunchKernelGGL((hier_select_kernel<DT, D, M, KMAX>), grid, dim3(SEL_WG), 0, s,
                       (const typename St<DT>::T *)q, qs[0], qs[1], qs[2], qgain, eps,
                       (const typename St<DT>::T *)S0, (const typename St<DT>::T *)S1, n, (int)Hq,
                       (int)Hkv, n / 64, W, (int)k, (int)F, (int)beam, scale, idx, val, cnt);
}

#define HBA_SEL_DISPATCH_K(FN, DT, D, M, ...)                   \
    do {                                                        \
        if (k <= 16) FN<DT, D, M, 16>(__VA_ARGS__);             \
        else if (k <= 32) FN<DT, D, M, 32>(__VA_ARGS__);        \
        else FN<DT, D, M, 64>(__VA_ARGS__);                     \
    } while (0)

#define HBA_SEL_DISPATCH_M(FN, DT, D, ...)                               \
    do {                                                                 \
        if (m == 1) HBA_SEL_DISPATCH_K(FN, DT, D, 1, __VA_ARGS__);       \
        else if (m == 2) HBA_SEL_DISPATCH_K(FN, DT, D, 2, __VA_ARGS__);  \
        else if (m == 4) HBA_SEL_DISPATCH_K(FN, DT, D, 4, __VA_ARGS__);  \
        else HBA_SEL_DISPATCH_K(FN, DT, D, 8, __VA_ARGS__);              \
    } while (0)

}  // namespace

extern "C" int hba_score_select(int dtype, const void *q, const int64_t q_strides[3],
                                const float *q_gain, float eps, const void *S0, int64_t B, int64_t n,
                                int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W,
                                int64_t k, float scale, int32_t *idx, float *val, int32_t *cnt,
                                float *scores, void *stream) {
    if (dtype == HBA_DTYPE_F32 &&
        (!tuned_shape(d, Bk) || k > 64 || !(m == 1 || m == 2 || m == 4 || m == 8) || m * d > SEL_LDS_FLOATS)) {
        // fp32 with another geometry, k or slot count: the generic kernel
        if (!q || !q_strides || !S0 || !idx || !val || !cnt) return HBA_ERR_INVALID_ARG;
        if (B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || W < 1 || k < 1 || m < 1)
            return HBA_ERR_INVALID_ARG;
        if (!gen_shape_ok(d, Bk)) return HBA_ERR_UNSUPPORTED;
        if (n % Bk != 0) return HBA_ERR_INVALID_ARG;
        if (B > 65535 || Hkv > 65535) return HBA_ERR_UNSUPPORTED;
        return gen_score_select((const float *)q, q_strides, q_gain, eps, (const float *)S0, B, n, Hq, Hkv, d, m,
                                Bk, W, k, scale, idx, val, cnt, scores, (hipStream_t)stream);
    }
    int st = select_checks(dtype, q, q_strides, S0, B, n, Hq, Hkv, d, m, Bk, W, k, idx, val, cnt);
    if (st) return st;
    hipStream_t s = (hipStream_t)stream;
#define HBA_FLAT(DT, D)                                                                            \
    HBA_SEL_DISPATCH_M(launch_flat, DT, D, q, q_strides, q_gain, eps, S0, B, n, Hq, Hkv, W, k, scale, \
                       idx, val, cnt, scores, s)
    HBA_DISPATCH_DT_D(dtype, d, HBA_FLAT);
#undef HBA_FLAT
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

extern "C" int hba_hier_select_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                                               int64_t d, int64_t m, int64_t k, int64_t fanout, int64_t beam,
                                               size_t *bytes) {
    if (!bytes || B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || d <= 0 || m <= 0 || k < 1 ||
        fanout < 1 || beam < 1)
        return HBA_ERR_INVALID_ARG;
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    *bytes = (dtype == HBA_DTYPE_BF16 && hier_grouped_ok(d, m, n, Hq, Hkv, k, fanout, beam))
                 ? hier_ws_bytes(B, n, Hkv, d)
                 : 0;
    return HBA_OK;
}

extern "C" int hba_hier_select(int dtype, const void *q, const int64_t q_strides[3],
                               const float *q_gain, float eps, const void *S0, const void *S1,
                               int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m,
                               int64_t Bk, int64_t W, int64_t k, int64_t fanout, int64_t beam,
                               float scale, int32_t *idx, float *val, int32_t *cnt, float *scores,
                               float *sup_scores, void *workspace, size_t ws_bytes, void *stream) {
    int st = select_checks(dtype, q, q_strides, S0, B, n, Hq, Hkv, d, m, Bk, W, k, idx, val, cnt);
    if (st) return st;
    if (!S1 || fanout < 1 || beam < 1) return HBA_ERR_INVALID_ARG;
    if (beam > 16 || fanout > 64) return HBA_ERR_UNSUPPORTED;
    // the grouped level 2 runs where a large enough workspace comes in
    size_t need = 0;
    hba_hier_select_workspace_bytes(dtype, B, n, Hq, Hkv, d, m, k, fanout, beam, &need);
    void *ws = (need > 0 && workspace && ws_bytes >= need) ? workspace : nullptr;
    if (ws && !abi::aligned16(ws)) return HBA_ERR_INVALID_ARG;
    hipStream_t s = (hipStream_t)stream;
#define HBA_HIER(DT, D)                                                                            \
    HBA_SEL_DISPATCH_M(launch_hier, DT, D, q, q_strides, q_gain, eps, S0, S1, B, n, Hq, Hkv, W, k,   \
                       fanout, beam, scale, idx, val, cnt, scores, sup_scores, ws, s)
    HBA_DISPATCH_DT_D(dtype, d, HBA_HIER);
#undef HBA_HIER
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

// ---------------------------------------------------------------------------
// hier_select with an arbitrary candidate mask: the reference function as
// hba_attention_eval and evals.hier_fidelity call it (src/hba/attention.py:
// 217-246, src/hba/evals.py:314).  One workgroup per (batch row, query row).
// Scores in fp32 in the declared order (dot over d in index order, slot max,
// times scale); a super is scored if one of its children is a candidate;
// the top b_eff = min(beam, ns) supers, then the top min(kk, b_eff * F)
// candidate children, each by block-wide argmax rounds under (score desc,
// block asc).
namespace hr {
constexpr int NT = 256;
constexpr int DMAX = 256, NSMAX = 4096, BEAMMAX = 64, CMAX = 1024;

template <int DT>
__device__ __forceinline__ float score(const float *q, const typename St<DT>::T *S, int m, int d, float scale) {
    float best = 0.0f;
    for (int s = 0; s < m; ++s) {
        float acc = 0.0f;
        for (int t = 0; t < d; ++t) acc = fmaf(q[t], St<DT>::ld(S, (int64_t)s * d + t), acc);
        best = (s == 0 || acc > best) ? acc : best;
    }
    return best * scale;
}

// Position of the best finite entry of vals[0..len) (ids: its block, null =
// the position), -1 if none; the same answer in every thread.  Ends with a
// barrier.
__device__ int argmax(const float *vals, const int *ids, int len, float *wv, int *wi, int *wj) {
    float bv = -INFINITY;
    int bi = 0, bj = -1;
    for (int j = threadIdx.x; j < len; j += NT) {
        const float v = vals[j];
        const int id = ids ? ids[j] : j;
        if (v != -INFINITY && v == v && (bj < 0 || better(v, id, bv, bi))) {
            bv = v;
            bi = id;
            bj = j;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64), oj = __shfl_xor(bj, o, 64);
        if (oj >= 0 && (bj < 0 || better(ov, oi, bv, bi))) {
            bv = ov;
            bi = oi;
            bj = oj;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        wv[w] = bv;
        wi[w] = bi;
        wj[w] = bj;
    }
    __syncthreads();
    float rv = wv[0];
    int ri = wi[0], rj = wj[0];
    for (int x = 1; x < NT / 64; ++x)
        if (wj[x] >= 0 && (rj < 0 || better(wv[x], wi[x], rv, ri))) {
            rv = wv[x];
            ri = wi[x];
            rj = wj[x];
        }
    __syncthreads();
    return rj;
}
}  // namespace hr

template <int DT>
__global__ __launch_bounds__(hr::NT) void hier_rows_kernel(
    const typename St<DT>::T *__restrict__ qn, const typename St<DT>::T *__restrict__ S0,
    const typename St<DT>::T *__restrict__ S1, const uint8_t *__restrict__ cand, int64_t c, int nb, int ns,
    int m, int d, int F, int beff, int kke, float scale, int64_t *__restrict__ top_idx,
    float *__restrict__ top_val) {
    using namespace hr;
    __shared__ float q[DMAX];
    __shared__ float ssc[NSMAX];
    __shared__ float csc[CMAX];
    __shared__ int cid[CMAX];
    __shared__ int par[BEAMMAX];
    __shared__ float wv[NT / 64];
    __shared__ int wi[NT / 64], wj[NT / 64];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x, b = blockIdx.y;
    for (int t = tid; t < d; t += NT) q[t] = St<DT>::ld(qn, (b * c + row) * d + t);
    const uint8_t *cr = cand + row * nb;
    const typename St<DT>::T *S0b = S0 + b * nb * m * d;
    const typename St<DT>::T *S1b = S1 + b * ns * m * d;
    __syncthreads();
    for (int p = tid; p < ns; p += NT) {
        bool has = false;
        for (int j = 0; j < F && p * F + j < nb; ++j) has = has || cr[p * F + j] != 0;
        ssc[p] = has ? score<DT>(q, S1b + (int64_t)p * m * d, m, d, scale) : -INFINITY;
    }
    __syncthreads();
    int np = 0;
    for (int a = 0; a < beff; ++a) {
        const int j = argmax(ssc, nullptr, ns, wv, wi, wj);
        if (j < 0) break;   // uniform
        if (tid == 0) {
            par[a] = j;
            ssc[j] = -INFINITY;
        }
        np = a + 1;
        __syncthreads();
    }
    const int nc = np * F;   // children in parent rank order
    for (int j = tid; j < nc; j += NT) {
        const int blk = par[j / F] * F + j % F;
        cid[j] = blk;
        csc[j] = (blk < nb && cr[blk]) ? score<DT>(q, S0b + (int64_t)blk * m * d, m, d, scale) : -INFINITY;
    }
    __syncthreads();
    int64_t *oi = top_idx + (b * c + row) * kke;
    float *ov = top_val + (b * c + row) * kke;
    for (int r = 0; r < kke; ++r) {
        const int j = argmax(csc, cid, nc, wv, wi, wj);
        if (j < 0) {   // uniform: no candidate child left
            for (int rr = r + tid; rr < kke; rr += NT) {
                oi[rr] = -1;
                ov[rr] = -INFINITY;
            }
            break;
        }
        if (tid == 0) {
            oi[r] = cid[j];
            ov[r] = csc[j];
            csc[j] = -INFINITY;
        }
        __syncthreads();
    }
}

extern "C" int hba_hier_select_rows(int dtype, const void *qn, const void *S0, const void *S1,
                                    const uint8_t *cand, int64_t B, int64_t c, int64_t nb, int64_t m,
                                    int64_t d, int64_t fanout, int64_t beam, int64_t kk, float scale,
                                    int64_t *top_idx, float *top_val, void *stream) {
    if (dtype != HBA_DTYPE_F32 && dtype != HBA_DTYPE_BF16) return HBA_ERR_UNSUPPORTED;
    if (!qn || !S0 || !S1 || !cand || !top_idx || !top_val) return HBA_ERR_INVALID_ARG;
    if (B < 1 || c < 0 || nb < 1 || m < 1 || d < 1 || fanout < 1 || beam < 1 || kk < 1) return HBA_ERR_INVALID_ARG;
    const int64_t ns = (nb + fanout - 1) / fanout;
    const int64_t beff = beam < ns ? beam : ns;
    if (d > hr::DMAX || ns > hr::NSMAX || beff > hr::BEAMMAX || beff * fanout > hr::CMAX) return HBA_ERR_UNSUPPORTED;
    if (c > 0x7fffffff || B > 65535) return HBA_ERR_UNSUPPORTED;
    if (c == 0) return HBA_OK;
    const int64_t kke = kk < beff * fanout ? kk : beff * fanout;
    dim3 grid((unsigned)c, (unsigned)B);
    hipStream_t s = (hipStream_t)stream;
    if (dtype == HBA_DTYPE_F32)
        hipLaunchKernelGGL(hier_rows_kernel<0>, grid, dim3(hr::NT), 0, s, (const float *)qn, (const float *)S0,
                           (const float *)S1, cand, c, (int)nb, (int)ns, (int)m, (int)d, (int)fanout, (int)beff,
                           (int)kke, scale, top_idx, top_val);
    else
        hipLaunchKernelGGL(hier_rows_kernel<1>, grid, dim3(hr::NT), 0, s, (const bf16_t *)qn, (const bf16_t *)S0,
                           (const bf16_t *)S1, cand, c, (int)nb, (int)ns, (int)m, (int)d, (int)fanout, (int)beff,
                           (int)kke, scale, top_idx, top_val);
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}

// ---------------------------------------------------------------------------
// The routing queries alone: qg[b, i, g, :] = the sum over the G heads of KV
// group g of QKNorm(q[b, i, h, :]), in the declared order and storage roundings
// of the selection kernels (grouped_query src/hba/summarizer.py:50-54 on
// _HeadRMSNorm's output src/hba/attention.py:88-94).  qg [B, n, Hkv, d] is a
// valid q for hba_score_select / hba_hier_select with Hq = Hkv and no gain:
// their routing query of a one-head group without QKNorm is the row itself,
// so precomputed and inline routing queries select identically.
// bf16: one 256-thread workgroup per (64 queries, KV head, batch), the
// selection kernels' routing_queries_tile; fp32: one thread per (query, KV
// head), routing_query.
template <int D>
__global__ __launch_bounds__(256) void route_queries_bf16_kernel(const bf16_t *__restrict__ q, int64_t qsb,
                                                                 int64_t qsn, int64_t qsh,
                                                                 const float *__restrict__ qgain, float eps,
                                                                 int64_t n, int Hq, int Hkv,
                                                                 bf16_t *__restrict__ qg) {
    __shared__ __align__(16) bf16_t rows[64 * D];
    const int tid = threadIdx.x;
    const int64_t i0 = (int64_t)blockIdx.x * 64;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    routing_queries_tile<D, D>(q, qsb, qsn, qsh, qgain, eps, b, i0, n, g, Hq / Hkv, rows, tid);
    __syncthreads();
    for (int c = tid; c < 64 * D / 8; c += 256) {   // 16-byte chunks of the tile's rows
        const int r = c / (D / 8), k = c % (D / 8);
        const int64_t i = i0 + r;
        if (i < n)
            *reinterpret_cast<uint4 *>(qg + ((b * n + i) * Hkv + g) * D + 8 * k) =
                *reinterpret_cast<const uint4 *>(rows + r * D + 8 * k);
    }
}

template <int D>
__global__ __launch_bounds__(64) void route_queries_f32_kernel(const float *__restrict__ q, int64_t qsb,
                                                               int64_t qsn, int64_t qsh,
                                                               const float *__restrict__ qgain, float eps,
                                                               int64_t n, int Hq, int Hkv, float *__restrict__ qg) {
    const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
    const int g = blockIdx.y;
    const int64_t b = blockIdx.z;
    if (i >= n) return;
    float x[D];
    routing_query<0, D>(q, qsb, qsn, qsh, qgain, eps, b, i, g, Hq / Hkv, x);
    float *dst = qg + ((b * n + i) * Hkv + g) * D;
#pragma unroll
    for (int t = 0; t < D; ++t) dst[t] = x[t];
}

extern "C" int hba_route_queries(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
                                 float eps, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, void *qg,
                                 void *stream) {
    if (dtype == HBA_DTYPE_F32 && (!(d == 64 || d == 128) || (Hkv > 0 && Hq / Hkv > 16))) {
        // fp32, another head dim or group size: the generic kernel
        if (!q || !q_strides || !qg || B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
            return HBA_ERR_INVALID_ARG;
        if (!gen_shape_ok(d, 1)) return HBA_ERR_UNSUPPORTED;
        return gen_route_queries((const float *)q, q_strides, q_gain, eps, B, n, Hq, Hkv, d, (float *)qg,
                                 (hipStream_t)stream);
    }
    int st = abi::check_dtype_dim(dtype, d);
    if (st) return st;
    if (!q || !q_strides || !qg || B <= 0 || n <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
        return HBA_ERR_INVALID_ARG;
    if (Hq / Hkv > 16) return HBA_ERR_UNSUPPORTED;
    if (!abi::rows_aligned(dtype, q, q_strides) || !abi::aligned16(qg)) return HBA_ERR_UNSUPPORTED;
    if (B > 65535 || Hkv > 65535 || (n + 63) / 64 > 0x7fffffff) return HBA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)Hkv, (unsigned)B);
    hipStream_t s = (hipStream_t)stream;
    if (dtype == HBA_DTYPE_BF16) {
        if (d == 64)
            hipLaunchKernelGGL(route_queries_bf16_kernel<64>, grid, dim3(256), 0, s, (const bf16_t *)q, q_strides[0],
                               q_strides[1], q_strides[2], q_gain, eps, n, (int)Hq, (int)Hkv, (bf16_t *)qg);
        else
            hipLaunchKernelGGL(route_queries_bf16_kernel<128>, grid, dim3(256), 0, s, (const bf16_t *)q,
                               q_strides[0], q_strides[1], q_strides[2], q_gain, eps, n, (int)Hq, (int)Hkv,
                               (bf16_t *)qg);
    } else {
        if (d == 64)
            hipLaunchKernelGGL(route_queries_f32_kernel<64>, grid, dim3(64), 0, s, (const float *)q, q_strides[0],
                               q_strides[1], q_strides[2], q_gain, eps, n, (int)Hq, (int)Hkv, (float *)qg);
        else
            hipLaunchKernelGGL(route_queries_f32_kernel<128>, grid, dim3(64), 0, s, (const float *)q, q_strides[0],
                               q_strides[1], q_strides[2], q_gain, eps, n, (int)Hq, (int)Hkv, (float *)qg);
    }
    HBA_LAUNCH_CHECK();
    return HBA_OK;
}
