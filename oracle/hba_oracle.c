/*
 * CPU oracle for the HBA forward path: the integer / declared-order parts.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, to check the kernels' results.
 *
 * It restates, in plain C with an explicitly declared fp32 operation order,
 * the parts of the reference whose results must be bit-exact between the
 * oracle and the HIP kernels (block selection):
 *
 *   _HeadRMSNorm.forward      src/hba/attention.py:88-94
 *   grouped_query             src/hba/summarizer.py:50-54
 *   slot_block_scores         src/hba/summarizer.py:45-47
 *   _route_candidates         src/hba/attention.py:250-256
 *   route_topk (mask + topk)  src/hba/attention.py:295-302, eval :695-698
 *   build_super               src/hba/attention.py:202-214
 *   hier_select               src/hba/attention.py:217-246
 *
 * Declared order (the kernels follow it operation for operation):
 *   QKNorm   ss = fmaf(x_t, x_t, ss) for t = 0..d-1 (from +0), ms = ss / d,
 *            ms = max(ms, eps), r = sqrtf(ms), y_t = (x_t / r) * gain,
 *            then rounded to the storage dtype (bf16: round-to-nearest-even).
 *   group    qg_t = ((qc_0,t + qc_1,t) + qc_2,t) + ... in fp32, then rounded.
 *   dot      acc = fmaf(q_t, s_t, acc) for t = 0..d-1 (from +0).
 *   score    best = dot(slot 0); best = (dot(slot j) > best) ? dot : best for
 *            j = 1..m-1; score = best * scale.
 *   super    sum = S0[F*p + 0] + S0[F*p + 1] + ... (children that exist, in
 *            order) in fp32, rounded to dtype, divided by the child count,
 *            rounded to dtype.
 *   top-k    order by (score descending, block index ascending); -inf
 *            (non-candidate) entries are never selected; cnt = number kept.
 *
 * The reference itself leaves reduction order and torch.topk tie order
 * unspecified; the oracle-vs-reference agreement is therefore checked with a
 * tolerance on scores and a margin rule on indices (tests/test_oracle_golden.py),
 * and the oracle-vs-kernel agreement bit-exactly.
 */
#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

static inline float rnd_bf16(float x)
{
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u; /* keep NaN quiet */
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    memcpy(&x, &u, 4);
    return x;
}

static inline float rnd(float x, int bf16) { return bf16 ? rnd_bf16(x) : x; }

/* Round a float array to bf16 in place (storage emulation helper). */
void hba_oracle_round_bf16(float *x, int64_t count)
{
    for (int64_t i = 0; i < count; ++i) x[i] = rnd_bf16(x[i]);
}

/* QKNorm rows: x [rows, d]; row r uses gain[r % heads].  attention.py:88-94 */
void hba_oracle_qknorm(const float *x, int64_t rows, int d, int heads,
                       const float *gain, float eps, int bf16, float *y)
{
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * d;
        float *yr = y + r * d;
        float ss = 0.0f;
        for (int t = 0; t < d; ++t) ss = fmaf(xr[t], xr[t], ss);
        float ms = ss / (float)d;
        if (ms < eps) ms = eps;
        float rr = sqrtf(ms);
        float g = gain[r % heads];
        for (int t = 0; t < d; ++t) {
            float q = xr[t] / rr;
            yr[t] = rnd(q * g, bf16);
        }
    }
}

/* grouped_query: qc [n, Hq, d] -> qg [Hkv, n, d].  summarizer.py:50-54 */
void hba_oracle_group_sum(const float *qc, int64_t n, int Hq, int Hkv, int d,
                          int bf16, float *qg)
{
    int G = Hq / Hkv;
    for (int g = 0; g < Hkv; ++g)
        for (int64_t i = 0; i < n; ++i)
            for (int t = 0; t < d; ++t) {
                float s = qc[(i * Hq + g * G) * d + t];
                for (int h = 1; h < G; ++h) s = s + qc[(i * Hq + g * G + h) * d + t];
                qg[((int64_t)g * n + i) * d + t] = rnd(s, bf16);
            }
}

/* Largest candidate block index for query position i (-1 or 0: none).
 * Candidate(i, b) <=> b >= 1 and (b + 1) * Bk <= i - W + 1.  attention.py:250-256 */
static inline int64_t cand_bmax(int64_t i, int Bk, int W)
{
    int64_t lim = i - W + 1;
    if (lim < 2 * (int64_t)Bk) return 0;
    return lim / Bk - 1;
}

int64_t hba_oracle_cand_bmax(int64_t i, int Bk, int W) { return cand_bmax(i, Bk, W); }

static inline float dot_decl(const float *a, const float *b, int d)
{
    float acc = 0.0f;
    for (int t = 0; t < d; ++t) acc = fmaf(a[t], b[t], acc);
    return acc;
}

static inline float slot_score(const float *q, const float *S, int m, int d, float scale)
{
    float best = dot_decl(q, S, d);
    for (int s = 1; s < m; ++s) {
        float v = dot_decl(q, S + (int64_t)s * d, d);
        best = (v > best) ? v : best;
    }
    return best * scale;
}

/* Block scores for the given query positions.
 * qg [n, d] (one KV head), S [nb, m, d]; out [nrows, nb] with -inf at
 * non-candidates.  summarizer.py:45-47 + attention.py:298 */
void hba_oracle_block_scores(const float *qg, const float *S, const int64_t *pos,
                             int64_t nrows, int nb, int m, int d, float scale,
                             int Bk, int W, float *out)
{
    for (int64_t r = 0; r < nrows; ++r) {
        int64_t i = pos[r];
        int64_t bmax = cand_bmax(i, Bk, W);
        const float *q = qg + i * d;
        for (int b = 0; b < nb; ++b) {
            float v = -INFINITY;
            if (b >= 1 && b <= bmax) v = slot_score(q, S + (int64_t)b * m * d, m, d, scale);
            out[r * nb + b] = v;
        }
    }
}

static inline int better(float va, int ia, float vb, int ib)
{
    return (va > vb) || (va == vb && ia < ib);
}

/* top-k of one row of scores under (score desc, index asc); -inf never kept. */
static int topk_row(const float *sc, const int *ids, int len, int kk,
                    int32_t *idx, float *val)
{
    int c = 0;
    for (int j = 0; j < len; ++j) {
        float v = sc[j];
        int id = ids ? ids[j] : j;
        if (v == -INFINITY || v != v) continue;
        if (c == kk && !better(v, id, val[kk - 1], idx[kk - 1])) continue;
        int p = (c < kk) ? c++ : kk - 1;
        while (p > 0 && better(v, id, val[p - 1], idx[p - 1])) {
            val[p] = val[p - 1];
            idx[p] = idx[p - 1];
            --p;
        }
        val[p] = v;
        idx[p] = id;
    }
    for (int j = c; j < kk; ++j) {
        idx[j] = -1;
        val[j] = -INFINITY;
    }
    return c;
}

/* Row-wise top-k.  scores [rows, nb] -> idx/val [rows, kk], cnt [rows]. */
void hba_oracle_topk(const float *scores, int64_t rows, int nb, int kk,
                     int32_t *idx, float *val, int32_t *cnt)
{
    for (int64_t r = 0; r < rows; ++r)
        cnt[r] = topk_row(scores + r * nb, 0, nb, kk, idx + r * kk, val + r * kk);
}

/* build_super: S0 [nb, m, d] -> S1 [ns, m, d].  attention.py:202-214 */
void hba_oracle_build_super(const float *S0, int nb, int m, int d, int F, int bf16,
                            float *S1)
{
    int ns = (nb + F - 1) / F;
    for (int p = 0; p < ns; ++p) {
        int c0 = p * F;
        int cn = (c0 + F <= nb) ? F : nb - c0;
        for (int s = 0; s < m; ++s)
            for (int t = 0; t < d; ++t) {
                float acc = S0[((int64_t)c0 * m + s) * d + t];
                for (int c = 1; c < cn; ++c) acc = acc + S0[((int64_t)(c0 + c) * m + s) * d + t];
                acc = rnd(acc, bf16);
                S1[((int64_t)p * m + s) * d + t] = rnd(acc / (float)cn, bf16);
            }
    }
}

/* hier_select for the given query positions (one KV head).
 * qg [n, d], S0 [nb, m, d], S1 [ns, m, d] -> idx/val [nrows, kk], cnt [nrows].
 * Picks are the top min(kk, b_eff*F) children of the top b_eff = min(beam, ns)
 * candidate-bearing supers.  attention.py:217-246 */
void hba_oracle_hier_select(const float *qg, const float *S0, const float *S1,
                            const int64_t *pos, int64_t nrows, int nb, int m, int d,
                            int F, int beam, int kk, float scale, int Bk, int W,
                            int32_t *idx, float *val, int32_t *cnt)
{
    int ns = (nb + F - 1) / F;
    int beff = beam < ns ? beam : ns;
    float ssc[4096];
    int32_t pidx[64];
    float pval[64];
    float csc[64 * 64];
    int cid[64 * 64];
    for (int64_t r = 0; r < nrows; ++r) {
        int64_t i = pos[r];
        int64_t bmax = cand_bmax(i, Bk, W);
        const float *q = qg + i * d;
        for (int p = 0; p < ns; ++p) {
            /* cand_sup: any child in [p*F, p*F+F) is a candidate */
            int64_t lo = (int64_t)p * F, hi = lo + F - 1;
            if (hi > nb - 1) hi = nb - 1;
            int has = (bmax >= 1) && (lo <= bmax) && (hi >= 1);
            ssc[p] = has ? slot_score(q, S1 + (int64_t)p * m * d, m, d, scale) : -INFINITY;
        }
        int np = topk_row(ssc, 0, ns, beff, pidx, pval);
        int nc = 0;
        for (int a = 0; a < np; ++a)
            for (int c = 0; c < F; ++c) {
                int b = pidx[a] * F + c;
                if (b >= nb) continue;
                float v = -INFINITY;
                if (b >= 1 && b <= bmax) v = slot_score(q, S0 + (int64_t)b * m * d, m, d, scale);
                csc[nc] = v;
                cid[nc] = b;
                ++nc;
            }
        int kke = kk < beff * F ? kk : beff * F;
        cnt[r] = topk_row(csc, cid, nc, kke, idx + r * kk, val + r * kk);
        for (int j = kke; j < kk; ++j) {
            idx[r * kk + j] = -1;
            val[r * kk + j] = -INFINITY;
        }
    }
}

/* hier_select with an arbitrary candidate mask, for one batch row: qn [r, d]
 * (the routing queries), cand [r, nb] (1 = candidate).  A super is scored if
 * any of its children is a candidate (cand_sup); the children of the top
 * b_eff = min(beam, ns) supers are scored if they are candidates, and the
 * top min(kk, b_eff*F) children are the picks.  attention.py:217-246 */
void hba_oracle_hier_select_mask(const float *qn, const float *S0, const float *S1,
                                 const uint8_t *cand, int64_t nrows, int nb, int m, int d,
                                 int F, int beam, int kk, float scale,
                                 int32_t *idx, float *val, int32_t *cnt)
{
    int ns = (nb + F - 1) / F;
    int beff = beam < ns ? beam : ns;
    int kke = kk < beff * F ? kk : beff * F;
    float *ssc = (float *)malloc(sizeof(float) * (size_t)ns);
    int32_t *pidx = (int32_t *)malloc(sizeof(int32_t) * (size_t)beff);
    float *pval = (float *)malloc(sizeof(float) * (size_t)beff);
    float *csc = (float *)malloc(sizeof(float) * (size_t)beff * F);
    int *cid = (int *)malloc(sizeof(int) * (size_t)beff * F);
    for (int64_t r = 0; r < nrows; ++r) {
        const float *q = qn + r * d;
        const uint8_t *cr = cand + r * nb;
        for (int p = 0; p < ns; ++p) {
            int has = 0;
            for (int c = 0; c < F && p * F + c < nb; ++c) has |= cr[p * F + c] != 0;
            ssc[p] = has ? slot_score(q, S1 + (int64_t)p * m * d, m, d, scale) : -INFINITY;
        }
        int np = topk_row(ssc, 0, ns, beff, pidx, pval);
        int nc = 0;
        for (int a = 0; a < np; ++a)
            for (int c = 0; c < F; ++c) {
                int b = pidx[a] * F + c;
                if (b >= nb) continue;
                csc[nc] = cr[b] ? slot_score(q, S0 + (int64_t)b * m * d, m, d, scale) : -INFINITY;
                cid[nc] = b;
                ++nc;
            }
        cnt[r] = topk_row(csc, cid, nc, kke, idx + r * kke, val + r * kke);
        for (int j = cnt[r]; j < kke; ++j) {
            idx[r * kke + j] = -1;
            val[r * kke + j] = -INFINITY;
        }
    }
    free(ssc);
    free(pidx);
    free(pval);
    free(csc);
    free(cid);
}
