/*
 * hba_amd.h -- C-ABI of the MI355X (gfx950) Hierarchical Block Attention
 * forward path.
 *
 * Conventions
 *   - Every pointer argument named as a tensor is a DEVICE pointer; stride and
 *     size arguments are host values in ELEMENTS.  No C++ types cross the
 *     boundary.
 *   - `dtype` is HBA_DTYPE_F32 or HBA_DTYPE_BF16 and applies to the q/k/v and
 *     summary tensors; gains, probes, proj, RoPE tables, scores and scales are
 *     always fp32; indices are int32.
 *   - All calls are asynchronous on `stream` (a hipStream_t; NULL = the null
 *     stream).  No call allocates memory, keeps global mutable state or
 *     synchronises; calls on distinct streams are independent.  Scratch space
 *     (bf16 attention, decode) is passed in by the caller, sized by the *_workspace_size
 *     query.
 *   - Return value: HBA_OK (0) or a negative status (invalid argument,
 *     unsupported shape/dtype/architecture, launch failure);
 *     hba_status_string() names it.  Nothing is launched when a status other
 *     than HBA_OK or HBA_ERR_LAUNCH is returned.
 *   - Layouts: q [B, n, Hq, d] and k, v [B, n, Hkv, d] are the reference's
 *     token-major views (model.py:121-123) with arbitrary strides for the
 *     first three dims and a contiguous last dim; prepared keys are
 *     head-major: kc, kr [B, Hkv, n, d], vt [B, Hkv, d, n]; summaries
 *     S0 [B, Hkv, nb, m, d], supers S1 [B, Hkv, ns, m, d]; selections
 *     idx, val [B, Hkv, n, k] and cnt [B, Hkv, n].
 *   - Head h uses KV head h / (Hq / Hkv) (heads group-contiguous,
 *     summarizer.py:50-54).
 */
#ifndef HBA_AMD_H
#define HBA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HBA_ABI_VERSION 1

enum {
    HBA_OK = 0,
    HBA_ERR_INVALID_ARG = -1,   /* null pointer, bad size, n % block != 0, ... */
    HBA_ERR_UNSUPPORTED = -2,   /* shape/dtype outside what the kernels implement */
    HBA_ERR_DEVICE = -3,        /* no device, or the current device is not gfx950 */
    HBA_ERR_LAUNCH = -4,        /* the kernel launch itself failed */
    HBA_ERR_SCRATCH = -5        /* a no-allocation call needs more than its fixed scratch */
};

enum { HBA_DTYPE_F32 = 0, HBA_DTYPE_BF16 = 1 };

/* Version of this ABI (HBA_ABI_VERSION). */
int hba_abi_version(void);

/* Static description of a status code. */
const char *hba_status_string(int status);

/* HBA_OK when the current HIP device is a gfx950 (MI355X-class) GPU. */
int hba_device_check(void);

/*
 * Key preparation: QKNorm of k (per-head RMS normalisation, scalar gain; the
 * key half of _content_qk), its RoPE rotation for the window branch, and V
 * transposed for the attention kernel.
 *   replaces: _HeadRMSNorm.forward  src/hba/attention.py:88-94 (via _content_qk :185)
 *             apply_rope            src/hba/attention.py:40-44 (k_rope, :633)
 * k_gain == NULL means qknorm=False (kc = k unchanged).  cos_tab/sin_tab are
 * fp32 [>= n, d] tables (rope_tables, attention.py:27-32).  kr or vt may be
 * NULL when not needed.
 */
int hba_prep_keys(int dtype, const void *k, const int64_t k_strides[3],
                  const void *v, const int64_t v_strides[3],
                  const float *k_gain, float eps,
                  const float *cos_tab, const float *sin_tab,
                  int64_t B, int64_t n, int64_t Hkv, int64_t d,
                  void *kc, void *kr, void *vt, void *stream);

/*
 * Slot summaries of every full block of kc.
 *   replaces: SlotSummarizer.summarize  src/hba/summarizer.py:34-42
 * probes fp32 [Hkv, m, d]; proj fp32 [Hkv, d, d]; S0 [B, Hkv, n/Bk, m, d].
 */
int hba_summarize(int dtype, const void *kc, int64_t B, int64_t Hkv, int64_t n,
                  int64_t d, int64_t Bk, const float *probes, const float *proj,
                  int64_t m, void *S0, void *stream);

/*
 * hba_prep_keys and hba_summarize (64-key blocks) in one launch: the
 * workgroup of a 64-key tile summarises the kc rows it has just written, so
 * that S0 is bit-identical to hba_summarize over that kc; tuned geometry
 * only (bf16 or fp32, d = 64 or 128; 1 <= m <= 8).
 *   replaces: _content_qk's key half + apply_rope  src/hba/attention.py:88-94, :40-44
 *             SlotSummarizer.summarize            src/hba/summarizer.py:34-42
 * Arguments as hba_prep_keys, then probes fp32 [Hkv, m, d], proj fp32
 * [Hkv, d, d] and S0 [B, Hkv, n/64, m, d].
 */
int hba_prep_keys_summarize(int dtype, const void *k, const int64_t k_strides[3],
                            const void *v, const int64_t v_strides[3],
                            const float *k_gain, float eps,
                            const float *cos_tab, const float *sin_tab,
                            int64_t B, int64_t n, int64_t Hkv, int64_t d,
                            void *kc, void *kr, void *vt, const float *probes,
                            const float *proj, int64_t m, void *S0, void *stream);

/*
 * Super-summaries: per-slot mean of `fanout` consecutive block summaries.
 *   replaces: build_super  src/hba/attention.py:202-214
 * S1 [B, Hkv, ceil(nb/fanout), m, d].
 */
int hba_build_super(int dtype, const void *S0, int64_t B, int64_t Hkv, int64_t nb,
                    int64_t m, int64_t d, int64_t fanout, void *S1, void *stream);

/*
 * Flat block selection: QKNorm of q, grouped routing query, slot scores
 * (max over slots, times `scale`), candidate mask, top-k per (query, KV head)
 * with ties broken by lowest block index.
 *   replaces: route_topk            src/hba/attention.py:272-303
 *             eval flat selection   src/hba/attention.py:695-698
 *             grouped_query / slot_block_scores  src/hba/summarizer.py:45-54
 * q_gain == NULL means qknorm=False.  Invalid picks (fewer than k
 * candidates) get idx -1 / val -inf; cnt holds the number of valid picks.
 * 1 <= k <= 64.  fp32 inputs are scored with sequential fp32 FMAs over d (the
 * oracle's declared order: bit-exact); bf16 inputs with m == 4 and k <= 32 as
 * a bf16 MFMA GEMM with fp32 accumulation.  scores (optional, NULL to skip):
 * fp32 [B, Hkv, n, n/Bk] receiving the score of every candidate the kernel
 * ranked (other entries are left untouched), so the top-k can be checked on
 * identical score arrays.
 */
int hba_score_select(int dtype, const void *q, const int64_t q_strides[3],
                     const float *q_gain, float eps, const void *S0,
                     int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                     int64_t m, int64_t Bk, int64_t W, int64_t k, float scale,
                     int32_t *idx, float *val, int32_t *cnt, float *scores, void *stream);

/*
 * Two-level selection: score the super-summaries, keep the top
 * min(beam, ns) supers that hold a candidate, score their children, keep the
 * top min(k, beam*fanout).  Same outputs and tie rule as hba_score_select.
 *   replaces: hier_select  src/hba/attention.py:217-246 (eval :690-693)
 * 1 <= beam <= 16, fanout <= 64.  fp32 inputs follow the oracle bit-exactly;
 * bf16 inputs with m == 4, k <= 32 and at most 2048 supers are scored as bf16
 * MFMA GEMMs.  Optional dumps (NULL to skip), entries written only where the
 * kernel ranked a score: sup_scores fp32 [B, Hkv, n, ns] with the score of
 * every super holding a candidate child, scores fp32 [B, Hkv, n, n/Bk] with
 * the score of every candidate child of a kept super.  sup_scores is written
 * by the MFMA path only.  workspace (16-byte aligned, no initial contents;
 * NULL allowed): with at least hba_hier_select_workspace_bytes bytes, the
 * bf16 descent scores its second level per group of a few hundred queries
 * (each super's children loaded once for the group's queries that kept it);
 * otherwise per 64-query tile.  The same picks either way.
 */
int hba_hier_select(int dtype, const void *q, const int64_t q_strides[3],
                    const float *q_gain, float eps, const void *S0, const void *S1,
                    int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                    int64_t m, int64_t Bk, int64_t W, int64_t k, int64_t fanout,
                    int64_t beam, float scale, int32_t *idx, float *val, int32_t *cnt,
                    float *scores, float *sup_scores, void *workspace, size_t ws_bytes,
                    void *stream);

/* Workspace bytes hba_hier_select can use for this geometry: bf16 with m == 4,
 * k <= 32, fanout 4, 8 or 16 and min(beam, ns) * fanout <= 256, the routing
 * queries (B*Hkv*n*d bf16) and the kept supers (B*Hkv*n*16 int16); 0 where
 * the grouped second level does not apply. */
int hba_hier_select_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                                    int64_t d, int64_t m, int64_t k, int64_t fanout, int64_t beam,
                                    size_t *bytes);

/*
 * Routing queries: qg [B, n, Hkv, d] (contiguous, storage dtype) = per KV
 * group, the sum of QKNorm(q) over its Hq/Hkv heads, in the declared order
 * and storage roundings the selection kernels use (QKNorm skipped when q_gain
 * is NULL).  qg is a valid q for hba_score_select / hba_hier_select with
 * Hq = Hkv and q_gain = NULL, which then select exactly as on q itself.
 *   replaces: grouped_query  src/hba/summarizer.py:50-54 applied to the
 *             QKNorm'd queries (_HeadRMSNorm, src/hba/attention.py:88-94)
 * bf16: d 64 or 128, Hq/Hkv <= 16; fp32: any even d <= 256, any Hq/Hkv
 * (other than d 64 / 128 with Hq/Hkv <= 16: a generic one-thread-per-row
 * kernel, same order).
 */
int hba_route_queries(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
                      float eps, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d, void *qg,
                      void *stream);

/*
 * hier_select with the reference's own signature and an arbitrary candidate
 * mask: qn [B, c, d] routing queries (already grouped and QKNorm'd, as the
 * reference's eval path passes them), S0 [B, nb, m, d], S1 [B, ns, m, d] with
 * ns = ceil(nb / fanout), cand uint8 [c, nb] (nonzero = candidate).  Writes
 * top_idx int64 / top_val fp32 [B, c, kk_eff], kk_eff = min(kk, min(beam, ns)
 * * fanout): the picks in order (score desc, block asc), then -1 / -inf.
 * Scores are fp32 in the declared order (dot in index order, slot max, times
 * scale), also for bf16 inputs.
 *   replaces: hier_select  src/hba/attention.py:217-246 (called by
 *             evals.hier_fidelity, src/hba/evals.py:314)
 * d <= 256, ns <= 4096, min(beam, ns) <= 64, min(beam, ns) * fanout <= 1024.
 */
int hba_hier_select_rows(int dtype, const void *qn, const void *S0, const void *S1,
                         const uint8_t *cand, int64_t B, int64_t c, int64_t nb, int64_t m,
                         int64_t d, int64_t fanout, int64_t beam, int64_t kk, float scale,
                         int64_t *top_idx, float *top_val, void *stream);

/*
 * Union attention forward: one softmax per (query, head) over the NoPE sinks
 * j < min(S, i+1), the RoPE window max(S, i-W+1) <= j <= i, and the NoPE keys
 * of the valid selected blocks idx[b, h/G, i, 0..cnt).
 *   replaces: hba_attention_dense forward  src/hba/attention.py:306-356
 *             hba_attention_eval           src/hba/attention.py:610-713
 *             hba_attention_fused forward  src/hba/attention.py:552-603
 * q is the raw query (QKNorm and RoPE are applied in the kernel); kc, kr, vt
 * come from hba_prep_keys.  `scale` is the union scale (content scale times
 * the log-length temperature).  k_gain (the gains hba_prep_keys applied; NULL
 * if none) lets the kernel bound the logits by d*max(q_gain)*k_gain*scale
 * and use that bound as the softmax shift.  out [B, n, Hq, d] with
 * out_strides.  Requires n % Bk == 0.  A routed block's keys below S are
 * sinks and count once, as the union mask of hba_attention_dense counts
 * them (src/hba/attention.py:351-352).  bf16: Bk == 64, d in {64, 128},
 * S <= 128.  fp32: any S; d 64 / 128 with Bk 64 on the tuned kernel,
 * otherwise any even d <= 256 and Bk <= 256 on the generic one.
 */
int hba_attn_fwd(int dtype, const void *q, const int64_t q_strides[3],
                 const float *q_gain, const float *k_gain, float eps,
                 const void *kc, const void *kr, const void *vt,
                 const float *cos_tab, const float *sin_tab,
                 const int32_t *idx, const int32_t *cnt,
                 int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                 int64_t S, int64_t W, int64_t Bk, int64_t k, float scale,
                 void *workspace, size_t ws_bytes,
                 void *out, const int64_t out_strides[3], void *stream);

/* Scratch bytes hba_attn_fwd needs: bf16, the RoPE query operand of the
 * window tiles, B*n*Hq*d bf16 (rounded up to 256 bytes; the one launch
 * parks it between its routed blocks and its window tiles); fp32, none.
 * workspace must be 16-byte aligned; no initial contents. */
int hba_attn_fwd_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t d, size_t *bytes);

/* Scratch bytes of the split launches below (bf16: the window's LSE,
 * B*Hq*n fp32; fp32: none).  workspace must be 16-byte aligned. */
int hba_attn_workspace_size(int dtype, int64_t B, int64_t n, int64_t Hq, size_t *bytes);

/*
 * The bf16 union attention as two launches, for callers that run the window
 * (which needs no selection) concurrently with summarisation and selection
 * on another stream.  Same arguments and checks as hba_attn_fwd (bf16 only);
 * workspace sized by hba_attn_workspace_size.
 *   hba_attn_window_fwd: the RoPE window region
 *     (attention.py:342-356 window term); writes its normalised rows into
 *     out and their log-sum-exp into workspace.
 *   hba_attn_routed_fwd: the sinks and the routed blocks (the rest of the
 *     union softmax), merged by LSE into out.  It must be ordered after
 *     hba_attn_window_fwd on the same out and workspace (same stream, or an
 *     event wait).
 * The same softmax as hba_attn_fwd's one launch, except that the window rows
 * are rounded to bf16 once before the merge.
 */
int hba_attn_window_fwd(const void *q, const int64_t q_strides[3],
                        const float *q_gain, const float *k_gain, float eps,
                        const void *kr, const void *vt,
                        const float *cos_tab, const float *sin_tab,
                        int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                        int64_t S, int64_t W, int64_t Bk, float scale,
                        void *workspace, size_t ws_bytes,
                        void *out, const int64_t out_strides[3], void *stream);
int hba_attn_routed_fwd(const void *q, const int64_t q_strides[3],
                        const float *q_gain, const float *k_gain, float eps,
                        const void *kc, const void *vt,
                        const int32_t *idx, const int32_t *cnt,
                        int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                        int64_t S, int64_t Bk, int64_t k, float scale,
                        void *workspace, size_t ws_bytes,
                        void *out, const int64_t out_strides[3], void *stream);

/*
 * Paged KV cache (decode).  Page = Bk = 64 tokens of one sequence; all
 * tensors page-major:  kc_pages [P, Hkv, 64*d] (QKNorm'd NoPE keys), kr_pages
 * [P, Hkv, 64*d] (the same keys rotated at their own positions: hba_prep_keys'
 * kr), v_pages [P, Hkv, 64*d] (values), summ_pages [P, Hkv, m, d] (slot
 * summaries of full pages);
 * page_table int32 [Bd, max_pages] (logical page -> physical page);
 * seq_lens int32 [Bd] (tokens already in the cache, including the current one).
 * Within a page and KV head, token j's element t lies at
 *   keys:   ((mt * (d/32) + t/32) * 64 + l16 + 16 * ((t%32)/8)) * 8 + t%8,
 *           mt = 2*(j/32) + (j/4)%2, l16 = 4*((j%32)/8) + j%4;
 *   values: (((t/16) * 2 + j/32) * 64 + t%16 + 16 * ((j%32)/8)) * 8 + j%8,
 * the order in which the decode kernel's MFMA tiles read them (each operand
 * load of a wave is one contiguous 1 KB run).
 * There is no reference function for these: the decode step is defined as row
 * L-1 of hba_attention_eval (src/hba/attention.py:610-713) for a sequence of
 * length L.
 */

/*
 * Append one token per sequence at position pos = seq_lens[s]-1: QKNorm of
 * k_new into kc_pages and its rotation at pos (as hba_prep_keys) into
 * kr_pages, v_new into v_pages.  k_new, v_new [Bd, Hkv, d] contiguous;
 * cos_tab/sin_tab fp32 [n_tab, d] (a position >= n_tab is not appended).
 * k_gain == NULL means qknorm=False.
 */
int hba_kv_append(int dtype, const void *k_new, const void *v_new, const float *k_gain,
                  float eps, const float *cos_tab, const float *sin_tab, int64_t n_tab,
                  const int32_t *page_table, int64_t max_pages, const int32_t *seq_lens,
                  int64_t Bd, int64_t Hkv, int64_t d, int64_t Bk, void *kc_pages,
                  void *kr_pages, void *v_pages, void *stream);

/*
 * The decode loop's append, one launch: for each sequence s, the token goes
 * to position pos = seq_lens[s] (QKNorm, rotation and writes as
 * hba_kv_append); when it fills its page (pos % Bk == Bk-1) that page's slot
 * summaries are written (as hba_summarize_pages); then seq_lens[s] becomes
 * pos+1 and, when scales is not NULL, scales[s] = scale_tab[pos+1] (a table
 * of the step scale by length, n_scale entries, the last one used past its
 * end).  A position outside the page table or at/after n_tab appends nothing
 * and leaves seq_lens[s] (scales[s] is still written).  seq_lens is read and
 * written on the device, so a decode loop of this and hba_decode_fwd needs no
 * host round trip per token and can be captured in a graph.  No counterpart
 * in the reference, which has no KV cache.
 */
int hba_kv_append_advance(int dtype, const void *k_new, const void *v_new, const float *k_gain,
                          float eps, const float *cos_tab, const float *sin_tab, int64_t n_tab,
                          const int32_t *page_table, int64_t max_pages, int32_t *seq_lens,
                          int64_t Bd, int64_t Hkv, int64_t d, int64_t Bk, void *kc_pages,
                          void *kr_pages, void *v_pages, const float *probes, const float *proj,
                          int64_t m, void *summ_pages, const float *scale_tab, int64_t n_scale,
                          float *scales, void *stream);

/*
 * Slot summaries of the listed physical pages (SlotSummarizer.summarize on
 * one block each): pages int32 [npages]; writes summ_pages[pages[i]].
 */
int hba_summarize_pages(int dtype, const void *kc_pages, const int32_t *pages,
                        int64_t npages, int64_t Hkv, int64_t d, int64_t Bk,
                        const float *probes, const float *proj, int64_t m,
                        void *summ_pages, void *stream);

/*
 * Slot summaries of the pages the last append filled, found on the device:
 * for each sequence s whose seq_lens[s] is a positive multiple of Bk, the
 * page page_table[s][seq_lens[s]/Bk - 1] (SlotSummarizer.summarize on that
 * block, src/hba/summarizer.py:34-42); other sequences are left alone.  No
 * host-side page list, so a decode loop that appends on the device (and a
 * captured graph of it) needs no host round trip.  No counterpart in the
 * reference, which has no KV cache.
 */
int hba_summarize_filled(int dtype, const void *kc_pages, const int32_t *page_table,
                         int64_t max_pages, const int32_t *seq_lens, int64_t Bd, int64_t Hkv,
                         int64_t d, int64_t Bk, const float *probes, const float *proj, int64_t m,
                         void *summ_pages, void *stream);

/*
 * The summarizer auxiliary loss of the training path (aux-KL,
 * hba_attention_dense src/hba/attention.py:366-389; the fused path's chunked
 * teacher :478-549, the same value) and, when dprobes / dproj are given, its
 * gradient with respect to the summarizer's probes [Hkv, m, d] and proj
 * [Hkv, d, d] (fp32; the only gradient it has: the routing runs on detached
 * q/k, so nothing flows into q, k or v).
 *   q       [B, n, Hq, d] raw queries (element strides; QKNorm'd inside with
 *           q_gain, NULL = qknorm off); k_gain the keys' QKNorm gains (NULL
 *           when off: they bound the logits); kc [B, Hkv, n, d] content keys and
 *           S0 [B, Hkv, n/Bk, m, d] their summaries (hba_prep_keys,
 *           hba_summarize);
 *   scale_u the union scale of the teacher's content logits (_content_qk),
 *   scale_r route_topk's scale of the block scores;
 *   aux     one fp32 on the device: -mean over (batch, KV head, queries with
 *           a candidate block) of sum_b p*_b log softmax_b(bsc), 0 when no
 *           query has a candidate.
 * Work is O(n^2 d) (the teacher scores every candidate key).  ws: at least
 * hba_aux_kl_workspace_size bytes, 16-byte aligned, no initial contents.
 * Every reduction runs in a fixed order (deterministic).  bf16: Bk = 64,
 * d = 64 / 128, m <= 8, Hq / Hkv <= 16.  fp32 also takes any block size
 * 1..256 dividing n, even d <= 256, m <= 32 and Hq / Hkv <= 64 (scalar
 * kernels in the oracle's arithmetic, one thread per query row).
 */
int hba_aux_kl_workspace_size(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                              int64_t m, int64_t Bk, size_t *bytes);
int hba_aux_kl(int dtype, const void *q, const int64_t q_strides[3], const float *q_gain,
               const float *k_gain, float eps,
               const void *kc, const void *S0, const float *probes, const float *proj, int64_t B,
               int64_t n, int64_t Hq, int64_t Hkv, int64_t d, int64_t m, int64_t Bk, int64_t W,
               float scale_u, float scale_r, void *ws, size_t ws_bytes, float *aux,
               float *dprobes, float *dproj, void *stream);

/*
 * Scratch bytes hba_decode_fwd needs for these sizes (max_len = max seq_len).
 * The workspace must be zero-filled before its first call: it opens with
 * per-(sequence, KV head) completion counters of the one-launch bf16 step,
 * which every call leaves zero again, so a workspace is reused as is by later
 * calls on the same stream (calls that overlap on it race).
 */
int hba_decode_workspace_size(int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d, int64_t k,
                              int64_t Bk, int64_t W, int64_t max_len, size_t *bytes);

/*
 * Decode step: for each sequence s of length L = seq_lens[s], the union
 * attention of its new query q[s] (raw; QKNorm and RoPE at position L-1 are
 * applied in the kernel) over the cached keys, with flat top-k selection
 * over the full pages that lie before the window.  scales fp32 [Bd] holds
 * each sequence's union scale (content scale times the temperature at n=L).
 * out [Bd, Hq, d].  Optional sel_idx int32 [Bd, Hkv, k] / sel_cnt
 * int32 [Bd, Hkv] receive the selection (NULL to skip).  max_len bounds
 * every seq_lens[s] (a longer length is read as max_len); cos_tab/sin_tab
 * fp32 [>= max_len, d].
 */
int hba_decode_fwd(int dtype, const void *q, const float *q_gain, float eps,
                   const void *kc_pages, const void *kr_pages, const void *v_pages,
                   const void *summ_pages, const int32_t *page_table, int64_t max_pages,
                   const int32_t *seq_lens, const float *cos_tab, const float *sin_tab,
                   const float *scales, int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d,
                   int64_t m, int64_t S, int64_t W, int64_t Bk, int64_t k, int64_t max_len,
                   void *workspace, size_t ws_bytes, void *out,
                   int32_t *sel_idx, int32_t *sel_cnt, void *stream);

/*
 * hba_decode_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, which
 * has no decode path.  The workspace is a fixed device array of
 * HBA_DECODE_SCRATCH_BYTES per GPU, held until the process ends; a call whose
 * hba_decode_workspace_size exceeds it returns HBA_ERR_SCRATCH and launches
 * nothing (32 sequences of 32K tokens at 14/2 heads, d = 64, k = 16 need
 * 4.8 MB).  The call allocates nothing.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (e.g. on two streams) race;
 * consecutive calls on one stream are safe.  Same arguments, checks and
 * results as hba_decode_fwd otherwise.
 */
#define HBA_DECODE_SCRATCH_BYTES (16u << 20)
int hba_decode_fwd_noalloc(int dtype, const void *q, const float *q_gain, float eps,
                           const void *kc_pages, const void *kr_pages, const void *v_pages,
                           const void *summ_pages, const int32_t *page_table, int64_t max_pages,
                           const int32_t *seq_lens, const float *cos_tab, const float *sin_tab,
                           const float *scales, int64_t Bd, int64_t Hq, int64_t Hkv, int64_t d,
                           int64_t m, int64_t S, int64_t W, int64_t Bk, int64_t k, int64_t max_len,
                           void *out, int32_t *sel_idx, int32_t *sel_cnt, void *stream);

/*
 * Backward of the union attention (replaces the autograd backward of
 * hba_attention_dense / hba_attention_fused, src/hba/attention.py:306-356,
 * 552-607; the routing is on detached q/k there, :288-303, so the selection
 * idx/cnt is an input and gets no gradient).  Given the forward's raw q
 * [B, n, Hq, d], k, v [B, n, Hkv, d], its prepared keys kc, kr [B, Hkv, n, d]
 * (hba_prep_keys), its selection, its output out and the output cotangent
 * dout [B, n, Hq, d] (all contiguous, storage dtype), writes dq, dk, dv
 * (contiguous, storage dtype) and ADDS the QKNorm gain gradients into
 * dq_gain fp32 [Hq] and dk_gain fp32 [Hkv] (q_gain == NULL: no QKNorm, the
 * gain outputs are ignored).  scale is the union scale of the forward.
 * fp32 storage: fp32 VALU arithmetic.  bf16 storage: bf16 MFMA products
 * with fp32 accumulation; the probabilities and dS enter the dk/dv/dq
 * products rounded to bf16, and dk/dv are summed with fp32 atomics, so the
 * bf16 result is not bit-reproducible from run to run.  bf16: 64-key
 * blocks, d = 64 / 128, S <= 64, k <= 64, G = Hq/Hkv <= 16.  fp32 takes every
 * geometry the fp32 forward takes (any block size Bk dividing n up to 256,
 * even d <= 256, any S, k and G): off the tuned one, one thread per (query,
 * head) recomputes the union softmax and the key sides are summed with fp32
 * atomics (not bit-reproducible either); its workspace is three fp32
 * [B, Hkv, n, d] accumulators, included in hba_attn_bwd_workspace_bytes.
 */
int hba_attn_bwd(int dtype, const void *q, const void *k, const void *v,
                 const void *kc, const void *kr,
                 const float *q_gain, const float *k_gain, float eps,
                 const float *cos_tab, const float *sin_tab,
                 const int32_t *idx, const int32_t *cnt,
                 const void *out, const void *dout,
                 int64_t B, int64_t n, int64_t Hq, int64_t Hkv, int64_t d,
                 int64_t S, int64_t W, int64_t Bk, int64_t k_blocks, float scale,
                 void *workspace, size_t ws_bytes,
                 void *dq, void *dk, void *dv, float *dq_gain, float *dk_gain, void *stream);

/* Scratch bytes hba_attn_bwd needs for this dtype and Hkv: the QKNorm'd and
 * rotated query rows (2*B*n*Hq*d in the storage type), the per-row LSE and
 * <dout, out> (2*B*Hq*n fp32), the sink-key accumulators (2*B*Hkv*64*d
 * fp32); on the bf16 path also the transposed prepared keys (2*B*Hkv*n*d
 * bf16), the dk/dv accumulators (3*B*Hkv*n*d fp32) and the routed-row bits
 * (B*Hkv*ceil(n/4096)*(n/64)*512 bytes: one bit per query row of each
 * 4096-row range and key block); each part rounded up to 256 bytes. */
int hba_attn_bwd_workspace_bytes(int dtype, int64_t B, int64_t n, int64_t Hq, int64_t Hkv,
                                 int64_t d, size_t *bytes);

/* An upper bound of hba_attn_bwd_workspace_bytes over both dtypes and every
 * Hkv <= Hq (for callers that size one workspace for any call). */
int hba_attn_bwd_workspace_size(int64_t B, int64_t n, int64_t Hq, int64_t d, size_t *bytes);

#ifdef __cplusplus
}
#endif

#endif /* HBA_AMD_H */
