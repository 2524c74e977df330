/*
 * ssa_hip.h -- C ABI of libssa_hip.so, the MI355X (gfx950) implementation of
 * the SSA forward hot path (codebook routing, inverted index, candidate
 * selection, gathered exact attention).
 *
 * Conventions
 *   - Every pointer is device memory owned by the caller (the PyTorch caching
 *     allocator in ssa_amd).  The library allocates nothing and never
 *     synchronises: each call enqueues kernels on `stream` (a hipStream_t;
 *     NULL = the default stream) and returns.
 *   - Strides are in ELEMENTS; the last (feature) dimension is contiguous.
 *   - Every function returns SSA_OK (0) or an error status; argument checks run
 *     on the host before any launch.  ssa_last_error() gives the detail of the
 *     last failure on the calling thread.
 *   - Selections are bit-exact with the CPU oracle (oracle/ssa_oracle.c):
 *     fp32 scoring in one canonical fmaf order, ties to the lowest index.
 *
 * Reference interfaces replaced (chenxingqiang/SSA):
 *   CodebookRouter.forward        ssa/router.py:73-149
 *     _select_candidates          ssa/router.py:151-214
 *     _build_candidate_mask       ssa/router.py:216-259
 *     get_code_assignment         ssa/router.py:261-275
 *   sparse_exact_attention        ssa/attention.py:12-115
 */
#ifndef SSA_HIP_H
#define SSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define SSA_OK 0
#define SSA_ERR_INVALID_ARGUMENT 1
#define SSA_ERR_UNSUPPORTED 2
#define SSA_ERR_WORKSPACE 3
#define SSA_ERR_HIP 4

/* element types of q / k / v / attention output */
#define SSA_DTYPE_F32 0
#define SSA_DTYPE_BF16 1

/* index element types */
#define SSA_INDEX_I32 0
#define SSA_INDEX_I64 1

/* candidate masks for ssa_select */
#define SSA_MASK_NONE 0   /* causal_mask=None: every key is eligible            */
#define SSA_MASK_CAUSAL 1 /* build_causal_mask(n): key j eligible iff j <= i     */
#define SSA_MASK_DENSE 2  /* any bool [n][n] mask: eligible iff mask[i][j] != 0  */

int ssa_version(void);
const char* ssa_status_str(int status);
const char* ssa_last_error(void);

/* rotary-embedding angle rows for ssa_rope */
#define SSA_ROPE_BY_POSITION 0 /* table row = token position (Hugging Face Qwen2)        */
#define SSA_ROPE_BY_HEAD 1     /* table row = head index (SSAAttention's apply_rope call) */

/* ---- layer prologue: rotary embedding ----------------------------------- */

/* Rotary embedding of q or k rows: features j < rot rotate in pairs
 * (j, j + rot/2), out = x * cos + rotate_half(x) * sin, and features j >= rot
 * pass through.  Replaces apply_rope (ssa/utils.py:7-41) as SSAAttention calls
 * it on [n, heads, d] per batch element (ssa/ssa_layer.py:115-120: rot = d/2,
 * angle row = head index, table freqs[:, :d/2]) and Hugging Face's
 * apply_rotary_pos_emb in the Qwen2 path (training/train_qwen.py:134-135:
 * rot = d, angle row = position, the model's cos/sin tables).
 *   x   [batch][n][h][d] strides (x_sb, x_sn, x_sh), type dtype
 *   cos_table, sin_table  [batch or 1][table_rows][>= rot], row stride t_sr,
 *       batch stride t_sb (0 = one table for every batch element), type table_dtype
 *   angle_axis  SSA_ROPE_BY_POSITION (row = token i) or SSA_ROPE_BY_HEAD (row = head)
 *   inverse != 0 applies the transpose of the rotation (the backward)
 *   out [batch][n][h][d] strides (o_sb, o_sn, o_sh), type out_dtype; out == x
 *       (same strides and type) rotates in place and leaves features >= rot alone.
 * Arithmetic matches torch's ops: bf16 x with bf16 tables rounds every product
 * and the sum to bf16; otherwise fp32 intermediates, the result rounded once. */
int ssa_rope(const void* x, int dtype, int64_t batch, int64_t n, int h, int d, int64_t x_sb,
             int64_t x_sn, int64_t x_sh, const void* cos_table, const void* sin_table,
             int table_dtype, int64_t t_sb, int64_t t_sr, int64_t table_rows, int rot,
             int angle_axis, int inverse, void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
             int64_t o_sh, void* stream);

/* ---- stage (a): routing ------------------------------------------------- */

/* Routing vectors: out[b][h][i] = normalize(mean_{gg<group}(x[b][i][h*group+gg] . w^T)).
 * Replaces the W_qr / W_kr projection, the GQA mean and F.normalize of
 * ssa/router.py:102-117 (group = h_q/h_kv for queries, 1 for keys).
 *   x   [batch][n][h_in][d]  strides (x_sb, x_sn, x_sh)
 *   w   fp32 [d_s][d] contiguous (nn.Linear weight)
 *   out fp32 [batch][h_in/group][n][d_s] contiguous */
int ssa_route_vectors(const void* x, int dtype, int64_t batch, int64_t n, int h_in, int group,
                      int d, int64_t x_sb, int64_t x_sn, int64_t x_sh, const float* w, int d_s,
                      float* out, void* stream);

/* Row-wise F.normalize(x, dim=-1) of a fp32 [rows][d_s] matrix (the codebook,
 * ssa/router.py:118). */
int ssa_normalize_rows(const float* x, int64_t rows, int d_s, float* out, void* stream);

/* Codebook scoring and top-`top` codes per row (score desc, code asc).
 * Replaces einsum("shd,hcd->shc") / temperature and topk of ssa/router.py:121-130
 * (keys, top = b) and :141 (queries, top = a).
 *   xhat  fp32 [batch][h][rows][d_s]; chat fp32 [h][n_c][d_s]
 *   codes int32 [batch][h][rows][top]
 * With a workspace (ssa_code_topk_workspace_bytes) and top <= 32, d_s <= 32,
 * scores are screened on the matrix cores (bf16) with a proven error bound and
 * the survivors rescored exactly; workspace = NULL scores every code exactly.
 * Both give identical codes. */
size_t ssa_code_topk_workspace_bytes(int64_t batch, int h, int64_t rows, int n_c);
int ssa_code_topk(const float* xhat, int64_t batch, int h, int64_t rows, const float* chat,
                  int n_c, int d_s, float temperature, int top, int32_t* codes, void* workspace,
                  size_t workspace_bytes, void* stream);

/* Stage (a) end to end: q_codes = top-a query codes, k_codes = top-b key codes.
 * Replaces ssa/router.py:102-141.  The workspace holds the normalized routing
 * vectors and codebook (ssa_route_workspace_bytes).
 *   q [batch][n][h_q][d], k [batch][n][h_kv][d]; codebook fp32 [h_kv][n_c][d_s]
 *   q_codes int32 [batch][h_kv][n][a]; k_codes int32 [batch][h_kv][n][b] */
size_t ssa_route_workspace_bytes(int64_t batch, int64_t n, int h_kv, int n_c, int d_s);
int ssa_route_codes(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int h_q,
                    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                    int64_t k_sn, int64_t k_sh, const float* w_qr, const float* w_kr,
                    const float* codebook, int d_s, int n_c, int a, int b, float temperature,
                    int32_t* q_codes, int32_t* k_codes, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ---- stage (b): inverted index ------------------------------------------ */

/* Bucket c of head h lists every key j with c in k_codes[b][h][j][:], ascending.
 * No reference counterpart: it replaces the O(n^2) broadcast compare of
 * _build_candidate_mask (ssa/router.py:241-257) and reproduces its set.
 *   offsets  int32 [batch][h_kv][n_c+1]; postings int32 [batch][h_kv][n*b] */
size_t ssa_index_workspace_bytes(int64_t batch, int64_t n, int h_kv, int b, int n_c);
int ssa_build_index(const int32_t* k_codes, int64_t batch, int64_t n, int h_kv, int b, int n_c,
                    int32_t* offsets, int32_t* postings, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Processing order for ssa_sparse_attention's row_order: the query positions of
 * each (batch, kv head) sorted by their smallest code min_t q_codes[b][h][i][t]
 * (stable, so ascending positions within a code).  Rows that share that code
 * share its bucket and much of their candidates, so processing them together
 * keeps the gathered K/V rows in cache.
 * No reference counterpart (the reference has no processing order; results do
 * not depend on it).  q_codes must lie in [0, n_c), as ssa_route_codes writes.
 *   q_codes int32 [batch][h_kv][n][a]; order int32 [batch][h_kv][n] */
size_t ssa_query_order_workspace_bytes(int64_t batch, int64_t n, int h_kv, int n_c);
int ssa_query_order(const int32_t* q_codes, int64_t batch, int64_t n, int h_kv, int a, int n_c,
                    int32_t* order, void* workspace, size_t workspace_bytes, void* stream);

/* ---- stage (c): candidate selection ------------------------------------- */

/* Top-k candidate keys per (query, kv head): union of the query's a buckets,
 * masked, deduplicated, rescored as mean_g(q.k / score_div) in fp32, ranked
 * (score desc, index asc); fewer than k candidates are followed by the lowest
 * non-candidate indices; k > n pads with 0.  Replaces
 * CodebookRouter._select_candidates (ssa/router.py:151-214).
 *   sorted != 0: selected keys by (score desc, index asc), as torch.topk orders
 *                them; sorted == 0: the same set, selected keys ascending (rows
 *                with at most k candidates then need no rescoring).  The filler
 *                and padding are the same in both orders.
 *   out    [batch][n][h_kv][top_k], index type out_index_dtype
 *   mask   (SSA_MASK_DENSE only) uint8 [batch][n][n], strides (mask_sb, mask_si); mask_sb may be 0
 *   stats  (nullable) int32 [batch][h_kv][n][2] = (candidates, postings read
 *          inside the mask window: j <= i when causal, all otherwise)
 *   row_prefix (nullable) int32 [batch][h_kv][n]: X per row such that the
 *          row's indices hold each key of [0, X) exactly once -- the last
 *          filler key + 1 for a row with filler, 0 otherwise (and 0 with k > n
 *          padding).  ssa_sparse_attention takes it to attend those keys in a
 *          dense pass.  No reference counterpart.
 *   workspace (nullable): with it, index order runs one wave per row; a row
 *          with more than k candidates leaves its candidate list in the
 *          workspace, which bf16 inputs with d = 64 or 128 then screen on the
 *          matrix cores (approximate scores with a proven error bound; only the
 *          keys near the k-th score are rescored exactly), and the remaining
 *          such rows (lists that do not fit, other types) take an exact
 *          one-block-per-row pass.  ssa_select_workspace_bytes(.., top_k) is
 *          the recommended size, (.., 0) the minimum (no lists).  Without a
 *          workspace, one block per row.  Results are identical in every case.
 *   row_order (nullable) int32 [batch][h_kv][n]: the order in which query rows
 *          are processed, as for ssa_sparse_attention (ssa_query_order groups
 *          rows that share buckets and candidate keys, which then hit in
 *          cache).  Results do not depend on it; a row never listed is not
 *          written and an entry outside [0, n) is skipped.
 * Limits: top_k <= 4096, g = h_q/h_kv <= 16, d <= 256 (d % 8 == 0), n < 2^31. */
size_t ssa_select_workspace_bytes(int64_t batch, int64_t n, int h_kv, int top_k);

/* Where ssa_select places its regions inside a workspace of workspace_bytes
 * (no reference counterpart; for tests and for callers that size or share
 * workspaces).  layout[11] receives byte offsets of the counter block, the
 * exact-pass row list, the screened-row entries, the per-row error bounds,
 * the candidate lists and their approximate scores, then the entries per
 * shard, the list entries per shard (0 = no screen), the shard count, the
 * counter block's size and the offset of the per-row candidate counts (one
 * int32 per row, between the error bounds and the lists).  Nothing is
 * launched or dereferenced. */
int ssa_select_workspace_layout(int64_t batch, int64_t n, int h_kv, size_t workspace_bytes,
                                int screen, int64_t* layout);

int ssa_select(const void* q, const void* k, int dtype, int64_t batch, int64_t n, int h_q,
               int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
               int64_t k_sn, int64_t k_sh, const int32_t* q_codes, int a, const int32_t* offsets,
               const int32_t* postings, int n_c, int b, int top_k, int mask_mode,
               const uint8_t* mask, int64_t mask_sb, int64_t mask_si, float score_div, int sorted,
               const int32_t* row_order, void* out, int out_index_dtype, int32_t* stats,
               int32_t* row_prefix, void* workspace, size_t workspace_bytes, void* stream);

/* ssa_select for a block of n_q query rows at key positions q_pos0 .. q_pos0 +
 * n_q - 1 against all n keys (0 <= q_pos0, q_pos0 + n_q <= n): q, q_codes,
 * out, stats and row_order hold n_q rows ([batch][n_q]..., [batch][h_kv][n_q]...);
 * the causal window and the dense mask use the key position.  n_q = n with
 * q_pos0 = 0 is ssa_select.  No reference counterpart: it serves incremental
 * decoding (new tokens against a key cache, ssa_design.md:225-234) and chunked
 * prefill.  Workspace: ssa_select_workspace_bytes(batch, n_q, h_kv, top_k). */
int ssa_select_block(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                     int64_t n_q, int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb,
                     int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh,
                     const int32_t* q_codes, int a, const int32_t* offsets,
                     const int32_t* postings, int n_c, int b, int top_k, int mask_mode,
                     const uint8_t* mask, int64_t mask_sb, int64_t mask_si, float score_div,
                     int sorted, const int32_t* row_order, void* out, int out_index_dtype,
                     int32_t* stats, int32_t* row_prefix, void* workspace, size_t workspace_bytes,
                     void* stream);

/* ssa_select_block without a workspace argument: no counterpart in the
 * reference; for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  The workspace is a static
 * device array of ssa_select_noalloc_scratch_bytes() bytes (64 MiB) that the
 * library holds on every device it runs on until the process ends; the call
 * allocates nothing and uses min(that, ssa_select_workspace_bytes(batch, n_q,
 * h_kv, top_k)) of it (rows whose candidate lists do not fit take the exact
 * pass, with identical results).  Shapes whose minimum workspace
 * (ssa_select_workspace_bytes(batch, n_q, h_kv, 0), about 20 bytes per
 * (batch, query row, kv head)) exceeds the array are rejected with
 * SSA_ERR_WORKSPACE.  Every call on one device shares the array: calls that
 * overlap on one device (other streams, other threads) race. */
size_t ssa_select_noalloc_scratch_bytes(void);
int ssa_select_block_noalloc(const void* q, const void* k, int dtype, int64_t batch, int64_t n,
                             int64_t n_q, int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb,
                             int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh,
                             const int32_t* q_codes, int a, const int32_t* offsets,
                             const int32_t* postings, int n_c, int b, int top_k, int mask_mode,
                             const uint8_t* mask, int64_t mask_sb, int64_t mask_si,
                             float score_div, int sorted, const int32_t* row_order, void* out,
                             int out_index_dtype, int32_t* stats, int32_t* row_prefix, void* stream);

/* ---- incremental decoding ----------------------------------------------- */

/* One decoding step for m new tokens against a key/value cache: no reference
 * counterpart (the reference runs whole sequences; ssa_design.md:225-234
 * describes decode-time routing against the cached keys' inverted index,
 * "maintained incrementally, avoiding re-scanning the full KV cache").
 * The caller owns the cache state:
 *   k_cache, v_cache [batch][max_len][h_kv][d] (strides kc_*, vc_*), holding
 *       n0 tokens; the step writes the new rows at n0 .. n0 + m - 1;
 *   k_codes int32 [batch][h_kv][max_len][b]: the keys' codes (written likewise);
 *   offsets/postings: an ssa_build_index index over keys 0 .. n_base - 1
 *       ([batch][h_kv][n_c + 1], [batch][h_kv][n_base * b]; n_base <= n0);
 *   tail_offsets int32 [batch][h_kv][n_c + 1], tail_postings int32
 *       [batch][h_kv][tail_cap]: rebuilt by the step over keys n_base ..
 *       n0 + m - 1 ((n0 + m - n_base) * b <= tail_cap, else SSA_ERR_WORKSPACE:
 *       rebuild the main index over every cached key and start a new tail);
 *   prep: the codebook prepared by ssa_decode_prepare (normalized rows, their
 *       bf16 copy and largest norm; prepare again when the codebook changes).
 * q [batch][m][h_q][d], k, v [batch][m][h_kv][d] (strided) are the new tokens.
 * The step routes them (top-a query and top-b key codes), selects each new
 * query's top_k keys among all cached keys from both indices (causal, index
 * order, the same selection as ssa_select_block over the whole cache) into
 * indices (nullable int32 [batch][m][h_kv][top_k]) and attends them
 * (ssa_sparse_attention_block; causal != 0 drops selected keys past the
 * query) into out [batch][m][h_q][d] (strides o_*, type out_dtype).  Limits
 * as the stages', plus a <= 32, d_s <= 32, n_c <= 16384, rows of 16 bytes. */
size_t ssa_decode_prepare_bytes(int h_kv, int n_c, int d_s);
int ssa_decode_prepare(const float* codebook, int h_kv, int n_c, int d_s, void* prep,
                       size_t prep_bytes, void* stream);
size_t ssa_decode_workspace_bytes(int64_t batch, int64_t m, int h_kv, int d_s, int n_c, int a,
                                  int b, int top_k);
int ssa_decode_step(const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t m,
                    int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
                    int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh,
                    void* k_cache, void* v_cache, int64_t max_len, int64_t kc_sb, int64_t kc_sn,
                    int64_t kc_sh, int64_t vc_sb, int64_t vc_sn, int64_t vc_sh, int64_t n0,
                    const float* w_qr, const float* w_kr, const void* prep, int d_s, int n_c, int a,
                    int b, float temperature, int32_t* k_codes, const int32_t* offsets,
                    const int32_t* postings, int64_t n_base, int32_t* tail_offsets,
                    int32_t* tail_postings, int64_t tail_cap, int top_k, float score_div,
                    float scale_div, int causal, int32_t* indices, void* out, int out_dtype,
                    int64_t o_sb, int64_t o_sn, int64_t o_sh, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- stage (d): gathered exact attention -------------------------------- */

/* out[b][i][hq] = softmax_m(q[b][i][hq] . k[b][idx[b][i][h][m]][h] / scale_div) . v[...]
 * with h = hq / (h_q/h_kv).  Replaces sparse_exact_attention (ssa/attention.py:12-115):
 * `scale_div` is the reference's `scale` (a divisor); duplicates count twice.
 * causal != 0 drops slots with idx > i (a row with no slot left outputs zeros).
 * Indices outside [0, n) are dropped and set *error_flag (nullable) to 1.
 * row_order (nullable) int32 [batch][h_kv][n]: a permutation of 0..n-1 per
 *   (batch, kv head) giving the order in which query rows are processed (e.g.
 *   grouped by routing code so that rows sharing candidates run together and
 *   hit in cache).  Results do not depend on it; a row never listed is not
 *   written, and an entry outside [0, n) is skipped and sets *error_flag.
 *   idx [batch][n][h_kv][top_k] strides (idx_sb, idx_sn, idx_sh)
 *   out [batch][n][h_q][d] strides (o_sb, o_sn, o_sh), type out_dtype
 * workspace (nullable) of ssa_sparse_attention_workspace_bytes(...) bytes: with
 *   it, the keys [0, X) that a row's indices hold exactly once (the lowest-key
 *   filler of a row with few candidates) are attended by a pass that streams
 *   them once per block of neighbouring rows, and the row pass skips them.
 *   The result is the same attention (a different summation order).
 * row_prefix (nullable) int32 [batch][h_kv][n]: X per row as ssa_select
 *   writes it (the caller vouches that the row's indices hold [0, X) once);
 *   without it the dense pass finds X from the indices (a bitmap per row).
 * row_stats (nullable) fp32 [batch][h_kv][n][g][2]: the bf16 matrix-core path
 *   (d 64 / 128, g <= 8) writes each (row, query head)'s softmax reference
 *   (the running maximum of q.k / scale_div in log2 units, 0 for a row with
 *   no slot) and 1 / sum there; other paths leave it as it was.  Given to the
 *   backward, it saves that kernel's first pass over the slots (fill it with
 *   NaN first: rows still NaN are recomputed).  No reference counterpart.
 * Limits: d a multiple of 8 in [8, 256], g <= 16. */
int ssa_sparse_attention(const void* q, const void* k, const void* v, int dtype, int64_t batch,
                         int64_t n, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn,
                         int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh, int64_t v_sb,
                         int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype, int top_k,
                         int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div,
                         int causal, const int32_t* row_order, const int32_t* row_prefix,
                         void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
                         int64_t o_sh, int32_t* error_flag, float* row_stats, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Bytes of ssa_sparse_attention's optional workspace for n_q query rows; 0
 * where the dense-prefix pass does not run (fp32 inputs, d other than 64 or
 * 128, g > 8, top_k < 64).  No reference counterpart. */
size_t ssa_sparse_attention_workspace_bytes(int dtype, int64_t batch, int64_t n_q, int h_q, int h_kv,
                                            int d, int top_k);

/* ssa_sparse_attention for a block of n_q query rows at key positions q_pos0
 * .. q_pos0 + n_q - 1 (0 <= q_pos0, q_pos0 + n_q <= n): q, idx, out and
 * row_order hold n_q rows; `causal` compares indices with the key position.
 * n_q = n with q_pos0 = 0 is ssa_sparse_attention.  No reference counterpart:
 * it serves incremental decoding and chunked prefill. */
int ssa_sparse_attention_block(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int64_t n_q,
    int64_t q_pos0, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb,
    int64_t k_sn, int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx,
    int idx_dtype, int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div,
    int causal, const int32_t* row_order, const int32_t* row_prefix, void* out, int out_dtype,
    int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag, float* row_stats, void* workspace,
    size_t workspace_bytes, void* stream);

/* Key blocks per query block: replaces convert_indices_to_blocks
 * (ssa/triton_kernel.py:226-294).  idx [batch][n][h_kv][top_k] (strides
 * idx_sb, idx_sn, idx_sh; int32 or int64 by idx_dtype) -> out
 * [batch][nb][h_kv][n_k_blocks] (strides o_sb, o_sq, o_sh; SSA_INDEX_I32 or
 * _I64 by out_dtype), nb = ceil(n / block_size), n_k_blocks <= nb (the
 * reference takes min(top_k, nb)).  For each query block, the key blocks
 * (key j -> block j / block_size) its rows reference most often, by count
 * descending and then block id ascending (the reference leaves the order of
 * equal counts to torch.topk); rows of the last query block past n count as
 * top_k references to block 0 each, as in the reference.  block_size: a power
 * of 2 in [2, 256]; nb <= 8192.  Indices outside [0, n) are skipped and set
 * *error_flag (nullable) to 1. */
int ssa_block_indices(const void* idx, int idx_dtype, int64_t batch, int64_t n, int h_kv, int top_k,
                      int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, int block_size, int n_k_blocks,
                      void* out, int out_dtype, int64_t o_sb, int64_t o_sq, int64_t o_sh,
                      int32_t* error_flag, void* stream);

/* Block-sparse exact attention: replaces ssa_triton_attention
 * (ssa/triton_kernel.py:141-223).  Query row i attends, causally (keys j <=
 * i), to every key of the n_k_blocks key blocks listed for its query block
 * i / block_size in blocks [batch][nb][h_kv][n_k_blocks] (strides b_sb, b_sq,
 * b_sh; int32 or int64 by idx_dtype).  Keys past n in the last block are
 * skipped; a block id outside [0, nb) sets *error_flag.  The softmax is exact
 * and normalised (the reference's kernel rescales and normalises its running
 * sums incorrectly, so its outputs are not a target); scores are q.k /
 * scale_div (the reference's default scale 1/sqrt(d) is scale_div =
 * sqrt(d)).  Other arguments as ssa_sparse_attention; it runs the same
 * kernels with the listed blocks expanded to keys on load. */
int ssa_block_sparse_attention(const void* q, const void* k, const void* v, int dtype, int64_t batch,
                               int64_t n, int h_q, int h_kv, int d, int64_t q_sb, int64_t q_sn,
                               int64_t q_sh, int64_t k_sb, int64_t k_sn, int64_t k_sh, int64_t v_sb,
                               int64_t v_sn, int64_t v_sh, const void* blocks, int idx_dtype,
                               int block_size, int n_k_blocks, int64_t b_sb, int64_t b_sq,
                               int64_t b_sh, float scale_div, void* out, int out_dtype,
                               int64_t o_sb, int64_t o_sn, int64_t o_sh, int32_t* error_flag,
                               void* stream);

/* Gradients of ssa_sparse_attention with respect to q, k and v, given the
 * forward output `out` and the output gradient `dout`.  Replaces the autograd
 * backward of sparse_exact_attention (gather -> einsum -> / scale -> softmax ->
 * einsum, ssa/attention.py:64-113), which the reference's training path runs
 * (tests/test_integration.py:32-49).  Same arguments as ssa_sparse_attention
 * for q, k, v, idx, scale_div, causal and row_order (duplicated slots count
 * once each, dropped slots not at all; an index outside [0, n) sets
 * *error_flag).  out and dout: [batch][n][h_q][d] with their own strides and
 * types (out_dtype, dout_dtype: f32 or bf16).
 *   dq fp32 [batch][n][h_q][d] contiguous: each processed row writes its own
 *      (a row never listed in row_order is not written);
 *   dk, dv fp32 [batch][n][h_kv][d] contiguous: zeroed, then accumulated.
 * Arithmetic is fp32 (softmax recomputed from q and k).  row_stats
 * (nullable): the forward's per-row softmax stats (ssa_sparse_attention's
 * row_stats); the matrix-core path then skips its first pass for every row
 * whose entry is not NaN.
 * Limits: d in [1, 256], g <= 16. */
int ssa_sparse_attention_backward(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
    int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
    const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
    int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
    float* dq, float* dk, float* dv, int32_t* error_flag, const int32_t* row_prefix,
    const float* row_stats, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of ssa_sparse_attention_backward's optional workspace (4 floats per
 * (row, query head)); 0 where the dense-prefix pass does not run (fp32 q/k/v
 * or dO, d other than 64 or 128, g > 8).  With row_prefix (X per row, as
 * ssa_select writes it) and this workspace, the keys [0, X) of each row are
 * differentiated by blocks of 8 neighbouring rows, whose dK/dV sums meet in
 * LDS before one fp32 atomic per (key, dim) and block.  No reference
 * counterpart. */
size_t ssa_sparse_attention_backward_workspace_bytes(int dtype, int dout_dtype, int64_t batch, int64_t n,
                                                     int h_q, int h_kv, int d);

/* ssa_sparse_attention_backward for indices that ssa_select produced (index
 * or score order, n >= top_k) from q_codes [batch][h_kv][n][a] and k_codes
 * [batch][h_kv][n][b] (ssa_route_codes), offsets / postings of
 * ssa_build_index, its row_prefix (required) and its causal routing flag
 * (router_causal: the mask was causal, else none).  Same results as
 * ssa_sparse_attention_backward (which pairs the indices hold is read from the
 * codes, row_prefix and the indices, never from scores).  dk and dv of the
 * candidate slots come from one pass per codebook
 * bucket: the rows holding a code and the keys holding it form a dense tile
 * (a pair sharing several codes counts in its smallest one), differentiated on
 * the matrix cores with one fp32 atomic per (key, dim) and 32-key chunk of a
 * bucket instead of one per selecting row.  Rows without filler (at least
 * top_k candidates) look their keys up in a bitmap of n bits each; the
 * workspace holds ssa_sparse_attention_backward_routed_workspace_bytes(...)
 * bytes, and rows past its bitmap capacity keep per-row atomics.  Shapes the
 * bucket pass does not take (fp32, d other than 64 / 128, g > 8, a > 32,
 * b > 8, N_c > 16384) run ssa_sparse_attention_backward's path.  No reference
 * counterpart (the reference's backward is autograd, ssa/attention.py:64-113). */
int ssa_sparse_attention_backward_routed(
    const void* q, const void* k, const void* v, int dtype, int64_t batch, int64_t n, int h_q,
    int h_kv, int d, int64_t q_sb, int64_t q_sn, int64_t q_sh, int64_t k_sb, int64_t k_sn,
    int64_t k_sh, int64_t v_sb, int64_t v_sn, int64_t v_sh, const void* idx, int idx_dtype,
    int top_k, int64_t idx_sb, int64_t idx_sn, int64_t idx_sh, float scale_div, int causal,
    const int32_t* row_order, const void* out, int out_dtype, int64_t o_sb, int64_t o_sn,
    int64_t o_sh, const void* dout, int dout_dtype, int64_t do_sb, int64_t do_sn, int64_t do_sh,
    float* dq, float* dk, float* dv, int32_t* error_flag, const int32_t* row_prefix,
    const float* row_stats, const int32_t* q_codes, int a, const int32_t* k_codes, int b,
    const int32_t* offsets,
    const int32_t* postings, int n_c, int router_causal, void* workspace, size_t workspace_bytes,
    void* stream);

/* Bytes of ssa_sparse_attention_backward_routed's workspace with key bitmaps
 * for bitmap_rows rows without filler (negative: half of the batch x kv head
 * x n rows); ssa_sparse_attention_backward_workspace_bytes(...) where the
 * bucket pass does not run.  No reference counterpart. */
size_t ssa_sparse_attention_backward_routed_workspace_bytes(int dtype, int dout_dtype, int64_t batch,
                                                            int64_t n, int h_q, int h_kv, int d, int top_k,
                                                            int a, int b, int n_c, int64_t bitmap_rows);

#ifdef __cplusplus
}
#endif

#endif /* SSA_HIP_H */
