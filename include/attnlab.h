/*
 * attnlab.h - C ABI of the MI355X (gfx950) sparse-decode hot path.
 *
 * Every entry point takes raw device pointers, plain integer shapes/strides and a hipStream_t (passed as void*),
 * launches asynchronously on that stream, never synchronises and never allocates device memory. The return value
 * is a status code:
 *   ATTNLAB_OK (0)            work enqueued;
 *   ATTNLAB_EINVAL (1)        an argument violates the contract (the Python layer raises ValueError);
 *   ATTNLAB_ERUNTIME (2)      the HIP runtime reported an error (the Python layer raises RuntimeError).
 * attnlab_last_error() returns a message for the last non-zero status of the calling thread.
 *
 * Tensor layouts follow the reference (paths relative to wlvh/attention-lab):
 *   K, V cache       [B, G, C, d] bf16, row = one position (src/attention_lab/qwen_wrap.py:68-70)
 *   index table zT   [B, G, r, C] (src/attention_lab/indexer.py:15-17, qwen_wrap.py:74-75)
 *   query            [B, G, h, d] bf16 (q_main[B,G,h,1,d] of decode.py:145-147 with T == 1)
 *   selection        F = [0, lo) U [hi, legal), candidates [lo, hi) (src/attention_lab/selection.py:69-86)
 * bf16 and fp16 buffers are passed as uint16_t*. All pointers must be device pointers of the current device.
 */
#ifndef ATTNLAB_H
#define ATTNLAB_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATTNLAB_OK 0
#define ATTNLAB_EINVAL 1
#define ATTNLAB_ERUNTIME 2

/* Row-list order of attnlab_select_rows / attnlab_sparse_decode_step. */
#define ATTNLAB_ORDER_POSITION 0 /* every row list ascending by position (canonical_order=True, decode.py:160-161) */
#define ATTNLAB_ORDER_SCORE 1    /* F ascending, then the top-k by descending score, ties lowest index first
                                    (cat(fixed_rows, topk.indices) of decode.py:86-93); any k: up to
                                    ATTNLAB_LDS_SORT_K pairs are sorted in LDS, more by a radix pass through the
                                    select scratch */

/* Largest k whose score order is sorted in one workgroup's LDS (attnlab_topk takes score order up to this k). */
#define ATTNLAB_LDS_SORT_K 8192

/* Index-key element types of the score kernels. */
#define ATTNLAB_DT_BF16 0
#define ATTNLAB_DT_F16 1
#define ATTNLAB_DT_F32 2

/* Words per row of the select state shared by attnlab_score_grouped and attnlab_select_rows: the first-digit
 * histogram (2048 bins), then 64 super-bin counts (sums of 32 consecutive bins), then 64 arrival counters that the
 * fused step's attend uses to merge its split-K partials in-kernel. Zero on entry; every call leaves it zero. */
#define ATTNLAB_SELECT_STATE_WORDS 2176

/* ABI version; bumped on any signature change. */
int attnlab_abi_version(void);

/* Message of the last failing call on this thread ("" when none). */
const char* attnlab_last_error(void);

/* gfx target name of the device the library was built for ("gfx950"). */
const char* attnlab_target(void);

/*
 * Grouped-indexer score, parity mode. Replaces MetalScore.fused / MetalScore.two_launch
 * (src/attention_lab/metal_score.py:294-330, kernels :44-246) and, batched, the project_keys column write +
 * project_queries + candidate_scores sequence of sparse_decode_step_kernel (decode.py:156-158, indexer.py:15-29).
 *
 * For every (b, g):
 *   if k_new != NULL:  zT[b,g,j,write_col] = bf16_rne(sum_e wk[g,j,e] * k_new[b,g,e])          (j < r)
 *   u[j]  = sum_f q_cat[b,g,f] * wq_t[g,f,j]   (fp32; 1/sqrt(r) is already folded into wq_t)   or u_in[b,g,j]
 *   out[b,g,m] = sum_j u[j] * zT[b,g,j,lo+m]   (fp32) for m in [0, hi-lo)
 * zT: [B,G,r,C] bf16 contiguous. k_new: [B,G,d] (nullable: no column write). wk: [G,r,d]. q_cat: [B,G,hd] with
 * q_cat[f = i*d + e] = q_pre[b,g,i,e] (project_queries order). wq_t: [G,hd,r]. u_in: [B,G,r] fp32 (nullable; when
 * given, q_cat/wq_t are not read). u_out: [B,G,r] fp32 (nullable; receives u). out: row (b,g) at out + bg*out_stride.
 * Requires r <= 32, 0 <= lo <= hi <= C, 0 <= write_col < C and write_col outside [lo, hi) when k_new != NULL.
 * vector != 0 selects the 16-byte-load scan (used when C % 8 == 0 and zT is 16-byte aligned; otherwise the 2-byte
 * scan runs, the counterpart of the reference's v1 fallback, metal_score.py:289-292).
 * state (nullable): select state [B*G, ATTNLAB_SELECT_STATE_WORDS] uint32, zero on entry; receives, per (b,g), the
 * histogram of the scores' first radix digit (top 11 bits of the order-preserving key) in its first 2048 words, which
 * attnlab_select_rows consumes and clears.
 */
int attnlab_score_grouped(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                          const uint16_t* wq_t, const float* u_in, float* u_out, float* out, int64_t out_stride,
                          int B, int G, int r, int C, int d, int hd, int lo, int hi, int write_col, int vector,
                          uint32_t* state, void* stream);

/*
 * Prologue only: u (and the z column when k_new != NULL). The first launch of MetalScore.two_launch
 * (metal_score.py:314-321, kernel `prologue` :101-123). u_out: [B,G,r] fp32.
 */
int attnlab_score_prologue(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                           const uint16_t* wq_t, float* u_out, int B, int G, int r, int C, int d, int hd,
                           int write_col, void* stream);

/*
 * Bulk index-table build: zT[b,g,j,col0+t] = bf16_rne(sum_e wk[g,j,e] * k_pre[b,g,t,e]) for t < T. Replaces
 * project_keys (indexer.py:15-17) and the chunked table writes of the prefill (qwen_wrap.py:320-324).
 * k_pre: row t of (b,g) at k_pre + bg*k_bg_stride + t*k_row_stride (elements, 16-byte aligned rows), d <= 128,
 * d % 8 == 0. zT: [B,G,r,C] bf16. Requires 0 <= col0, col0 + T <= C.
 */
int attnlab_project_keys(const uint16_t* k_pre, int64_t k_bg_stride, int64_t k_row_stride, const uint16_t* wk,
                         uint16_t* zT, int B, int G, int T, int r, int d, int C, int col0, void* stream);

/*
 * Float32 index tables (a trained bank's cache: FrozenIndexer keeps wq/wk in float32, trained.py:11-18, and the
 * state's cache is built with index_dtype=float32, trained.py:78-81; FrozenBank.guard refuses anything else,
 * trained.py:45-46). The same contract as attnlab_score_grouped with every index-side operand in fp32:
 *   if k_new != NULL:  zT[b,g,j,write_col] = sum_e wk[g,j,e] * k_new[b,g,e]   (fp32, no rounding to bf16)
 *   u[j] = sum_f q_cat[b,g,f] * wq_t[g,f,j]   or u_in;   out[b,g,m] = sum_j u[j] * zT[b,g,j,lo+m]
 * zT: [B,G,r,C] fp32 (16-byte loads when C % 4 == 0 and zT is 16-byte aligned, 4-byte loads otherwise);
 * k_new [B,G,d], wk [G,r,d], q_cat [B,G,hd],
 * wq_t [G,hd,r] fp32. u_out, when given without u_in, receives u (q_cat and wq_t required); the scan of hi > lo
 * reads u from u_in or u_out, so one of them is required then. A call with k_new == NULL and lo == hi is a pure query
 * projection (project_queries, indexer.py:20-24) and may pass zT == NULL, C == 0. No vector flag: the load width
 * follows the table's alignment. state as in attnlab_score_grouped.
 */
int attnlab_score_grouped_f32(float* zT, const float* k_new, const float* wk, const float* q_cat, const float* wq_t,
                              const float* u_in, float* u_out, float* out, int64_t out_stride, int B, int G, int r,
                              int C, int d, int hd, int lo, int hi, int write_col, uint32_t* state, void* stream);

/*
 * Bulk fp32 index-table build (project_keys, indexer.py:15-17, on a float32 cache): zT[b,g,j,col0+t] =
 * sum_e wk[g,j,e] * k_pre[b,g,t,e] in fp32. k_pre rows 16-byte aligned (strides in elements, multiples of 4),
 * d % 4 == 0, d <= 128. zT: [B,G,r,C] fp32. Requires 0 <= col0, col0 + T <= C.
 */
int attnlab_project_keys_f32(const float* k_pre, int64_t k_bg_stride, int64_t k_row_stride, const float* wk,
                             float* zT, int B, int G, int T, int r, int d, int C, int col0, void* stream);

/*
 * Lightning-indexer score (no reference kernel: the generalisation north_star names; the grouped score of
 * indexer.py:27-29 is the special case nh=1, w=1, relu=0, keys transposed):
 *   out[b,kg,t] = sum_i w[b,kg,i] * act(sum_j q[b,kg,i,j] * key[b,kg,t,j])   for t in [lo, hi), act = ReLU or identity
 * keys: [B,KG,Lk,r] (row layout, one r-vector per position) in key_dtype (ATTNLAB_DT_F16 or ATTNLAB_DT_BF16);
 * q: [B,KG,nh,r] fp32; w: [B,KG,nh] fp32; out row (b,kg) at out + bkg*out_stride holds hi-lo fp32 scores.
 * r must be 32; 1 <= nh <= 8.
 */
int attnlab_score_lightning(const uint16_t* keys, int key_dtype, const float* q, const float* w, float* out,
                            int64_t out_stride, int B, int KG, int Lk, int r, int nh, int lo, int hi, int relu,
                            void* stream);

/*
 * Batched (prefill) lightning-indexer score on the matrix cores: the T-query form of attnlab_score_lightning, the
 * "batched/prefill score contraction" north_star puts on MFMA (no reference kernel; per query it is the formula of
 * attnlab_score_lightning, and with nh=1, w=1, relu=0 the grouped score of indexer.py:27-29 for T queries):
 *   out[b,kg,t,m-lo] = sum_i w[b,kg,t,i] * act(sum_j q[b,kg,t,i,j] * key[b,kg,m,j])
 * for m in [lo, hi) and, when q_pos0 >= 0, m <= q_pos0 + t (causal: query t sits at position q_pos0 + t); entries
 * past a query's causal bound are not written. keys: [B,KG,Lk,32] fp16/bf16, 16-byte aligned; q: [B,KG,T,nh,32]
 * fp32, 16-byte aligned; w: [B,KG,T,nh] fp32; out row (b,kg,t) at out + ((b*KG+kg)*T+t)*out_stride, 16-byte aligned,
 * out_stride a multiple of 4. r must be 32; nh in {1, 2, 4, 8}.
 */
int attnlab_score_lightning_batched(const uint16_t* keys, int key_dtype, const float* q, const float* w, float* out,
                                    int64_t out_stride, int B, int KG, int Lk, int r, int nh, int T, int lo, int hi,
                                    int q_pos0, int relu, void* stream);

/*
 * Top-k selection with lowest-index tie-break, no reference kernel (the reference calls torch.topk,
 * decode.py:86-93 / :161-166; the planned P2 kernel was never built). For each of R rows of M fp32 scores
 * (row i at scores + i*score_stride) selects the k largest; equal scores resolve to the lower index; NaN ranks below
 * every number; -0.0 equals +0.0. Writes, when non-NULL, top_idx[i, 0..k) (int32 candidate-relative indices) and
 * top_val[i, 0..k) (the scores), row stride top_stride, in `order`: ATTNLAB_ORDER_POSITION (ascending index) or
 * ATTNLAB_ORDER_SCORE (descending score, then ascending index). Requires 0 <= k <= M, and k <= ATTNLAB_LDS_SORT_K in
 * score order (larger k: attnlab_topk_tiled, which has the scratch for the radix pass).
 */
int attnlab_topk(const float* scores, int64_t score_stride, int R, int M, int k, int order, int32_t* top_idx,
                 float* top_val, int64_t top_stride, void* stream);

/*
 * attnlab_topk spread over the chip for long rows (the same selection, bit for bit): a histogram pass, a classify
 * pass over tiles of 4096 scores and one resolve workgroup per row, instead of one workgroup per row for every pass.
 * Replaces the same torch.topk call (decode.py:86-93), for any k in either order. state: [R,
 * ATTNLAB_SELECT_STATE_WORDS] uint32, 16-byte aligned, zero on entry and left zero; scratch: 256-byte aligned, at least
 * attnlab_select_scratch_bytes(R, M, k, order) bytes, no initialisation. Rows longer than 262144 scores run the
 * single-workgroup select.
 */
int attnlab_topk_tiled(const float* scores, int64_t score_stride, int R, int M, int k, int order, int32_t* top_idx,
                       float* top_val, int64_t top_stride, uint32_t* state, void* scratch, int64_t scratch_bytes,
                       void* stream);

/*
 * Selection of one decode step: top-k over the candidate scores merged with the fixed set F, written as the row
 * list the attend kernel reads. Replaces select_rows_kernel + the optional canonical sort
 * (decode.py:86-93, :160-161) and DecodeRequest.select_positions (decode.py:50-56).
 * scores: [B*G] rows of M = hi - lo candidate scores (row stride score_stride). F = [0, lo) U [hi, legal).
 * S = lo + (legal - hi) + k. rows: [B*G, S] int32 positions (row stride rows_stride; nullable). rows_flat: [B*G*S]
 * int64 flat row ids pos + (b*G+g)*C of the flattened [B*G*C, d] cache (sparse.py:14-16; nullable).
 * order: ATTNLAB_ORDER_POSITION or ATTNLAB_ORDER_SCORE.
 * state (nullable): the select state [B*G, ATTNLAB_SELECT_STATE_WORDS] attnlab_score_grouped filled for these scores;
 * when given, the first radix pass is skipped and the state is left zeroed for the next call.
 * scratch (256-byte aligned, no zeroing needed; nullable except in score order with k > ATTNLAB_LDS_SORT_K): with
 * state, 0 < k, hi - lo <= 262144 and scratch_bytes >= attnlab_select_scratch_bytes(B*G, hi - lo, k, order), the keys
 * are classified by a grid of 4096-key tiles and each row resolved by one workgroup (two launches) instead of one
 * workgroup per row reading every key three times; the result is the same. Every argument check runs before the first
 * launch.
 */
int attnlab_select_rows(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k,
                        int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                        void* scratch, int64_t scratch_bytes, void* stream);

/*
 * The list select, the two stages attnlab_sparse_decode_step runs where it applies (no reference counterpart: the
 * reference's step is indexer + torch.topk, decode.py:86-93 and :145-163). attnlab_score_grouped_lists is the
 * one-launch attnlab_score_grouped (bf16 table, r = 32, h*d <= 512, C % 8 == 0, 16-byte aligned zT, u built from q_cat
 * and wq_t) that also writes, for every score workgroup, a list of its largest keys into `lists` (256-byte aligned,
 * attnlab_list_bytes(B, G, lo, hi, k, order) bytes, no initialisation); `state` is required; `out` may be NULL (key
 * lists only, no score stored: what the fused step runs in position order), and then u_out must be given.
 * attnlab_select_lists then writes what attnlab_select_rows writes for the same scores, state and arguments, reading
 * the lists instead of every score, in one launch, and leaves the state zeroed. A tile whose list cannot hold its part
 * of the selection (and a row whose threshold bin holds more than 8192 keys) is read from `scores`; with scores NULL
 * it is recomputed from the index table zT (z_dtype ATTNLAB_DT_BF16 or ATTNLAB_DT_F32, the score stage's table) and
 * the score stage's u_out, in the score kernel's exact fp32 operation order, so the result is the same; that takes
 * ATTNLAB_ORDER_POSITION (score order reads the picks' scores back). zT and u are ignored when scores are given. attnlab_list_bytes returns 0 where the list select does not apply (hi - lo > 32768, or k large
 * against hi - lo, or `order` ATTNLAB_ORDER_SCORE with k > ATTNLAB_LDS_SORT_K, which the list select does not sort;
 * both functions then fail with ATTNLAB_EINVAL before any launch) and -1 for invalid sizes. `order` is the row order
 * the select stage will be asked for: the score stage refuses a combination the select stage would refuse, because
 * the score stage adds into `state`, which only a completed select stage clears. attnlab_select_lists checks its
 * arguments again; called with other arguments than its score stage (another order, k or shape), it can refuse after
 * the state was filled, and the caller must then zero the state itself. attnlab_sparse_decode_step takes the tiled
 * select itself for score order with k > ATTNLAB_LDS_SORT_K.
 */
int64_t attnlab_list_bytes(int B, int G, int lo, int hi, int k, int order);
int attnlab_score_grouped_lists(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                                const uint16_t* wq_t, float* u_out, float* out, int64_t out_stride, int B, int G,
                                int r, int C, int d, int hd, int lo, int hi, int write_col, int k, int order,
                                uint32_t* state, void* lists, int64_t lists_bytes, void* stream);
int attnlab_select_lists(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k,
                         int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                         const void* lists, int64_t lists_bytes, const void* zT, int z_dtype, const float* u,
                         void* stream);

/* Scratch bytes of attnlab_select_rows / attnlab_topk_tiled for R rows of M candidates and top-k in `order`: the
 * tiled select's bitmaps and candidate entries, plus the radix pass's buffers in score order with
 * k > ATTNLAB_LDS_SORT_K (-1 for negative sizes or k outside [0, M]). */
int64_t attnlab_select_scratch_bytes(int R, int M, int k, int order);

/*
 * Gather-free sparse attention. Replaces MetalAttend.__call__ (metal_attend.py:226-250, kernels :46-169) and the
 * index_select + subset SDPA of gathered_decode_step_kernel (decode.py:131-142, sparse.py:40-60):
 *   out[b,g,i] = softmax_s(scale * q[b,g,i] . K[b,g,rows[b,g,s]]) @ V[b,g,rows[b,g,s]]   over s < S
 * K/V: position p of (b,g) at K + bg*kv_bg_stride + p*kv_row_stride (elements; V likewise), d = 128 contiguous
 * values per position. The interleaved diagnostic layout [G,C,2,d] is K = base, V = base + 128, row stride 256.
 * q: [B,G,h,128] bf16 contiguous, 1 <= h <= 8. rows: [B*G, S] int32 positions (row stride rows_stride), S >= 1,
 * positions outside [0, C) are skipped (never read). P split-K partitions (1..256); when P > 1, part must hold
 * B*G*P*h*130 floats and a second small kernel merges the partials. out: [B,G,h,128], bf16 (RNE) when out_bf16
 * else fp32.
 */
int attnlab_attend(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                   const uint16_t* q, const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S, int C,
                   int P, float scale, void* out, int out_bf16, float* part, void* stream);

/*
 * Dense decode attention over positions [0, L): the control read A. Replaces full_attention(backend="sdpa_fold")
 * for one decode query at the last legal position (full.py:17-34) and dense_decode_step (decode.py:174-176).
 * Same layouts and partials contract as attnlab_attend.
 */
int attnlab_dense_decode(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                         const uint16_t* q, int B, int G, int h, int L, int C, int P, float scale, void* out,
                         int out_bf16, float* part, void* stream);

/*
 * attnlab_attend over a paged K/V cache (the layout option of the attend, metal_attend.py:226-235; no reference
 * kernel reads pages). K_pages, V_pages: pools [num_pages, G, page_size, 128] bf16 shared by all sequences;
 * block_table: int32 [B, bt_stride], entry j of sequence b = the pool page holding its positions
 * [j * page_size, (j + 1) * page_size) for all G groups (j < max_pages). Position p of (b, g) is read from pool row
 * (block_table[b][p / page_size] * G + g) * page_size + p % page_size. rows as in attnlab_attend (positions, row
 * stride rows_stride), or NULL for the positions [0, S) (the dense read of a paged cache); listed positions outside
 * [0, max_pages * page_size) or on a page entry outside [0, num_pages) are skipped, never read. page_size a power of
 * two up to 65536; the pool at most 2^31 rows. q, out, P, part, scale as in attnlab_attend.
 */
int attnlab_attend_paged(const uint16_t* K_pages, const uint16_t* V_pages, int num_pages, int page_size,
                         const int32_t* block_table, int64_t bt_stride, int max_pages, const uint16_t* q,
                         const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S, int P, float scale,
                         void* out, int out_bf16, float* part, void* stream);

/*
 * Causal prefill read on the matrix cores: full_attention (full.py:17-44) for a chunk of T > 1 queries, with the
 * reference's legality rule (reference.py:41-48). Query t sits at position q_pos0 + t and reads the cache rows
 * j <= q_pos0 + t, j < legal:
 *   out[b,g,i,t,:] = sum_j softmax_j(scale * q[b,g,i,t,:] . K[b,g,j,:]) V[b,g,j,:]
 * q, out: [B,G,h,T,d] bf16 contiguous; K/V row j of (b,g) at K + (b*G+g)*kv_bg_stride + j*kv_row_stride (elements).
 * d must be 128; h one of 1, 2, 4, 8, 16; 16-byte aligned pointers and rows; 0 < legal <= C.
 */
int attnlab_prefill_attend(const uint16_t* q, const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride,
                           int kv_row_stride, uint16_t* out, int B, int G, int h, int T, int d, int q_pos0, int legal,
                           int C, float scale, void* stream);

/*
 * The same read with the keys of every query tile split into `splits` (1..16) ranges of whole 64-key blocks, for
 * grids that one workgroup per tile leaves mostly idle: a short chunk after a long history, as the reference's chunked
 * prefill runs (qwen_wrap.py:320-324 calls full_attention per chunk). Each split writes its rows' partial (running
 * max, sum, unnormalised outputs) to `part`, a second kernel merges them into `out` in split order. The result equals
 * attnlab_prefill_attend's up to the summation order. part: 16-byte aligned, at least attnlab_prefill_part_bytes
 * bytes, no initialisation; splits == 1 takes no part and is attnlab_prefill_attend.
 */
int64_t attnlab_prefill_part_bytes(int B, int G, int h, int T, int splits);
int attnlab_prefill_attend_split(const uint16_t* q, const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride,
                                 int kv_row_stride, uint16_t* out, int B, int G, int h, int T, int d, int q_pos0,
                                 int legal, int C, float scale, int splits, float* part, int64_t part_bytes,
                                 void* stream);

/*
 * Workspace (bytes) of attnlab_sparse_decode_step for these sizes: candidate scores, row list, u, tiled-select
 * scratch and split-K partials, each 256-byte aligned. Its contents need no initialisation.
 */
int64_t attnlab_sparse_decode_workspace(int B, int G, int h, int lo, int hi, int legal, int k, int P);

/*
 * One layer's sparse decode read for one new query: z column write, u projection, candidate scan, top-k, merge with
 * F, gather-free attention. Replaces sparse_decode_step_kernel (decode.py:145-163) with a few launches on `stream`:
 * the score (u, z column, scan and, with `state`, the key lists of the list select), then the select and the attend.
 * With neither rows_out nor rows_flat, and the list select applying, those two are one launch: every attend
 * workgroup selects its row from the key lists and attends its partition (the output bits of the separate launches).
 * The attend merges split-K partials in-kernel with `state`, else a combine launch does when P > 1. Calls sharing a
 * workspace or a select state must be ordered on one stream.
 * q_main: [B,G,h,128] bf16 (post-RoPE query); q_cat: [B,G,h*128] bf16 (pre-RoPE query, project_queries order);
 * K/V: [B,G,C,128] bf16; zT: [B,G,r,C] bf16; wq_t: [G,h*128,r]; wk: [G,r,128]; k_new: [B,G,128] (nullable: the
 * z column is not written). F = [0, lo) U [hi, legal); k top candidates; write_col = legal - 1 for the reference's
 * plan. rows_out: [B*G, S] int32 positions (nullable: kept in the workspace); rows_flat: [B*G*S] int64 flat ids
 * (nullable). out: [B,G,h,128] bf16. P: split-K partitions of the attend (1..64). order as in attnlab_select_rows;
 * with neither rows_out nor rows_flat given the row order is not observable (attention is the same over any order of
 * its rows, up to the summation's rounding), and the step runs the position-order select, the faster one.
 * state: select state [B*G, ATTNLAB_SELECT_STATE_WORDS] uint32, zero before the first call; the score kernel fills
 * it and the select kernels (in the one-launch form, the row's last workgroup to read it) clear it, so it stays zero
 * between calls with no memset (the launches stay capturable in a HIP graph). Nullable: the select kernel then runs its own first radix pass on one workgroup per row.
 */
int attnlab_sparse_decode_step(const uint16_t* q_main, const uint16_t* q_cat, const uint16_t* K, const uint16_t* V,
                               uint16_t* zT, const uint16_t* wq_t, const uint16_t* wk, const uint16_t* k_new,
                               int B, int G, int h, int r, int C, int lo, int hi, int legal, int k, int write_col,
                               float scale, int order, int P, uint32_t* state, void* workspace,
                               int64_t workspace_bytes, int32_t* rows_out, int64_t* rows_flat, uint16_t* out,
                               void* stream);

/*
 * attnlab_sparse_decode_step over a float32 index table (sparse_decode_step_kernel, decode.py:145-163, with a trained
 * bank's fp32 wq_t_scaled/wk and fp32 z cache, trained.py:78-81): q_cat [B,G,h*128], zT [B,G,r,C],
 * wq_t [G,h*128,r], wk [G,r,128] and k_new [B,G,128] are fp32; q_main, K, V and out stay bf16. Same workspace size
 * (attnlab_sparse_decode_workspace), state, order and row-list contract.
 */
int attnlab_sparse_decode_step_f32(const uint16_t* q_main, const float* q_cat, const uint16_t* K, const uint16_t* V,
                                   float* zT, const float* wq_t, const float* wk, const float* k_new, int B, int G,
                                   int h, int r, int C, int lo, int hi, int legal, int k, int write_col, float scale,
                                   int order, int P, uint32_t* state, void* workspace, int64_t workspace_bytes,
                                   int32_t* rows_out, int64_t* rows_flat, uint16_t* out, void* stream);

/*
 * attnlab_sparse_decode_step with no allocation and no caller buffers beyond its inputs and outputs. No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The select state and the workspace live in a 32 MiB file-scope device array
 * that each device holds until the process ends; its first 256 * ATTNLAB_SELECT_STATE_WORDS words are the select state
 * (B*G <= 256), the rest the workspace (attnlab_sparse_decode_workspace of these sizes must fit, or the call returns
 * ATTNLAB_EINVAL). Arguments and outputs as in attnlab_sparse_decode_step (bf16 index table). Every call on a device
 * shares that device's array: calls that overlap on one device race, so order them on one stream.
 */
int attnlab_sparse_decode_step_noalloc(const uint16_t* q_main, const uint16_t* q_cat, const uint16_t* K,
                                       const uint16_t* V, uint16_t* zT, const uint16_t* wq_t, const uint16_t* wk,
                                       const uint16_t* k_new, int B, int G, int h, int r, int C, int lo, int hi,
                                       int legal, int k, int write_col, float scale, int order, int P,
                                       int32_t* rows_out, int64_t* rows_flat, uint16_t* out, void* stream);

/*
 * Measurement only (no reference counterpart): the read ceiling of attnlab_attend. Reads the K/V rows attnlab_attend
 * would read for these rows, with its grid (B*G*Q*P workgroups of 256 threads: Q head groups, P partitions), lane
 * layout and load pipeline, and folds the loaded words into one word per thread, stored to sink [B*G*Q*P*256] uint32.
 * Nothing else is computed. Positions outside [0, C) read row 0, as attnlab_attend masks them.
 */
int attnlab_gather_probe(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                         const int32_t* rows, int64_t rows_stride, int B, int G, int S, int C, int Q, int P,
                         uint32_t* sink, void* stream);

/*
 * Measurement only (no reference counterpart): the read ceiling of the one-launch score (score_scan_fused, the fused
 * step's score). Runs its grid, u prologue (q_cat [B*G, hd] . wq_t [G, hd, 32]), table loads of zT [B*G, 32, C] over
 * candidate columns [lo, hi) and load pipeline, with the multiply, reduction, histogram and key lists replaced by an
 * XOR fold of the loaded words; one word per thread goes to sink, which must hold
 * B*G*ceil((hi - lo + 16) / 512)*256 uint32. Needs the one-launch layout: C % 8 == 0, zT and wq_t 16-byte aligned,
 * 1 <= hd <= 512.
 */
int attnlab_scan_probe(const uint16_t* zT, const uint16_t* q_cat, const uint16_t* wq_t, int B, int G, int C, int hd,
                       int lo, int hi, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTNLAB_H */
