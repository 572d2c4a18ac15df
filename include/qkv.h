/*
 * qkv.h -- C ABI of libqkv, the MI355X (gfx950) kernels of the Qwen3
 * sparse-attention KV-retrieval path.
 *
 * Every entry point takes plain device pointers, sizes and strides, launches
 * asynchronously on the caller's HIP stream (`stream` is a hipStream_t, NULL
 * for the default stream), never allocates and never synchronises.  Outputs
 * and workspaces are owned by the caller.  Each returns QKV_OK or a negative
 * status; qkv_last_error() then holds this thread's message.
 *
 * Reference citations are to littlexi001/kv_cache:
 *   QK = ymluo/projects/qwen3_top2_head_limit3_ppl/src/qabs_cuda_kernels.py
 *   EV = ymluo/projects/qwen3_top2_head_limit3_ppl/src/evaluate_qwen3_top2_head_limit3_ppl.py
 *
 * Strides are in elements of the tensor's own type.  The innermost (channel)
 * axis is always contiguous unless a stride argument for it is given.
 */
#ifndef QKV_H_
#define QKV_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QKV_OK 0
#define QKV_ERR_INVALID (-1)     /* bad shape, pointer, alignment or value  */
#define QKV_ERR_LAUNCH (-2)      /* HIP reported an error at launch         */
#define QKV_ERR_UNSUPPORTED (-3) /* valid request outside what is built     */

#define QKV_DTYPE_BF16 0
#define QKV_DTYPE_FP16 1
#define QKV_DTYPE_FP32 2

/* Block-metadata selector kinds (qkv_block_*). */
#define QKV_BLOCK_QBB 0  /* Quest-style per-block channel min/max bounds */
#define QKV_BLOCK_BREP 1 /* per-block representative tokens */

/* Candidate selections of the reuse step (--qabs_candidate_selection,
 * EV:3958-3989). */
#define QKV_CAND_TOPK 0               /* the row's k-th largest value             */
#define QKV_CAND_SAMPLE_QUANTILE 1    /* the k-th largest of sampled columns      */
#define QKV_CAND_PREVIOUS_THRESHOLD 2 /* the previous step's threshold            */

/* Refresh tests of the lagged reuse modes (qkv_reuse_lag_flags, EV:4026-4087). */
#define QKV_LAG_DIMS 0    /* record the top-|q| dims and values only               */
#define QKV_LAG_OVERLAP 1 /* qdrift[maj|head|share]: top dims shared with the last */
#define QKV_LAG_COS 2     /* qdriftcos[head]: overlap, or cosine on the last dims  */
#define QKV_LAG_ESS 3     /* pconf{T}: effective sample size of the last selection */

/* Which rows of a lagged step take new candidates (qkv_reuse_lag_union). */
#define QKV_REFRESH_NONE 0     /* none: the previous final selection alone       */
#define QKV_REFRESH_ALL 1      /* every row                                      */
#define QKV_REFRESH_PER_ROW 2  /* the rows whose flag is set                     */
#define QKV_REFRESH_ANY 3      /* every row when any flag is set                 */
#define QKV_REFRESH_MAJORITY 4 /* every row when more than half the flags are    */

#define QKV_ABI_VERSION 2

/* ABI version of the loaded library (QKV_ABI_VERSION it was built with). */
int qkv_abi_version(void);

/* Message of this thread's most recent failed call ("" if none).  Replaces
 * the TORCH_CHECK messages the reference raises (QK:425-430, 576-593). */
const char* qkv_last_error(void);

/* ======================================================================
 * Reference-signature family: the four kernels behind the reference's
 * Python module, fp32 results, inputs in bf16 / fp16 / fp32 (dtype).
 * ====================================================================== */

/* Replaces qabs_partial_scores_forward (QK:421-459, kernel QK:98-158,
 * Python partial_scores QK:654-656).
 * query [B,H,D] contiguous; key [B,H,T,D] with k_strides = {b,h,t,d};
 * out f32 [B,H,T] contiguous.  Per (b,h): the min(max(dim_count,1),D,128)
 * dims of largest |q| (ties to the lower dim), then out = sum_s q*k in
 * selection order, fp32. */
int qkv_partial_scores(const void* query, const void* key, float* out, int dtype,
                       int64_t batch, int64_t heads, int64_t keys, int64_t head_dim,
                       const int64_t* k_strides, int64_t dim_count, void* stream);

/* Replaces qabs_partial_scores_dim_major_forward (QK:461-504, kernel
 * QK:63-96, Python partial_scores_dim_major QK:659-665).
 * query [B,H,D] contiguous; key_dim_major [B,H,D,T] with kdm_strides =
 * {b,h,d,t}; dim_indices int64 [B,H,S] contiguous; out f32 [B,H,T]. */
int qkv_partial_scores_dim_major(const void* query, const void* key_dim_major,
                                 const int64_t* dim_indices, float* out, int dtype,
                                 int64_t batch, int64_t heads, int64_t keys, int64_t head_dim,
                                 int64_t selected, const int64_t* kdm_strides, void* stream);

/* Replaces qabs_candidate_full_scores_forward (QK:506-567, kernel
 * QK:160-216, Python candidate_full_scores QK:668-691).
 * Masks are uint8 [B,H,T] contiguous; previous / previous_final may be NULL.
 * out f32 [B,H,T]: full-D dot * scaling where selected, else -inf. */
int qkv_candidate_full_scores(const void* query, const void* key, const uint8_t* current,
                              const uint8_t* previous, const uint8_t* previous_final,
                              float* out, int dtype, int64_t batch, int64_t heads,
                              int64_t keys, int64_t head_dim, const int64_t* k_strides,
                              int64_t protect_sink, int64_t protect_recent, float scaling,
                              void* stream);

/* Replaces qabs_final_attention_forward (QK:569-638, kernel QK:335-419,
 * Python final_attention QK:694-705).
 * query [B,H,D], key/value [B,H,T,D], indices int64 [B,H,N], valid uint8
 * [B,H,N], out [B,H,D] in dtype; all contiguous.  N <= 16384. */
int qkv_final_attention(const void* query, const void* key, const void* value,
                        const int64_t* indices, const uint8_t* valid, void* out, int dtype,
                        int64_t batch, int64_t heads, int64_t keys, int64_t selected,
                        int64_t head_dim, float scaling, void* stream);

/* ======================================================================
 * int4 family (no reference counterpart: the reference scores fp32 over
 * GQA-expanded bf16 K).  K/V/q are bf16 or fp16, named by the last
 * argument before the stream (QKV_DTYPE_BF16 / QKV_DTYPE_FP16; FP32 fails
 * with QKV_ERR_UNSUPPORTED).  A "row" r = b * Hkv + j is one
 * (sequence, KV head).  Packed K, scales and the subset slab are laid out
 * [rows, capacity, ...] with capacity a multiple of 64 tokens.
 * ====================================================================== */

/* Quantize tokens [t_begin, t_end) of K [B,Hkv,*,D] (k_strides = {b,h,t},
 * channels contiguous, rows 16-byte aligned) to symmetric int4 in groups of
 * `group` channels (32, 64 or 128): packed uint8 [rows,capacity,D/2],
 * scales fp16 bits [rows,capacity,D/group].  Nearest reference layout: the
 * dim-major K copy kept per layer (EV:2018-2042). */
int qkv_int4_pack_k(const void* key, const int64_t* k_strides, int64_t batch, int64_t kv_heads,
                    int64_t t_begin, int64_t t_end, int64_t head_dim, int64_t group,
                    uint8_t* packed, uint16_t* scales, int64_t capacity, int dtype, void* stream);

/* Static channel subset per row: stats[r,c] = sum_t |code| * scale * 2^24
 * (exact uint64, T <= 2^20), then the `selected` channels of largest stat,
 * ties to the lower channel, written ascending to chan_idx int32
 * [rows,selected].  stats uint64 [rows,D] is an output the call overwrites.
 * Replaces the per-step top-|q| dims of EV:4428 / QK:123-145 with a
 * per-KV-head choice made once per prefill. */
int qkv_int4_select_channels(const uint8_t* packed, const uint16_t* scales, int64_t rows,
                             int64_t tokens, int64_t capacity, int64_t head_dim, int64_t group,
                             int64_t selected, uint64_t* stats, int32_t* chan_idx, void* stream);

/* Subset slab of tokens [t_begin, t_end): the `selected` channels chan_idx
 * of each K row re-quantized as one int4 group.  slab holds rows *
 * capacity * selected/2 bytes, each row's codes in 4096-byte tiles of
 * 8192/selected keys: lane l of a tile owns keys [l*128/S, (l+1)*128/S) =
 * 64 logical bytes, whose logical byte b is stored at tile offset
 * (64*(b/16) + l)*16 + b%16 (b = (key % (128/S)) * S/2 + code byte).
 * slab_scales fp16 bits [rows,capacity] in key order.  selected in
 * {16,32,64,128}; capacity a multiple of 8192/selected.  int4 analogue of
 * the reference's dim-major K copy (EV:2018-2042). */
int qkv_int4_build_slab(const void* key, const int64_t* k_strides, int64_t batch,
                        int64_t kv_heads, int64_t t_begin, int64_t t_end, int64_t head_dim,
                        const int32_t* chan_idx, int64_t selected, uint8_t* slab,
                        uint16_t* slab_scales, int64_t capacity, int dtype, void* stream);

/* Per-row int8 query of decode scoring.  query [B,Hq,D] contiguous,
 * Hq = G * Hkv.  The G query heads of a row are summed over the row's
 * channels chan_idx (fp32, head order), quantized to int8 q8[s] =
 * rint(qg[s] / (amax/127)), and packed as qwords uint32 [rows, selected/4]:
 * dword 2d holds q8 of channels 8d, 8d+2, 8d+4, 8d+6 (bytes 0..3), dword
 * 2d+1 channels 8d+1, 8d+3, ...  qscale f32 [rows] (optional) receives
 * amax/127.  qkv_int4_decode_scores computes the same words itself; this
 * entry point exposes them.  The reference picks top-|q| dims per query head
 * instead (EV:4428, QK:123-145). */
int qkv_int4_query_words(const void* query, int64_t batch, int64_t q_heads, int64_t kv_heads,
                         int64_t head_dim, const int32_t* chan_idx, int64_t selected,
                         uint32_t* qwords, float* qscale, int dtype, void* stream);

/* Decode scoring over tokens [0, tokens) of every row, fused with block
 * max-pooling.  Replaces qabs_partial_scores_dim_major_forward (QK:63-96)
 * plus the block pool of EV:5038-5044.
 * query [B,Hq,D] contiguous, Hq = G * Hkv; chan_idx int32
 * [rows,selected].  I[t] = sum_s q8[s] * code[t,s] (int32) with q8 as
 * qkv_int4_query_words defines it; the ranking key is fp32(slab_scale[t]) *
 * fp32(I[t]).  bmax f32 [rows, ceil(tokens/block)] (block a power of two,
 * 1..8192/S).  isum int32 [rows,tokens] and keys f32 [rows,tokens] are
 * optional (NULL to skip); bmax may be NULL when both are given.  qscale f32
 * [rows] optional.  The slab is the tile layout qkv_int4_build_slab writes
 * (capacity a multiple of 8192/S). */
int qkv_int4_decode_scores(const void* query, int64_t batch, int64_t q_heads, int64_t kv_heads,
                           int64_t head_dim, const int32_t* chan_idx, int64_t selected,
                           const uint8_t* slab, const uint16_t* slab_scales, int64_t capacity,
                           int64_t tokens, int64_t block, float* bmax, int32_t* isum,
                           float* keys, float* qscale, int dtype, void* stream);

/* Top-k per row with the lowest-index tie-break: out int32 [rows,k] holds the
 * k indices first in (value descending, index ascending) order, written in
 * ascending index order.  values f32 [rows, n] with row stride ld; 1 <= k <= n.
 * -0 equals +0; NaN is outside the contract.  Replaces torch.topk at EV:4448
 * and EV:5046. */
int qkv_topk(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k,
             int32_t* out, void* stream);

/* Bytes of workspace qkv_topk_ws needs: 0 when qkv_topk's one workgroup per
 * row is used (n <= 4096 or k > 1024); for rows of at most 64 chunks of 4096
 * keys with ceil(n/4096) * k <= 32768, per chunk a 66-word histogram window
 * and a list of k (value, index) pairs with its count; otherwise two
 * candidate buffers of rows * (k * ceil(n/4096)) (value, index) pairs and
 * rows * ceil(n/4096) uint32 chunk bounds; -1 for bad sizes. */
int64_t qkv_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k);

/* qkv_topk with a caller-owned workspace (16-byte aligned, contents
 * irrelevant; calls sharing a workspace must not overlap in time): rows
 * longer than 4096 keys with k <= 1024 are split into 4096-key chunks.  Rows
 * of at most 64 chunks with chunks * k <= 32768: every chunk histograms its
 * keys (1/8-octave bins) around its own k-th key, the row's floor is the bin
 * where the merged count from the top reaches k, each chunk keeps its keys
 * at or above it (its exact top-k among them when more than k pass), and
 * the row's last chunk to finish selects from those lists -- one launch when
 * rows * chunks <= 256 (every workgroup resident at once; the row's chunks
 * count in ticket words the library keeps per GPU, 4 MiB held until the
 * process ends, in 4096 slots taken in turn: calls in flight together on one
 * GPU collide only when 4096 other calls were made between them; a call made
 * under stream capture keeps its slot for the graph's lifetime and the
 * process's, so at most 4095 captured calls per GPU), three otherwise.
 * Longer rows: stages
 * in which each chunk keeps its local
 * top-k until the candidates fit one chunk or one 1024-thread workgroup
 * (40960), keys below a lower bound of the row's k-th key left out after the
 * first stage.  The result equals qkv_topk's.  Same replaced call sites as
 * qkv_topk (EV:4448 token-level top-k over long contexts). */
int qkv_topk_ws(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                void* workspace, int64_t workspace_bytes, void* stream);

/* Token-level decode selection in one call: qkv_int4_decode_scores with
 * block 1 into scores f32 [batch * kv_heads, tokens], then qkv_topk_ws over
 * those rows into out int32 [rows, k] (the same result as the two calls).
 * workspace: qkv_topk_workspace_bytes(rows, tokens, k) bytes, 16-byte
 * aligned, contents irrelevant.  Where qkv_topk_ws takes its
 * histogram-and-filter path, the scoring launch (one workgroup per
 * 4096-token chunk) also builds each chunk's histogram window, so the top-k
 * starts at the row's floor.  Replaces the reference's partial scores plus
 * torch.topk at EV:5038-5046 for block 1 (no counterpart as one call). */
int qkv_int4_decode_topk(const void* query, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                         const int32_t* chan_idx, int64_t selected, const uint8_t* slab,
                         const uint16_t* slab_scales, int64_t capacity, int64_t tokens, int64_t k, float* scores,
                         int32_t* out, void* workspace, int64_t workspace_bytes, int dtype, void* stream);

/* No counterpart in the reference; for tests of qkv_topk_ws's one-launch
 * path.  Sets how long (ticks of the 100 MHz real-time clock) a chunk waits
 * for the other chunks of its row before keeping its exact top-k instead of
 * filtering by the row's floor (the result is the same either way); ticks < 0
 * restores the default (131072, about 1.3 ms).  Process-wide; takes effect
 * for launches after the call. */
int qkv_topk_set_wait_limit(int64_t ticks);

/* Bytes of workspace qkv_sparse_attention needs for these sizes: 65536
 * uint32 row tickets (the same words for every call shape), then G*(D+2)
 * floats per split.  The size also covers every call with the same batch
 * and heads and fewer selected slots (n_sel * block), so one workspace
 * serves all of them. */
int64_t qkv_sparse_attention_workspace_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads,
                                             int64_t head_dim, int64_t n_sel, int64_t block);

/* GQA-native sparse gather attention.  Replaces the reference's
 * gather/matmul/softmax fallback (EV:4490-4502) and final-attention kernel
 * (QK:335-419) without expanding K/V to the query heads (EV:6248-6251).
 * query [B,Hq,D] contiguous; key/value [B,Hkv,*,D] with
 * kv_strides = {b,h,t} (rows 16-byte aligned); block_ids int32 [rows,n_sel]
 * (ids outside [0, ceil(tokens/block)) are skipped); each block covers
 * tokens [id*block, min(tokens,(id+1)*block)).  Every query head of a row
 * attends, with softmax(scaling * q.k), over the union of the row's blocks.
 * out [B,Hq,D]; a head with no valid token gets zeros (QK:388, 404).
 * query, key, value and out share `dtype` (QKV_DTYPE_BF16 or
 * QKV_DTYPE_FP16; P is rounded to it before P.V, as the reference's
 * attention in that dtype does).
 * D must be 128.  One launch: the last workgroup of each row merges the
 * row's split partials.  The workspace's ticket words must be zero before
 * the first call that uses it (allocate it zero-filled); each completed call
 * leaves them zero.  Calls sharing a workspace must not overlap in time. */
int qkv_sparse_attention(const void* query, const void* key, const void* value,
                         const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                         int64_t kv_heads, int64_t tokens, int64_t head_dim,
                         const int32_t* block_ids, int64_t n_sel, int64_t block, float scaling,
                         float* workspace, int64_t workspace_bytes, void* out, int dtype, void* stream);

/* qkv_sparse_attention with the block selection fused in: replaces the
 * reference's top-k over pooled block scores (EV:5046) followed by its
 * final-attention kernel (QK:335-419).  bmax f32 [rows, >= bmax_ld] holds
 * the row's ceil(tokens/block) block maxima (as qkv_int4_decode_scores writes
 * them); each workgroup selects the n_sel largest (lowest index wins ties,
 * ascending -- exactly qkv_topk's selection) and attends over those blocks.
 * sel_out int32 [rows,n_sel], when not NULL, receives the selection.  At
 * most 4096 blocks per row (longer rows: qkv_topk_ws, then
 * qkv_sparse_attention).  Workspace as for qkv_sparse_attention. */
int qkv_sparse_attention_select(const void* query, const void* key, const void* value,
                                const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                int64_t kv_heads, int64_t tokens, int64_t head_dim, const float* bmax,
                                int64_t bmax_ld, int64_t n_sel, int64_t block, float scaling,
                                float* workspace, int64_t workspace_bytes, int32_t* sel_out, void* out,
                                int dtype, void* stream);

/* qkv_sparse_attention / qkv_sparse_attention_select with the reference's
 * protected tokens (EV:2938-2982, applied at EV:4460): the n_sel blocks are
 * chosen over the history [0, history) -- given in block_ids, or selected
 * in the kernel from bmax when block_ids is NULL (exactly one of the two) --
 * and the attention set is those blocks' tokens minus the sink range
 * [0, min(protect_sink, history)) and the recent range
 * [max(0, history - protect_recent), history), plus both ranges in full and,
 * when keep_self, the current token `history`; every token once.  K/V hold
 * at least history + 1 tokens when keep_self.  Workspace: at least
 * qkv_sparse_attention_workspace_bytes(B, Hq, Hkv, D, n_sel +
 * ceil(n_protected / block), block) with n_protected = sink + recent
 * tokens (not overlapping) + keep_self.  sel_out (with bmax only, may be
 * NULL) receives the selection. */
int qkv_sparse_attention_protected(const void* query, const void* key, const void* value,
                                   const int64_t* kv_strides, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                   int64_t history, int64_t head_dim, const int32_t* block_ids, const float* bmax,
                                   int64_t bmax_ld, int64_t n_sel, int64_t block, int64_t protect_sink,
                                   int64_t protect_recent, int keep_self, float scaling, float* workspace,
                                   int64_t workspace_bytes, int32_t* sel_out, void* out, int dtype,
                                   void* stream);

/* Streaming-read probe, no counterpart in the reference: reads `bytes` (a
 * positive multiple of 16 KiB, 16-byte aligned) once with the access shape
 * of qkv_int4_decode_scores -- whole 4 KiB tiles per wave, 16-byte
 * non-temporal loads, the next tile in flight -- and stores one fold word
 * per wave into sink (qkv_hbm_read_probe_sink_words words).  Its time is the
 * read ceiling of one launch of that size; the benchmark reports it. */
int64_t qkv_hbm_read_probe_sink_words(int64_t bytes);
int qkv_hbm_read_probe(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words, void* stream);

/* Bytes of the static device scratch behind
 * qkv_sparse_attention_select_noalloc (one copy per GPU, held until the
 * process ends). */
#define QKV_NOALLOC_SCRATCH_BYTES (8LL << 20)

/* qkv_sparse_attention_select without a workspace argument and without any
 * allocation: no counterpart in the reference.  It is for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  The workspace lives in a
 * static device array of QKV_NOALLOC_SCRATCH_BYTES per GPU; sizes whose
 * qkv_sparse_attention_workspace_bytes exceeds it fail with
 * QKV_ERR_UNSUPPORTED.  All calls on one GPU share that array, so calls that
 * overlap in time on one GPU (other streams, other threads) race; serialize
 * them.  Arguments and results as for qkv_sparse_attention_select. */
int qkv_sparse_attention_select_noalloc(const void* query, const void* key, const void* value,
                                        const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                        int64_t kv_heads, int64_t tokens, int64_t head_dim, const float* bmax,
                                        int64_t bmax_ld, int64_t n_sel, int64_t block, float scaling,
                                        int32_t* sel_out, void* out, int dtype, void* stream);

/* qkv_sparse_attention with one token list per query head (group size 1,
 * one-token blocks): row (b, h) attends over token_ids [B,Hq,n_ids] (ids
 * outside [0, tokens) skipped) of K/V head h / (Hq/Hkv).  Replaces the
 * reference's final-attention kernel (QK:335-419) on GQA-shaped K/V without
 * the repeat_interleave of EV:6248-6251.  Workspace:
 * qkv_sparse_attention_workspace_bytes(B, Hq, Hq, D, n_ids, 1). */
int qkv_token_attention(const void* query, const void* key, const void* value, const int64_t* kv_strides,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t tokens, int64_t head_dim,
                        const int32_t* token_ids, int64_t n_ids, float scaling, float* workspace,
                        int64_t workspace_bytes, void* out, int dtype, void* stream);

/* ======================================================================
 * Candidate reuse and exact rerank (the qabs{S}cand{pct}reuse[final|2set]
 * decode step, EV:3991-4397).  Rows are (sequence, query head)
 * r = b * Hq + h; a row reads K head h / (Hq/Hkv).  dtype selects bf16,
 * fp16 or fp32 for query and K.  Masks are uint8 0/1 (torch.bool) with
 * row stride mask_ld.
 * ====================================================================== */

/* Entries per row of the final index list: keep + sink range + recent
 * range (not overlapping the sink) + 1 when keep_self, with
 * keep = min(history, max(1, ceil(top_fraction * history))) (EV:4270,
 * 2938-2982).  -1 for history <= 0. */
int64_t qkv_reuse_final_count(int64_t history, int64_t protect_sink, int64_t protect_recent,
                              double top_fraction, int keep_self);

/* Workspace bytes of qkv_reuse_select for rows x history. */
int64_t qkv_reuse_select_workspace_bytes(int64_t rows, int64_t history, double top_fraction);

/* The reference's absent reuse_select kernel (EV:3881-3919, called at
 * EV:4200-4216), with the semantics of the fallback it replaces
 * (EV:4257-4365): full-D fp32 scores * scaling of the union current |
 * previous | previous_final (previous masks may be NULL; no sink/recent
 * protection in the union), the keep largest (lowest index wins ties),
 * valid where finite; history_final = the valid selections plus the first
 * protect_sink and last protect_recent history positions; final_indices /
 * final_valid [rows, n_out] = the selection in ascending index order with
 * protected entries invalid, then the sink range, the recent range and the
 * current token key_count - 1 (when keep_self).  attn_ids (optional) int32
 * [rows, n_out] holds the same list with -1 for invalid entries, ready for
 * qkv_token_attention.  query [B,Hq,D]; key [B,Hkv,key_count,D] with
 * k_strides {b,h,t,d} (d contiguous); history = key_count - 1.
 * history_final (row stride history_final_ld) may be the previous_final
 * buffer: it is written after every read of the masks. */
int qkv_reuse_select(const void* query, const void* key, const int64_t* k_strides, int dtype, int64_t batch,
                     int64_t q_heads, int64_t kv_heads, int64_t key_count, int64_t head_dim,
                     const uint8_t* current, const uint8_t* previous, const uint8_t* previous_final,
                     int64_t mask_ld, int64_t protect_sink, int64_t protect_recent, double top_fraction,
                     int keep_self, float scaling, void* workspace, int64_t workspace_bytes,
                     int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                     uint8_t* history_final, int64_t history_final_ld, void* stream);

/* qkv_reuse_select on bitsets: current, previous, previous_final and
 * history_final are bitsets (bit t % 64 of uint64 word t / 64, row stride
 * words_ld / history_final_ld words, 8-byte aligned) instead of byte masks;
 * everything else as qkv_reuse_select.  The compact state the reference
 * names for its reuse step (bitset OR of the masks, no dense per-token byte
 * mask); no reference counterpart as a kernel.  With value and out (may be
 * NULL): value [B,Hkv,key_count,D] with key's strides, out [B,Hq,D] in the
 * query's dtype -- the attention of qkv_token_attention over attn_ids is
 * run by the final selection's own workgroups (the reference's suggested
 * fusion of rerank and final attention) when the rows allow it (history <=
 * 40960, n_out <= 4096, D = 128, bf16 / fp16, 16-byte aligned rows);
 * *attended (host int, may be NULL) says whether it ran, else the caller
 * runs qkv_token_attention on attn_ids. */
int qkv_reuse_select_bits(const void* query, const void* key, const int64_t* k_strides, int dtype, int64_t batch,
                          int64_t q_heads, int64_t kv_heads, int64_t key_count, int64_t head_dim,
                          const uint64_t* current, const uint64_t* previous, const uint64_t* previous_final,
                          int64_t words_ld, int64_t protect_sink, int64_t protect_recent, double top_fraction,
                          int keep_self, float scaling, void* workspace, int64_t workspace_bytes,
                          int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                          uint64_t* history_final, int64_t history_final_ld, const void* value, void* out,
                          int* attended, void* stream);

/* qkv_reuse_select_bits followed by qkv_reuse_expand_blocks in one launch,
 * for the reuse...blk{bs} modes on bitsets (EV:4270-4316 with the block
 * expansion of EV:2914-2922): the final selection's bitset is expanded to
 * aligned blocks of `block` positions (1 <= block <= 4096) before it is
 * stored in history_final, and final_indices / final_valid / attn_ids
 * (optional) [rows, n_out] hold the expanded list exactly as
 * qkv_reuse_expand_blocks writes it (n_out = qkv_reuse_block_final_count).
 * Histories of at most 40960 positions (else QKV_ERR_UNSUPPORTED: run
 * qkv_reuse_select on byte masks and qkv_reuse_expand_blocks).  Workspace:
 * qkv_reuse_select_workspace_bytes.  No reference counterpart as a kernel
 * (the reference expands in PyTorch after its selection). */
int qkv_reuse_select_bits_blocks(const void* query, const void* key, const int64_t* k_strides, int dtype,
                                 int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                                 int64_t head_dim, const uint64_t* current, const uint64_t* previous,
                                 const uint64_t* previous_final, int64_t words_ld, int64_t protect_sink,
                                 int64_t protect_recent, double top_fraction, int keep_self, float scaling,
                                 int64_t block, void* workspace, int64_t workspace_bytes, int64_t* final_indices,
                                 uint8_t* final_valid, int32_t* attn_ids, int64_t n_out, uint64_t* history_final,
                                 int64_t history_final_ld, void* stream);

/* Workspace bytes of qkv_qabs_candidate_select (0 for histories of at most
 * 40960 positions, which one workgroup per row selects; -1 for bad sizes). */
int64_t qkv_qabs_candidate_select_workspace_bytes(int64_t rows, int64_t history, double candidate_fraction);

/* The candidate selection of the qabs{S}cand{pct}attn / appendattn modes
 * (_qabs_candidate_attention_forward EV:4419-4464): the keep =
 * min(history, max(1, ceil(candidate_fraction * history))) largest of
 * scores [rows, history] (row stride scores_ld; the fp32 partial scores of
 * qkv_reuse_partial_scores or partial_scores; lowest index wins ties), then
 * the final list of _qabs_final_indices_from_selected (EV:2938-2982) or,
 * with append, _qabs_final_indices_append_protected (EV:2985-3022, the
 * selected copies of protected tokens stay valid): final_indices /
 * final_valid / attn_ids (optional, -1 where invalid) [rows, n_out] = the
 * selection in ascending index order, then the sink range, the recent range
 * and the current token key_count - 1 (when keep_self); n_out =
 * qkv_reuse_final_count(history, protect_sink, protect_recent,
 * candidate_fraction, keep_self).  history_final [rows, history] (row stride
 * history_final_ld) = the selection plus the protected ranges.  workspace:
 * qkv_qabs_candidate_select_workspace_bytes bytes. */
int qkv_qabs_candidate_select(const float* scores, int64_t rows, int64_t key_count, int64_t scores_ld,
                              double candidate_fraction, int64_t protect_sink, int64_t protect_recent,
                              int keep_self, int append, void* workspace, int64_t workspace_bytes,
                              int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                              uint8_t* history_final, int64_t history_final_ld, void* stream);

/* Workspace bytes of qkv_qabs_candidates (-1 for bad arguments). */
int64_t qkv_qabs_candidates_workspace_bytes(int64_t rows, int64_t history, double candidate_fraction);

/* The exact candidate attention's selection in one call (EV:4400-4465):
 * qkv_reuse_partial_scores into partial over the history key_count - 1,
 * then qkv_qabs_candidate_select on those scores, the same outputs.  Rows of
 * at most 40960 history tokens and fewer than 128 rows: the partial scores
 * also count each row's leading 12 bits, and the selection runs across
 * several workgroups per row (the row's last workgroup resolves the
 * boundary and writes the list).  workspace:
 * qkv_qabs_candidates_workspace_bytes(batch * q_heads, key_count - 1,
 * candidate_fraction) bytes, 16-byte aligned, zero-filled before the first
 * call that uses it (allocate it zero-filled): it holds per-row counts and
 * tickets that every completed call leaves zero again.  Calls that share a
 * workspace use the same batch * q_heads and must not overlap in time.  No
 * reference counterpart as one call (QK:63-96, then EV:4448-4465). */
int qkv_qabs_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides, int dtype,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count, int64_t head_dim,
                        int64_t dim_count, double candidate_fraction, int64_t protect_sink, int64_t protect_recent,
                        int keep_self, int append, float* partial, int64_t partial_ld, void* workspace,
                        int64_t workspace_bytes, int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                        int64_t n_out, uint8_t* history_final, int64_t history_final_ld, void* stream);

/* The final index list of a given selection (_qabs_final_indices_from_selected
 * EV:2938-2982), as the periodic qabs{S}cand{pct}r{N}attn mode rebuilds it
 * from the indices the last refreshing step kept (EV:4535-4548, 4592-4600):
 * final_indices / final_valid / attn_ids (optional, -1 where invalid) [rows,
 * n_out] = selected[r, :n_sel] (row stride selected_ld), valid where the
 * index lies in [0, history) outside the first protect_sink and last
 * protect_recent history positions, then the sink range, the recent range
 * (not overlapping the sink) and the current token key_count - 1 (when
 * keep_self); n_out = n_sel + that many protected entries. */
int qkv_final_indices_from_selected(const int64_t* selected, int64_t selected_ld, int64_t n_sel, int64_t rows,
                                    int64_t key_count, int64_t protect_sink, int64_t protect_recent, int keep_self,
                                    int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                                    void* stream);

/* Workspace bytes of qkv_candidate_mask (0 for previous_threshold, -1 for
 * bad arguments). */
int64_t qkv_candidate_mask_workspace_bytes(int64_t rows, int64_t n, int selection, int64_t k, int64_t n_sample);

/* Candidate mask of the reuse step under each candidate selection of the
 * reference (_select_qabs_candidate_from_partial_scores EV:3958-3989):
 * mask[r, t] = values[r, t] >= thresholds[r] for t < n, where the
 * threshold is
 *   QKV_CAND_TOPK: the row's k-th largest value (EV:3988; written to
 *     thresholds when that is not NULL);
 *   QKV_CAND_SAMPLE_QUANTILE: the k-th largest of values[r, sample_cols[i]],
 *     i < n_sample (EV:3972-3987; the caller passes the sampled columns,
 *     the reference's rounded linspace, each in [0, n) - they are device
 *     data and not checked - and k = the sample's budget), written to
 *     thresholds;
 *   QKV_CAND_PREVIOUS_THRESHOLD: thresholds[r] as given (EV:3967-3971).
 * values f32 [rows, ld]; mask uint8 row stride mask_ld, or bits (a bitset:
 * bit t % 64 of uint64 word t / 64, row stride bits_ld words, 8-byte
 * aligned) -- exactly one of the two; thresholds f32 [rows] (required for
 * the last two). */
int qkv_candidate_mask(const float* values, int64_t rows, int64_t n, int64_t ld, int selection, int64_t k,
                       const int32_t* sample_cols, int64_t n_sample, float* thresholds, uint8_t* mask,
                       int64_t mask_ld, uint64_t* bits, int64_t bits_ld, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* The refresh test of the lagged reuse modes (lagtop2 / lagrefresh{N} /
 * qdrift[maj|head|share|cos|coshead] / pconf{T} before qabs{S}cand{pct},
 * _qabs_reuse_fast_attention_forward EV:4020-4087).  One row per (sequence,
 * query head).  Always writes the row's top-|q| dims (count = clamp(dim_count,
 * 1, head_dim); descending |q|, equal magnitudes to the lower dim, EV:4026)
 * to dims_out and q at them to values_out, both [rows, count]: the state the
 * next step's test reads as previous_dims / previous_values.  Then, into
 * flags[r] (1 = the row refreshes):
 *   QKV_LAG_OVERLAP: fewer than max(1, ceil(count / 2)) of the dims are among
 *     previous_dims[r] (EV:4045-4048);
 *   QKV_LAG_COS: that, or the cosine of q on previous_dims[r] with
 *     previous_values[r] (denominator clamped to 1e-6) is below 0.5
 *     (EV:4049-4056);
 *   QKV_LAG_ESS: over the set positions t < history of previous_final[r]
 *     (row stride mask_ld), s_t = q . K[t] rounded to the input dtype, times
 *     scaling rounded again; weights softmax(s); flagged when the mask is
 *     empty or (1 / sum w^2) / count > ess_threshold (EV:4068-4087).
 * query [B,Hq,D] (D <= 128); key [B,Hkv,>=history,D] with k_strides
 * {b,h,t,d} (d contiguous), read by QKV_LAG_ESS only.  history < 2^30.
 * QKV_LAG_ESS also takes a workspace of
 * qkv_reuse_lag_flags_workspace_bytes(batch * q_heads, history) bytes (its
 * per-span partial sums; contents need no clearing); the other tests none. */
int qkv_reuse_lag_flags(const void* query, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t dim_count, int test, const int32_t* previous_dims,
                        const float* previous_values, int32_t* dims_out, float* values_out, const void* key,
                        const int64_t* k_strides, int64_t history, const uint8_t* previous_final, int64_t mask_ld,
                        float scaling, float ess_threshold, uint8_t* flags, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* Workspace bytes of qkv_reuse_lag_flags' QKV_LAG_ESS test (-1 for bad sizes). */
int64_t qkv_reuse_lag_flags_workspace_bytes(int64_t rows, int64_t history);

/* The candidates of a lagged reuse step (EV:4089-4145): qkv_reuse_partial_scores
 * into partial, then qkv_threshold_mask (mask = partial >= the row's k-th
 * largest; workspace of qkv_threshold_mask_workspace_bytes(batch * q_heads,
 * history, k) bytes), for the rows that refresh under `refresh`
 * (QKV_REFRESH_*, from flags [batch * q_heads] for the last three; nothing
 * runs under QKV_REFRESH_NONE).  The other rows' partial and mask rows are
 * left as they were (qkv_reuse_lag_union clears their candidates); rows
 * longer than 40960 positions are all computed. */
int qkv_reuse_lag_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides, int dtype,
                             int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history, int64_t head_dim,
                             int64_t dim_count, int64_t k, const uint8_t* flags, int refresh, float* partial,
                             int64_t partial_ld, uint8_t* mask, int64_t mask_ld, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* The candidate union of a lagged reuse step (EV:4089-4175), for
 * qkv_reuse_select with no previous masks.  A row refreshes per `refresh`
 * (QKV_REFRESH_*, from flags [batch * q_heads] for the last three); the
 * current candidates of a row that does not refresh are set to 0 (read
 * only for rows that refresh).  union_out[r, t] = current[r, t] (refreshed
 * rows) | previous_final[r, t] (when not NULL) | (with share) current[r', t]
 * for any refreshed row r' of the same sequence | t < protect_sink | t >=
 * history - protect_recent, for t < history.  current, previous_final row
 * stride mask_ld; union_out row stride union_ld. */
int qkv_reuse_lag_union(uint8_t* current, const uint8_t* previous_final, int64_t mask_ld, const uint8_t* flags,
                        int64_t batch, int64_t q_heads, int64_t history, int refresh, int share,
                        int64_t protect_sink, int64_t protect_recent, uint8_t* union_out, int64_t union_ld,
                        void* stream);

/* The lagged modes' three calls on bitset state (bit t % 64 of uint64 word
 * t / 64, row strides in words, 8-byte aligned), everything else as the
 * byte-mask calls above; no reference counterparts as kernels (the
 * reference keeps these masks as torch bool tensors, EV:4020-4198).
 * qkv_reuse_lag_flags_bits: QKV_LAG_ESS reads previous_final as a bitset.
 * qkv_reuse_lag_candidates_bits: the candidate bits of the refreshing rows
 * (the rows that do not refresh are left as they were), with the workspace
 * of qkv_reuse_candidates_workspace_bytes(batch * q_heads, history, k)
 * bytes, zero-filled before the first call and left zero by every call
 * (rows of up to 40960 positions select across several workgroups).
 * qkv_reuse_lag_union_bits: the union of qkv_reuse_lag_union into a bitset
 * (words past the history are not written). */
int qkv_reuse_lag_flags_bits(const void* query, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t head_dim, int64_t dim_count, int test, const int32_t* previous_dims,
                             const float* previous_values, int32_t* dims_out, float* values_out, const void* key,
                             const int64_t* k_strides, int64_t history, const uint64_t* previous_final,
                             int64_t words_ld, float scaling, float ess_threshold, uint8_t* flags, void* workspace,
                             int64_t workspace_bytes, void* stream);
int qkv_reuse_lag_candidates_bits(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                  int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history,
                                  int64_t head_dim, int64_t dim_count, int64_t k, const uint8_t* flags, int refresh,
                                  float* partial, int64_t partial_ld, uint64_t* bits, int64_t bits_ld,
                                  void* workspace, int64_t workspace_bytes, void* stream);
int qkv_reuse_lag_union_bits(uint64_t* current, const uint64_t* previous_final, int64_t words_ld,
                             const uint8_t* flags, int64_t batch, int64_t q_heads, int64_t history, int refresh,
                             int share, int64_t protect_sink, int64_t protect_recent, uint64_t* union_out,
                             int64_t union_ld, void* stream);

/* qkv_reuse_expand_blocks on a bitset final selection (bit t % 64 of uint64
 * word t / 64, row stride history_final_ld words, 8-byte aligned), any
 * history: the same expanded bitset and list. */
int qkv_reuse_expand_blocks_bits(uint64_t* history_final, int64_t history_final_ld, int64_t rows,
                                 int64_t key_count, int64_t block, int64_t protect_sink, int64_t protect_recent,
                                 double top_fraction, int keep_self, int64_t* final_indices, uint8_t* final_valid,
                                 int32_t* attn_ids, int64_t n_out, void* stream);

/* Entries per row of the final index list of a block-expanded reuse step
 * (the qabs{S}cand{pct}reuse[final|2set]blk{block} modes): body + sink
 * range + recent range (not overlapping the sink) + 1 when keep_self, where
 * body = min(history positions outside the protected ranges,
 * keep * block + 2 * (block - 1)) bounds the expanded selection outside the
 * protected ranges.  -1 for history <= 0 or block < 1. */
int64_t qkv_reuse_block_final_count(int64_t history, int64_t block, int64_t protect_sink,
                                    int64_t protect_recent, double top_fraction, int keep_self);

/* Block expansion of a reuse step's final selection, replacing the
 * reference's mask-level steps for the blk modes (EV:4314-4316:
 * _expand_history_keep_to_aligned_blocks EV:2914-2922, then the selection
 * re-read by _indices_from_keep_mask EV:2896-2911 and the final list of
 * EV:2938-2982).  history_final [rows, history] (row stride
 * history_final_ld, as qkv_reuse_select left it) is expanded in place:
 * every aligned block of `block` positions (1 <= block <= 4096; the last
 * block cut at the history) that holds a set flag becomes wholly set.
 * final_indices / final_valid / attn_ids (optional) [rows, n_out] are
 * rewritten: the expanded positions outside the sink and recent ranges in
 * ascending order (the reference lists them descending; the set is the
 * same), padded to the body bound of qkv_reuse_block_final_count with
 * (0, invalid, -1), then the sink range, the recent range and the current
 * token key_count - 1 (when keep_self). */
int qkv_reuse_expand_blocks(uint8_t* history_final, int64_t history_final_ld, int64_t rows, int64_t key_count,
                            int64_t block, int64_t protect_sink, int64_t protect_recent, double top_fraction,
                            int keep_self, int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                            int64_t n_out, void* stream);

/* Partial scores of the reuse step (EV:4123-4135 on the dim-major copy,
 * partial_scores_dim_major QK:63-96 with the dims of QK:120-145): for each
 * row, the top-|q| dim_count dims (descending |q|, lower dim first on ties,
 * clamped to [1, min(D, 128)]) and out[r, t] = sum_s q[d_s] * K[d_s, t] in
 * selection order, fp32.  key_dim_major [B,Hkv,D,*] with strides {b,h,d,t}
 * (t contiguous); out row stride out_ld. */
int qkv_reuse_partial_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides, int dtype,
                             int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history, int64_t head_dim,
                             int64_t dim_count, float* out, int64_t out_ld, void* stream);

/* Workspace bytes of qkv_threshold_mask. */
int64_t qkv_threshold_mask_workspace_bytes(int64_t rows, int64_t n, int64_t k);

/* Candidate mask of the reuse step (EV:4136-4144, 3988-3989):
 * mask[r, t] = values[r, t] >= the row's k-th largest value (ties at the
 * threshold all kept).  values f32 [rows, >= ld]; mask uint8 row stride
 * mask_ld. */
int qkv_threshold_mask(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, uint8_t* mask,
                       int64_t mask_ld, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of qkv_reuse_candidates for rows = batch * q_heads (-1
 * for bad arguments). */
int64_t qkv_reuse_candidates_workspace_bytes(int64_t rows, int64_t history, int64_t k);

/* The reuse step's candidates (EV:3988, 4136-4144): qkv_reuse_partial_scores
 * into partial (row stride partial_ld), then mask = partial >= the row's
 * k-th largest (qkv_threshold_mask), as a byte mask (mask, row stride
 * mask_ld) or a bitset (bits: bit t % 64 of uint64 word t / 64, row stride
 * bits_ld words, 8-byte aligned) -- exactly one of the two; thr_out f32
 * [batch * q_heads] (optional) receives the k-th largest.  Rows of at most
 * 40960 history tokens: one launch per call for 128 rows and more
 * (head_dim <= 128, a 16-byte aligned copy); for fewer rows with a bitset
 * the partial scores also count each row's leading 12 bits and a second
 * launch selects with several workgroups per row; otherwise the two
 * launches of qkv_reuse_partial_scores and qkv_threshold_mask.
 * workspace: qkv_reuse_candidates_workspace_bytes(batch * q_heads, history,
 * k) bytes, 16-byte aligned, zero-filled before the first call that uses
 * it (allocate it zero-filled): it holds per-row counts and tickets that
 * every completed call leaves zero again.  Calls that share a workspace use
 * the same batch * q_heads and must not overlap in time.  No reference counterpart as one call: the
 * reference runs the two steps separately (QK:63-96, then torch.topk at
 * EV:3988). */
int qkv_reuse_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides, int dtype,
                         int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history, int64_t head_dim,
                         int64_t dim_count, int64_t k, float* partial, int64_t partial_ld, uint8_t* mask,
                         int64_t mask_ld, uint64_t* bits, int64_t bits_ld, float* thr_out, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* Dim-major copy of K tokens [t_begin, t_end): key_dim_major[b, j, d, t] =
 * key[b, j, t, d] (the reference's incremental transposed copy,
 * EV:2018-2042, kept per KV head).  k_strides {b,h,t,d} (d contiguous);
 * kdm_strides {b,h,d,t} (t contiguous).  head_dim <= 512 (256 for fp32). */
int qkv_dim_major_append(const void* key, const int64_t* k_strides, int dtype, int64_t batch, int64_t kv_heads,
                         int64_t head_dim, int64_t t_begin, int64_t t_end, void* key_dim_major,
                         const int64_t* kdm_strides, void* stream);

/* ======================================================================
 * Block-metadata selectors: the qbb{bs}q{S}s{scan}cand{c} (Quest-style
 * channel bounds, EV:5508-5617) and brep{bs}r{R}q{S}s{scan}cand{c} (block
 * representatives, EV:5361-5505, BlockRepState EV:1853-1918) decode steps.
 * K/V [B,Hkv,*,128] with k_strides {b,h,t,d} (d contiguous, rows 16-byte
 * aligned); rows r = b * Hq + h read K head h / (Hq/Hkv).  Query, K and the
 * dim-major copy share `dtype` (QKV_DTYPE_BF16 or QKV_DTYPE_FP16), the last
 * argument before the stream; qbb metadata is stored in that dtype.
 * ====================================================================== */

/* Bytes of block metadata for meta_blocks blocks per (sequence, KV head):
 * qbb 512 per block ([min(128) | max(128)] in K's dtype), brep 4*reps per block
 * (int32 token ids).  -1 for a bad kind or size. */
int64_t qkv_block_meta_bytes(int kind, int64_t batch, int64_t kv_heads, int64_t meta_blocks, int64_t reps);

/* Rebuilds the metadata of the blocks holding tokens [t_begin, t_end) from
 * K's tokens below t_end: per-channel min/max (qbb), or the reps tokens of
 * largest squared norm (fp32 sum in channel order), descending, lower index
 * on ties, -1 padding (brep; 1 <= reps <= min(block, 64), any block).  The reference recomputes these
 * every step (EV:5536-5553) or per new block (EV:1884-1918). */
int qkv_block_meta_update(int kind, const void* key, const int64_t* k_strides, int64_t batch, int64_t kv_heads,
                          int64_t head_dim, int64_t block, int64_t reps, int64_t t_begin, int64_t t_end, void* meta,
                          int64_t meta_blocks, int dtype, void* stream);

/* Block scores of each row over ceil(history/block) blocks: qbb the bound
 * sum_s q_s * (q_s >= 0 ? max : min) over the row's top-|q| dims (EV:5554),
 * brep the largest partial score of the block's representatives
 * (EV:5431-5435).  Dims as qkv_reuse_partial_scores.  out f32 [rows, out_ld]. */
int qkv_block_scores(int kind, const void* query, const void* key, const int64_t* k_strides, const void* meta,
                     int64_t meta_blocks, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history,
                     int64_t head_dim, int64_t block, int64_t reps, int64_t dim_count, float* out, int64_t out_ld,
                     int dtype, void* stream);

/* Partial scores of the tokens of each row's chosen blocks (EV:5576-5581):
 * position p is token blocks[r, p / block] * block + p % block, scored on
 * the row's top-|q| dims from the dim-major K copy (qkv_dim_major_append);
 * positions at or past history get -inf.  out f32 [rows, >= n_scan*block].
 * full (optional, same layout and out_ld; NULL: not written): each
 * position's full-D score scaling * q.K in the reference's fp32 order, read
 * from key ([B,Hkv,*,D] with k_strides, rows 16-byte aligned) -- the
 * scores qkv_block_rerank ranks its candidates by, computed here across the
 * launch's workgroups instead of in one workgroup per row. */
int qkv_block_scan_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                          const void* key, const int64_t* k_strides, int64_t batch, int64_t q_heads,
                          int64_t kv_heads, int64_t history, int64_t head_dim, const int32_t* blocks, int64_t n_scan,
                          int64_t block, int64_t dim_count, float scaling, float* out, float* full, int64_t out_ld,
                          int dtype, void* stream);

/* Block scores of the qboracle selector (EV:5030-5044): out[r, j] = the
 * largest partial score, on row r's top-|q| dims (ties to the lower dim,
 * summed in selection order), of block j's history tokens
 * [j*block, min(history, (j+1)*block)), read from the dim-major K copy
 * (qkv_dim_major_append).  query [B,Hq,D]; out f32 [rows, >= out_ld],
 * rows = B*Hq; any block length. */
int qkv_block_max_partial_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                 int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history, int64_t head_dim,
                                 int64_t block, int64_t dim_count, float* out, int64_t out_ld, int dtype,
                                 void* stream);

/* Replaces brep_partial_scores, which the reference imports from its
 * extension module but never shipped (wrapper EV:3847-3877, call
 * EV:5419-5431, signature `brep_partial_scores(query, key_history,
 * rep_indices, rep_valid, block_size, dim_count, scan_fraction)`).
 * query f32 [B,H,D] contiguous (the reference passes the fp32 query);
 * key_history [B,H,T,D] of key_dtype with k_strides {b,h,t,d}, d contiguous;
 * rep_indices int64 and rep_valid u8, both [B,H,ceil(T/block_size),reps]
 * contiguous (the reference's BlockRepState, EV:1857-1918).  out f32
 * [B,H,T]: the partial score over the row's min(max(dim_count,1), D, 128)
 * largest-|q| dims (ties to the lower dim), summed in that order, for every
 * token of the min(blocks, max(1, ceil(scan_fraction * T / block_size)))
 * blocks whose best valid representative scores highest (a block without
 * one scores finfo(float32).min; ties to the lower block); -inf elsewhere.
 * At most 40960 blocks per row. */
int qkv_brep_partial_scores(const float* query, const void* key_history, const int64_t* rep_indices,
                            const uint8_t* rep_valid, float* out, int key_dtype, int64_t batch, int64_t heads,
                            int64_t history, int64_t head_dim, const int64_t* k_strides, int64_t reps,
                            int64_t block_size, int64_t dim_count, double scan_fraction, void* stream);

/* Entries of a final token list: n_keep + sink range + recent range (not
 * overlapping the sink) + 1 when keep_self.  -1 for history <= 0. */
int64_t qkv_final_list_count(int64_t history, int64_t n_keep, int64_t protect_sink, int64_t protect_recent,
                             int keep_self);

/* Rerank of each row (EV:5583-5605): the n_cand best scanned history tokens
 * by partial score -- with unscanned != 0 (qboracle) every history token
 * ranks, the unscanned ones at finfo(float32).min behind every scanned one
 * (EV:5055-5058), so candidates past the scanned tokens are the lowest
 * unscanned ones -- their full-D fp32 scores * scaling, the n_keep best of
 * those (ties to the lower token throughout), then keep_mask [rows,
 * key_count] (kept tokens, the first protect_sink and last protect_recent
 * history tokens, the current token when keep_self; EV:5607-5615) and
 * attn_ids [rows, n_out] for qkv_token_attention: the kept tokens ascending
 * (-1 where protected or not filled), the sink range, the recent range, the
 * current token.  n_keep <= n_cand.  Rows of at most 40960 scanned positions
 * and 4096 candidates (and, with unscanned, no more candidates than
 * scanned history tokens) take one workgroup each and no workspace; full
 * (optional, partial's layout) then holds the full scores
 * qkv_block_scan_scores wrote (NULL: computed here from key).  Other rows
 * take five launches over `workspace` (256-byte aligned, at least
 * qkv_block_rerank_workspace_bytes; full unused). */
int qkv_block_rerank(const void* query, const void* key, const int64_t* k_strides, int64_t batch, int64_t q_heads,
                     int64_t kv_heads, int64_t key_count, int64_t head_dim, const float* partial, const float* full,
                     int64_t partial_ld, const int32_t* blocks, int64_t n_scan, int64_t block, int64_t n_cand,
                     int64_t n_keep,
                     int64_t protect_sink, int64_t protect_recent, int keep_self, float scaling, uint8_t* keep_mask,
                     int64_t keep_ld, int32_t* attn_ids, int64_t n_out, int unscanned, void* workspace,
                     int64_t workspace_bytes, int dtype, void* stream);

/* Bytes of workspace qkv_block_rerank needs for these sizes: 0 when every
 * row fits one workgroup, -1 for bad sizes (rows = B*Hq, history =
 * key_count - 1). */
int64_t qkv_block_rerank_workspace_bytes(int64_t rows, int64_t history, int64_t n_scan, int64_t block,
                                         int64_t n_cand, int64_t n_keep, int unscanned);

/* ======================================================================
 * Chunked-prefill block selection (no reference counterpart: the reference
 * prefills with dense attention, EV:7079-7111, dense QK at EV:6602-6604).
 * ====================================================================== */

/* Per-row int8 quantization of prefill queries: query rows of 128
 * channels (row_stride elements apart), q8 = clamp(rint(q / (amax/127)),
 * +-127) per row, written as int8 [rows,128] in the permuted order the MFMA
 * scoring kernel consumes: channel c at byte 32*(c/32) + 16*((c/16)%2) +
 * 8*((c%16)/8) + 4*(c%2) + (c%8)/2 (q8 2-byte aligned).  qscale f32 [rows]
 * optional.  dtype: QKV_DTYPE_BF16 or QKV_DTYPE_FP16. */
int qkv_prefill_quantize_query(const void* query, int64_t rows, int64_t head_dim, int64_t row_stride,
                               int8_t* q8, float* qscale, int dtype, void* stream);

/* Block maxima of a query chunk against the whole cached K, on int8 MFMA.
 * q8 [B,Hq,queries,128] from qkv_prefill_quantize_query; packed uint8
 * [B,Hkv,capacity,64] and scales fp16 bits [B,Hkv,capacity] are K packed
 * with group 128 (qkv_int4_pack_k).  Query i sits at position q_pos0 + i and
 * sees keys t <= q_pos0 + i, t < tokens.  key = fp32(scale[t]) * fp32(I),
 * I = sum over 128 channels of q8 * code (exact int32); bmax f32
 * [B,Hq,queries,ceil(tokens/block)] is the max over each block's visible
 * keys (-inf if none), -0 read as +0.  block must be 64. */
int qkv_prefill_block_scores(const int8_t* q8, int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t queries, const uint8_t* packed, const uint16_t* scales,
                             int64_t capacity, int64_t tokens, int64_t q_pos0, int64_t head_dim,
                             int64_t block, float* bmax, void* stream);

/* Top-k blocks per row of bmax f32 [rows,n] (row stride ld, n <= 4096) as
 * qkv_topk does it, except that blocks whose value is -inf are never
 * selected: a row with fewer than k finite blocks lists those in ascending
 * order and pads with -1.  out int32 [rows,k]. */
int qkv_prefill_block_topk(const float* bmax, int64_t rows, int64_t n, int64_t ld, int64_t k,
                           int32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QKV_H_ */
