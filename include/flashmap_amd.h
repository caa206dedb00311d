/*
 * flashmap_amd.h - C ABI of the MI355X (gfx950) kernels for the FlashMap drafter's
 * cross-attention hot path: the per-layer QK-RMSNorm + RoPE prologue, the block
 * attention of K draft slots onto the target's context keys/values (contiguous,
 * block-paged and token-paged KV), the in-block self-attention and the context-KV
 * writers that produce the paged layouts.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers unless stated; tensors are bf16 (passed as void*),
 *     float32 (float*) or integer as typed. Strides are in ELEMENTS, not bytes.
 *   - Nothing is allocated and nothing synchronizes: work is enqueued on `stream`
 *     (a hipStream_t passed as void*; NULL = the legacy default stream).
 *   - Return FM_OK (0) or an FM_ERR_* code; fm_last_error() then describes the
 *     failure (thread-local string owned by the library).
 *   - RoPE rotates interleaved channel pairs (2i, 2i+1). A rotary table is given as
 *     two float32 arrays: cos and sin of pair i at table row r are
 *       rope_cos[r * rope_row_stride + i * rope_pair_stride]   (same for rope_sin).
 *     The row of token t is positions[t] when `positions` is non-NULL, else t.
 *     rope_rows (> 0) bounds the row index (rows are clamped into [0, rope_rows)).
 *   - RMSNorm is x * bf16(w * rsqrt(mean(x^2) + eps)), the product rounded to bf16.
 */
#ifndef FLASHMAP_AMD_H
#define FLASHMAP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FM_OK = 0,
  FM_ERR_INVALID = 1,     /* bad shape, stride, dtype contract or NULL pointer */
  FM_ERR_UNSUPPORTED = 2, /* a shape the kernels do not implement (e.g. head_dim) */
  FM_ERR_WORKSPACE = 3,   /* workspace missing or smaller than fm_*_workspace_bytes */
  FM_ERR_HIP = 4          /* a HIP runtime call failed (launch, attribute query) */
};

#define FM_ABI_VERSION 1

/* Library metadata and errors. No reference counterpart (the reference raises Python
 * exceptions: assert / ValueError in flashmap/vllm/kernels.py:51,112,341-342). */
const char *fm_last_error(void);
int fm_abi_version(void);
/* Compute units of `device` (the split-KV planner sizes its grid from it). */
int fm_device_cus(int device, int *num_cus);

/* ---------------------------------------------------------------------------------
 * a2/a3  Q prologue: RMSNorm of every (token, head) row of x, then RoPE.
 * Replaces flashmap_vllm::rms_norm_rope (flashmap/vllm/kernels.py:101-124; table
 * rows gathered at positions) and flashmap_sglang::rms_norm_rope
 * (flashmap/sglang/kernels.py:171-189; one table row per token, positions = NULL);
 * same math as FlashMapAttention's q_norm + apply_rope
 * (flashmap/modeling_flashmap.py:61-80,145). x and out: (tokens, heads, head_dim)
 * bf16 with the given token/head strides (unit stride inside a head).
 * head_dim in {64, 128}.
 */
int fm_rms_norm_rope(const void *x, void *out, int64_t tokens, int32_t heads, int32_t head_dim,
                     int64_t x_stride_token, int64_t x_stride_head, int64_t out_stride_token,
                     int64_t out_stride_head, const float *weight, const float *rope_cos,
                     const float *rope_sin, int64_t rope_row_stride, int64_t rope_pair_stride,
                     int64_t rope_rows, const int64_t *positions, float eps, void *stream);

/* ---------------------------------------------------------------------------------
 * a5/a6/a7  Block attention: for each sequence b, its q_len(b) draft rows of every
 * query head attend, non-causally, to the first seqlen(b) context positions:
 *   out = softmax(Q K^T * softmax_scale) V
 * in fp32 with P rounded to bf16 before P.V, output rounded to bf16 once.
 * GQA: query head hq attends to KV head hq / (num_q_heads / num_kv_heads).
 *
 * Query / output rows: token t of sequence b is row cu_seqlens_q[b] + t when
 * cu_seqlens_q is non-NULL (varlen, strides *_stride_token / *_stride_head), else
 * b * *_stride_batch + t * *_stride_token. q_len(b) = cu_seqlens_q[b+1] -
 * cu_seqlens_q[b] (<= max_seqlen_q) or max_seqlen_q.
 *
 * Optional fused Q prologue: with q_norm_weight non-NULL the call reads the
 * pre-norm projection q and applies fm_rms_norm_rope's math itself, bit-identically
 * (the rope row of query token row i is q_positions[i] or i, i being the varlen row
 * index cu_seqlens_q[b] + t, or b * max_seqlen_q + t without cu_seqlens_q).
 *
 * One call enqueues three kernels: the query pass (each (sequence, KV head) unit's
 * G x q_len rows packed contiguously in the workspace, with the prologue applied), the
 * split-KV attention and the fp32 log-sum-exp combine that writes `out`. Split-KV:
 * the context of all sequences is cut into equal shares over a persistent grid (one
 * share per workgroup); every (unit, share) segment leaves a partial (fp16 values
 * with a per-row scale, fp32 log-sum-exp) that the combine merges. `plan` is fm_attn_plan's output for this step (it depends only on
 * the context lengths, so every layer of a step may share it); NULL plans inside the
 * call, in the workspace. `workspace` must hold fm_attn_workspace_bytes(...) bytes for
 * the same arguments (packed queries, partials, plan); it is scratch that concurrent
 * calls must not share.
 * head_dim in {64, 128}; num_q_heads % num_kv_heads == 0.
 * A sequence with seqlen(b) == 0 gets zeros (vLLM's seqused_k = 0 rows).
 * ------------------------------------------------------------------------------ */

/* Bytes of the plan buffer for `batch` sequences: 2 (batch + 1) int32, the prefixes of the
 * sequences' tile counts for bf16 K/V (tiles of 32 positions) and for e4m3 K/V (tiles of 64
 * positions), so one step plan serves calls onto caches of either kind. */
size_t fm_attn_plan_bytes(int32_t batch);
/* Writes the step's plan from seqlens (batch,) int32 into `plan` (device, int32).
 * Replaces get_scheduler_metadata (flashmap/vllm/model.py:967-989,
 * flashmap/sglang/model.py:189-204). */
int fm_attn_plan(const int32_t *seqlens, int32_t batch, int32_t *plan, void *stream);

/* Workspace bytes an attention call with these sizes needs on `device`. */
size_t fm_attn_workspace_bytes(int32_t batch, int32_t max_seqlen_q, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t max_seqlen_k,
                               int device);

/* a5: contiguous KV, the FlashMapCache layout (flashmap/modeling_flashmap.py:195-219):
 * K and V views (batch, kv_heads, positions, head_dim) with arbitrary strides.
 * seqlens_k NULL: every sequence attends to kv_len positions (FlashMapCache.context(end)).
 * Replaces F.scaled_dot_product_attention in FlashMapAttention.forward
 * (flashmap/modeling_flashmap.py:144-147). */
int fm_block_attn_contig(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *k, int64_t k_stride_batch, int64_t k_stride_head,
    int64_t k_stride_pos, const void *v, int64_t v_stride_batch, int64_t v_stride_head,
    int64_t v_stride_pos, const int32_t *seqlens_k, int32_t kv_len, int32_t batch,
    int32_t max_seqlen_q, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream);

/* a6: block-paged KV, vLLM's FlashAttention cache as the FlashMap plugin views it
 * ((num_blocks, kv_heads, page_size, 2 * head_dim): K then V in every token row;
 * flashmap/vllm/model.py:93-139,707-733). Position p of sequence b lives in page
 * block_table[b * block_table_stride + p / page_size] at token p % page_size:
 *   K = kv_cache + page * stride_block + head * stride_head + (p % page) * stride_token
 *   V = K + v_offset.
 * Page ids are clamped into [0, num_blocks), block-table columns into
 * [0, block_table_width). Replaces flashmap_vllm::paged_cross_attention
 * (flashmap/vllm/model.py:93-134, i.e. vllm_flash_attn.flash_attn_varlen_func with
 * causal=False). */
int fm_block_attn_paged(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
    int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream);

/* fm_block_attn_paged for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). It has no
 * counterpart in the reference. It takes fm_block_attn_paged's arguments without the
 * workspace and uses instead a scratch array the library holds in device memory
 * (fm_static_scratch_bytes() = 32 MiB per GPU it runs on, kept until the process ends);
 * it allocates nothing and never synchronizes. A call whose split-KV scratch would exceed
 * the array fails with FM_ERR_WORKSPACE. Every call on one GPU shares that GPU's array:
 * calls that may overlap in time on one GPU (two streams, two threads) race on it. No
 * part of the array has to start cleared (each call writes what it later reads). Every
 * process that loads the library holds the array on each GPU it uses, whether or not it
 * calls this entry point. Before the first call on a device is captured into a graph,
 * call fm_static_scratch_init() with that device current (or make one eager call): it
 * resolves the array's address and fills the host-side caches a first call would query. */
size_t fm_static_scratch_bytes(void);
int fm_static_scratch_init(void);
int fm_block_attn_paged_static(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks, int64_t stride_block,
    int64_t stride_head, int64_t stride_token, int64_t v_offset, int32_t page_size,
    const int32_t *block_table, int64_t block_table_stride, int64_t block_table_width,
    const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *stream);

/* f4: one drafter layer's paged attention over vLLM's virtual context-cache layout
 * (flashmap/vllm/context_cache.py:33-73), where the layer's KV heads lie in runs across
 * several caches of one geometry and one block table: run r holds the next run_count[r]
 * KV heads (in order, from head 0) at head slots run_first_slot[r] .. of the cache at
 * run_caches[r] (a host array of device pointers; heads_per_cache heads per cache). One
 * launch replaces attend_by_segments' per-run flashmap_vllm::paged_cross_attention calls
 * and the concatenation of their outputs (flashmap/vllm/context_cache.py:120-139, called
 * at flashmap/vllm/model.py:874-893). The other arguments are fm_block_attn_paged's. */
int fm_block_attn_paged_runs(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *const *run_caches, const int32_t *run_first_slot,
    const int32_t *run_count, int32_t num_runs, int32_t heads_per_cache, int64_t num_blocks,
    int64_t stride_block, int64_t stride_head, int64_t stride_token, int64_t v_offset,
    int32_t page_size, const int32_t *block_table, int64_t block_table_stride,
    int64_t block_table_width, const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q,
    int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream);

/* a7: token-paged KV, SGLang's pool ((pool_size, kv_heads, head_dim) key and value
 * buffers): position p of sequence b is pool row page_table[b * page_table_stride + p]
 * (flashmap/sglang/model.py:127-151, 785-786, 861-864). Pool rows are clamped into
 * [0, pool_size). Replaces flashmap_sglang::paged_cross_attention
 * (flashmap/sglang/model.py:127-146, i.e. sgl_kernel flash_attn_with_kvcache with
 * page size 1, causal=False). */
int fm_block_attn_token_paged(
    const void *q, int64_t q_stride_batch, int64_t q_stride_token, int64_t q_stride_head,
    void *out, int64_t out_stride_batch, int64_t out_stride_token, int64_t out_stride_head,
    const int32_t *cu_seqlens_q, const void *key_buffer, const void *value_buffer,
    int64_t pool_size, int64_t k_stride_slot, int64_t k_stride_head, int64_t v_stride_slot,
    int64_t v_stride_head, const int32_t *page_table, int64_t page_table_stride,
    int64_t page_table_width, const int32_t *cache_seqlens, int32_t batch, int32_t max_seqlen_q,
    int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream);

/* FP8 (OCP e4m3) K/V: the same calls onto caches holding one byte per element (strides
 * in elements = bytes, multiples of 16), with FlashAttention's descale convention:
 * descales (3, batch, num_kv_heads) float32 at [kind * descale_stride_kind + b *
 * descale_stride_batch + h * descale_stride_head], kind 0 = query, 1 = key, 2 = value
 * (NULL: all 1). Scores are (q8 . k8) * q_descale * k_descale * softmax_scale, values
 * v8 * v_descale; P is rounded to bf16 before P.V, the output to bf16 once.
 * q_fp8 != 0: q holds e4m3 bytes (the caller quantized them; strides in bytes), no
 * prologue. q_fp8 == 0: q is bf16 (with the optional prologue) and the call quantizes
 * each (sequence, query head)'s rows with scale max(amax |q|, 1e-12) / 448, as
 * flashmap/sglang/model.py:167-169 does (the query part of descales is not read;
 * max_seqlen_q must be a multiple of 16). Workspace: fm_attn_workspace_bytes.
 * fm_block_attn_paged_fp8 replaces flashmap_vllm::paged_cross_attention with descales
 * (flashmap/vllm/model.py:93-134, 863-873); fm_block_attn_token_paged_fp8 replaces
 * flashmap_sglang::paged_cross_attention_fp8 (flashmap/sglang/model.py:154-181).
 */
int fm_block_attn_paged_fp8(
    const void *q, int32_t q_fp8, int64_t q_stride_batch, int64_t q_stride_token,
    int64_t q_stride_head, void *out, int64_t out_stride_batch, int64_t out_stride_token,
    int64_t out_stride_head, const int32_t *cu_seqlens_q, const void *kv_cache, int64_t num_blocks,
    int64_t stride_block, int64_t stride_head, int64_t stride_token, int64_t v_offset,
    int32_t page_size, const int32_t *block_table, int64_t block_table_stride,
    int64_t block_table_width, const int32_t *seqused_k, int32_t batch, int32_t max_seqlen_q,
    int32_t max_seqlen_k, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, const float *descales, int64_t descale_stride_kind,
    int64_t descale_stride_batch, int64_t descale_stride_head, const float *q_norm_weight,
    const float *rope_cos, const float *rope_sin, int64_t rope_row_stride,
    int64_t rope_pair_stride, int64_t rope_rows, const int64_t *q_positions, float eps,
    const int32_t *plan, void *workspace, size_t workspace_bytes, void *stream);
int fm_block_attn_token_paged_fp8(
    const void *q, int32_t q_fp8, int64_t q_stride_batch, int64_t q_stride_token,
    int64_t q_stride_head, void *out, int64_t out_stride_batch, int64_t out_stride_token,
    int64_t out_stride_head, const int32_t *cu_seqlens_q, const void *key_buffer,
    const void *value_buffer, int64_t pool_size, int64_t k_stride_slot, int64_t k_stride_head,
    int64_t v_stride_slot, int64_t v_stride_head, const int32_t *page_table,
    int64_t page_table_stride, int64_t page_table_width, const int32_t *cache_seqlens,
    int32_t batch, int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_q_heads,
    int32_t num_kv_heads, int32_t head_dim, float softmax_scale, const float *descales,
    int64_t descale_stride_kind, int64_t descale_stride_batch, int64_t descale_stride_head,
    const float *q_norm_weight, const float *rope_cos, const float *rope_sin,
    int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
    const int64_t *q_positions, float eps, const int32_t *plan, void *workspace,
    size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------------
 * Target verify attention: the step after the draft. Each request b has verify_len (L)
 * tokens -- the draft and its root, as a chain or a tree -- that attend to the
 * request's cached context and, among themselves, to what the mask allows. Replaces
 * SplitKVVerify (flashmap/sglang/verify_attention.py:251-474; its kernels :35-233,
 * installed as the target's verify_splitkv_fwd by flashmap/sglang/tree_worker.py:79-99),
 * taking sglang's extend_attention_fwd arguments as plain pointers:
 *   q, out: (batch * L, num_q_heads, head_dim), row of token b * L + t;
 *   k_ext, v_ext: the verify tokens' own keys/values (batch * L, num_kv_heads, head_dim);
 *   key_buffer, value_buffer: the pool (pool_size, num_kv_heads, head_dim);
 *   context of request b: pool rows kv_indices[kv_indptr[b] .. kv_indptr[b + 1]),
 *     kv_indices int32 or int64 (kv_index_bytes 4 / 8), kv_indptr int32 (batch + 1);
 *   mask_mode 0: causal among the verify tokens (token t sees tokens 0..t);
 *     1: sglang's custom mask, request b's rows at custom_mask[mask_indptr[b]], each
 *        context + L bytes of which the last L apply (the context is always visible);
 *     2: EAGLE's QLEN_ONLY layout, request b's L x L block at custom_mask[b * L * L];
 *     custom_mask bytes: nonzero = visible; mask_indptr int64 (batch + 1).
 * Context scores are scaled by sm_scale * k_scale and context values by v_scale; the
 * verify tokens' by sm_scale alone. A row that sees nothing gets zeros. Query heads
 * h * G .. h * G + G - 1 (G = num_q_heads / num_kv_heads) read KV head h.
 * max_context (> 0) bounds every request's context for grid planning; <= 0 uses
 * pool_size. Only sizes are read on the host. head_dim in {64, 128}, bf16.
 */
size_t fm_verify_workspace_bytes(int32_t batch, int32_t verify_len, int32_t num_q_heads,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t max_context,
                                 int64_t pool_size, int device);
int fm_verify_attention(
    const void *q, int64_t q_stride_token, int64_t q_stride_head, const void *k_ext,
    int64_t k_ext_stride_token, int64_t k_ext_stride_head, const void *v_ext,
    int64_t v_ext_stride_token, int64_t v_ext_stride_head, void *out, int64_t out_stride_token,
    int64_t out_stride_head, const void *key_buffer, const void *value_buffer, int64_t pool_size,
    int64_t k_stride_slot, int64_t k_stride_head, int64_t v_stride_slot, int64_t v_stride_head,
    const int32_t *kv_indptr, const void *kv_indices, int32_t kv_index_bytes,
    const uint8_t *custom_mask, const int64_t *mask_indptr, int32_t mask_mode, int32_t batch,
    int32_t verify_len, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float sm_scale, float k_scale, float v_scale, int32_t max_context, void *workspace,
    size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------------
 * a8  Block self-attention with fused q/k RMSNorm + RoPE: qkv (blocks, block_size,
 * 3, heads, head_dim) bf16 contiguous -> out (blocks, block_size, heads, head_dim)
 * bf16 contiguous (the same bytes as vLLM's (blocks * block_size, heads * head_dim)).
 * Rope row of slot token i (= block * block_size + t) is positions[i] or i.
 * block_size <= 16, head_dim in {64, 128}. Replaces flashmap_vllm::block_self_attention
 * (flashmap/vllm/kernels.py:194-232) and flashmap_sglang::block_self_attention
 * (flashmap/sglang/kernels.py:84-120).
 */
int fm_block_self_attention(const void *qkv, void *out, int64_t blocks, int32_t block_size,
                            int32_t heads, int32_t head_dim, const float *q_norm_weight,
                            const float *k_norm_weight, const float *rope_cos,
                            const float *rope_sin, int64_t rope_row_stride,
                            int64_t rope_pair_stride, int64_t rope_rows,
                            const int64_t *positions, float eps, float softmax_scale,
                            void *stream);

/* ---------------------------------------------------------------------------------
 * a4  Context KV writers (the K side of the QK-norm prologue). Every layer's keys are
 * k-normed (k_norm_weight row = layer, float32 (layers, head_dim)) and rotated at
 * their context position, then stored as bf16 together with the values.
 *
 * fm_write_context_kv: kv (tokens, layers, 2, heads, head_dim) bf16 contiguous into
 * vLLM-layout paged caches. Head h of layer l is global head gh = l * heads + h and
 * lives in cache gh / heads_per_cache (device array cache_ptrs[num_caches] of data
 * pointers) at cache head gh % heads_per_cache, token slot s = slots[t]:
 *   K = cache + (s / page_size) * stride_block + head * stride_head
 *       + (s % page_size) * stride_token,  V = K + v_offset.
 * slots[t] < 0 skips token t. Replaces write_context_kv
 * (flashmap/vllm/kernels.py:311-364) for bf16 caches.
 */
int fm_write_context_kv(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                        int32_t head_dim, const int64_t *positions, const int64_t *slots,
                        const float *k_norm_weight, const float *rope_cos, const float *rope_sin,
                        int64_t rope_row_stride, int64_t rope_pair_stride, int64_t rope_rows,
                        const int64_t *cache_ptrs, int32_t num_caches, int32_t heads_per_cache,
                        int64_t stride_block, int64_t stride_head, int64_t stride_token,
                        int64_t v_offset, int32_t page_size, float eps, void *stream);

/* fm_write_context_kv_pool: kv (tokens, layers * 2 * heads * head_dim) bf16
 * contiguous (per layer: keys of all heads, then values) into SGLang-layout pools.
 * meta (layers, 4) int64 device array: key buffer pointer, value buffer pointer, key
 * row stride, value row stride (elements); head h of a row at h * head_dim.
 * locs[t] < 0 skips token t; with commit_lens non-NULL, token t is skipped when
 * t % locs_row_width >= commit_lens[t / locs_row_width] (uncommitted verify columns).
 * Replaces sglang's fused_kv_norm_rope_write as the plugin calls it
 * (flashmap/sglang/model.py:746-766, is_neox_style=False) for bf16 pools, with the
 * reference rounding (scale rounded to bf16 before the multiply).
 */
int fm_write_context_kv_pool(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                             int32_t head_dim, const int64_t *meta, const float *k_norm_weight,
                             const float *rope_cos, const float *rope_sin,
                             int64_t rope_row_stride, int64_t rope_pair_stride,
                             int64_t rope_rows, const int64_t *positions, const int64_t *locs,
                             const int32_t *commit_lens, int64_t locs_row_width, float eps,
                             void *stream);

/* FP8 (OCP e4m3, one byte per element) versions of the two writers. Keys are k-normed
 * and rotated as above but kept in fp32 through the rotation; keys and values are then
 * divided by the cache's scale, rounded to nearest even and saturated to +-448.
 * fm_write_context_kv_fp8: scales (layers, 2) float32 device array of per-layer (key,
 * value) scales; strides in elements (= bytes). Replaces write_context_kv for fp8 caches
 * (flashmap/vllm/kernels.py:292-299, 311-364).
 * fm_write_context_kv_pool_fp8: one (k_scale, v_scale) pair, and the pool writer's norm
 * rounding bf16(x * r * w) (r = 1 / sqrt(mean(x^2) + eps)); meta strides in elements.
 * Replaces kv_norm_rope_write_fp8 (flashmap/sglang/kernels.py:283-357).
 */
int fm_write_context_kv_fp8(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                            int32_t head_dim, const int64_t *positions, const int64_t *slots,
                            const float *k_norm_weight, const float *rope_cos,
                            const float *rope_sin, int64_t rope_row_stride,
                            int64_t rope_pair_stride, int64_t rope_rows,
                            const int64_t *cache_ptrs, int32_t num_caches,
                            int32_t heads_per_cache, int64_t stride_block, int64_t stride_head,
                            int64_t stride_token, int64_t v_offset, int32_t page_size,
                            const float *scales, float eps, void *stream);
int fm_write_context_kv_pool_fp8(const void *kv, int64_t tokens, int32_t layers, int32_t heads,
                                 int32_t head_dim, const int64_t *meta,
                                 const float *k_norm_weight, const float *rope_cos,
                                 const float *rope_sin, int64_t rope_row_stride,
                                 int64_t rope_pair_stride, int64_t rope_rows,
                                 const int64_t *positions, const int64_t *locs,
                                 const int32_t *commit_lens, int64_t locs_row_width,
                                 float k_scale, float v_scale, float eps, void *stream);

/* ---------------------------------------------------------------------------------
 * f3: the draft step's token selection and noise. Logits are (rows, vocab) with
 * row_stride elements between rows, dtype 0 bf16, 1 fp16, 2 fp32; out is int64 (rows,).
 * The selection calls use a caller workspace of fm_select_workspace_bytes(rows, vocab)
 * bytes. The random stream is Triton's tl.rand / tl.randn (Philox-4x32-10 keyed by the
 * seed's words, counter (offset, 0, 0, 0)) word for word.
 */
size_t fm_select_workspace_bytes(int64_t rows, int64_t vocab);
/* split_argmax (flashmap/vllm/fold.py:117-128, called at flashmap/vllm/speculator.py:218):
 * per row the index of the largest logit, the first among equals (a NaN counts as the
 * largest). */
int fm_argmax_rows(const void *logits, int32_t dtype, int64_t rows, int64_t vocab,
                   int64_t row_stride, int64_t *out, void *workspace, size_t workspace_bytes,
                   void *stream);
/* sample_rows (flashmap/sglang/kernels.py:195-247, called at flashmap/sglang/sampler.py:169):
 * per row the argmax of its logits where greedy[row] != 0, else of
 * logit / temperatures[row] - log(-log(u)), u = tl.rand(*seed, row * vocab + col) with
 * int32 offsets (Gumbel-max); the first index among equals. seed: a device int64. */
int fm_sample_rows(const void *logits, int32_t dtype, int64_t rows, int64_t vocab,
                   int64_t row_stride, const float *temperatures, const uint8_t *greedy,
                   const int64_t *seed, int64_t *out, void *workspace, size_t workspace_bytes,
                   void *stream);
/* seeded_normal (flashmap/vllm/kernels.py:367-410, called at flashmap/vllm/model.py:965):
 * out[i, j] = scale * tl.randn(key_i, j), key_i = seeds[rows[i]] * 1000003 + positions[i]
 * (int64, wrapping; seed 0 where rows[i] < 0). rows / positions are int64 where their
 * flag is nonzero, else int32; rows[i] must index seeds. */
int fm_seeded_normal(const int64_t *seeds, const void *rows, int32_t rows_int64,
                     const void *positions, int32_t positions_int64, int64_t num_rows,
                     int64_t n_cols, float scale, float *out, int64_t out_row_stride,
                     void *stream);

/* ---------------------------------------------------------------------------------
 * f3: the DiT's residual stream between sublayers. Replaces the eager ops of
 * FlashMapAdaLayerNorm.forward and the gated residuals of FlashMapLayer.forward
 * (flashmap/modeling_flashmap.py:114-117, 185-192) and of the vLLM draft step's _dit
 * (flashmap/vllm/model.py:829-903):
 *   x' = x + gate * y                          (when y is non-NULL; else x' = x)
 *   h  = LN(x') * (1 + scale) + shift          (when scale is non-NULL)
 * with every op rounded to bf16 as torch's eager bf16 ops round; LN has no affine
 * weights (biased variance, eps inside the rsqrt). x, y, x_out, h_out: (rows, dim) bf16
 * with row strides (elements, multiples of 8); x_stride 0 reads one (dim,) row for every
 * row; scale, shift: (dim,) bf16 shared by all rows; gate: (dim,) bf16 shared by all
 * rows, or with gate_per_row nonzero one bf16 value per row (rows,); x_out may alias x
 * (not a shared x row). dim a multiple of 8, at most 8192.
 */
int fm_adaln_residual(const void *x, int64_t x_stride, const void *y, int64_t y_stride,
                      const void *gate, int32_t gate_per_row, const void *scale, const void *shift,
                      void *x_out, int64_t x_out_stride, void *h_out, int64_t h_out_stride,
                      int64_t rows, int32_t dim, float eps, void *stream);

/* The row pass of the one-jump draft's folded noise read-out (flashmap/vllm/model.py:
 * 915-925 with the folds of flashmap/vllm/fold.py:45-75): for z (rows, hidden) fp32 with a
 * row stride, scale[r] = bf16(gain * rsqrt(sum_i z[r,i]^2 eigvals[i] + eps)) (bf16, rows)
 * and z_bf16 = z rounded to bf16 (the folded GEMM's operand). The read-out is then
 * noise = z_bf16 @ M^T and hidden = first_hidden + scale * noise (fm_adaln_residual with
 * a shared x row and a per-row gate). hidden a multiple of 4, at most 16384.
 */
int fm_noise_rows(const float *z, int64_t rows, int32_t hidden, int64_t z_stride,
                  const float *eigvals, float eps, float gain, void *z_bf16,
                  int64_t z_bf16_stride, void *scale, void *stream);

/* The several-jump draft's state over the vocabulary (flashmap/vllm/model.py:944-956,
 * `_embed_state`): for state (rows, vocab) fp32 with a row stride and posterior nonzero,
 * out rows r < rows get bf16(softmax(evidence * state[r])) and rows rows + r get
 * bf16(state[r]) -- the operand of the one GEMM through the state vocabulary's embedding
 * (torch.cat([posterior, state]).to(bf16)); out is (2 rows, vocab) bf16 with a row
 * stride. With posterior zero (a jump starting at time 0, whose posterior is uniform),
 * out is (rows, vocab): the state rows only. Strides multiples of 4; state 16-byte
 * aligned, out 8-byte aligned.
 */
int fm_state_embed_rows(const float *state, int64_t rows, int64_t vocab, int64_t state_stride,
                        float evidence, int32_t posterior, void *out, int64_t out_stride, void *stream);

/* The state update between two jumps (flashmap/vllm/model.py:1031-1036): with logits
 * (rows, vocab) bf16 (the jump head's output) and the jump's times start <= end, start < 1:
 * state = ((1 - end) * state + (end - start) * softmax(logits)) / (1 - start) in place,
 * in float32 with torch's rounding points (the scalars rounded from double to float).
 * Strides multiples of 4; state 16-byte aligned, logits 8-byte aligned.
 */
int fm_state_update(float *state, int64_t rows, int64_t vocab, int64_t state_stride, const void *logits,
                    int64_t logits_stride, double start, double end, void *stream);

/* ---------------------------------------------------------------------------------
 * Measurement hook. No reference counterpart: it lets a benchmark time the main
 * split-KV attention kernel alone with HIP events on the stream it runs on, without
 * changing the work any call does. While enabled, every attention call records an
 * event pair around its main kernel; fm_profile_read synchronizes those events and
 * returns the summed milliseconds and the number of launches, then clears them.
 */
int fm_profile_enable(int enable);
/* Measurement hook, no reference counterpart: one wavefront on `stream` spins for
 * spin_ticks (at most 2^24) ticks of the shader-clock counter and stores, at out[0] and
 * out[1] (device, 16-byte aligned), the shader-clock ticks and the 100 MHz real-time ticks
 * that passed: their ratio is the shader clock (SCLK) at that point of the stream. Used
 * to follow the clock under sustained load. */
int fm_clock_probe(uint64_t *out, uint64_t spin_ticks, void *stream);
int fm_profile_read(double *total_ms, int64_t *launches);
/* Tuning hook, no reference counterpart: the attention calls read their FLASHMAP_*
 * overrides (split-KV workgroups and minimum tiles, the small-call kernel's tiles per
 * share, the query pass, the share cost, the combine's batch) from the environment once,
 * at the first call; this re-reads them (for tests and sweeps that change them within a
 * process). Not to be called while another thread launches attention calls. */
int fm_tuning_reload(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASHMAP_AMD_H */
