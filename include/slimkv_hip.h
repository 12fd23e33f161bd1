/*
 * slimkv_hip.h -- C ABI of the MI355X (gfx950) compressed-cache attention library.
 *
 * Every entry point enqueues work on the caller's HIP stream (passed as `void*`,
 * a hipStream_t), allocates nothing, never synchronises the host, and returns 0 on
 * success or a negative error code; `slimkv_last_error()` then holds a message
 * for the calling thread.  Tensors are device pointers.  bf16 data is passed as
 * its 16-bit pattern.  Strides are in elements, the last dimension of every
 * tensor is contiguous, and bf16 rows must start on 16-byte boundaries
 * (strides and widths are multiples of 8 elements).  Workspaces are owned by the
 * caller and sized by the matching `*_workspace` query; they need no clearing.
 */
#ifndef SLIMKV_HIP_H
#define SLIMKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SLIMKV_OK 0
#define SLIMKV_EINVAL (-1)   /* invalid shape, stride or argument */
#define SLIMKV_EUNSUP (-2)   /* supported by the reference, not by this build */
#define SLIMKV_EWORKSPACE (-3) /* workspace too small */
#define SLIMKV_EHIP (-4)     /* HIP runtime error */

/* Block tables follow torch's indexing rules, like the reference's page I/O
 * (slimkv/vllm_plugin/paged_cache.py:60-67, :111-127): an entry in
 * [-num_pages, 0) counts from the end of the pool; a row whose table column
 * lies past the table or whose entry lies outside [-num_pages, num_pages) is an
 * index error (the reference raises IndexError).  Kernels reading such a row
 * use no data from it, kernels writing it write nothing, and when the
 * argument struct's `status` (device int32, optional) is set they store
 * SLIMKV_STATUS_BAD_PAGE there with an ordinary store; nothing clears it. */
#define SLIMKV_STATUS_BAD_PAGE 1
/* slimkv_decode_qkv: the cache slot lies outside [0, capacity); no cache row
 * is written (the reference's index_copy_ raises IndexError).
 * slimkv_paged_step_rows: a request's raw set does not fit the dense rows. */
#define SLIMKV_STATUS_BAD_SLOT 2

/* Message describing the last failure on the calling thread ("" if none). */
const char* slimkv_last_error(void);

/* ABI version of this header (bumped on any struct change). */
int slimkv_abi_version(void);

/* Stages of a decode call, for the *_stages entry points (bit mask).  A
 * decode runs three kernels that hand over through the caller's workspace:
 *   SLIMKV_STAGE_PROLOGUE  query RoPE (and, for the latent decode, the query
 *                          absorption into U_K and the K-bias LSE shift);
 *   SLIMKV_STAGE_ATTEND    the split-K attention: per-split partials;
 *   SLIMKV_STAGE_COMBINE   the LSE merge of the partials, the V lift, out/lse.
 * A *_stages call runs the selected stages in that order.  Calls with the
 * same arguments and workspace that together run every stage once, in order,
 * write exactly what one full call writes.  No counterpart in the reference,
 * whose decode runs as one sequence of launches (slimkv/llama3/fa2_decode.py:
 * 143-164); callers use it to place the stages themselves, e.g. to time the
 * attention kernel of many layers back to back. */
#define SLIMKV_STAGE_PROLOGUE 1
#define SLIMKV_STAGE_ATTEND 2
#define SLIMKV_STAGE_COMBINE 4
#define SLIMKV_STAGE_ALL 7

/* ------------------------------------------------------------------------
 * Split-K decode attention with GQA, bottom-right causality and LSE.
 *
 * Replaces the native forward of the reference decode extension,
 *   slimkv_fa2_decode_320.forward(q, k, v, softmax_scale, causal, num_splits,
 *                                 pack_q, cache_seqlens)
 *   (kernels/fa2_decode/binding.cpp:35-121, exported at :123-130), and the
 *   flash_attn call inside flash_forward (slimkv/llama3/fa2_decode.py:15-38).
 * Semantics follow the reference eager attention
 *   (slimkv/llama3/latent_decode.py:16-41): query head j uses KV head
 *   j / (heads / kv_heads); with `causal` query i sees keys
 *   [0, keys_b - queries + i]; a row that sees no key gets output 0 and
 *   LSE -inf.  K and V widths may differ; no padding is needed.
 * q   [B, Lq, Hq, Wk]  k [B, N, Hk, Wk]  v [B, N, Hk, Wv]  (BSHD, bf16)
 * out [B, Lq, Hq, Wv]  bf16;  lse [B, Hq, Lq] fp32 contiguous (may be NULL)
 * seqlens: optional device int32 [B] key counts (each <= keys).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_attention_args {
    const void* q;  int64_t q_sb, q_sl, q_sh;
    const void* k;  int64_t k_sb, k_sn, k_sh;
    const void* v;  int64_t v_sb, v_sn, v_sh;
    void* out;      int64_t o_sb, o_sl, o_sh;
    float* lse;
    const int32_t* seqlens;
    int64_t batch, queries, heads, kv_heads, keys, width_k, width_v;
    double scale;
    int32_t causal;
    int32_t splits; /* 0 = automatic */
} slimkv_attention_args;

size_t slimkv_attention_workspace(const slimkv_attention_args* a);
int slimkv_attention_forward(const slimkv_attention_args* a, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused reconstruction-free latent beacon decode for one attention layer.
 *
 * Replaces the attention core of slimkv.llama3.fa2_decode.decode
 *   (slimkv/llama3/fa2_decode.py:143-164): query RoPE (optional, bf16-exact as
 *   decode_kernels.py:44-51), raw branch over RoPE'd full-dim K/V
 *   (:146-148), query absorption into U_K (project_query :41-46), latent branch
 *   over un-RoPE'd beacon latents (:152-154), V lift through U_V
 *   (project_value :49-54), bias folding (:157-163) and the LSE merge
 *   (merge_attention :57-66) -- all under one online softmax.
 * q       [B, Lq, Hq, D] bf16; rotated in-kernel at q_positions [B, Lq] when
 *         `cos`/`sin` ([rope_rows, D] fp32) are given, else already rotated.
 *         With cos/sin but no q_positions, the tables are the rows already
 *         taken at the query positions: row b * Lq + l (rope_rows >= B * Lq),
 *         as a model's rotary embedding returns them once per decode step.
 * raw_k/v [B, Nr, Hkv, D] bf16, K already rotated (sinks, tail, current token).
 * lat_k   [B, Nl, Rk] bf16 and lat_v [B, Nl, Rv] bf16: global latent rows.
 * up_k    [Hkv*D, Rk], up_v [Hkv*D, Rv]: nn.Linear weights of the beacon
 *         up-projections, optional biases [Hkv*D].
 * block_diagonal = 1 asserts that every off-diagonal (D x Rk/Hkv) block of
 *         up_k and (D x Rv/Hkv) block of up_v is zero (per-KV-head bases); the
 *         latent branch then reads only each head's own latent slice.
 * lat_causal: bottom-right causal latent branch (the beacon-insertion step).
 * out [B, Lq, Hq, D] bf16; lse [B, Hq, Lq] fp32 (may be NULL).
 * up_k_t  optional [Hkv, Rk/Hkv, D] per-head transposed K bases made by
 *         slimkv_prepare_latent_bases; with block_diagonal the query
 *         absorption then runs on MFMA in one wavefront per (b, KV head).
 * lat_k2 / lat_v2 optional second latent segment: rows [lat_split, lat_keys)
 *         of every sequence lie there (row i at index i - lat_split, strides
 *         lk2_sb/lk2_sn, lv2_sb/lv2_sn) and rows [0, lat_split) at lat_k /
 *         lat_v, so a growing history and the current window are read where
 *         they lie instead of being joined each step (fa2_decode.py:133-135
 *         concatenates them); 0 < lat_split < lat_keys; dense rows only.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_latent_decode_args {
    const void* q;  int64_t q_sb, q_sl, q_sh;
    const int64_t* q_positions; int64_t pos_sb;
    const float* cos; const float* sin; int64_t rope_rows;
    const void* raw_k; int64_t rk_sb, rk_sn, rk_sh;
    const void* raw_v; int64_t rv_sb, rv_sn, rv_sh;
    const int32_t* raw_lengths;
    int64_t raw_keys;
    const void* lat_k; int64_t lk_sb, lk_sn;
    const void* lat_v; int64_t lv_sb, lv_sn;
    const int32_t* lat_lengths;
    int64_t lat_keys;
    int32_t lat_causal;
    int32_t block_diagonal;
    const void* up_k; const void* up_k_bias;
    const void* up_v; const void* up_v_bias;
    int64_t batch, queries, heads, kv_heads, head_dim, rank_k, rank_v;
    double scale;
    void* out; int64_t o_sb, o_sl, o_sh;
    float* lse;
    int32_t raw_splits, lat_splits; /* 0 = automatic */
    const void* up_k_t;
    const void* lat_k2; int64_t lk2_sb, lk2_sn;
    const void* lat_v2; int64_t lv2_sb, lv2_sn;
    int64_t lat_split;
} slimkv_latent_decode_args;

size_t slimkv_latent_decode_workspace(const slimkv_latent_decode_args* a);
int slimkv_latent_decode(const slimkv_latent_decode_args* a, void* workspace,
                         size_t workspace_bytes, void* stream);
/* slimkv_latent_decode restricted to `stages` (SLIMKV_STAGE_*). */
int slimkv_latent_decode_stages(const slimkv_latent_decode_args* a, int stages, void* workspace,
                                size_t workspace_bytes, void* stream);

/* Allocation-free slimkv_latent_decode (no counterpart in the reference): for
 * callers that cannot allocate -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The workspace is a device array of
 * SLIMKV_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held until the
 * process ends), so the call allocates nothing; a call whose workspace
 * (slimkv_latent_decode_workspace) would exceed it fails with
 * SLIMKV_EWORKSPACE before launching anything.  The stream must belong to the
 * current device.  Every call on one GPU uses that GPU's one array: calls that
 * overlap on a GPU (other streams, other threads) race and must be ordered by
 * the caller.  The array needs no clearing between calls.  Results equal
 * slimkv_latent_decode's. */
#define SLIMKV_NOALLOC_SCRATCH_BYTES (32u << 20)
int slimkv_latent_decode_noalloc(const slimkv_latent_decode_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Paged latent decode: slimkv_latent_decode with the beacon rows read straight
 * out of beacon pages, no restore/gather step.  Replaces the page gather of
 *   restore_memory (slimkv/vllm_plugin/paged_model.py:36-52, through
 *   BeaconPages.read, slimkv/vllm_plugin/paged_cache.py:60-87) followed by the
 *   latent decode of the gathered rows (slimkv/llama3/fa2_decode.py:77-166).
 * Page format (BeaconPageLayout, paged_cache.py:27-44): page = [sink_elements
 * | slots x (rank_k + rank_v)] bf16; beacon i of sequence b sits in page
 * table[b * t_sb + i / slots] (t_cols entries per row, at least
 * ceil(lat_keys / slots), like the reference's IndexError) at column sink_elements + (i % slots) *
 * (rank_k + rank_v), K first, then V.  Page ids follow the block-table rules
 * above (an out-of-pool id is reported through `status`; the row then reads
 * page 0 so every access stays inside the pool, and the output is not
 * meaningful).  base.lat_k / lat_v and their strides are ignored;
 * base.lat_lengths (beacons per sequence) is required and base.lat_keys is
 * the largest count.  rows_total: the sum of lat_lengths when the host knows
 * it (sizes the key splits; 0 = unknown), never needed for correctness.
 * With the same base.lat_splits the result is bit-identical to gathering the
 * rows and calling slimkv_latent_decode.
 * raw_pages (optional): the raw rows (sinks, tail, current token) read through
 * raw pages as well, replacing RawPages.read (paged_cache.py:111-127) into
 * base.raw_k / raw_v (then ignored, NULL allowed): row r of sequence b is
 * token r % raw_block_size (a power of two, at least 16) of block
 * raw_table[b * raw_t_sb + r / raw_block_size] (raw_t_cols entries per row,
 * at least ceil(base.raw_keys / raw_block_size)); K at raw_pages +
 * block * raw_block_stride + token * raw_token_stride + head *
 * raw_head_stride, V raw_kind_stride further (RawPages' [blocks, block, 2,
 * Hkv, D] pages).  Block ids follow the same rules; base.raw_lengths holds
 * the raw rows per sequence.  With the same split counts the result is
 * bit-identical to reading the raw rows into dense tensors first.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_paged_latent_decode_args {
    slimkv_latent_decode_args base;
    const void* pages; int64_t num_pages, page_stride;
    const int64_t* table; int64_t t_sb, t_cols;
    int64_t slots, sink_elements;
    int64_t rows_total;
    int32_t* status;   /* optional: SLIMKV_STATUS_BAD_PAGE on an index error */
    const void* raw_pages; int64_t raw_num_blocks, raw_block_size;
    int64_t raw_block_stride, raw_token_stride, raw_kind_stride, raw_head_stride;
    const int64_t* raw_table; int64_t raw_t_sb, raw_t_cols;
} slimkv_paged_latent_decode_args;

size_t slimkv_paged_latent_decode_workspace(const slimkv_paged_latent_decode_args* a);
int slimkv_paged_latent_decode(const slimkv_paged_latent_decode_args* a, void* workspace,
                               size_t workspace_bytes, void* stream);
/* slimkv_paged_latent_decode restricted to `stages` (SLIMKV_STAGE_*). */
int slimkv_paged_latent_decode_stages(const slimkv_paged_latent_decode_args* a, int stages, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* One-time re-layout of block-diagonal K bases for slimkv_latent_decode (no
 * counterpart in the reference, whose project_query reads U_K as stored,
 * slimkv/llama3/fa2_decode.py:41-46): out[h, c, d] = up_k[h*D + d, h*r + c]
 * with r = rank/kv_heads.  up_k [kv_heads*D, rank] bf16 row-major; out
 * [kv_heads, r, D] bf16. */
int slimkv_prepare_latent_bases(const void* up_k, int64_t kv_heads, int64_t head_dim, int64_t rank, void* out,
                                void* stream);

/* ------------------------------------------------------------------------
 * Beacon reconstruction: the up-projection of latent rows to full-dim K or V.
 * Replaces the up-projection inside ReconstructionCache.materialize
 *   (slimkv/llama3/memory.py:29-36) and the per-step history rebuild of the
 *   reconstruction route (tools/benchmark/context_decode_runtime.py:318-332).
 * out[b, dst(n), h, :] = rope?(bf16(latent[b, n, :] @ W[h*D:(h+1)*D, :]^T + bias[h*D:...]))
 * latent [B, n, R]; weight [Hkv*D, R] (nn.Linear); bias [Hkv*D] or NULL;
 * out: 4-D with strides (batch, row, head), last dim contiguous.
 * dst_rows [n] int64 scatters rows (the window/raw interleave of materialize),
 * NULL = identity.  positions [B, n] int64 applies bf16-exact RoPE (beacon K
 * with RoPE, modeling_llama.py:1144-1145), NULL = none.  block_diagonal = 1
 * contracts each head with its own R/Hkv latent slice only.  head_dim 128.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_reconstruct_args {
    const void* latent; int64_t l_sb, l_sn;
    const void* weight; const void* bias;
    void* out; int64_t o_sb, o_sn, o_sh;
    const int64_t* dst_rows;
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* positions; int64_t pos_sb;
    int64_t batch, rows, rank, kv_heads, head_dim;
    int32_t block_diagonal;
} slimkv_reconstruct_args;

int slimkv_reconstruct(const slimkv_reconstruct_args* a, void* stream);

/* Two reconstructions in one launch where both take the streaming kernel (a
 * contracted latent width up to 64) at the same width -- the K and the V
 * rebuild of one set of beacon rows -- else in two launches; the results are
 * those of two slimkv_reconstruct calls, bit for bit.  The reference runs the
 * K and V up-projections of ReconstructionCache.materialize as two nn.Linear
 * calls (slimkv/llama3/memory.py:29-36); this saves a launch where both are
 * rebuilt together (a prefill window's beacon rows, modeling_llama.py:1347-1367). */
int slimkv_reconstruct_pair(const slimkv_reconstruct_args* a, const slimkv_reconstruct_args* b, void* stream);

/* ------------------------------------------------------------------------
 * Reconstruction decode for one attention layer: rebuild every beacon's K
 * (RoPE'd at `beacon_positions` when given) and V from the latents, then one
 * split-K online softmax over [reconstructed beacons ; raw rows].
 * Replaces the reconstruction route of LlamaAttention.forward
 *   (slimkv/llama3/modeling_llama.py:1405-1483) and
 *   OptimizedDecodeRuntime.reconstruction_attention
 *   (tools/benchmark/context_decode_runtime.py:298-344).
 * Argument meaning as slimkv_latent_decode; lat_causal makes the beacon
 * segment bottom-right causal (the raw query of an insertion step does not
 * see the new beacon).  With block-diagonal bases (per-head K rank 16, 32 or
 * 48, V rank 32 or 64; lat_k and up_k 16-byte aligned with row strides a
 * multiple of 8 elements at K ranks 32 and 48, 8-byte and 4 at rank 16) each
 * K tile is rebuilt and rotated inside the attention kernel and V is lifted
 * after the weighted sum; rotated beacon keys then
 * need rope_pairs (slimkv_prepare_rope_pairs of the same cos/sin tables) and
 * rope_repeats = 1 (rotate-half tables, cos/sin = cat(f, f): the reference's
 * RotaryEmbedding, modeling_utils.py:369-376).  Otherwise the workspace holds
 * the rebuilt K (and V).
 * ---------------------------------------------------------------------- */
/* rope_fp32 (fused route with rotated beacon keys): 0 rebuilds and rotates
 * each key with the reference's bf16 steps (bf16(acc + bias), then
 * bf16(bf16(x c) + bf16(rotate_half(x) s)): the bits ReconstructionCache
 * .materialize writes); 1 adds the bias and rotates in fp32 and rounds once
 * (about a third of the per-key arithmetic; keys within one bf16 rounding of
 * the exact rotation). */
typedef struct slimkv_recon_decode_args {
    slimkv_latent_decode_args base;
    const int64_t* beacon_positions; int64_t bpos_sb;   /* [B, Nl] or NULL */
    const uint32_t* rope_pairs;                          /* [rope_rows, 128] or NULL */
    int32_t rope_repeats;                                /* 1: every cos/sin row is its first half twice */
    int32_t rope_fp32;                                   /* 1: fp32 rotation, one rounding */
} slimkv_recon_decode_args;

/* One-time packing of RoPE tables for the fused reconstruction decode (no
 * counterpart in the reference, whose RoPE reads cos/sin and rounds them to
 * bf16 at every use, slimkv/llama3/decode_kernels.py:7-51):
 * out[r, d] = bf16(cos[r, d]) | bf16(sin[r, d]) << 16.  cos, sin [rows, dim]
 * fp32 contiguous; out [rows, dim] uint32. */
int slimkv_prepare_rope_pairs(const float* cos, const float* sin, int64_t rows, int64_t dim, uint32_t* out,
                              void* stream);

size_t slimkv_recon_decode_workspace(const slimkv_recon_decode_args* a);
int slimkv_recon_decode(const slimkv_recon_decode_args* a, void* workspace, size_t workspace_bytes, void* stream);
/* slimkv_recon_decode restricted to `stages` (SLIMKV_STAGE_*): the prologue
 * rotates the query, except on the fused route (K rebuilt per tile inside the
 * split kernel), whose split kernel rotates its query rows itself and whose
 * prologue stage does nothing; the attend stage rebuilds what the route
 * rebuilds and runs the split kernel. */
int slimkv_recon_decode_stages(const slimkv_recon_decode_args* a, int stages, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Decode RoPE of the query and the raw K cache, bf16-exact.
 * Replaces decode_ops.fused_rope (slimkv/llama3/decode_ops.py:14-31) and its
 * kernel (slimkv/llama3/decode_kernels.py:7-51).
 * q [B, Hq, Lq, D], k [B, Hk, Nk, D] (BHSD, strided); outputs contiguous.
 * Query position: q_positions[b*pos_sb + s].  Key position of slot s:
 * s < sink -> s; s == Nk-1 -> q_positions[b*pos_sb]; else
 * raw_indices[s - sink] + sink + history.
 * out = bf16(bf16(x*bf16(cos)) + bf16(rotate_half(x)*bf16(sin))).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_rope_decode_args {
    const void* q; int64_t q_sb, q_sh, q_ss;
    const void* k; int64_t k_sb, k_sh, k_ss;
    void* out_q; void* out_k;
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* q_positions; int64_t pos_sb;
    const int64_t* raw_indices; /* may be NULL when no slot needs it */
    int64_t raw_index_count;
    int64_t batch, heads, kv_heads, queries, keys, dim, sink, history;
} slimkv_rope_decode_args;

int slimkv_rope_decode(const slimkv_rope_decode_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Prefill RoPE that leaves beacon K unrotated.
 * Replaces prefill_ops.fused_prefill_rope (slimkv/llama3/prefill_ops.py:48-73)
 * and prefill_rope_kernel (slimkv/llama3/prefill_kernels.py:7-53).
 * Query slot s uses positions[b*pos_sb + Nk - Lq + s]; key slot s uses
 * positions[b*pos_sb + s] unless it is a beacon: s in [sink, Nk-role_len) or
 * roles[s - (Nk-role_len)] in {1, 2}, which is copied unchanged.  queries = 0
 * (q and out_q may then be NULL) rotates the keys alone, for callers whose
 * attention rotates its queries itself (slimkv_prefill_attention).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_prefill_rope_args {
    const void* q; int64_t q_sb, q_sh, q_ss;
    const void* k; int64_t k_sb, k_sh, k_ss;
    void* out_q; int64_t oq_sb, oq_sh, oq_ss;
    void* out_k; int64_t ok_sb, ok_sh, ok_ss;
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* positions; int64_t pos_sb;
    const int64_t* roles; int64_t role_len;
    int64_t batch, heads, kv_heads, queries, keys, dim, sink;
    /* optional (v NULL: none): value rows [B, Hk, Nk, D] copied unchanged
     * into out_v in the same launch, row for row with the keys -- the window's
     * V written into the attention's value set beside its rotated keys */
    const void* v; int64_t v_sb, v_sh, v_ss;
    void* out_v; int64_t ov_sb, ov_sh, ov_ss;
} slimkv_prefill_rope_args;

int slimkv_prefill_rope(const slimkv_prefill_rope_args* a, void* stream);

/* ------------------------------------------------------------------------
 * LSE merge of two attention branches.
 * Replaces decode_ops.fused_merge (slimkv/llama3/decode_ops.py:34-48) and
 * merge_kernel (slimkv/llama3/decode_kernels.py:53-75):
 * t = max(r,l) + log1p(exp(-|r-l|)); out = exp(r-t)*raw + exp(l-t)*latent.
 * raw/latent [B, H, L, D] bf16 (strided), lse [B, H, L] fp32 (strided);
 * out contiguous [B, H, L, D] bf16.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_merge_args {
    const void* raw; int64_t r_sb, r_sh, r_sl;
    const void* latent; int64_t l_sb, l_sh, l_sl;
    const float* raw_lse; int64_t rl_sb, rl_sh, rl_sl;
    const float* latent_lse; int64_t ll_sb, ll_sh, ll_sl;
    void* out;
    int64_t batch, heads, length, dim;
} slimkv_merge_args;

int slimkv_merge(const slimkv_merge_args* a, void* stream);

/* Element types of the dtype-generic entry points below. */
#define SLIMKV_DTYPE_BF16 0
#define SLIMKV_DTYPE_F16 1
#define SLIMKV_DTYPE_F32 2

/* slimkv_merge for bf16, fp16 or fp32 branch outputs of type `dtype`, out in
 * the same type (contiguous [B, H, L, D]; any width, element strides).
 * Replaces merge_attention's torch arithmetic (slimkv/llama3/fa2_decode.py:
 * 57-66), which the reference runs wherever its fused merge does not apply. */
int slimkv_merge_typed(const slimkv_merge_args* a, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * fp32 eager attention.
 * Replaces latent_decode.eager_forward (slimkv/llama3/latent_decode.py:16-41),
 * the reference's fp32 attention: q [B, Lq, Hq, R], k [B, N, Hk, R],
 * v [B, N, Hk, Rv] of one dtype (element strides, last dim contiguous) meet in
 * fp32; bottom-right causal mask when `causal`; rows that see no key give LSE
 * -inf and a zero output.  out [B, Lq, Hq, Rv] in the inputs' dtype (element
 * strides), lse [B, Hq, Lq] fp32 contiguous; `scores` is a workspace of
 * B * Hq * Lq * N floats.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_eager_attention_args {
    const void* q; int64_t q_sb, q_sl, q_sh;
    const void* k; int64_t k_sb, k_sn, k_sh;
    const void* v; int64_t v_sb, v_sn, v_sh;
    void* out; int64_t o_sb, o_sl, o_sh;
    float* lse;
    float* scores;
    int64_t batch, queries, heads, kv_heads, keys, rank, rank_v;
    double scale;
    int32_t dtype, causal;
} slimkv_eager_attention_args;

int slimkv_eager_attention(const slimkv_eager_attention_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Projections of a decode step's rows (one token per sequence of a lockstep
 * batch, m <= 4): out[m, n] = x[m, :] . W[n, :] (+ bias[n]), W the
 * nn.Linear weight [N, K] bf16 row-major, fp32 accumulation, one bf16
 * rounding.  N a multiple of 128, K a multiple of 8; x rows and W 16-byte
 * aligned.  Replaces the nn.Linear calls on the step's rows, such as o_proj
 * in StaticDecode.forward (slimkv/llama3/static_decode.py:193-198).
 * x [m, K] (row stride x_sm), out [m, N] (row stride o_sm).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_linear_rows_args {
    const void* x; int64_t x_sm;
    const void* weight; const void* bias;   /* [N, K]; bias [N] or NULL */
    void* out; int64_t o_sm;
    int64_t m, n, k;
} slimkv_linear_rows_args;

int slimkv_linear_rows(const slimkv_linear_rows_args* a, void* stream);

/* ------------------------------------------------------------------------
 * The new token's query/key/value projection with its key RoPE and raw-cache
 * appends, one launch.  Over W = [W_q; W_k; W_v] ([(Hq + 2 Hkv) * 128, K],
 * bias likewise or NULL) it writes q = x W_q^T (+ b_q) to `q` (unrotated:
 * the decode rotates it), the key k = bf16(x W_k^T (+ b_k)) rotated at
 * positions[m] with the reference's bf16 steps (the bits of
 * slimkv_rope_decode) to raw_k[m, slot], the unrotated key to
 * plain_k[m, slot] (when given) and v = x W_v^T (+ b_v) to raw_v[m, slot],
 * slot = *slot_index (device int64).  Replaces q_proj / k_proj / v_proj,
 * fused_rope and the raw-cache index_copy_ appends of StaticDecode.forward
 * (slimkv/llama3/static_decode.py:148-163).  head_dim 128; x [m, K], m <= 4;
 * q [m, Hq * 128] (row stride q_sm); the caches [m, capacity, Hkv, 128] share
 * strides (c_sm, c_sn); cos/sin [rope_rows, 128] fp32; positions [m] (stride
 * pos_sm), clamped into the tables.  `capacity` (> 0) is the caches' slot
 * count: a slot outside [0, capacity) writes no cache row, and when `status`
 * (device int32, optional) is set SLIMKV_STATUS_BAD_SLOT is stored there
 * (q is still written).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_decode_qkv_args {
    const void* x; int64_t x_sm;
    const void* weight; const void* bias;
    void* q; int64_t q_sm;
    void* raw_k; void* plain_k; void* raw_v; int64_t c_sm, c_sn;
    const int64_t* slot_index;
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* positions; int64_t pos_sm;
    int64_t m, k, heads, kv_heads, head_dim;
    int64_t capacity;
    int32_t* status;   /* optional: SLIMKV_STATUS_BAD_SLOT on a slot outside the caches */
} slimkv_decode_qkv_args;

int slimkv_decode_qkv(const slimkv_decode_qkv_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Prefill attention: causal (bottom-right aligned) GQA attention over a full
 * window, head_dim 128, bf16 in/out, fp32 accumulation and softmax.
 * Replaces the flash_attn_func call of LlamaFlashAttention2._flash_attention_forward
 * (slimkv/llama3/modeling_llama.py:1752-1809) made by the prefill forward
 * (modeling_llama.py:1632-1750) over [sink | up(history) | window | current].
 * q [B, Lq, Hq, 128]  k, v [B, Nk, Hk, 128]  out [B, Lq, Hq, 128] (BSHD);
 * lse [B, Hq, Lq] fp32 contiguous (may be NULL).  With `causal` query i sees
 * keys [0, n_b - Lq + i] where n_b = seqlens_k ? seqlens_k[b] : keys; a row
 * that sees no key gets output 0 and LSE -inf.  Strides are multiples of 8
 * elements, tensors 16-byte aligned, k_sn and v_sn in [128, 2^23) (SLIMKV_EUNSUP
 * otherwise), scale > 0.
 * Optional query RoPE (rope_pairs non-NULL): each query row is rotated as it
 * is loaded, at q_positions[b * qpos_sb + i] clamped into [0, rope_rows)
 * (qpos_sb 0: the same positions for every batch entry), with the
 * reference's bf16 steps (the prefill RoPE of _apply_rotary_with_beacon,
 * modeling_llama.py:1108-1216): rope_pairs [rope_rows, 128] from
 * slimkv_prepare_rope_pairs of the cos/sin tables, rope_repeats = 1 when every
 * row is its first half twice.  The same bits as rotating q with
 * slimkv_prefill_rope first.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_prefill_attention_args {
    const void* q; int64_t q_sb, q_sl, q_sh;
    const void* k; int64_t k_sb, k_sn, k_sh;
    const void* v; int64_t v_sb, v_sn, v_sh;
    void* out; int64_t o_sb, o_sl, o_sh;
    float* lse;
    const int32_t* seqlens_k;
    int64_t batch, queries, heads, kv_heads, keys, head_dim;
    double scale;
    int32_t causal;
    const uint32_t* rope_pairs; int64_t rope_rows;   /* optional query RoPE */
    int32_t rope_repeats;
    const int64_t* q_positions; int64_t qpos_sb;
} slimkv_prefill_attention_args;

int slimkv_prefill_attention(const slimkv_prefill_attention_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Beacon down-projection of the selected rows of a window.
 * Replaces beacon_{k,v}_down_proj inside _project_beacon_key/_value and the
 * beacon-row selection of _incremental_cache
 * (slimkv/llama3/modeling_llama.py:383-390,444-451,1347-1367):
 *   out[b, i, :] = bf16(x[b, rows[i], :] @ weight^T)
 * x [B, length, in_features] bf16 (row strides x_sb, x_sl); rows: device int64
 * [row_count] indices into length (NULL: rows 0..row_count-1; an index
 * outside [0, length) yields a zero row); weight [out_features, in_features]
 * contiguous (nn.Linear layout); out [B, row_count, out_features] bf16.
 * blocks > 1 declares a block-diagonal weight with `blocks` diagonal blocks
 * (per-KV-head bases): each output block contracts its own input block only.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_down_project_args {
    const void* x; int64_t x_sb, x_sl;
    const int64_t* rows; int64_t row_count, length;
    const void* weight;
    void* out; int64_t o_sb, o_sn;
    int64_t batch, in_features, out_features, blocks;
} slimkv_down_project_args;

size_t slimkv_down_project_workspace(const slimkv_down_project_args* a);
int slimkv_down_project(const slimkv_down_project_args* a, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Two down-projections (the K and V latents of one set of beacon rows,
 * beacon_k_down_proj and beacon_v_down_proj at modeling_llama.py:383-390,
 * 444-451) in one launch where neither splits its contraction into partials,
 * else one after the other; the results are those of two slimkv_down_project
 * calls, bit for bit.  The workspace holds
 * slimkv_down_project_pair_workspace(a, b) bytes. */
size_t slimkv_down_project_pair_workspace(const slimkv_down_project_args* a, const slimkv_down_project_args* b);
int slimkv_down_project_pair(const slimkv_down_project_args* a, const slimkv_down_project_args* b, void* workspace,
                             size_t workspace_bytes, void* stream);

/* The down-projection with its epilogue writing the latents straight into
 * beacon pages (no dense staging, no separate append).  Replaces the
 * projection of the window's beacon rows (modeling_llama.py:1347-1367)
 * followed by flush_memory's BeaconPages.append of those rows
 * (slimkv/vllm_plugin/paged_model.py:55-84, paged_cache.py:69-87).
 * Row i of request b is beacon start + i: page table[b*t_sb + (start+i)/slots]
 * (t_cols entries per row), columns sink_elements + ((start+i) % slots) *
 * slot_width + column + [0, out_features); column is 0 for the K latent and
 * key_rank for the V latent (BeaconPageLayout, paged_cache.py:27-44).  Table
 * entries follow the block-table rules above: a row with an index error is
 * not written and is reported through dst->status.
 * a->out / o_sb / o_sn are ignored; workspace as slimkv_down_project. */
typedef struct slimkv_page_rows {
    void* pages; int64_t num_pages, page_stride;
    const int64_t* table; int64_t t_sb, t_cols;
    int64_t slots, sink_elements, slot_width, column;
    int64_t start;
    int32_t* status;   /* optional: SLIMKV_STATUS_BAD_PAGE on an index error */
} slimkv_page_rows;

int slimkv_down_project_to_pages(const slimkv_down_project_args* a, const slimkv_page_rows* dst, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Beacon-page I/O: exact bf16 copies between engine-owned pages and dense
 * latent rows, for `batch` requests at once.
 * Replaces BeaconPages._indices/read/append (slimkv/vllm_plugin/paged_cache.py:60-87)
 * with the layout of BeaconPageLayout (paged_cache.py:11-44).
 * pages: bf16 [num_pages, page_stride] (each page's features contiguous).
 * Logical beacon i of request b lives in physical page
 *   p = table[b*t_sb + i / slots]
 * at columns sink_elements + (i % slots)*(key_rank + value_rank) + [0, key_rank)
 * (K latent), followed by [key_rank, key_rank + value_rank) (V latent).
 * Beacons start .. start+count-1 map to dense row i - start:
 *   K at dense_k[b*dk_sb + (i-start)*dk_sn + c], V likewise.
 * lengths: optional device int32 [batch]; request b moves only beacons
 * i < lengths[b] (the rest of its dense rows and pages are untouched).
 * Each table row holds t_cols entries; entries follow the block-table rules
 * above (a row with an index error moves nothing and sets `status`).
 * to_pages = 1 appends (dense -> pages), 0 reads (pages -> dense).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_beacon_pages_args {
    void* pages; int64_t num_pages, page_stride;
    const int64_t* table; int64_t t_sb, t_cols;
    void* dense_k; int64_t dk_sb, dk_sn;
    void* dense_v; int64_t dv_sb, dv_sn;
    const int32_t* lengths;
    int64_t batch, start, count;
    int64_t slots, key_rank, value_rank, sink_elements;
    int32_t to_pages;
    int32_t* status;   /* optional: SLIMKV_STATUS_BAD_PAGE on an index error */
    const int64_t* starts;   /* optional [batch]: request b's rows start at start + starts[b] */
} slimkv_beacon_pages_args;

int slimkv_beacon_pages(const slimkv_beacon_pages_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Raw-page I/O: exact bf16 copies between raw KV blocks and dense K/V.
 * Replaces RawPages.read/write (slimkv/vllm_plugin/paged_cache.py:102-127).
 * pages: bf16 [blocks, block_size, 2, kv_heads, head_dim] with strides
 * (p_sblk, p_stok, p_skind, p_sh, 1).  Token position t of request b lives in
 * block table[b*t_sb + t / block_size], row t % block_size; positions
 * start .. start+count-1 map to dense row t - start:
 *   K at dense_k[b*dk_sb + h*dk_sh + (t-start)*dk_sn + d], V likewise.
 * lengths: optional device int32 [batch] token counts (positions >= lengths[b]
 * are skipped).  Each table row holds t_cols entries; entries follow the
 * block-table rules above with num_blocks as the pool size.
 * to_pages = 1 writes, 0 reads.
 * ---------------------------------------------------------------------- */
typedef struct slimkv_raw_pages_args {
    void* pages; int64_t num_blocks, p_sblk, p_stok, p_skind, p_sh;
    const int64_t* table; int64_t t_sb, t_cols;
    void* dense_k; int64_t dk_sb, dk_sh, dk_sn;
    void* dense_v; int64_t dv_sb, dv_sh, dv_sn;
    const int32_t* lengths;
    int64_t batch, start, count, block_size, kv_heads, head_dim;
    int32_t to_pages;
    int32_t* status;   /* optional: SLIMKV_STATUS_BAD_PAGE on an index error */
    const int64_t* starts;   /* optional [batch]: request b's positions start at start + starts[b] */
} slimkv_raw_pages_args;

int slimkv_raw_pages(const slimkv_raw_pages_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Raw rows of one decode step over vLLM pages, and flush_memory's raw and
 * sink writes, in one launch for a batch of requests.  No single counterpart
 * in the reference, which rebuilds each request's memory on its own
 * (restore_memory, slimkv/vllm_plugin/paged_model.py:7-52: RawPages.read and
 * BeaconPages.read_sink, paged_cache.py:102-127, 89-99), rotates the raw keys
 * in fa2_decode.decode (slimkv/llama3/fa2_decode.py:107-142) and writes back
 * in flush_memory (paged_model.py:55-84).
 * For request b the dense raw set [sink | window rows | new token] goes to
 * out_k / out_v [B, rows, Hkv, 128] (head stride 128): the sink (sink = 1) from
 * the first 2 * Hkv * 128 elements of the root beacon page beacon_table[b, 0]
 * (K, then V), window row j from the raw pages at position window_start[b] + j
 * (j < raw_count[b]), the new token from new_k / new_v [B, Hkv, 128]; K rotated
 * at positions[b, r] with the reference's bf16 steps (fp32 cos/sin tables
 * [rope_rows, 128]), V copied.  Rows past sink + raw_count[b] + 1 are not
 * written.  With `flush` set, afterwards: the new token's K/V (unrotated) into
 * the raw page at position window_start[b] + raw_count[b] when that is below
 * raw_write_end[b], and the root page's sink replaced by the new token where
 * sink_update[b] (one byte per request) is non-zero.  Table entries follow
 * torch's indexing; an entry outside the pool moves nothing for its row and
 * stores SLIMKV_STATUS_BAD_PAGE in the optional status word.  A request whose
 * raw set (sink + raw_count[b] + 1 rows) exceeds `rows` stores
 * SLIMKV_STATUS_BAD_SLOT there (its rows past `rows`, the new token's among
 * them, are neither gathered nor flushed).
 * ---------------------------------------------------------------------- */
typedef struct slimkv_paged_step_rows_args {
    void* raw_pages; int64_t num_blocks, p_sblk, p_stok, p_skind, p_sh;
    const int64_t* raw_table; int64_t rt_sb, rt_cols, block_size;
    void* beacon_pages; int64_t num_pages, page_stride;
    const int64_t* beacon_table; int64_t bt_sb;
    const void* new_k; int64_t nk_sb;
    const void* new_v; int64_t nv_sb;
    const int64_t* window_start; const int32_t* raw_count;
    const int64_t* positions; int64_t pos_sb;
    const float* cos; const float* sin; int64_t rope_rows;
    void* out_k; int64_t ok_sb, ok_sn;
    void* out_v; int64_t ov_sb, ov_sn;
    int64_t batch, rows, kv_heads, head_dim, sink;
    int32_t flush;
    const int32_t* raw_write_end; const uint8_t* sink_update;
    int32_t* status;
} slimkv_paged_step_rows_args;

int slimkv_paged_step_rows(const slimkv_paged_step_rows_args* a, void* stream);

/* The measurement probes (HBM and LDS read ceilings, the launch floor) are in
 * libslimkv_probe.so, declared in slimkv_probe.h. */

#ifdef __cplusplus
}
#endif

#endif /* SLIMKV_HIP_H */
