/* C-ABI of libabridgekv_amd.so: the MI355X (gfx950) abridged-KV hot path.
 *
 * Plain pointers and sizes only. Device pointers refer to HIP device memory of the current device; `stream` is a
 * hipStream_t (0 = the null stream). Kernel entry points return 0 on success or a hipError_t code; they never
 * synchronise. Planner entry points are pure host code and return the ABKV_* codes below.
 *
 * Cache geometry of the kernels (the served Qwen3-4B attention): a layer's paged KV cache is
 * [num_pages, 2 (K,V), 16 slots, 8 KV heads, 128] bf16 -- the FlashInfer NHD layout the reference's worker allocates
 * (third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1215-1217). 32 query heads (GQA 4).
 */
#ifndef ABRIDGEKV_AMD_H
#define ABRIDGEKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* abkv_stream_t; /* == hipStream_t */

/* Library error codes (negative; kernel entry points otherwise return 0 or a positive hipError_t code). */
enum {
  ABKV_OK = 0,
  ABKV_ERR_ARG = -1,         /* bad argument (null handle, out-of-range group, ...) */
  ABKV_ERR_NO_REQUEST = -2,  /* unknown request id */
  ABKV_ERR_SPAN = -3,        /* the reference's SpanRemovalResult(success=False); message in abkv_planner_last_error */
  ABKV_ERR_POOL = -4,        /* page pool exhausted inside an allocation that passed the total check */
  ABKV_ERR_CAPACITY = -5,    /* output buffer too small */
  ABKV_ERR_SCRATCH = -6      /* abkv_decode_attn_noalloc: the call needs more than the static scratch holds */
};

/* ---------------------------------------------------------------------------------------------------------------
 * Decode attention (kernel 1).
 * Replaces the FlashInfer BatchDecodeWithPagedKVCache call of the stock vLLM backend that the reference's overlay
 * drives with per-group metadata (third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1872-1887, 2184-2276;
 * backend chosen at scripts/bench_decode.py:70) and the pure-torch consumer
 * third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:564-616 (_attend_decode_batched).
 * q [num_seqs, 32, 128] bf16 (strides in elements), block_table [num_seqs, block_table_stride] int32 (group's page
 * table), seq_lens [num_seqs] int32 (physical rows of the group), out [num_seqs, 32, 128] bf16, lse [num_seqs, 32]
 * fp32 natural log (may be NULL). num_pages: pages in kv_cache (page ids are clamped into range).
 * split_pages: even number of pages per split, at most 64. max_pages_per_seq (<= block_table_stride) bounds ceil(seq_len/16);
 * longer sequences are truncated to max_pages_per_seq * 16 rows. workspace: >= abkv_decode_workspace_size(num_seqs, ceil(max_pages/split_pages))
 * bytes when a sequence can need more than one split (may be NULL otherwise); it holds each split's normalised
 * output in fp16 and an fp32 (m, l, scale) record per query head.
 * ------------------------------------------------------------------------------------------------------------- */
size_t abkv_decode_workspace_size(int num_seqs, int max_splits);
int abkv_decode_attn(const void* q, long q_stride_seq, long q_stride_head, const void* kv_cache, int num_pages,
                     const int32_t* block_table, long block_table_stride, const int32_t* seq_lens, int num_seqs,
                     int max_pages_per_seq, int split_pages, float scale, void* out, long out_stride_seq,
                     long out_stride_head, float* lse, void* workspace, size_t workspace_bytes,
                     abkv_stream_t stream);

/* abkv_decode_attn without a workspace argument and without any allocation. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The split partials live in a static device array of ABKV_DECODE_NOALLOC_SCRATCH_BYTES that the
 * library image holds on every GPU it runs on until the process ends; a call whose partials need more
 * (abkv_decode_workspace_size(num_seqs, ceil(max_pages_per_seq / split_pages)) bytes when that is > 1 split) returns
 * ABKV_ERR_SCRATCH and launches nothing. Nothing in the scratch has to start at zero (every partial a launch reads
 * was written by that launch). Every call on one GPU shares that GPU's scratch: calls that overlap on one GPU (other
 * streams, other host threads) race and must be serialised by the caller. */
#define ABKV_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int abkv_decode_attn_noalloc(const void* q, long q_stride_seq, long q_stride_head, const void* kv_cache,
                             int num_pages, const int32_t* block_table, long block_table_stride,
                             const int32_t* seq_lens, int num_seqs, int max_pages_per_seq, int split_pages,
                             float scale, void* out, long out_stride_seq, long out_stride_head, float* lse,
                             abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * KV-cache row movement for compaction (kernel 2, device half).
 * Replaces GPUModelRunner._execute_kv_copy_group (gpu_model_runner.py:1194-1224): ops [n, 4] int32 rows
 * (src_block, src_off, dst_block, dst_off) applied to each of n_layers layer caches (<= 16) with gather-then-scatter
 * semantics. abkv_kv_move_segments: ops are split into segments (seg_offsets [n_segments + 1] int32, device) touching
 * disjoint pages; inside a segment no op may read a slot written by an earlier op of that segment (true for
 * compaction ops: increasing source, dst < src, single_type_kv_cache_manager.py:378-381). abkv_kv_copy_staged: any op
 * list, rows staged through `stage` (>= abkv_kv_stage_bytes). page_bytes / half_bytes / slot_bytes describe the cache
 * (64 KiB / 32 KiB / 2 KiB for the served geometry); ops naming a page outside [0, num_pages) or an offset outside
 * [0, block_size) are skipped.
 * ------------------------------------------------------------------------------------------------------------- */
int abkv_kv_move_segments(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                          long half_bytes, int slot_bytes, const int32_t* ops, const int32_t* seg_offsets, int n_segments, abkv_stream_t stream);
/* abkv_kv_move_mixed: one launch over the ordered segments of abkv_kv_move_segments (n_segments >= 0; ops /
 * seg_offsets may be NULL when 0) and n_free independent ops free_ops [n_free, 4]: ops that read or write no slot
 * another op of the launch writes, so they run in any order (the layout abkv_moves_pack builds from a planner step's
 * fused moves; the same executor, gpu_model_runner.py:1194-1224). */
int abkv_kv_move_mixed(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                       long half_bytes, int slot_bytes, const int32_t* ops, const int32_t* seg_offsets, int n_segments,
                       const int32_t* free_ops, int n_free, abkv_stream_t stream);
size_t abkv_kv_stage_bytes(int n_layers, int n_ops, int slot_bytes);
int abkv_kv_copy_staged(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                        long half_bytes, int slot_bytes, const int32_t* ops, int n_ops, void* stage, size_t stage_bytes, abkv_stream_t stream);

/* KV append: replaces the stock vLLM compiled op reshape_and_cache(_flash) fed by slot maps from
 * third_party/vllm_overlay/vllm/v1/worker/block_table.py:186-197. key/value [num_tokens, slot_bytes] (row strides in
 * bytes); slot_mapping [num_tokens] int64, negative or >= num_pages * block_size = skip. */
int abkv_kv_append(const void* key, long key_stride, const void* value, long value_stride,
                   const int64_t* slot_mapping, int num_tokens, void* kv_cache, int num_pages, long page_bytes,
                   long half_bytes, int slot_bytes, int block_size, abkv_stream_t stream);

/* Fused rotary embedding + KV append (served geometry: 32 query / 8 KV heads, head size 128, NeoX halves).
 * Replaces the model's rotary op followed by reshape_and_cache on the overlay's attention path (positions from
 * third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1593-1598 via config/compresslm.py:208-216; slots from
 * block_table.py:186-197). q [T, 32, 128] (strides in elements, dims contiguous) and key [T, 8, 128] are rotated in
 * place; rotated key and value rows are written at slot_mapping[t] (NULL: rotate only; < 0 or past the cache: skip).
 * positions [T] int64: RoPE positions when block_c == 0; otherwise logical positions of the abridged layout (period
 * block_c + codes_k, codes_k a power of two <= block_c) mapped on the device to block * block_c + (offset < block_c ?
 * offset : floor(bitrev(offset - block_c) * span / codes_k)) with span = code_span, the in-block range the codes
 * summarize (0: block_c; block_c - T with a retained tail of T rows, config/compresslm.py:192-206; codes_k <=
 * span <= block_c). cos_sin [max_pos, 128] fp32: cos of the 64 rotary
 * frequencies then their sin. The caller guarantees every RoPE position is < max_pos (the Python wrapper checks it);
 * the kernel clamps positions into [0, max_pos) only so that no read leaves the table. */
int abkv_rope_kv_append(void* q, long q_stride_t, long q_stride_h, void* key, long key_stride_t, const void* value,
                        long value_stride_t, const int64_t* positions, int num_tokens, int block_c, int codes_k,
                        int code_span, const float* cos_sin, long max_pos, const int64_t* slot_mapping,
                        void* kv_cache, int num_pages, abkv_stream_t stream);

/* Slot mapping on device: BlockTable.compute_slot_mapping (block_table.py:186-197, non-CP branch) on the physical
 * positions of one KV-cache group (gpu_model_runner.py:1579-1590: phys = logical - compacted[req, group]).
 * slot = table[r][p / block_size] * block_size + p % block_size with r = req_idx[t], p = positions[t] -
 * compacted[r] (compacted NULL: positions are physical); -1 when p < 0, p is past the table row
 * (block_table_stride pages) or r is outside [0, num_reqs). */
int abkv_slot_mapping(const int32_t* req_idx, const int64_t* positions, int num_tokens, const int32_t* block_table,
                      int num_reqs, long block_table_stride, int block_size, const int32_t* compacted,
                      int64_t* slot_mapping, abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Block-masked teacher-forced attention (kernel 3).
 * Replaces the FlexAttention call of CompressLM.forward (abridgekv/compress_forward.py:1134-1230) with the mask of
 * _arith_mask_mod (abridgekv/compress_forward.py:695-727) and the per-query-head code quota (:725-726, :230-236):
 * layout N blocks of [block_c content | pause_passes passes of codes_k codes], seq_len = N * (block_c + pause_passes
 * * codes_k) (L = pause_passes, compress_forward.py:20-31, 566-649: pass l of a block reads its block's content, its
 * pass l - 1 and its own pass (by pause_xattn); later blocks read only the final pass; the quota counts a code row's
 * slot within its pass; L > 1 runs the per-element mask).
 * q [batch, seq_len, 32, 128], k/v [batch, seq_len, 8, 128], out [batch, seq_len, 32, 128] bf16 with element strides
 * (dims contiguous); prompt_len [batch] int32 raw-prompt content tokens (NULL: none); head_quota [32] int32 code slots
 * visible per query head (NULL: all); retain_tail = T of a retained tail (retain_tail_kv; 0: none; 0 <= T <
 * block_c): a block's codes never see its own last T content rows (:714-715, :721-722), and tail_policy
 * (retain_tail_policy, _retained_tail_visible :99-124) names the later rows that see them: ABKV_TAIL_STATIC every
 * later row, ABKV_TAIL_STICKY every content row of the next block, ABKV_TAIL_ROLLING content row i of the next block
 * from tail row i on (key in-block offset >= block_c - T + i); ABKV_TAIL_RAW is CompressLM's raw_tail = T
 * (_raw_tail_visible, compress_forward.py:89-96; 0 <= T <= block_c): the rolling window, with the codes seeing their
 * whole block (code_excluded_tail = 0, :309-311), on the per-element mask; lse [batch, 32, seq_len] fp32 natural log
 * (NULL: not written).
 * ------------------------------------------------------------------------------------------------------------- */
#define ABKV_TAIL_STATIC 0
#define ABKV_TAIL_ROLLING 1
#define ABKV_TAIL_STICKY 2
#define ABKV_TAIL_RAW 3
/* pause_xattn: a code row's attention to its own block's code rows (compress_forward.py:313-314, 622-625): all of
 * them (ABKV_XATTN_FULL, the served setting), those at or before its own row (ABKV_XATTN_CAUSAL), none
 * (ABKV_XATTN_NONE). The non-full settings run the per-element mask on every tile up to the query's block. */
#define ABKV_XATTN_FULL 0
#define ABKV_XATTN_CAUSAL 1
#define ABKV_XATTN_NONE 2
/* replay_rows = R (replay_tail, compress_forward.py:20-31, 594-603): after each block's codes, R rows replaying its
 * last R content tokens (block period block_c + pause_passes * codes_k + R): a replay row sees its block's content,
 * final pass and replay rows (causally), and content row i of the next block sees the previous block's replay rows
 * from row i on; replay_exclude (code_exclude_replay_tail) hides a block's last R content rows from its codes.
 * Exclusive with retain_tail.
 * copy_rows: a copy region after the N blocks (CompressLM.forward's copy_lambda, compress_forward.py:631-633,
 * 1185-1189), seq_len = N * (block_c + pause_passes * codes_k + replay_rows) + copy_rows: its rows see the last block's final pass
 * (slots < quota) and the copy rows up to themselves, and no other row sees them. codes_k = 0 (pause_passes 1, no
 * copy rows): plain causal attention within blocks of block_c rows (the full-context baseline and teacher,
 * compress_forward.py:952-956, 1095-1105). */
int abkv_prefill_masked_attn(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                             long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                             long v_stride_s, long v_stride_h, int batch, int block_c, int codes_k, int num_blocks,
                             int seq_len, const int32_t* prompt_len, const int32_t* head_quota, int retain_tail,
                             int tail_policy, int pause_xattn, int pause_passes, int copy_rows, int replay_rows,
                             int replay_exclude, float scale, void* out, long out_stride_b, long out_stride_s,
                             long out_stride_h, float* lse, abkv_stream_t stream);

/* Backward of abkv_prefill_masked_attn: the gradients dq [batch, seq_len, 32, 128] and dk, dv [batch, seq_len, 8,
 * 128] (bf16, element strides, dims contiguous; written, not accumulated) of sum(dout * out) under the same mask,
 * from the forward's out and lse (lse required). Replaces the FlexAttention backward the reference trains through
 * (abridgekv/compress_forward.py:1134-1230 under autograd; its self-test calls backward at :1329).
 * workspace >= abkv_prefill_masked_bwd_workspace_size(batch, seq_len) bytes. */
size_t abkv_prefill_masked_bwd_workspace_size(int batch, int seq_len);
int abkv_prefill_masked_attn_bwd(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                                 long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                                 long v_stride_s, long v_stride_h, const void* out, long out_stride_b,
                                 long out_stride_s, long out_stride_h, const void* dout, long dout_stride_b,
                                 long dout_stride_s, long dout_stride_h, const float* lse, int batch, int block_c,
                                 int codes_k, int num_blocks, int seq_len, const int32_t* prompt_len,
                                 const int32_t* head_quota, int retain_tail, int tail_policy, int pause_xattn,
                                 int pause_passes, int copy_rows, int replay_rows, int replay_exclude, float scale,
                                 void* dq,
                                 long dq_stride_b, long dq_stride_s, long dq_stride_h, void* dk, long dk_stride_b,
                                 long dk_stride_s, long dk_stride_h, void* dv, long dv_stride_b, long dv_stride_s,
                                 long dv_stride_h, void* workspace, size_t workspace_bytes, abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Multi-query attention over the paged cache: prompt-chunk prefill (causal) and the CompressLM code step.
 * Replaces the FlashInfer paged-prefill call with a custom mask that the overlay routes code steps to
 * (third_party/vllm_overlay/patch_stock_flashinfer.py:30-152, masks from
 * third_party/vllm_overlay/vllm/v1/worker/compresslm_masks.py:165-239 and gpu_model_runner.py:2042-2107): in a group's
 * physical layout the code step's mask is "keys < code_start + q_g", so each request carries a key limit.
 * q [T, 32, 128] (token stride, head stride), request r's queries are tokens [q_start[r], q_start[r+1]) at physical
 * positions kv_start[r] + i and see keys < kv_limit[r] (and <= their position when request r is causal: causal[r] != 0,
 * or causal_default when causal is NULL), except the keys of kv_excluded[r] = [start, end) (NULL: none; the code
 * step's own-block retained tail, gpu_model_runner.py:2086-2094 "excluded" ranges, compresslm_masks.py:206-213;
 * start >= end: none). tile_req / tile_q0 [num_tiles] list the 64-row query tiles (request, first
 * row). All index arrays are device int32. lse [T, 32] or NULL. num_splits > 1 splits every tile's keys into
 * num_splits ranges of split_tiles 64-key tiles (split z covers tiles [z * split_tiles, (z + 1) * split_tiles); the
 * ranges must cover every request's keys) computed by separate workgroups and merged; the partials use workspace
 * (>= abkv_paged_prefill_workspace_size(num_tokens, num_splits) bytes). num_tokens = q_start[num_reqs], the rows
 * the launch covers: the split merge writes exactly those rows, and rows of q / out past them are never touched.
 * num_splits <= 1: no split, no workspace.
 * ------------------------------------------------------------------------------------------------------------- */
size_t abkv_paged_prefill_workspace_size(int num_tokens, int num_splits);
int abkv_paged_prefill_attn(const void* q, long q_stride_t, long q_stride_h, const void* kv_cache, int num_pages,
                            const int32_t* block_table, long block_table_stride, int block_table_width,
                            const int32_t* q_start, const int32_t* kv_start, const int32_t* kv_limit,
                            const int32_t* kv_excluded, const int32_t* tile_req, const int32_t* tile_q0, int num_tiles,
                            const int32_t* causal,
                            int causal_default, float scale, void* out, long out_stride_t, long out_stride_h, float* lse,
                            int num_tokens, int num_splits, int split_tiles, void* workspace, size_t workspace_bytes,
                            abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Per-head packed code pages (the reference's packed KV sidecar for per-head quota schedules:
 * third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:12-155 PackedKVLayout, :214-284 PackedKVSidecar
 * capture, :564-616 batched decode consumer, :648-741 per-request consumer). A packed page holds one closed block's
 * code rows of one layer as [2 (K,V)][rows][128] bf16, KV head h's first q_h code rows at rows off_h .. off_h+q_h-1,
 * off_h = q_0 + ... + q_{h-1}, rows = the sum of the layer's 8 head quotas (each in [1, 2048]). A layer's pool is
 * [pool_pages, 2, rows, 128]; a sequence lists its packed page ids (one per captured block, the same id in every
 * layer) in packed_table [num_seqs, packed_table_stride] with packed_count [num_seqs] entries (device int32).
 *
 * abkv_packed_capture: for capture c and layer l, copy the K_max code rows at physical positions code_start[c] ..
 * (block_table row c) of layer_kv[l] into page dst_page[c] of layer_pool[l]. layer_kv / layer_pool: device arrays of
 * num_layers device pointers; layer_rows [num_layers], layer_quota [num_layers, 8]: device int32.
 *
 * abkv_decode_attn_packed: decode attention over the paged rows [0, seq_len) (as abkv_decode_attn) plus, for KV
 * head h, the sequence's side rows (q_h rows of each of its packed pages). head_quota: HOST int32 [8] (this layer's
 * quotas; packed_rows must equal their sum). side_split_rows: abkv_decode_side_split_rows(min quota).
 * max_packed_per_seq * max quota < 2^21. workspace >= abkv_decode_packed_workspace_size(...) bytes (always needed).
 *
 * abkv_paged_prefill_attn_packed: as abkv_paged_prefill_attn (always split: num_splits >= 1 ranges of split_tiles
 * paged tiles) plus the side rows, visible to every query of the request, in side_splits ranges of side_split_tiles
 * 64-row tiles (side_splits * side_split_tiles * 64 >= max_packed_per_seq * max quota); a non-causal request (code
 * step) sees paged keys < min(kv_limit, kv_start + q_h) for KV head h (head_quota_dev: device int32 [8], the same
 * quotas as the host head_quota). max_packed_per_seq <= 2048. workspace >=
 * abkv_paged_prefill_workspace_size(num_tokens, num_splits + side_splits).
 * ------------------------------------------------------------------------------------------------------------- */
int abkv_packed_capture(const void* const* layer_kv, void* const* layer_pool, const int32_t* layer_rows,
                        const int32_t* layer_quota, int num_layers, int num_pages, int pool_pages,
                        const int32_t* block_table, long block_table_stride, int block_table_width,
                        const int32_t* code_start, const int32_t* dst_page, int num_captures, abkv_stream_t stream);
int abkv_decode_side_split_rows(int q_min);
size_t abkv_decode_packed_workspace_size(int num_seqs, int max_pages_per_seq, int split_pages, int max_side_pages,
                                         int side_q_max, int side_split_rows);
int abkv_decode_attn_packed(const void* q, long q_stride_seq, long q_stride_head, const void* kv_cache, int num_pages,
                            const int32_t* block_table, long block_table_stride, const int32_t* seq_lens,
                            int num_seqs, int max_pages_per_seq, int split_pages, const void* packed_kv,
                            int packed_pool_pages, int packed_rows, const int32_t* head_quota,
                            const int32_t* packed_table, long packed_table_stride, const int32_t* packed_count,
                            int max_packed_per_seq, int side_split_rows, float scale, void* out, long out_stride_seq,
                            long out_stride_head, float* lse, void* workspace, size_t workspace_bytes,
                            abkv_stream_t stream);
int abkv_paged_prefill_attn_packed(const void* q, long q_stride_t, long q_stride_h, const void* kv_cache,
                                   int num_pages, const int32_t* block_table, long block_table_stride,
                                   int block_table_width, const int32_t* q_start, const int32_t* kv_start,
                                   const int32_t* kv_limit, const int32_t* kv_excluded, const int32_t* tile_req,
                                   const int32_t* tile_q0, int num_tiles, const int32_t* causal, int causal_default,
                                   const int32_t* head_quota_dev, const void* packed_kv, int packed_pool_pages,
                                   int packed_rows, const int32_t* head_quota, const int32_t* packed_table,
                                   long packed_table_stride, const int32_t* packed_count, int max_packed_per_seq,
                                   float scale, void* out, long out_stride_t, long out_stride_h, float* lse,
                                   int num_tokens, int num_splits, int split_tiles, int side_splits,
                                   int side_split_tiles, void* workspace, size_t workspace_bytes,
                                   abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * fp32 mode of the three attention paths (same semantics as the bf16 entry points above, fp32 q / K / V / out,
 * fp32 accumulation and accurate exp/log): the reference's PyTorch attention run in fp32
 * (abridgekv/gen_compress.py:359-360, 555; compresslm_packed_kv.py:608-613; compress_forward.py:695-727).
 * Caches are [num_pages, 2, 16, 8, 128] fp32. A correctness mode, not a tuned path.
 * ------------------------------------------------------------------------------------------------------------- */
/* Decode over the group page table: out [B, 32, 128] fp32 (strides), lse [B, 32] or NULL. */
int abkv_decode_attn_f32(const float* q, long q_stride_seq, long q_stride_head, const float* kv_cache, int num_pages,
                         const int32_t* block_table, long block_table_stride, const int32_t* seq_lens, int num_seqs,
                         int max_pages_per_seq, float scale, float* out, long out_stride_seq, long out_stride_head,
                         float* lse, abkv_stream_t stream);

/* Paged multi-query attention (prompt chunks, code steps): as abkv_paged_prefill_attn, with tok_req [num_tokens]
 * (request of every query token) in place of the tile list. lse [T, 32] or NULL. */
int abkv_paged_prefill_attn_f32(const float* q, long q_stride_t, long q_stride_h, const float* kv_cache, int num_pages,
                                const int32_t* block_table, long block_table_stride, int block_table_width,
                                const int32_t* q_start, const int32_t* kv_start, const int32_t* kv_limit,
                                const int32_t* kv_excluded, const int32_t* tok_req, int num_tokens,
                                const int32_t* causal, int causal_default, float scale, float* out, long out_stride_t,
                                long out_stride_h, float* lse, abkv_stream_t stream);

/* Compression-masked teacher-forced attention: as abkv_prefill_masked_attn (strides in elements, head dims
 * contiguous and 16-byte aligned rows). lse [B, 32, seq_len] or NULL. */
int abkv_prefill_masked_attn_f32(const float* q, long q_sb, long q_ss, long q_sh, const float* k, long k_sb,
                                 long k_ss, long k_sh, const float* v, long v_sb, long v_ss, long v_sh, int batch,
                                 int block_c, int codes_k, int num_blocks, int seq_len, const int32_t* prompt_len,
                                 const int32_t* head_quota, int retain_tail, int tail_policy, int pause_xattn,
                                 int pause_passes, int copy_rows, int replay_rows, int replay_exclude, float scale,
                                 float* out, long o_sb, long o_ss, long o_sh, float* lse,
                                 abkv_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Compaction planner (kernel 2, host half). Bit-exact restatement of the reference's scheduler/KV-manager
 * bookkeeping: Scheduler.mask_token_span (third_party/vllm_overlay/vllm/v1/core/sched/scheduler.py:2060-2204),
 * SingleTypeKVCacheManager.compact_kv_cache_span/_truncate_compacted_blocks/allocate_new_blocks/free
 * (v1/core/single_type_kv_cache_manager.py:122-145, 173-188, 358-452), BlockPool.get_new_blocks/free_blocks/
 * copy_kv_slots (v1/core/block_pool.py:295-325, 385-399, 488-550), FreeKVCacheBlockQueue (v1/core/kv_cache_utils.py:
 * 157-345), KVCacheManager.allocate_slots (v1/core/kv_cache_manager.py:206-340), CompactedSpanIndex
 * (v1/compacted_spans.py:8-68). One planner = one page pool shared by num_groups KV-cache groups.
 * ------------------------------------------------------------------------------------------------------------- */

/* free_order: NULL (pages 1..num_blocks-1 in id order, page 0 null -- the reference's construction) or a
 * permutation of 1..num_blocks-1 giving the initial free-queue order. */
void* abkv_planner_create(int num_blocks, int num_groups, int block_size, const int32_t* free_order,
                          int64_t max_model_len);
void abkv_planner_destroy(void* planner);
/* 1 (default): build the reference-format op batches; 0: skip them (the bookkeeping and the fused moves are unchanged;
 * take_step_outputs then returns no op rows). The reference always builds them (single_type_kv_cache_manager.py:
 * 378-381, consumed by gpu_model_runner.py:1194-1224); a caller that executes the fused moves only turns them off. */
int abkv_planner_set_op_rows(void* planner, int enabled);
const char* abkv_planner_last_error(void* planner);
int abkv_planner_add_request(void* planner, int64_t rid);
int abkv_planner_free_request(void* planner, int64_t rid);
int abkv_planner_set_num_computed(void* planner, int64_t rid, int64_t num_computed_tokens);
int64_t abkv_planner_get_num_computed(void* planner, int64_t rid);
/* 1 = allocated, 0 = pool cannot cover it (reference returns None), < 0 = error. */
int abkv_planner_allocate_slots(void* planner, int64_t rid, int64_t num_new_tokens);
int abkv_planner_mask_token_span(void* planner, int64_t rid, int64_t start, int64_t end, const int32_t* groups,
                                 int n_groups, int64_t* tokens_removed, int64_t* blocks_freed);
int abkv_planner_pending_sizes(void* planner, int64_t* n_op_rows, int64_t* n_trunc_rows, int64_t* n_fused_rows);
/* op_rows [n,7] (rid, group, batch, src_block, src_off, dst_block, dst_off); trunc_rows [n, 1+G];
 * fused_rows [n,6] (rid, group, src_block, src_off, dst_block, dst_off): the step's removals composed per
 * (request, group), rows truncated later in the same step are not moved. */
int abkv_planner_take_step_outputs(void* planner, int64_t* op_rows, int64_t op_cap, int64_t* n_ops,
                                   int64_t* trunc_rows, int64_t trunc_cap, int64_t* n_trunc, int64_t* fused_rows,
                                   int64_t fused_cap, int64_t* n_fused);
/* Device-ready move lists from fused_rows [n, 6] (host; the host side of the executor above,
 * gpu_model_runner.py:1194-1224, for the fused form): per group g < num_groups, back to back in `out` (capacity
 * >= 5 n + 4 num_groups int32), the ops [n_g, 4] -- first the ordered segments, one per (request, group) run holding
 * the run's ops that lie on a dependency (an op whose destination is another op's source, and that op), in emission
 * order; then every other op, independent of all others -- and the segment offsets [n_segments + 1], each group's
 * section 16-byte aligned. index [num_groups, 5] = (ops_at, n_ops, offs_at, n_segments, n_free) in int32 elements of
 * `out`; feeds abkv_kv_move_mixed. Returns the elements written, ABKV_ERR_CAPACITY or ABKV_ERR_ARG (group out of
 * range, a run split in two, an offset outside [0, 65536), a slot read twice, or an op that reads a slot an earlier
 * op of its run writes). */
int64_t abkv_moves_pack(const int64_t* fused_rows, int64_t n, int num_groups, int32_t* out, int64_t out_cap,
                        int64_t* index);
/* The step outputs for a caller that executes fused moves: trunc_rows as abkv_planner_take_step_outputs, and the
 * device move lists of abkv_moves_pack written directly into `out` (capacity >= 5 x the fused bound of
 * abkv_planner_pending_sizes + 4 num_groups int32; index [num_groups, 5] as abkv_moves_pack). Clears the step.
 * Returns the int32 elements written, ABKV_ERR_CAPACITY or ABKV_ERR_ARG. (The reference's scheduler output,
 * scheduler.py:2060-2204 and sched/output.py:221-225, in the fused form.) */
int64_t abkv_planner_take_moves_packed(void* planner, int64_t* trunc_rows, int64_t trunc_cap, int64_t* n_trunc,
                                       int32_t* out, int64_t out_cap, int64_t* index);
/* Capacities of abkv_planner_take_move_runs for the pending step: run records and page-window entries. */
int abkv_planner_pending_run_sizes(void* planner, int64_t* n_runs, int64_t* n_pages);
/* The same step outputs as abkv_planner_take_moves_packed with the per-row work left to the device: trunc_rows and
 * index as there, and per (request, group) run with moved rows one record of 30 int32 (the run's row count, its first
 * row in its page window, output positions and counts of its ordered and independent ops, its segment entry, and the
 * run's row map in closed form: up to 8 thresholds with their running removal lengths), the runs' page windows and
 * groups [num_groups, 4] (segment-offset position, n_segments, end of padding, 0). abkv_moves_expand turns them into
 * the int32 move lists take_moves_packed writes, element for element. sizes = (records, page entries, int32 elements
 * of the move lists). Clears the step. Returns 0, ABKV_ERR_CAPACITY (nothing cleared) or ABKV_ERR_ARG (page size not
 * a power of two, more than 8 removals of one request and group in one step, rows past a page list, or a step
 * interleaved with an allocation). (scheduler.py:2060-2204 and gpu_model_runner.py:1194-1224, the op rows generated
 * on the device.) */
int abkv_planner_take_move_runs(void* planner, int64_t* trunc_rows, int64_t trunc_cap, int64_t* n_trunc,
                                int32_t* runs, int64_t runs_cap, int32_t* pages, int64_t pages_cap, int32_t* groups,
                                int64_t* index, int64_t* sizes);
/* Device expansion of abkv_planner_take_move_runs' outputs (runs, pages, groups on the device; n_runs = sizes[0],
 * the records that call wrote -- record slots past it are not cleared and must not be passed; n_pages = entries of
 * `pages`; out_elems = sizes[2]) into `out`, ready for abkv_kv_move_mixed. page_shift = log2(page size). One launch of
 * n_runs + num_groups workgroups on `stream`; every store is bounds-checked against the record's counts and
 * out_elems, every page read against the record's window and n_pages, and negative positions are skipped. */
int abkv_moves_expand(const int32_t* runs, int n_runs, const int32_t* pages, long n_pages, const int32_t* groups,
                      int num_groups, int page_shift, int32_t* out, long out_elems, abkv_stream_t stream);
int64_t abkv_planner_num_free(void* planner);
int64_t abkv_planner_free_queue(void* planner, int32_t* out, int64_t cap);
int64_t abkv_planner_block_ids(void* planner, int64_t rid, int group, int32_t* out, int64_t cap);
int abkv_planner_fill_block_table(void* planner, const int64_t* rids, int n, int group, int32_t* table,
                                  int64_t stride, int32_t pad);
int64_t abkv_planner_compacted(void* planner, int64_t rid, int group);
int64_t abkv_planner_spans(void* planner, int64_t rid, int group, int64_t* out, int64_t cap);
int64_t abkv_planner_logical_to_physical(void* planner, int64_t rid, int group, int64_t pos);
int64_t abkv_planner_physical_to_logical(void* planner, int64_t rid, int group, int64_t pos);
int abkv_planner_is_token_active(void* planner, int64_t rid, int group, int64_t pos);
/* events [n, 6] int64 (kind, rid, a, b, group_mask, 0): 0 add, 1 schedule a tokens, 2 mask [a, b) in the groups of
 * group_mask (< 0: all), 3 free, 4 drop step outputs. Returns n, or -(failing index + 1). */
int64_t abkv_planner_apply_events(void* planner, const int64_t* events, int64_t n);

#ifdef __cplusplus
}
#endif
#endif /* ABRIDGEKV_AMD_H */
