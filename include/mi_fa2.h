/*
 * mi_fa2.h -- C ABI of the MI355X (gfx950) FlashAttention-2 forward library, libmi_fa2.so.
 *
 * The library replaces the attention hot path of shubhav1/my-inference-engine:
 *   - the Triton kernel `fa2_forward`            (kernels/fa2.py:14-162),
 *   - its launcher `FlashAttention2Function`     (kernels/fa2.py:164-214),
 *   - the per-step dense K/V gather it is fed by (kv_cache.py:117-121, called at model.py:97),
 * with hand-written HIP kernels: an MFMA/LDS-tiled prefill kernel, a split-KV decode kernel that
 * reads K/V straight out of the paged cache's blocks, and a split combine kernel (head_dim 128,
 * bf16/fp16), a general kernel for the launcher's other head dims and fp32; and the steps either
 * side of it: a fused RoPE + paged cache write and a fused last-position token sampler.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers except the stride arrays, which are host arrays.
 *   - Strides are in ELEMENTS, int64.  The innermost (head_dim) stride must be 1, every other stride
 *     a multiple of 8 elements and every tensor base 16-byte aligned (16-byte vector loads).  The
 *     token stride of K and V (the slot stride of a pool) is also the row pitch of their loads:
 *     at least head_dim, also where seqlen_k is 1 (rows must not overlap).
 *   - `dtype` is MI_FA2_BF16 or MI_FA2_FP16; q, k, v and o share it (the sampler also takes
 *     MI_FA2_FP32 logits, mi_fa2_fwd_general MI_FA2_FP32 inputs).  Softmax and accumulation
 *     are fp32; `lse` is fp32 (natural log, like the reference's L, kernels/fa2.py:158,189).
 *   - head_dim must be 128 (the Qwen2.5 shape) except in mi_fa2_fwd_general; heads_q must be a
 *     multiple of heads_kv and query head h reads kv head h / (heads_q / heads_kv)
 *     (kernels/fa2.py:53, model.py:70-75).
 *   - Causal masking is bottom-right aligned per row: query i of a row sees key j iff
 *     j <= i + kv_len - seqlen_q (kernels/fa2.py:109-111,132-138).  Keys j >= kv_len are never read
 *     as data: their loads are predicated off, so padding may hold anything, NaN included.
 *   - A query that sees no key gets an output of 0 and an lse of -inf.  This matches the
 *     reference's fp32 SDPA path (model.py:104-107, kernels/test_fa2.py:28-35); the reference's
 *     Triton kernel would produce 0/0 = NaN there.
 *   - Launches are asynchronous on `stream` (a hipStream_t); nothing is synchronised and nothing
 *     is allocated.  Entry points that need scratch take a caller-owned workspace whose size the
 *     matching *_workspace_size() returns; its contents need no initialisation.  Calls that
 *     overlap in time (other streams) must not share one workspace.
 *   - Return value: MI_FA2_OK (0) or an error code; mi_fa2_last_error() then describes it.
 */
#ifndef MI_FA2_H
#define MI_FA2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_FA2_API __attribute__((visibility("default")))

typedef struct ihipStream_t* mi_fa2_stream_t; /* the same handle type as hipStream_t */

enum mi_fa2_status {
  MI_FA2_OK = 0,
  MI_FA2_ERR_INVALID = 1,     /* bad pointer, shape, stride or alignment */
  MI_FA2_ERR_UNSUPPORTED = 2, /* valid request outside the kernels' envelope (e.g. head_dim 64) */
  MI_FA2_ERR_WORKSPACE = 3,   /* workspace missing or smaller than *_workspace_size() */
  MI_FA2_ERR_LAUNCH = 4       /* the HIP runtime refused the launch */
};

enum mi_fa2_dtype { MI_FA2_BF16 = 0, MI_FA2_FP16 = 1, MI_FA2_FP32 = 2 };

/* Library version string, e.g. "mi_fa2 0.1.0 gfx950". */
MI_FA2_API const char* mi_fa2_version(void);

/* Message describing the most recent failing call on this thread ("" if none). */
MI_FA2_API const char* mi_fa2_last_error(void);

/*
 * How the launches are sized for a device: no counterpart in the reference, whose Triton launcher
 * sizes its grid from the shapes alone (kernels/fa2.py:192) and leaves the rest to the autotuner.
 * The kernels size their grids from the device's compute units and deal work-groups over its XCDs
 * (each XCD has its own L2); MI355X has 256 CUs in 8 XCDs, a partitioned device reports its own
 * share.  num_cus <= 0: the plan of the current device (read once per device); otherwise the plan
 * the library would use on a device of num_cus CUs in num_xcds XCDs (no GPU needed).
 *   xcds_mapped: XCDs the prefill grid deals work-groups over (num_xcds if a power of two, else 1)
 *   decode_work_groups_*: split-decode work-groups per launch (3 or 2 per CU; MI_FA2_DECODE_WGS
 *   overrides both), capped at run time by the launch's 128-key chunk count.
 *   prefill_one_stream_min_work_groups, prefill_one_stream_max_keys: prefill launches of at
 *   least that many work-groups (two per CU) whose query tiles see at most that many keys take
 *   the one-stream work-group shape (4 waves, two work-groups per CU), the others the two-stream
 *   shape (8 waves, one per CU); MI_FA2_PREFILL_STREAMS=1 or 2 forces one shape.
 */
typedef struct mi_fa2_plan {
  int32_t num_cus;
  int32_t num_xcds;
  int32_t xcds_mapped;
  int32_t decode_work_groups_paged;
  int32_t decode_work_groups_dense;
  int32_t prefill_one_stream_min_work_groups;
  int32_t prefill_one_stream_max_keys;
} mi_fa2_plan;
MI_FA2_API int mi_fa2_launch_plan(int32_t num_cus, int32_t num_xcds, mi_fa2_plan* out);

/*
 * Measurement support, no counterpart in the reference (which publishes no kernel timings): the
 * shader clock the attention kernels actually run at.  With probe set (device memory, 16 uint64,
 * zeroed by the caller), every later prefill, decode and general-kernel launch adds, for thread 0
 * of each of its first 8 work-groups, the shader cycles its CU counted (s_memtime) and the
 * 100 MHz real-time ticks (s_memrealtime) between that work-group's start and end to
 * probe[2 x] and probe[2 x + 1], x = the work-group's XCD (0-7; the first 8 work-groups of a
 * launch run one per XCD on MI355X).  The clock XCD x ran those kernels at is
 * probe[2 x] / probe[2 x + 1] x 100 MHz.  The counts of different CUs are never compared (each
 * CU counts its own clocks and stops while clock-gated).  probe NULL turns it off (the default);
 * the setting is process-wide and applies to launches made after the call.  Measurement only:
 * calls that overlap in time accumulate into the same sums.
 */
MI_FA2_API int mi_fa2_set_clock_probe(uint64_t* probe);

/*
 * Padded forward.  Replaces FlashAttention2Function.forward (kernels/fa2.py:164-214) and the Triton
 * launch at kernels/fa2.py:192-207, same argument meaning:
 *   q [batch, heads_q, seqlen_q, 128], k/v [batch, heads_kv, seqlen_k, 128], o like q,
 *   lse [batch, heads_q, seqlen_q] fp32 (may be NULL), kv_lens [batch] int32 (may be NULL: every
 *   row uses all seqlen_k keys, kernels/fa2.py:182-183; values are clamped to [0, seqlen_k]).
 *   q_strides/k_strides/v_strides/o_strides: 4 strides each; lse_strides: 3 (ignored if lse NULL).
 * seqlen_q == 1 runs the split-KV decode kernel, which needs the workspace; seqlen_q > 1 runs the
 * MFMA prefill kernel, which needs none.
 */
MI_FA2_API size_t mi_fa2_fwd_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                 int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim);
MI_FA2_API int mi_fa2_fwd(int32_t dtype, const void* q, const void* k, const void* v, void* o, float* lse,
               const int32_t* kv_lens, int32_t batch, int32_t heads_q, int32_t heads_kv,
               int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim,
               const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
               const int64_t* o_strides, const int64_t* lse_strides, int32_t is_causal,
               float sm_scale, void* workspace, size_t workspace_bytes, mi_fa2_stream_t stream);

/*
 * Padded forward over the rest of the launcher's envelope.  Replaces FlashAttention2Function.forward
 * (kernels/fa2.py:164-214) for the inputs mi_fa2_fwd does not take: head dims that are any powers of
 * two from 16 to 256 (kernels/fa2.py:185), with d_v (V and O) allowed to differ from d (Q and K),
 * and fp32 inputs, whose dots stay fp32 (input_precision="ieee", kernels/fa2.py:129,147).
 *   dtype: MI_FA2_BF16, MI_FA2_FP16 or MI_FA2_FP32 (q, k, v and o share it);
 *   q [batch, heads_q, seqlen_q, head_dim], k [batch, heads_kv, seqlen_k, head_dim],
 *   v [batch, heads_kv, seqlen_k, head_dim_v], o [batch, heads_q, seqlen_q, head_dim_v];
 *   everything else as in mi_fa2_fwd (kv_lens clamped to [0, seqlen_k], bottom-right causal mask,
 *   lse may be NULL).  batch and heads_q are at most 65535.  One kernel family (16x16 MFMAs, no
 *   workspace) serves every seqlen_q; bf16/fp16 at head_dim = head_dim_v = 128 is faster through
 *   mi_fa2_fwd, which this entry point does not dispatch to.
 */
MI_FA2_API int mi_fa2_fwd_general(int32_t dtype, const void* q, const void* k, const void* v, void* o,
                       float* lse, const int32_t* kv_lens, int32_t batch, int32_t heads_q,
                       int32_t heads_kv, int32_t seqlen_q, int32_t seqlen_k, int32_t head_dim,
                       int32_t head_dim_v, const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides,
                       const int64_t* lse_strides, int32_t is_causal, float sm_scale,
                       mi_fa2_stream_t stream);

/*
 * Packed variable-length forward.  The reference has no packed entry point: it pads a ragged
 * batch to the longest row and masks each row to its kv_lens (kv_cache.py:93-98,
 * kernels/fa2.py:107,133).  This entry point computes the same per-row attention without the
 * padding: row b owns query tokens [cu_seqlens_q[b], cu_seqlens_q[b+1]) of
 *   q [total_q, heads_q, 128] and key tokens [cu_seqlens_k[b], cu_seqlens_k[b+1]) of
 *   k/v [total_k, heads_kv, 128]; o like q; lse [heads_q, total_q] fp32 (may be NULL).
 *   *_strides: 2 strides each (token, head); lse_strides: 2 (head, token).
 * max_seqlen_q bounds every row's query count (it sizes the grid).
 */
MI_FA2_API int mi_fa2_fwd_varlen(int32_t dtype, const void* q, const void* k, const void* v, void* o,
                      float* lse, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                      int32_t batch, int32_t heads_q, int32_t heads_kv, int32_t max_seqlen_q,
                      int32_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      const int64_t* lse_strides, int32_t is_causal, float sm_scale,
                      mi_fa2_stream_t stream);

/*
 * Paged forward: attention whose K/V are read in-kernel from the paged KV cache.  Replaces
 * KVCache.read (kv_cache.py:117-121) + FlashAttention2Function.apply (model.py:97,103).
 *   k_pool/v_pool: one layer of KVCache.buf, i.e. buf[layer, 0] and buf[layer, 1], each
 *     [num_blocks * block_size, heads_kv, 128] (kv_cache.py:20-22); pool_strides: (slot, head)
 *     strides, shared by k_pool and v_pool.
 *   block_table [batch, >= ceil(kv_len/block_size)] int32, row stride block_table_stride:
 *     logical token p of row b lives in slot block_table[b][p / block_size] * block_size +
 *     p % block_size (kv_cache.py:15-16).  Entries past a row's kv_len are never read.  An entry
 *     outside [0, num_blocks) is a caller bug; as a guard it is never dereferenced and its keys
 *     read as zero vectors.
 *   kv_lens [batch] int32: keys held by each row, this step's included (model.py:175).
 *   max_kv_len: an upper bound of kv_lens (sizes the grid and the workspace).
 *   q/o [batch, heads_q, seqlen_q, 128] with 4 strides; lse [batch, heads_q, seqlen_q] (may be NULL).
 * block_size must be a multiple of 16.  seqlen_q == 1 is the decode regime (split-KV, uses the
 * workspace); seqlen_q > 1 is a prefill over cached context (bottom-right causal if is_causal).
 */
MI_FA2_API size_t mi_fa2_fwd_paged_workspace_size(int32_t batch, int32_t heads_q, int32_t heads_kv,
                                       int32_t seqlen_q, int32_t max_kv_len, int32_t head_dim);
MI_FA2_API int mi_fa2_fwd_paged(int32_t dtype, const void* q, const void* k_pool, const void* v_pool,
                     void* o, float* lse, const int32_t* block_table, int64_t block_table_stride,
                     const int32_t* kv_lens, int32_t batch, int32_t heads_q, int32_t heads_kv,
                     int32_t seqlen_q, int32_t max_kv_len, int32_t head_dim, int32_t block_size,
                     int32_t num_blocks, const int64_t* q_strides, const int64_t* pool_strides,
                     const int64_t* o_strides, const int64_t* lse_strides, int32_t is_causal,
                     float sm_scale, void* workspace, size_t workspace_bytes,
                     mi_fa2_stream_t stream);

/*
 * The paged forward without a workspace: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, hosts that forbid hipMalloc).  It has no
 * counterpart in the reference.  Same arguments, kernels and results as mi_fa2_fwd_paged, minus
 * workspace / workspace_bytes: the split-decode partials live in a scratch array of 32 MiB
 * (33,554,432 bytes) that the library holds on every GPU it runs on until the process ends
 * (e.g. 64 rows x 12 query heads at max_kv_len 8,192 use 25.6 MB).  A call that needs more
 * (mi_fa2_fwd_paged_workspace_size() above 32 MiB) returns MI_FA2_ERR_WORKSPACE without launching.
 * The caller still passes every input and output; nothing is allocated or freed, on the device or
 * the host.  All calls on one GPU share its scratch (its contents need no clearing: every slot
 * read is written by the same launch), so calls that overlap in time on one GPU, e.g. on two
 * streams, race: serialise them.
 */
MI_FA2_API int mi_fa2_fwd_paged_noalloc(int32_t dtype, const void* q, const void* k_pool,
                                        const void* v_pool, void* o, float* lse,
                                        const int32_t* block_table, int64_t block_table_stride,
                                        const int32_t* kv_lens, int32_t batch, int32_t heads_q,
                                        int32_t heads_kv, int32_t seqlen_q, int32_t max_kv_len,
                                        int32_t head_dim, int32_t block_size, int32_t num_blocks,
                                        const int64_t* q_strides, const int64_t* pool_strides,
                                        const int64_t* o_strides, const int64_t* lse_strides,
                                        int32_t is_causal, float sm_scale, mi_fa2_stream_t stream);

/*
 * Packed prefill over the paged cache: several rows, each with its own number of new query tokens,
 * attend to their cached keys in one launch.  The reference has no counterpart: its scheduler runs
 * one un-chunked prompt per forward (chat.py:247-253, model.py:157-199); this entry point lets a
 * scheduler pack the prompts admitted in one step (and the single tokens of rows that only decode)
 * into one batch.  Rows are as in mi_fa2_fwd_paged (block_table, kv_lens with this step's tokens
 * included, bottom-right causal per row), queries packed as in mi_fa2_fwd_varlen: row b owns query
 * tokens [cu_seqlens_q[b], cu_seqlens_q[b+1]) of q [total_q, heads_q, 128]; o like q;
 * lse [heads_q, total_q] (may be NULL).  q/o strides: 2 (token, head); lse_strides: 2 (head, token).
 * max_seqlen_q bounds every row's query count, max_kv_len every kv_len.  No workspace.
 */
MI_FA2_API int mi_fa2_fwd_paged_varlen(int32_t dtype, const void* q, const void* k_pool,
                                       const void* v_pool, void* o, float* lse,
                                       const int32_t* cu_seqlens_q, const int32_t* block_table,
                                       int64_t block_table_stride, const int32_t* kv_lens,
                                       int32_t batch, int32_t heads_q, int32_t heads_kv,
                                       int32_t max_seqlen_q, int32_t max_kv_len, int32_t head_dim,
                                       int32_t block_size, int32_t num_blocks,
                                       const int64_t* q_strides, const int64_t* pool_strides,
                                       const int64_t* o_strides, const int64_t* lse_strides,
                                       int32_t is_causal, float sm_scale, mi_fa2_stream_t stream);

/*
 * Merge of attention partials over disjoint key ranges.  The reference keeps no partials: its
 * kernel walks every key of a row in one program (kernels/fa2.py:122-158).  This is the split-KV
 * reduction of the decode path made callable on its own, for partials that other calls produced:
 * each partial i of (row r, head h) is what a forward over a sub-range of the row's keys returns,
 * its normalised output and its log-sum-exp (the O and L of kernels/fa2.py:155-158, L in natural
 * log), e.g. one per GPU when a long row's keys are spread over several GPUs.  Writes
 *   lse[r][h] = log sum_i exp(L_i),   o[r][h] = sum_i exp(L_i - lse[r][h]) O_i,
 * the output and L of one pass over all the keys.  A partial with L_i = -inf saw no key and is
 * skipped (its O_i is not read); a (row, head) with none left gets o = 0 and lse = -inf.
 *   part_o [max_parts, n_rows, heads, 128] fp32, part_o_strides: 3 (part, row, head), even;
 *   part_lse [max_parts, n_rows, heads] fp32, part_lse_strides: 3 (part, row, head);
 *   n_parts [n_rows] int32 partials used per row (the first n_parts[r]; clamped to
 *     [0, max_parts]), or NULL: max_parts each;
 *   o [n_rows, heads, 128] in out_dtype (MI_FA2_BF16, MI_FA2_FP16 or MI_FA2_FP32), o_strides: 2
 *     (row, head), even; lse [n_rows, heads] fp32 (may be NULL), lse_strides: 2.
 * n_rows <= 65535 (e.g. batch x query tokens flattened).  No workspace.  Asynchronous on `stream`.
 */
MI_FA2_API int mi_fa2_combine(int32_t out_dtype, const float* part_o, const float* part_lse,
                              const int32_t* n_parts, int32_t n_rows, int32_t heads,
                              int32_t max_parts, int32_t head_dim, const int64_t* part_o_strides,
                              const int64_t* part_lse_strides, void* o, const int64_t* o_strides,
                              float* lse, const int64_t* lse_strides, mi_fa2_stream_t stream);

/*
 * Fused rotary embedding + paged KV-cache write, the step before attention.  Replaces apply_rope
 * (model.py:62-65, applied at model.py:92) and KVCache.write (kv_cache.py:108-115, called at
 * model.py:96) on the GPU path, with bitwise the same results (the reference's 16-bit rounding
 * after each multiply and after the add):
 *   qkv [n_tokens, (heads_q + 2*heads_kv) * 128] with row stride qkv_row_stride: the fused q|k|v
 *     projection of every new token (q heads, then k heads, then v heads);
 *   cos, sin [n_tokens, 128] with row stride cs_row_stride: the model's RoPE tables for each
 *     token's position (model.py:151-155), in the same dtype;
 *   slot_mapping [n_tokens] int32: the cache slot of each token (kv_cache.py:15-16); a slot outside
 *     [0, num_slots) is skipped (a caller bug, guarded);
 *   q_out [n_tokens, heads_q * 128] with row stride q_row_stride: receives the rotated q;
 *   k_pool, v_pool: one layer of KVCache.buf (buf[layer, 0] and buf[layer, 1]), [num_slots,
 *     heads_kv, 128] with pool_strides (slot, head): receive the rotated k and the v.
 * Strides in elements, multiples of 8; pointers 16-byte aligned.  Asynchronous on `stream`.
 */
MI_FA2_API int mi_fa2_rope_kv_write(int32_t dtype, const void* qkv, int64_t qkv_row_stride,
                                    const void* cos, const void* sin, int64_t cs_row_stride,
                                    const int32_t* slot_mapping, int32_t n_tokens, int32_t heads_q,
                                    int32_t heads_kv, int32_t head_dim, void* q_out,
                                    int64_t q_row_stride, void* k_pool, void* v_pool,
                                    const int64_t* pool_strides, int32_t num_slots,
                                    mi_fa2_stream_t stream);

/*
 * Fused token sampler.  Replaces the reference's batched sampling (chat.py:103-107:
 * probs = softmax(logits.float() / temperature); torch.multinomial(probs, 1)) applied to the
 * last-position logits (model.py:204-207): draws one token per row of logits [batch, vocab]
 * (row stride `row_stride` elements, dtype bf16, fp16 or fp32) into tokens [batch] int32.
 *   temperature > 0: token = argmax_v(logit_v / temperature - ln E_v), E_v ~ Exp(1) -- the
 *     exponential race torch.multinomial uses for one sample, so the distribution is
 *     softmax(logits / temperature); E_v = -ln U_v with U_v from Philox4x32-10 keyed by `seed`,
 *     counter (v / 4, row, offset): advance `offset` by one per call for fresh draws.
 *   temperature <= 0: greedy argmax.
 * Ties go to the lowest index; NaN logits never win; a row with no candidate (all -inf or NaN)
 * gets -1 (torch.multinomial raises there).  batch <= 65535.  Needs the workspace that
 * mi_fa2_sample_workspace_size() returns (0 when vocab <= 8192).  Asynchronous on `stream`.
 */
MI_FA2_API size_t mi_fa2_sample_workspace_size(int32_t batch, int32_t vocab);
MI_FA2_API int mi_fa2_sample(int32_t dtype, const void* logits, int64_t row_stride, int32_t batch,
                             int32_t vocab, float temperature, uint64_t seed, uint64_t offset,
                             int32_t* tokens, void* workspace, size_t workspace_bytes,
                             mi_fa2_stream_t stream);

/*
 * Per-step paged-cache metadata from device-resident block tables.  Replaces the host side of
 * KVCache.prepare (kv_cache.py:74-101: a Python loop over every new token for slot_mapping, a
 * dense gather index, two host-to-device copies per step, consumed at model.py:168-175):
 *   tables [max_seqs, table_stride] int32: each sequence slot's block ids, kept on the device and
 *     written only when blocks are allocated; seq_lens [max_seqs] int32: tokens each slot holds,
 *     ADVANCED IN PLACE by this call (row b's slot grows by its token count);
 *   row_slots [batch] int32: the slot of each row (< 0: a padding row: no keys, slot -1 for its
 *     tokens, no advance); distinct rows must name distinct slots;
 *   cu [batch + 1] int32: row b's new tokens are [cu[b], cu[b+1]) of the packed batch, or NULL:
 *     every row has tokens_per_row tokens, row b's at b * tokens_per_row;
 * and writes starts [batch] (length before the step), kv_lens [batch] (= starts + count),
 * block_table [batch, width] (the first ceil(kv_len / block_size) entries of the slot's table,
 * then 0), slots [tokens] (cache slot of every new token, kv_cache.py:15-16), and optionally
 * positions [tokens] and last_idx [batch] (packed index of each row's last token).  A row whose
 * keys would not fit its table row is treated as padding.  All pointers are device pointers; one
 * launch, asynchronous on `stream`, safe to capture in a graph.
 */
MI_FA2_API int mi_fa2_step_metadata(const int32_t* row_slots, const int32_t* cu,
                                    int32_t tokens_per_row, int32_t batch, int32_t* seq_lens,
                                    int32_t max_seqs, const int32_t* tables, int64_t table_stride,
                                    int32_t block_size, int32_t width, int32_t* starts,
                                    int32_t* kv_lens, int32_t* block_table, int32_t* slots,
                                    int32_t* positions, int32_t* last_idx, mi_fa2_stream_t stream);

/*
 * Fused residual add + RMSNorm.  Replaces, on the GPU path, the reference's residual add
 * (model.py:128-138: x = x + attn / x = x + mlp) followed by the next RMSNorm (model.py:49-55: eight
 * torch ops), keeping their rounding points:
 *   r = round(x + y)                       (r = x when y is NULL), written to residual_out;
 *   out = round(weight * round(float(r) * rsqrt(mean(float(r)^2) + eps))).
 * x, y, residual_out, out [rows, hidden] with row strides (elements, multiples of 8, 16-byte
 * aligned bases); weight [hidden].  hidden: a multiple of 8, at most 8192.  residual_out may be x
 * itself (in place).  Asynchronous on `stream`.
 */
MI_FA2_API int mi_fa2_add_rmsnorm(int32_t dtype, const void* x, int64_t x_stride, const void* y,
                                  int64_t y_stride, const void* weight, void* residual_out,
                                  int64_t residual_stride, void* out, int64_t out_stride,
                                  int32_t rows, int32_t hidden, float eps, mi_fa2_stream_t stream);

/*
 * SwiGLU activation.  Replaces F.silu(gate) * up (model.py:112-120) on the fused gate|up
 * projection: gate_up [rows, 2 * inter] (gate columns first) -> out [rows, inter],
 * out = round(round(g / (1 + exp(-g))) * u).  inter: a multiple of 8.  Asynchronous on `stream`.
 */
MI_FA2_API int mi_fa2_silu_mul(int32_t dtype, const void* gate_up, int64_t gate_up_stride,
                               void* out, int64_t out_stride, int32_t rows, int32_t inter,
                               mi_fa2_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_FA2_H */
