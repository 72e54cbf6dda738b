/*
 * flexengine_amd.h -- C ABI of the MI355X (gfx950) paged-attention library
 * (libfe_paged.so).
 *
 * This is the drop-in boundary for FlexEngine's paged-attention hot path.
 * Every entry point takes plain device pointers, element counts and a HIP
 * stream; no PyTorch type crosses the boundary.  All buffers are owned by the
 * caller.  Every entry point is asynchronous on `stream`, performs no host
 * synchronisation and no device allocation, so it may be recorded into a HIP
 * graph.  Return value: 0 on success, a negative FE_ERR_* code for an argument
 * the library rejects before launching anything, or a positive hipError_t
 * returned by the launch.
 *
 * Tensor layouts (fp16 = IEEE binary16, row-major, contiguous unless a stride
 * argument says otherwise):
 *   KV pool of one layer   k_pool, v_pool : [num_blocks, block_size, kv_heads, head_dim]
 *       (the layout of PagedKVCache.k[layer] in
 *        src/flexengine/engine/kv_cache/allocator.py:30-32)
 *   block tables           int32 [batch, table_stride]; row b lists the
 *       physical blocks of sequence b in logical order.
 *   context lengths        int32 [batch]; tokens of sequence b that attention
 *       covers, INCLUDING the token being decoded.  0 marks an inactive row,
 *       whose output is exact zeros (paged_attention.py:131,138).
 *
 * Supported shapes: num_q_heads a multiple of kv_heads; block_size a power
 * of two.  head_dim 64 and 128 with a decode group (num_q_heads / kv_heads)
 * of at most 16 run on the matrix-core kernels, as does the prefill at any
 * group size; so do the fp16 / bf16 decode (group <= 16, no shared prefix) and
 * prefill at head_dim 256, unplanned, and an unplanned decode (no shared
 * prefix) whose group above 16 has a divisor from 8 to 16: it is split into
 * that many-headed virtual KV heads, each reading its pool head's K/V; an
 * unplanned fp16 / bf16 decode (no shared prefix, block_size a multiple of 16)
 * at any other head_dim that is a multiple of 8 below 256 runs on the
 * matrix-core decode padded to the next of 64 / 128 / 256 (the dims past
 * head_dim are zeros, never read from the pool nor written to the output;
 * its workspace is sized at the padded head_dim), and so does the 16-bit
 * prefill at any block size; fp32 runs padded on its own engine at 64 / 128
 * (any block size): the decode at multiples of 8 up to 64 and from 96 to 120,
 * the prefill at every multiple of 8 below 128.  Every other head_dim from 1 to 512, and decode groups of 17
 * to 128, run on a generic kernel (key splits of a row or tiles of prefill
 * tokens per workgroup, fp32 arithmetic) as long as group * head_dim <= 8192
 * (head_dim rounded up to a multiple of 8): same entry points, same results
 * to the same tolerances; the decode's key-split partials use the workspace
 * (fe_paged_decode_workspace_size covers them), the prefill none; no plan is
 * taken (the _planned calls return FE_ERR_UNSUPPORTED there), and a
 * shared-prefix decode at any shape but head_dim 64 / 128 with a group <= 16
 * attends each row over its own table (a plain decode, on whichever kernel
 * takes the shape).  The KV page movers need
 * head_dim % 8 == 0 (fp16 / bf16) or % 4 == 0 (fp32).
 * Element types: fp16 (the unsuffixed entry points), bfloat16 (_bf16) and
 * fp32 (_f32: the KV movers, the decode and the prefill).
 */
#ifndef FLEXENGINE_AMD_H
#define FLEXENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* fe_stream_t;

#define FE_OK 0
#define FE_ERR_INVALID_ARGUMENT (-1)  /* null pointer, bad size, misalignment */
#define FE_ERR_UNSUPPORTED (-2)       /* head_dim / group size / block size not built */
#define FE_ERR_WORKSPACE (-3)         /* workspace missing or smaller than required */
#define FE_ERR_SCRATCH_LIMIT (-4)     /* more scratch than fe_paged_decode_noalloc holds */

/* Bytes of the static per-GPU scratch array of fe_paged_decode_noalloc. */
#define FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES (16u << 20)

/*
 * A planned launch (fe_paged_decode_planned, fe_prefill_paged_planned and their
 * bf16 forms) checks its plan before using it and reports a mismatch in the
 * plan's error word: an int32 at these byte offsets of the plan buffer, zeroed
 * by the plan call, set by the planned launch (the planned calls therefore take
 * the plan as writable).  The launch itself has returned FE_OK: the check runs
 * on the device, so the caller reads the word after the stream's work is done.
 */
#define FE_DECODE_PLAN_ERROR_OFFSET 60
#define FE_PREFILL_PLAN_ERROR_OFFSET 124
#define FE_PLAN_ERR_SIZES 1  /* other sizes, block_tables / q_offsets / context_lens tensors */
#define FE_PLAN_ERR_STALE 2  /* the lengths changed since the plan was computed */

/* Library version (major*10000 + minor*100 + patch). */
int fe_version(void);

/* Human-readable text for any return code of this library. */
const char* fe_error_string(int code);

/*
 * KV page write ("reshape and cache"): for every new token t,
 *   k_pool[slot_block[t], slot_offset[t], h, :] = k_new[t, h, :]   (and v)
 * Rows whose slot_block is negative are skipped (inactive / padded rows).
 * Bit-exact byte copy.  k_new/v_new rows are `new_token_stride` elements
 * apart (>= kv_heads*head_dim), heads within a row are contiguous.
 * Replaces PagedKVCache._locators + PagedKVCache.write
 * (src/flexengine/engine/kv_cache/allocator.py:107-127): the caller passes the
 * (block, offset) pairs that _locators builds on the host.
 */
int fe_write_kv(const void* k_new, const void* v_new, int64_t new_token_stride,
                void* k_pool, void* v_pool, int num_blocks,
                const int32_t* slot_block, const int32_t* slot_offset,
                int num_tokens, int kv_heads, int head_dim, int block_size,
                fe_stream_t stream);

/*
 * Decode-step KV page write with device-side slot mapping: for each row b
 * with context_lens[b] = L > 0, writes k_new[b] / v_new[b] ([kv_heads,
 * head_dim], rows new_batch_stride elements apart) at logical position L-1,
 * i.e. block block_tables[b, (L-1)/bs], offset (L-1)%bs.  Rows with L == 0 are left untouched.
 * Replaces the graph-path write in decode_static
 * (src/flexengine/inference/models/qwen2.py:156-161), with inactive rows
 * skipped instead of rewritten.
 */
int fe_write_kv_decode(const void* k_new, const void* v_new, int64_t new_batch_stride,
                       void* k_pool, void* v_pool, int num_blocks,
                       const int32_t* block_tables, int table_stride,
                       const int32_t* context_lens, int batch,
                       int kv_heads, int head_dim, int block_size,
                       fe_stream_t stream);

/*
 * Ragged-chunk KV page write with device-side slot mapping: sequence s owns
 * new rows q_offsets[s] .. q_offsets[s+1]-1 of k_new / v_new ([total_tokens,
 * kv_heads, head_dim], rows new_token_stride elements apart), which are the
 * last n_s = q_offsets[s+1] - q_offsets[s] positions of its context of
 * context_lens[s] tokens; row i goes to position p = context_lens[s] - n_s +
 * (i - q_offsets[s]), block block_tables[s, p / block_size], offset
 * p % block_size (the same arrays fe_prefill_paged takes).  Rows whose page
 * or block id is out of range are skipped.  Bit-exact copy.
 * Replaces the per-request cache.write of the ragged forward
 * (src/flexengine/inference/models/qwen2.py:117-126) and its slot map
 * PagedKVCache._locators / write (src/flexengine/engine/kv_cache/allocator.py:
 * 107-127): no host-built slot list, no device-to-host synchronisation.
 */
int fe_write_kv_ragged(const void* k_new, const void* v_new, int64_t new_token_stride,
                       void* k_pool, void* v_pool, int num_blocks,
                       const int32_t* block_tables, int table_stride,
                       const int32_t* q_offsets, const int32_t* context_lens,
                       int num_seqs, int total_tokens, int kv_heads, int head_dim,
                       int block_size, fe_stream_t stream);

/*
 * Block tables of a batch built on the device from a device-resident mirror
 * of the allocator's tables: mirror is int32 [mirror_rows, mirror_stride]
 * with row r holding row_len[r] valid block ids; for b < batch and j < width,
 *   out[b, j] = mirror[rows[b], j]            if j < row_len[rows[b]],
 *             = pad_block                      otherwise (pad_block >= 0),
 *             = the row's last block (0 if empty)  otherwise (pad_block < 0);
 * rows[b] < 0 gives a row of padding.  out rows are out_stride apart.
 * Replaces the per-step host fill of the padded block tables
 * (src/flexengine/engine/runtime.py:205-213, _graph_inputs) and
 * PagedKVCache.block_table: a step copies `batch` row indices instead of
 * batch * width table entries.
 */
int fe_gather_tables(const int32_t* mirror, int mirror_stride, const int32_t* row_len,
                     int mirror_rows, const int32_t* rows, int batch, int width,
                     int pad_block, int32_t* out, int out_stride, fe_stream_t stream);

/*
 * Block-table gather ("materialize"): for every sequence b and position
 * t < context_lens[b],
 *   k_out[out_offsets[b] + t] = k_pool[block_tables[b, t/bs], t%bs]   (and v)
 * k_out/v_out are [total_tokens, kv_heads, head_dim]; out_offsets has batch+1
 * entries (exclusive prefix sum of context_lens; out_offsets[batch] =
 * total_tokens).  Bit-exact byte copy.
 * Replaces PagedKVCache.materialize (allocator.py:129-134), batched.
 */
int fe_gather_kv(const void* k_pool, const void* v_pool, int num_blocks,
                 const int32_t* block_tables, int table_stride,
                 const int32_t* context_lens, const int32_t* out_offsets,
                 void* k_out, void* v_out, int batch, int total_tokens,
                 int kv_heads, int head_dim, int block_size, fe_stream_t stream);

/*
 * fp32 forms of the four KV movers above: the same arguments and byte-exact
 * results for float32 pools and rows (strides in float32 elements; head_dim a
 * multiple of 4).  The reference's PagedKVCache defaults to float32
 * (src/flexengine/engine/kv_cache/allocator.py:26) and the engine builds the
 * cache in the model's dtype, float32 among them (engine/runtime.py:37-40,
 * inference/models/qwen2.py:54); its write and materialize
 * (allocator.py:116-134) move those rows.
 */
int fe_write_kv_f32(const void* k_new, const void* v_new, int64_t new_token_stride,
                    void* k_pool, void* v_pool, int num_blocks,
                    const int32_t* slot_block, const int32_t* slot_offset,
                    int num_tokens, int kv_heads, int head_dim, int block_size,
                    fe_stream_t stream);
int fe_write_kv_decode_f32(const void* k_new, const void* v_new, int64_t new_batch_stride,
                           void* k_pool, void* v_pool, int num_blocks,
                           const int32_t* block_tables, int table_stride,
                           const int32_t* context_lens, int batch,
                           int kv_heads, int head_dim, int block_size, fe_stream_t stream);
int fe_write_kv_ragged_f32(const void* k_new, const void* v_new, int64_t new_token_stride,
                           void* k_pool, void* v_pool, int num_blocks,
                           const int32_t* block_tables, int table_stride,
                           const int32_t* q_offsets, const int32_t* context_lens,
                           int num_seqs, int total_tokens, int kv_heads, int head_dim,
                           int block_size, fe_stream_t stream);
int fe_gather_kv_f32(const void* k_pool, const void* v_pool, int num_blocks,
                     const int32_t* block_tables, int table_stride,
                     const int32_t* context_lens, const int32_t* out_offsets,
                     void* k_out, void* v_out, int batch, int total_tokens,
                     int kv_heads, int head_dim, int block_size, fe_stream_t stream);

/*
 * Bytes of caller-owned workspace that fe_paged_decode needs for a given
 * batch / head configuration, table capacity (max_context = table_stride *
 * block_size) and split target (0 = library default).
 * It must be zero-filled before its first use; every call leaves it ready
 * for the next (the split counters it holds return to zero), so consecutive
 * calls on one stream may share it.  Calls that overlap in time (several
 * streams) need separate workspaces.
 */
size_t fe_paged_decode_workspace_size(int batch, int num_q_heads, int head_dim,
                                      int max_context, int target_splits);

/*
 * Fused single-token paged decode attention over one layer:
 *   out[b, hq, :] = softmax_t(scale * q[b,hq,:] . K[b,t,hq/G,:]) V[b,t,hq/G,:]
 * for t < context_lens[b], K/V rows fetched through block_tables; G =
 * num_q_heads / kv_heads.  Rows with context_lens[b] == 0 get exact zeros.
 * Work is split over the keys ("split-K") into about `target_splits` equal
 * pieces per KV head (0 = library default); partial results are combined by a
 * log-sum-exp merge inside the same kernel launch (the last piece of a
 * sequence to finish merges).  Tables may address at most 262144 tokens
 * (table_stride * block_size) and batch * kv_heads may not exceed 65536.
 * If k_new and v_new are non-null ([batch, kv_heads, head_dim], rows
 * new_batch_stride elements apart) the kernel
 * also performs the decode-step page write of fe_write_kv_decode and uses
 * those rows for position L-1, so one call is "write KV, then attend".
 * q and out are [batch, num_q_heads, head_dim]; q rows are q_batch_stride
 * elements apart.
 * Replaces triton_paged_decode_batch / _paged_decode_batch_kernel
 * (src/flexengine/inference/kernels/paged_attention.py:99-155) and the batched
 * backend signature shared with flashinfer_paged_decode_batch
 * (src/flexengine/inference/attention/flashinfer_backend.py:33-72); the
 * reference's positions/active_mask pair maps to context_lens =
 * (positions + 1) * active.
 */
int fe_paged_decode(const void* q, int64_t q_batch_stride, void* out,
                    const void* k_new, const void* v_new, int64_t new_batch_stride,
                    void* k_pool, void* v_pool, int num_blocks,
                    const int32_t* block_tables, int table_stride,
                    const int32_t* context_lens,
                    void* workspace, size_t workspace_bytes,
                    int batch, int num_q_heads, int kv_heads, int head_dim,
                    int block_size, float scale, int target_splits,
                    fe_stream_t stream);

/*
 * Decode plan of one step, shared by every layer's fe_paged_decode_planned:
 * the split-K partition of the sequences (from context_lens) and each
 * workgroup's block rows (from block_tables), which fe_paged_decode otherwise
 * derives at the start of every launch.  A model's decode step computes it
 * once and its 28 layers reuse it, since tables and lengths do not change
 * between layers.  No counterpart in the reference: its decode
 * (src/flexengine/inference/kernels/paged_attention.py:99-155) has no split-K
 * partition to plan.  Block sizes must be multiples of 16.
 * fe_paged_decode_plan_size: bytes of the plan for these sizes (the same
 * table capacity max_context = table_stride * block_size and target_splits
 * as the decode calls).
 */
size_t fe_paged_decode_plan_size(int batch, int kv_heads, int max_context, int target_splits);
int fe_paged_decode_plan(const int32_t* block_tables, int table_stride,
                         const int32_t* context_lens, int num_blocks, int batch, int kv_heads,
                         int block_size, int target_splits, void* plan, size_t plan_bytes,
                         fe_stream_t stream);

/*
 * fe_paged_decode with the partition and first block rows read from `plan`
 * (written by fe_paged_decode_plan on the same block_tables, table_stride,
 * context_lens, num_blocks, batch, kv_heads, block_size and target_splits,
 * earlier on the stream): same results, one dependent load fewer before the
 * first K/V loads.  A plan_bytes below fe_paged_decode_plan_size returns
 * FE_ERR_WORKSPACE.  A plan recorded for other sizes or other block_tables /
 * context_lens addresses is not used: every output row is NaN and the error
 * word is FE_PLAN_ERR_SIZES.  A row whose live context length is not the
 * plan's (lengths changed after the plan call) writes nothing to the pools and
 * gives NaN, and the error word is FE_PLAN_ERR_STALE; other rows are exact.
 * Block-table contents are not checked: the plan's block rows are used.
 */
int fe_paged_decode_planned(const void* q, int64_t q_batch_stride, void* out,
                            const void* k_new, const void* v_new, int64_t new_batch_stride,
                            void* k_pool, void* v_pool, int num_blocks,
                            const int32_t* block_tables, int table_stride,
                            const int32_t* context_lens,
                            void* workspace, size_t workspace_bytes,
                            int batch, int num_q_heads, int kv_heads, int head_dim,
                            int block_size, float scale, int target_splits,
                            void* plan, size_t plan_bytes, fe_stream_t stream);

/*
 * bf16 forms of fe_paged_decode and fe_paged_decode_planned: the same
 * arguments and results with q, out, k_new, v_new and the pools in bfloat16
 * (products on v_mfma_f32_16x16x16_bf16, probabilities rounded to bf16 for
 * the PV product, fp32 accumulation and merge).  Replace the same reference
 * routes for the bfloat16 models and caches the reference builds
 * (src/flexengine/inference/models/qwen2.py:54, engine/kv_cache/allocator.py:24);
 * the plan and the workspace are the fp16 forms' (dtype-free).
 */
int fe_paged_decode_bf16(const void* q, int64_t q_batch_stride, void* out,
                         const void* k_new, const void* v_new, int64_t new_batch_stride,
                         void* k_pool, void* v_pool, int num_blocks,
                         const int32_t* block_tables, int table_stride,
                         const int32_t* context_lens,
                         void* workspace, size_t workspace_bytes,
                         int batch, int num_q_heads, int kv_heads, int head_dim,
                         int block_size, float scale, int target_splits,
                         fe_stream_t stream);
int fe_paged_decode_planned_bf16(const void* q, int64_t q_batch_stride, void* out,
                                 const void* k_new, const void* v_new, int64_t new_batch_stride,
                                 void* k_pool, void* v_pool, int num_blocks,
                                 const int32_t* block_tables, int table_stride,
                                 const int32_t* context_lens,
                                 void* workspace, size_t workspace_bytes,
                                 int batch, int num_q_heads, int kv_heads, int head_dim,
                                 int block_size, float scale, int target_splits,
                                 void* plan, size_t plan_bytes, fe_stream_t stream);

/*
 * fp32 form of fe_paged_decode: the same arguments (strides in float32
 * elements) and workspace, with q, out, k_new, v_new and the pools in float32,
 * any power-of-two block size; fp32 products on v_mfma_f32_16x16x4_f32, fp32
 * probabilities, softmax and merge -- no rounding below fp32.  Replaces the
 * reference's Triton decode for the float32 caches it serves
 * (src/flexengine/inference/kernels/paged_attention.py:99-155, which loads K,
 * V and q as float32 at :116,126,134).  No plan and no shared-prefix form.
 */
int fe_paged_decode_f32(const void* q, int64_t q_batch_stride, void* out,
                        const void* k_new, const void* v_new, int64_t new_batch_stride,
                        void* k_pool, void* v_pool, int num_blocks,
                        const int32_t* block_tables, int table_stride,
                        const int32_t* context_lens,
                        void* workspace, size_t workspace_bytes,
                        int batch, int num_q_heads, int kv_heads, int head_dim,
                        int block_size, float scale, int target_splits,
                        fe_stream_t stream);

/*
 * fe_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference.
 * Same arguments (minus workspace / workspace_bytes), kernels and results as
 * fe_paged_decode; the split-K tickets and partials live in a static device
 * array of FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES (16 MiB) that each GPU the
 * library runs on holds until the process ends.  The call allocates nothing
 * (no hipMalloc / hipFree); the first call on a device looks up that
 * device's array and clears its split counters with a kernel on `stream`.
 * A call needing more scratch than the array holds -- what
 * fe_paged_decode_workspace_size reports for the same arguments -- returns
 * FE_ERR_SCRATCH_LIMIT before launching anything (C2-sized batches need
 * about 4 MiB).  Every call on one GPU shares that GPU's array and leaves the
 * last call's partials in it: calls that overlap in time on one GPU (several
 * streams, or host threads without ordering) race and must not be issued.
 * The current device must be the device of `stream` and of the pointers.
 */
int fe_paged_decode_noalloc(const void* q, int64_t q_batch_stride, void* out,
                            const void* k_new, const void* v_new, int64_t new_batch_stride,
                            void* k_pool, void* v_pool, int num_blocks,
                            const int32_t* block_tables, int table_stride,
                            const int32_t* context_lens,
                            int batch, int num_q_heads, int kv_heads, int head_dim,
                            int block_size, float scale, int target_splits,
                            fe_stream_t stream);

/*
 * Bytes of device workspace fe_paged_decode_shared_prefix needs; zero-filled
 * before first use, reusable like fe_paged_decode's.
 */
size_t fe_paged_decode_shared_prefix_workspace_size(int batch, int num_q_heads, int kv_heads,
                                                    int head_dim, int max_context,
                                                    int num_groups, int target_splits);

/*
 * fe_paged_decode for a batch in which groups of sequences share a prefix
 * of KV blocks (FlexEngine's prefix cache attaches the same physical blocks
 * to every request that reuses a prompt: PrefixCache.insert / attach_prefix,
 * src/flexengine/engine/kv_cache/prefix.py:75-96,
 * src/flexengine/engine/kv_cache/allocator.py:83-94).  Same result as
 * fe_paged_decode on the same arguments, computed in cascade:
 *   group s = sequences group_offsets[s] .. group_offsets[s+1]-1 (device
 *   arrays; ascending offsets, groups contiguous in the batch), whose first
 *   P_s = group_prefix_lens[s] keys (rounded down to whole blocks) are the
 *   blocks of row group_offsets[s]'s table.  The shared keys are attended
 *   once per group, all members' query heads together (a matrix-core
 *   product, K/V read once per group instead of once per sequence); each
 *   sequence's own decode covers only keys P_s .. L-1 and merges the two by
 *   their log-sum-exp.  A member whose context does not reach past P_s is
 *   decoded without sharing.  Sequences outside every group are decoded as
 *   by fe_paged_decode.  The caller guarantees that members' tables really
 *   hold the group's blocks in their first P_s / block_size entries, and a
 *   decode-step write (k_new) must not target a shared block (the reference
 *   refuses such writes, allocator.py:124-125).  Block size a multiple of 16.
 */
int fe_paged_decode_shared_prefix(const void* q, int64_t q_batch_stride, void* out,
                                  const void* k_new, const void* v_new, int64_t new_batch_stride,
                                  void* k_pool, void* v_pool, int num_blocks,
                                  const int32_t* block_tables, int table_stride,
                                  const int32_t* context_lens,
                                  const int32_t* group_offsets, const int32_t* group_prefix_lens,
                                  int num_groups,
                                  void* workspace, size_t workspace_bytes,
                                  int batch, int num_q_heads, int kv_heads, int head_dim,
                                  int block_size, float scale, int target_splits,
                                  fe_stream_t stream);

/*
 * bf16 form of fe_paged_decode_shared_prefix: the same arguments, workspace
 * and results with q, out, the pools and the new rows in bfloat16 (the
 * prefix pass and the suffix decode on the bf16 matrix-core products,
 * probabilities rounded to bf16, fp32 merge).  Replaces the same route for the
 * bfloat16 models the reference builds (qwen2.py:54).
 */
int fe_paged_decode_shared_prefix_bf16(const void* q, int64_t q_batch_stride, void* out,
                                       const void* k_new, const void* v_new,
                                       int64_t new_batch_stride, void* k_pool, void* v_pool,
                                       int num_blocks, const int32_t* block_tables,
                                       int table_stride, const int32_t* context_lens,
                                       const int32_t* group_offsets,
                                       const int32_t* group_prefix_lens, int num_groups,
                                       void* workspace, size_t workspace_bytes,
                                       int batch, int num_q_heads, int kv_heads, int head_dim,
                                       int block_size, float scale, int target_splits,
                                       fe_stream_t stream);

/*
 * fp32 form of fe_paged_decode_shared_prefix: the same arguments, workspace
 * and results with q, out, the pools and the new rows in float32 (the prefix
 * pass on the fp32 matrix-core engine of fe_prefill_paged_f32, the suffix
 * decode on fe_paged_decode_f32's, fp32 softmax and merge).  Replaces the same
 * route for the float32 caches the reference allocates by default
 * (allocator.py:26; runtime.py:37-40 builds the cache in the model's dtype).
 */
int fe_paged_decode_shared_prefix_f32(const void* q, int64_t q_batch_stride, void* out,
                                      const void* k_new, const void* v_new,
                                      int64_t new_batch_stride, void* k_pool, void* v_pool,
                                      int num_blocks, const int32_t* block_tables,
                                      int table_stride, const int32_t* context_lens,
                                      const int32_t* group_offsets,
                                      const int32_t* group_prefix_lens, int num_groups,
                                      void* workspace, size_t workspace_bytes,
                                      int batch, int num_q_heads, int kv_heads, int head_dim,
                                      int block_size, float scale, int target_splits,
                                      fe_stream_t stream);

/*
 * Log-sum-exp merge of split attention results:
 *   LSE[r]   = log(sum_s exp(part_lse[s, r]))
 *   out[r,:] = sum_s exp(part_lse[s, r] - LSE[r]) * part_out[s, r, :]
 * part_out fp32 [num_splits, rows, head_dim] (each normalised by its own
 * softmax denominator), part_lse fp32 [num_splits, rows] (natural log),
 * out fp16 [rows, head_dim]; out_lse (fp32 [rows], nullable) receives LSE.
 * A split whose lse is -inf contributes nothing; a row whose every split is
 * -inf gets zeros.  This is the combine step of split-K decode; the
 * reference has no split-K, its single-pass online softmax
 * (src/flexengine/inference/attention/paged.py:50-70) is the quantity the
 * merge reproduces.
 */
int fe_lse_merge(const float* part_out, const float* part_lse, int num_splits,
                 int rows, int head_dim, void* out, float* out_lse,
                 fe_stream_t stream);

/* bf16 form of fe_lse_merge: the same arguments, out bfloat16 [rows, head_dim]
 * (rounded to nearest even) for the bfloat16 models of qwen2.py:54. */
int fe_lse_merge_bf16(const float* part_out, const float* part_lse, int num_splits,
                      int rows, int head_dim, void* out, float* out_lse, fe_stream_t stream);

/*
 * Ragged chunked-prefill attention over paged KV (causal), fp16 MFMA:
 * sequence s owns query rows [q_offsets[s], q_offsets[s+1]) of q/out
 * ([total_q, num_q_heads, head_dim]); its context length is
 * context_lens[s] (cached tokens + its new tokens, whose K/V must already be
 * in the pool).  Query row j of sequence s sits at absolute position
 * context_lens[s] - n_s + j and attends to keys t <= that position.
 * Replaces the per-request materialized route that the reference takes for
 * every multi-token chunk (src/flexengine/inference/attention/paged.py:27-40,
 * called per request from qwen2.py:117-126).
 */
int fe_prefill_paged(const void* q, void* out,
                     const void* k_pool, const void* v_pool, int num_blocks,
                     const int32_t* block_tables, int table_stride,
                     const int32_t* q_offsets, const int32_t* context_lens,
                     int num_seqs, int total_q, int max_q_len,
                     int num_q_heads, int kv_heads, int head_dim,
                     int block_size, float scale,
                     void* workspace, size_t workspace_bytes, fe_stream_t stream);

/*
 * bf16 form of fe_prefill_paged: the same arguments, block sizes and results
 * with q, out and the pools in bfloat16 (v_mfma_f32_16x16x32_bf16,
 * probabilities rounded to bf16 for the PV product, fp32 accumulation and row
 * sums of the rounded probabilities); the workspace is
 * fe_prefill_workspace_size's.  Replaces the same per-request route for the
 * bfloat16 models the reference builds (qwen2.py:54).
 */
int fe_prefill_paged_bf16(const void* q, void* out,
                          const void* k_pool, const void* v_pool, int num_blocks,
                          const int32_t* block_tables, int table_stride,
                          const int32_t* q_offsets, const int32_t* context_lens,
                          int num_seqs, int total_q, int max_q_len,
                          int num_q_heads, int kv_heads, int head_dim,
                          int block_size, float scale,
                          void* workspace, size_t workspace_bytes, fe_stream_t stream);

/*
 * fp32 form of fe_prefill_paged: the same arguments and results with q, out
 * and the pools in float32, any power-of-two block size; fp32 products on
 * v_mfma_f32_16x16x4_f32 and an fp32 softmax, one wave per 16 (token, query
 * head) rows over its whole causal key range (no key splits).  The workspace
 * arguments are accepted and unused (null is allowed).  Replaces the
 * reference's per-request prefill route on a float32 cache
 * (src/flexengine/inference/attention/paged.py:27-36: materialize, then
 * scaled_dot_product_attention in the cache's dtype).
 */
int fe_prefill_paged_f32(const void* q, void* out,
                         const void* k_pool, const void* v_pool, int num_blocks,
                         const int32_t* block_tables, int table_stride,
                         const int32_t* q_offsets, const int32_t* context_lens,
                         int num_seqs, int total_q, int max_q_len,
                         int num_q_heads, int kv_heads, int head_dim,
                         int block_size, float scale,
                         void* workspace, size_t workspace_bytes, fe_stream_t stream);

/*
 * Prefill plan of one model step: the stream-K work split of fe_prefill_paged
 * -- every workgroup's range of key blocks and its first unit -- depends only
 * on q_offsets, context_lens and the sizes, which all layers of a step share.
 * fe_prefill_plan computes it once into a caller-owned device buffer of
 * fe_prefill_plan_size(...) bytes (16-byte aligned); fe_prefill_paged_planned
 * (and its bf16 form) is fe_prefill_paged reading the split from it, with the
 * same results.  The plan must come from the same q_offsets, context_lens,
 * table_stride, block_size and head counts, and be complete (stream order)
 * before the planned calls.  A planned launch compares the plan's record of
 * the sizes, of the q_offsets / context_lens addresses and of a digest of
 * their contents with its own; on a mismatch every output row is NaN and the
 * error word is FE_PLAN_ERR_SIZES (sizes, addresses) or FE_PLAN_ERR_STALE
 * (contents).  Sizes the stream-K kernel does not take (block
 * sizes not a multiple of 16, or beyond its 32-bit work split) return
 * FE_ERR_UNSUPPORTED from fe_prefill_plan; such steps call fe_prefill_paged.
 * No counterpart in the reference: its prefill has no work split to plan; one
 * plan serves the 28 per-layer calls of qwen2.py:117-126's ragged forward.
 */
size_t fe_prefill_plan_size(int num_seqs, int total_q, int num_q_heads, int kv_heads);
int fe_prefill_plan(const int32_t* q_offsets, const int32_t* context_lens, int num_seqs,
                    int total_q, int num_q_heads, int kv_heads, int table_stride,
                    int block_size, void* plan, size_t plan_bytes, fe_stream_t stream);
int fe_prefill_paged_planned(const void* q, void* out,
                             const void* k_pool, const void* v_pool, int num_blocks,
                             const int32_t* block_tables, int table_stride,
                             const int32_t* q_offsets, const int32_t* context_lens,
                             int num_seqs, int total_q, int max_q_len,
                             int num_q_heads, int kv_heads, int head_dim,
                             int block_size, float scale,
                             void* workspace, size_t workspace_bytes,
                             void* plan, size_t plan_bytes, fe_stream_t stream);
int fe_prefill_paged_planned_bf16(const void* q, void* out,
                                  const void* k_pool, const void* v_pool, int num_blocks,
                                  const int32_t* block_tables, int table_stride,
                                  const int32_t* q_offsets, const int32_t* context_lens,
                                  int num_seqs, int total_q, int max_q_len,
                                  int num_q_heads, int kv_heads, int head_dim,
                                  int block_size, float scale,
                                  void* workspace, size_t workspace_bytes,
                                  void* plan, size_t plan_bytes, fe_stream_t stream);

/*
 * Bytes of device workspace fe_prefill_paged needs for these sizes (its key
 * splits keep fp32 partial outputs there).  Like the decode workspace it must
 * be zero-filled before its first use; every call leaves its ticket region
 * zero again, so one allocation serves every later call on the stream.
 */
size_t fe_prefill_workspace_size(int num_seqs, int total_q, int num_q_heads, int kv_heads,
                                 int head_dim);

#ifdef __cplusplus
}
#endif

#endif /* FLEXENGINE_AMD_H */
