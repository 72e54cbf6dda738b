// KV page write ("reshape and cache") and block-table gather for gfx950.
//
// Both are pure byte movement: each thread moves one 16-byte chunk (8 fp16
// elements) of one (token, kv-head) row, so a 256-byte row (head_dim 128) is
// one fully coalesced 256-byte segment per 16 lanes.  Bound: HBM bandwidth.
#include "fe_common.h"

using namespace fe;

namespace {

__device__ __forceinline__ int clamp_block(int blk, int nb) {
  return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
}

// Scatter of new rows to explicit (block, offset) slots
// (PagedKVCache.write, src/flexengine/engine/kv_cache/allocator.py:116-127).
__global__ __launch_bounds__(256) void write_kv_slots_kernel(
    const f16* __restrict__ k_new, const f16* __restrict__ v_new, int64_t src_stride,
    f16* __restrict__ k_pool, f16* __restrict__ v_pool, int nb,
    const int32_t* __restrict__ slot_block, const int32_t* __restrict__ slot_off,
    int T, int Hkv, int D, int BS) {
  const int chunks_per_tok = Hkv * (D >> 3);
  const int64_t total = (int64_t)T * chunks_per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(i / chunks_per_tok);
    const int r = (int)(i - (int64_t)t * chunks_per_tok);  // = h*(D/8) + c
    const int blk = slot_block[t];
    const int off = slot_off[t];
    if (blk < 0 || blk >= nb || off < 0 || off >= BS) continue;
    const int64_t dst = ((int64_t)blk * BS + off) * Hkv * D + (int64_t)r * 8;
    const int64_t src = (int64_t)t * src_stride + (int64_t)r * 8;
    st16(k_pool + dst, ld16(k_new + src));
    st16(v_pool + dst, ld16(v_new + src));
  }
}

// Decode-step write at position L-1 of every active row
// (decode_static, src/flexengine/inference/models/qwen2.py:156-161).
__global__ __launch_bounds__(256) void write_kv_decode_kernel(
    const f16* __restrict__ k_new, const f16* __restrict__ v_new, int64_t src_stride,
    f16* __restrict__ k_pool, f16* __restrict__ v_pool, int nb,
    const int32_t* __restrict__ tables, int W, const int32_t* __restrict__ ctx,
    int B, int Hkv, int D, int BS, int bs_log2) {
  const int chunks_per_tok = Hkv * (D >> 3);
  const int total = B * chunks_per_tok;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const int b = i / chunks_per_tok;
    const int r = i - b * chunks_per_tok;
    const int L = ctx[b];
    if (L <= 0) continue;
    const int pos = L - 1;
    int page = pos >> bs_log2;
    page = page < W ? page : W - 1;
    const int blk = clamp_block(tables[(int64_t)b * W + page], nb);
    const int64_t dst = ((int64_t)blk * BS + (pos & (BS - 1))) * Hkv * D + (int64_t)r * 8;
    const int64_t src = (int64_t)b * src_stride + (int64_t)r * 8;
    st16(k_pool + dst, ld16(k_new + src));
    st16(v_pool + dst, ld16(v_new + src));
  }
}

// Ragged-chunk write with device-side slot mapping (the per-request write of
// the ragged forward, src/flexengine/inference/models/qwen2.py:117-126, with
// PagedKVCache._locators, allocator.py:107-114, computed here): token i of
// sequence s (q_off[s] <= i < q_off[s+1], n_s tokens) is the sequence's
// position ctx[s] - n_s + (i - q_off[s]) -- the new rows are the last n_s of
// its context -- in block tables[s][pos / BS], offset pos % BS.  Tokens whose
// position or block falls outside the table or the pool are skipped.
__global__ __launch_bounds__(256) void write_kv_ragged_kernel(
    const f16* __restrict__ k_new, const f16* __restrict__ v_new, int64_t src_stride,
    f16* __restrict__ k_pool, f16* __restrict__ v_pool, int nb,
    const int32_t* __restrict__ tables, int W, const int32_t* __restrict__ q_off,
    const int32_t* __restrict__ ctx, int S, int T, int Hkv, int D, int BS, int bs_log2) {
  const int chunks_per_tok = Hkv * (D >> 3);
  const int64_t total = (int64_t)T * chunks_per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int tok = (int)(i / chunks_per_tok);
    const int r = (int)(i - (int64_t)tok * chunks_per_tok);
    // sequence of token `tok`: last s with q_off[s] <= tok
    int lo = 0, hi = S - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (q_off[mid] <= tok) lo = mid; else hi = mid - 1;
    }
    const int s = lo;
    const int first = q_off[s], end = q_off[s + 1];
    if (tok < first || tok >= end) continue;
    const int pos = ctx[s] - (end - first) + (tok - first);
    if (pos < 0) continue;
    const int page = pos >> bs_log2;
    if (page >= W) continue;
    const int blk = tables[(int64_t)s * W + page];
    if (blk < 0 || blk >= nb) continue;
    const int64_t dst = ((int64_t)blk * BS + (pos & (BS - 1))) * Hkv * D + (int64_t)r * 8;
    const int64_t src = (int64_t)tok * src_stride + (int64_t)r * 8;
    st16(k_pool + dst, ld16(k_new + src));
    st16(v_pool + dst, ld16(v_new + src));
  }
}

// Block tables of a batch gathered from a device-resident table mirror
// (PagedKVCache.block_table, allocator.py / runtime.py:205-213, where the
// engine fills every row on the host each step): out[b][j] = mirror[rows[b]][j]
// for j < len[rows[b]]; past it (and for rows[b] < 0) pad_block, or the row's
// last block when pad_block < 0 (0 for an empty row).
__global__ __launch_bounds__(256) void gather_tables_kernel(
    const int32_t* __restrict__ mirror, int mstride, const int32_t* __restrict__ row_len,
    int nrows, const int32_t* __restrict__ rows, int B, int W, int pad_block,
    int32_t* __restrict__ out, int ostride) {
  const int64_t total = (int64_t)B * W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int b = (int)(i / W);
    const int j = (int)(i - (int64_t)b * W);
    const int row = rows[b];
    const bool ok = row >= 0 && row < nrows;
    int len = ok ? row_len[row] : 0;
    len = len < mstride ? len : mstride;
    int v;
    if (j < len) v = mirror[(int64_t)row * mstride + j];
    else if (pad_block >= 0) v = pad_block;
    else v = len > 0 ? mirror[(int64_t)row * mstride + len - 1] : 0;
    out[(int64_t)b * ostride + j] = v;
  }
}

// Batched block-table gather (PagedKVCache.materialize, allocator.py:129-134).
__global__ __launch_bounds__(256) void gather_kv_kernel(
    const f16* __restrict__ k_pool, const f16* __restrict__ v_pool, int nb,
    const int32_t* __restrict__ tables, int W, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ out_off, f16* __restrict__ k_out, f16* __restrict__ v_out,
    int B, int total_tokens, int Hkv, int D, int BS, int bs_log2) {
  const int chunks_per_tok = Hkv * (D >> 3);
  const int64_t total = (int64_t)total_tokens * chunks_per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int tok = (int)(i / chunks_per_tok);
    const int r = (int)(i - (int64_t)tok * chunks_per_tok);
    // sequence owning output row `tok`: last b with out_off[b] <= tok
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (out_off[mid] <= tok) lo = mid; else hi = mid - 1;
    }
    const int b = lo;
    const int t = tok - out_off[b];
    if (t < 0 || t >= ctx[b]) continue;
    int page = t >> bs_log2;
    page = page < W ? page : W - 1;
    const int blk = clamp_block(tables[(int64_t)b * W + page], nb);
    const int64_t src = ((int64_t)blk * BS + (t & (BS - 1))) * Hkv * D + (int64_t)r * 8;
    const int64_t dst = (int64_t)tok * chunks_per_tok * 8 + (int64_t)r * 8;
    st16(k_out + dst, ld16(k_pool + src));
    st16(v_out + dst, ld16(v_pool + src));
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}
inline int grid_for(int64_t work, int threads) {
  int64_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (int)g;
}

}  // namespace

extern "C" int fe_write_kv(const void* k_new, const void* v_new, int64_t new_token_stride,
                           void* k_pool, void* v_pool, int num_blocks,
                           const int32_t* slot_block, const int32_t* slot_offset,
                           int num_tokens, int kv_heads, int head_dim, int block_size,
                           fe_stream_t stream) {
  FE_CHECK_ARG(num_tokens >= 0 && kv_heads > 0 && head_dim > 0 && block_size > 0 && num_blocks > 0);
  FE_CHECK_ARG(head_dim % 8 == 0 && new_token_stride % 8 == 0 &&
               new_token_stride >= (int64_t)kv_heads * head_dim);
  if (num_tokens == 0) return FE_OK;
  FE_CHECK_ARG(k_new && v_new && k_pool && v_pool && slot_block && slot_offset);
  FE_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool));
  const int64_t work = (int64_t)num_tokens * kv_heads * (head_dim / 8);
  hipLaunchKernelGGL(write_kv_slots_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)k_new, (const f16*)v_new, new_token_stride,
                     (f16*)k_pool, (f16*)v_pool, num_blocks, slot_block, slot_offset, num_tokens,
                     kv_heads, head_dim, block_size);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_write_kv_decode(const void* k_new, const void* v_new,
                                  int64_t new_batch_stride, void* k_pool, void* v_pool,
                                  int num_blocks, const int32_t* block_tables,
                                  int table_stride, const int32_t* context_lens, int batch,
                                  int kv_heads, int head_dim, int block_size, fe_stream_t stream) {
  FE_CHECK_ARG(batch >= 0 && kv_heads > 0 && head_dim > 0 && num_blocks > 0 && table_stride > 0);
  FE_CHECK_ARG(head_dim % 8 == 0 && new_batch_stride % 8 == 0 &&
               new_batch_stride >= (int64_t)kv_heads * head_dim);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  if (batch == 0) return FE_OK;
  FE_CHECK_ARG(k_new && v_new && k_pool && v_pool && block_tables && context_lens);
  FE_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool));
  const int64_t work = (int64_t)batch * kv_heads * (head_dim / 8);
  hipLaunchKernelGGL(write_kv_decode_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)k_new, (const f16*)v_new, new_batch_stride,
                     (f16*)k_pool, (f16*)v_pool, num_blocks, block_tables, table_stride,
                     context_lens, batch,
                     kv_heads, head_dim, block_size, bs_log2);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_write_kv_ragged(const void* k_new, const void* v_new, int64_t new_token_stride,
                                  void* k_pool, void* v_pool, int num_blocks,
                                  const int32_t* block_tables, int table_stride,
                                  const int32_t* q_offsets, const int32_t* context_lens,
                                  int num_seqs, int total_tokens, int kv_heads, int head_dim,
                                  int block_size, fe_stream_t stream) {
  FE_CHECK_ARG(num_seqs >= 0 && total_tokens >= 0 && kv_heads > 0 && head_dim > 0 &&
               num_blocks > 0 && table_stride > 0);
  FE_CHECK_ARG(head_dim % 8 == 0 && new_token_stride % 8 == 0 &&
               new_token_stride >= (int64_t)kv_heads * head_dim);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  if (num_seqs == 0 || total_tokens == 0) return FE_OK;
  FE_CHECK_ARG(k_new && v_new && k_pool && v_pool && block_tables && q_offsets && context_lens);
  FE_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool));
  const int64_t work = (int64_t)total_tokens * kv_heads * (head_dim / 8);
  hipLaunchKernelGGL(write_kv_ragged_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)k_new, (const f16*)v_new, new_token_stride,
                     (f16*)k_pool, (f16*)v_pool, num_blocks, block_tables, table_stride,
                     q_offsets, context_lens, num_seqs, total_tokens, kv_heads, head_dim,
                     block_size, bs_log2);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_gather_tables(const int32_t* mirror, int mirror_stride, const int32_t* row_len,
                                int mirror_rows, const int32_t* rows, int batch, int width,
                                int pad_block, int32_t* out, int out_stride, fe_stream_t stream) {
  FE_CHECK_ARG(mirror_stride > 0 && mirror_rows >= 0 && batch >= 0 && width > 0 &&
               out_stride >= width);
  if (batch == 0) return FE_OK;
  FE_CHECK_ARG(mirror && row_len && rows && out);
  const int64_t work = (int64_t)batch * width;
  hipLaunchKernelGGL(gather_tables_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, mirror, mirror_stride, row_len, mirror_rows, rows, batch,
                     width, pad_block, out, out_stride);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_gather_kv(const void* k_pool, const void* v_pool, int num_blocks,
                            const int32_t* block_tables, int table_stride,
                            const int32_t* context_lens, const int32_t* out_offsets, void* k_out,
                            void* v_out, int batch, int total_tokens, int kv_heads, int head_dim,
                            int block_size, fe_stream_t stream) {
  FE_CHECK_ARG(batch >= 0 && total_tokens >= 0 && kv_heads > 0 && head_dim > 0 &&
               num_blocks > 0 && table_stride > 0);
  FE_CHECK_ARG(head_dim % 8 == 0);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  if (batch == 0 || total_tokens == 0) return FE_OK;
  FE_CHECK_ARG(k_pool && v_pool && block_tables && context_lens && out_offsets && k_out && v_out);
  FE_CHECK_ARG(aligned16(k_out) && aligned16(v_out) && aligned16(k_pool) && aligned16(v_pool));
  const int64_t work = (int64_t)total_tokens * kv_heads * (head_dim / 8);
  hipLaunchKernelGGL(gather_kv_kernel, dim3(grid_for(work, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const f16*)k_pool, (const f16*)v_pool, num_blocks,
                     block_tables, table_stride, context_lens, out_offsets, (f16*)k_out,
                     (f16*)v_out, batch, total_tokens, kv_heads, head_dim, block_size, bs_log2);
  return FE_LAUNCH_STATUS();
}

// ---- fp32 pools -------------------------------------------------------------
// The movers above copy 16-byte chunks and never look at the values, so an fp32
// row of head_dim elements is a 16-bit row of 2 * head_dim: the fp32 forms call
// them with the widths and strides (given in fp32 elements) doubled.

extern "C" int fe_write_kv_f32(const void* k_new, const void* v_new, int64_t new_token_stride,
                               void* k_pool, void* v_pool, int num_blocks,
                               const int32_t* slot_block, const int32_t* slot_offset,
                               int num_tokens, int kv_heads, int head_dim, int block_size,
                               fe_stream_t stream) {
  FE_CHECK_ARG(head_dim > 0 && head_dim % 4 == 0 && head_dim <= (1 << 28) &&
               new_token_stride % 4 == 0 && new_token_stride >= 0);
  return fe_write_kv(k_new, v_new, 2 * new_token_stride, k_pool, v_pool, num_blocks, slot_block,
                     slot_offset, num_tokens, kv_heads, 2 * head_dim, block_size, stream);
}

extern "C" int fe_write_kv_decode_f32(const void* k_new, const void* v_new,
                                      int64_t new_batch_stride, void* k_pool, void* v_pool,
                                      int num_blocks, const int32_t* block_tables,
                                      int table_stride, const int32_t* context_lens, int batch,
                                      int kv_heads, int head_dim, int block_size,
                                      fe_stream_t stream) {
  FE_CHECK_ARG(head_dim > 0 && head_dim % 4 == 0 && head_dim <= (1 << 28) &&
               new_batch_stride % 4 == 0 && new_batch_stride >= 0);
  return fe_write_kv_decode(k_new, v_new, 2 * new_batch_stride, k_pool, v_pool, num_blocks,
                            block_tables, table_stride, context_lens, batch, kv_heads,
                            2 * head_dim, block_size, stream);
}

extern "C" int fe_write_kv_ragged_f32(const void* k_new, const void* v_new,
                                      int64_t new_token_stride, void* k_pool, void* v_pool,
                                      int num_blocks, const int32_t* block_tables,
                                      int table_stride, const int32_t* q_offsets,
                                      const int32_t* context_lens, int num_seqs,
                                      int total_tokens, int kv_heads, int head_dim,
                                      int block_size, fe_stream_t stream) {
  FE_CHECK_ARG(head_dim > 0 && head_dim % 4 == 0 && head_dim <= (1 << 28) &&
               new_token_stride % 4 == 0 && new_token_stride >= 0);
  return fe_write_kv_ragged(k_new, v_new, 2 * new_token_stride, k_pool, v_pool, num_blocks,
                            block_tables, table_stride, q_offsets, context_lens, num_seqs,
                            total_tokens, kv_heads, 2 * head_dim, block_size, stream);
}

extern "C" int fe_gather_kv_f32(const void* k_pool, const void* v_pool, int num_blocks,
                                const int32_t* block_tables, int table_stride,
                                const int32_t* context_lens, const int32_t* out_offsets,
                                void* k_out, void* v_out, int batch, int total_tokens,
                                int kv_heads, int head_dim, int block_size, fe_stream_t stream) {
  FE_CHECK_ARG(head_dim > 0 && head_dim % 4 == 0 && head_dim <= (1 << 28));
  return fe_gather_kv(k_pool, v_pool, num_blocks, block_tables, table_stride, context_lens,
                      out_offsets, k_out, v_out, batch, total_tokens, kv_heads, 2 * head_dim,
                      block_size, stream);
}
