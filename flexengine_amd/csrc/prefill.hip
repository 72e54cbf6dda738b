// Ragged chunked-prefill attention over paged KV for gfx950 (MI355X).
//
// Every sequence s contributes n_s new query rows (q_offsets[s] ..
// q_offsets[s+1]) that sit at absolute positions ctx_s - n_s .. ctx_s - 1 and
// attend causally to keys t <= position over the paged K/V of the sequence
// (the new rows' own K/V are already in the pool).
//
// grid = (64-row query blocks of all sequences, num_q_heads); 256 threads.
// Wave w of a workgroup owns 16 query rows of one query head: they are the 16
// MFMA columns of the tile engine in attn_core.h, each column with its own
// causal limit (position + 1).  The QK^T and PV contractions run on
// v_mfma_f32_16x16x16_f16 with fp32 accumulation.
#include "attn_core.h"

using namespace fe;

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 16;
constexpr int kRowsPerBlock = 64;

struct PrefillArgs {
  const f16* q;
  f16* out;
  f16* k_pool;
  f16* v_pool;
  const int32_t* tables;
  const int32_t* q_off;
  const int32_t* ctx;
  int W, S, total_q, Hq, Hkv, G, BS, bs_log2, NB;
  float scale_log2;
};

struct QBlock {
  int s;     // sequence
  int qb;    // 64-row block index within the sequence
  int n;     // query rows of the sequence
  int q0;    // first query row of the sequence in q/out
  int ctx;   // context length of the sequence
};

__device__ __forceinline__ int seq_rows(const PrefillArgs& a, int s, int& q0) {
  q0 = a.q_off[s];
  const int n = a.q_off[s + 1] - q0;
  return n > 0 ? n : 0;
}

// Maps a workgroup id onto (sequence, query block); false past the last block.
__device__ __forceinline__ bool locate_qblock(const PrefillArgs& a, int item, QBlock& qb) {
  const int lane = lane_id();
  int carry = 0;
  for (int base = 0; base < a.S; base += kWave) {
    const int s = base + lane;
    int q0 = 0, n = 0;
    if (s < a.S) n = seq_rows(a, s, q0);
    const int nb = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    const int incl = wave_scan_incl_i(nb) + carry;
    const int excl = incl - nb;
    const unsigned long long hit = __ballot(s < a.S && item >= excl && item < incl);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      qb.s = base + src;
      qb.qb = item - readlane_i(excl, src);
      qb.n = readlane_i(n, src);
      qb.q0 = readlane_i(q0, src);
      qb.ctx = clamp_len(a.ctx[qb.s]);
      return true;
    }
    carry = readlane_i(incl, kWave - 1);
  }
  return false;
}

template <int D>
__global__ __launch_bounds__(kThreads) void prefill_kernel(const PrefillArgs a) {
  using C = TileCfg<D>;
  __shared__ __align__(16) unsigned char smem[4 * C::STAGE];

  QBlock qb;
  if (!locate_qblock(a, blockIdx.x, qb)) return;
  const int hq = blockIdx.y;
  const int h = hq / a.G;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int row0 = qb.qb * kRowsPerBlock + w * kRowsPerWave;  // first row of this wave
  if (row0 >= qb.n) return;                                   // wave without rows
  const int cached = qb.ctx >= qb.n ? qb.ctx - qb.n : 0;
  const int row = row0 + n;
  const bool valid = row < qb.n;
  const int last_row = (row0 + kRowsPerWave - 1 < qb.n ? row0 + kRowsPerWave : qb.n) - 1;

  TileCore<D> core;
  core.k_pool = a.k_pool;
  core.v_pool = a.v_pool;
  core.trow = a.tables + (int64_t)qb.s * a.W;
  core.rs = (int64_t)a.Hkv * D;
  core.hoff = h * D;
  core.W = a.W;
  core.NB = a.NB;
  core.BS = a.BS;
  core.bs_log2 = a.bs_log2;
  core.tok_end = cached + last_row + 1;
  core.limit = valid ? cached + row + 1 : 0;
  core.scale_log2 = a.scale_log2;
  core.knew_row = nullptr;
  core.vnew_row = nullptr;
  core.new_pos = -1;
  core.stage = smem + w * C::STAGE;

  int qrow_idx = qb.q0 + (valid ? row : last_row);
  qrow_idx = qrow_idx < a.total_q ? qrow_idx : a.total_q - 1;
  {
    const f16* qrow = a.q + ((int64_t)qrow_idx * a.Hq + hq) * D;
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      const f16x8 v = ld16(qrow + (4 * s + g) * 8);
      core.qv[s] = valid ? v : f16x8{};
    }
  }
  core.init_acc();
  core.run(0, 1, (core.tok_end + kTile - 1) / kTile);

  const float l = core.l_total();
  if (valid) {
    const float inv = 1.f / l;
    f16* orow = a.out + ((int64_t)qrow_idx * a.Hq + hq) * D;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) {
      const f16x4 v = {(f16)(core.o[x][0] * inv), (f16)(core.o[x][1] * inv),
                       (f16)(core.o[x][2] * inv), (f16)(core.o[x][3] * inv)};
      *reinterpret_cast<f16x4*>(orow + 16 * x + 4 * g) = v;
    }
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

}  // namespace

extern "C" int fe_prefill_paged(const void* q, void* out, const void* k_pool, const void* v_pool,
                                int num_blocks, const int32_t* block_tables, int table_stride,
                                const int32_t* q_offsets, const int32_t* context_lens,
                                int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                int kv_heads, int head_dim, int block_size, float scale,
                                fe_stream_t stream) {
  FE_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 &&
               kv_heads > 0 && num_blocks > 0 && table_stride > 0);
  if (head_dim != 64 && head_dim != 128) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  if (num_seqs == 0 || total_q == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && q_offsets && context_lens);
  FE_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(k_pool) && aligned16(v_pool));

  PrefillArgs a;
  a.q = (const f16*)q;
  a.out = (f16*)out;
  a.k_pool = (f16*)k_pool;
  a.v_pool = (f16*)v_pool;
  a.tables = block_tables;
  a.q_off = q_offsets;
  a.ctx = context_lens;
  a.W = table_stride;
  a.S = num_seqs;
  a.total_q = total_q;
  a.Hq = num_q_heads;
  a.Hkv = kv_heads;
  a.G = num_q_heads / kv_heads;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.scale_log2 = scale * kLog2e;
  // upper bound on the number of 64-row blocks: sum_s ceil(n_s/64) <= total_q/64 + num_seqs
  const int blocks = (total_q + kRowsPerBlock - 1) / kRowsPerBlock + num_seqs;
  const dim3 grid(blocks, num_q_heads);
  if (head_dim == 64)
    hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  return FE_LAUNCH_STATUS();
}
