// Fused single-token paged decode attention for gfx950 (MI355X).
//
// Work decomposition
//   grid = (target + 2*batch, kv_heads); one 256-thread workgroup (4 waves)
//   per (piece of a sequence's keys, KV head).  The pieces come from the
//   device-side split-K partition in fe_common.h, so every workgroup gets an
//   equal share of keys whatever the context-length mix.  Wave w takes the
//   16-token tiles w, w+4, w+8, ... of the piece (tile engines: attn_core.h)
//   and the four waves are merged through LDS.  Workgroups past the last piece
//   write the zero rows of inactive sequences.
//
// Split-K merge, in the same launch: a sequence cut into several pieces has
// each piece write its fp32 partial output plus a base-2 log-sum-exp per query
// head to the workspace, then draw a ticket from a per-(sequence, KV head)
// counter; the workgroup drawing the last ticket merges all pieces and resets
// the counter, so the workspace is ready for the next call without a memset.
// Cross-workgroup visibility uses device-coherent accesses only: partials are
// written and read with agent-scope atomic stores/loads (which bypass the
// per-XCD L2), and the writer waits for its stores to complete before taking
// its ticket.  The agent-scope fences of the language memory model would
// instead write back and invalidate the whole L2 of the XCD per workgroup.
//
// The grid is flattened as x = piece * kv_heads + kv_head, so the kv_heads
// workgroups of one piece are dispatched together: they read interleaved
// halves of the same 512-byte pool rows.
//
// One wave serves all G = Hq/Hkv query heads of its KV head (the 16 MFMA
// columns), so every K/V byte is read from HBM once per step; the reference's
// Triton kernel reads it G times, once per query head
// (src/flexengine/inference/kernels/paged_attention.py:99-139).
#include "attn_core.h"

using namespace fe;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// Default split target: about FE_DECODE_WORKGROUPS working workgroups in total,
// i.e. that many / kv_heads pieces per KV head.  512 = two per CU of MI355X's
// 256, all resident at once at the two waves per SIMD the kernel runs at.
#ifndef FE_DECODE_WORKGROUPS
#define FE_DECODE_WORKGROUPS 512
#endif
constexpr int kDefaultWorkgroups = FE_DECODE_WORKGROUPS;
constexpr int kMaxGroup = 16;

// The occupancy the register allocation is held to (waves per SIMD).
#ifndef FE_DECODE_WAVES_PER_EU
#define FE_DECODE_WAVES_PER_EU 2
#endif
// LDS of the piece kernel: per-wave V staging, then every wave's parked state
// (o, m, l) for the combine, and a ticket flag.
template <int D>
struct PieceLds {
  static constexpr size_t stage = 0;
  static constexpr size_t park = stage + (size_t)kWaves * TileCfg<D>::STAGE;
  static constexpr size_t park_m = park + (size_t)kWaves * TileCfg<D>::NX * kWave * 16;
  static constexpr size_t park_l = park_m + (size_t)kWaves * kWave * sizeof(float);
  static constexpr size_t flag = park_l + (size_t)kWaves * kWave * sizeof(float);
  static constexpr size_t bytes = flag + sizeof(int);
};

struct DecodeArgs {
  const f16* q;
  f16* out;
  const f16* k_new;
  const f16* v_new;
  f16* k_pool;
  f16* v_pool;
  const int32_t* tables;
  const int32_t* ctx;
  float* ws_o;       // [pieces, Hq, D]
  float* ws_lse;     // [pieces, Hq]  (base 2)
  int* tickets;      // [B, Hkv], zero between calls
  // shared-prefix decode: sequence b attends only keys tok0[b].. here and
  // merges the prefix attention (pre_o [B*Hq][D], base-2 pre_lse [B*Hq]) in;
  // all three null otherwise
  const int32_t* tok0;
  const float* pre_o;
  const float* pre_lse;
  int64_t q_stride;
  int64_t new_stride;
  int W, B, Hq, Hkv, G, BS, bs_log2, NB, target;
  int max_len;       // W * BS: longest context the tables can address
  float scale_log2;  // softmax scale * log2(e)
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // buffer-instruction cache policy: sc1 (device-coherent)

__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Combines the ns pieces (slots first .. first+ns-1) of sequence b, KV head h:
// per query head, out = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M).
// Each thread owns 4 consecutive output elements (one 16-byte device-coherent
// load per piece) and computes their weights itself from the LSE it loads
// alongside; pieces are taken kMergeBatch at a time with an online max, so the
// common case (ns <= kMergeBatch) is one round trip to memory and no barrier.
constexpr int kMergeBatch = 16;

template <int D>
__device__ __forceinline__ void merge_pieces(const DecodeArgs& a, int b, int h, int first,
                                             int ns, bool pre = false) {
  const int G = a.G;
  const int n4 = G * D / 4;
  const int o_step = a.Hq * D;  // floats per slot
  const float* lse_base = a.ws_lse + (int64_t)first * a.Hq + h * G;
  // one descriptor over the ns slots (the host keeps the partial area < 2 GiB)
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o + ((int64_t)first * a.Hq + h * G) * D, 0, ns * o_step * (int)sizeof(float),
      0x00020000);
  for (int e4 = threadIdx.x; e4 < n4; e4 += kThreads) {
    const int hh = e4 * 4 / D;
    float M = kNegInf, den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += kMergeBatch) {
      // only the live slots are loaded (nb is wave-uniform)
      const int nb = ns - s0 < kMergeBatch ? ns - s0 : kMergeBatch;
      float lv[kMergeBatch];
      f32x4 ov[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        lv[u] = kNegInf;
        ov[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (u < nb) {
          const int sidx = s0 + u;
          lv[u] = load_coherent(lse_base + (int64_t)sidx * a.Hq + hh);
          ov[u] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         ro, (uint32_t)((sidx * o_step + e4 * 4) * sizeof(float)), 0, kSc1));
        }
      }
      float bm = kNegInf;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) bm = fmaxf(bm, lv[u]);
      const float newM = fmaxf(M, bm);
      const float alpha = M == kNegInf ? 0.f : exp2f(M - newM);
      num *= alpha;
      den *= alpha;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const float wv = lv[u] == kNegInf ? 0.f : exp2f(lv[u] - newM);
        num += wv * ov[u];
        den += wv;
      }
      M = newM;
    }
    if (pre) {
      // the shared-prefix part, written by the launch before this one
      const int64_t r = (int64_t)b * a.Hq + h * G;
      const float lv = a.pre_lse[r + hh];
      const f32x4 ov = *reinterpret_cast<const f32x4*>(a.pre_o + r * D + e4 * 4);
      if (lv != kNegInf) {
        const float newM = fmaxf(M, lv);
        const float alpha = M == kNegInf ? 0.f : exp2f(M - newM);
        num = num * alpha + exp2f(lv - newM) * ov;
        den = den * alpha + exp2f(lv - newM);
        M = newM;
      }
    }
    const float inv = 1.f / den;
    *reinterpret_cast<f16x4*>(a.out + ((int64_t)b * a.Hq + h * G) * D + e4 * 4) =
        f16x4{(f16)(num[0] * inv), (f16)(num[1] * inv), (f16)(num[2] * inv),
              (f16)(num[3] * inv)};
  }
}

template <int D, class Core>
__device__ __forceinline__ void setup_core(Core& core, const DecodeArgs& a, const Piece& pc, int h,
                                           unsigned char* stage) {
  core.trow = a.tables + (int64_t)pc.b * a.W;
  core.rs = a.Hkv * D;
  core.hoff = h * D;
  core.W = a.W;
  core.NB = a.NB;
  core.BS = a.BS;
  core.bs_log2 = a.bs_log2;
  core.tok_end = pc.tok_end;
  core.limit = pc.tok_end;
  core.scale_log2 = a.scale_log2;
  if (a.k_new != nullptr) {
    core.knew_row = a.k_new + (int64_t)pc.b * a.new_stride + (int64_t)h * D;
    core.vnew_row = a.v_new + (int64_t)pc.b * a.new_stride + (int64_t)h * D;
    core.new_pos = pc.L - 1;
  } else {
    core.knew_row = nullptr;
    core.vnew_row = nullptr;
    core.new_pos = -1;
  }
  core.stage = stage;
}

template <int D, bool PAGE16>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(PAGE16 ? FE_DECODE_WAVES_PER_EU : 2, 8)))
void piece_decode_kernel(const DecodeArgs a) {
  using C = TileCfg<D>;
  extern __shared__ __align__(16) unsigned char smem[];

  const int h = blockIdx.x % a.Hkv;
  const int item = blockIdx.x / a.Hkv;
  Piece pc;
  int total = 0;
  if (!find_piece(a.ctx, a.tok0, a.B, a.max_len, a.target, item, pc, total)) {
    // spare workgroup: zero rows of inactive sequences
    const int b = item - total;
    if (b < a.B && seq_len(a.ctx, b, a.max_len) == 0) {
      for (int e = threadIdx.x; e < a.G * D; e += kThreads)
        a.out[((int64_t)b * a.Hq + h * a.G) * D + e] = (f16)0.f;
    }
    return;
  }
  using Lds = PieceLds<D>;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int G = a.G;
  const int b = pc.b;
  const int t_first = pc.tok_begin / kTile + w;
  const int t_end = (pc.tok_end + kTile - 1) / kTile;

  f16x8 qv[C::NK];
  {
    const int hq = h * G + (n < G ? n : G - 1);
    const f16* qrow = a.q + (int64_t)b * a.q_stride + (int64_t)hq * D;
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      const f16x8 v = ld16(qrow + (4 * s + g) * 8);
      qv[s] = n < G ? v : f16x8{};
    }
  }

  float m_run, l_tot;
  f32x4 o[C::NX];
  if constexpr (PAGE16) {
    // the wave's tiles t_first, t_first + 4, ... of the piece as a tile list
    TileListCore<D> core;
    core.k_pool = a.k_pool;
    core.v_pool = a.v_pool;
    core.rs = a.Hkv * D;
    core.hoff = h * D;
    core.scale_log2 = a.scale_log2;
    core.stage = smem + w * C::STAGE;
    const int ntiles = t_first < t_end ? (t_end - t_first + kWaves - 1) / kWaves : 0;
    core.ntiles = ntiles;
    {
      const int tok = (t_first + lane * kWaves) * kTile;
      int blk = 0;
      if (lane < ntiles) blk = clamp_block(a.tables[(int64_t)b * a.W + (tok >> a.bs_log2)], a.NB);
      const int rem = pc.tok_end - tok;
      core.row_vec = blk * a.BS + (tok & (a.BS - 1));
      core.rows_vec = lane < ntiles ? (rem < kTile ? rem : kTile) : 0;
    }
    core.new_tile = -1;
    core.new_row = 0;
    if (a.k_new != nullptr && pc.tok_end == pc.L) {
      // the piece holds the decoded token (position L-1); the wave whose list
      // holds its tile takes the row from k_new / v_new, loaded here
      // alongside the tables
      const int tn = (pc.L - 1) / kTile - t_first;
      if (tn >= 0 && tn % kWaves == 0) {
        core.new_tile = tn / kWaves;
        core.new_row = (pc.L - 1) & (kTile - 1);
        const f16* kr = a.k_new + (int64_t)b * a.new_stride + (int64_t)h * D;
        const f16* vr = a.v_new + (int64_t)b * a.new_stride + (int64_t)h * D;
#pragma unroll
        for (int s = 0; s < C::NK; ++s) core.knew[s] = ld16(kr + (4 * s + g) * 8);
        core.vnew = ld16(vr + (lane % C::CPR) * 8);
      }
    }
#pragma unroll
    for (int s = 0; s < C::NK; ++s) core.qv[s] = qv[s];
    core.init_acc();
    core.run();
    core.store_new_row(a.k_pool, a.v_pool);
    m_run = core.m_run;
    l_tot = core.l_total();
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = core.o[x];
  } else {
    TileCore<D> core;
    setup_core<D>(core, a, pc, h, smem + w * C::STAGE);
    core.k_pool = a.k_pool;
    core.v_pool = a.v_pool;
#pragma unroll
    for (int s = 0; s < C::NK; ++s) core.qv[s] = qv[s];
    core.init_acc();
    core.run(t_first, kWaves, t_end);
    m_run = core.m_run;
    l_tot = core.l_total();
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = core.o[x];
  }

  // a sequence with a shared prefix always merges (its prefix part is a partial)
  const bool split = pc.nsplit > 1 || pc.tok0 > 0;
  f32x4* park = reinterpret_cast<f32x4*>(smem + Lds::park);  // [4][NX][64]
  float* park_m = reinterpret_cast<float*>(smem + Lds::park_m);
  float* park_l = reinterpret_cast<float*>(smem + Lds::park_l);
  int* flag = reinterpret_cast<int*>(smem + Lds::flag);
  // ---- combine the four waves: every wave parks (o, m, l) in LDS (lane-major,
  // conflict-free); wave w then combines output tiles [w*XW, (w+1)*XW) of all
  // four in the register layout of the loop: lane (g, n) holds
  // O[head n][16x + 4g + i], so the per-head scale factors are per lane.
  {
#pragma unroll
    for (int x = 0; x < C::NX; ++x) park[(w * C::NX + x) * kWave + lane] = o[x];
    park_m[w * kWave + lane] = m_run;
    park_l[w * kWave + lane] = l_tot;
    __syncthreads();
    float M = kNegInf;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) M = fmaxf(M, park_m[v * kWave + lane]);
    float sc[kWaves];
    float den = 0.f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      const float mv = park_m[v * kWave + lane];
      sc[v] = mv == kNegInf ? 0.f : exp2f(mv - M);
      den += sc[v] * park_l[v * kWave + lane];
    }
    const float inv = 1.f / den;
    constexpr int XW = C::NX / kWaves;  // output tiles per wave
    f32x4 ox[XW];
#pragma unroll
    for (int xi = 0; xi < XW; ++xi) {
      const int x = w * XW + xi;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < kWaves; ++v) acc += sc[v] * park[(v * C::NX + x) * kWave + lane];
      ox[xi] = acc * inv;
    }
    if (n < G) {
      const int hq = h * G + n;
      if (!split) {
        f16* orow = a.out + ((int64_t)b * a.Hq + hq) * D + 4 * g;
#pragma unroll
        for (int xi = 0; xi < XW; ++xi)
          *reinterpret_cast<f16x4*>(orow + 16 * (w * XW + xi)) =
              f16x4{(f16)ox[xi][0], (f16)ox[xi][1], (f16)ox[xi][2], (f16)ox[xi][3]};
      } else {
        // device-coherent (sc1) 16-byte stores of this piece's partial output
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            a.ws_o + ((int64_t)item * a.Hq + h * G) * D, 0, G * D * (int)sizeof(float),
            0x00020000);
        const uint32_t off = (uint32_t)((n * D + 4 * g) * sizeof(float));
#pragma unroll
        for (int xi = 0; xi < XW; ++xi)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, ox[xi]), r,
              off + 16 * (w * XW + xi) * (uint32_t)sizeof(float), 0, kSc1);
        if (w == 0 && g == 0) store_coherent(a.ws_lse + (int64_t)item * a.Hq + hq, M + log2f(den));
      }
    }
  }
  if (!split) return;

  // ---- split-K: the last piece of (b, h) to finish merges all pieces ----
  wait_stores();  // this wave's partials are complete at the device-coherent level
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(a.tickets + b * a.Hkv + h, 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == pc.nsplit - 1;
  __syncthreads();
  if (!*flag) return;
  if (threadIdx.x == 0)
    __hip_atomic_store(a.tickets + b * a.Hkv + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  merge_pieces<D>(a, b, h, item - pc.split, pc.nsplit, pc.tok0 > 0);
}

// General LSE merge of S partial results (natural-log LSE at the boundary).
__global__ __launch_bounds__(kThreads) void lse_merge_kernel(const float* __restrict__ po,
                                                             const float* __restrict__ plse,
                                                             int S, int R, int D, f16* out,
                                                             float* out_lse) {
  const int r = blockIdx.x;
  float M = kNegInf;
  for (int s = 0; s < S; ++s) M = fmaxf(M, plse[(int64_t)s * R + r] * kLog2e);
  if (M == kNegInf) {
    for (int d = threadIdx.x; d < D; d += blockDim.x) out[(int64_t)r * D + d] = (f16)0.f;
    if (out_lse && threadIdx.x == 0) out_lse[r] = kNegInf;
    return;
  }
  float den = 0.f;
  for (int s = 0; s < S; ++s) den += exp2f(plse[(int64_t)s * R + r] * kLog2e - M);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float num = 0.f;
    for (int s = 0; s < S; ++s)
      num += exp2f(plse[(int64_t)s * R + r] * kLog2e - M) * po[((int64_t)s * R + r) * D + d];
    out[(int64_t)r * D + d] = (f16)(num / den);
  }
  if (out_lse && threadIdx.x == 0) out_lse[r] = (M + log2f(den)) / kLog2e;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// workspace = [tickets (fixed region) | partial outputs | partial lse].  The
// ticket region sits at offset 0 with a fixed size, so calls of any shape
// share it and find it zero.
constexpr int kMaxTickets = 65536;
constexpr size_t kTicketBytes = kMaxTickets * sizeof(int);
inline size_t ws_o_bytes(int batch, int hq, int d, int target) {
  return align256((size_t)(target + batch) * hq * d * sizeof(float));
}
inline size_t ws_lse_bytes(int batch, int hq, int target) {
  return align256((size_t)(target + batch) * hq * sizeof(float));
}

// Pieces per KV head the kernel aims for.  Raised above the request when the
// tables allow very long contexts, so that no piece holds more than 64 quads
// (256 tiles: one staged pool row per thread of the workgroup).
inline int effective_target(int batch, int kv_heads, int max_context, int target_splits) {
  const int target =
      target_splits > 0 ? target_splits : (kDefaultWorkgroups + kv_heads - 1) / kv_heads;
  const int64_t max_quads = ((int64_t)max_context + 63) / 64;
  const int64_t need = ((int64_t)batch * max_quads + 63) / 64;
  return need > target ? (int)need : target;
}

template <int D>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((a.target + 2 * a.B) * a.Hkv);
  if (a.BS % kTile == 0)
    hipLaunchKernelGGL((piece_decode_kernel<D, true>), grid, dim3(kThreads), PieceLds<D>::bytes,
                       stream, a);
  else
    hipLaunchKernelGGL((piece_decode_kernel<D, false>), grid, dim3(kThreads), PieceLds<D>::bytes,
                       stream, a);
  return FE_LAUNCH_STATUS();
}

}  // namespace

extern "C" size_t fe_paged_decode_workspace_size(int batch, int num_q_heads, int head_dim,
                                                 int max_context, int target_splits) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_context < 0 || target_splits < 0)
    return 0;
  // sized for the largest default (kv_heads = 1): valid for every kv_heads
  const int target = effective_target(batch, 1, max_context, target_splits);
  return kTicketBytes + ws_o_bytes(batch, num_q_heads, head_dim, target) +
         ws_lse_bytes(batch, num_q_heads, target);
}

namespace {

// Everything fe_paged_decode and fe_paged_decode_shared_prefix share: argument
// checks, workspace carving and the decode launch.  `cascade` (null for plain
// decode) is filled with the workspace regions of the shared-prefix half and
// launched first.
int decode_impl(const void* q, int64_t q_batch_stride, void* out, const void* k_new,
                const void* v_new, int64_t new_batch_stride, void* k_pool, void* v_pool,
                int num_blocks, const int32_t* block_tables, int table_stride,
                const int32_t* context_lens, void* workspace, size_t workspace_bytes, int batch,
                int num_q_heads, int kv_heads, int head_dim, int block_size, float scale,
                int target_splits, CascadePrefix* cascade, hipStream_t stream) {
  FE_CHECK_ARG(batch >= 0 && num_q_heads > 0 && kv_heads > 0 && num_blocks > 0 &&
               table_stride > 0 && target_splits >= 0);
  if (head_dim != 64 && head_dim != 128) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  const int G = num_q_heads / kv_heads;
  if (G > kMaxGroup) return FE_ERR_UNSUPPORTED;
  if ((int64_t)batch * kv_heads > kMaxTickets) return FE_ERR_UNSUPPORTED;
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  // the shared-prefix split needs 16-token-aligned suffixes (block-size-16k path)
  if (cascade && block_size % kTile != 0) return FE_ERR_UNSUPPORTED;
  if (batch == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && context_lens);
  FE_CHECK_ARG((k_new == nullptr) == (v_new == nullptr));
  FE_CHECK_ARG(q_batch_stride % 8 == 0 && q_batch_stride >= (int64_t)num_q_heads * head_dim);
  FE_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(k_pool) && aligned16(v_pool));
  // lane offsets inside a block are 32-bit
  FE_CHECK_ARG((int64_t)block_size * kv_heads * head_dim < (int64_t)1 << 30);
  if (k_new) {
    FE_CHECK_ARG(aligned16(k_new) && aligned16(v_new) && new_batch_stride % 8 == 0 &&
                 new_batch_stride >= (int64_t)kv_heads * head_dim);
  }
  // a piece holds at most 64 quads (64 tiles per wave) and a sequence at most
  // kMaxPieces pieces: contexts up to 64 * 64 * 64 = 262144 tokens
  if ((int64_t)table_stride * block_size > 262144) return FE_ERR_UNSUPPORTED;
  const int max_len = table_stride * block_size;
  const int target = effective_target(batch, kv_heads, max_len, target_splits);
  if ((int64_t)(target + batch) * num_q_heads * head_dim * (int64_t)sizeof(float) >= ((int64_t)1 << 31))
    return FE_ERR_UNSUPPORTED;
  const size_t need = fe_paged_decode_workspace_size(batch, num_q_heads, head_dim, max_len, target);
  const size_t need_all =
      cascade ? fe_paged_decode_shared_prefix_workspace_size(batch, num_q_heads, kv_heads, head_dim,
                                                             max_len, cascade->num_groups, target)
              : need;
  if (workspace == nullptr || workspace_bytes < need_all || !aligned16(workspace))
    return FE_ERR_WORKSPACE;

  DecodeArgs a;
  a.q = (const f16*)q;
  a.out = (f16*)out;
  a.k_new = (const f16*)k_new;
  a.v_new = (const f16*)v_new;
  a.k_pool = (f16*)k_pool;
  a.v_pool = (f16*)v_pool;
  a.tables = block_tables;
  a.ctx = context_lens;
  char* ws = (char*)workspace;
  a.tickets = (int*)ws;
  ws += kTicketBytes;
  a.ws_o = (float*)ws;
  ws += ws_o_bytes(batch, num_q_heads, head_dim, target);
  a.ws_lse = (float*)ws;
  a.tok0 = nullptr;
  a.pre_o = nullptr;
  a.pre_lse = nullptr;
  a.q_stride = q_batch_stride;
  a.new_stride = new_batch_stride;
  a.W = table_stride;
  a.B = batch;
  a.Hq = num_q_heads;
  a.Hkv = kv_heads;
  a.G = G;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.target = target;
  a.max_len = max_len;
  a.scale_log2 = scale * kLog2e;
  const hipStream_t s = (hipStream_t)stream;
  if (cascade) {
    char* cw = (char*)workspace + need;
    CascadePrefix& c = *cascade;
    c.q = q;
    c.q_stride = q_batch_stride;
    c.k_pool = k_pool;
    c.v_pool = v_pool;
    c.num_blocks = num_blocks;
    c.tables = block_tables;
    c.table_stride = table_stride;
    c.ctx = context_lens;
    c.batch = batch;
    c.hq = num_q_heads;
    c.hkv = kv_heads;
    c.d = head_dim;
    c.bs = block_size;
    c.scale = scale;
    c.tickets = a.tickets;  // each launch leaves the tickets it used at zero
    c.tok0 = (int32_t*)cw;
    cw += align256((size_t)batch * sizeof(int32_t));
    c.pre_o = (float*)cw;
    cw += align256((size_t)batch * num_q_heads * head_dim * sizeof(float));
    c.pre_lse = (float*)cw;
    cw += align256((size_t)batch * num_q_heads * sizeof(float));
    c.scratch = cw;
    const int rc = cascade_prefix_launch(c, s);
    if (rc != FE_OK) return rc;
    a.tok0 = c.tok0;
    a.pre_o = c.pre_o;
    a.pre_lse = c.pre_lse;
  }
  if (head_dim == 64) return launch_decode<64>(a, s);
  return launch_decode<128>(a, s);
}

}  // namespace

extern "C" int fe_paged_decode(const void* q, int64_t q_batch_stride, void* out,
                               const void* k_new, const void* v_new, int64_t new_batch_stride,
                               void* k_pool, void* v_pool, int num_blocks,
                               const int32_t* block_tables, int table_stride,
                               const int32_t* context_lens, void* workspace,
                               size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
                               int head_dim, int block_size, float scale, int target_splits,
                               fe_stream_t stream) {
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, nullptr, (hipStream_t)stream);
}

extern "C" size_t fe_paged_decode_shared_prefix_workspace_size(int batch, int num_q_heads,
                                                               int kv_heads, int head_dim,
                                                               int max_context, int num_groups,
                                                               int target_splits) {
  if (batch < 0 || num_q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || max_context < 0 ||
      num_groups < 0 || target_splits < 0 || num_q_heads % kv_heads)
    return 0;
  return fe_paged_decode_workspace_size(batch, num_q_heads, head_dim, max_context, target_splits) +
         align256((size_t)batch * sizeof(int32_t)) +
         align256((size_t)batch * num_q_heads * head_dim * sizeof(float)) +
         align256((size_t)batch * num_q_heads * sizeof(float)) +
         cascade_prefix_scratch_bytes(num_groups, batch, num_q_heads, kv_heads, head_dim);
}

extern "C" int fe_paged_decode_shared_prefix(
    const void* q, int64_t q_batch_stride, void* out, const void* k_new, const void* v_new,
    int64_t new_batch_stride, void* k_pool, void* v_pool, int num_blocks,
    const int32_t* block_tables, int table_stride, const int32_t* context_lens,
    const int32_t* group_offsets, const int32_t* group_prefix_lens, int num_groups,
    void* workspace, size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
    int head_dim, int block_size, float scale, int target_splits, fe_stream_t stream) {
  FE_CHECK_ARG(num_groups >= 0 && num_groups <= batch + 1);
  if (num_groups == 0 || batch == 0)
    return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                       num_blocks, block_tables, table_stride, context_lens, workspace,
                       workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                       target_splits, nullptr, (hipStream_t)stream);
  FE_CHECK_ARG(group_offsets && group_prefix_lens);
  CascadePrefix c{};
  c.group_offsets = group_offsets;
  c.prefix_len = group_prefix_lens;
  c.num_groups = num_groups;
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, &c, (hipStream_t)stream);
}

extern "C" int fe_lse_merge(const float* part_out, const float* part_lse, int num_splits,
                            int rows, int head_dim, void* out, float* out_lse,
                            fe_stream_t stream) {
  FE_CHECK_ARG(num_splits > 0 && rows >= 0 && head_dim > 0);
  if (rows == 0) return FE_OK;
  FE_CHECK_ARG(part_out && part_lse && out);
  const int threads = head_dim >= 256 ? 256 : (head_dim >= 128 ? 128 : 64);
  hipLaunchKernelGGL(lse_merge_kernel, dim3(rows), dim3(threads), 0, (hipStream_t)stream,
                     part_out, part_lse, num_splits, rows, head_dim, (f16*)out, out_lse);
  return FE_LAUNCH_STATUS();
}
