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

// Register stages of the K/V prefetch pipeline and the occupancy the register
// allocation is held to (waves per SIMD); tuned on MI355X for head_dim 128.
#ifndef FE_DECODE_STAGES
#define FE_DECODE_STAGES 2
#endif
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
      float lv[kMergeBatch];
      f32x4 ov[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int sidx = s0 + u < ns ? s0 + u : ns - 1;  // clamped: always a written slot
        lv[u] = load_coherent(lse_base + (int64_t)sidx * a.Hq + hh);
        ov[u] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       ro, (uint32_t)((sidx * o_step + e4 * 4) * sizeof(float)), 0, kSc1));
      }
      float bm = kNegInf;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (s0 + u >= ns) lv[u] = kNegInf;
        bm = fmaxf(bm, lv[u]);
      }
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
  const int chunk = split_chunk_quads(a.ctx, a.tok0, a.B, a.max_len, a.target);
  Piece pc;
  int total = 0;
  if (!locate_piece(a.ctx, a.tok0, a.B, a.max_len, chunk, item, pc, total)) {
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
    TileListCore<D> core;
    core.k_pool = a.k_pool;
    core.v_pool = a.v_pool;
    core.k_pool_w = a.k_pool;
    core.v_pool_w = a.v_pool;
    core.rs = a.Hkv * D;
    core.hoff = h * D;
    core.scale_log2 = a.scale_log2;
    core.stage = smem + w * C::STAGE;
    // the wave's tiles t_first, t_first + 4, ... of the piece as a tile list
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
    if (a.k_new != nullptr) {
      const int tn = (pc.L - 1) / kTile - t_first;  // list index of the decoded token's tile
      if (tn >= 0 && tn % kWaves == 0 && tn / kWaves < ntiles)
        core.write_new_row(tn / kWaves, (pc.L - 1) & (kTile - 1),
                           a.k_new + (int64_t)b * a.new_stride + (int64_t)h * D,
                           a.v_new + (int64_t)b * a.new_stride + (int64_t)h * D);
    }
#pragma unroll
    for (int s = 0; s < C::NK; ++s) core.qv[s] = qv[s];
    core.init_acc();
    if (ntiles > 0) {
      typename TileListCore<D>::template Buffers<FE_DECODE_STAGES> buf;
      core.prologue(buf);
      auto more = [&](TileListCore<D>&, int k) { return k + 1 < ntiles; };
      core.template run<FE_DECODE_STAGES>(buf, more);
    }
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

// ---- equal-tile ("lean") decode for block sizes divisible by 16 -------------
//
// The keys of every sequence are cut into 16-token tiles; per KV head the tiles
// of all sequences, in sequence order, form one list of T tiles.  Workgroup j
// (of P per KV head) takes the contiguous range [j*ceil(T/P), ...) whatever the
// sequence boundaries, so every workgroup -- and every CU -- gets the same
// number of tiles within one.  Wave w of the workgroup takes a contiguous
// quarter of the range; consecutive tiles of a wave can belong to different
// sequences, and at each sequence boundary the wave's state (o, m, l) for that
// sequence is flushed:
//   - the wave saw the whole sequence: normalise and write the output row;
//   - the sequence started in an earlier wave of this workgroup: park the state
//     in LDS for that wave;
//   - the sequence continues in a later wave of this workgroup: keep it in
//     registers, and after the loop merge in the later waves' parked states;
//   - otherwise (or after that merge) the sequence spans several workgroups:
//     write a partial output and its LSE to slot j + b, draw a ticket, and the
//     last of its ceil-divided pieces merges them (merge_pieces).
// A workgroup has at most two such pieces: the sequences at either end of its
// range.  Slots j + b are distinct for distinct (range, sequence) pairs since
// both indices only grow along the tile list.
template <int D>
struct LeanLds {
  using C = TileCfg<D>;
  static constexpr size_t park = (size_t)kWaves * C::STAGE;
  static constexpr size_t park_m = park + (size_t)(kWaves - 1) * C::NX * kWave * 16;
  static constexpr size_t park_l = park_m + (size_t)(kWaves - 1) * kWave * sizeof(float);
  static constexpr size_t flags = park_l + (size_t)(kWaves - 1) * kWave * sizeof(float);
  static constexpr size_t bytes = flags + 8 * sizeof(int);
};

template <int D>
__device__ __forceinline__ void store_rows_final(const DecodeArgs& a, int b, int h,
                                                 const f32x4 (&o)[TileCfg<D>::NX], float inv,
                                                 int lane) {
  const int g = lane >> 4;
  const int n = lane & 15;
  if (n < a.G) {
    f16* orow = a.out + ((int64_t)b * a.Hq + h * a.G + n) * D + 4 * g;
#pragma unroll
    for (int x = 0; x < TileCfg<D>::NX; ++x)
      *reinterpret_cast<f16x4*>(orow + 16 * x) =
          f16x4{(f16)(o[x][0] * inv), (f16)(o[x][1] * inv), (f16)(o[x][2] * inv),
                (f16)(o[x][3] * inv)};
  }
}

// Partial output (normalised) and base-2 LSE of one piece, written with
// device-coherent (sc1) stores.
template <int D>
__device__ __forceinline__ void store_rows_partial(const DecodeArgs& a, int slot, int h,
                                                   const f32x4 (&o)[TileCfg<D>::NX], float inv,
                                                   float lse, int lane) {
  const int g = lane >> 4;
  const int n = lane & 15;
  const int G = a.G;
  if (n < G) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_o + ((int64_t)slot * a.Hq + h * G) * D, 0, G * D * (int)sizeof(float), 0x00020000);
    const uint32_t off = (uint32_t)((n * D + 4 * g) * sizeof(float));
#pragma unroll
    for (int x = 0; x < TileCfg<D>::NX; ++x)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[x] * inv), r,
                                             off + 16 * x * sizeof(float), 0, kSc1);
    if (g == 0) store_coherent(a.ws_lse + (int64_t)slot * a.Hq + h * G + n, lse);
  }
}

template <int D>
__device__ __forceinline__ void zero_row(const DecodeArgs& a, int b, int h) {
  f16* row = a.out + ((int64_t)b * a.Hq + h * a.G) * D;
  for (int e = lane_id() * 8; e < a.G * D; e += kWave * 8) st16(row + e, f16x8{});
}

// Query vectors of sequence b for the MFMA B operand: lane (g, n) holds chunks
// 4s+g of query head n of the group (zeros for n >= G).
template <int D>
__device__ __forceinline__ void load_q(const DecodeArgs& a, int b, int h, int lane,
                                       f16x8 (&qv)[TileCfg<D>::NK]) {
  const int g = lane >> 4;
  const int n = lane & 15;
  const int nn = n < a.G ? n : a.G - 1;
  const f16* qr = a.q + (int64_t)b * a.q_stride + (int64_t)(h * a.G + nn) * D + g * 8;
#pragma unroll
  for (int s = 0; s < TileCfg<D>::NK; ++s) {
    const f16x8 v = ld16(qr + s * 32);
    qv[s] = n < a.G ? v : f16x8{};
  }
}

template <int D>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(FE_DECODE_WAVES_PER_EU, 8)))
void lean_decode_kernel(const DecodeArgs a) {
  using C = TileCfg<D>;
  using Lds = LeanLds<D>;
  using Core = TileListCore<D>;
  extern __shared__ __align__(16) unsigned char smem[];

  const int h = blockIdx.x % a.Hkv;
  const int j = blockIdx.x / a.Hkv;
  const int P = a.target;  // ranges per KV head
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id();

  int* mflag = reinterpret_cast<int*>(smem + Lds::flags);  // [2][b, first, ns]
  if (tid < 6) mflag[tid] = -1;  // read only after later barriers

  // ---- tiles in total; zero rows of inactive sequences b = j (mod P).  The
  //      first 64 sequences stay in registers for the second pass. ----
  const int L0 = lane < a.B ? seq_len(a.ctx, lane, a.max_len) : 0;
  const int nt0 = (L0 + kTile - 1) / kTile;
  const int incl0 = wave_scan_incl_i(nt0);
  int T = readlane_i(incl0, kWave - 1);
  for (int base = 0; base < a.B; base += kWave) {
    const int bb = base + lane;
    const int L = base == 0 ? L0 : (bb < a.B ? seq_len(a.ctx, bb, a.max_len) : 0);
    if (base > 0) T += wave_sum_i((L + kTile - 1) / kTile);
    if (w == 0) {
      unsigned long long z = __ballot(bb < a.B && L == 0 && bb % P == j);
      while (z) {
        const int zb = base + __builtin_ctzll(z);
        z &= z - 1;
        zero_row<D>(a, zb, h);
      }
    }
  }
  T = __builtin_amdgcn_readfirstlane(T);
  if (T == 0) return;
  const int tpr = (T + P - 1) / P;
  const int r0 = j * tpr;
  if (r0 >= T) return;
  const int r1 = min(r0 + tpr, T);
  // wave w: a contiguous sub-range; the first (len % 4) waves take one more tile
  const int len = r1 - r0;
  const int qw = len / kWaves;
  const int qr = len % kWaves;
  auto wave_begin = [&](int v) { return r0 + v * qw + (v < qr ? v : qr); };
  const int wa = wave_begin(w);
  const int we = wave_begin(w + 1);
  const int ntiles = we - wa;  // <= 64: the host keeps ceil(T/P) <= 256

  // ---- lane k: sequence, first tile and length of the sequence of tile wa+k;
  //      the sequences at both ends of the workgroup's range ----
  int seq_v = 0, s0_v = 0, len_v = 0;
  int S0_first = 0, S1_last = 0;
  auto visit = [&](int base, int L, int nt, int incl) __attribute__((always_inline)) {
    const int excl = incl - nt;
    unsigned long long mk = __ballot(nt > 0 && excl < we && incl > wa);
    while (mk) {
      const int i = __builtin_ctzll(mk);
      mk &= mk - 1;
      const int sb = readlane_i(excl, i);
      const int lb = readlane_i(L, i);
      if (wa + lane >= sb) {
        seq_v = base + i;
        s0_v = sb;
        len_v = lb;
      }
    }
    const unsigned long long m0 = __ballot(excl <= r0 && r0 < incl);
    if (m0) S0_first = readlane_i(excl, __builtin_ctzll(m0));
    const unsigned long long m1 = __ballot(excl < r1 && r1 <= incl);
    if (m1) S1_last = readlane_i(incl, __builtin_ctzll(m1));
  };
  visit(0, L0, nt0, incl0);
  for (int base = kWave, carry = readlane_i(incl0, kWave - 1); base < a.B && carry < r1;
       base += kWave) {
    const int bb = base + lane;
    const int L = bb < a.B ? seq_len(a.ctx, bb, a.max_len) : 0;
    const int nt = (L + kTile - 1) / kTile;
    const int incl = wave_scan_incl_i(nt) + carry;
    visit(base, L, nt, incl);
    carry = readlane_i(incl, kWave - 1);
  }
  const bool wg_partial = S0_first < r0 || S1_last > r1;  // some sequence leaves the range

  // ---- query vectors of the wave's first two sequences, block ids of its
  //      tiles, and the new K/V rows of the sequences ending in its tiles ----
  Core core;
  core.k_pool = a.k_pool;
  core.v_pool = a.v_pool;
  core.k_pool_w = a.k_pool;
  core.v_pool_w = a.v_pool;
  core.rs = a.Hkv * D;
  core.hoff = h * D;
  core.scale_log2 = a.scale_log2;
  core.stage = smem + w * C::STAGE;
  core.ntiles = ntiles;
  const int b_seg0 = readlane_i(seq_v, 0);
  const unsigned long long second = __ballot(lane < ntiles && seq_v != b_seg0);
  const int b_seg1 = second ? readlane_i(seq_v, __builtin_ctzll(second)) : -1;
  f16x8 qn[C::NK];
  if (ntiles > 0) load_q<D>(a, b_seg0, h, lane, core.qv);
  if (b_seg1 >= 0) load_q<D>(a, b_seg1, h, lane, qn);
  int blk = 0;
  if (lane < ntiles) {
    const int tok = (wa + lane - s0_v) * kTile;
    blk = clamp_block(a.tables[(int64_t)seq_v * a.W + (tok >> a.bs_log2)], a.NB);
  }
  {
    const int tok = (wa + lane - s0_v) * kTile;
    const int rem = len_v - tok;
    core.row_vec = blk * a.BS + (tok & (a.BS - 1));
    core.rows_vec = lane < ntiles ? (rem < kTile ? rem : kTile) : 0;
  }
  if (a.k_new != nullptr) {
    // tiles holding a sequence's last key: write the decoded token's K/V row
    unsigned long long mk =
        __ballot(lane < ntiles && wa + lane == s0_v + (len_v + kTile - 1) / kTile - 1);
    while (mk) {
      const int k = __builtin_ctzll(mk);
      mk &= mk - 1;
      const int bn = readlane_i(seq_v, k);
      const int r = (readlane_i(len_v, k) - 1) & (kTile - 1);
      core.write_new_row(k, r, a.k_new + (int64_t)bn * a.new_stride + (int64_t)h * D,
                         a.v_new + (int64_t)bn * a.new_stride + (int64_t)h * D);
    }
  }

  f32x4* park = reinterpret_cast<f32x4*>(smem + Lds::park);
  float* park_m = reinterpret_cast<float*>(smem + Lds::park_m);
  float* park_l = reinterpret_cast<float*>(smem + Lds::park_l);
  int keep_b = -1, keep_S0 = 0, keep_S1 = 0;
  int pend_b[2] = {-1, -1}, pend_first[2] = {0, 0}, pend_ns[2] = {0, 0};
  auto add_pending = [&](int b, int S0, int S1) __attribute__((always_inline)) {
    const int first = S0 / tpr + b;
    const int ns = (S1 - 1) / tpr - S0 / tpr + 1;
    if (S1 > r1) {
      pend_b[1] = b; pend_first[1] = first; pend_ns[1] = ns;
    } else {
      pend_b[0] = b; pend_first[0] = first; pend_ns[0] = ns;
    }
  };

  if (ntiles > 0) {
    typename Core::template Buffers<FE_DECODE_STAGES> buf;
    core.prologue(buf);
    core.init_acc();
    auto tile_end = [&](Core& c, int k) __attribute__((always_inline)) -> bool {
      const int b = readlane_i(seq_v, k);
      const bool last = k + 1 >= ntiles;
      if (!last && readlane_i(seq_v, k + 1) == b) return true;
      // The wave's tiles of sequence b end here.  The lane index goes through
      // an opaque copy so that the addresses derived from it are computed
      // here, on this rarely taken path, instead of being hoisted out of the
      // loop and held in registers across it.
      int ol = lane;
      asm volatile("" : "+v"(ol));
      const int S0 = readlane_i(s0_v, k);
      const int S1 = S0 + (readlane_i(len_v, k) + kTile - 1) / kTile;
      const float l_tot = c.l_total();
      if (S0 >= wa && S1 <= we) {
        store_rows_final<D>(a, b, h, c.o, 1.f / l_tot, ol);
      } else if (S0 < wa && w > 0) {
#pragma unroll
        for (int x = 0; x < C::NX; ++x) park[((w - 1) * C::NX + x) * kWave + ol] = c.o[x];
        park_m[(w - 1) * kWave + ol] = c.m_run;
        park_l[(w - 1) * kWave + ol] = l_tot;
      } else if (S1 > we && we < r1) {
        keep_b = b;  // the accumulators stay in c until the later waves have parked
        keep_S0 = S0;
        keep_S1 = S1;
      } else {
        store_rows_partial<D>(a, j + b, h, c.o, 1.f / l_tot, c.m_run + log2f(l_tot), ol);
        add_pending(b, S0, S1);
      }
      if (last) return false;
      c.init_acc();
      const int bn = readlane_i(seq_v, k + 1);
      if (bn == b_seg1) {
#pragma unroll
        for (int s = 0; s < C::NK; ++s) c.qv[s] = qn[s];
      } else {
        load_q<D>(a, bn, h, ol, c.qv);
      }
      return true;
    };
    core.template run<FE_DECODE_STAGES>(buf, tile_end);
  }
  __syncthreads();  // parked states are visible

  if (keep_b >= 0) {
    // merge the parked states of the later waves that saw sequence keep_b
    const int end_t = min(keep_S1, r1);
    float M = core.m_run;
    for (int v = w + 1; v < kWaves && wave_begin(v) < end_t; ++v)
      M = fmaxf(M, park_m[(v - 1) * kWave + lane]);
    const float sc0 = core.m_run == kNegInf ? 0.f : exp2f(core.m_run - M);
    float den = sc0 * core.l_total();
#pragma unroll
    for (int x = 0; x < C::NX; ++x) core.o[x] *= sc0;
    for (int v = w + 1; v < kWaves && wave_begin(v) < end_t; ++v) {
      const float mv = park_m[(v - 1) * kWave + lane];
      const float sc = mv == kNegInf ? 0.f : exp2f(mv - M);
      den += sc * park_l[(v - 1) * kWave + lane];
#pragma unroll
      for (int x = 0; x < C::NX; ++x) core.o[x] += sc * park[((v - 1) * C::NX + x) * kWave + lane];
    }
    if (keep_S0 >= r0 && keep_S1 <= r1) {
      store_rows_final<D>(a, keep_b, h, core.o, 1.f / den, lane);
    } else {
      store_rows_partial<D>(a, j + keep_b, h, core.o, 1.f / den, M + log2f(den), lane);
      add_pending(keep_b, keep_S0, keep_S1);
    }
  }
  if (!wg_partial) return;

  // ---- pieces shared with other workgroups: the last of each merges ----
  if (pend_b[0] >= 0 || pend_b[1] >= 0) {
    wait_stores();  // this wave's partials are complete at the device-coherent level
    if (lane == 0) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (pend_b[s] >= 0 &&
            __hip_atomic_fetch_add(a.tickets + pend_b[s] * a.Hkv + h, 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == pend_ns[s] - 1) {
          mflag[3 * s] = pend_b[s];
          mflag[3 * s + 1] = pend_first[s];
          mflag[3 * s + 2] = pend_ns[s];
        }
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int mb = __builtin_amdgcn_readfirstlane(mflag[3 * s]);
    if (mb >= 0) {
      if (tid == 0)
        __hip_atomic_store(a.tickets + mb * a.Hkv + h, 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      merge_pieces<D>(a, mb, h, __builtin_amdgcn_readfirstlane(mflag[3 * s + 1]),
                      __builtin_amdgcn_readfirstlane(mflag[3 * s + 2]));
    }
  }
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

// Pieces (ranges) per KV head the kernel aims for.  Raised above the request
// when the tables allow very long contexts, so that no wave gets more than 64
// tiles (one block-id fetch per wave): a piece of the generic path holds at
// most 64 quads, a range of the equal-tile path at most 256 tiles.
inline int effective_target(int batch, int kv_heads, int max_context, int target_splits) {
  const int target =
      target_splits > 0 ? target_splits : (kDefaultWorkgroups + kv_heads - 1) / kv_heads;
  const int64_t max_quads = ((int64_t)max_context + 63) / 64;
  const int64_t max_tiles = ((int64_t)max_context + kTile - 1) / kTile;
  int64_t need = ((int64_t)batch * max_quads + 63) / 64;
  const int64_t need_tiles = ((int64_t)batch * max_tiles + 255) / 256;
  need = need > need_tiles ? need : need_tiles;
  return need > target ? (int)need : target;
}

template <int D>
size_t piece_lds_bytes() {
  return PieceLds<D>::bytes;
}

// FE_DECODE_LEAN selects the partition of the block-size-16 path: 1 = equal
// tile ranges per workgroup (lean_decode_kernel), 0 = per-sequence pieces.
#ifndef FE_DECODE_LEAN
#define FE_DECODE_LEAN 0
#endif

template <int D>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 piece_grid((a.target + 2 * a.B) * a.Hkv);
  if (a.BS % kTile == 0) {
    if (FE_DECODE_LEAN)
      hipLaunchKernelGGL((lean_decode_kernel<D>), dim3(a.target * a.Hkv), dim3(kThreads),
                         LeanLds<D>::bytes, stream, a);
    else
      hipLaunchKernelGGL((piece_decode_kernel<D, true>), piece_grid, dim3(kThreads),
                         piece_lds_bytes<D>(), stream, a);
  } else {
    hipLaunchKernelGGL((piece_decode_kernel<D, false>), piece_grid, dim3(kThreads),
                       piece_lds_bytes<D>(), stream, a);
  }
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
  if (cascade && (block_size % kTile != 0 || FE_DECODE_LEAN)) return FE_ERR_UNSUPPORTED;
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
