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
#include <algorithm>
#include <mutex>

#include "attn_core.h"

// Diagnostic build only (python -m flexengine_amd.build --timeline, which
// defines FE_TIMELINE and writes libfe_paged_timeline.so): thread 0 of every
// piece_decode_kernel workgroup records s_memrealtime stamps (100 MHz) of its
// phases into fe_tl_stamps, read back by flexengine_amd/timeline_c2.py.  The
// product library compiles the marks to nothing.
#ifdef FE_TIMELINE
constexpr int kTlWgs = 4096;
constexpr int kTlSlots = 16;
__device__ unsigned long long fe_tl_stamps[kTlWgs * kTlSlots];
#define FE_TL_SET(slot, v)                                                     \
  do {                                                                         \
    if (threadIdx.x == 0 && blockIdx.x < kTlWgs)                               \
      fe_tl_stamps[blockIdx.x * kTlSlots + (slot)] = (unsigned long long)(v);  \
  } while (0)
#define FE_TL_MARK(slot) FE_TL_SET(slot, __builtin_amdgcn_s_memrealtime())
#else
#define FE_TL_SET(slot, v) \
  do {                     \
  } while (0)
#define FE_TL_MARK(slot) \
  do {                   \
  } while (0)
#endif

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
  // merges the prefix attention in -- pre_splits slots per query-head row r of
  // normalised outputs (slot s at pre_o + (r*pre_splits + s)*D) and base-2
  // LSEs (pre_lse[r*pre_splits + s]); null and 0 otherwise
  const int32_t* tok0;
  const float* pre_o;
  const float* pre_lse;
  int pre_splits;
  int64_t q_stride;
  int64_t new_stride;
  int W, B, Hq, Hkv, G, BS, bs_log2, NB, target;
  // virtual KV heads per pool head (1, or a group above 16 split into hdiv
  // groups of G query heads: virtual head h reads pool head h / hdiv, whose
  // rows are (Hkv / hdiv) * D elements apart)
  int hdiv;
  // head dims computed as the next of 64 / 128 / 256 (the padded kernels): the
  // real head_dim, by which q, the pools, the new rows and the outputs are laid
  // out; the dims past it are zeros in q and K and never stored
  int dr;
  int max_len;       // W * BS: longest context the tables can address
  float scale_log2;  // softmax scale * log2(e)
  int nwg;           // balanced kernel: workgroups sharing the tile order (= grid size)
  int states;        // balanced kernel: parked-state slots in LDS
  // decode plan (fe_paged_decode_plan): per workgroup item the piece header
  // [kPlanHdr ints], then per item, wave and lane the pool row of the lane's
  // tile; null for the unplanned decode
  int* plan;
  uint32_t plan_key_lo, plan_key_hi;  // plan_key() of the call's sizes and tensors
};

// The decode plan of one step, for items = target + 2 * batch (the grid of the
// piece kernel over kv_heads):
// * a descriptor of kPlanDesc ints: the 64-bit plan_key() of the sizes and
//   tensors it was computed for (the word pair a planned call compares), the
//   same fields in the clear for inspection (magic, batch, kv heads, table
//   stride, block size, pool blocks, target, the block-table and
//   context-length addresses), zero padding, and last the error word the
//   planned kernel sets (kPlanErrSizes, kPlanErrStale);
// * a header per item -- the Piece fields b, id, split, nsplit, L, tok0,
//   tok_begin, tok_end; b = -1 for an item without a piece, whose id field is
//   then the row it zero-fills when inactive;
// * the tile list of each item's four waves (lane k: pool row of tile k).
constexpr int kPlanDesc = 16;
constexpr int kPlanFields = 13;         // key (2 words) + the fields in the clear
constexpr int kPlanHdr = 8;
constexpr int kPlanMagic = 0x46504450;  // "PDPF"
constexpr int kPlanErrSizes = 1;        // error word: the call's sizes are not the plan's
constexpr int kPlanErrStale = 2;        // error word: a row's context length is not the plan's
static_assert((kPlanDesc - 1) * 4 == FE_DECODE_PLAN_ERROR_OFFSET &&
              kPlanErrSizes == FE_PLAN_ERR_SIZES && kPlanErrStale == FE_PLAN_ERR_STALE);
inline size_t plan_bytes(int items) {
  return ((size_t)kPlanDesc + (size_t)items * (kPlanHdr + kWaves * kWave)) * sizeof(int32_t);
}
// The key of the fields a plan is tied to (computed on the host).
inline void set_plan_key(DecodeArgs& a) {
  const uint64_t f[] = {(uint64_t)kPlanMagic, (uint64_t)a.B, (uint64_t)a.Hkv, (uint64_t)a.W,
                        (uint64_t)a.BS, (uint64_t)a.NB, (uint64_t)a.target,
                        (uint64_t)(uintptr_t)a.tables, (uint64_t)(uintptr_t)a.ctx};
  const uint64_t h = plan_key(f, (int)(sizeof(f) / sizeof(f[0])));
  a.plan_key_lo = (uint32_t)h;
  a.plan_key_hi = (uint32_t)(h >> 32);
}

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

// Folds the shared-prefix result of query-head row r (dims d0 .. d0 + 3; every
// slot the prefix launch wrote, loaded in one round trip: a row's slots are
// adjacent) into an online merge state: running maximum M (base 2),
// denominator den and numerator num.  Called for rows with a shared prefix,
// so pre_splits >= 1.
template <int D>
__device__ __forceinline__ void fold_prefix(const DecodeArgs& a, int64_t r, int d0, float& M,
                                            float& den, f32x4& num) {
  const int64_t r0 = r * a.pre_splits;
  float lv[kMaxPrefixSlots];
  f32x4 ov[kMaxPrefixSlots];
  // every load unconditional (slots past the last repeat it and get weight 0):
  // guarded loads were issued one branch at a time, a round trip each
#pragma unroll
  for (int s = 0; s < kMaxPrefixSlots; ++s) {
    const int sc = s < a.pre_splits ? s : a.pre_splits - 1;
    lv[s] = a.pre_lse[r0 + sc];
    ov[s] = *reinterpret_cast<const f32x4*>(a.pre_o + (r0 + sc) * D + d0);
  }
#pragma unroll
  for (int s = 0; s < kMaxPrefixSlots; ++s)
    if (s >= a.pre_splits) lv[s] = kNegInf;
  // no early exit when every slot is -inf (the loads above would sink below
  // it): newM is then M, and alpha 1 (or 0 for a state that is still empty)
  float bm = kNegInf;
#pragma unroll
  for (int s = 0; s < kMaxPrefixSlots; ++s) bm = fmaxf(bm, lv[s]);
  const float newM = fmaxf(M, bm);
  const float alpha = M == kNegInf ? 0.f : exp2f(M - newM);
  num *= alpha;
  den *= alpha;
#pragma unroll
  for (int s = 0; s < kMaxPrefixSlots; ++s) {
    const float wv = lv[s] == kNegInf ? 0.f : exp2f(lv[s] - newM);
    num += wv * ov[s];
    den += wv;
  }
  M = newM;
}

template <int D, class E = Fp16, bool PAD = false>
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
    // the shared-prefix part, written by the launch before this one
    if (pre) fold_prefix<D>(a, (int64_t)b * a.Hq + h * G + hh, (e4 * 4) % D, M, den, num);
    const float inv = 1.f / den;
    if constexpr (PAD) {
      const int d = e4 * 4 - hh * D;  // the partials keep the padded layout
      if (d < a.dr)
        store_out4<E>(a.out, ((int64_t)b * a.Hq + h * G + hh) * a.dr + d, num * inv);
    } else {
      store_out4<E>(a.out, ((int64_t)b * a.Hq + h * G) * D + e4 * 4, num * inv);
    }
  }
}

template <int D, class Core>
__device__ __forceinline__ void setup_core(Core& core, const DecodeArgs& a, const Piece& pc, int h,
                                           unsigned char* stage) {
  const int hp = h / a.hdiv;  // the pool's KV head
  core.trow = a.tables + (int64_t)pc.b * a.W;
  core.rs = (a.Hkv / a.hdiv) * D;
  core.hoff = hp * D;
  core.W = a.W;
  core.NB = a.NB;
  core.BS = a.BS;
  core.bs_log2 = a.bs_log2;
  core.tok_end = pc.tok_end;
  core.limit = pc.tok_end;
  core.scale_log2 = a.scale_log2;
  if (a.k_new != nullptr) {
    core.knew_row = a.k_new + (int64_t)pc.b * a.new_stride + (int64_t)hp * D;
    core.vnew_row = a.v_new + (int64_t)pc.b * a.new_stride + (int64_t)hp * D;
    core.new_pos = pc.L - 1;
  } else {
    core.knew_row = nullptr;
    core.vnew_row = nullptr;
    core.new_pos = -1;
  }
  core.stage = stage;
}

// Tile list of wave w of piece pc (block sizes that are multiples of 16):
// lane k < ntiles gets the pool row (block * BS + offset) of the first key of
// the wave's tile k, i.e. of piece tile w + 4k.
__device__ __forceinline__ int tile_list_row(const DecodeArgs& a, const Piece& pc, int w) {
  const int lane = lane_id();
  const int t_first = pc.tok_begin / kTile + w;
  const int t_end = (pc.tok_end + kTile - 1) / kTile;
  const int ntiles = t_first < t_end ? (t_end - t_first + kWaves - 1) / kWaves : 0;
  const int tok = (t_first + lane * kWaves) * kTile;
  int blk = 0;
  if (lane < ntiles) blk = clamp_block(a.tables[(int64_t)pc.b * a.W + (tok >> a.bs_log2)], a.NB);
  return blk * a.BS + (tok & (a.BS - 1));
}

// The decode plan: workgroup `item` (256 threads) finds its piece as the piece
// kernel would and writes the header and its four waves' tile lists.
__global__ __launch_bounds__(kThreads) void decode_plan_kernel(const DecodeArgs a) {
  const int item = blockIdx.x;
  const int items = a.target + 2 * a.B;
  if (item == 0 && threadIdx.x < kPlanDesc) {
    const int desc[kPlanFields] = {(int)a.plan_key_lo, (int)a.plan_key_hi, kPlanMagic, a.B,
                                   a.Hkv, a.W, a.BS, a.NB, a.target, lo32(a.tables),
                                   hi32(a.tables), lo32(a.ctx), hi32(a.ctx)};
    int v = 0;  // padding and the error word
#pragma unroll
    for (int i = 0; i < kPlanFields; ++i) v = (int)threadIdx.x == i ? desc[i] : v;
    a.plan[threadIdx.x] = v;
  }
  Piece pc;
  int total = 0;
  const bool found = find_piece(a.ctx, nullptr, a.B, a.max_len, a.target, item, pc, total);
  int* hdr = a.plan + kPlanDesc + (int64_t)item * kPlanHdr;
  if (threadIdx.x == 0) {
    hdr[0] = found ? pc.b : -1;
    hdr[1] = found ? pc.id : item - total;
    hdr[2] = found ? pc.split : 0;
    hdr[3] = found ? pc.nsplit : 0;
    hdr[4] = found ? pc.L : 0;
    hdr[5] = found ? pc.tok0 : 0;
    hdr[6] = found ? pc.tok_begin : 0;
    hdr[7] = found ? pc.tok_end : 0;
  }
  if (!found) return;
  const int w = threadIdx.x / kWave;
  a.plan[kPlanDesc + (int64_t)items * kPlanHdr + ((int64_t)item * kWaves + w) * kWave + lane_id()] =
      tile_list_row(a, pc, w);
}

template <int D, bool PAGE16, bool PLANNED = false, class E = Fp16, bool PAD = false>
__global__ __launch_bounds__(kThreads)
// (fp32 and head_dim 256: one wave per SIMD, the rest of the register file held
// as AGPRs -- at two waves D = 256 spilled 168-388 bytes per lane to scratch and
// ran 1.6-1.8x slower)
__attribute__((amdgpu_waves_per_eu(kIsF32<E> || D > 128 ? 1 : (PAGE16 ? FE_DECODE_WAVES_PER_EU : 2),
                                   8)))
void piece_decode_kernel(const DecodeArgs a) {
  using C = TileCfg<D>;
  extern __shared__ __align__(16) unsigned char smem[];

  FE_TL_MARK(0);  // start
  // the real head_dim (layout of q, pools, new rows, outputs)
  const int DR = PAD ? a.dr : D;
  const int h = blockIdx.x % a.Hkv;
  const int item = blockIdx.x / a.Hkv;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Piece pc;
  int planned_row = 0;
  bool found;
  int spare_row;
  bool plan_ok = true;
  if constexpr (PLANNED) {
    // The plan's key, the header and this lane's tile row, all loads in flight
    // at once (the host checked that the plan holds the call's items, so the
    // header and row loads stay inside it whatever the plan is for).  The key's
    // verdict joins `found` instead of branching here: a branch on it would let
    // the compiler sink the header and row loads behind the key's round trip.
    // A plan computed for other sizes or tables addresses other partial slots
    // and rows, so none of it is used (see the spare-workgroup branch).
    const int lane = lane_id();
    const uint32_t key_lo = (uint32_t)a.plan[0], key_hi = (uint32_t)a.plan[1];
    const int* hdr = a.plan + kPlanDesc + (int64_t)item * kPlanHdr;
    planned_row = a.plan[kPlanDesc + (int64_t)(a.target + 2 * a.B) * kPlanHdr +
                         ((int64_t)item * kWaves + w) * kWave + lane];
    const int h0 = hdr[0], h1 = hdr[1], h2 = hdr[2], h3 = hdr[3];
    const int h4 = hdr[4], h5 = hdr[5], h6 = hdr[6], h7 = hdr[7];
    plan_ok = ((key_lo ^ a.plan_key_lo) | (key_hi ^ a.plan_key_hi)) == 0;
    pc.b = __builtin_amdgcn_readfirstlane(h0);
    pc.id = __builtin_amdgcn_readfirstlane(h1);
    pc.split = __builtin_amdgcn_readfirstlane(h2);
    pc.nsplit = __builtin_amdgcn_readfirstlane(h3);
    pc.L = __builtin_amdgcn_readfirstlane(h4);
    pc.tok0 = __builtin_amdgcn_readfirstlane(h5);
    pc.tok_begin = __builtin_amdgcn_readfirstlane(h6);
    pc.tok_end = __builtin_amdgcn_readfirstlane(h7);
    // (the row is consumed here -- the plan kernel never writes a negative row --
    // so that its load is issued beside the header's rather than sunk behind them)
    found = plan_ok & (pc.b >= 0) & (__builtin_amdgcn_readfirstlane(planned_row) >= 0);
    spare_row = pc.id;
  } else {
    int total = 0;
    found = find_piece(a.ctx, a.tok0, a.B, a.max_len, a.target, item, pc, total);
    spare_row = item - total;
  }
  FE_TL_MARK(1);  // the piece is known (plan header, or the partition scan)
  FE_TL_SET(6, found ? 1 : 0);
  if (!found) {
    if (PLANNED && !plan_ok) {
      // not this call's plan: every workgroup of the grid (items >= batch, so one
      // per row and kv head) fills its row's heads with NaN; the error word is set
      if (item < a.B) {
        for (int e = threadIdx.x; e < a.G * DR; e += kThreads)
          store_out1<E>(a.out, ((int64_t)item * a.Hq + h * a.G) * DR + e, __builtin_nanf(""));
      }
      if (item == 0 && h == 0 && threadIdx.x == 0)
        __hip_atomic_store(a.plan + kPlanDesc - 1, kPlanErrSizes, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    // spare workgroup: zero rows of inactive sequences
    const int b = spare_row;
    if (b < a.B && seq_len(a.ctx, b, a.max_len) == 0) {
      for (int e = threadIdx.x; e < a.G * DR; e += kThreads)
        store_out1<E>(a.out, ((int64_t)b * a.Hq + h * a.G) * DR + e, 0.f);
    }
    return;
  }
  using Lds = PieceLds<D>;

  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int G = a.G;
  const int b = pc.b;
  // A plan of the same sizes computed for other context lengths would put the
  // fused page write at a stale position: the row's live length is loaded here
  // (its wait falls after the loop) and a piece whose length is not the plan's
  // writes nothing to the pool and contributes NaN.
  int live_len = pc.L;
  if constexpr (PLANNED) live_len = seq_len(a.ctx, b, a.max_len);
  const int t_first = pc.tok_begin / kTile + w;
  const int t_end = (pc.tok_end + kTile - 1) / kTile;

  float m_run, l_tot;
  f32x4 o[C::NX];
  if constexpr (kIsF32<E>) {
    // fp32 pools: the fp32 engine (tile lists for block sizes that are multiples
    // of 16, a table lookup per key row otherwise; no plan)
    F32Core<D, PAGE16, PAD> core;
    core.k_pool = reinterpret_cast<const float*>(a.k_pool);
    core.v_pool = reinterpret_cast<const float*>(a.v_pool);
    core.k_pool_w = reinterpret_cast<float*>(a.k_pool);
    core.v_pool_w = reinterpret_cast<float*>(a.v_pool);
    core.trow = a.tables + (int64_t)b * a.W;
    core.rs = (a.Hkv / a.hdiv) * DR;
    core.hoff = (h / a.hdiv) * DR;
    core.dr = DR;
    core.W = a.W;
    core.NB = a.NB;
    core.BS = a.BS;
    core.bs_log2 = a.bs_log2;
    core.tok_end = pc.tok_end;
    core.limit = pc.tok_end;
    core.scale_log2 = a.scale_log2;
    core.new_pos = -1;
    core.knew_row = nullptr;
    core.vnew_row = nullptr;
    if (a.k_new != nullptr) {
      const int64_t nr = (int64_t)b * a.new_stride + (int64_t)(h / a.hdiv) * DR;
      core.knew_row = reinterpret_cast<const float*>(a.k_new) + nr;
      core.vnew_row = reinterpret_cast<const float*>(a.v_new) + nr;
      core.new_pos = pc.L - 1;
    }
    {
      const int hq = h * G + (n < G ? n : G - 1);
      const float* qrow =
          reinterpret_cast<const float*>(a.q) + (int64_t)b * a.q_stride + (int64_t)hq * DR;
#pragma unroll
      for (int c = 0; c < F32Core<D, PAGE16, PAD>::NC; ++c) {
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (!PAD || 16 * c + 4 * g < DR) v = *reinterpret_cast<const f32x4*>(qrow + 16 * c + 4 * g);
        core.qv[c] = n < G ? v : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    core.init_acc();
    core.run(t_first, kWaves, t_end);
    m_run = core.m_run;
    l_tot = core.l_total();
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = core.o[x];
  } else {
  f16x8 qv[C::NK];
  {
    const int hq = h * G + (n < G ? n : G - 1);
    const f16* qrow = a.q + (int64_t)b * a.q_stride + (int64_t)hq * DR;
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      if constexpr (PAD) {
        // chunks past the real head_dim are zeros (and not loaded)
        const bool in = (4 * s + g) * 8 < DR;
        const f16x8 v = in ? ld16(qrow + (4 * s + g) * 8) : f16x8{};
        qv[s] = n < G ? v : f16x8{};
      } else {
        const f16x8 v = ld16(qrow + (4 * s + g) * 8);
        qv[s] = n < G ? v : f16x8{};
      }
    }
  }
  if constexpr (PAGE16) {
    // the wave's tiles t_first, t_first + 4, ... of the piece as a tile list
    TileListCore<D, E, PAD> core;
    core.k_pool = a.k_pool;
    core.v_pool = a.v_pool;
    core.rs = (a.Hkv / a.hdiv) * DR;
    core.hoff = (h / a.hdiv) * DR;
    core.nch = DR / 8;
    core.scale_log2 = a.scale_log2;
    core.stage = smem + w * C::STAGE;
    const int ntiles = t_first < t_end ? (t_end - t_first + kWaves - 1) / kWaves : 0;
    core.ntiles = ntiles;
    {
      const int tok = (t_first + lane * kWaves) * kTile;
      const int rem = pc.tok_end - tok;
      if constexpr (PLANNED)
        core.row_vec = planned_row;
      else
        core.row_vec = tile_list_row(a, pc, w);
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
        const f16* kr = a.k_new + (int64_t)b * a.new_stride + (int64_t)(h / a.hdiv) * DR;
        const f16* vr = a.v_new + (int64_t)b * a.new_stride + (int64_t)(h / a.hdiv) * DR;
        if constexpr (PAD) {
#pragma unroll
          for (int s = 0; s < C::NK; ++s)
            core.knew[s] = (4 * s + g) * 8 < DR ? ld16(kr + (4 * s + g) * 8) : f16x8{};
          core.vnew = (lane % C::CPR) * 8 < DR ? ld16(vr + (lane % C::CPR) * 8) : f16x8{};
        } else {
#pragma unroll
          for (int s = 0; s < C::NK; ++s) core.knew[s] = ld16(kr + (4 * s + g) * 8);
          core.vnew = ld16(vr + (lane % C::CPR) * 8);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < C::NK; ++s) core.qv[s] = qv[s];
    core.init_acc();
    core.run();
    if (live_len == pc.L) core.store_new_row(a.k_pool, a.v_pool);
    m_run = core.m_run;
    l_tot = core.l_total();
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = core.o[x];
  } else {
    TileCore<D, E> core;
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
  }
  FE_TL_MARK(2);  // wave 0's tile loop has ended
  FE_TL_SET(7, pc.tok_end - pc.tok_begin);
  FE_TL_SET(8, pc.b);
  FE_TL_SET(9, pc.nsplit);

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
  constexpr int XW = C::NX / kWaves;  // output tiles per wave
  f32x4 ox[XW];
  float M = kNegInf, den = 0.f;
  {
#pragma unroll
    for (int x = 0; x < C::NX; ++x) park[(w * C::NX + x) * kWave + lane] = o[x];
    park_m[w * kWave + lane] = m_run;
    park_l[w * kWave + lane] = l_tot;
    __syncthreads();
#pragma unroll
    for (int v = 0; v < kWaves; ++v) M = fmaxf(M, park_m[v * kWave + lane]);
    float sc[kWaves];
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      const float mv = park_m[v * kWave + lane];
      sc[v] = mv == kNegInf ? 0.f : exp2f(mv - M);
      den += sc[v] * park_l[v * kWave + lane];
    }
    const float inv = 1.f / den;
#pragma unroll
    for (int xi = 0; xi < XW; ++xi) {
      const int x = w * XW + xi;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < kWaves; ++v) acc += sc[v] * park[(v * C::NX + x) * kWave + lane];
      ox[xi] = acc * inv;
    }
  }
  if (PLANNED && live_len != pc.L) {
#pragma unroll
    for (int xi = 0; xi < XW; ++xi) ox[xi] = f32x4{1.f, 1.f, 1.f, 1.f} * __builtin_nanf("");
    if (threadIdx.x == 0)
      __hip_atomic_store(a.plan + kPlanDesc - 1, kPlanErrStale, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  FE_TL_MARK(3);  // the four waves are combined
  const int hq = h * G + (n < G ? n : G - 1);
  if (!split) {
    if (n < G) {
      const int64_t orow = ((int64_t)b * a.Hq + hq) * DR + 4 * g;
#pragma unroll
      for (int xi = 0; xi < XW; ++xi)
        if (!PAD || 16 * (w * XW + xi) + 4 * g < DR)
          store_out4<E>(a.out, orow + 16 * (w * XW + xi), ox[xi]);
    }
    FE_TL_MARK(4);  // output stores issued
    return;
  }
  // device-coherent (sc1) 16-byte stores of this piece's partial output and LSE
  auto store_partial = [&]() __attribute__((always_inline)) {
    if (n >= G) return;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        a.ws_o + ((int64_t)pc.id * a.Hq + h * G) * D, 0, G * D * (int)sizeof(float), 0x00020000);
    const uint32_t off = (uint32_t)((n * D + 4 * g) * sizeof(float));
#pragma unroll
    for (int xi = 0; xi < XW; ++xi)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ox[xi]), r,
                                             off + 16 * (w * XW + xi) * (uint32_t)sizeof(float),
                                             0, kSc1);
    if (w == 0 && g == 0) store_coherent(a.ws_lse + (int64_t)pc.id * a.Hq + hq, M + log2f(den));
  };
  // ---- split-K: every piece stores its partial and waits for it before its
  // ticket; the last piece of (b, h) to finish merges them all ----
  int* const ticket = a.tickets + b * a.Hkv + h;
  store_partial();
  wait_stores();  // this wave's partials are complete at the device-coherent level
  __syncthreads();
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            pc.nsplit - 1;
  __syncthreads();
  FE_TL_MARK(4);  // partial stored, ticket drawn
  FE_TL_SET(6, *flag ? 7 : 3);
  if (!*flag) return;
  if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  merge_pieces<D, E, PAD>(a, b, h, pc.id - pc.split, pc.nsplit, pc.tok0 > 0);
  FE_TL_MARK(5);  // merge stores issued
}

// ---- balanced decode (block sizes that are multiples of 16) ----------------------
//
// Runs the suffix pass of the shared-prefix decode at large batches (many short
// private suffixes, each read once: its page loads are non-temporal).
//
// Work is cut at 16-token tile granularity over one global order of all
// (sequence, KV head, tile) triples -- sequence-major, then KV head, then
// tile -- so every workgroup receives the same number of tiles whatever the
// context-length mix.  The grid is one 512-thread workgroup (8 waves) per
// compute unit, and each workgroup asks for more than half of the CU's LDS so
// that no CU receives two: the HBM bandwidth a CU achieves does not grow with
// the number of workgroups it holds, so equal bytes per CU is what balances
// the launch.
//
// Workgroup w owns tiles [w*T/N, (w+1)*T/N) of the order (T tiles in total, N
// workgroups), and each of its waves a contiguous eighth of that range.  A
// wave's tiles may cross from one (sequence, KV head) "segment" into the
// next: it parks the finished segment's state (o, m, l of its live query
// heads) in an LDS slot and goes on without waiting for the other waves, its
// next tile's loads still in flight.  After the loop the workgroup meets once
// and combines every segment from the slots of the waves that touched it.  A
// segment entirely inside the range is written directly as fp16; the first
// and last segment of a range can be shared with the neighbouring
// workgroups, and those go through the split-K ticket protocol of the piece
// kernel (partials with device-coherent stores, the last contributing
// workgroup merges).  The queries of all segments of the range are staged in
// LDS during set-up, alongside the block-table loads.  A range with more
// segments than there are slots (many very short sequences) falls back to
// combining each segment as soon as all waves are past it, with a barrier
// per segment.
constexpr int kBThreads = 512;
constexpr int kBWaves = kBThreads / kWave;
constexpr int kBMaxBatch = 2048;      // per-sequence arrays kept in LDS
constexpr int kBMaxTilesPerWave = 64; // a wave's tile list is held one tile per lane
constexpr int kBMinLds = 84 * 1024;   // > half of a CU's 160 KB: one workgroup per CU

// Compact parked state of one wave for one segment: o of the G live columns
// ([NX][4][G] x 16 bytes, the MFMA register layout), then m[G] and l[G].
__host__ __device__ constexpr int bstate_bytes(int D, int G) {
  return ((D / 16) * 4 * G * 16 + 2 * G * 4 + 15) & ~15;
}

template <int D>
struct BLds {
  static constexpr size_t stage = 0;
  static constexpr size_t misc = stage + (size_t)kBWaves * TileCfg<D>::STAGE;  // 64 ints
  static constexpr size_t arrays = misc + 64 * sizeof(int);
  // arrays: tile prefix P[B+1], context lengths Ls[B], suffix starts S0[B];
  // then each wave's second-segment queries [8][NK][64 lanes] x 16 bytes,
  // then parked states [states][bstate_bytes]
  static constexpr size_t kQw = (size_t)TileCfg<D>::NK * kWave * 16;
  __host__ __device__ static size_t qw_off(int B) {
    return (arrays + (size_t)(3 * B + 1) * sizeof(int) + 15) & ~size_t(15);
  }
  __host__ __device__ static size_t states_off(int B) { return qw_off(B) + kBWaves * kQw; }
  static size_t bytes(int B, int G, int states) {
    const size_t n = states_off(B) + (size_t)states * bstate_bytes(D, G);
    return n > (size_t)kBMinLds ? n : (size_t)kBMinLds;
  }
};

template <int D, class E = Fp16>
__global__ __launch_bounds__(kBThreads) void balanced_decode_kernel(const DecodeArgs a) {
  using C = TileCfg<D>;
  using Lds = BLds<D>;
  extern __shared__ __align__(16) unsigned char smem[];
  int* misc = reinterpret_cast<int*>(smem + Lds::misc);
  int* P = reinterpret_cast<int*>(smem + Lds::arrays);
  int* Ls = P + a.B + 1;
  int* S0 = Ls + a.B;
  unsigned char* states = smem + Lds::states_off(a.B);
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int G = a.G;
  const int Hkv = a.Hkv;
  const int SB = bstate_bytes(D, G);
  unsigned char* qw = smem + Lds::qw_off(a.B) + w * Lds::kQw;  // this wave's query area

  // ---- tiles of every sequence and their exclusive prefix sum, in LDS ----
  int carry = 0;
  for (int base = 0; base < a.B; base += kBThreads) {
    const int b = base + tid;
    int L = 0, t0 = 0;
    if (b < a.B) {
      L = seq_len(a.ctx, b, a.max_len);
      t0 = suffix_start(a.tok0, b, L);
      Ls[b] = L;
      S0[b] = t0;
    }
    const int nt = (L - t0 + kTile - 1) / kTile;
    const int incl = wave_scan_incl_i(nt);
    if (lane == kWave - 1) misc[w] = incl;
    __syncthreads();
    int off = carry, tot = 0;
#pragma unroll
    for (int v = 0; v < kBWaves; ++v) {
      const int c = misc[v];
      off += v < w ? c : 0;
      tot += c;
    }
    if (b < a.B) P[b] = off + incl - nt;
    carry += tot;
    __syncthreads();
  }
  carry = __builtin_amdgcn_readfirstlane(carry);
  if (tid == 0) P[a.B] = carry;
  __syncthreads();

  // rows of inactive sequences are zeros (every launched workgroup takes a share)
  for (int b = blockIdx.x; b < a.B; b += gridDim.x) {
    if (Ls[b] == 0) {
      for (int e = tid; e < a.Hq * D; e += kBThreads) a.out[(int64_t)b * a.Hq * D + e] = (f16)0.f;
    }
  }
  const int T = Hkv * carry;
  // at least one tile per wave: tiny batches use fewer workgroups
  int nwg = a.nwg;
  if (T / kBWaves < nwg) nwg = T / kBWaves > 0 ? T / kBWaves : 1;
  const int wg = blockIdx.x;
  if (T == 0 || wg >= nwg) return;
  const int lo = (int)((int64_t)wg * T / nwg);
  const int hi = (int)((int64_t)(wg + 1) * T / nwg);

  // the workgroup whose range holds tile x
  auto wg_of = [&](int x) { return (int)(((int64_t)(x + 1) * nwg + T - 1) / T) - 1; };
  auto seg_start = [&](int sg) {
    const int b = sg / Hkv;
    return Hkv * P[b] + (sg - b * Hkv) * (P[b + 1] - P[b]);
  };

  // ---- this wave's contiguous share of the range, one tile per lane ----
  const int R = hi - lo;  // >= kBWaves unless the whole batch has fewer tiles
  const int wlo = lo + (w * R) / kBWaves;
  const int whi = lo + ((w + 1) * R) / kBWaves;
  const int ntiles = whi - wlo;
  // One pass of binary searches: lane k < ntiles locates tile wlo + k; lanes
  // 0..7 (8..15) also locate the first (last) tile of wave lane % 8, so every
  // wave knows all waves' segments -- its state slots -- without a barrier.
  int b1, b2;
  {
    const int x1 = wlo + (lane < ntiles ? lane : 0);
    const int v = lane & (kBWaves - 1);
    const int x2 = lane < kBWaves ? lo + (v * R) / kBWaves : lo + ((v + 1) * R) / kBWaves - 1;
    int l1 = 0, r1 = a.B - 1, l2 = 0, r2 = a.B - 1;
    while (l1 < r1 || l2 < r2) {
      const int m1 = (l1 + r1 + 1) >> 1, m2 = (l2 + r2 + 1) >> 1;
      const int p1 = Hkv * P[m1], p2 = Hkv * P[m2];
      if (l1 < r1) {
        if (p1 <= x1) l1 = m1;
        else r1 = m1 - 1;
      }
      if (l2 < r2) {
        if (p2 <= x2) l2 = m2;
        else r2 = m2 - 1;
      }
    }
    b1 = l1;
    b2 = l2;
  }
  int row_vec = 0, rows_vec = 0, seg_vec = 0x7fffffff, newrow_vec = -1;
  if (lane < ntiles) {
    const int b = b1;
    const int nt = P[b + 1] - P[b];
    const int r = wlo + lane - Hkv * P[b];
    const int h = r / nt;
    const int t = r - h * nt;
    const int L = Ls[b];
    const int tok = S0[b] + kTile * t;
    const int rem = L - tok;
    const int blk = clamp_block(a.tables[(int64_t)b * a.W + (tok >> a.bs_log2)], a.NB);
    row_vec = blk * a.BS + (tok & (a.BS - 1));
    rows_vec = rem < kTile ? rem : kTile;
    seg_vec = b * Hkv + h;
    if (a.k_new != nullptr && rem <= kTile) newrow_vec = rem - 1;
  }
  auto load_qg = [&](int sg, f16x8 (&dst)[C::NK]) {
    const int hh = n < G ? n : G - 1;
    const int b = sg / Hkv;
    const f16* qrow = a.q + (int64_t)b * a.q_stride + (int64_t)((sg - b * Hkv) * G + hh) * D;
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      const f16x8 v = ld16(qrow + (4 * s + g) * 8);
      dst[s] = n < G ? v : f16x8{};
    }
  };
  // the wave's first two segments (their queries load alongside the tables);
  // a wave without tiles (ranges shorter than 8) has none
  const int sa = ntiles > 0 ? __builtin_amdgcn_readlane(seg_vec, 0) : 0x7fffffff;
  int s2 = 0x7fffffff;
  {
    const unsigned long long other = __ballot(lane < ntiles && seg_vec != sa);
    if (other) s2 = __builtin_amdgcn_readlane(seg_vec, __builtin_ctzll(other));
  }
  int bnd = -1;  // -1: wave lane % 8 holds no tiles
  {
    const int nt = P[b2 + 1] - P[b2];
    const int v = lane & (kBWaves - 1);
    const int vlo = lo + (v * R) / kBWaves;
    const int vhi = lo + ((v + 1) * R) / kBWaves;
    const int x2 = lane < kBWaves ? vlo : vhi - 1;
    if (vhi > vlo) bnd = b2 * Hkv + (x2 - Hkv * P[b2]) / (nt > 0 ? nt : 1);
  }
  int wsa[kBWaves], wsb[kBWaves], wslot[kBWaves];
  int nstates = 0, s_first = 0x7fffffff, s_last = -1;
#pragma unroll
  for (int v = 0; v < kBWaves; ++v) {
    wsa[v] = __builtin_amdgcn_readlane(bnd, v);
    wsb[v] = __builtin_amdgcn_readlane(bnd, kBWaves + v);
    if (wsa[v] < 0) {
      wsa[v] = 0x7fffffff;
      wsb[v] = -1;
    }
    wslot[v] = nstates;
    if (wsb[v] >= wsa[v]) {
      nstates += wsb[v] - wsa[v] + 1;
      s_first = wsa[v] < s_first ? wsa[v] : s_first;
      s_last = wsb[v];
    }
  }
  int sb = -1, slot0 = 0;
#pragma unroll
  for (int v = 0; v < kBWaves; ++v) {
    if (v == w) {
      sb = wsb[v];
      slot0 = wslot[v];
    }
  }
  // slot mode: every wave's states fit the LDS state slots; otherwise one
  // barrier per segment (slots 0..7)
  const bool slots = nstates <= a.states;
  f16x8 qv[C::NK], q2[C::NK];
  int cur = slots ? sa : s_first;
  if (!slots || ntiles > 0) load_qg(cur, qv);
  if (!slots || sb == sa) s2 = 0x7fffffff;
  if (s2 != 0x7fffffff) load_qg(s2, q2);

  auto seg_tiles = [&](int sg) {
    const int b = sg / Hkv;
    return P[b + 1] - P[b];
  };
  // next segment after sg holding at least one tile (sequences with no keys hold none)
  auto next_seg = [&](int sg) {
    for (++sg; sg <= s_last; ++sg)
      if (seg_tiles(sg) > 0) break;
    return sg;
  };

  const int rs = Hkv * D;
  unsigned char* stage = smem + Lds::stage + w * C::STAGE;
  auto tile_rows = [&](int k) {
    const int r = __builtin_amdgcn_readlane(rows_vec, k & (kWave - 1));
    return k < ntiles ? r : 0;
  };
  auto tile_seg = [&](int k) { return __builtin_amdgcn_readlane(seg_vec, k & (kWave - 1)); };
  auto tile_base = [&](int k) {
    const int s = tile_seg(k);
    const int h = s - (s / Hkv) * Hkv;
    return (int64_t)__builtin_amdgcn_readlane(row_vec, k & (kWave - 1)) * rs + h * D;
  };
  auto tile_newrow = [&](int k) {
    return k < ntiles ? __builtin_amdgcn_readlane(newrow_vec, k & (kWave - 1)) : -1;
  };
  auto rsrc = [&](const f16* pool, int64_t base, int rows) {
    const uint64_t addr = reinterpret_cast<uint64_t>(pool + base);
    const uint32_t lo32 = __builtin_amdgcn_readfirstlane((uint32_t)addr);
    const uint32_t hi32 = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
    const int nrec = __builtin_amdgcn_readfirstlane(rows * rs * 2);
    void* p = reinterpret_cast<void*>(((uint64_t)hi32 << 32) | lo32);
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, nrec, 0x00020000);
  };
  const uint32_t k_off0 = (uint32_t)(((lane & 15) * rs + (lane >> 4) * 8) * 2);
  const uint32_t v_off0 = (uint32_t)(((lane / C::CPR) * rs + (lane % C::CPR) * 8) * 2);
  const int vrow = lane / C::CPR;

  // Issues the K/V loads of tile k (zero extent past the list).  The tile
  // holding the decoded token takes that row from k_new / v_new instead of
  // the pool, in the same batch of loads.
  auto load_tile = [&](int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) {
    const int64_t base = tile_base(k);
    const int rows = tile_rows(k);
    const __amdgpu_buffer_rsrc_t kr = rsrc(a.k_pool, base, rows);
    const __amdgpu_buffer_rsrc_t vr = rsrc(a.v_pool, base, rows);
    const int nr = tile_newrow(k);
    if (nr < 0) {
#pragma unroll
      for (int s = 0; s < C::NK; ++s)
        kk[s] = __builtin_bit_cast(
            f16x8, __builtin_amdgcn_raw_buffer_load_b128(kr, k_off0, s * 64, kStreamPolicy));
#pragma unroll
      for (int j = 0; j < C::NK; ++j)
        vv[j] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                              vr, v_off0, j * C::RPI * rs * 2, kStreamPolicy));
    } else {
      const int sg = tile_seg(k);
      const int b = sg / Hkv;
      const int h = sg - b * Hkv;
      const f16* kn = a.k_new + (int64_t)b * a.new_stride + h * D;
      const f16* vn = a.v_new + (int64_t)b * a.new_stride + h * D;
#pragma unroll
      for (int s = 0; s < C::NK; ++s) {
        if ((lane & 15) == nr)
          kk[s] = ld16(kn + (4 * s + g) * 8);
        else
          kk[s] = __builtin_bit_cast(
              f16x8, __builtin_amdgcn_raw_buffer_load_b128(kr, k_off0, s * 64, kStreamPolicy));
      }
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        if (j * C::RPI + vrow == nr)
          vv[j] = ld16(vn + (lane % C::CPR) * 8);
        else
          vv[j] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                                vr, v_off0, j * C::RPI * rs * 2, kStreamPolicy));
      }
    }
  };

  // ---- per-segment state ----
  auto load_q = [&](int sg) {
    if (sg == s2) {
#pragma unroll
      for (int s = 0; s < C::NK; ++s) qv[s] = *reinterpret_cast<const f16x8*>(qw + (s * kWave + lane) * 16);
    } else {
      load_qg(sg, qv);
    }
  };
  float m_run = kNegInf, l_run = 0.f;
  f32x4 o[C::NX];
  auto reset = [&]() {
    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  reset();

  // parks this wave's state in a slot (live columns only)
  auto park = [&](int slot) {
    float l_tot = l_run + shfl_xor_f(l_run, 16);
    l_tot += shfl_xor_f(l_tot, 32);
    unsigned char* st = states + slot * SB;
    if (n < G) {
#pragma unroll
      for (int x = 0; x < C::NX; ++x)
        *reinterpret_cast<f32x4*>(st + ((x * 4 + g) * G + n) * 16) = o[x];
      if (g == 0) {
        float* ml = reinterpret_cast<float*>(st + C::NX * 4 * G * 16);
        ml[n] = m_run;
        ml[G + n] = l_tot;
      }
    }
  };

  // Combines segments s_first + j, j0 <= j < j1, from the parked slots of the
  // waves that touched them and writes them: fp16 output for a segment inside
  // the range, a partial (normalised o and base-2 LSE, device-coherent) for a
  // shared one.  One thread per (segment, 16-byte output chunk).
  auto combine = [&](int j0, int j1, bool by_wave) {
    constexpr int kNE = C::NX * 4;  // 16-byte chunks of one query head's output
    const int ne = kNE * G;
    for (int it = tid; it < (j1 - j0) * ne; it += kBThreads) {
      const int sg = s_first + j0 + it / ne;
      if (seg_tiles(sg) == 0) continue;
      const int e = it % ne;
      const int nn = e % G;
      const int xg = e / G;  // x * 4 + g: dims 16x + 4g .. +3
      const int b = sg / Hkv;
      const int h = sg - b * Hkv;
      int sl[kBWaves];
      float mv[kBWaves];
      float M = kNegInf;
#pragma unroll
      for (int v = 0; v < kBWaves; ++v) {
        const int slot = by_wave ? v : (wsa[v] <= sg && sg <= wsb[v] ? wslot[v] + sg - wsa[v] : -1);
        sl[v] = slot;
        mv[v] = slot >= 0 ? reinterpret_cast<const float*>(states + slot * SB + kNE * G * 16)[nn]
                          : kNegInf;
        M = fmaxf(M, mv[v]);
      }
      float den = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < kBWaves; ++v) {
        if (mv[v] == kNegInf) continue;
        const unsigned char* st = states + sl[v] * SB;
        const float sc = exp2f(mv[v] - M);
        den += sc * reinterpret_cast<const float*>(st + kNE * G * 16)[G + nn];
        acc += sc * *reinterpret_cast<const f32x4*>(st + (xg * G + nn) * 16);
      }
      acc *= 1.f / den;
      const float lse = M + log2f(den);
      const int64_t r = (int64_t)b * a.Hq + h * G + nn;
      const int d0 = (xg >> 2) * 16 + (xg & 3) * 4;
      const int start = seg_start(sg);
      if (start >= lo && start + seg_tiles(sg) <= hi) {
        if (S0[b] > 0) {  // fold in the shared-prefix result of the launch before
          float M = lse, dsum = 1.f;
          fold_prefix<D>(a, r, d0, M, dsum, acc);
          if (dsum > 0.f) acc *= 1.f / dsum;
        }
        *reinterpret_cast<f16x4*>(a.out + r * D + d0) = to16x4<E>(acc);
      } else {
        const int slot = 2 * wg + (sg == s_first ? 0 : 1);
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            a.ws_o + (int64_t)slot * G * D, 0, G * D * (int)sizeof(float), 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc), ro,
                                               (uint32_t)((nn * D + d0) * sizeof(float)), 0,
                                               kSc1);
        if (xg == 0) store_coherent(a.ws_lse + slot * G + nn, lse);
      }
    }
  };

  // barrier mode: all waves park in slot w, meet, combine, move on together
  auto finish = [&]() {
    park(w);
    __syncthreads();
    combine(cur - s_first, cur - s_first + 1, true);
    cur = next_seg(cur);
    if (cur <= s_last) load_q(cur);
    __syncthreads();
    reset();
  };

  // One tile: scores, V staging, softmax and PV.  In slot mode a tile of a
  // later segment first parks the current one.
  auto step = [&](int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK], bool switching) {
    if (switching) {
      const int sk = tile_seg(k);
      if (sk != cur) {
        park(slot0 + cur - sa);
        cur = sk;
        load_q(cur);
        reset();
      }
    }
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      sacc = mma16<E>(lo4(kk[s]), lo4(qv[s]), sacc);
      sacc = mma16<E>(hi4(kk[s]), hi4(qv[s]), sacc);
    }
    compiler_fence();
    {
      const int cv = lane % C::CPR;
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        unsigned char* dst = stage + (j * C::RPI + vrow) * C::ROWB + cv * 16;
        *reinterpret_cast<f16x8*>(dst) = vv[j];
      }
    }
    compiler_fence();
    softmax_pv_tile<D, E>(sacc, 0, tile_rows(k), a.scale_log2, stage, m_run, l_run, o);
    compiler_fence();
    const int nr = tile_newrow(k);
    if (nr >= 0) {  // write the decoded token's row to the pool
      char* kb = reinterpret_cast<char*>(a.k_pool + tile_base(k));
      char* vb = reinterpret_cast<char*>(a.v_pool + tile_base(k));
      if ((lane & 15) == nr) {
#pragma unroll
        for (int s = 0; s < C::NK; ++s)
          *reinterpret_cast<f16x8*>(kb + k_off0 + s * 64) = kk[s];
      }
#pragma unroll
      for (int j = 0; j < C::NK; ++j)
        if (j * C::RPI + vrow == nr)
          *reinterpret_cast<f16x8*>(vb + v_off0 + j * C::RPI * rs * 2) = vv[j];
    }
  };

  // Tiles k0 .. k1-1 of the list with one tile of prefetch (loads past k1
  // have zero extent, so every wait is exact).
  auto run = [&](int k0, int k1, bool switching) {
    f16x8 ka[C::NK], va[C::NK], kb[C::NK], vb[C::NK];
    auto ld = [&](int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) {
      if (k < k1) load_tile(k, kk, vv);
      else load_tile(ntiles, kk, vv);
    };
    ld(k0, ka, va);
    if (switching && s2 != 0x7fffffff) {
      // the second segment's queries go to the wave's LDS area once the first
      // tile's loads are in flight (they were issued before those loads)
#pragma unroll
      for (int s = 0; s < C::NK; ++s)
        *reinterpret_cast<f16x8*>(qw + (s * kWave + lane) * 16) = q2[s];
    }
    for (int k = k0;; k += 2) {
      ld(k + 1, kb, vb);
      if (k >= k1) break;
      step(k, ka, va, switching);
      ld(k + 2, ka, va);
      if (k + 1 >= k1) break;
      step(k + 1, kb, vb, switching);
    }
  };
  if (slots) {
    // one pipeline across the wave's segments; states parked as it goes
    run(0, ntiles, true);
    if (ntiles > 0) park(slot0 + cur - sa);
    __syncthreads();
    combine(0, s_last - s_first + 1, false);
  } else {
    // a pipeline per segment, the workgroup meeting after each
    int k0 = 0;
    while (cur <= s_last) {
      const int k1 = k0 + __builtin_popcountll(__ballot(lane < ntiles && seg_vec == cur));
      run(k0, k1, false);
      k0 = k1;
      finish();
    }
  }

  // ---- split segments: the last contributing workgroup merges ----
  // the segments combine() wrote as partials: s_first (side 0) and s_last
  // (side 1) when they reach past the range
  const bool st0 = seg_start(s_first) < lo || seg_start(s_first) + seg_tiles(s_first) > hi;
  const bool st1 = s_last != s_first && seg_start(s_last) + seg_tiles(s_last) > hi;
  if (!st0 && !st1) return;
  wait_stores();
  __syncthreads();
  int* flag = misc + 40;
  if (tid < 2) {
    const int side = tid;
    flag[side] = 0;
    if (side == 0 ? st0 : st1) {
      const int sg = side == 0 ? s_first : s_last;
      const int start = seg_start(sg);
      const int nsplit = wg_of(start + seg_tiles(sg) - 1) - wg_of(start) + 1;
      flag[side] = __hip_atomic_fetch_add(a.tickets + sg, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
    }
  }
  __syncthreads();
  const int n4 = G * D / 4;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.ws_o, 0, 2 * nwg * G * D * (int)sizeof(float), 0x00020000);
  // both merges at once: item = side * n4 + e4
  for (int item = tid; item < 2 * n4; item += kBThreads) {
    const int side = item >= n4 ? 1 : 0;
    if (!flag[side]) continue;
    const int e4 = item - side * n4;
    const int sg = side == 0 ? s_first : s_last;
    const int b = sg / Hkv;
    const int h = sg - b * Hkv;
    const int start = seg_start(sg);
    const int w0 = wg_of(start);
    const int ns = wg_of(start + seg_tiles(sg) - 1) - w0 + 1;
    // the first contributor kept the segment in side 1 when its range began earlier
    const int side0 = (int)((int64_t)w0 * T / nwg) < start ? 1 : 0;
    if (e4 == 0) __hip_atomic_store(a.tickets + sg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int hh = e4 * 4 / D;
    float M = kNegInf, den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += kMergeBatch) {
      const int nb = ns - s0 < kMergeBatch ? ns - s0 : kMergeBatch;
      float lv[kMergeBatch];
      f32x4 ov[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        lv[u] = kNegInf;
        ov[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (u < nb) {
          const int c = s0 + u;
          const int slot = 2 * (w0 + c) + (c == 0 ? side0 : 0);
          lv[u] = load_coherent(a.ws_lse + slot * G + hh);
          ov[u] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         ro, (uint32_t)((slot * G * D + e4 * 4) * sizeof(float)), 0, kSc1));
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
    const int64_t r = (int64_t)b * a.Hq + h * G;
    if (S0[b] > 0) fold_prefix<D>(a, r + hh, (e4 * 4) % D, M, den, num);  // the shared prefix
    const float inv = 1.f / den;
    *reinterpret_cast<f16x4*>(a.out + r * D + e4 * 4) = to16x4<E>(num * inv);
  }
}

// General LSE merge of S partial results (natural-log LSE at the boundary).
template <class E>
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
    out[(int64_t)r * D + d] = to16<E>(num / den);
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

// Compute units and LDS bytes per workgroup of the current device (queried
// once per device).
struct DeviceLimits {
  int cus;
  int lds;
};
DeviceLimits device_limits() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  static DeviceLimits cache[64] = {};
  if (dev >= 0 && dev < 64 && cache[dev].cus > 0) return cache[dev];
  DeviceLimits d{0, 0};
  if (hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      d.cus <= 0)
    d.cus = 256;
  if (hipDeviceGetAttribute(&d.lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
          hipSuccess ||
      d.lds <= 0)
    d.lds = 64 * 1024;
  if (dev >= 0 && dev < 64) cache[dev] = d;
  return d;
}

#ifndef FE_DECODE_BALANCED
#define FE_DECODE_BALANCED 1
#endif
// The balanced kernel runs the suffix pass of the shared-prefix decode for
// batches of this many rows and more: there it measured faster than the piece
// kernel (B = 256 with 8 groups of 32 sharing 2048 tokens: 83 vs 99 us per
// step; its suffixes are many and short).  The plain decode keeps the piece
// kernel at every batch size: with default-cached loads it measured faster
// (same B = 256 batch without the cascade: 110 vs 115 us; B = 8: 7.1 vs
// 11.5 us; B = 64: 20.8 vs 25.0 us).
#ifndef FE_DECODE_BALANCED_MIN_BATCH
#define FE_DECODE_BALANCED_MIN_BATCH 128
#endif

// Launch shape of the balanced kernel for these sizes; nwg = 0 when the piece
// kernel handles them (block size below 16, very large batches, LDS too
// small, or partials that do not fit the workspace that
// fe_paged_decode_workspace_size describes).
struct BalancedPlan {
  int nwg = 0;
  int states = 0;
  size_t lds = 0;
};
template <int D>
BalancedPlan plan_balanced(int batch, int hkv, int G, int block_size, int max_len,
                           size_t ws_limit) {
  BalancedPlan p;
  if (!FE_DECODE_BALANCED || block_size % kTile != 0 || batch > kBMaxBatch ||
      batch < FE_DECODE_BALANCED_MIN_BATCH)
    return p;
  const DeviceLimits dl = device_limits();
  const size_t cap = dl.lds < 160 * 1024 ? (size_t)dl.lds : (size_t)160 * 1024;
  const size_t sb = bstate_bytes(D, G);
  const size_t base = BLds<D>::states_off(batch);
  if (base + (size_t)kBWaves * sb > cap) return p;  // the barrier fallback needs 8 slots
  int states = (int)((cap - base) / sb);
  if (states > 64) states = 64;
  const int64_t tiles_max = (int64_t)hkv * batch * ((max_len + kTile - 1) / kTile);
  const int64_t per_wg = (int64_t)kBWaves * kBMaxTilesPerWave;
  int64_t n = dl.cus;
  if ((tiles_max + per_wg - 1) / per_wg > n) n = (tiles_max + per_wg - 1) / per_wg;
  const size_t need = kTicketBytes + align256((size_t)2 * n * G * D * sizeof(float)) +
                      align256((size_t)2 * n * G * sizeof(float));
  if (n > (1 << 20) || need > ws_limit) return p;
  p.nwg = (int)n;
  p.states = states;
  p.lds = BLds<D>::bytes(batch, G, states);
  return p;
}

template <int D, class E>
int launch_decode(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((a.target + 2 * a.B) * a.Hkv);
  if constexpr (kIsF32<E>) {
    // fp32 pools: the fp32 engine, unplanned
    if (a.BS % kTile == 0)
      hipLaunchKernelGGL((piece_decode_kernel<D, true, false, E>), grid, dim3(kThreads),
                         PieceLds<D>::bytes, stream, a);
    else
      hipLaunchKernelGGL((piece_decode_kernel<D, false, false, E>), grid, dim3(kThreads),
                         PieceLds<D>::bytes, stream, a);
  } else if (a.nwg > 0) {
    hipLaunchKernelGGL((balanced_decode_kernel<D, E>), dim3(a.nwg), dim3(kBThreads),
                       BLds<D>::bytes(a.B, a.G, a.states), stream, a);
  } else if (a.plan != nullptr) {
    hipLaunchKernelGGL((piece_decode_kernel<D, true, true, E>), grid, dim3(kThreads),
                       PieceLds<D>::bytes, stream, a);
  } else if (a.BS % kTile == 0) {
    hipLaunchKernelGGL((piece_decode_kernel<D, true, false, E>), grid, dim3(kThreads),
                       PieceLds<D>::bytes, stream, a);
  } else {
    hipLaunchKernelGGL((piece_decode_kernel<D, false, false, E>), grid, dim3(kThreads),
                       PieceLds<D>::bytes, stream, a);
  }
  return FE_LAUNCH_STATUS();
}

// Padded head dims, unplanned: 16-bit pools with block sizes that are multiples
// of 16, fp32 pools (D 64 / 128) at any block size.
template <int D, class E>
int launch_decode_padded(const DecodeArgs& a, hipStream_t stream) {
  const dim3 grid((a.target + 2 * a.B) * a.Hkv);
  if (a.BS % kTile == 0)
    hipLaunchKernelGGL((piece_decode_kernel<D, true, false, E, true>), grid, dim3(kThreads),
                       PieceLds<D>::bytes, stream, a);
  else if constexpr (kIsF32<E>)
    hipLaunchKernelGGL((piece_decode_kernel<D, false, false, E, true>), grid, dim3(kThreads),
                       PieceLds<D>::bytes, stream, a);
  return FE_LAUNCH_STATUS();
}

}  // namespace

// The generic kernel's split partials: [batch * hq][splits] outputs and LSEs
inline size_t generic_ws_bytes(int batch, int hq, int d, int splits) {
  return align256((size_t)batch * hq * splits * d * sizeof(float)) +
         align256((size_t)batch * hq * splits * sizeof(float));
}
constexpr int kGenericWsSplits = 16;  // splits per row the workspace size allows for

extern "C" size_t fe_paged_decode_workspace_size(int batch, int num_q_heads, int head_dim,
                                                 int max_context, int target_splits) {
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || max_context < 0 || target_splits < 0)
    return 0;
  // sized for the largest default (kv_heads = 1): valid for every kv_heads
  const int target = effective_target(batch, 1, max_context, target_splits);
  // the padded kernels keep their partials at the computed head_dim
  const size_t pieces = kTicketBytes +
                        ws_o_bytes(batch, num_q_heads, mfma_padded_head_dim(head_dim), target) +
                        ws_lse_bytes(batch, num_q_heads, target);
  // head dims other than 64 / 128 run on the generic kernel: room for its splits
  if (head_dim != 64 && head_dim != 128) {
    const size_t gen =
        kTicketBytes + generic_ws_bytes(batch, num_q_heads, head_dim, kGenericWsSplits);
    return gen > pieces ? gen : pieces;
  }
  return pieces;
}

namespace {

bool aligned_to(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }
constexpr int kGenericWorkgroups = 2048;  // the generic decode's default launch size

// Shapes the matrix-core decode does not take (head_dim other than 64 / 128,
// or more than 16 query heads per KV head): the generic kernel, no plan.  Each
// row's keys are cut into as many splits as fit the workspace region the
// piece partials would use ((target + batch) rows of partials: 1 + target /
// batch splits per row, at most 32 and one per 64 keys of the table width).
// A shared-prefix call lands here as a plain decode: every row attends its own
// table, whose first pages are the shared ones, so the result is the same.
int decode_generic(const void* q, int64_t q_batch_stride, void* out, const void* k_new,
                   const void* v_new, int64_t new_batch_stride, void* k_pool, void* v_pool,
                   int num_blocks, const int32_t* block_tables, int table_stride,
                   const int32_t* context_lens, void* workspace, size_t workspace_bytes,
                   int batch, int num_q_heads, int kv_heads, int head_dim, int block_size,
                   float scale, int target_splits, hipStream_t stream, bool planned, int elem) {
  if (!generic_shape(num_q_heads, kv_heads, head_dim) || planned) return FE_ERR_UNSUPPORTED;
  if (log2_exact(block_size) < 0) return FE_ERR_UNSUPPORTED;
  // key indices and pool rows (block * block_size + offset) are 32-bit in the kernel
  if ((int64_t)table_stride * block_size >= ((int64_t)1 << 31) ||
      (int64_t)num_blocks * block_size >= ((int64_t)1 << 31))
    return FE_ERR_UNSUPPORTED;
  if (batch == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && context_lens);
  FE_CHECK_ARG((k_new == nullptr) == (v_new == nullptr));
  const size_t el = elem == 2 ? 4 : 2;
  FE_CHECK_ARG(q_batch_stride >= (int64_t)num_q_heads * head_dim);
  FE_CHECK_ARG(aligned_to(q, el) && aligned_to(out, el) && aligned_to(k_pool, el) &&
               aligned_to(v_pool, el));
  if (k_new) {
    FE_CHECK_ARG(new_batch_stride >= (int64_t)kv_heads * head_dim && aligned_to(k_new, el) &&
                 aligned_to(v_new, el));
  }
  const int max_len = table_stride * block_size;
  const int target = effective_target(batch, kv_heads, max_len, target_splits);
  const size_t need = fe_paged_decode_workspace_size(batch, num_q_heads, head_dim, max_len, target);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return FE_ERR_WORKSPACE;
  // key splits per row: about kGenericWorkgroups workgroups in all (or
  // target_splits per KV head when given), no more than the documented
  // workspace size holds (so a larger workspace does not change the result)
  // nor one per 64 keys of the table width
  const int64_t want = target_splits > 0 ? (int64_t)target_splits * kv_heads : kGenericWorkgroups;
  int64_t splits = (want + (int64_t)batch * kv_heads - 1) / ((int64_t)batch * kv_heads);
  splits = std::min<int64_t>(splits, kGenericWsSplits);
  splits = std::min<int64_t>(splits, (max_len + 63) / 64);
  while (splits > 1 &&
         kTicketBytes + generic_ws_bytes(batch, num_q_heads, head_dim, (int)splits) > need)
    --splits;
  if (splits < 1) splits = 1;
  GenericAttn g{};
  g.splits = (int)splits;
  // past the split-K tickets, which the other decode kernels need at zero and
  // this one leaves alone
  char* const parts = (char*)workspace + kTicketBytes;
  g.part_o = (float*)parts;
  g.part_lse =
      (float*)(parts + align256((size_t)batch * num_q_heads * splits * head_dim * sizeof(float)));
  g.q = q;
  g.q_stride = q_batch_stride;
  g.out = out;
  g.out_stride = (int64_t)num_q_heads * head_dim;
  g.k_new = k_new;
  g.v_new = v_new;
  g.new_stride = new_batch_stride;
  g.k_pool = k_pool;
  g.v_pool = v_pool;
  g.num_blocks = num_blocks;
  g.tables = block_tables;
  g.table_stride = table_stride;
  g.ctx = context_lens;
  g.q_offsets = nullptr;
  g.num_seqs = batch;
  g.rows = batch;
  g.hq = num_q_heads;
  g.hkv = kv_heads;
  g.d = head_dim;
  g.bs = block_size;
  g.scale = scale;
  g.elem = elem;
  return generic_attention(g, stream);
}

// Everything fe_paged_decode and fe_paged_decode_shared_prefix share: argument
// checks, workspace carving and the decode launch.  `cascade` (null for plain
// decode) is filled with the workspace regions of the shared-prefix half and
// launched first.
int decode_impl(const void* q, int64_t q_batch_stride, void* out, const void* k_new,
                const void* v_new, int64_t new_batch_stride, void* k_pool, void* v_pool,
                int num_blocks, const int32_t* block_tables, int table_stride,
                const int32_t* context_lens, void* workspace, size_t workspace_bytes, int batch,
                int num_q_heads, int kv_heads, int head_dim, int block_size, float scale,
                int target_splits, CascadePrefix* cascade, hipStream_t stream,
                void* plan = nullptr, size_t plan_len = 0, bool bf16 = false,
                bool f32 = false) {
  FE_CHECK_ARG(batch >= 0 && num_q_heads > 0 && kv_heads > 0 && num_blocks > 0 &&
               table_stride > 0 && target_splits >= 0);
  // fp32 pools: the unplanned piece kernel only (no plan; a shared-prefix call
  // runs its suffix pass on the piece kernel too)
  if (f32 && plan != nullptr) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  const int G = num_q_heads / kv_heads;
  // the shared-prefix kernels take head_dim 64 / 128 and groups <= 16: at other
  // shapes a shared-prefix call is a plain decode of every row over its own
  // table (whose first pages are the shared ones), on whichever kernel takes it
  if (cascade && ((head_dim != 64 && head_dim != 128) || G > kMaxGroup)) cascade = nullptr;
  // head_dim 256 in 16 bits runs on the piece kernel too (unplanned, no shared
  // prefix; one wave per SIMD with its spills in AGPRs: 1.9-2.4x the generic
  // kernel's rate)
  const bool mfma256 = head_dim == 256 && !f32 && plan == nullptr && cascade == nullptr;
  // a group above 16 (unplanned, no shared prefix) is split into hdiv virtual
  // KV heads of G / hdiv <= 16 query heads, each reading its pool head's K/V;
  // splits that would leave fewer than 8 query heads per read of the K/V (a
  // group with no divisor in 8..16) stay on the generic kernel
  int hdiv = 1;
  if (G > kMaxGroup && plan == nullptr && cascade == nullptr) {
    for (int v = 2; v <= G; ++v) {
      if (G % v == 0 && G / v <= kMaxGroup) {
        if (G / v >= 8) hdiv = v;
        break;
      }
    }
  }
  const int hkv_v = kv_heads * hdiv;  // KV heads as the kernels see them
  const int G_v = G / hdiv;
  // other multiples of 8 below 256 (16-bit, unplanned, no shared prefix, pages
  // of 16k tokens): the piece kernel at the next of 64 / 128 / 256, the dims
  // past head_dim zeros in q and K and never stored
  // (fp32: the fp32 engine at 64 / 128, any block size; padded to 128 only when
  // head_dim fills 3/4 of it -- the engine runs one wave per SIMD there, and at
  // D 80 (32/8) it measured 186.5 us against the generic kernel's 173.0)
  const int dpad = mfma_padded_head_dim(head_dim);
  const bool padded = dpad != head_dim && plan == nullptr && cascade == nullptr &&
                      (f32 ? dpad == 64 || (dpad == 128 && 4 * head_dim >= 3 * dpad)
                           : block_size % kTile == 0);
  if ((head_dim != 64 && head_dim != 128 && !mfma256 && !padded) || G_v > kMaxGroup)
    return decode_generic(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                          num_blocks, block_tables, table_stride, context_lens, workspace,
                          workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size,
                          scale, target_splits, stream, plan != nullptr, bf16 ? 1 : (f32 ? 2 : 0));
  if ((int64_t)batch * hkv_v > kMaxTickets) return FE_ERR_UNSUPPORTED;
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
  const int target = effective_target(batch, hkv_v, max_len, target_splits);
  const int dc = padded ? dpad : head_dim;  // head_dim as computed
  if ((int64_t)(target + batch) * num_q_heads * dc * (int64_t)sizeof(float) >= ((int64_t)1 << 31))
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
  ws += ws_o_bytes(batch, num_q_heads, dc, target);
  a.ws_lse = (float*)ws;
  a.tok0 = nullptr;
  a.pre_o = nullptr;
  a.pre_lse = nullptr;
  a.pre_splits = 0;
  a.q_stride = q_batch_stride;
  a.new_stride = new_batch_stride;
  a.W = table_stride;
  a.B = batch;
  a.Hq = num_q_heads;
  a.Hkv = hkv_v;
  a.G = G_v;
  a.hdiv = hdiv;
  a.dr = head_dim;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.target = target;
  a.max_len = max_len;
  a.scale_log2 = scale * kLog2e;
  // the balanced kernel's partials ([2N][G][D] and [2N][G]) replace the piece
  // partials inside the same region of the workspace
  a.nwg = 0;
  a.states = 0;
  a.plan = nullptr;
  if (plan != nullptr) {
    // the planned piece kernel: tile lists need block sizes that are multiples of 16
    if (cascade || block_size % kTile != 0) return FE_ERR_UNSUPPORTED;
    if (plan_len < plan_bytes(target + 2 * batch) || !aligned16(plan)) return FE_ERR_WORKSPACE;
    a.plan = (int*)plan;
    set_plan_key(a);
  }
  if (cascade && !f32) {  // the balanced kernel has 16-bit forms only
    const BalancedPlan bp =
        head_dim == 64 ? plan_balanced<64>(batch, kv_heads, G, block_size, max_len, need)
                       : plan_balanced<128>(batch, kv_heads, G, block_size, max_len, need);
    a.nwg = bp.nwg;
    a.states = bp.states;
  }
  if (a.nwg > 0)
    a.ws_lse = a.ws_o + align256((size_t)2 * a.nwg * G * head_dim * sizeof(float)) / sizeof(float);
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
    c.bf16 = bf16;
    c.f32 = f32;
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
    a.pre_o = c.out_o;
    a.pre_lse = c.out_lse;
    a.pre_splits = c.splits;
  }
  if (f32 && padded)
    return dpad == 64 ? launch_decode_padded<64, F32>(a, s) : launch_decode_padded<128, F32>(a, s);
  if (f32) return head_dim == 64 ? launch_decode<64, F32>(a, s) : launch_decode<128, F32>(a, s);
  if (padded) {
    if (dpad == 64)
      return bf16 ? launch_decode_padded<64, Bf16>(a, s) : launch_decode_padded<64, Fp16>(a, s);
    if (dpad == 128)
      return bf16 ? launch_decode_padded<128, Bf16>(a, s) : launch_decode_padded<128, Fp16>(a, s);
    return bf16 ? launch_decode_padded<256, Bf16>(a, s) : launch_decode_padded<256, Fp16>(a, s);
  }
  if (head_dim == 256) return bf16 ? launch_decode<256, Bf16>(a, s) : launch_decode<256, Fp16>(a, s);
  if (bf16) return head_dim == 64 ? launch_decode<64, Bf16>(a, s) : launch_decode<128, Bf16>(a, s);
  return head_dim == 64 ? launch_decode<64, Fp16>(a, s) : launch_decode<128, Fp16>(a, s);
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

extern "C" size_t fe_paged_decode_plan_size(int batch, int kv_heads, int max_context,
                                            int target_splits) {
  if (batch < 0 || kv_heads <= 0 || max_context < 0 || target_splits < 0) return 0;
  return plan_bytes(effective_target(batch, kv_heads, max_context, target_splits) + 2 * batch);
}

extern "C" int fe_paged_decode_plan(const int32_t* block_tables, int table_stride,
                                    const int32_t* context_lens, int num_blocks, int batch,
                                    int kv_heads, int block_size, int target_splits, void* plan,
                                    size_t plan_len, fe_stream_t stream) {
  FE_CHECK_ARG(batch >= 0 && kv_heads > 0 && num_blocks > 0 && table_stride > 0 &&
               target_splits >= 0);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0 || block_size % kTile != 0) return FE_ERR_UNSUPPORTED;
  if ((int64_t)table_stride * block_size > 262144) return FE_ERR_UNSUPPORTED;
  if (batch == 0) return FE_OK;
  FE_CHECK_ARG(block_tables && context_lens);
  const int max_len = table_stride * block_size;
  const int target = effective_target(batch, kv_heads, max_len, target_splits);
  if (plan == nullptr || plan_len < plan_bytes(target + 2 * batch) || !aligned16(plan))
    return FE_ERR_WORKSPACE;
  DecodeArgs a{};
  a.tables = block_tables;
  a.ctx = context_lens;
  a.W = table_stride;
  a.B = batch;
  a.Hkv = kv_heads;
  a.hdiv = 1;
  a.dr = 0;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.target = target;
  a.max_len = max_len;
  a.plan = (int*)plan;
  set_plan_key(a);
  hipLaunchKernelGGL(decode_plan_kernel, dim3(target + 2 * batch), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_paged_decode_planned(const void* q, int64_t q_batch_stride, void* out,
                                       const void* k_new, const void* v_new,
                                       int64_t new_batch_stride, void* k_pool, void* v_pool,
                                       int num_blocks, const int32_t* block_tables,
                                       int table_stride, const int32_t* context_lens,
                                       void* workspace, size_t workspace_bytes, int batch,
                                       int num_q_heads, int kv_heads, int head_dim,
                                       int block_size, float scale, int target_splits,
                                       void* plan, size_t plan_len, fe_stream_t stream) {
  if (plan == nullptr) return FE_ERR_INVALID_ARGUMENT;
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, nullptr, (hipStream_t)stream, plan, plan_len);
}

extern "C" int fe_paged_decode_bf16(const void* q, int64_t q_batch_stride, void* out,
                                    const void* k_new, const void* v_new,
                                    int64_t new_batch_stride, void* k_pool, void* v_pool,
                                    int num_blocks, const int32_t* block_tables, int table_stride,
                                    const int32_t* context_lens, void* workspace,
                                    size_t workspace_bytes, int batch, int num_q_heads,
                                    int kv_heads, int head_dim, int block_size, float scale,
                                    int target_splits, fe_stream_t stream) {
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, nullptr, (hipStream_t)stream, nullptr, 0, true);
}

extern "C" int fe_paged_decode_f32(const void* q, int64_t q_batch_stride, void* out,
                                   const void* k_new, const void* v_new,
                                   int64_t new_batch_stride, void* k_pool, void* v_pool,
                                   int num_blocks, const int32_t* block_tables, int table_stride,
                                   const int32_t* context_lens, void* workspace,
                                   size_t workspace_bytes, int batch, int num_q_heads,
                                   int kv_heads, int head_dim, int block_size, float scale,
                                   int target_splits, fe_stream_t stream) {
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, nullptr, (hipStream_t)stream, nullptr, 0, false, true);
}

extern "C" int fe_paged_decode_planned_bf16(const void* q, int64_t q_batch_stride, void* out,
                                            const void* k_new, const void* v_new,
                                            int64_t new_batch_stride, void* k_pool, void* v_pool,
                                            int num_blocks, const int32_t* block_tables,
                                            int table_stride, const int32_t* context_lens,
                                            void* workspace, size_t workspace_bytes, int batch,
                                            int num_q_heads, int kv_heads, int head_dim,
                                            int block_size, float scale, int target_splits,
                                            void* plan, size_t plan_len,
                                            fe_stream_t stream) {
  if (plan == nullptr) return FE_ERR_INVALID_ARGUMENT;
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, nullptr, (hipStream_t)stream, plan, plan_len, true);
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

namespace {

int shared_prefix_impl(const void* q, int64_t q_batch_stride, void* out, const void* k_new,
                       const void* v_new, int64_t new_batch_stride, void* k_pool, void* v_pool,
                       int num_blocks, const int32_t* block_tables, int table_stride,
                       const int32_t* context_lens, const int32_t* group_offsets,
                       const int32_t* group_prefix_lens, int num_groups, void* workspace,
                       size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
                       int head_dim, int block_size, float scale, int target_splits,
                       fe_stream_t stream, bool bf16, bool f32 = false) {
  FE_CHECK_ARG(num_groups >= 0 && num_groups <= batch + 1);
  if (num_groups == 0 || batch == 0)
    return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                       num_blocks, block_tables, table_stride, context_lens, workspace,
                       workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                       target_splits, nullptr, (hipStream_t)stream, nullptr, 0, bf16, f32);
  FE_CHECK_ARG(group_offsets && group_prefix_lens);
  CascadePrefix c{};
  c.group_offsets = group_offsets;
  c.prefix_len = group_prefix_lens;
  c.num_groups = num_groups;
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, workspace,
                     workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size, scale,
                     target_splits, &c, (hipStream_t)stream, nullptr, 0, bf16, f32);
}

}  // namespace

extern "C" int fe_paged_decode_shared_prefix(
    const void* q, int64_t q_batch_stride, void* out, const void* k_new, const void* v_new,
    int64_t new_batch_stride, void* k_pool, void* v_pool, int num_blocks,
    const int32_t* block_tables, int table_stride, const int32_t* context_lens,
    const int32_t* group_offsets, const int32_t* group_prefix_lens, int num_groups,
    void* workspace, size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
    int head_dim, int block_size, float scale, int target_splits, fe_stream_t stream) {
  return shared_prefix_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool,
                            v_pool, num_blocks, block_tables, table_stride, context_lens,
                            group_offsets, group_prefix_lens, num_groups, workspace,
                            workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size,
                            scale, target_splits, stream, false);
}

extern "C" int fe_paged_decode_shared_prefix_bf16(
    const void* q, int64_t q_batch_stride, void* out, const void* k_new, const void* v_new,
    int64_t new_batch_stride, void* k_pool, void* v_pool, int num_blocks,
    const int32_t* block_tables, int table_stride, const int32_t* context_lens,
    const int32_t* group_offsets, const int32_t* group_prefix_lens, int num_groups,
    void* workspace, size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
    int head_dim, int block_size, float scale, int target_splits, fe_stream_t stream) {
  return shared_prefix_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool,
                            v_pool, num_blocks, block_tables, table_stride, context_lens,
                            group_offsets, group_prefix_lens, num_groups, workspace,
                            workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size,
                            scale, target_splits, stream, true);
}

extern "C" int fe_paged_decode_shared_prefix_f32(
    const void* q, int64_t q_batch_stride, void* out, const void* k_new, const void* v_new,
    int64_t new_batch_stride, void* k_pool, void* v_pool, int num_blocks,
    const int32_t* block_tables, int table_stride, const int32_t* context_lens,
    const int32_t* group_offsets, const int32_t* group_prefix_lens, int num_groups,
    void* workspace, size_t workspace_bytes, int batch, int num_q_heads, int kv_heads,
    int head_dim, int block_size, float scale, int target_splits, fe_stream_t stream) {
  return shared_prefix_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool,
                            v_pool, num_blocks, block_tables, table_stride, context_lens,
                            group_offsets, group_prefix_lens, num_groups, workspace,
                            workspace_bytes, batch, num_q_heads, kv_heads, head_dim, block_size,
                            scale, target_splits, stream, false, true);
}

// ---------------------------------------------------------------------------
// Allocation-free decode (fe_paged_decode_noalloc)
// ---------------------------------------------------------------------------

namespace {

// fe_paged_decode_noalloc's split-K tickets and partials: one copy of this
// array per GPU, zero-initialised when the code object is loaded and held
// until the process ends.  Host code never uses the name itself (on the host
// it is a stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES];

__global__ void clear_words_kernel(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

struct ScratchTable {
  std::mutex mu;
  void* ptr[64] = {};
};
ScratchTable& scratch_table() {
  static ScratchTable t;
  return t;
}

// Device address of the current device's scratch.  The first call on a device
// looks it up and clears the ticket region with a fill kernel on `stream` (a
// kernel rather than hipMemsetAsync, so a first call under graph capture
// records a kernel node); every later call finds the tickets at zero because
// each decode leaves them so.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= 64) return FE_ERR_UNSUPPORTED;
  ScratchTable& t = scratch_table();
  std::lock_guard<std::mutex> lock(t.mu);
  if (t.ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr || !aligned16(p)) return (int)hipErrorInvalidSymbol;
    hipLaunchKernelGGL(clear_words_kernel, dim3(64), dim3(256), 0, stream, (int*)p,
                       (int)(kTicketBytes / sizeof(int)));
    const int rc = FE_LAUNCH_STATUS();
    if (rc != FE_OK) return rc;
    t.ptr[dev] = p;
  }
  *out = t.ptr[dev];
  return FE_OK;
}

}  // namespace

extern "C" int fe_paged_decode_noalloc(const void* q, int64_t q_batch_stride, void* out,
                                       const void* k_new, const void* v_new,
                                       int64_t new_batch_stride, void* k_pool, void* v_pool,
                                       int num_blocks, const int32_t* block_tables,
                                       int table_stride, const int32_t* context_lens, int batch,
                                       int num_q_heads, int kv_heads, int head_dim,
                                       int block_size, float scale, int target_splits,
                                       fe_stream_t stream) {
  // the scratch the call would need, checked before anything is launched
  // (decode_impl validates the remaining arguments the same way as for
  // fe_paged_decode)
  if (batch > 0 && num_q_heads > 0 && kv_heads > 0 && head_dim > 0 && table_stride > 0 &&
      block_size > 0 && target_splits >= 0 &&
      (int64_t)table_stride * block_size <= 262144) {
    const int max_len = table_stride * block_size;
    const int target = effective_target(batch, kv_heads, max_len, target_splits);
    if (fe_paged_decode_workspace_size(batch, num_q_heads, head_dim, max_len, target) >
        (size_t)FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES)
      return FE_ERR_SCRATCH_LIMIT;
  }
  void* ws = nullptr;
  if (batch > 0) {
    const int rc = scratch_for_current_device((hipStream_t)stream, &ws);
    if (rc != FE_OK) return rc;
  }
  return decode_impl(q, q_batch_stride, out, k_new, v_new, new_batch_stride, k_pool, v_pool,
                     num_blocks, block_tables, table_stride, context_lens, ws,
                     (size_t)FE_PAGED_DECODE_NOALLOC_SCRATCH_BYTES, batch, num_q_heads,
                     kv_heads, head_dim, block_size, scale, target_splits, nullptr,
                     (hipStream_t)stream);
}

namespace {

template <class E>
int lse_merge_impl(const float* part_out, const float* part_lse, int num_splits, int rows,
                   int head_dim, void* out, float* out_lse, fe_stream_t stream) {
  FE_CHECK_ARG(num_splits > 0 && rows >= 0 && head_dim > 0);
  if (rows == 0) return FE_OK;
  FE_CHECK_ARG(part_out && part_lse && out);
  const int threads = head_dim >= 256 ? 256 : (head_dim >= 128 ? 128 : 64);
  hipLaunchKernelGGL(lse_merge_kernel<E>, dim3(rows), dim3(threads), 0, (hipStream_t)stream,
                     part_out, part_lse, num_splits, rows, head_dim, (f16*)out, out_lse);
  return FE_LAUNCH_STATUS();
}

}  // namespace

extern "C" int fe_lse_merge(const float* part_out, const float* part_lse, int num_splits,
                            int rows, int head_dim, void* out, float* out_lse,
                            fe_stream_t stream) {
  return lse_merge_impl<Fp16>(part_out, part_lse, num_splits, rows, head_dim, out, out_lse,
                              stream);
}

extern "C" int fe_lse_merge_bf16(const float* part_out, const float* part_lse, int num_splits,
                                 int rows, int head_dim, void* out, float* out_lse,
                                 fe_stream_t stream) {
  return lse_merge_impl<Bf16>(part_out, part_lse, num_splits, rows, head_dim, out, out_lse,
                              stream);
}

#ifdef FE_TIMELINE
// Diagnostic build only (not declared in include/): the stamps of the last
// launches, and their reset.
extern "C" int fe_timeline_read(void* host, int wgs) {
  if (wgs < 0 || wgs > kTlWgs) return FE_ERR_INVALID_ARGUMENT;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(fe_tl_stamps),
                                  (size_t)wgs * kTlSlots * sizeof(unsigned long long));
}
extern "C" int fe_timeline_clear() {
  static unsigned long long zeros[kTlWgs * kTlSlots];
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(fe_tl_stamps), zeros, sizeof(zeros));
}
#endif
