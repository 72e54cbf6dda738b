// Ragged chunked-prefill attention over paged KV for gfx950 (MI355X).
//
// Every sequence s contributes n_s new query rows (q_offsets[s] ..
// q_offsets[s+1]) that sit at absolute positions ctx_s - n_s .. ctx_s - 1 and
// attend causally to keys t <= position over the paged K/V of the sequence
// (the new rows' own K/V are already in the pool).
//
// Work decomposition.  For one KV head h, the query rows of a sequence are the
// pairs (position, query head of the group) flattened position-major: row
// r -> position r / G, query head h*G + r % G.  A workgroup (4 waves) owns
// 64*RT consecutive rows of one sequence and KV head, so all G query heads of
// the group share every K/V block it loads.  K/V are walked in blocks of 32
// keys: the workgroup stages a block in LDS (double-buffered; the next block's
// global loads, and the block ids of the one after, are in flight while the
// current one is computed, one barrier
// per block), and every wave computes its RT tiles of 16 rows against it:
//
//   S^T[16 keys x 16 rows] = K . Q^T    v_mfma_f32_16x16x32_f16, k = 32 dims
//     A = K: lane (g,n) reads key n, dims 32c + 8g .. +7 (16 bytes, LDS)
//     B = Q: lane (g,n) holds row n's query, same dims (registers)
//   base-2 online softmax with lazy rescale (attn_core.h), causal mask only on
//   the blocks that cross the workgroup's first position
//   O^T[16 dims x 16 rows] += V^T . P^T  v_mfma_f32_16x16x32_f16, k = 32 keys
//     B = P^T: lane (g,n) holds keys 4g..4g+3 of two 16-key tiles (the score
//       layout itself), A = V^T: two transposing LDS reads (ds_read_b64_tr_b16)
//       give lane (g,n) the same keys for dim n.
//
// Key splits: when the row blocks alone give too few workgroups to fill the
// chip, grid.z = KS workgroups share a row block, each taking an equal share
// of its key blocks.  A split writes its normalised fp32 partial output and
// base-2 LSE with device-coherent stores, waits for them, and draws a ticket
// of (row block, KV head); the last split to arrive merges the KS partials
// into the fp16 output and resets the ticket, so the workspace needs no clear
// between calls.
//
// The reference runs a materialized gather + SDPA per request for every
// multi-token chunk (src/flexengine/inference/attention/paged.py:27-40,
// called per request from qwen2.py:117-126).
#include "attn_core.h"

using namespace fe;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// Keys staged per block (a multiple of 32).  64 measured slower: its LDS stages
// leave two workgroups per CU instead of four (C4: ~70 vs ~59 us).
constexpr int kBlockKeys = 32;
constexpr int kKT = kBlockKeys / 16;    // 16-key S tiles per block
constexpr int kPS = kBlockKeys / 32;    // 32-key PV steps per block
// Key splits per row block (plan() clamps to it).  The merge loads all kMaxSplits
// slots at once, so the bound is also its load count: 4 measured best (C4 prefill
// 55 us; 8: 61 us, 8 with loads only for the live splits: 57.5 us, 2: 63 us; the
// C3 shared-prefix decode 81 us at 4 and 8, 91 us at 2).
constexpr int kMaxSplits = 4;
static_assert(kMaxSplits <= kMaxPrefixSlots, "the cascade prefix writes one slot per key split");
// Rows of the split merge whose partials are loaded in one round trip: the C3
// shared-prefix pass took 24.15 us with 1 (a round trip per 8 rows), 23.79 with
// 2, 23.06 with 4 and 23.14 with 8.
constexpr int kMergeRows = 4;
// Two 16-row tiles per wave (RT = 2) once the rows fill this many 128-row blocks;
// below it the extra blocks of RT = 1 fill the CUs better (measured: 1377 new tokens
// x 12 heads run slower with RT = 2).
constexpr int kRt2Blocks = 512;

template <int D, int RT>
struct PCfg {
  static constexpr int NC = D / 32;                 // 32-dim k-chunks of QK^T
  static constexpr int NX = D / 16;                 // 16-dim output tiles
  static constexpr int KP = D * 2 + 16;             // K row pitch in LDS (bytes)
  static constexpr int VP = D * 2 + 32;             // V row pitch (transposing reads)
  static constexpr int KBYTES = kBlockKeys * KP;
  static constexpr int STAGE = KBYTES + kBlockKeys * VP;
  static constexpr int ROWS = kWaves * 16 * RT;     // rows per workgroup
  static constexpr int CPR = D / 8;                 // 16-byte chunks per K/V row
  static constexpr int KPL = kThreads / CPR;        // key rows covered by one load round
  static constexpr int LOADS = kBlockKeys / KPL;    // load rounds per matrix per block
};

struct PrefillArgs {
  const f16* q;
  f16* out;
  const f16* k_pool;
  const f16* v_pool;
  const int32_t* tables;
  const int32_t* q_off;
  const int32_t* ctx;
  float* part_o;     // [KS][total_q * Hq][D] normalised partial outputs (KS > 1); the
                     // stream-K kernel's partials [2 * nwg_max * 128][D]
  float* part_lse;   // [KS][total_q * Hq] base-2 LSE of each partial
  int* tickets;      // [row blocks * Hkv] (stream-K kernel: [nwg_max]), zero between calls
  // stream-K kernel: the step's plan (fe_prefill_plan), null to derive the
  // work split in the launch, and the key of the call's sizes and tensors
  int* plan;
  uint32_t plan_key_lo, plan_key_hi;
  int64_t q_stride;  // elements from one query row (token or sequence) to the next
  int W, S, total_q, Hq, Hkv, G, BS, bs_log2, NB, KS;
  int nwg_max;       // stream-K kernel: workgroups of the launch
  int dr;            // padded tile kernel: the real head_dim (layout of q, pools, out)
  float scale_log2;
  // shared-prefix (cascade) mode: "sequence" s is a group of decode rows
  // q_off[s] .. q_off[s+1]-1 sharing the first prefix_len[s] keys of row
  // q_off[s]'s table; the result per (row, query head) is an fp32 output
  // normalised over those keys plus its base-2 LSE (pre_o, pre_lse), and
  // tok0[b] (for every decode row b < total_q) receives the first key the
  // row's own decode still has to attend.
  const int32_t* prefix_len;
  float* pre_o;      // [total_q * Hq][D]
  float* pre_lse;    // [total_q * Hq]
  int32_t* tok0;     // [total_q]
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // buffer-instruction cache policy: sc1 (device-coherent)

struct RowBlock {
  int s;      // sequence
  int rb;     // row block of the sequence
  int n;      // new rows (positions) of the sequence
  int q0;     // first query row of the sequence in q/out
  int ctx;    // context length (cached + new)
};

// Shared prefix of group s as the kernels use it: whole blocks only.
__device__ __forceinline__ int group_prefix(const PrefillArgs& a, int s) {
  return clamp_len(a.prefix_len[s]) & ~(a.BS - 1);
}

// Context length of decode row b in cascade mode, clamped to what the table
// addresses (the decode kernel clamps the same way).
__device__ __forceinline__ int member_len(const PrefillArgs& a, int b) {
  const int L = clamp_len(a.ctx[b]);
  return L < a.W * a.BS ? L : a.W * a.BS;
}

// Maps a workgroup id onto (sequence, row block); false past the last block.
template <int ROWS, bool CASCADE>
__device__ __forceinline__ bool locate_rows(const PrefillArgs& a, int item, RowBlock& rb) {
  const int lane = lane_id();
  int carry = 0;
  for (int base = 0; base < a.S; base += kWave) {
    const int s = base + lane;
    int q0 = 0, n = 0, cx = 0;
    if (s < a.S) {
      // rows outside [0, total_q) are dropped: every row the kernel touches
      // (q, out, the context and table of a decode row) stays in its array
      q0 = min(max(a.q_off[s], 0), a.total_q);
      n = min(a.q_off[s + 1], a.total_q) - q0;
      n = n > 0 ? n : 0;
      // the context length (group prefix) loaded with the offsets: the hit
      // lane's is read below without another round trip
      cx = CASCADE ? group_prefix(a, s) : clamp_len(a.ctx[s]);
    }
    const int nb = (n * a.G + ROWS - 1) / ROWS;
    const int incl = wave_scan_incl_i(nb) + carry;
    const int excl = incl - nb;
    const unsigned long long hit = __ballot(s < a.S && item >= excl && item < incl);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      rb.s = base + src;
      rb.rb = item - readlane_i(excl, src);
      rb.n = readlane_i(n, src);
      rb.q0 = readlane_i(q0, src);
      rb.ctx = readlane_i(cx, src);
      return true;
    }
    carry = readlane_i(incl, kWave - 1);
  }
  return false;
}

// Cascade mode: the decode row b shares group s's prefix when its context
// reaches past it; its own decode then starts at the prefix end.  Written by
// one workgroup for every decode row (0 = no shared prefix).  offs: the group
// offsets q_off[0 .. S], in global memory or a copy in LDS.
template <class Offs>
__device__ void write_suffix_starts(const PrefillArgs& a, Offs offs) {
  for (int b = threadIdx.x; b < a.total_q; b += blockDim.x) {
    int lo = 0, hi = a.S;  // last group s with q_off[s] <= b
    while (hi - lo > 1) {
      const int mid = (lo + hi) / 2;
      if (offs[mid] <= b) lo = mid; else hi = mid;
    }
    int t = 0;
    if (a.S > 0 && offs[lo] <= b && b < offs[lo + 1]) {
      const int pl = group_prefix(a, lo);
      t = member_len(a, b) > pl ? pl : 0;
    }
    a.tok0[b] = t;
  }
}

// The end of a key split of the tile kernel.  Lane (g, n) holds
// O[row n][dims 16x + 4g + i] of its RT row tiles, the row's running maximum
// m_run (base 2) and its sum l.  One split: normalise and store.  Several:
// write this split's partial (device-coherent stores), draw the row block's
// ticket; the last split merges all of them.
template <int D, int RT, class E, bool PAD = false, int DC = D>
__device__ __forceinline__ void finish_split(const PrefillArgs& a, const RowBlock& rb, int item,
                                             int h, int ks, int wr0, int r0, int r_last,
                                             const bool (&valid)[RT], const float (&m_run)[RT],
                                             const float (&l)[RT], const f32x4 (&o)[RT][DC / 16],
                                             int* last) {
  constexpr int NX = DC / 16;  // output tiles computed
  const int DR = PAD ? a.dr : D;  // output row length
  const int G = a.G;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const bool split = a.KS > 1;
  const int64_t split_stride = (int64_t)a.total_q * a.Hq;  // rows per split
  // (only used when split; the host keeps KS * rows * D floats under 2 GiB)
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.part_o, 0, split ? (int)(a.KS * split_stride * D * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      a.part_lse, 0, split ? (int)(a.KS * split_stride * 4) : 0, 0x00020000);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    if (!valid[rt]) continue;
    const int row = wr0 + 16 * rt + n;
    const int64_t orow_idx = (int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G;
    const float inv = l[rt] > 0.f ? 1.f / l[rt] : 0.f;
    if (!split) {
      f16* orow = a.out + orow_idx * DR + 4 * g;
#pragma unroll
      for (int x = 0; x < NX; ++x)
        if (!PAD || 16 * x + 4 * g < DR)
          *reinterpret_cast<f16x4*>(orow + 16 * x) = to16x4<E>(o[rt][x] * inv);
    } else {
      // device-coherent stores through one wave-uniform descriptor per array
      // (the host keeps the partial arrays under 2 GiB)
      const uint32_t prow = (uint32_t)((int64_t)ks * a.total_q * a.Hq + orow_idx);
#pragma unroll
      for (int x = 0; x < NX; ++x)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[rt][x] * inv), ro,
                                               (prow * D + 16 * x + 4 * g) * (uint32_t)sizeof(float),
                                               0, kSc1);
      if (g == 0)
        __builtin_amdgcn_raw_buffer_store_b32(
            __builtin_bit_cast(uint32_t, l[rt] > 0.f ? m_run[rt] + log2f(l[rt]) : kNegInf), rl,
            prow * (uint32_t)sizeof(float), 0, kSc1);
    }
  }
  if (!split) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are complete
  __syncthreads();
  if (tid == 0)
    *last = __hip_atomic_fetch_add(a.tickets + item * a.Hkv + h, 1, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) == a.KS - 1;
  __syncthreads();
  if (!*last) return;
  if (tid == 0)
    __hip_atomic_store(a.tickets + item * a.Hkv + h, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  // merge: thread -> (row of the block, 4 consecutive dims).  All KS LSEs and
  // partial outputs of kMergeRows of the thread's rows are loaded at once
  // (indices past KS repeat the last split and get weight 0; rows past the
  // block repeat its last row and are not stored), so the block's rows cost
  // ceil(rows / (RPS * kMergeRows)) round trips to memory.
  constexpr int TPR = D / 4;             // threads per row
  constexpr int RPS = kThreads / TPR;    // rows per pass
  const int d4 = (tid % TPR) * 4;
  for (int row0 = r0 + tid / TPR; row0 <= r_last; row0 += RPS * kMergeRows) {
    float lse[kMergeRows][kMaxSplits];
    f32x4 ov[kMergeRows][kMaxSplits];
    int64_t orow_idx[kMergeRows];
#pragma unroll
    for (int u = 0; u < kMergeRows; ++u) {
      const int row = min(row0 + u * RPS, r_last);
      orow_idx[u] = (int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G;
#pragma unroll
      for (int k = 0; k < kMaxSplits; ++k) {
        const int kc = k < a.KS ? k : a.KS - 1;
        const uint32_t prow = (uint32_t)(kc * split_stride + orow_idx[u]);
        lse[u][k] = __builtin_bit_cast(
            float,
            __builtin_amdgcn_raw_buffer_load_b32(rl, prow * (uint32_t)sizeof(float), 0, kSc1));
        ov[u][k] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       ro, (prow * D + d4) * (uint32_t)sizeof(float), 0, kSc1));
      }
    }
#pragma unroll
    for (int u = 0; u < kMergeRows; ++u) {
      if (row0 + u * RPS > r_last) break;
      float M = kNegInf;
#pragma unroll
      for (int k = 0; k < kMaxSplits; ++k)
        if (k < a.KS) M = fmaxf(M, lse[u][k]);
      f32x4 num = {0.f, 0.f, 0.f, 0.f};
      float den = 0.f;
#pragma unroll
      for (int k = 0; k < kMaxSplits; ++k) {
        const float wgt = k < a.KS && lse[u][k] != kNegInf ? exp2f(lse[u][k] - M) : 0.f;
        num += wgt * ov[u][k];
        den += wgt;
      }
      const float inv = den > 0.f ? 1.f / den : 0.f;
      if (!PAD || d4 < DR)
        *reinterpret_cast<f16x4*>(a.out + orow_idx[u] * DR + d4) = to16x4<E>(num * inv);
    }
  }
}

// (head_dim 256: one wave per SIMD, 174 VGPRs + 72 AGPRs, no scratch)
//
// PAD: head_dim a.dr below D (a multiple of 8): q, the pools and the output are
// laid out by a.dr; the dims past it are zeros in q, K and V (never loaded)
// and never stored.  DC (a multiple of 32, a.dr <= DC <= D): the dims the
// products compute -- the K/V staging keeps D's layout, q.K runs DC / 32
// k-chunks and P.V DC / 16 output tiles, so the all-zero ones drop out at
// compile time.
template <int D, int RT, class E = Fp16, bool PAD = false, int DC = D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D > 128 ? 1 : 2, 8)))
void prefill_kernel(const PrefillArgs a) {
  using P = PCfg<D, RT>;
  static_assert(DC % 32 == 0 && DC <= D && (PAD || DC == D), "computed dims");
  constexpr int NCC = DC / 32;  // k-chunks of q.K computed
  constexpr int NXC = DC / 16;  // output tiles computed
  const int DR = PAD ? a.dr : D;
  extern __shared__ __align__(16) unsigned char smem[];

  // workgroup i: (KV head, key split) pair i % P, row block i / P (P = Hkv * KS);
  // the hardware places workgroup i on XCD i % 8, so when P divides 8 or is a
  // multiple of it every XCD serves fixed pairs -- one KV head and one key
  // range of every sequence -- and its L2 holds the K/V its row blocks share
  const int npair = a.Hkv * a.KS;
  const int item = blockIdx.x / npair;
  const int pair = blockIdx.x - item * npair;
  RowBlock rb;
  if (!locate_rows<P::ROWS, false>(a, item, rb)) return;
  const int h = pair % a.Hkv;
  const int G = a.G;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int total_rows = rb.n * G;
  const int cached = rb.ctx >= rb.n ? rb.ctx - rb.n : 0;
  const int r0 = rb.rb * P::ROWS;
  const int r_last = min(r0 + P::ROWS, total_rows) - 1;
  // keys the row block reads: causal up to its last position
  const int key_end = cached + r_last / G + 1;
  // split ks of KS takes an equal share of the row block's key blocks
  const int ks = pair / a.Hkv;
  const int nblocks_all = (key_end + kBlockKeys - 1) / kBlockKeys;
  const int per_split = (nblocks_all + a.KS - 1) / a.KS;
  const int kb_lo = min(ks * per_split, nblocks_all);
  const int kb_hi = min(kb_lo + per_split, nblocks_all);
  const int wr0 = r0 + w * 16 * RT;                               // first row of this wave

  // ---- this lane's rows: query vectors (B operand), last key each may see
  //      (its position) ----
  f16x8 qv[RT][NCC];
  int pos[RT];
  bool valid[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = wr0 + 16 * rt + n;
    valid[rt] = row < total_rows;
    const int rc = valid[rt] ? row : r_last;
    pos[rt] = valid[rt] ? cached + rc / G : -1;
    const f16* qrow = a.q + (int64_t)(rb.q0 + rc / G) * a.q_stride + (h * G + rc % G) * DR + 8 * g;
#pragma unroll
    for (int c = 0; c < NCC; ++c) {
      const f16x8 v = !PAD || 32 * c + 8 * g < DR ? ld16(qrow + 32 * c) : f16x8{};
      qv[rt][c] = valid[rt] ? v : f16x8{};
    }
  }

  // blocks whose last key is <= every row's position need no mask
  const int unmasked_blocks = (cached + min(wr0, r_last) / G + 1) / kBlockKeys;

  float m_run[RT], l_run[RT];
  f32x4 o[RT][NXC];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = kNegInf;
    l_run[rt] = 0.f;
#pragma unroll
    for (int x = 0; x < NXC; ++x) o[rt][x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- K/V block staging: thread t loads 16-byte chunk t % CPR of key rows
  //      t / CPR + KPL * i (keys at or past key_end repeat key_end - 1).  The
  //      block ids a block needs are fetched one iteration before its K/V
  //      loads, so no table access sits in front of a K/V load. ----
  const int32_t* trow = a.tables + (int64_t)rb.s * a.W;
  const int chunk = tid % P::CPR;
  const int krow = tid / P::CPR;
  const bool chunk_in = !PAD || chunk * 8 < DR;  // a real chunk of the row
  f16x8 kst[P::LOADS], vst[P::LOADS];
  int ids[P::LOADS];
  auto fetch_ids = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::LOADS; ++i) {
      const int key = min(kb * kBlockKeys + krow + P::KPL * i, key_end - 1);
      int page = key >> a.bs_log2;
      page = page < a.W ? page : a.W - 1;
      ids[i] = trow[page];
    }
  };
  auto load_block = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < P::LOADS; ++i) {
      // a key at or past key_end reads key key_end - 1 instead: a written
      // row, so finite, and past every row's position, so the causal mask
      // gives it probability 0 (no block below unmasked_blocks reaches it)
      const int kc = min(kb * kBlockKeys + krow + P::KPL * i, key_end - 1);
      const int blk = clamp_block(ids[i], a.NB);
      const int64_t off = (int64_t)(blk * a.BS + (kc & (a.BS - 1))) * (a.Hkv * DR) + h * DR + chunk * 8;
      if (PAD) {
        kst[i] = f16x8{};
        vst[i] = f16x8{};
      }
      if (chunk_in) {
        kst[i] = ld16(a.k_pool + off);
        vst[i] = ld16(a.v_pool + off);
      }
    }
  };
  auto store_block = [&](int stage) __attribute__((always_inline)) {
    unsigned char* kbase = smem + stage * P::STAGE;
    unsigned char* vbase = kbase + P::KBYTES;
#pragma unroll
    for (int i = 0; i < P::LOADS; ++i) {
      const int r = krow + P::KPL * i;
      *reinterpret_cast<f16x8*>(kbase + r * P::KP + chunk * 16) = kst[i];
      *reinterpret_cast<f16x8*>(vbase + r * P::VP + chunk * 16) = vst[i];
    }
  };

  if (kb_lo < kb_hi) {
    fetch_ids(kb_lo);
    load_block(kb_lo);
    fetch_ids(kb_lo + 1);
    store_block(0);
  }
  __syncthreads();

  // Loading two blocks ahead (a second register set) was measured slower: the
  // extra registers cost a wave per SIMD of occupancy.
  for (int kb = kb_lo; kb < kb_hi; ++kb) {
    const bool more = kb + 1 < kb_hi;
    if (more) {
      load_block(kb + 1);
      fetch_ids(kb + 2);
    }
    const unsigned char* kbase = smem + ((kb - kb_lo) & 1) * P::STAGE;
    const unsigned char* vbase = kbase + P::KBYTES;

    // S^T tiles: kKT key tiles x RT row tiles
    f32x4 st[RT][kKT];
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st[rt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCC; ++c) {
        const f16x8 kv =
            *reinterpret_cast<const f16x8*>(kbase + (16 * kt + n) * P::KP + (32 * c + 8 * g) * 2);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st[rt][kt] = mma32<E>(kv, qv[rt][c], st[rt][kt]);
      }
    }

    // online softmax per row tile; P^T of each 32 keys as one f16x8 B operand
    f16x8 pb[RT][kPS];
    // scores stay unscaled up to the exponent: the row max is taken on them and
    // scaled once (scale > 0 keeps the order), and exp2(s * scale - m) is one
    // fma per score; the causal mask only runs on blocks that need it
    const bool need_mask = kb >= unmasked_blocks;  // wave-uniform
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      float sv[kKT][4];
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[kt][i] = st[rt][kt][i];
      if (need_mask) {
#pragma unroll
        for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kb * kBlockKeys + 16 * kt + 4 * g + i > pos[rt]) sv[kt][i] = kNegInf;
      }
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt)
        mx = fmaxf(mx, fmaxf(fmaxf(sv[kt][0], sv[kt][1]), fmaxf(sv[kt][2], sv[kt][3])));
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      mx *= a.scale_log2;
      if (__ballot(mx > m_run[rt] + kRescaleSlack)) {  // wave-uniform
        const float m_new = fmaxf(m_run[rt], mx);
        const float alpha = m_new == kNegInf ? 1.f : exp2_fast(m_run[rt] - m_new);
        l_run[rt] *= alpha;
#pragma unroll
        for (int x = 0; x < NXC; ++x) o[rt][x] *= alpha;
        m_run[rt] = m_new;
      }
      const float neg_m = m_run[rt] == kNegInf ? 0.f : -m_run[rt];
      float lsum = 0.f;
#pragma unroll
      for (int ps = 0; ps < kPS; ++ps) {
        f16x8 p;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float e = exp2_fast(__builtin_fmaf(sv[2 * ps + kt][i], a.scale_log2, neg_m));
            const f16 pe = to16<E>(e);
            p[4 * kt + i] = pe;
            // bf16: the row sum takes the rounded weights that multiply V (the
            // fp16 rounding error is small enough to sum e itself)
            if constexpr (__is_same(E, Bf16))
              lsum += (float)__builtin_bit_cast(__bf16, pe);
            else
              lsum += e;
          }
        pb[rt][ps] = p;
      }
      l_run[rt] += lsum;
    }

    // O^T += V^T . P^T: one 32-key step per 16-dim tile and PV step
#pragma unroll
    for (int ps = 0; ps < kPS; ++ps) {
      const unsigned char* vb = vbase + (32 * ps + 4 * g + (n >> 2)) * P::VP + (n & 3) * 8;
#pragma unroll
      for (int x = 0; x < NXC; ++x) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vb + 32 * x));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vb + 16 * P::VP + 32 * x));
        const f16x4 l4 = __builtin_bit_cast(f16x4, lo), h4 = __builtin_bit_cast(f16x4, hi);
        const f16x8 va = {l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[rt][x] = mma32<E>(va, pb[rt][ps], o[rt][x]);
      }
    }

    if (more) store_block((kb + 1 - kb_lo) & 1);
    __syncthreads();
  }

  // ---- normalise and store, or the split's partial and the merge ----
  float lt[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    lt[rt] = l_run[rt] + shfl_xor_f(l_run[rt], 16);
    lt[rt] += shfl_xor_f(lt[rt], 32);
  }
  __shared__ int last;
  finish_split<D, RT, E, PAD, DC>(a, rb, item, h, ks, wr0, r0, r_last, valid, m_run, lt, o, &last);
}

// ---------------------------------------------------------------------------
// prefill_f32_kernel: fp32 pools (fe_prefill_paged_f32)
// ---------------------------------------------------------------------------
//
// The rows of a sequence's KV-head group in the tile kernel's order (row r:
// token r / G, query head hG + r % G), 16 per wave and 64 per workgroup.  Each
// wave walks every key tile up to its last row's position on the fp32 engine
// (F32Core: fp32 products on v_mfma_f32_16x16x4_f32, fp32 softmax), every
// column masking the keys past its own position, then normalises and stores
// its 16 rows: no LDS, no key splits.
//
// CASCADE: the prefix pass of the fp32 shared-prefix decode.  "Sequence" s is
// a group of decode rows (locate_rows' cascade mode), every row reads the
// group's whole-block prefix from the group's first table row (none for a row
// whose context does not pass it), and the result is one prefix slot per
// (row, query head): the normalised output in pre_o and its base-2 LSE in
// pre_lse; the grid's last workgroup writes the suffix starts.
//
// PAD: head_dim a.dr below D (a multiple of 8): q, the pools and the output laid
// out by a.dr, the dims past it zeros in q, K and V and never stored.
template <int D, bool LIST, bool CASCADE = false, bool PAD = false>
__global__ __launch_bounds__(kThreads) void prefill_f32_kernel(const PrefillArgs a) {
  constexpr int ROWS = kWaves * 16;
  const int DR = PAD ? a.dr : D;
  if constexpr (CASCADE) {
    if (blockIdx.x == gridDim.x - 1) {
      write_suffix_starts(a, a.q_off);
      return;
    }
  }
  const int item = blockIdx.x / a.Hkv;
  const int h = blockIdx.x - item * a.Hkv;
  RowBlock rb;
  if (!locate_rows<ROWS, CASCADE>(a, item, rb)) return;
  const int G = a.G;
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int total_rows = rb.n * G;
  const int cached = CASCADE ? 0 : (rb.ctx >= rb.n ? rb.ctx - rb.n : 0);
  const int wr0 = rb.rb * ROWS + 16 * w;
  if (wr0 >= total_rows) return;
  const int r_last = min(wr0 + 16, total_rows) - 1;
  const int row = wr0 + n;
  const bool valid = row < total_rows;
  const int rc = valid ? row : r_last;

  F32Core<D, LIST, PAD> core;
  core.k_pool = reinterpret_cast<const float*>(a.k_pool);
  core.v_pool = reinterpret_cast<const float*>(a.v_pool);
  core.k_pool_w = nullptr;
  core.v_pool_w = nullptr;
  core.trow = a.tables + (int64_t)(CASCADE ? rb.q0 : rb.s) * a.W;
  core.rs = a.Hkv * DR;
  core.hoff = h * DR;
  core.dr = DR;
  core.W = a.W;
  core.NB = a.NB;
  core.BS = a.BS;
  core.bs_log2 = a.bs_log2;
  if constexpr (CASCADE) {
    core.tok_end = rb.ctx;  // the group's prefix
    core.limit = valid && member_len(a, rb.q0 + rc / G) > rb.ctx ? rb.ctx : 0;
  } else {
    core.tok_end = cached + r_last / G + 1;  // the wave's last row reads the most keys
    core.limit = valid ? cached + rc / G + 1 : 0;
  }
  core.scale_log2 = a.scale_log2;
  core.knew_row = nullptr;
  core.vnew_row = nullptr;
  core.new_pos = -1;
  {
    const float* qrow = reinterpret_cast<const float*>(a.q) +
                        (int64_t)(rb.q0 + rc / G) * a.q_stride + (int64_t)(h * G + rc % G) * DR;
#pragma unroll
    for (int c = 0; c < F32Core<D, LIST, PAD>::NC; ++c) {
      core.qv[c] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (!PAD || 16 * c + 4 * g < DR)
        core.qv[c] = *reinterpret_cast<const f32x4*>(qrow + 16 * c + 4 * g);
    }
  }
  core.init_acc();
  core.run(0, 1, (core.tok_end + kTile - 1) / kTile);
  const float l = core.l_total();
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (valid) {
    const int64_t r = (int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G;
    if constexpr (CASCADE) {
      float* orow = a.pre_o + r * D + 4 * g;
#pragma unroll
      for (int x = 0; x < F32Core<D, LIST, PAD>::NX; ++x)
        *reinterpret_cast<f32x4*>(orow + 16 * x) = core.o[x] * inv;
      if (g == 0) a.pre_lse[r] = l > 0.f ? core.m_run + log2f(l) : kNegInf;
    } else {
#pragma unroll
      for (int x = 0; x < F32Core<D, LIST, PAD>::NX; ++x)
        if (!PAD || 4 * g + 16 * x < DR)
          store_out4<F32>(a.out, r * DR + 4 * g + 16 * x, core.o[x] * inv);
    }
  }
}

// ---------------------------------------------------------------------------
// prefill_dma_kernel: 32 rows per wave, 64-key blocks staged by buffer->LDS DMA
// ---------------------------------------------------------------------------
//
// Used for block sizes that are multiples of 16 (every 16-key run of a block
// lies in one page).  Differences from prefill_kernel:
//
// * Each wave owns 32 rows (two 16-row MFMA tiles), a workgroup 128 rows, so
//   every K/V fragment read from LDS feeds two MFMAs: 32 flops per LDS byte
//   (one tile per wave, as in prefill_kernel, is 16 flops per byte, which caps
//   the MFMA pipes at about half of their peak on LDS bandwidth alone).
// * Keys come in blocks of 64.  Wave w stages keys 16w .. 16w+15 of a block --
//   one run of one page -- with buffer_load_dwordx4 ... lds: one scalar buffer
//   descriptor per run (its range ends at the last key the row block reads, so
//   later keys arrive as zeros; the causal mask covers them), loop-invariant
//   lane offsets, and no registers or address arithmetic per staged byte.  The
//   next block's DMA runs while the current block is computed.
// * LDS rows are not padded (a DMA instruction fills 1 KiB contiguously); bank
//   conflicts are avoided by XOR-swizzling the 16-byte chunks of each row (see
//   swz_k / swz_v): the QK^T operand read puts consecutive lanes on consecutive
//   key rows of one chunk, a transposing V read puts each 16-lane group on 4
//   consecutive rows x 32 bytes.
// * Row sums come from the PV MFMA: a tile of ones as the V^T operand gives
//   sum_k P[row][k] in every element, from the same fp16 probabilities the
//   output uses, and takes the place of a VALU add per score.

constexpr int kDmaKeys = 64;                       // keys per staged block
constexpr int kDmaRows = 128;                      // rows per unit

template <int D>
struct DCfg {
  static constexpr int NC = D / 32;          // 32-dim k-chunks of QK^T
  static constexpr int NX = D / 16;          // 16-dim output tiles
  static constexpr int ROWB = D * 2;         // LDS bytes per staged key row
  static constexpr int MAT = kDmaKeys * ROWB;
  static constexpr int STAGE = 2 * MAT;      // K rows, then V rows
  static constexpr int CPR = D / 8;          // 16-byte chunks per row
  static constexpr int RPI = kWave / CPR;    // rows per DMA instruction
  static constexpr int NI = 16 / RPI;        // DMA instructions per 16-key run and matrix
};

// Chunk swizzles of staged key row r.  gfx950's LDS serves 256 bytes per clock
// (64 banks of 4 bytes): 16 lanes of a 16-byte read, 32 lanes of an 8-byte read.
// K (16 consecutive rows, one chunk each): D = 128 rows are 256 bytes, so
// chunk c goes to slot c ^ (r & 15); D = 64 rows are 128 bytes, row parity
// already picks the half of the 256 bytes, so slot c ^ ((r >> 1) & 7).
// V (transposing reads: 8 consecutive rows x 32 bytes per 32 lanes): 32-byte
// pairs of chunks move together, slot c ^ ((r & 7) << 1) for D = 128 and
// c ^ (((r >> 1) & 3) << 1) for D = 64.  The D = 128 forms are also
// conflict-free with 32 banks (8 and 16 lanes per clock).
template <int D>
__device__ __forceinline__ int swz_k(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
template <int D>
__device__ __forceinline__ int swz_v(int r) { return D == 128 ? ((r & 7) << 1) : (((r >> 1) & 3) << 1); }

// Row maxima of scores (finite or -inf, never NaN): IEEE maximum, which gfx950
// computes three operands at a time (v_maximum3_f32) straight from the MFMA
// results -- fmaxf would first canonicalise every operand, one v_max_f32
// x, x, x each, under the IEEE mode.  Written as the compiler's own operation,
// not inline asm: an MFMA result read by a VALU instruction needs wait states
// that the compiler inserts only for instructions it can see (an inline-asm
// max read a score tile two instructions after its MFMA, before the MFMA had
// written every lane, and overwrote a register that MFMA was still reading).
// The cross-lane steps use gfx950's permlane swaps (VALU, no LDS round trip).
// Each swap returns both halves and both are used: permlane32_swap(x, x) gives
// lane l the values of lanes l % 32 and l % 32 + 32, permlane16_swap(x, x)
// those of the two 16-lane rows l / 16 pairs with.
__device__ __forceinline__ float vmax2(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax2(vmax2(a, b), c); }
__device__ __forceinline__ float max_over_lane_rows(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// max of the 16 values sv[4][4]
__device__ __forceinline__ float max16(const float (&v)[4][4]) {
  const float a = vmax3(v[0][0], v[0][1], v[0][2]);
  const float b = vmax3(v[0][3], v[1][0], v[1][1]);
  const float c = vmax3(v[1][2], v[1][3], v[2][0]);
  const float d = vmax3(v[2][1], v[2][2], v[2][3]);
  const float e = vmax3(v[3][0], v[3][1], v[3][2]);
  return vmax2(vmax3(a, b, c), vmax3(d, e, v[3][3]));
}

// max of the 8 values sv[0..1][4]
__device__ __forceinline__ float max8(const float (&v)[4][4]) {
  const float a = vmax3(v[0][0], v[0][1], v[0][2]);
  const float b = vmax3(v[0][3], v[1][0], v[1][1]);
  return vmax3(a, b, vmax2(v[1][2], v[1][3]));
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(4))) const int32_t const_i32;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t run_rsrc(const f16* base, uint32_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

// DMA of one wave's RUN-key run of block kb (first key t0, RUN dividing 16, so
// the run lies in one page) into rows RUN * w .. of the K and V stages: one
// buffer descriptor per matrix whose range ends at the run's last key before
// key_end (later rows arrive as zeros).
template <int D, int RUN = 16>
__device__ __forceinline__ void dma_run(const PrefillArgs& a, int h, int w, int t0, int key_end,
                                        int id, const uint32_t* voff_k, const uint32_t* voff_v,
                                        unsigned char* kst, unsigned char* vst, int wv = -1) {
  using P = DCfg<D>;
  static_assert(16 % RUN == 0 && RUN % P::RPI == 0, "whole DMA instructions within a page");
  const int rs = a.Hkv * D * 2;
  int nv = key_end - t0;
  nv = nv < 0 ? 0 : (nv > RUN ? RUN : nv);
  const uint32_t nrec = nv > 0 ? (uint32_t)((nv - 1) * rs + D * 2) : 0u;
  const int64_t row0 = (int64_t)id * a.BS + (t0 & (a.BS - 1));
  const int64_t off = row0 * a.Hkv * D + h * D;
  const __amdgpu_buffer_rsrc_t rk = run_rsrc(a.k_pool + off, nrec);
  const __amdgpu_buffer_rsrc_t rv = run_rsrc(a.v_pool + off, nrec);
  unsigned char* kl = kst + RUN * w * P::ROWB;
  unsigned char* vl = vst + RUN * (wv < 0 ? w : wv) * P::ROWB;  // V rows: run wv, if given
#pragma unroll
  for (int i = 0; i < RUN / P::RPI; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(kl + i * P::RPI * P::ROWB), 16,
                                             voff_k[i], 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(vl + i * P::RPI * P::ROWB), 16,
                                             voff_v[i], 0, 0, 0);
  }
}

// NKT 16-key tiles of a staged 64-key block for a wave's RT 16-row tiles (the
// stream-K kernel's step: the whole block; the cascade prefix kernel's: one
// half, NKT = 2, kbase and koff moved to key 32 for the second, vbase at
// that half's V rows):
// S^T = K.Q^T with v_mfma_f32_16x16x32, base-2 online softmax with the lazy
// rescale (the causal mask only on blocks at or past unmasked_blocks: key
// kb * 64 + koff + j is masked past the row's pos), P as fp16 / bf16,
// O^T += V^T.P^T, and the row sums from a tile of ones (every element of
// lsum[rt] is the row's sum of P).  A move by 32 keys keeps the chunk
// swizzles (they depend on the key row mod 16, or mod 32 halved).
template <int D, int RT, class E, int NKT = 4>
__device__ __forceinline__ void dma_block(int kb, const unsigned char* kbase,
                                          const unsigned char* vbase, int unmasked_blocks,
                                          float scale_log2, const f16x8 (&qv)[RT][DCfg<D>::NC],
                                          const int (&pos)[RT], float (&m_run)[RT],
                                          f32x4 (&lsum)[RT], f32x4 (&o)[RT][DCfg<D>::NX],
                                          int koff = 0) {
  static_assert(NKT == 4 || NKT == 2, "a whole block or one half");
  constexpr int NPS = NKT / 2;  // 32-key PV steps
  using P = DCfg<D>;
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const f16 one = to16<E>(1.f);
  const f16x8 ones = {one, one, one, one, one, one, one, one};
  // K fragments (16 keys x 32 dims, A operand): all reads issued ahead of
  // the MFMAs that use them
  f16x8 kf[NKT][P::NC];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int c = 0; c < P::NC; ++c)
      kf[kt][c] = *reinterpret_cast<const f16x8*>(
          kbase + (16 * kt + n) * P::ROWB + (((4 * c + g) ^ swz_k<D>(16 * kt + n)) * 16));
  // one row tile: the scheduler would otherwise interleave the reads with the
  // MFMAs to save registers, and each MFMA would wait for its read
  if constexpr (RT == 1) __builtin_amdgcn_sched_barrier(0);
  f32x4 st[RT][NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) st[rt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int c = 0; c < P::NC; ++c)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) st[rt][kt] = mma32<E>(kf[kt][c], qv[rt][c], st[rt][kt]);
  // V fragments (transposing reads): lane (g, n) of a read addresses V[key
  // 32ps + 4g + n/4][dims 16x + 4(n%4) .. +3] (and the same 16 keys further
  // for the second half of the k = 32 operand; 32ps and 16 keep the row's
  // swizzle).  The first 32 keys' fragments are read before the softmax,
  // whose VALU work hides their latency.
  const int vrow = 4 * g + (n >> 2);
  const int vswz = swz_v<D>(vrow);
  auto vfrag = [&](int ps, int x) __attribute__((always_inline)) {
    const unsigned char* vb = vbase + (32 * ps + vrow) * P::ROWB + (n & 1) * 8;
    const unsigned char* vh = vbase + (32 * ps + 16 + vrow) * P::ROWB + (n & 1) * 8;
    const int slot = (2 * x + ((n & 3) >> 1)) ^ vswz;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vb + slot * 16));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vh + slot * 16));
    const f16x4 l4 = __builtin_bit_cast(f16x4, lo), h4 = __builtin_bit_cast(f16x4, hi);
    return f16x8{l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
  };
  f16x8 vf[P::NX];
#pragma unroll
  for (int x = 0; x < P::NX; ++x) vf[x] = vfrag(0, x);

  const bool need_mask = kb >= unmasked_blocks;  // wave-uniform
  f16x8 pb[RT][NPS];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float sv[4][4];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[kt][i] = st[rt][kt][i];
    if (need_mask) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kb * kDmaKeys + koff + 16 * kt + 4 * g + i > pos[rt]) sv[kt][i] = kNegInf;
    }
    const float mx = max_over_lane_rows(NKT == 4 ? max16(sv) : max8(sv)) * scale_log2;
    if (__ballot(mx > m_run[rt] + kRescaleSlack)) {  // wave-uniform
      const float m_new = fmaxf(m_run[rt], mx);
      const float alpha = m_new == kNegInf ? 1.f : exp2_fast(m_run[rt] - m_new);
      lsum[rt] *= alpha;
#pragma unroll
      for (int x = 0; x < P::NX; ++x) o[rt][x] *= alpha;
      m_run[rt] = m_new;
    }
    const float neg_m = m_run[rt] == kNegInf ? 0.f : -m_run[rt];
#pragma unroll
    for (int ps = 0; ps < NPS; ++ps) {
      f16x8 p;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p[4 * kt + i] =
              to16<E>(exp2_fast(__builtin_fmaf(sv[2 * ps + kt][i], scale_log2, neg_m)));
      pb[rt][ps] = p;
    }
  }
#pragma unroll
  for (int ps = 0; ps < NPS; ++ps) {
#pragma unroll
    for (int x = 0; x < P::NX; ++x) {
      const f16x8 va = vf[x];
      if (ps + 1 < NPS) vf[x] = vfrag(ps + 1, x);  // the next 32 keys' fragment, in flight meanwhile
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) o[rt][x] = mma32<E>(va, pb[rt][ps], o[rt][x]);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) lsum[rt] = mma32<E>(ones, pb[rt][ps], lsum[rt]);
  }
}

// ---- stream-K work split -------------------------------------------------
//
// Units are (sequence, KV head, 128-row block) in that order; unit u has nb_u
// key blocks of 64 (through its last row's position).  The grid is a fixed
// number of workgroups (two per CU); logical workgroup g takes blocks
// [g*T/NWG, (g+1)*T/NWG) of the concatenated key blocks of all units (T in
// total), so every workgroup gets the same number of blocks whatever the mix
// of context lengths.  A unit covered by one workgroup is written directly; a
// unit split between workgroups gets a normalised fp32 partial and base-2 LSE
// from each contributor (slot 2g, or 2g + 1 for the last unit of a range that
// started in an earlier one), written with device-coherent stores that the
// contributor waits for before drawing a ticket; the contributor drawing the
// last ticket merges the partials (device-coherent loads) into the output and
// resets the ticket (the protocol of the decode's split-K merge).  A split
// unit starts in the range of exactly one workgroup x0 (it runs past the end
// of that range), so its ticket is tickets[x0] and its contributors are the
// workgroups x0 .. owner(last block).
//
// Key blocks per row block, in closed form: a row block whose last row is y
// (row = position * G + head) reads keys up to c + y / G, so it has
// floor((G * (c + 64) + y) / (64 * G)) blocks of 64 (c cached tokens), and
// the row blocks 0 .. R-2 of a sequence (all but the last, whose y is cut at
// the sequence's last row) have floor_sum(R - 1, 64G, 128, G * (c + 64) + 127)
// blocks together.

// sum_{i < n} floor((a * i + b) / m) (the Euclidean-like reduction).  The
// divisions are 32-bit: fe_prefill_paged accepts sizes with a * n + b < 2^29
// on the first call, and y = a * n + b does not grow from one step to the
// next (a < m after the first reduction, b < m).
__device__ __forceinline__ int64_t floor_sum(uint32_t n, uint32_t m, uint32_t a, uint32_t b) {
  int64_t ans = 0;
  while (true) {
    if (a >= m) {
      ans += (int64_t)((uint64_t)n * (n - 1) / 2) * (a / m);
      a %= m;
    }
    if (b >= m) {
      ans += (int64_t)n * (b / m);
      b %= m;
    }
    const uint32_t y = a * n + b;
    if (y < m) break;
    n = y / m;
    b = y % m;
    const uint32_t t = m;
    m = a;
    a = t;
  }
  return ans;
}

// A sequence as the work split sees it.
struct SeqWork {
  int q0;      // first query row in q / out
  int n;       // new tokens (positions)
  int cached;  // keys before the first new token
  int R;       // 128-row blocks
  int tb;      // key blocks of all row blocks of one KV head
};

__device__ __forceinline__ SeqWork seq_work(const PrefillArgs& a, int s) {
  SeqWork w;
  w.q0 = min(max(a.q_off[s], 0), a.total_q);
  w.n = min(a.q_off[s + 1], a.total_q) - w.q0;
  w.n = w.n > 0 ? w.n : 0;
  const int ctx = min(clamp_len(a.ctx[s]), a.W * a.BS);  // what the table addresses
  w.cached = ctx >= w.n ? ctx - w.n : 0;
  w.R = (w.n * a.G + kDmaRows - 1) / kDmaRows;
  w.tb = 0;
  if (w.R > 0) {
    const uint32_t G = (uint32_t)a.G, m = (uint32_t)kDmaKeys * G;
    const uint32_t b = G * (uint32_t)(w.cached + kDmaKeys) + kDmaRows - 1;
    w.tb = (int)(floor_sum((uint32_t)(w.R - 1), m, kDmaRows, b) +
                 (G * (uint32_t)(w.cached + kDmaKeys) + (uint32_t)(w.n * a.G) - 1) / m);
  }
  return w;
}

// key blocks of row block rb of a sequence
__device__ __forceinline__ int rb_blocks(const PrefillArgs& a, const SeqWork& w, int rb) {
  const int y = min(kDmaRows * (rb + 1), w.n * a.G) - 1;
  return (a.G * (w.cached + kDmaKeys) + y) / (kDmaKeys * a.G);
}

// Where block x of the concatenation lies: sequence s, head h, row block rb
// and block kb of that unit.  Every wave computes it (wave-parallel over
// sequences and row blocks, results uniform).
struct StreamPos {
  int s, h, rb, kb;
  SeqWork w;
};
// The ranges of the nwg workgroups: [start(g), start(g + 1)) with start(g) =
// floor(g * T / nwg), in 32-bit arithmetic (fe_prefill_paged keeps T < 2^31
// and nwg < 2^13, so g * q < T and g * r < nwg^2).
struct Ranges {
  int T, nwg, q, r;  // T = q * nwg + r
  __device__ __forceinline__ int start(int g) const { return g * q + (g * r) / nwg; }
  // the workgroup whose range holds block x (0 <= x < T): a float estimate
  // within one of the answer, then exact steps
  __device__ __forceinline__ int owner(int x) const {
    int g = (int)((float)x * (float)nwg / (float)T);
    g = min(max(g, 0), nwg - 1);
    while (g + 1 < nwg && start(g + 1) <= x) ++g;
    while (g > 0 && start(g) > x) --g;
    return g;
  }
};

// The split every workgroup (and the step's plan) derives from the sizes: the
// ranges (T key blocks in all, nwg workgroups, a multiple of 8 from 8 on) and
// this lane's sequence of the first 64 (kept for stream_locate).
struct StreamPlan {
  Ranges rg;
  SeqWork w0;
};

// Contributors of one split unit at most kMaxContrib: ranges of at least
// ceil(nb_max / (kMaxContrib - 2)) blocks, so a unit of nb_max blocks meets at
// most kMaxContrib - 1 of them.
constexpr int kMaxContrib = 32;
// Partials a split unit's merging lanes load per round trip.
constexpr int kMergeBatch = 2;
// Stream-K workgroups at most (a split unit's ticket is tickets[x0], x0 < nwg).
constexpr int kMaxStreamWgs = 1024;

__device__ __forceinline__ StreamPlan stream_plan(const PrefillArgs& a) {
  const int lane = lane_id();
  StreamPlan p;
  int T = 0;
  p.w0 = SeqWork{};
  int nb_max = 0;
  for (int base = 0; base < a.S; base += kWave) {
    int blocks = 0, most = 0;
    if (base + lane < a.S) {
      const SeqWork w = seq_work(a, base + lane);
      if (base == 0) p.w0 = w;
      blocks = w.tb * a.Hkv;
      if (w.R > 0) most = rb_blocks(a, w, w.R - 1);  // the last row block reads the most keys
    }
    T += wave_sum_i(blocks);
    nb_max = max(nb_max, wave_max_i(most));
  }
  const int min_range = max((nb_max + kMaxContrib - 3) / (kMaxContrib - 2), 1);
  int nwg = max(1, min(a.nwg_max, T / min_range));
  nwg = nwg >= 8 ? nwg & ~7 : nwg;
  p.rg = Ranges{T, nwg, T / nwg, T % nwg};
  return p;
}

// Logical workgroup of workgroup g < nwg: the dispatcher deals workgroups to
// the 8 XCDs in turn (g % 8), so logical ranges (g % 8) * nwg / 8 + g / 8 put
// consecutive key blocks -- the same sequence and KV head, mostly -- on one
// XCD and its L2.
__device__ __forceinline__ int logical_wg(int g, int nwg) {
  return nwg >= 8 ? (g & 7) * (nwg >> 3) + (g >> 3) : g;
}

__device__ __forceinline__ bool stream_locate(const PrefillArgs& a, const SeqWork& w0, int x,
                                              StreamPos& p) {
  const int lane = lane_id();
  int bcarry = 0;
  for (int base = 0; base < a.S; base += kWave) {
    const int s = base + lane;
    SeqWork w{};
    if (base == 0) w = w0;
    else if (s < a.S) w = seq_work(a, s);
    const int blocks = w.tb * a.Hkv;
    const int incl = wave_scan_incl_i(blocks);
    const int lo = bcarry + incl - blocks;
    const unsigned long long hit = __ballot(s < a.S && blocks > 0 && x >= lo && x < lo + blocks);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      p.s = base + src;
      p.w.q0 = readlane_i(w.q0, src);
      p.w.n = readlane_i(w.n, src);
      p.w.cached = readlane_i(w.cached, src);
      p.w.R = readlane_i(w.R, src);
      p.w.tb = readlane_i(w.tb, src);
      const int o = x - (bcarry + readlane_i(incl - blocks, src));
      p.h = o / p.w.tb;
      const int o2 = o - p.h * p.w.tb;
      // row block: scan of the row blocks' key blocks, 64 row blocks at a time
      // (one division per lane and chunk)
      int rcarry = 0;
      for (int rb0 = 0; rb0 < p.w.R; rb0 += kWave) {
        const int rb = rb0 + lane;
        const int nbl = rb < p.w.R ? rb_blocks(a, p.w, rb) : 0;
        const int rincl = wave_scan_incl_i(nbl);
        const int rlo = rcarry + rincl - nbl;
        const unsigned long long rhit = __ballot(nbl > 0 && o2 >= rlo && o2 < rlo + nbl);
        if (rhit) {
          const int rsrc = __builtin_ctzll(rhit);
          p.rb = rb0 + rsrc;
          p.kb = o2 - readlane_i(rlo, rsrc);
          return true;
        }
        rcarry += readlane_i(rincl, kWave - 1);
      }
      return false;
    }
    bcarry += readlane_i(incl, kWave - 1);
  }
  return false;
}


// The split units' partial slots (2 per workgroup of 128 rows): one buffer
// descriptor per array over all of them (the host keeps them < 2 GiB).
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc_o(const PrefillArgs& a, int nwg) {
  return __builtin_amdgcn_make_buffer_rsrc(a.part_o, 0, (int)(2 * nwg * kDmaRows * D * sizeof(float)),
                                           0x00020000);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc_lse(const PrefillArgs& a, int nwg) {
  return __builtin_amdgcn_make_buffer_rsrc(a.part_lse, 0, (int)(2 * nwg * kDmaRows * sizeof(float)),
                                           0x00020000);
}

// Merges rows of a split unit into the fp16 output: lane (g, n) owns one row
// (urow within the unit, output row orow) and dims 16x + 4g .. +3.  Contributor
// k of the unit's ncontrib (workgroups x0 + k) left its normalised partial in
// slot slot_x0 (k = 0) or 2 (x0 + k); contributor `self` (-1: none) did not,
// and its values (own_o, own_lse: exactly what it would have stored) are used
// in its place.  Contributors are combined in slot order, kMergeBatch per round
// trip with a running maximum, so the result does not depend on which
// contributor merges.
template <int D, class E>
__device__ __forceinline__ void merge_split_rows(const PrefillArgs& a, __amdgpu_buffer_rsrc_t ro,
                                                 __amdgpu_buffer_rsrc_t rl, int x0, int ncontrib,
                                                 uint32_t slot_x0, int self, uint32_t urow,
                                                 int64_t orow, const f32x4 (&own_o)[D / 16],
                                                 float own_lse) {
  constexpr int NX = D / 16;
  const int g = lane_id() >> 4;
  float M = kNegInf, den = 0.f;
  f32x4 num[NX];
#pragma unroll
  for (int xx = 0; xx < NX; ++xx) num[xx] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < ncontrib; c0 += kMergeBatch) {
    float lv[kMergeBatch];
    f32x4 ov[kMergeBatch][NX];
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      lv[k] = kNegInf;
      const int kc = c0 + k;
      if (kc == self) {  // wave-uniform
        lv[k] = own_lse;
#pragma unroll
        for (int xx = 0; xx < NX; ++xx) ov[k][xx] = own_o[xx];
      } else if (kc < ncontrib) {  // wave-uniform
        const uint32_t prow = (kc == 0 ? slot_x0 : 2u * (x0 + kc)) * kDmaRows + urow;
        lv[k] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rl, prow * (uint32_t)sizeof(float), 0,
                                                        kSc1));
#pragma unroll
        for (int xx = 0; xx < NX; ++xx)
          ov[k][xx] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         ro, (prow * D + 16 * xx + 4 * g) * (uint32_t)sizeof(float), 0, kSc1));
      } else {
#pragma unroll
        for (int xx = 0; xx < NX; ++xx) ov[k][xx] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    float bm = kNegInf;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) bm = fmaxf(bm, lv[k]);
    const float newM = fmaxf(M, bm);
    const float alpha = M == kNegInf ? 0.f : exp2f(M - newM);
    den *= alpha;
#pragma unroll
    for (int xx = 0; xx < NX; ++xx) num[xx] *= alpha;
#pragma unroll
    for (int k = 0; k < kMergeBatch; ++k) {
      const float wv = lv[k] != kNegInf ? exp2f(lv[k] - newM) : 0.f;
      den += wv;
#pragma unroll
      for (int xx = 0; xx < NX; ++xx) num[xx] += wv * ov[k][xx];
    }
    M = newM;
  }
  const float dinv = den > 0.f ? 1.f / den : 0.f;
  f16* out = a.out + orow * D + 4 * g;
#pragma unroll
  for (int xx = 0; xx < NX; ++xx)
    *reinterpret_cast<f16x4*>(out + 16 * xx) = to16x4<E>(num[xx] * dinv);
}

// The stream-K kernel's workgroup: two halves of kHalfWaves waves, each wave
// 32 rows (RT = 2 tiles of 16) of the unit's 128.  Half H takes the unit's
// blocks kb_lo + H, kb_lo + H + 2, ... with its own two LDS stages, so the
// workgroup keeps 128 rows in flight per CU with two waves per SIMD, and the
// halves' online-softmax states of each row meet in LDS at the unit's end.
constexpr int kHalfWaves = kDmaRows / 32;
constexpr int kDmaThreads = 2 * kHalfWaves * kWave;

constexpr int kPPlanInts = 16;
constexpr int kPPlanMagic = 0x46505046;  // "FPPF"
constexpr int kPPlanFields = 15;         // descriptor words: key (2), fields in the clear, digest
constexpr int kPPlanDigest = 14;         // descriptor word of the digest
constexpr int kPPlanErrSizes = 1;        // error word: the call's sizes or tensors are not the plan's
constexpr int kPPlanErrStale = 2;        // error word: q_offsets / context_lens changed since the plan
static_assert((2 * kPPlanInts - 1) * 4 == FE_PREFILL_PLAN_ERROR_OFFSET &&
              kPPlanErrSizes == FE_PLAN_ERR_SIZES && kPPlanErrStale == FE_PLAN_ERR_STALE);
inline size_t pplan_bytes() { return (size_t)(2 + kMaxStreamWgs) * kPPlanInts * sizeof(int32_t); }
inline void set_pplan_key(PrefillArgs& a) {
  const uint64_t f[] = {(uint64_t)kPPlanMagic, (uint64_t)a.S, (uint64_t)a.total_q,
                        (uint64_t)a.Hq, (uint64_t)a.Hkv, (uint64_t)a.W, (uint64_t)a.BS,
                        (uint64_t)a.nwg_max, (uint64_t)(uintptr_t)a.q_off,
                        (uint64_t)(uintptr_t)a.ctx};
  const uint64_t h = plan_key(f, (int)(sizeof(f) / sizeof(f[0])));
  a.plan_key_lo = (uint32_t)h;
  a.plan_key_hi = (uint32_t)(h >> 32);
}

// lowbias32 (C. Wellons' published 32-bit integer hash)
__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
// Digest of q_offsets[0..S] and context_lens[0..S), uniform over the wave: lane
// s of a pass loads q_offsets[s] (s <= S) and context_lens[s] (s < S), both
// loads unconditional (indices clamped, results selected), so for up to 63
// sequences all of it is one round trip.  S >= 1 (the callers return earlier
// for an empty batch).
__device__ __forceinline__ int lens_digest(const PrefillArgs& a) {
  const int lane = lane_id();
  uint32_t d = 0;
  for (int base = 0; base <= a.S; base += kWave) {
    const int s = base + lane;
    const uint32_t qo = (uint32_t)a.q_off[min(s, a.S)];
    const uint32_t cx = (uint32_t)a.ctx[min(s, a.S - 1)];
    const uint32_t mq = mix32(qo + 0x9e3779b9u * (uint32_t)(s + 1));
    const uint32_t mc = mix32(cx + 0x85ebca6bu * (uint32_t)(s + 1));
    d += s <= a.S ? (s < a.S ? mq ^ mc : mq) : 0u;
  }
  return wave_sum_i((int)d);
}

// A planned launch whose plan is not for the call: every workgroup of the grid
// writes NaN to its grid-stride share of the output (so the whole of it is
// NaN), and workgroup 0 sets the plan's error word.
template <int D, class E>
__device__ __forceinline__ void refuse_plan(const PrefillArgs& a, int err) {
  const f16 nan = to16<E>(__builtin_nanf(""));
  const int64_t n = (int64_t)a.total_q * a.Hq * D;
  for (int64_t e = (int64_t)blockIdx.x * kDmaThreads + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kDmaThreads)
    a.out[e] = nan;
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(a.plan + 2 * kPPlanInts - 1, err, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// The units of workgroup gid's range [x_begin, x_end) for the waves of half H
// (wave r of the half); k0 .. v1 are the half's stage objects, pk1 / pv1 the
// partner half's stage-1 objects, xml the exchange of row maxima and sums and
// last the workgroup's ticket result.  Units follow each other without a
// pipeline bubble: after a unit's last step the next unit's block ids, queries
// and first block (into stage 0) are loaded while the halves exchange their
// states (in the stage-1 objects) and store.  PLANNED: the live lengths'
// digest is checked against the plan's (plan_digest) while the first unit's
// loads are in flight -- they stay in bounds for a stale plan of the call's
// sizes -- and before anything is stored or any ticket drawn.
template <int D, int RT, int H, class E, bool PLANNED = false>
__device__ __forceinline__ void run_units(const PrefillArgs& a, const StreamPlan& pl, int gid,
                                          int x_begin, int x_end, StreamPos sp, int r,
                                          unsigned char* k0, unsigned char* v0,
                                          unsigned char* k1, unsigned char* v1,
                                          const unsigned char* pk1, const unsigned char* pv1,
                                          float* xml, int* last, int plan_digest = 0) {
  using P = DCfg<D>;
  static_assert(RT == 2, "each half's wave exchanges one of its two row tiles");
  static_assert(2 * P::NX * kWave * 16 <= P::MAT, "two waves' tiles per stage object");
  const int G = a.G;
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int rs = a.Hkv * D * 2;  // pool bytes from one key row to the next
  uint32_t voff_k[P::NI], voff_v[P::NI];  // loop-invariant DMA lane offsets
#pragma unroll
  for (int i = 0; i < P::NI; ++i) {
    const int rr = P::RPI * i + lane / P::CPR;
    const int sl = lane % P::CPR;
    voff_k[i] = (uint32_t)(rr * rs + (sl ^ swz_k<D>(rr)) * 16);
    voff_v[i] = (uint32_t)(rr * rs + (sl ^ swz_v<D>(rr)) * 16);
  }

  // ---- the current unit (wave-uniform, except the lanes' rows) ----
  int x = x_begin;
  int h = 0, q0 = 0, total_rows = 0, cached = 0, r0 = 0, r_last = 0, key_end = 0;
  int kb_lo = 0, kb_hi = 0, kb_first = 0, unit_start = 0, nb = 0, wr0 = 0, unmasked_blocks = 0;
  bool split = false, has_rows = false;
  const int32_t* trow = a.tables;
  int kb_base = 0, idv = 0;
  f16x8 qv[RT][P::NC];
  int pos[RT];
  bool valid[RT];
  // block ids of the wave's run for blocks base .. base + 63 (lane j: block base + j)
  auto load_ids = [&](int base) __attribute__((always_inline)) {
    int page = ((base + lane) * kDmaKeys + 16 * r) >> a.bs_log2;
    page = page < a.W ? page : a.W - 1;
    return trow[page];
  };
  auto block_id = [&](int kb) __attribute__((always_inline)) {
    return clamp_block(__builtin_amdgcn_readlane(idv, kb - kb_base), a.NB);
  };
  // takes the unit at (x, sp) and issues its block ids, the lanes' queries and
  // the DMA of the half's first block into stage 0
  auto open_unit = [&]() __attribute__((always_inline)) {
    h = sp.h;
    q0 = sp.w.q0;
    total_rows = sp.w.n * G;
    cached = sp.w.cached;
    r0 = sp.rb * kDmaRows;
    r_last = min(r0 + kDmaRows, total_rows) - 1;
    key_end = cached + r_last / G + 1;  // keys the row block reads
    nb = rb_blocks(a, sp.w, sp.rb);
    kb_lo = sp.kb;
    kb_hi = min(nb, kb_lo + (x_end - x));
    unit_start = x - kb_lo;
    split = kb_lo > 0 || kb_hi < nb;  // other workgroups hold blocks of the unit
    wr0 = r0 + r * 16 * RT;  // first row of this wave
    has_rows = wr0 <= r_last;
    trow = a.tables + (int64_t)sp.s * a.W;
    kb_first = kb_lo + H;  // this half's blocks: kb_first, kb_first + 2, ...
    kb_base = kb_first;
    idv = load_ids(kb_first);  // before the queries: the DMA below waits for the ids only
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int row = wr0 + 16 * rt + n;
      valid[rt] = row < total_rows;
      const int rc = valid[rt] ? row : r_last;
      pos[rt] = cached + rc / G;
      const f16* qrow = a.q + (int64_t)(q0 + rc / G) * a.q_stride + (h * G + rc % G) * D + 8 * g;
#pragma unroll
      for (int c = 0; c < P::NC; ++c) {
        const f16x8 v = ld16(qrow + 32 * c);
        qv[rt][c] = valid[rt] ? v : f16x8{};
      }
    }
    // blocks whose last key is <= every row's position of this wave need no mask
    unmasked_blocks = (cached + min(wr0, r_last) / G + 1) / kDmaKeys;
    if (kb_first < kb_hi)
      dma_run<D>(a, h, r, kb_first * kDmaKeys + 16 * r, key_end, block_id(kb_first), voff_k,
                 voff_v, k0, v0);
  };
  // moves sp to the unit after the current one: next row block, head, then
  // sequence; false past the last sequence
  auto next_unit = [&]() __attribute__((always_inline)) {
    sp.kb = 0;
    if (++sp.rb == sp.w.R) {
      sp.rb = 0;
      if (++sp.h == a.Hkv) {
        sp.h = 0;
        do {
          ++sp.s;
        } while (sp.s < a.S && (sp.w = seq_work(a, sp.s)).tb == 0);
        if (sp.s >= a.S) return false;
      }
    }
    return true;
  };

  // the range's first unit when it is split and the range holds more: its
  // ticket is drawn one barrier later, and its merge, if it falls to this
  // workgroup, waits for the end of the range
  bool pend = false;

  open_unit();
  if constexpr (PLANNED) {
    // one wave reads the lengths and posts the verdict for the barrier below
    if (H == 0 && r == 0) {
      const int stale = lens_digest(a) != plan_digest;
      if (lane == 0) last[9] = stale;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if constexpr (PLANNED) {
    if (last[9]) {  // workgroup-uniform; nothing stored yet, no ticket drawn
      refuse_plan<D, E>(a, kPPlanErrStale);
      return;
    }
  }
  while (true) {
    float m_run[RT];
    f32x4 o[RT][P::NX];
    f32x4 lsum[RT];  // ones-tile accumulators: every element is the row's sum of P
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      m_run[rt] = kNegInf;
      lsum[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int xx = 0; xx < P::NX; ++xx) o[rt][xx] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // ---- one block: S^T = K.Q^T, online softmax, O^T += V^T.P^T ----
    auto compute = [&](int kb, const unsigned char* kbase,
                       const unsigned char* vbase) __attribute__((always_inline)) {
      dma_block<D, RT, E>(kb, kbase, vbase, unmasked_blocks, a.scale_log2, qv, pos, m_run, lsum, o);
    };

    // ---- pipeline: the DMA of the half's next block (kb + 2) runs while block
    //      kb is computed; the loop is unrolled by two so each step names its
    //      stage objects; both halves take the same number of steps ----
    const int nsteps = (kb_hi - kb_lo + 1) / 2;
    auto step = [&](int j, unsigned char* kc, unsigned char* vc, unsigned char* kn,
                    unsigned char* vn) __attribute__((always_inline)) {
      const int kb = kb_first + 2 * j;
      if (kb + 2 < kb_hi) {
        if (kb + 2 - kb_base >= kWave) {
          kb_base = kb + 2;
          idv = load_ids(kb_base);
        }
        dma_run<D>(a, h, r, (kb + 2) * kDmaKeys + 16 * r, key_end, block_id(kb + 2), voff_k,
                   voff_v, kn, vn);
      }
      if (has_rows && kb < kb_hi) compute(kb, kc, vc);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
    };
    for (int j = 0; j < nsteps; j += 2) {
      step(j, k0, v0, k1, v1);
      if (j + 1 < nsteps) step(j + 1, k1, v1, k0, v0);
    }

    // ---- what the store of this unit needs; then the next unit's loads ----
    const bool st_ok = has_rows && valid[H];
    const int st_row = wr0 + 16 * H + n;
    const int st_q0 = q0, st_h = h, st_r0 = r0, total_rows_st = total_rows;
    const bool st_split = split;
    const uint32_t slot = 2u * gid + (x_begin < unit_start ? 1u : 0u);
    // a split unit's contributors: workgroups x0 .. x0 + ncontrib - 1
    const int x0 = st_split ? pl.rg.owner(unit_start) : 0;
    const int ncontrib = st_split ? pl.rg.owner(unit_start + nb - 1) - x0 + 1 : 1;
    const uint32_t slot_x0 = 2u * x0 + (pl.rg.start(x0) < unit_start ? 1u : 0u);
    const int x_next = x + (kb_hi - kb_lo);
    const bool more = x_next < x_end && next_unit();
    if (more) {
      x = x_next;
      open_unit();
    }

    // ---- the two halves' states of the unit's rows meet in LDS (stage 1 is
    //      idle: the next unit's first block goes to stage 0): tile rt = H
    //      stays, tile 1 - H goes to the partner wave (1 - H, r), which holds
    //      the same rows ----
    {
      float* xo = reinterpret_cast<float*>((r < 2 ? k1 : v1) + (r & 1) * P::NX * kWave * 16);
#pragma unroll
      for (int xx = 0; xx < P::NX; ++xx)
        *reinterpret_cast<f32x4*>(xo + (xx * kWave + lane) * 4) = o[1 - H][xx];
      float* xm = xml + (H * kHalfWaves + r) * 2 * kWave;
      xm[lane] = m_run[1 - H];
      xm[kWave + lane] = lsum[1 - H][0];
    }
    __syncthreads();
    {
      const float* xp =
          reinterpret_cast<const float*>((r < 2 ? pk1 : pv1) + (r & 1) * P::NX * kWave * 16);
      const float* xm = xml + ((1 - H) * kHalfWaves + r) * 2 * kWave;
      const float pm = xm[lane];
      const float pl = xm[kWave + lane];
      const float mm = fmaxf(m_run[H], pm);
      const float a0 = m_run[H] == kNegInf ? 0.f : exp2_fast(m_run[H] - mm);
      const float a1 = pm == kNegInf ? 0.f : exp2_fast(pm - mm);
#pragma unroll
      for (int xx = 0; xx < P::NX; ++xx)
        o[H][xx] = a0 * o[H][xx] + a1 * *reinterpret_cast<const f32x4*>(xp + (xx * kWave + lane) * 4);
      lsum[H][0] = a0 * lsum[H][0] + a1 * pl;
      m_run[H] = mm;
    }

    // ---- the whole unit here: store.  Part of it: normalised partial and
    //      base-2 LSE (fp32, device-coherent stores), then the unit's ticket;
    //      the last contributor merges every partial of the unit's rows ----
    const int64_t st_orow =
        (int64_t)(st_q0 + st_row / G) * a.Hq + st_h * G + st_row % G;  // output row
    if (!st_split) {
      if (st_ok) {
        const float l = lsum[H][0];
        const float inv = l > 0.f ? 1.f / l : 0.f;
        f16* orow = a.out + st_orow * D + 4 * g;
#pragma unroll
        for (int xx = 0; xx < P::NX; ++xx)
          *reinterpret_cast<f16x4*>(orow + 16 * xx) = to16x4<E>(o[H][xx] * inv);
      }
    } else {
      const __amdgpu_buffer_rsrc_t ro = part_rsrc_o<D>(a, pl.rg.nwg);
      const __amdgpu_buffer_rsrc_t rl = part_rsrc_lse(a, pl.rg.nwg);
      const uint32_t urow = (uint32_t)(st_row - st_r0);  // row within the unit
      const float l = lsum[H][0];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float own_lse = l > 0.f ? m_run[H] + log2f(l) : kNegInf;
      // At the end of its range the workgroup is usually the unit's last
      // contributor (the others took the unit's later blocks at the start of
      // theirs): if all of them have drawn their tickets, it merges from its
      // registers and stores no partial of its own.
      bool fast = false;
      if (!more) {
        if (threadIdx.x == 0)
          *last = __hip_atomic_load(a.tickets + x0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  ncontrib - 1;
        __syncthreads();
        fast = *last;  // workgroup-uniform
      }
      if (!fast) {
        if (st_ok) {
          const uint32_t prow = slot * kDmaRows + urow;
#pragma unroll
          for (int xx = 0; xx < P::NX; ++xx)
            __builtin_amdgcn_raw_buffer_store_b128(
                __builtin_bit_cast(u32x4, o[H][xx] * inv), ro,
                (prow * D + 16 * xx + 4 * g) * (uint32_t)sizeof(float), 0, kSc1);
          if (g == 0)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, own_lse), rl,
                                                  prow * (uint32_t)sizeof(float), 0, kSc1);
        }
        if (more) {
          // the range's first unit: what its merge needs, kept in LDS
          pend = true;
          if (threadIdx.x == 0) {
            last[2] = x0;
            last[3] = ncontrib;
            last[4] = (int)slot_x0;
            last[5] = st_q0;
            last[6] = st_h;
            last[7] = st_r0;
            last[8] = total_rows_st;
          }
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial is complete
          __syncthreads();  // every thread has read *last
          if (threadIdx.x == 0)
            *last = __hip_atomic_fetch_add(a.tickets + x0, 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) == ncontrib - 1;
          __syncthreads();
        }
      }
      if (fast || (!more && *last)) {  // workgroup-uniform
        if (threadIdx.x == 0)
          __hip_atomic_store(a.tickets + x0, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (st_ok) {
          f32x4 own[P::NX];
#pragma unroll
          for (int xx = 0; xx < P::NX; ++xx) own[xx] = o[H][xx] * inv;
          merge_split_rows<D, E>(a, ro, rl, x0, ncontrib, slot_x0, fast ? gid - x0 : -1, urow,
                                 st_orow, own, own_lse);
        }
      }
    }
    if (!more) break;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next unit's ids, queries, block
    __syncthreads();  // ... and the exchange has been read before stage 1 is refilled
    // the first unit's partial is complete in every wave: draw its ticket (the
    // result is read at the end of the range)
    if (st_split && threadIdx.x == 0)
      last[1] = __hip_atomic_fetch_add(a.tickets + x0, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == ncontrib - 1;
  }
  if (pend) {
    __syncthreads();  // last[1] was written before a barrier of a later step
    if (last[1]) {
      // the merge of the range's first unit fell to this workgroup (its other
      // contributors finished later)
      const int f_x0 = __builtin_amdgcn_readfirstlane(last[2]);
      const int f_n = __builtin_amdgcn_readfirstlane(last[3]);
      const uint32_t f_slot_x0 = (uint32_t)__builtin_amdgcn_readfirstlane(last[4]);
      const int f_q0 = __builtin_amdgcn_readfirstlane(last[5]);
      const int f_h = __builtin_amdgcn_readfirstlane(last[6]);
      const int f_r0 = __builtin_amdgcn_readfirstlane(last[7]);
      const int f_rows = min(f_r0 + kDmaRows, __builtin_amdgcn_readfirstlane(last[8])) - f_r0;
      if (threadIdx.x == 0)
        __hip_atomic_store(a.tickets + f_x0, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int urow = r * 16 * RT + 16 * H + n;
      if (urow < f_rows) {
        const int row = f_r0 + urow;
        const f32x4 none[P::NX] = {};
        merge_split_rows<D, E>(a, part_rsrc_o<D>(a, pl.rg.nwg), part_rsrc_lse(a, pl.rg.nwg), f_x0,
                               f_n, f_slot_x0, -1, (uint32_t)urow,
                               (int64_t)(f_q0 + row / G) * a.Hq + f_h * G + row % G, none,
                               kNegInf);
      }
    }
  }
}

// ---- per-step plan of the stream-K kernel (fe_prefill_plan) -----------------
//
// The work split depends only on q_offsets, context_lens and the sizes, which
// every layer of a model step shares: fe_prefill_plan computes it once -- the
// ranges and, per workgroup, its range and first unit -- and
// fe_prefill_paged_planned reads it with one load instead of the scans of
// stream_plan and stream_locate.  Layout (int32): a header of kPPlanInts
// (nwg, T, q, r of the Ranges), a descriptor of kPPlanInts (what the plan was
// computed for: the 64-bit key of the sizes and tensors, the same fields in
// the clear -- magic, the sizes, the q_offsets and context_lens addresses --,
// a digest of their contents, and last an error word the planned kernel
// sets), then kPPlanInts per workgroup: x_begin, x_end, has work, logical id,
// then the StreamPos s, h, rb, kb, q0, n, cached, R, tb.
//
// A planned launch checks the descriptor before anything else: every unit after
// a workgroup's first is located from the live q_offsets / context_lens, so a
// plan of other contents would make workgroups disagree on a unit's size and
// leave its ticket set for the next launch.  On a mismatch the launch writes
// NaN to every output row, sets the error word and returns.
// One wave per workgroup entry of the launch the plan is for (grid nwg_max).
__global__ __launch_bounds__(kWave) void prefill_plan_kernel(const PrefillArgs a, int* plan) {
  const StreamPlan pl = stream_plan(a);
  const int nwg = pl.rg.nwg;
  const int lane = lane_id();
  if (blockIdx.x == 0) {
    const int digest = lens_digest(a);
    const int hdr[4] = {nwg, pl.rg.T, pl.rg.q, pl.rg.r};
    const int desc[kPPlanFields] = {(int)a.plan_key_lo, (int)a.plan_key_hi, kPPlanMagic, a.S,
                                    a.total_q, a.Hq, a.Hkv, a.W, a.BS, a.nwg_max,
                                    lo32(a.q_off), hi32(a.q_off), lo32(a.ctx), hi32(a.ctx),
                                    digest};
    static_assert(kPPlanDigest == kPPlanFields - 1, "the digest closes the descriptor");
    int v = 0;  // zero padding and the error word
#pragma unroll
    for (int i = 0; i < 4; ++i) v = lane == i ? hdr[i] : v;
#pragma unroll
    for (int i = 0; i < kPPlanFields; ++i) v = lane == kPPlanInts + i ? desc[i] : v;
    if (lane < 2 * kPPlanInts) plan[lane] = v;
  }
  int e[13] = {};
  if ((int)blockIdx.x < nwg) {
    const int gid = logical_wg(blockIdx.x, nwg);
    const int x_begin = pl.rg.start(gid);
    const int x_end = pl.rg.start(gid + 1);
    StreamPos sp{};
    if (x_begin < x_end && stream_locate(a, pl.w0, x_begin, sp)) {
      const int v[13] = {x_begin, x_end, 1, gid, sp.s, sp.h, sp.rb, sp.kb,
                         sp.w.q0, sp.w.n, sp.w.cached, sp.w.R, sp.w.tb};
#pragma unroll
      for (int i = 0; i < 13; ++i) e[i] = v[i];
    }
  }
  int out = 0;
#pragma unroll
  for (int i = 0; i < 13; ++i) out = lane == i ? e[i] : out;
  if (lane < kPPlanInts) plan[2 * kPPlanInts + (int)blockIdx.x * kPPlanInts + lane] = out;
}

template <int D, int RT, class E = Fp16, bool PLANNED = false>
__global__ __launch_bounds__(kDmaThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_dma_kernel(const PrefillArgs a) {
  using P = DCfg<D>;
  // K and V of two stages per half as eight LDS objects: the compiler's wait
  // for an LDS DMA before an LDS read is then limited to reads of the object
  // it fills
  __shared__ __align__(16) unsigned char k00[P::MAT];
  __shared__ __align__(16) unsigned char v00[P::MAT];
  __shared__ __align__(16) unsigned char k01[P::MAT];
  __shared__ __align__(16) unsigned char v01[P::MAT];
  __shared__ __align__(16) unsigned char k10[P::MAT];
  __shared__ __align__(16) unsigned char v10[P::MAT];
  __shared__ __align__(16) unsigned char k11[P::MAT];
  __shared__ __align__(16) unsigned char v11[P::MAT];
  __shared__ float xml[2 * kHalfWaves * 2 * kWave];  // row maxima and sums exchanged at unit ends
  // whether this workgroup drew the last ticket of its range's last unit [0]
  // and of its first unit [1], when split; [2..8]: the first unit's merge
  // parameters; [9]: a planned launch's verdict on the lengths (stale plan)
  __shared__ int last[10];

  StreamPlan pl;
  StreamPos sp;
  int gid, x_begin, x_end;
  int plan_digest = 0;
  if constexpr (PLANNED) {
    // the ranges and this workgroup's first unit from the plan: its entry,
    // header and descriptor in one round trip (lanes 0-15 the entry, 16-31 the
    // header, 32-47 the descriptor).  The key of the sizes and tensors is
    // checked here; the digest of the lengths while the first unit's loads
    // are in flight (run_units), or here by workgroups without work.
    const int lane = lane_id();
    const int v = lane < kPPlanInts ? a.plan[2 * kPPlanInts + (int)blockIdx.x * kPPlanInts + lane]
                                    : (lane < 3 * kPPlanInts ? a.plan[lane - kPPlanInts] : 0);
    const uint32_t diff_key = ((uint32_t)readlane_i(v, 2 * kPPlanInts) ^ a.plan_key_lo) |
                              ((uint32_t)readlane_i(v, 2 * kPPlanInts + 1) ^ a.plan_key_hi);
    if (diff_key) {
      refuse_plan<D, E>(a, kPPlanErrSizes);
      return;
    }
    plan_digest = readlane_i(v, 2 * kPPlanInts + kPPlanDigest);
    pl.rg = Ranges{readlane_i(v, 16 + 1), readlane_i(v, 16 + 0), readlane_i(v, 16 + 2),
                   readlane_i(v, 16 + 3)};
    pl.w0 = SeqWork{};
    if ((int)blockIdx.x >= pl.rg.nwg || readlane_i(v, 2) == 0) {
      if (lens_digest(a) != plan_digest) refuse_plan<D, E>(a, kPPlanErrStale);
      return;
    }
    x_begin = readlane_i(v, 0);
    x_end = readlane_i(v, 1);
    gid = readlane_i(v, 3);
    sp.s = readlane_i(v, 4);
    sp.h = readlane_i(v, 5);
    sp.rb = readlane_i(v, 6);
    sp.kb = readlane_i(v, 7);
    sp.w.q0 = readlane_i(v, 8);
    sp.w.n = readlane_i(v, 9);
    sp.w.cached = readlane_i(v, 10);
    sp.w.R = readlane_i(v, 11);
    sp.w.tb = readlane_i(v, 12);
  } else {
    pl = stream_plan(a);
    if ((int)blockIdx.x >= pl.rg.nwg) return;
    gid = logical_wg(blockIdx.x, pl.rg.nwg);
    x_begin = pl.rg.start(gid);
    x_end = pl.rg.start(gid + 1);
    if (x_begin >= x_end) return;
    if (!stream_locate(a, pl.w0, x_begin, sp)) return;
  }

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = w % kHalfWaves;
  if (w < kHalfWaves)
    run_units<D, RT, 0, E, PLANNED>(a, pl, gid, x_begin, x_end, sp, r, k00, v00, k01, v01, k11,
                                    v11, xml, last, plan_digest);
  else
    run_units<D, RT, 1, E, PLANNED>(a, pl, gid, x_begin, x_end, sp, r, k10, v10, k11, v11, k01,
                                    v01, xml, last, plan_digest);
}

// ---------------------------------------------------------------------------
// prefix_dma_kernel: the cascade prefix pass on LDS DMA (block sizes that are
// multiples of 16)
// ---------------------------------------------------------------------------
//
// The tile kernel's cascade work split -- workgroup i: (KV head, key split)
// pair i % P, 64-row block i / P of a group -- with the stream-K kernel's key
// staging and block step.  The group's prefix arrives in 64-key blocks (each
// wave brings an 8-key run by LDS DMA) in a ring of kPfxStages stages, so three
// blocks are in flight while one is computed.  Eight waves, two per SIMD: wave
// r of half H computes rows 16r .. 16r + 15 over keys 32H .. 32H + 31 of every
// block (dma_block on half a block), so the two waves of a SIMD share its
// MFMA and VALU time and hide each other's latencies; at the end the halves'
// states of the same rows meet in LDS.  Each key split writes its normalised
// output and base-2 LSE into its own slot of the prefix result (slot ks of
// query-head row r at r * KS + ks): the decode launch after it folds a row's
// adjacent slots into its own-key attention, so no split merge runs here.
//
// Measured at C3 against a first form with four waves (one per SIMD, whole
// blocks): 20.2 us, of which 8.8 us in the eight-block loop -- per block a
// wave spent ~0.78 us computing (0.23 us of it MFMA) and ~0.17 us issuing its
// DMA, with no second wave to cover either -- and ~4 us of split merge in the
// 48 merging workgroups.
constexpr int kPfxStages = 4;
constexpr int kPfxThreads = 2 * kThreads;  // two halves of four waves
constexpr int kPfxRun = 8;                 // keys of a block each wave brings in

// s_waitcnt operand that waits until at most n vector-memory operations of
// the wave are in flight (they complete in issue order); expcnt and lgkmcnt at
// their maxima, i.e. not waited for.  Issued through the builtin, the compiler
// sees the wait: it knows the LDS DMA of a stage being read has completed and
// adds no wait of its own before the reads.
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(vm_wait(N));
}
constexpr int kWaitVm0 = vm_wait(0);

template <int D, class E>
__global__ __launch_bounds__(kPfxThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefix_dma_kernel(const PrefillArgs a) {
  using P = DCfg<D>;
  constexpr int RT = 1;
  constexpr int ROWS = kWaves * 16;                    // 64 rows: wave r of each half owns 16
  constexpr int VM_BLOCK = 2 * kPfxRun / P::RPI;       // DMA instructions of one wave per block
  static_assert(kPfxStages == 4, "the step sequence below names four stages");
  static_assert(2 * kWaves * kPfxRun == kDmaKeys, "the eight runs cover a block");
  static_assert(2 * P::NX * kWave * 16 <= P::MAT && 2 * kWaves * kWave * 4 <= P::MAT / 2,
                "two waves' tiles per K stage object; the maxima and sums in a V one");
  // one LDS object per stage and matrix, V split by half (keys 0-31 and
  // 32-63): the compiler's wait for an LDS DMA before an LDS read is then
  // limited to reads of the object it fills (half 1's V reads at an offset
  // of 32 rows in a whole-block object were not told apart from the DMA into
  // the other stages, and waited for all of it)
  __shared__ __align__(16) unsigned char k0[P::MAT];
  __shared__ __align__(16) unsigned char k1[P::MAT];
  __shared__ __align__(16) unsigned char k2[P::MAT];
  __shared__ __align__(16) unsigned char k3[P::MAT];
  __shared__ __align__(16) unsigned char vl0[P::MAT / 2];
  __shared__ __align__(16) unsigned char vh0[P::MAT / 2];
  __shared__ __align__(16) unsigned char vl1[P::MAT / 2];
  __shared__ __align__(16) unsigned char vh1[P::MAT / 2];
  __shared__ __align__(16) unsigned char vl2[P::MAT / 2];
  __shared__ __align__(16) unsigned char vh2[P::MAT / 2];
  __shared__ __align__(16) unsigned char vl3[P::MAT / 2];
  __shared__ __align__(16) unsigned char vh3[P::MAT / 2];

  // the last workgroup of the grid writes the suffix starts (read by the
  // decode launch after this one), beside the others' work
  if (blockIdx.x == gridDim.x - 1) {
    typedef __attribute__((address_space(3))) int32_t lds_i32;
    if (a.S + 1 <= (int)(P::MAT / sizeof(int32_t))) {
      // the offsets staged in a stage buffer (one round trip), searched there
      lds_i32* offs = (lds_i32*)(int32_t*)k0;
      for (int i = threadIdx.x; i <= a.S; i += blockDim.x) offs[i] = a.q_off[i];
      __syncthreads();
      write_suffix_starts(a, offs);
    } else {
      write_suffix_starts(a, a.q_off);
    }
    return;
  }
  const int npair = a.Hkv * a.KS;
  const int item = blockIdx.x / npair;
  const int pair = blockIdx.x - item * npair;
  RowBlock rb;
  if (!locate_rows<ROWS, true>(a, item, rb)) return;
  const int h = pair % a.Hkv;
  const int ks = pair / a.Hkv;
  const int G = a.G;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = w / kWaves;  // half: keys 32H .. 32H + 31 of each block
  const int r = w % kWaves;  // row tile
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int total_rows = rb.n * G;
  const int r0 = rb.rb * ROWS;
  const int r_last = min(r0 + ROWS, total_rows) - 1;
  const int key_end = rb.ctx;  // the group's prefix (whole blocks)
  const int nblocks_all = (key_end + kDmaKeys - 1) / kDmaKeys;
  const int per_split = (nblocks_all + a.KS - 1) / a.KS;
  const int kb_lo = min(ks * per_split, nblocks_all);
  const int nb = min(kb_lo + per_split, nblocks_all) - kb_lo;  // this split's blocks
  const int wr0 = r0 + r * 16;
  const bool has_rows = wr0 <= r_last;
  const int32_t* trow = a.tables + (int64_t)rb.q0 * a.W;  // the group's first row

  // pool block of this wave's run of blocks base .. base + 63 (lane j: block
  // base + j; pages past the table repeat its last entry, unused)
  auto load_ids = [&](int base) __attribute__((always_inline)) {
    int page = ((base + lane) * kDmaKeys + kPfxRun * w) >> a.bs_log2;
    page = page < a.W ? page : a.W - 1;
    return trow[page];
  };
  int kb_base = kb_lo;
  int idv = load_ids(kb_lo);

  // this lane's row: query vector (B operand) and last key it may see (the
  // prefix end, or -1 for a row whose context does not pass the prefix)
  f16x8 qv[RT][P::NC];
  int pos[RT];
  bool valid[RT];
  {
    const int row = wr0 + n;
    valid[0] = row < total_rows;
    const int rc = valid[0] ? row : r_last;
    const int L = member_len(a, rb.q0 + rc / G);
    pos[0] = valid[0] && L > rb.ctx ? rb.ctx - 1 : -1;
    const f16* qrow = a.q + (int64_t)(rb.q0 + rc / G) * a.q_stride + (h * G + rc % G) * D + 8 * g;
#pragma unroll
    for (int c = 0; c < P::NC; ++c) {
      const f16x8 v = ld16(qrow + 32 * c);
      qv[0][c] = valid[0] ? v : f16x8{};
    }
  }
  // blocks whose last key is <= every row's position of the wave need no mask
  const int pos_lo = -wave_max_i(-(valid[0] ? min(pos[0], rb.ctx) : rb.ctx));
  const int unmasked_blocks = __builtin_amdgcn_readfirstlane((pos_lo + 1) / kDmaKeys);

  float m_run[RT] = {kNegInf};
  f32x4 lsum[RT] = {f32x4{0.f, 0.f, 0.f, 0.f}};
  f32x4 o[RT][P::NX];
#pragma unroll
  for (int x = 0; x < P::NX; ++x) o[0][x] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int rs = a.Hkv * D * 2;  // pool bytes from one key row to the next
  // loop-invariant DMA lane offsets: key rr of the wave's run lands on K row
  // 8w + rr and on V row 8r + rr of the half's object; the chunk swizzles
  // take those rows
  uint32_t voff_k[P::NI], voff_v[P::NI];
#pragma unroll
  for (int i = 0; i < P::NI; ++i) {
    const int rr = P::RPI * i + lane / P::CPR;
    const int sl = lane % P::CPR;
    voff_k[i] = (uint32_t)(rr * rs + (sl ^ swz_k<D>(kPfxRun * w + rr)) * 16);
    voff_v[i] = (uint32_t)(rr * rs + (sl ^ swz_v<D>(kPfxRun * r + rr)) * 16);
  }
  // wave w brings keys 8w .. 8w + 7 of block kb: K rows 8w of the stage, V
  // rows 8r of the half's V object
  auto issue = [&](int kb, unsigned char* kst, unsigned char* vlo,
                   unsigned char* vhi) __attribute__((always_inline)) {
    const int id = clamp_block(__builtin_amdgcn_readlane(idv, kb - kb_base), a.NB);
    dma_run<D, kPfxRun>(a, h, w, kb * kDmaKeys + kPfxRun * w, key_end, id, voff_k, voff_v, kst,
                        H == 0 ? vlo : vhi, r);
  };

  // the ids, the row's context length and the queries in one round trip;
  // then the first kPfxStages - 1 blocks
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  if (nb > 0) issue(kb_lo, k0, vl0, vh0);
  if (nb > 1) issue(kb_lo + 1, k1, vl1, vh1);
  if (nb > 2) issue(kb_lo + 2, k2, vl2, vh2);

  // step j: block kb_lo + j sits in stage j % 4; once every wave's run of it
  // has landed and every wave is done with block j - 1, block j + 3 goes into
  // the stage block j - 1 used
  auto step = [&](int j, const unsigned char* kc, const unsigned char* vlc,
                  const unsigned char* vhc, unsigned char* kn, unsigned char* vln,
                  unsigned char* vhn) __attribute__((always_inline)) {
    if (j + 2 < nb) wait_vm<2 * VM_BLOCK>();  // blocks j + 1 and j + 2 stay in flight
    else if (j + 1 < nb) wait_vm<VM_BLOCK>();
    else wait_vm<0>();
    // a bare barrier: __syncthreads()'s release fence would also wait for the
    // DMA of blocks j + 1 and j + 2.  The wait above has put this wave's run
    // of block j in LDS; LDS operations of a wave complete in order, and the
    // compiler fences keep every LDS access on its side of the barrier.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (j + 3 < nb) {
      if (j + 3 - (kb_base - kb_lo) >= kWave) {
        // the next 64 blocks' ids (splits past 61 blocks only): the wait is
        // an s_waitcnt the compiler sees, so no path that skips this load
        // carries a pending load into the readlane below
        kb_base = kb_lo + j + 3;
        idv = load_ids(kb_base);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
      }
      issue(kb_lo + j + 3, kn, vln, vhn);
    }
    // the half's keys: K at a constant offset of the stage object, V in the
    // half's own object
    if (has_rows) {
      if (H == 0)
        dma_block<D, RT, E, 2>(kb_lo + j, kc, vlc, unmasked_blocks, a.scale_log2, qv, pos, m_run,
                               lsum, o, 0);
      else
        dma_block<D, RT, E, 2>(kb_lo + j, kc + 32 * P::ROWB, vhc, unmasked_blocks, a.scale_log2,
                               qv, pos, m_run, lsum, o, 32);
    }
  };
  for (int j = 0; j < nb; j += 4) {
    step(j, k0, vl0, vh0, k3, vl3, vh3);
    if (j + 1 < nb) step(j + 1, k1, vl1, vh1, k0, vl0, vh0);
    if (j + 2 < nb) step(j + 2, k2, vl2, vh2, k1, vl1, vh1);
    if (j + 3 < nb) step(j + 3, k3, vl3, vh3, k2, vl2, vh2);
  }

  // ---- the halves' states of the same rows meet in the idle stages (tiles
  //      of waves 0-1 in k0, 2-3 in k1, maxima and sums in vl0): half 1
  //      parks, half 0 combines and writes the split's slot ----
  __syncthreads();  // every wave is done with the stages
  float* xo = reinterpret_cast<float*>(r < 2 ? k0 : k1) + (r & 1) * P::NX * kWave * 4;
  float* xm = reinterpret_cast<float*>(vl0) + r * 2 * kWave;
  if (H == 1) {
#pragma unroll
    for (int x = 0; x < P::NX; ++x)
      *reinterpret_cast<f32x4*>(xo + (x * kWave + lane) * 4) = o[0][x];
    xm[lane] = m_run[0];
    xm[kWave + lane] = lsum[0][0];
  }
  __syncthreads();
  if (H == 1 || !valid[0]) return;
  const float pm = xm[lane];
  const float mm = fmaxf(m_run[0], pm);
  const float a0 = m_run[0] == kNegInf ? 0.f : exp2_fast(m_run[0] - mm);
  const float a1 = pm == kNegInf ? 0.f : exp2_fast(pm - mm);
  const float l = a0 * lsum[0][0] + a1 * xm[kWave + lane];
  const float inv = l > 0.f ? 1.f / l : 0.f;
  const int row = wr0 + n;
  const int64_t slot_row =
      ((int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G) * a.KS + ks;
  float* orow = a.pre_o + slot_row * D + 4 * g;
#pragma unroll
  for (int x = 0; x < P::NX; ++x)
    *reinterpret_cast<f32x4*>(orow + 16 * x) =
        (a0 * o[0][x] + a1 * *reinterpret_cast<const f32x4*>(xo + (x * kWave + lane) * 4)) * inv;
  if (g == 0) a.pre_lse[slot_row] = l > 0.f ? mm + log2f(l) : kNegInf;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int log2_exact(int x) {
  if (x <= 0 || (x & (x - 1))) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

template <int D, int RT, class E = Fp16, bool PAD = false, int DC = D>
void launch_prefill(const PrefillArgs& a, int blocks, hipStream_t stream) {
  using P = PCfg<D, RT>;
  hipLaunchKernelGGL((prefill_kernel<D, RT, E, PAD, DC>), dim3(blocks * a.Hkv * a.KS),
                     dim3(kThreads), 2 * P::STAGE, stream, a);
}

// RT 16-row MFMA tiles per wave of the stream-K kernel: two, so every K/V
// fragment read from LDS feeds two MFMAs (VGPRs allow 2 waves per SIMD).
constexpr int kDmaRt = 2;

// Compute units of the current device (queried once per device).
int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  static int cache[64] = {};
  if (dev >= 0 && dev < 64 && cache[dev] > 0) return cache[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev >= 0 && dev < 64) cache[dev] = cus;
  return cus;
}
// One stream-K workgroup per CU (LDS: 128 KiB of stages at D = 128).
inline int stream_wgs() { return device_cus(); }

template <int D, class E>
void launch_prefill_dma(const PrefillArgs& a, hipStream_t stream) {
  constexpr int RT = kDmaRt;
  if (a.plan != nullptr)
    hipLaunchKernelGGL((prefill_dma_kernel<D, RT, E, true>), dim3(a.nwg_max), dim3(kDmaThreads),
                       0, stream, a);
  else
    hipLaunchKernelGGL((prefill_dma_kernel<D, RT, E>), dim3(a.nwg_max), dim3(kDmaThreads), 0,
                       stream, a);
}

constexpr int kMaxTickets = 65536;
constexpr size_t kTicketBytes = kMaxTickets * sizeof(int);
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Launch shape from host-side sizes only (context lengths live on the device):
// rows per workgroup (RT), an upper bound on the row blocks, and the key
// splits KS, aiming at about 1024 workgroups (four per CU).
struct Plan {
  int rt, blocks, ks;
};
// rt2: whether the kernel to launch has a two-row-tile form (head_dim 256 has
// one only: its row blocks, and so the grid, are then sized for one tile)
inline Plan plan(int num_seqs, int total_q, int num_q_heads, int kv_heads, bool rt2 = true) {
  const int64_t rows = (int64_t)total_q * num_q_heads;  // (token, query head) rows
  Plan p;
  p.rt = rt2 && rows >= (int64_t)kRt2Blocks * PCfg<128, 2>::ROWS ? 2 : 1;
  const int per = kWaves * 16 * p.rt;
  const int G = num_q_heads / kv_heads;
  p.blocks = (int)(((int64_t)total_q * G + per - 1) / per) + num_seqs;
  const int64_t wgs = (int64_t)((rows + per - 1) / per) * 1;
  int ks = (int)((1024 + wgs - 1) / (wgs > 0 ? wgs : 1));
  ks = ks < 1 ? 1 : (ks > kMaxSplits ? kMaxSplits : ks);
  // round KS up so that the (KV head, split) pairs divide 8 or fill a multiple
  // of 8 (the XCD-affine grid order of prefill_kernel), when that stays within
  // kMaxSplits
  for (int k = ks; k <= kMaxSplits; ++k) {
    const int pairs = kv_heads * k;
    if (8 % pairs == 0 || pairs % 8 == 0) {
      ks = k;
      break;
    }
  }
  p.ks = ks;
  // the split partials are addressed with 32-bit offsets (at most ~128K rows
  // split at all, ~256 MB)
  if (p.ks > 1 && (int64_t)p.ks * rows * 128 * (int64_t)sizeof(float) >= ((int64_t)1 << 31))
    p.ks = 1;
  return p;
}

// Whether the stream-K kernel takes a launch: block sizes that are multiples
// of 16 (every 16-key run of a 64-key block lies in one page), and sizes whose
// block counts stay within the 32-bit closed form of the work split.
inline bool stream_ok(int block_size, int table_stride, int total_q, int G, int num_seqs,
                      int kv_heads, int nwg) {
  if (block_size % 16 != 0 || nwg <= 0 || nwg > kMaxStreamWgs) return false;
  const int64_t max_ctx = (int64_t)table_stride * block_size;
  const int64_t units = ((int64_t)total_q * G + kDmaRows - 1) / kDmaRows + num_seqs;
  // closed-form operands within 32 bits; total key blocks within 31 bits (a
  // row block reads at most the context plus its own new rows' positions)
  return max_ctx * G < ((int64_t)1 << 28) && (int64_t)total_q * G < ((int64_t)1 << 28) &&
         units * kv_heads * ((max_ctx + total_q) / kDmaKeys + 2) < ((int64_t)1 << 31);
}

// Partial slots of the stream-K kernel: two per workgroup, 128 rows each.
inline size_t stream_ws_bytes(int head_dim) {
  const size_t rows = (size_t)2 * stream_wgs() * kDmaRows;
  return kTicketBytes + align256(rows * head_dim * sizeof(float)) + align256(rows * sizeof(float));
}

}  // namespace

extern "C" size_t fe_prefill_workspace_size(int num_seqs, int total_q, int num_q_heads,
                                            int kv_heads, int head_dim) {
  if (num_seqs < 0 || total_q < 0 || num_q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      num_q_heads % kv_heads)
    return 0;
  // enough for either kernel (the size does not depend on the block size)
  const Plan p = plan(num_seqs, total_q, num_q_heads, kv_heads);
  // the padded tile kernel keeps its partials at the computed head_dim
  const int dc = mfma_padded_head_dim(head_dim);
  size_t need = kTicketBytes;
  if (p.ks > 1) {
    const size_t rows = (size_t)p.ks * total_q * num_q_heads;
    need += align256(rows * dc * sizeof(float)) + align256(rows * sizeof(float));
  }
  const size_t sk = stream_ws_bytes(dc);
  return need > sk ? need : sk;
}

namespace {

bool aligned_to(const void* p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// head_dim other than 64 / 128: the generic kernel (one workgroup per token and
// KV head, causal over the sequence's cached keys and the chunk up to the
// token), no workspace and no plan.
int prefill_generic(const void* q, void* out, const void* k_pool, const void* v_pool,
                    int num_blocks, const int32_t* block_tables, int table_stride,
                    const int32_t* q_offsets, const int32_t* context_lens, int num_seqs,
                    int total_q, int num_q_heads, int kv_heads, int head_dim, int block_size,
                    float scale, hipStream_t stream, bool planned, int elem) {
  if (!generic_shape(num_q_heads, kv_heads, head_dim) || planned) return FE_ERR_UNSUPPORTED;
  if (log2_exact(block_size) < 0) return FE_ERR_UNSUPPORTED;
  // key indices and pool rows (block * block_size + offset) are 32-bit in the kernel
  if ((int64_t)table_stride * block_size >= ((int64_t)1 << 31) ||
      (int64_t)num_blocks * block_size >= ((int64_t)1 << 31))
    return FE_ERR_UNSUPPORTED;
  if (num_seqs == 0 || total_q == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && q_offsets && context_lens);
  const size_t el = elem == 2 ? 4 : 2;
  FE_CHECK_ARG(aligned_to(q, el) && aligned_to(out, el) && aligned_to(k_pool, el) &&
               aligned_to(v_pool, el));
  GenericAttn g{};
  g.q = q;
  g.q_stride = (int64_t)num_q_heads * head_dim;
  g.out = out;
  g.out_stride = g.q_stride;
  g.k_pool = const_cast<void*>(k_pool);
  g.v_pool = const_cast<void*>(v_pool);
  g.num_blocks = num_blocks;
  g.tables = block_tables;
  g.table_stride = table_stride;
  g.ctx = context_lens;
  g.q_offsets = q_offsets;
  g.num_seqs = num_seqs;
  g.rows = total_q;
  g.hq = num_q_heads;
  g.hkv = kv_heads;
  g.d = head_dim;
  g.bs = block_size;
  g.scale = scale;
  g.elem = elem;
  return generic_attention(g, stream);
}

// fe_prefill_paged and its bf16 form: argument checks, workspace carving, launch.
int prefill_impl(const void* q, void* out, const void* k_pool, const void* v_pool, int num_blocks,
                 const int32_t* block_tables, int table_stride, const int32_t* q_offsets,
                 const int32_t* context_lens, int num_seqs, int total_q, int max_q_len,
                 int num_q_heads, int kv_heads, int head_dim, int block_size, float scale,
                 void* workspace, size_t workspace_bytes, fe_stream_t stream, bool bf16,
                 void* step_plan = nullptr, size_t plan_bytes = 0, bool f32 = false) {
  FE_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 &&
               kv_heads > 0 && num_blocks > 0 && table_stride > 0);
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  // head_dim 256 in 16 bits runs on the tile kernel (one row tile per wave, no
  // plan); other head dims on the generic kernel
  const bool mfma256 = head_dim == 256 && !f32 && step_plan == nullptr;
  // other multiples of 8 below 256 in 16 bits (no plan): the tile kernel at the
  // next of 64 / 128 / 256, the dims past head_dim zeros
  // (fp32: the fp32 engine at 64 / 128)
  const int dpad = mfma_padded_head_dim(head_dim);
  const bool padded = dpad != head_dim && step_plan == nullptr && (!f32 || dpad <= 128);
  if (head_dim != 64 && head_dim != 128 && !mfma256 && !padded)
    return prefill_generic(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride,
                           q_offsets, context_lens, num_seqs, total_q, num_q_heads, kv_heads,
                           head_dim, block_size, scale, (hipStream_t)stream,
                           step_plan != nullptr, bf16 ? 1 : (f32 ? 2 : 0));
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  // pool rows (block * block_size + offset) are 32-bit in the kernel
  if ((int64_t)num_blocks * block_size >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(scale > 0.f);  // the kernel takes the row max on unscaled scores
  if (num_seqs == 0 || total_q == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && q_offsets && context_lens);
  FE_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(k_pool) && aligned16(v_pool));
  if (f32) {
    // fp32 pools: prefill_f32_kernel, 64 rows per workgroup, no workspace
    if (step_plan != nullptr) return FE_ERR_UNSUPPORTED;
    PrefillArgs a{};
    a.q = (const f16*)q;
    a.out = (f16*)out;
    a.k_pool = (const f16*)k_pool;
    a.v_pool = (const f16*)v_pool;
    a.tables = block_tables;
    a.q_off = q_offsets;
    a.ctx = context_lens;
    a.q_stride = (int64_t)num_q_heads * head_dim;
    a.W = table_stride;
    a.S = num_seqs;
    a.total_q = total_q;
    a.Hq = num_q_heads;
    a.Hkv = kv_heads;
    a.G = num_q_heads / kv_heads;
    a.BS = block_size;
    a.bs_log2 = bs_log2;
    a.NB = num_blocks;
    a.KS = 1;
    a.dr = head_dim;
    a.scale_log2 = scale * kLog2e;
    const int64_t blocks = ((int64_t)total_q * a.G + kWaves * 16 - 1) / (kWaves * 16) + num_seqs;
    if (blocks * kv_heads >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)(blocks * kv_heads));
    const hipStream_t s = (hipStream_t)stream;
    const bool list = block_size % kTile == 0;  // tile rows held per lane
    if (padded && dpad == 64 && list)
      hipLaunchKernelGGL((prefill_f32_kernel<64, true, false, true>), grid, dim3(kThreads), 0, s, a);
    else if (padded && dpad == 64)
      hipLaunchKernelGGL((prefill_f32_kernel<64, false, false, true>), grid, dim3(kThreads), 0, s, a);
    else if (padded && list)
      hipLaunchKernelGGL((prefill_f32_kernel<128, true, false, true>), grid, dim3(kThreads), 0, s, a);
    else if (padded)
      hipLaunchKernelGGL((prefill_f32_kernel<128, false, false, true>), grid, dim3(kThreads), 0, s, a);
    else if (head_dim == 64 && list)
      hipLaunchKernelGGL((prefill_f32_kernel<64, true>), grid, dim3(kThreads), 0, s, a);
    else if (head_dim == 64)
      hipLaunchKernelGGL((prefill_f32_kernel<64, false>), grid, dim3(kThreads), 0, s, a);
    else if (list)
      hipLaunchKernelGGL((prefill_f32_kernel<128, true>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((prefill_f32_kernel<128, false>), grid, dim3(kThreads), 0, s, a);
    return FE_LAUNCH_STATUS();
  }
  const int nwg = stream_wgs();
  const bool dma = head_dim != 256 && !padded &&
                   stream_ok(block_size, table_stride, total_q, num_q_heads / kv_heads, num_seqs,
                             kv_heads, nwg);
  // (the workspace size takes the two-tile plan: its key splits are never fewer)
  const Plan p = plan(num_seqs, total_q, num_q_heads, kv_heads, dpad != 256);
  // split-K tickets of prefill_kernel: one per (row block, KV head)
  if (!dma && (int64_t)p.blocks * kv_heads > kMaxTickets) return FE_ERR_UNSUPPORTED;
  // a plan is for the stream-K kernel (fe_prefill_plan refuses the sizes it cannot take)
  if (step_plan != nullptr && !dma) return FE_ERR_UNSUPPORTED;
  if (step_plan != nullptr && (plan_bytes < pplan_bytes() || !aligned16(step_plan)))
    return FE_ERR_WORKSPACE;
  const size_t need = fe_prefill_workspace_size(num_seqs, total_q, num_q_heads, kv_heads, head_dim);
  if (workspace == nullptr || workspace_bytes < need || !aligned16(workspace))
    return FE_ERR_WORKSPACE;

  PrefillArgs a;
  a.q = (const f16*)q;
  a.out = (f16*)out;
  a.k_pool = (const f16*)k_pool;
  a.v_pool = (const f16*)v_pool;
  a.tables = block_tables;
  a.q_off = q_offsets;
  a.ctx = context_lens;
  char* ws = (char*)workspace;
  a.tickets = (int*)ws;
  ws += kTicketBytes;
  const size_t rows = dma ? (size_t)2 * nwg * kDmaRows : (size_t)p.ks * total_q * num_q_heads;
  a.part_o = (float*)ws;
  ws += align256(rows * (padded ? dpad : head_dim) * sizeof(float));
  a.part_lse = (float*)ws;
  ws += align256(rows * sizeof(float));
  a.W = table_stride;
  a.S = num_seqs;
  a.total_q = total_q;
  a.Hq = num_q_heads;
  a.Hkv = kv_heads;
  a.G = num_q_heads / kv_heads;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.KS = dma ? 1 : p.ks;
  a.nwg_max = nwg;
  a.dr = head_dim;
  a.scale_log2 = scale * kLog2e;
  a.q_stride = (int64_t)num_q_heads * head_dim;
  a.prefix_len = nullptr;
  a.pre_o = nullptr;
  a.pre_lse = nullptr;
  a.tok0 = nullptr;
  a.plan = (int*)step_plan;
  if (a.plan != nullptr) set_pplan_key(a);
  hipStream_t s = (hipStream_t)stream;
  if (dma && bf16) {
    if (head_dim == 64) launch_prefill_dma<64, Bf16>(a, s); else launch_prefill_dma<128, Bf16>(a, s);
  } else if (dma) {
    if (head_dim == 64) launch_prefill_dma<64, Fp16>(a, s); else launch_prefill_dma<128, Fp16>(a, s);
  } else if (padded && dpad == 256) {
    // computed dims: 160 (head_dim 136-160), 192 (168-192), else all 256
    if (head_dim <= 160) {
      if (bf16) launch_prefill<256, 1, Bf16, true, 160>(a, p.blocks, s);
      else launch_prefill<256, 1, Fp16, true, 160>(a, p.blocks, s);
    } else if (head_dim <= 192) {
      if (bf16) launch_prefill<256, 1, Bf16, true, 192>(a, p.blocks, s);
      else launch_prefill<256, 1, Fp16, true, 192>(a, p.blocks, s);
    } else {
      if (bf16) launch_prefill<256, 1, Bf16, true>(a, p.blocks, s);
      else launch_prefill<256, 1, Fp16, true>(a, p.blocks, s);
    }
  } else if (padded && dpad == 128 && head_dim <= 96) {
    // head_dim 72-96: 96 computed dims of 128
    if (bf16) p.rt == 2 ? launch_prefill<128, 2, Bf16, true, 96>(a, p.blocks, s)
                        : launch_prefill<128, 1, Bf16, true, 96>(a, p.blocks, s);
    else p.rt == 2 ? launch_prefill<128, 2, Fp16, true, 96>(a, p.blocks, s)
                   : launch_prefill<128, 1, Fp16, true, 96>(a, p.blocks, s);
  } else if (padded) {
    const bool r2 = p.rt == 2;
    if (dpad == 64) {
      if (bf16) r2 ? launch_prefill<64, 2, Bf16, true>(a, p.blocks, s)
                   : launch_prefill<64, 1, Bf16, true>(a, p.blocks, s);
      else r2 ? launch_prefill<64, 2, Fp16, true>(a, p.blocks, s)
              : launch_prefill<64, 1, Fp16, true>(a, p.blocks, s);
    } else {
      if (bf16) r2 ? launch_prefill<128, 2, Bf16, true>(a, p.blocks, s)
                   : launch_prefill<128, 1, Bf16, true>(a, p.blocks, s);
      else r2 ? launch_prefill<128, 2, Fp16, true>(a, p.blocks, s)
              : launch_prefill<128, 1, Fp16, true>(a, p.blocks, s);
    }
  } else if (head_dim == 256) {
    if (bf16) launch_prefill<256, 1, Bf16>(a, p.blocks, s); else launch_prefill<256, 1>(a, p.blocks, s);
  } else if (bf16) {
    if (head_dim == 64) {
      if (p.rt == 2) launch_prefill<64, 2, Bf16>(a, p.blocks, s);
      else launch_prefill<64, 1, Bf16>(a, p.blocks, s);
    } else {
      if (p.rt == 2) launch_prefill<128, 2, Bf16>(a, p.blocks, s);
      else launch_prefill<128, 1, Bf16>(a, p.blocks, s);
    }
  } else if (head_dim == 64) {
    if (p.rt == 2) launch_prefill<64, 2>(a, p.blocks, s); else launch_prefill<64, 1>(a, p.blocks, s);
  } else {
    if (p.rt == 2) launch_prefill<128, 2>(a, p.blocks, s); else launch_prefill<128, 1>(a, p.blocks, s);
  }
  return FE_LAUNCH_STATUS();
}

}  // namespace

extern "C" int fe_prefill_paged(const void* q, void* out, const void* k_pool, const void* v_pool,
                                int num_blocks, const int32_t* block_tables, int table_stride,
                                const int32_t* q_offsets, const int32_t* context_lens,
                                int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                int kv_heads, int head_dim, int block_size, float scale,
                                void* workspace, size_t workspace_bytes, fe_stream_t stream) {
  return prefill_impl(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride, q_offsets,
                      context_lens, num_seqs, total_q, max_q_len, num_q_heads, kv_heads, head_dim,
                      block_size, scale, workspace, workspace_bytes, stream, false);
}

extern "C" int fe_prefill_paged_bf16(const void* q, void* out, const void* k_pool,
                                     const void* v_pool, int num_blocks,
                                     const int32_t* block_tables, int table_stride,
                                     const int32_t* q_offsets, const int32_t* context_lens,
                                     int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                     int kv_heads, int head_dim, int block_size, float scale,
                                     void* workspace, size_t workspace_bytes,
                                     fe_stream_t stream) {
  return prefill_impl(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride, q_offsets,
                      context_lens, num_seqs, total_q, max_q_len, num_q_heads, kv_heads, head_dim,
                      block_size, scale, workspace, workspace_bytes, stream, true);
}

extern "C" int fe_prefill_paged_f32(const void* q, void* out, const void* k_pool,
                                    const void* v_pool, int num_blocks,
                                    const int32_t* block_tables, int table_stride,
                                    const int32_t* q_offsets, const int32_t* context_lens,
                                    int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                    int kv_heads, int head_dim, int block_size, float scale,
                                    void* workspace, size_t workspace_bytes,
                                    fe_stream_t stream) {
  return prefill_impl(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride, q_offsets,
                      context_lens, num_seqs, total_q, max_q_len, num_q_heads, kv_heads, head_dim,
                      block_size, scale, workspace, workspace_bytes, stream, false, nullptr, 0,
                      true);
}

extern "C" size_t fe_prefill_plan_size(int num_seqs, int total_q, int num_q_heads,
                                       int kv_heads) {
  if (num_seqs < 0 || total_q < 0 || num_q_heads <= 0 || kv_heads <= 0) return 0;
  return pplan_bytes();
}

extern "C" int fe_prefill_plan(const int32_t* q_offsets, const int32_t* context_lens,
                               int num_seqs, int total_q, int num_q_heads, int kv_heads,
                               int table_stride, int block_size, void* plan, size_t plan_bytes,
                               fe_stream_t stream) {
  FE_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && num_q_heads > 0 && kv_heads > 0 &&
               table_stride > 0);
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  const int nwg = stream_wgs();
  if (!stream_ok(block_size, table_stride, total_q, num_q_heads / kv_heads, num_seqs, kv_heads,
                 nwg))
    return FE_ERR_UNSUPPORTED;
  if (plan == nullptr || plan_bytes < pplan_bytes() || !aligned16(plan)) return FE_ERR_WORKSPACE;
  if (num_seqs == 0 || total_q == 0) return FE_OK;
  FE_CHECK_ARG(q_offsets && context_lens);
  PrefillArgs a{};
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
  a.nwg_max = nwg;
  set_pplan_key(a);
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(nwg), dim3(kWave), 0, (hipStream_t)stream, a,
                     (int*)plan);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_prefill_paged_planned(const void* q, void* out, const void* k_pool,
                                        const void* v_pool, int num_blocks,
                                        const int32_t* block_tables, int table_stride,
                                        const int32_t* q_offsets, const int32_t* context_lens,
                                        int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                        int kv_heads, int head_dim, int block_size, float scale,
                                        void* workspace, size_t workspace_bytes, void* plan,
                                        size_t plan_bytes, fe_stream_t stream) {
  FE_CHECK_ARG(plan != nullptr);
  return prefill_impl(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride, q_offsets,
                      context_lens, num_seqs, total_q, max_q_len, num_q_heads, kv_heads, head_dim,
                      block_size, scale, workspace, workspace_bytes, stream, false, plan,
                      plan_bytes);
}

extern "C" int fe_prefill_paged_planned_bf16(
    const void* q, void* out, const void* k_pool, const void* v_pool, int num_blocks,
    const int32_t* block_tables, int table_stride, const int32_t* q_offsets,
    const int32_t* context_lens, int num_seqs, int total_q, int max_q_len, int num_q_heads,
    int kv_heads, int head_dim, int block_size, float scale, void* workspace,
    size_t workspace_bytes, void* plan, size_t plan_bytes, fe_stream_t stream) {
  FE_CHECK_ARG(plan != nullptr);
  return prefill_impl(q, out, k_pool, v_pool, num_blocks, block_tables, table_stride, q_offsets,
                      context_lens, num_seqs, total_q, max_q_len, num_q_heads, kv_heads, head_dim,
                      block_size, scale, workspace, workspace_bytes, stream, true, plan,
                      plan_bytes);
}

namespace fe {

size_t cascade_prefix_scratch_bytes(int num_groups, int batch, int hq, int hkv, int d) {
  const Plan p = plan(num_groups, batch, hq, hkv);
  if (p.ks == 1) return 0;
  const size_t rows = (size_t)p.ks * batch * hq;
  return align256(rows * d * sizeof(float)) + align256(rows * sizeof(float));
}

int cascade_prefix_launch(CascadePrefix& c, hipStream_t stream) {
  // prefix_dma_kernel: 64-row blocks, each 8-key run of a 64-key block in one
  // page (the shared-prefix decode takes block sizes that are multiples of 16)
  if (c.bs % 16 != 0) return FE_ERR_UNSUPPORTED;
  const Plan p = plan(c.num_groups, c.batch, c.hq, c.hkv);
  const int blocks =
      (int)(((int64_t)c.batch * (c.hq / c.hkv) + kWaves * 16 - 1) / (kWaves * 16)) + c.num_groups;
  if ((int64_t)blocks * c.hkv * p.ks + 1 >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  if ((int64_t)c.num_blocks * c.bs >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  if (!(c.scale > 0.f)) return FE_ERR_INVALID_ARGUMENT;  // row max on unscaled scores
  PrefillArgs a;
  a.plan = nullptr;
  a.q = (const f16*)c.q;
  a.out = nullptr;
  a.k_pool = (const f16*)c.k_pool;
  a.v_pool = (const f16*)c.v_pool;
  a.tables = c.tables;
  a.q_off = c.group_offsets;
  a.ctx = c.ctx;
  a.tickets = nullptr;
  a.part_o = nullptr;
  a.part_lse = nullptr;
  a.q_stride = c.q_stride;
  a.W = c.table_stride;
  a.S = c.num_groups;
  a.total_q = c.batch;
  a.Hq = c.hq;
  a.Hkv = c.hkv;
  a.G = c.hq / c.hkv;
  a.BS = c.bs;
  a.bs_log2 = log2_exact(c.bs);
  a.NB = c.num_blocks;
  a.KS = p.ks;
  a.nwg_max = 0;
  a.scale_log2 = c.scale * kLog2e;
  a.prefix_len = c.prefix_len;
  a.tok0 = c.tok0;
  // every key split writes its own slot (the decode launch folds them in):
  // one slot fits pre_o / pre_lse, several the key-split scratch
  if (p.ks > 1) {
    const size_t rows = (size_t)p.ks * c.batch * c.hq;
    a.pre_o = (float*)c.scratch;
    a.pre_lse = (float*)((char*)c.scratch + align256(rows * c.d * sizeof(float)));
  } else {
    a.pre_o = c.pre_o;
    a.pre_lse = c.pre_lse;
  }
  if (c.f32) {
    // fp32: the fp32 prefill kernel's cascade mode, one slot per row
    a.KS = 1;
    a.pre_o = c.pre_o;
    a.pre_lse = c.pre_lse;
    c.out_o = a.pre_o;
    c.out_lse = a.pre_lse;
    c.splits = 1;
    const dim3 grid(blocks * a.Hkv + 1);  // + the suffix-start workgroup
    if (c.d == 64)
      hipLaunchKernelGGL((prefill_f32_kernel<64, true, true>), grid, dim3(kThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_f32_kernel<128, true, true>), grid, dim3(kThreads), 0, stream, a);
    return FE_LAUNCH_STATUS();
  }
  c.out_o = a.pre_o;
  c.out_lse = a.pre_lse;
  c.splits = p.ks;
  const dim3 grid(blocks * a.Hkv * a.KS + 1);  // + the suffix-start workgroup
  const dim3 block(kPfxThreads);
  if (c.bf16) {
    if (c.d == 64) hipLaunchKernelGGL((prefix_dma_kernel<64, Bf16>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((prefix_dma_kernel<128, Bf16>), grid, block, 0, stream, a);
  } else {
    if (c.d == 64) hipLaunchKernelGGL((prefix_dma_kernel<64, Fp16>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((prefix_dma_kernel<128, Fp16>), grid, block, 0, stream, a);
  }
  return FE_LAUNCH_STATUS();
}

}  // namespace fe
