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
  float* part_o;     // [KS][total_q * Hq][D] normalised partial outputs (KS > 1)
  float* part_lse;   // [KS][total_q * Hq] base-2 LSE of each partial
  int* tickets;      // [row blocks * Hkv], zero between calls
  int64_t q_stride;  // elements from one query row (token or sequence) to the next
  int W, S, total_q, Hq, Hkv, G, BS, bs_log2, NB, KS;
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
    int q0 = 0, n = 0;
    if (s < a.S) {
      // rows outside [0, total_q) are dropped: every row the kernel touches
      // (q, out, the context and table of a decode row) stays in its array
      q0 = min(max(a.q_off[s], 0), a.total_q);
      n = min(a.q_off[s + 1], a.total_q) - q0;
      n = n > 0 ? n : 0;
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
      rb.ctx = __builtin_amdgcn_readfirstlane(CASCADE ? group_prefix(a, rb.s)
                                                      : clamp_len(a.ctx[rb.s]));
      return true;
    }
    carry = readlane_i(incl, kWave - 1);
  }
  return false;
}

__device__ __forceinline__ f32x4 mfma32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Cascade mode: the decode row b shares group s's prefix when its context
// reaches past it; its own decode then starts at the prefix end.  Written by
// the first workgroup for every decode row (0 = no shared prefix).
__device__ void write_suffix_starts(const PrefillArgs& a) {
  for (int b = threadIdx.x; b < a.total_q; b += kThreads) {
    int lo = 0, hi = a.S;  // last group s with q_off[s] <= b
    while (hi - lo > 1) {
      const int mid = (lo + hi) / 2;
      if (a.q_off[mid] <= b) lo = mid; else hi = mid;
    }
    int t = 0;
    if (a.S > 0 && a.q_off[lo] <= b && b < a.q_off[lo + 1]) {
      const int pl = group_prefix(a, lo);
      t = member_len(a, b) > pl ? pl : 0;
    }
    a.tok0[b] = t;
  }
}

template <int D, int RT, bool CASCADE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 8)))
void prefill_kernel(const PrefillArgs a) {
  using P = PCfg<D, RT>;
  extern __shared__ __align__(16) unsigned char smem[];

  if constexpr (CASCADE) {
    if (blockIdx.x == 0) write_suffix_starts(a);
  }
  // workgroup i: (KV head, key split) pair i % P, row block i / P (P = Hkv * KS);
  // the hardware places workgroup i on XCD i % 8, so when P divides 8 or is a
  // multiple of it every XCD serves fixed pairs -- one KV head and one key
  // range of every sequence -- and its L2 holds the K/V its row blocks share
  const int npair = a.Hkv * a.KS;
  const int item = blockIdx.x / npair;
  const int pair = blockIdx.x - item * npair;
  RowBlock rb;
  if (!locate_rows<P::ROWS, CASCADE>(a, item, rb)) return;
  const int h = pair % a.Hkv;
  const int G = a.G;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;

  const int total_rows = rb.n * G;
  const int cached = CASCADE ? 0 : (rb.ctx >= rb.n ? rb.ctx - rb.n : 0);
  const int r0 = rb.rb * P::ROWS;
  const int r_last = min(r0 + P::ROWS, total_rows) - 1;
  // keys the row block reads: causal up to its last position, or the prefix
  const int key_end = CASCADE ? rb.ctx : cached + r_last / G + 1;
  // split ks of KS takes an equal share of the row block's key blocks
  const int ks = pair / a.Hkv;
  const int nblocks_all = (key_end + kBlockKeys - 1) / kBlockKeys;
  const int per_split = (nblocks_all + a.KS - 1) / a.KS;
  const int kb_lo = min(ks * per_split, nblocks_all);
  const int kb_hi = min(kb_lo + per_split, nblocks_all);
  const int wr0 = r0 + w * 16 * RT;                               // first row of this wave

  // ---- this lane's rows: query vectors (B operand), last key each may see
  //      (its position; in cascade mode the prefix end, or -1 for a row whose
  //      context does not reach past the prefix) ----
  f16x8 qv[RT][P::NC];
  int pos[RT];
  bool valid[RT];
  int pos_lo = 0x7fffffff;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int row = wr0 + 16 * rt + n;
    valid[rt] = row < total_rows;
    const int rc = valid[rt] ? row : r_last;
    if constexpr (CASCADE) {
      const int L = member_len(a, rb.q0 + rc / G);
      pos[rt] = valid[rt] && L > rb.ctx ? rb.ctx - 1 : -1;
    } else {
      pos[rt] = valid[rt] ? cached + rc / G : -1;
    }
    if (valid[rt]) pos_lo = min(pos_lo, pos[rt]);
    const f16* qrow = a.q + (int64_t)(rb.q0 + rc / G) * a.q_stride + (h * G + rc % G) * D + 8 * g;
#pragma unroll
    for (int c = 0; c < P::NC; ++c) {
      const f16x8 v = ld16(qrow + 32 * c);
      qv[rt][c] = valid[rt] ? v : f16x8{};
    }
  }

  // blocks whose last key is <= every row's position need no mask
  int unmasked_blocks;
  if constexpr (CASCADE) {
    pos_lo = -wave_max_i(-min(pos_lo, rb.ctx));
    unmasked_blocks = __builtin_amdgcn_readfirstlane((pos_lo + 1) / kBlockKeys);
  } else {
    unmasked_blocks = (cached + min(wr0, r_last) / G + 1) / kBlockKeys;
  }

  float m_run[RT], l_run[RT];
  f32x4 o[RT][P::NX];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m_run[rt] = kNegInf;
    l_run[rt] = 0.f;
#pragma unroll
    for (int x = 0; x < P::NX; ++x) o[rt][x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // ---- K/V block staging: thread t loads 16-byte chunk t % CPR of key rows
  //      t / CPR + KPL * i (keys at or past key_end repeat key_end - 1).  The
  //      block ids a block needs are fetched one iteration before its K/V
  //      loads, so no table access sits in front of a K/V load. ----
  const int32_t* trow = a.tables + (int64_t)(CASCADE ? rb.q0 : rb.s) * a.W;
  const int chunk = tid % P::CPR;
  const int krow = tid / P::CPR;
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
      const int64_t off = (int64_t)(blk * a.BS + (kc & (a.BS - 1))) * (a.Hkv * D) + h * D + chunk * 8;
      kst[i] = ld16(a.k_pool + off);
      vst[i] = ld16(a.v_pool + off);
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
      for (int c = 0; c < P::NC; ++c) {
        const f16x8 kv =
            *reinterpret_cast<const f16x8*>(kbase + (16 * kt + n) * P::KP + (32 * c + 8 * g) * 2);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st[rt][kt] = mfma32(kv, qv[rt][c], st[rt][kt]);
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
        for (int x = 0; x < P::NX; ++x) o[rt][x] *= alpha;
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
            lsum += e;
            p[4 * kt + i] = (f16)e;
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
      for (int x = 0; x < P::NX; ++x) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vb + 32 * x));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(vb + 16 * P::VP + 32 * x));
        const f16x4 l4 = __builtin_bit_cast(f16x4, lo), h4 = __builtin_bit_cast(f16x4, hi);
        const f16x8 va = {l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) o[rt][x] = mfma32(va, pb[rt][ps], o[rt][x]);
      }
    }

    if (more) store_block((kb + 1 - kb_lo) & 1);
    __syncthreads();
  }

  // ---- normalise; one split: store.  Several: write this split's partial
  //      (device-coherent stores), draw a ticket; the last split of the row
  //      block merges all of them.  Lane (g,n) holds O[row n][dims 16x+4g+i]. ----
  const bool split = a.KS > 1;
  const int64_t split_stride = (int64_t)a.total_q * a.Hq;  // rows per split
  // (only used when split; the host keeps KS * rows * D floats under 2 GiB)
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.part_o, 0, split ? (int)(a.KS * split_stride * D * 4) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      a.part_lse, 0, split ? (int)(a.KS * split_stride * 4) : 0, 0x00020000);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float l = l_run[rt] + shfl_xor_f(l_run[rt], 16);
    l += shfl_xor_f(l, 32);
    if (!valid[rt]) continue;
    const int row = wr0 + 16 * rt + n;
    const int64_t orow_idx = (int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (CASCADE && !split) {
      float* orow = a.pre_o + orow_idx * D + 4 * g;
#pragma unroll
      for (int x = 0; x < P::NX; ++x) *reinterpret_cast<f32x4*>(orow + 16 * x) = o[rt][x] * inv;
      if (g == 0) a.pre_lse[orow_idx] = l > 0.f ? m_run[rt] + log2f(l) : kNegInf;
    } else if (!split) {
      f16* orow = a.out + orow_idx * D + 4 * g;
#pragma unroll
      for (int x = 0; x < P::NX; ++x)
        *reinterpret_cast<f16x4*>(orow + 16 * x) =
            f16x4{(f16)(o[rt][x][0] * inv), (f16)(o[rt][x][1] * inv),
                  (f16)(o[rt][x][2] * inv), (f16)(o[rt][x][3] * inv)};
    } else {
      // device-coherent stores through one wave-uniform descriptor per array
      // (the host keeps the partial arrays under 2 GiB)
      const uint32_t prow = (uint32_t)((int64_t)ks * a.total_q * a.Hq + orow_idx);
#pragma unroll
      for (int x = 0; x < P::NX; ++x)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[rt][x] * inv), ro,
                                               (prow * D + 16 * x + 4 * g) * (uint32_t)sizeof(float),
                                               0, kSc1);
      if (g == 0)
        __builtin_amdgcn_raw_buffer_store_b32(
            __builtin_bit_cast(uint32_t, l > 0.f ? m_run[rt] + log2f(l) : kNegInf), rl,
            prow * (uint32_t)sizeof(float), 0, kSc1);
    }
  }
  if (!split) return;
  __shared__ int last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partials are complete
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(a.tickets + item * a.Hkv + h, 1, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) == a.KS - 1;
  __syncthreads();
  if (!last) return;
  if (tid == 0)
    __hip_atomic_store(a.tickets + item * a.Hkv + h, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  // merge: thread -> (row of the block, 4 consecutive dims).  All KS LSEs and
  // partial outputs of a row are loaded at once (indices past KS repeat the
  // last split and get weight 0), so a row costs one round trip to memory.
  constexpr int TPR = D / 4;             // threads per row
  constexpr int RPS = kThreads / TPR;    // rows per pass
  const int d4 = (tid % TPR) * 4;
  for (int row = r0 + tid / TPR; row <= r_last; row += RPS) {
    const int64_t orow_idx = (int64_t)(rb.q0 + row / G) * a.Hq + h * G + row % G;
    float lse[kMaxSplits];
    f32x4 ov[kMaxSplits];
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k) {
      const int kc = k < a.KS ? k : a.KS - 1;
      const uint32_t prow = (uint32_t)(kc * split_stride + orow_idx);
      lse[k] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rl, prow * (uint32_t)sizeof(float), 0, kSc1));
      ov[k] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     ro, (prow * D + d4) * (uint32_t)sizeof(float), 0, kSc1));
    }
    float M = kNegInf;
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k)
      if (k < a.KS) M = fmaxf(M, lse[k]);
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k) {
      const float wgt = k < a.KS && lse[k] != kNegInf ? exp2f(lse[k] - M) : 0.f;
      num += wgt * ov[k];
      den += wgt;
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    if constexpr (CASCADE) {
      *reinterpret_cast<f32x4*>(a.pre_o + orow_idx * D + d4) = num * inv;
      if (d4 == 0) a.pre_lse[orow_idx] = den > 0.f ? M + log2f(den) : kNegInf;
    } else {
      *reinterpret_cast<f16x4*>(a.out + orow_idx * D + d4) =
          f16x4{(f16)(num[0] * inv), (f16)(num[1] * inv), (f16)(num[2] * inv),
                (f16)(num[3] * inv)};
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

template <int D, int RT, bool CASCADE = false>
void launch_prefill(const PrefillArgs& a, int blocks, hipStream_t stream) {
  using P = PCfg<D, RT>;
  hipLaunchKernelGGL((prefill_kernel<D, RT, CASCADE>), dim3(blocks * a.Hkv * a.KS),
                     dim3(kThreads), 2 * P::STAGE, stream, a);
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
inline Plan plan(int num_seqs, int total_q, int num_q_heads, int kv_heads) {
  const int64_t rows = (int64_t)total_q * num_q_heads;  // (token, query head) rows
  Plan p;
  p.rt = rows >= (int64_t)kRt2Blocks * PCfg<128, 2>::ROWS ? 2 : 1;
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

}  // namespace

extern "C" size_t fe_prefill_workspace_size(int num_seqs, int total_q, int num_q_heads,
                                            int kv_heads, int head_dim) {
  if (num_seqs < 0 || total_q < 0 || num_q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      num_q_heads % kv_heads)
    return 0;
  const Plan p = plan(num_seqs, total_q, num_q_heads, kv_heads);
  if (p.ks == 1) return kTicketBytes;
  const size_t rows = (size_t)p.ks * total_q * num_q_heads;
  return kTicketBytes + align256(rows * head_dim * sizeof(float)) + align256(rows * sizeof(float));
}

extern "C" int fe_prefill_paged(const void* q, void* out, const void* k_pool, const void* v_pool,
                                int num_blocks, const int32_t* block_tables, int table_stride,
                                const int32_t* q_offsets, const int32_t* context_lens,
                                int num_seqs, int total_q, int max_q_len, int num_q_heads,
                                int kv_heads, int head_dim, int block_size, float scale,
                                void* workspace, size_t workspace_bytes, fe_stream_t stream) {
  FE_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 &&
               kv_heads > 0 && num_blocks > 0 && table_stride > 0);
  if (head_dim != 64 && head_dim != 128) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(num_q_heads % kv_heads == 0);
  const int bs_log2 = log2_exact(block_size);
  if (bs_log2 < 0) return FE_ERR_UNSUPPORTED;
  // pool rows (block * block_size + offset) are 32-bit in the kernel
  if ((int64_t)num_blocks * block_size >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  FE_CHECK_ARG(scale > 0.f);  // the kernel takes the row max on unscaled scores
  if (num_seqs == 0 || total_q == 0) return FE_OK;
  FE_CHECK_ARG(q && out && k_pool && v_pool && block_tables && q_offsets && context_lens);
  FE_CHECK_ARG(aligned16(q) && aligned16(out) && aligned16(k_pool) && aligned16(v_pool));
  const Plan p = plan(num_seqs, total_q, num_q_heads, kv_heads);
  if ((int64_t)p.blocks * kv_heads > kMaxTickets) return FE_ERR_UNSUPPORTED;
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
  const size_t rows = (size_t)p.ks * total_q * num_q_heads;
  a.part_o = (float*)ws;
  ws += align256(rows * head_dim * sizeof(float));
  a.part_lse = (float*)ws;
  a.W = table_stride;
  a.S = num_seqs;
  a.total_q = total_q;
  a.Hq = num_q_heads;
  a.Hkv = kv_heads;
  a.G = num_q_heads / kv_heads;
  a.BS = block_size;
  a.bs_log2 = bs_log2;
  a.NB = num_blocks;
  a.KS = p.ks;
  a.scale_log2 = scale * kLog2e;
  a.q_stride = (int64_t)num_q_heads * head_dim;
  a.prefix_len = nullptr;
  a.pre_o = nullptr;
  a.pre_lse = nullptr;
  a.tok0 = nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 64) {
    if (p.rt == 2) launch_prefill<64, 2>(a, p.blocks, s); else launch_prefill<64, 1>(a, p.blocks, s);
  } else {
    if (p.rt == 2) launch_prefill<128, 2>(a, p.blocks, s); else launch_prefill<128, 1>(a, p.blocks, s);
  }
  return FE_LAUNCH_STATUS();
}

namespace fe {

size_t cascade_prefix_scratch_bytes(int num_groups, int batch, int hq, int hkv, int d) {
  const Plan p = plan(num_groups, batch, hq, hkv);
  if (p.ks == 1) return 0;
  const size_t rows = (size_t)p.ks * batch * hq;
  return align256(rows * d * sizeof(float)) + align256(rows * sizeof(float));
}

int cascade_prefix_launch(const CascadePrefix& c, hipStream_t stream) {
  const Plan p = plan(c.num_groups, c.batch, c.hq, c.hkv);
  if ((int64_t)p.blocks * c.hkv > kMaxTickets) return FE_ERR_UNSUPPORTED;
  if ((int64_t)c.num_blocks * c.bs >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  if (!(c.scale > 0.f)) return FE_ERR_INVALID_ARGUMENT;  // row max on unscaled scores
  PrefillArgs a;
  a.q = (const f16*)c.q;
  a.out = nullptr;
  a.k_pool = (const f16*)c.k_pool;
  a.v_pool = (const f16*)c.v_pool;
  a.tables = c.tables;
  a.q_off = c.group_offsets;
  a.ctx = c.ctx;
  a.tickets = c.tickets;
  const size_t rows = (size_t)p.ks * c.batch * c.hq;
  a.part_o = (float*)c.scratch;
  a.part_lse = p.ks > 1 ? (float*)((char*)c.scratch + align256(rows * c.d * sizeof(float)))
                        : nullptr;
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
  a.scale_log2 = c.scale * kLog2e;
  a.prefix_len = c.prefix_len;
  a.pre_o = c.pre_o;
  a.pre_lse = c.pre_lse;
  a.tok0 = c.tok0;
  if (c.d == 64) {
    if (p.rt == 2) launch_prefill<64, 2, true>(a, p.blocks, stream);
    else launch_prefill<64, 1, true>(a, p.blocks, stream);
  } else {
    if (p.rt == 2) launch_prefill<128, 2, true>(a, p.blocks, stream);
    else launch_prefill<128, 1, true>(a, p.blocks, stream);
  }
  return FE_LAUNCH_STATUS();
}

}  // namespace fe
