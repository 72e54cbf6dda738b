// Per-wave paged-attention tile engine shared by the decode and prefill kernels.
//
// A wave owns up to 16 "columns" n (decode: the G query heads of one KV head;
// prefill: 16 query rows of one query head) and walks 16-token key tiles of one
// sequence's paged K/V.  Lane l = 16g + n.
//
//   S^T[16 keys x 16 cols] = K[16 x D] . Q^T[D x 16]        (MFMA 16x16x16 f16)
//     A = K: lane (g,n) loads key n of the tile, 16-byte chunks 4s+g (s < D/32),
//            straight from the pool; each chunk feeds two MFMAs.
//     B = Q: lane (g,n) holds column n's query vector, same chunks.
//     -> lane (g,n) holds the scores of column n for keys 4g..4g+3.
//   online softmax in base 2 (scores scaled by scale*log2(e)); column n's
//     running max is shared by its four lanes (g = 0..3) via two xor-shuffles.
//   O^T[D x 16 cols] += V^T[D x 16 keys] . P^T[16 keys x 16 cols]  (D/16 MFMAs)
//     B = P^T is the score layout above, converted to fp16.
//     A = V^T: V rows are loaded with coalesced 16-byte loads (16 lanes per
//            256-byte row), staged in a per-wave LDS tile with a padded pitch
//            and read back column-wise.
//     -> lane (g,n) accumulates O[col n][d = 16x + 4g + i], so the softmax
//        rescale of column n never leaves the lane.
#pragma once

#include "fe_common.h"

namespace fe {

constexpr int kTile = 16;

template <int D>
struct TileCfg {
  static constexpr int NK = D / 32;       // K chunk loads per lane per tile (= V loads)
  static constexpr int NX = D / 16;       // PV output tiles of 16 dims
  static constexpr int CPR = D / 8;       // 16-byte chunks per K/V row
  static constexpr int RPI = kWave / CPR; // V rows covered by one load instruction
  // LDS pitch of a staged V row: D halves + 32 bytes = D/2 + 8 dwords, which is
  // 8 mod 32 for D = 64 and 128.  The transposing read of a 16-dim slice (see
  // softmax_pv_tile) has each 16-lane group fetch 8 bytes from 4 rows x 4
  // consecutive 8-byte columns; rows 8 dwords apart put those 16 fetches on
  // distinct bank pairs.
  static constexpr int ROWB = D * 2 + 32;
  static constexpr int STAGE = kTile * ROWB;
};

__device__ __forceinline__ int clamp_block(int blk, int nb) {
  return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
}

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Running-max slack of the online softmax, in base-2 units: the max a tile's
// scores are exponentiated against is only raised when some column's tile max
// exceeds it by more than this, so most tiles skip the rescale of o and l, and
// every probability stays <= 2^kRescaleSlack (exact in fp16 for the PV MFMA).
constexpr float kRescaleSlack = 8.f;

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Shared softmax + PV step of one 16-key tile (scores already in sacc).
// Lane (g,n): sacc[i] = raw score of key t0 + 4g + i for column n; keys at or
// past `limit` are masked.  V rows of the tile are in `stage` (row pitch ROWB).
//
// The PV product O^T[16 dims x 16 cols] += V^T . P^T takes its A operand
// (lane (g,n): V[key 4g+i][dim 16x+n], i = 0..3) from one transposing LDS read
// per 16-dim slice: ds_read_b64_tr_b16 returns to lane l of a 16-lane group
// the halves M[4j + l/4][l%4] (j = 0..3), M[r] being the 8 bytes addressed by
// lane r of the group; lane (g, r) therefore addresses
// V[key 4g + r/4][dims 16x + 4(r%4) .. +3].
template <int D, class E = Fp16>
__device__ __forceinline__ void softmax_pv_tile(f32x4 sacc, int t0, int limit, float scale_log2,
                                                const unsigned char* stage, float& m_run,
                                                float& l_run, f32x4 (&o)[TileCfg<D>::NX]) {
  using C = TileCfg<D>;
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  float sv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tok = t0 + 4 * g + i;
    sv[i] = tok < limit ? sacc[i] * scale_log2 : kNegInf;
  }
  float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mx = fmaxf(mx, shfl_xor_f(mx, 16));
  mx = fmaxf(mx, shfl_xor_f(mx, 32));
  if (__ballot(mx > m_run + kRescaleSlack)) {  // wave-uniform
    const float m_new = fmaxf(m_run, mx);
    const float alpha = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] *= alpha;
    m_run = m_new;
  }
  const float m_use = m_run == kNegInf ? 0.f : m_run;
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = exp2_fast(sv[i] - m_use);
  l_run += (p[0] + p[1]) + (p[2] + p[3]);
  const f16x4 pb = to16x4<E>(p[0], p[1], p[2], p[3]);
  const unsigned char* vb = stage + (4 * g + (n >> 2)) * C::ROWB + (n & 3) * 8;
#pragma unroll
  for (int x = 0; x < C::NX; ++x) {
    const s16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(vb + 32 * x));
    o[x] = mma16<E>(__builtin_bit_cast(f16x4, raw), pb, o[x]);
  }
}

template <int D, class E = Fp16>
struct TileCore {
  using C = TileCfg<D>;

  // sequence / pool geometry
  f16* k_pool;
  f16* v_pool;
  const int32_t* trow;  // block-table row of the sequence
  int64_t rs;           // elements per pool row (kv_heads * D)
  int hoff;             // kv_head * D
  int W, NB, BS, bs_log2;
  int tok_end;          // keys >= tok_end are never read
  int limit;            // this lane's column accepts keys < limit
  float scale_log2;
  // optional fused page write of the decode token (position new_pos)
  const f16* knew_row;
  const f16* vnew_row;
  int new_pos;          // -1: none

  unsigned char* stage; // per-wave LDS tile, C::STAGE bytes

  f16x8 qv[C::NK];
  float m_run;
  float l_run;
  f32x4 o[C::NX];

  __device__ __forceinline__ int64_t pool_row(int tok) const {
    int page = tok >> bs_log2;
    page = page < W ? page : W - 1;
    const int blk = clamp_block(trow[page], NB);
    return (int64_t)blk * BS + (tok & (BS - 1));
  }

  __device__ __forceinline__ void init_acc() {
    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  __device__ __forceinline__ void load_tile(int t, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) const {
    const int lane = lane_id();
    const int g = lane >> 4;
    const int n = lane & 15;
    const int t0 = t * kTile;
    {
      const int tk = t0 + n;
      const int tkc = tk < tok_end ? tk : tok_end - 1;
      f16* kp = k_pool + pool_row(tkc) * rs + hoff;
      if (tk == new_pos) {
#pragma unroll
        for (int s = 0; s < C::NK; ++s) {
          kk[s] = ld16(knew_row + (4 * s + g) * 8);
          st16(kp + (4 * s + g) * 8, kk[s]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < C::NK; ++s) kk[s] = ld16(kp + (4 * s + g) * 8);
      }
    }
    const int cv = lane % C::CPR;
#pragma unroll
    for (int j = 0; j < C::NK; ++j) {
      const int tv = t0 + j * C::RPI + lane / C::CPR;
      const bool ok = tv < tok_end;
      const int tvc = ok ? tv : tok_end - 1;
      f16* vp = v_pool + pool_row(tvc) * rs + hoff + cv * 8;
      f16x8 val;
      if (tv == new_pos) {
        val = ld16(vnew_row + cv * 8);
        st16(vp, val);
      } else {
        val = ld16(vp);
      }
      vv[j] = ok ? val : f16x8{};
    }
  }

  __device__ __forceinline__ void compute_tile(int t, const f16x8 (&kk)[C::NK],
                                               const f16x8 (&vv)[C::NK]) {
    const int lane = lane_id();
    const int t0 = t * kTile;
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      sacc = mma16<E>(lo4(kk[s]), lo4(qv[s]), sacc);
      sacc = mma16<E>(hi4(kk[s]), hi4(qv[s]), sacc);
    }
    // stage the V rows of this tile (row-major, padded pitch)
    compiler_fence();
    {
      const int cv = lane % C::CPR;
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        const int r = j * C::RPI + lane / C::CPR;
        unsigned char* dst = stage + r * C::ROWB + cv * 16;
        *reinterpret_cast<f16x8*>(dst) = vv[j];  // ROWB is a multiple of 16
      }
    }
    compiler_fence();
    softmax_pv_tile<D, E>(sacc, t0, limit, scale_log2, stage, m_run, l_run, o);
    compiler_fence();
  }

  // Tiles t_first, t_first + step, ... < t_end with one tile of prefetch.
  __device__ __forceinline__ void run(int t_first, int step, int t_end) {
    f16x8 ka[C::NK], va[C::NK], kb[C::NK], vb[C::NK];
    int t = t_first;
    if (t < t_end) load_tile(t, ka, va);
    while (t < t_end) {
      if (t + step < t_end) load_tile(t + step, kb, vb);
      compute_tile(t, ka, va);
      t += step;
      if (t >= t_end) break;
      if (t + step < t_end) load_tile(t + step, ka, va);
      compute_tile(t, kb, vb);
      t += step;
    }
  }

  // Softmax denominator of column n summed over the four lanes g.
  __device__ __forceinline__ float l_total() const {
    float l = l_run + shfl_xor_f(l_run, 16);
    return l + shfl_xor_f(l, 32);
  }
};

// fp32 tile engine (pools, q and output in fp32), in the 16-bit engines'
// register layout, so the decode kernel around it -- the cross-wave combine,
// the split-K partials and their merge -- is the same:
//   S^T = K . Q^T on v_mfma_f32_16x16x4_f32: lane (g,n) loads dims 16c+4g .. +3
//     of key n and of column n's query (one 16-byte load per chunk c); MFMA
//     (c, j) contracts dim 16c + 4g + j in k-slot g.  -> lane (g,n) holds the
//     scores of column n for keys 4g..4g+3.
//   O^T += V^T . P^T, MFMA r taking keys 4g + r in k-slot g: A = V[key 4g+r]
//     [dim 16x+n] (a dword per (r, x); the 16 lanes of a group read a 64-byte
//     run of one row), B = the lane's probability of key 4g + r.  -> lane (g,n)
//     accumulates O[col n][16x + 4g + i].
// Probabilities stay fp32; the online softmax is the 16-bit engines' (base 2,
// the same rescale slack).  Any block size: a table lookup per key row, or
// (LIST, block sizes that are multiples of 16) the wave's tile rows held one
// per lane.  Column n accepts keys < limit (decode: tok_end; prefill: its
// position + 1).
//
// PAD: the real head_dim dr is below D (a multiple of 4): rows are dr floats
// apart within a pool row, the dims past dr are zeros in K and V (not loaded,
// and not written by the page write), and q is zero there too.
template <int D, bool LIST = false, bool PAD = false>
struct F32Core {
  static constexpr int NC = D / 16;  // 16-byte K and q chunks per lane
  static constexpr int NX = D / 16;  // output tiles of 16 dims

  const float* k_pool;
  const float* v_pool;
  const int32_t* trow;  // block-table row of the sequence
  int64_t rs;           // elements per pool row (kv_heads * head_dim)
  int hoff;             // kv_head * head_dim
  int dr;               // PAD: the real head_dim
  int W, NB, BS, bs_log2;
  int tok_end;          // keys >= tok_end are never read
  int limit;            // this lane's column accepts keys < limit
  float scale_log2;
  // optional fused page write of the decode token (position new_pos)
  const float* knew_row;
  const float* vnew_row;
  float* k_pool_w;
  float* v_pool_w;
  int new_pos;          // -1: none
  // the wave's tiles: t_first, t_first + step, ... (LIST: block sizes that are
  // multiples of 16, so a tile's 16 keys are consecutive rows of one block;
  // lane j of row_vec holds the pool row of the first key of tile list_base + j,
  // refilled every 64 tiles, so no table load sits between two tiles' loads)
  int t_first, step;
  int row_vec, list_base;

  f32x4 qv[NC];
  float m_run;
  float l_run;
  f32x4 o[NX];

  __device__ __forceinline__ int64_t pool_row(int tok) const {
    int page = tok >> bs_log2;
    page = page < W ? page : W - 1;
    const int blk = clamp_block(trow[page], NB);
    return (int64_t)blk * BS + (tok & (BS - 1));
  }
  // LIST: the pool rows of tiles k0 .. k0 + 63 of the wave's list
  __device__ __forceinline__ void fill_list(int k0) {
    list_base = k0;
    row_vec = (int)pool_row((t_first + (k0 + lane_id()) * step) * kTile);
  }
  // Pool row of key t0 + r of the wave's k-th tile (key clamped below tok_end).
  __device__ __forceinline__ int64_t key_row(int k, int t0, int r) const {
    const int tok = t0 + r < tok_end ? t0 + r : tok_end - 1;
    if constexpr (LIST)
      return (int64_t)__builtin_amdgcn_readlane(row_vec, k - list_base) + (tok - t0);
    else
      return pool_row(tok);
  }

  __device__ __forceinline__ void init_acc() {
    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int x = 0; x < NX; ++x) o[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  __device__ __forceinline__ void load_tile(int k, f32x4 (&kk)[NC], float (&vv)[4][NX]) {
    const int lane = lane_id();
    const int g = lane >> 4;
    const int n = lane & 15;
    if constexpr (LIST) {
      if (k - list_base >= kWave) fill_list(k);  // wave-uniform
    }
    const int t0 = (t_first + k * step) * kTile;
    {
      const int tk = t0 + n;
      const int64_t off = key_row(k, t0, n) * rs + hoff + 4 * g;
      if (tk == new_pos) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          kk[c] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (!PAD || 16 * c + 4 * g < dr) {
            kk[c] = *reinterpret_cast<const f32x4*>(knew_row + 16 * c + 4 * g);
            *reinterpret_cast<f32x4*>(k_pool_w + off + 16 * c) = kk[c];
          }
        }
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          kk[c] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (!PAD || 16 * c + 4 * g < dr)
            kk[c] = *reinterpret_cast<const f32x4*>(k_pool + off + 16 * c);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tv = t0 + 4 * g + r;
      const bool ok = tv < tok_end;
      const int64_t off = key_row(k, t0, 4 * g + r) * rs + hoff + n;
      if (tv == new_pos) {
#pragma unroll
        for (int x = 0; x < NX; ++x) {
          vv[r][x] = 0.f;
          if (!PAD || 16 * x + n < dr) {
            vv[r][x] = vnew_row[16 * x + n];
            v_pool_w[off + 16 * x] = vv[r][x];
          }
        }
      } else {
#pragma unroll
        for (int x = 0; x < NX; ++x) {
          float val = 0.f;
          if (!PAD || 16 * x + n < dr) val = v_pool[off + 16 * x];
          vv[r][x] = ok ? val : 0.f;
        }
      }
    }
  }

  __device__ __forceinline__ void compute_tile(int k, const f32x4 (&kk)[NC],
                                               const float (&vv)[4][NX]) {
    const int lane = lane_id();
    const int g = lane >> 4;
    const int t0 = (t_first + k * step) * kTile;
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) sacc = mfma4_f32(kk[c][j], qv[c][j], sacc);
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = t0 + 4 * g + i;
      sv[i] = tok < limit ? sacc[i] * scale_log2 : kNegInf;
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, shfl_xor_f(mx, 16));
    mx = fmaxf(mx, shfl_xor_f(mx, 32));
    if (__ballot(mx > m_run + kRescaleSlack)) {  // wave-uniform
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int x = 0; x < NX; ++x) o[x] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == kNegInf ? 0.f : m_run;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = exp2_fast(sv[i] - m_use);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[x] = mfma4_f32(vv[r][x], p[r], o[x]);
  }

  // The wave's tiles t_first, t_first + step, ... below t_end, one tile of
  // prefetch: while tile k is computed, the loads of tile k + 1 are in flight.
  __device__ __forceinline__ void run(int first, int stride, int t_end) {
    t_first = first;
    step = stride;
    const int ntiles = first < t_end ? (t_end - first + stride - 1) / stride : 0;
    if (ntiles == 0) return;
    if constexpr (LIST) fill_list(0);
    f32x4 ka[NC], kb[NC];
    float va[4][NX], vb[4][NX];
    load_tile(0, ka, va);
    for (int k = 0;; k += 2) {
      if (k + 1 < ntiles) load_tile(k + 1, kb, vb);
      compute_tile(k, ka, va);
      if (k + 1 >= ntiles) break;
      if (k + 2 < ntiles) load_tile(k + 2, ka, va);
      compute_tile(k + 1, kb, vb);
      if (k + 2 >= ntiles) break;
    }
  }

  __device__ __forceinline__ float l_total() const {
    float l = l_run + shfl_xor_f(l_run, 16);
    return l + shfl_xor_f(l, 32);
  }
};

// Fast path for block sizes that are multiples of 16: the 16 keys of a tile
// share one physical block, so a tile is fully described by wave-uniform
// values -- the pool row of its first key and its key count.  A wave's tiles
// form a list held one per lane (lane k: tile k, k < 64), filled from the block
// tables before the first load, so no table access sits between two tiles'
// K/V loads.
//
// PAD: the real head_dim is below D (D = the next of 64 / 128 / 256 computed):
// rows are nch 16-byte chunks long in the pool, the chunks past them are zeros
// in the K and V registers (q is zero there too) and never written.
template <int D, class E = Fp16, bool PAD = false>
struct TileListCore {
  using C = TileCfg<D>;

  const f16* k_pool;
  const f16* v_pool;
  int rs;                 // elements per pool row (kv_heads * head_dim)
  int hoff;               // kv_head * head_dim
  int nch;                // PAD: 16-byte chunks of a real row
  float scale_log2;
  unsigned char* stage;   // per-wave LDS tile, C::STAGE bytes
  int ntiles;             // tiles in the list (<= 64)
  int row_vec;            // lane k < ntiles: pool row (block * BS + offset) of tile k's first key
  int rows_vec;           // lane k < ntiles: keys in tile k (1..16)

  // The decoded token's K/V row (row new_row of tile new_tile; -1: not in this
  // list) comes from these registers instead of the pool, so no load waits on
  // the page write; the caller writes the row to the pool (store_new_row).
  int new_tile;
  int new_row;
  f16x8 knew[C::NK];      // lane (g, n): chunks 4s+g of the new K row
  f16x8 vnew;             // lane l: chunk l % CPR of the new V row

  f16x8 qv[C::NK];
  float m_run;
  float l_run;
  f32x4 o[C::NX];

  __device__ __forceinline__ void init_acc() {
    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Element offset of row 0 of tile k (kv head included); wave-uniform.
  __device__ __forceinline__ int64_t tile_base(int k) const {
    return (int64_t)__builtin_amdgcn_readlane(row_vec, k & (kWave - 1)) * rs + hoff;
  }
  // Keys of tile k; 0 past the end of the list.
  __device__ __forceinline__ int tile_rows(int k) const {
    const int r = __builtin_amdgcn_readlane(rows_vec, k & (kWave - 1));
    return k < ntiles ? r : 0;
  }

  // Tile loads are raw buffer loads: a scalar descriptor per tile (base = row
  // 0 of the tile for this KV head, extent = the tile's keys) and a
  // loop-invariant 32-bit byte offset per lane.  Rows past the extent read as
  // zeros, so stale pool contents beyond a context never reach the
  // accumulators, and a tile past the list loads nothing.
  __device__ __forceinline__ uint32_t k_off0() const {
    const int lane = lane_id();
    return (uint32_t)(((lane & 15) * rs + (lane >> 4) * 8) * 2);
  }
  __device__ __forceinline__ static uint32_t k_soff(int s) { return (uint32_t)(s * 64); }
  __device__ __forceinline__ uint32_t v_off0() const {
    const int lane = lane_id();
    return (uint32_t)(((lane / C::CPR) * rs + (lane % C::CPR) * 8) * 2);
  }
  __device__ __forceinline__ uint32_t v_soff(int j) const { return (uint32_t)(j * C::RPI * rs * 2); }
  __device__ __forceinline__ static f16x8 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff) {
    return __builtin_bit_cast(f16x8,
                              __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kPagePolicy));
  }
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const f16* pool, int64_t base,
                                                             int rows) const {
    // Every field goes through readfirstlane: the values are wave-uniform, and
    // a descriptor held in vector registers would make the backend wrap each
    // load in a waterfall loop.
    const uint64_t addr = reinterpret_cast<uint64_t>(pool + base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
    // PAD: the extent ends at the real end of the last key's row, so the
    // chunks past it in that row read as zeros rather than past the pool
    const int nrec = __builtin_amdgcn_readfirstlane(
        PAD ? (rows > 0 ? ((rows - 1) * rs + nch * 8) * 2 : 0) : rows * rs * 2);
    void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    // dword 3 = 0x00020000: 32-bit data format, the gfx9 setting for raw dword access
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, nrec, 0x00020000);
  }

  // Issues the K/V loads of tile k; nothing here waits for data.
  __device__ __forceinline__ void load_tile(int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) const {
    const int64_t base = tile_base(k);
    const int rows = tile_rows(k);
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(k_pool, base, rows);
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(v_pool, base, rows);
    const uint32_t ko = k_off0();
    const uint32_t vo = v_off0();
    if constexpr (PAD) {
      // only the real chunks of a row are loaded: the rest stay zeros
      const int lane = lane_id();
#pragma unroll
      for (int s = 0; s < C::NK; ++s) {
        kk[s] = f16x8{};
        if (4 * s + (lane >> 4) < nch) kk[s] = buf_ld16(kr, ko, k_soff(s));
      }
      const bool vin = lane % C::CPR < nch;
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        vv[j] = f16x8{};
        if (vin) vv[j] = buf_ld16(vr, vo, v_soff(j));
      }
    } else {
#pragma unroll
      for (int s = 0; s < C::NK; ++s) kk[s] = buf_ld16(kr, ko, k_soff(s));
#pragma unroll
      for (int j = 0; j < C::NK; ++j) vv[j] = buf_ld16(vr, vo, v_soff(j));
    }
  }

  // One tile held in kk / vv: scores, V staging, softmax and PV.
  __device__ __forceinline__ void compute_tile(int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) {
    const int lane = lane_id();
    const int vrow = lane / C::CPR;
    if (k == new_tile) {  // wave-uniform: substitute the decoded token's row
      const bool krow = (lane & 15) == new_row;
#pragma unroll
      for (int s = 0; s < C::NK; ++s) kk[s] = krow ? knew[s] : kk[s];
#pragma unroll
      for (int j = 0; j < C::NK; ++j) vv[j] = j * C::RPI + vrow == new_row ? vnew : vv[j];
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
        const int r = j * C::RPI + vrow;
        unsigned char* dst = stage + r * C::ROWB + cv * 16;
        *reinterpret_cast<f16x8*>(dst) = vv[j];  // ROWB is a multiple of 16
      }
    }
    compiler_fence();
    softmax_pv_tile<D, E>(sacc, 0, tile_rows(k), scale_log2, stage, m_run, l_run, o);
    compiler_fence();
  }

  // Two register stages: while tile k is computed, the loads of tile k+1 are
  // in flight.  Loads are issued unconditionally (zero extent past the end of
  // the list), so the loop has no join points and every wait is exact.
  __device__ __forceinline__ void run() {
    f16x8 ka[C::NK], va[C::NK], kb[C::NK], vb[C::NK];
    load_tile(0, ka, va);
    for (int k = 0;; k += 2) {
      load_tile(k + 1, kb, vb);
      if (k >= ntiles) break;
      compute_tile(k, ka, va);
      load_tile(k + 2, ka, va);
      if (k + 1 >= ntiles) break;
      compute_tile(k + 1, kb, vb);
    }
  }

  // Writes the decoded token's K/V row to the pool (the wave holding its tile).
  __device__ __forceinline__ void store_new_row(f16* k_pool_w, f16* v_pool_w) const {
    if (new_tile < 0) return;
    const int lane = lane_id();
    const int64_t base = tile_base(new_tile);
    char* kb = reinterpret_cast<char*>(k_pool_w + base);
    char* vb = reinterpret_cast<char*>(v_pool_w + base);
    if ((lane & 15) == new_row) {
#pragma unroll
      for (int s = 0; s < C::NK; ++s)
        if (!PAD || 4 * s + (lane >> 4) < nch)
          *reinterpret_cast<f16x8*>(kb + k_off0() + k_soff(s)) = knew[s];
    }
    const int vrow = lane / C::CPR;
#pragma unroll
    for (int j = 0; j < C::NK; ++j)
      if (j * C::RPI + vrow == new_row && (!PAD || lane % C::CPR < nch))
        *reinterpret_cast<f16x8*>(vb + v_off0() + v_soff(j)) = vnew;
  }

  __device__ __forceinline__ float l_total() const {
    float l = l_run + shfl_xor_f(l_run, 16);
    return l + shfl_xor_f(l, 32);
  }
};

}  // namespace fe
