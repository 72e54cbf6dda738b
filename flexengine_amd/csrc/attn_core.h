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
  // LDS pitch of a staged V row: D halves + 8 bytes = D/2 + 2 dwords, which is
  // 2 mod 32 for D = 64 and 128.  Row r then starts at bank 2r mod 32, so the
  // four rows 4g+i (g = 0..3) that one column read touches start at banks
  // 8g + 2i and their 8-dword spans are disjoint: no bank conflicts.
  static constexpr int ROWB = D * 2 + 8;
  static constexpr int STAGE = kTile * ROWB;
};

__device__ __forceinline__ int clamp_block(int blk, int nb) {
  return blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
}

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Shared softmax + PV step of one 16-key tile (scores already in sacc).
// Lane (g,n): sacc[i] = raw score of key t0 + 4g + i for column n; keys at or
// past `limit` are masked.  V rows of the tile are in `stage` (row pitch ROWB).
template <int D>
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
  const float m_new = fmaxf(m_run, mx);
  const float m_use = m_new == kNegInf ? 0.f : m_new;
  const float alpha = exp2f(m_run - m_use);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = exp2f(sv[i] - m_use);
  l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  m_run = m_new;
  const f16x4 pb = {(f16)p[0], (f16)p[1], (f16)p[2], (f16)p[3]};
#pragma unroll
  for (int x = 0; x < C::NX; ++x) {
    o[x] *= alpha;
    f16x4 va;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      va[i] = *reinterpret_cast<const f16*>(stage + (4 * g + i) * C::ROWB + (16 * x + n) * 2);
    o[x] = mfma16(va, pb, o[x]);
  }
}

template <int D>
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
      sacc = mfma16(lo4(kk[s]), lo4(qv[s]), sacc);
      sacc = mfma16(hi4(kk[s]), hi4(qv[s]), sacc);
    }
    // stage the V rows of this tile (row-major, padded pitch)
    compiler_fence();
    {
      const int cv = lane % C::CPR;
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        const int r = j * C::RPI + lane / C::CPR;
        unsigned char* dst = stage + r * C::ROWB + cv * 16;
        const uint4 bits = *reinterpret_cast<const uint4*>(&vv[j]);
        *reinterpret_cast<uint2*>(dst) = uint2{bits.x, bits.y};
        *reinterpret_cast<uint2*>(dst + 8) = uint2{bits.z, bits.w};
      }
    }
    compiler_fence();
    softmax_pv_tile<D>(sacc, t0, limit, scale_log2, stage, m_run, l_run, o);
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

// Fast path for block sizes that are multiples of 16: the 16 keys of a tile
// share one physical block, so the block id and the row base are wave-uniform
// (scalar registers) and each lane only carries a 32-bit offset.  The block
// ids of all of a wave's tiles are fetched with one vector load before the
// first tile, so no table access sits between two tiles' K/V loads.
template <int D>
struct Page16Core {
  using C = TileCfg<D>;

  const f16* k_pool;
  const f16* v_pool;
  f16* k_pool_w;          // writable aliases for the fused page write
  f16* v_pool_w;
  const int32_t* trow;
  int rs;                 // elements per pool row (kv_heads * D)
  int hoff;               // kv_head * D
  int W, NB, BS, bs_log2;
  int tok_end;
  int limit;
  float scale_log2;
  const f16* knew_row;
  const f16* vnew_row;
  int new_pos;
  unsigned char* stage;

  f16x8 qv[C::NK];
  float m_run;
  float l_run;
  f32x4 o[C::NX];

  int t_first;            // first tile of this wave
  int step;               // tile stride (waves per workgroup)
  int blk_vec;            // lane k: physical block of tile t_first + k*step (k < 64)

  __device__ __forceinline__ void init_acc() {
    m_run = kNegInf;
    l_run = 0.f;
#pragma unroll
    for (int x = 0; x < C::NX; ++x) o[x] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Lane k (< ntiles <= 64) fetches the physical block of tile k; other lanes 0.
  __device__ __forceinline__ void fetch_blocks(int ntiles) {
    const int k = lane_id();
    int blk = 0;
    if (k < ntiles) {
      int page = ((t_first + k * step) * kTile) >> bs_log2;
      page = page < W ? page : W - 1;
      blk = clamp_block(trow[page], NB);
    }
    blk_vec = blk;
  }

  // Row base (element offset of row 0 of the tile, kv head included), uniform.
  __device__ __forceinline__ int64_t tile_base(int k) const {
    const int t0 = (t_first + k * step) * kTile;
    const int blk = __builtin_amdgcn_readlane(blk_vec, k & (kWave - 1));
    return ((int64_t)blk * BS + (t0 & (BS - 1))) * rs + hoff;
  }

  __device__ __forceinline__ int tile_t0(int k) const { return (t_first + k * step) * kTile; }

  // Tile loads are raw buffer loads: a scalar descriptor per tile (base = row
  // 0 of the tile for this KV head, extent = rows still inside the piece) and
  // a loop-invariant 32-bit byte offset per lane.  Rows past the piece fall
  // outside the descriptor's range and read as zeros, so stale pool contents
  // beyond the context never reach the accumulators.
  __device__ __forceinline__ uint32_t k_off0() const {
    const int lane = lane_id();
    return (uint32_t)(((lane & 15) * rs + (lane >> 4) * 8) * 2);
  }
  __device__ __forceinline__ static uint32_t k_soff(int s) { return (uint32_t)(s * 64); }
  __device__ __forceinline__ uint32_t k_off(int s) const { return k_off0() + k_soff(s); }
  __device__ __forceinline__ uint32_t v_off0() const {
    const int lane = lane_id();
    return (uint32_t)(((lane / C::CPR) * rs + (lane % C::CPR) * 8) * 2);
  }
  __device__ __forceinline__ uint32_t v_soff(int j) const { return (uint32_t)(j * C::RPI * rs * 2); }
  __device__ __forceinline__ static f16x8 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff) {
    return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  }
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const f16* pool, int64_t base,
                                                             int rows) const {
    // Every field goes through readfirstlane: the values are wave-uniform, and
    // a descriptor held in vector registers would make the backend wrap each
    // load in a waterfall loop.
    const uint64_t addr = reinterpret_cast<uint64_t>(pool + base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)addr);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
    const int nrec = __builtin_amdgcn_readfirstlane(rows * rs * 2);
    void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    // dword 3 = 0x00020000: 32-bit data format, the gfx9 setting for raw dword access
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, nrec, 0x00020000);
  }

  // Issues the K/V loads of tile k; nothing here waits for data.
  __device__ __forceinline__ void load_tile(int k, f16x8 (&kk)[C::NK], f16x8 (&vv)[C::NK]) const {
    const int64_t base = tile_base(k);
    const int rem = tok_end - tile_t0(k);
    const int rows = rem < 0 ? 0 : (rem < kTile ? rem : kTile);
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc(k_pool, base, rows);
    const __amdgpu_buffer_rsrc_t vr = tile_rsrc(v_pool, base, rows);
    const uint32_t ko = k_off0();
#pragma unroll
    for (int s = 0; s < C::NK; ++s) kk[s] = buf_ld16(kr, ko, k_soff(s));
    const uint32_t vo = v_off0();
#pragma unroll
    for (int j = 0; j < C::NK; ++j) vv[j] = buf_ld16(vr, vo, v_soff(j));
  }

  // Fused page write of the decoded token (position new_pos, inside this
  // wave's tile k): each lane that will load a 16-byte chunk of that row first
  // stores the new chunk to the same address, so its later load (same thread,
  // same address, program order) returns the new bytes.  Issued right after the
  // block-id fetch, whose latency the k_new / v_new loads overlap.
  __device__ __forceinline__ void write_new_row(int k) const {
    const int lane = lane_id();
    const int g = lane >> 4;
    const int n = lane & 15;
    const int r = new_pos - tile_t0(k);
    const int64_t base = tile_base(k);
    char* kb = reinterpret_cast<char*>(k_pool_w + base);
    char* vb = reinterpret_cast<char*>(v_pool_w + base);
    if (n == r) {
#pragma unroll
      for (int s = 0; s < C::NK; ++s)
        *reinterpret_cast<f16x8*>(kb + k_off(s)) = ld16(knew_row + (4 * s + g) * 8);
    }
    const int vrow = lane / C::CPR;
#pragma unroll
    for (int j = 0; j < C::NK; ++j)
      if (j * C::RPI + vrow == r)
        *reinterpret_cast<f16x8*>(vb + v_off0() + v_soff(j)) = ld16(vnew_row + (lane % C::CPR) * 8);
    // The same lanes load these addresses later: a wave's memory operations to
    // one address are performed in order, so only the compiler needs holding
    // back (it may not move the buffer loads above these stores).
    compiler_fence();
  }

  __device__ __forceinline__ void compute_tile(int k, const f16x8 (&kk)[C::NK],
                                               f16x8 (&vv)[C::NK]) {
    const int lane = lane_id();
    const int t0 = tile_t0(k);
    const int vrow = lane / C::CPR;
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < C::NK; ++s) {
      sacc = mfma16(lo4(kk[s]), lo4(qv[s]), sacc);
      sacc = mfma16(hi4(kk[s]), hi4(qv[s]), sacc);
    }
    compiler_fence();
    {
      const int cv = lane % C::CPR;
#pragma unroll
      for (int j = 0; j < C::NK; ++j) {
        const int r = j * C::RPI + vrow;
        unsigned char* dst = stage + r * C::ROWB + cv * 16;
        const uint4 bits = *reinterpret_cast<const uint4*>(&vv[j]);
        *reinterpret_cast<uint2*>(dst) = uint2{bits.x, bits.y};
        *reinterpret_cast<uint2*>(dst + 8) = uint2{bits.z, bits.w};
      }
    }
    compiler_fence();
    softmax_pv_tile<D>(sacc, t0, limit, scale_log2, stage, m_run, l_run, o);
    compiler_fence();
  }

  // All tiles t_first + k*step < t_end (at most 64 per wave: the host bounds
  // the piece size).  NSTAGE register stages: while tile k is computed, the
  // loads of tiles k+1 .. k+NSTAGE-1 are in flight.  Loads are issued
  // unconditionally (tiles past the end have a zero-extent descriptor and touch
  // no memory), so the loop has no join points and every wait is exact.
  template <int NSTAGE>
  __device__ __forceinline__ void run(int t_end) {
    static_assert(NSTAGE >= 2, "need at least two register stages");
    const int ntiles = t_first < t_end ? (t_end - t_first + step - 1) / step : 0;
    if (ntiles == 0) return;
    fetch_blocks(ntiles);
    if (new_pos >= 0) {
      // tile index (within this wave) holding the decoded token, if any
      const int tn = new_pos / kTile - t_first;
      if (tn >= 0 && tn % step == 0 && tn / step < ntiles) write_new_row(tn / step);
    }
    f16x8 kbuf[NSTAGE][C::NK], vbuf[NSTAGE][C::NK];
#pragma unroll
    for (int u = 0; u < NSTAGE - 1; ++u) load_tile(u, kbuf[u], vbuf[u]);
    int k = 0;
    while (true) {
#pragma unroll
      for (int u = 0; u < NSTAGE; ++u) {
        load_tile(k + NSTAGE - 1, kbuf[(u + NSTAGE - 1) % NSTAGE], vbuf[(u + NSTAGE - 1) % NSTAGE]);
        compute_tile(k, kbuf[u], vbuf[u]);
        if (++k >= ntiles) return;
      }
    }
  }

  __device__ __forceinline__ float l_total() const {
    float l = l_run + shfl_xor_f(l_run, 16);
    return l + shfl_xor_f(l, 32);
  }
};

}  // namespace fe
