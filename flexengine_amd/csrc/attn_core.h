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
    const int g = lane >> 4;
    const int n = lane & 15;
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
    // a column with no valid key so far keeps m = -inf; use 0 as the shift so
    // that alpha and p evaluate to 0 instead of NaN
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

}  // namespace fe
