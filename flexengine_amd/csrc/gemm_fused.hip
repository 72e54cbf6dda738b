// Decode-step GEMMs of the Qwen2 layer with their element-wise neighbours fused
// (gfx950).  At decode batch sizes every kernel boundary of the layer costs a
// few microseconds on its own (the launch, the ramp of the grid, the drain),
// more than the element-wise work between the projections, so these kernels
// take that work into the GEMM that consumes or produces it:
//
//   prologue  RMSNorm of the operand: x is the un-normalised residual stream
//             r [M][K] (fp16) plus the per-tile sums of r^2 that the producing
//             GEMM wrote, and the operand is fp16(w * fp16(r * rsqrt(mean + eps)))
//             -- each workgroup normalises only the K range it multiplies.
//   epilogue  F16    out = fp16(x W^T + bias)
//             RESID  r = fp16(fp16(x W^T) + residual), and sum(r^2) over the
//                    tile's 16 columns (the next GEMM's prologue input)
//             SILU   act = fp16(fp16(silu(gate)) * up) for W = [gate; up]
//             ROPE   q, k, v of W = [q; k; v] with bias and rotate-half RoPE
//
// Work: one workgroup per 16-row tile of the output; its waves cut K into
// contiguous slices and add their products through LDS.  When the tiles alone
// leave the chip short of ~192 workgroups (q/k/v 128 tiles, o and down 96), ks_for()
// gives each tile several workgroups over disjoint K ranges: each writes its
// fp32 partial tile with device-coherent stores and takes a per-tile ticket,
// and the last one adds the partials in split order and runs the epilogue, so
// the element-wise epilogue still sees the whole sum.  The 16 weight
// rows of a tile are the A operand of v_mfma_f32_16x16x16_f16 loaded straight
// from HBM (lane (g, n): row n, 16 bytes at k0 + 32j + 8g), x the B operand.
// For SILU a tile holds 8 gate rows and the 8 up rows of the same columns, for
// ROPE 8 rows of the first half of a head and the 8 rows D/2 further, so the
// pairs the epilogue combines sit in one workgroup (the weights keep their
// PyTorch Linear layout; only the row map differs).
//
// Rounding follows the PyTorch fp16 semantics of the unfused chains (each
// element-wise op computes in fp32 and rounds to fp16), as the element-wise
// kernels of model_ops.hip do; no multiply-add contraction in this file.
// Replaces, per layer, the rmsnorm/rope/silu launches between the projections
// of the reference's decode step (src/flexengine/inference/models/qwen2.py:
// 139-186 with the HF Qwen2RMSNorm / Qwen2MLP it calls).
#include "fe_common.h"

using namespace fe;

#pragma clang fp contract(off)

namespace {

constexpr int kStepK = 128;  // keys per pipeline step (4 MFMA k-groups of 32)
constexpr int kMaxSsPerLane = 64;  // RMSNorm prologue: up to 256 tile sums per row
#ifndef FE_WEIGHT_POLICY
#define FE_WEIGHT_POLICY 0
#endif

enum Epi { kEpiF16 = 0, kEpiResid = 1, kEpiSilu = 2, kEpiRope = 3, kEpiResidNorm = 4 };

struct FusedArgs {
  const f16* W;        // [N][K]
  int N, K, M;
  int kslice;          // keys per wave (a multiple of 32)
  const f16* x;        // [M][K]: the operand, or the residual r when x_ss is set
  const float* x_ss;   // [ss_tiles][M] sums of r^2, or null (plain operand)
  int ss_tiles;
  const f16* norm_w;   // [K]
  float eps;
  const f16* bias;     // [N] or null
  f16* out;            // F16, RESID: [M][N]; SILU: [M][N/2]; ROPE: q [M][hq][d]
  const f16* residual; // RESID: [M][N]
  float* out_ss;       // RESID: [N/16][M]
  f16* k_out;          // ROPE: [M][hkv][d]
  f16* v_out;
  const int64_t* positions;  // ROPE: [M]
  const float* inv_freq;     // ROPE: [d/2]
  int hq, hkv, d;
  // split-K across workgroups: `ks_count` workgroups per tile, each over
  // `kslice_wg` keys; their partial tiles meet in the workspace
  int tiles, ks_count, kslice_wg;
  f32x4* part;    // [tiles][ks_count][MT][64] lane-layout partial tiles
  int* tickets;   // [tiles], zero between calls
  // RESID + RMSNorm (kEpiResidNorm): the tile that finishes last normalises
  // every row of r into tail_out
  const f16* tail_w;  // [N]
  float tail_eps;
  f16* tail_out;      // [M][N]
  int* grid_ticket;   // zero between calls
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int kSc1 = 16;  // buffer-instruction cache policy: sc1 (device-coherent)

__device__ __forceinline__ float round16(float x) { return (float)(f16)x; }

// Weight row held by tile-local row r (0..15) of tile `tile`; -1 past the end.
template <int EPI>
__device__ __forceinline__ int tile_row(const FusedArgs& a, int tile, int r) {
  if (EPI == kEpiSilu) {
    const int inter = a.N / 2;
    const int c = tile * 8 + (r & 7);
    return c < inter ? (r < 8 ? c : inter + c) : -1;
  }
  if (EPI == kEpiRope) {
    const int per_head = a.d / 16;
    const int hh = tile / per_head;
    const int j = tile - hh * per_head;
    return hh * a.d + (r < 8 ? 0 : a.d / 2) + 8 * j + (r & 7);
  }
  const int row = tile * 16 + r;
  return row < a.N ? row : -1;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

template <int MT, bool NORM>
struct Stage {
  f16x8 w[4];
  f16x8 x[MT][4];
  f16x8 nw[NORM ? 4 : 1];  // norm weight of the step's keys (RMSNorm prologue)
};

// RMSNorm of the finished residual stream r = out [M][N], run by the waves of
// the workgroup that completed the launch's last tile (wave w: rows
// kTailRows * w .. and every waves * kTailRows after): inv = rsqrt(sum of the
// row's tile sums of r^2 / N + eps), h = fp16(w * fp16(r * inv)), the rounding
// of fe_rmsnorm and transformers' Qwen2RMSNorm.  r and the tile sums were
// written by other workgroups with device-coherent stores before their
// tickets, so they are read device-coherently here.  N <= 64 * 8 * kTailChunks
// and N / 16 <= 64 * kTailSs (the host checks).
constexpr int kTailChunks = 4;  // 16-byte chunks of a row per lane
constexpr int kTailSs = 2;      // tile sums of a row per lane
constexpr int kTailRows = 2;    // rows of a wave whose loads are in flight together

__device__ __forceinline__ void norm_tail(const FusedArgs& a, int w, int waves, int lane) {
  const int N = a.N, M = a.M;
  const uint32_t r_bytes = (uint32_t)M * N * 2;
  const __amdgpu_buffer_rsrc_t rr = rsrc(a.out, r_bytes);
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.out_ss, (uint32_t)a.tiles * M * 4);
  f16x8 wv[kTailChunks];
#pragma unroll
  for (int c = 0; c < kTailChunks; ++c) {
    const int e0 = (c * kWave + lane) * 8;
    wv[c] = e0 < N ? ld16(a.tail_w + e0) : f16x8{};
  }
  for (int m0 = w * kTailRows; m0 < M; m0 += waves * kTailRows) {
    f16x8 rv[kTailRows][kTailChunks];
    float sp[kTailRows][kTailSs];
#pragma unroll
    for (int r = 0; r < kTailRows; ++r) {
      const int m = m0 + r;  // rows past M read as zeros (offsets past the range)
#pragma unroll
      for (int c = 0; c < kTailChunks; ++c) {
        const int e0 = (c * kWave + lane) * 8;
        const uint32_t off = m < M && e0 < N ? (uint32_t)(m * N + e0) * 2 : r_bytes;
        rv[r][c] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, kSc1));
      }
#pragma unroll
      for (int j = 0; j < kTailSs; ++j) {
        const int t = j * kWave + lane;
        const uint32_t off = m < M && t < a.tiles ? (uint32_t)(t * M + m) * 4 : (uint32_t)a.tiles * M * 4;
        sp[r][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kSc1));
      }
    }
#pragma unroll
    for (int r = 0; r < kTailRows; ++r) {
      const int m = m0 + r;
      float ssum = 0.f;
#pragma unroll
      for (int j = 0; j < kTailSs; ++j) ssum += sp[r][j];
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) ssum += __shfl_xor(ssum, sh, kWave);
      const float inv = rsqrtf(ssum / (float)N + a.tail_eps);
      if (m >= M) continue;
#pragma unroll
      for (int c = 0; c < kTailChunks; ++c) {
        const int e0 = (c * kWave + lane) * 8;
        if (e0 >= N) continue;
        f16x8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (f16)((float)wv[c][e] * round16((float)rv[r][c][e] * inv));
        st16(a.tail_out + (int64_t)m * N + e0, o);
      }
    }
  }
}

template <int MT, int WAVES, int EPI, bool NORM>
__global__ __launch_bounds__(WAVES * kWave) void gemm_fused_kernel(const FusedArgs a) {
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x % a.tiles;
  const int ks = blockIdx.x / a.tiles;
  const int wg_end = min(a.K, (ks + 1) * a.kslice_wg);
  const int k_begin = ks * a.kslice_wg + w * a.kslice;
  const int k_end = min(wg_end, k_begin + a.kslice);
  const int M = a.M;

  // weight rows through one descriptor over W; a row past the end reads zeros
  const uint32_t wbytes = (uint32_t)a.N * a.K * 2;
  const __amdgpu_buffer_rsrc_t rw = rsrc(a.W, wbytes);
  const int my_row = tile_row<EPI>(a, tile, n);
  const uint32_t w_off = my_row >= 0 ? (uint32_t)(my_row * a.K * 2 + g * 16) : wbytes;
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (uint32_t)M * a.K * 2);
  uint32_t x_off[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) x_off[mt] = (uint32_t)((mt * 16 + n) * a.K * 2 + g * 16);

  const __amdgpu_buffer_rsrc_t rn = rsrc(NORM ? a.norm_w : a.x, NORM ? (uint32_t)a.K * 2 : 0u);
  auto load = [&](Stage<MT, NORM>& s, int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      s.w[j] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                             rw, w_off, (uint32_t)(k0 + 32 * j) * 2, FE_WEIGHT_POLICY));
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s.x[mt][j] = __builtin_bit_cast(
            f16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, x_off[mt], (uint32_t)(k0 + 32 * j) * 2, 0));
    if constexpr (NORM) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s.nw[j] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                                rn, (uint32_t)g * 16, (uint32_t)(k0 + 32 * j) * 2, 0));
    }
  };

  // first weight step in flight before the prologue's loads
  Stage<MT, NORM> sa, sb;
  int k0 = k_begin;
  if (k0 < k_end) load(sa, k0);

  // RMSNorm prologue: 1/rms of every x row this lane multiplies (row mt*16 + n)
  float inv[MT];
  if constexpr (NORM) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + n;
      // all of this lane's tile sums in one batch of loads (ss_tiles <= 4 * 64)
      float part[kMaxSsPerLane];
#pragma unroll
      for (int i = 0; i < kMaxSsPerLane; ++i) {
        const int t = g + 4 * i;
        part[i] = m < M && t < a.ss_tiles ? a.x_ss[t * M + m] : 0.f;
      }
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < kMaxSsPerLane; ++i) s += part[i];
      s += shfl_xor_f(s, 16);
      s += shfl_xor_f(s, 32);
      inv[mt] = rsqrtf(s / (float)a.K + a.eps);
    }
  }
  // operand transform of one 8-key chunk of row mt*16 + n (nw: its norm weights)
  auto operand = [&](f16x8 v, int mt, f16x8 nw) __attribute__((always_inline)) {
    if constexpr (!NORM) {
      return v;
    } else {
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f16)((float)nw[e] * round16((float)v[e] * inv[mt]));
      return o;
    }
  };

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Stage<MT, NORM>& s, int nj) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nj) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f16x8 xv = operand(s.x[mt][j], mt, s.nw[NORM ? j : 0]);
          acc[mt] = mfma16(lo4(s.w[j]), lo4(xv), acc[mt]);
          acc[mt] = mfma16(hi4(s.w[j]), hi4(xv), acc[mt]);
        }
      }
    }
  };

  // two register stages: step t+1's loads are in flight while step t is computed
  while (k0 < k_end) {
    const int nja = min(4, (k_end - k0) / 32);
    load(sb, min(k0 + kStepK, k_end - 32));
    compute(sa, nja);
    k0 += kStepK;
    if (k0 >= k_end) break;
    const int njb = min(4, (k_end - k0) / 32);
    load(sa, min(k0 + kStepK, k_end - 32));
    compute(sb, njb);
    k0 += kStepK;
  }

  // KEEP: every wave stays to the end (the norm tail uses all of them); the
  // workgroup's decisions then go through LDS so that all waves take them
  constexpr bool KEEP = EPI == kEpiResidNorm;
  __shared__ int wg_flag[2];
  auto broadcast = [&](int v, int slot) __attribute__((always_inline)) {
    if (w == 0 && lane == 0) wg_flag[slot] = v;
    __syncthreads();
    return wg_flag[slot];
  };

  // the waves' K slices are added through LDS, in wave order
  if constexpr (WAVES > 1) {
    __shared__ f32x4 red[WAVES - 1][MT][kWave];
    if (w > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) red[w - 1][mt][lane] = acc[mt];
    }
    __syncthreads();
    if (!KEEP && w != 0) return;
    if (w == 0) {
#pragma unroll
      for (int v = 0; v < WAVES - 1; ++v)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] += red[v][mt][lane];
    }
  }

  // ---- split-K: the last workgroup of the tile to finish adds all partial
  // tiles, in split order (the same sum whichever workgroup is last) ----
  if (a.ks_count > 1) {
    const __amdgpu_buffer_rsrc_t rp = rsrc(a.part + (int64_t)tile * a.ks_count * MT * kWave,
                                           (uint32_t)a.ks_count * MT * kWave * 16);
    int last = 0;
    if (w == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt]), rp,
                                               (uint32_t)(((ks * MT + mt) * kWave + lane) * 16),
                                               0, kSc1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial complete device-wide
      if (lane == 0)
        last = __hip_atomic_fetch_add(a.tickets + tile, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == a.ks_count - 1;
      last = __builtin_amdgcn_readfirstlane(last);
    }
    if constexpr (KEEP) last = broadcast(last, 0);
    if (!last) return;
    if (w == 0) {
      if (lane == 0)
        __hip_atomic_store(a.tickets + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      // the partials are loaded MB splits at a time, all in flight together
      // (a load-add loop would wait out one round trip per split), and added
      // in split order
      constexpr int MB = 8 / MT;
      for (int s0 = 0; s0 < a.ks_count; s0 += MB) {
        f32x4 pv[MB][MT];
#pragma unroll
        for (int u = 0; u < MB; ++u)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            pv[u][mt] = s0 + u < a.ks_count
                            ? __builtin_bit_cast(
                                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rp, (uint32_t)((((s0 + u) * MT + mt) * kWave + lane) * 16),
                                             0, kSc1))
                            : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < MB; ++u)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            if (s0 + u < a.ks_count) acc[mt] += pv[u][mt];
      }
    }
  }

  // ---- epilogue (wave 0): lane (g, n) holds out[m = mt*16 + n][tile row 4g + i] ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (KEEP && w != 0) break;  // the other waves wait for the norm tail
    const int m = mt * 16 + n;
    if constexpr (EPI == kEpiF16 || EPI == kEpiResid || EPI == kEpiResidNorm) {
      constexpr bool RES = EPI != kEpiF16;
      const int row0 = tile * 16 + 4 * g;
      float r[4];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + i;
        const bool ok = m < M && row < a.N;
        float v = acc[mt][i];
        if (!RES) {
          if (a.bias && row < a.N) v += (float)a.bias[row];
          r[i] = round16(v);
        } else {
          const float res = ok ? (float)a.residual[(int64_t)m * a.N + row] : 0.f;
          r[i] = round16(round16(v) + res);
          ss += ok ? r[i] * r[i] : 0.f;
        }
        if (EPI != kEpiResidNorm && ok) a.out[(int64_t)m * a.N + row] = (f16)r[i];
      }
      if constexpr (EPI == kEpiResidNorm) {
        // device-coherent: the workgroup that finishes last reads them (N % 16 == 0)
        if (m < M) {
          const f16x4 h4 = {(f16)r[0], (f16)r[1], (f16)r[2], (f16)r[3]};
          __builtin_amdgcn_raw_buffer_store_b64(
              __builtin_bit_cast(u32x2, h4), rsrc(a.out, (uint32_t)M * a.N * 2),
              (uint32_t)(m * a.N + row0) * 2, 0, kSc1);
        }
      }
      if constexpr (RES) {
        ss += shfl_xor_f(ss, 16);
        ss += shfl_xor_f(ss, 32);
        if (g == 0 && m < M) {
          if constexpr (EPI == kEpiResidNorm)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ss),
                                                  rsrc(a.out_ss, (uint32_t)a.tiles * M * 4),
                                                  (uint32_t)(tile * M + m) * 4, 0, kSc1);
          else
            a.out_ss[tile * M + m] = ss;
        }
      }
    } else if constexpr (EPI == kEpiSilu) {
      // lanes g = 0, 1 hold gate columns 8*tile + 4g + i, lanes g + 2 the up values
      float up[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) up[i] = shfl_xor_f(acc[mt][i], 32);
      const int inter = a.N / 2;
      if (g < 2 && m < M) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = tile * 8 + 4 * g + i;
          if (c < inter) {
            const float gv = round16(acc[mt][i] + (a.bias ? (float)a.bias[c] : 0.f));
            const float uv = round16(up[i] + (a.bias ? (float)a.bias[inter + c] : 0.f));
            const float s = round16(gv / (1.f + expf(-gv)));
            a.out[(int64_t)m * inter + c] = (f16)(s * uv);
          }
        }
      }
    } else {  // kEpiRope
      // lanes g = 0, 1: dims 8j + 4g + i of head hh (first half), lanes g + 2
      // the dims D/2 further
      float hi_v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) hi_v[i] = shfl_xor_f(acc[mt][i], 32);
      const int per_head = a.d / 16;
      const int hh = tile / per_head;
      const int j = tile - hh * per_head;
      if (g < 2 && m < M) {
        f16* dst;
        if (hh < a.hq) dst = a.out + ((int64_t)m * a.hq + hh) * a.d;
        else if (hh < a.hq + a.hkv) dst = a.k_out + ((int64_t)m * a.hkv + hh - a.hq) * a.d;
        else dst = a.v_out + ((int64_t)m * a.hkv + hh - a.hq - a.hkv) * a.d;
        const bool rot = hh < a.hq + a.hkv;
        const float pos = (float)a.positions[m];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dim = 8 * j + 4 * g + i;
          const int row_lo = hh * a.d + dim;
          const float x1 = round16(acc[mt][i] + (a.bias ? (float)a.bias[row_lo] : 0.f));
          const float x2 =
              round16(hi_v[i] + (a.bias ? (float)a.bias[row_lo + a.d / 2] : 0.f));
          f16 o1 = (f16)x1, o2 = (f16)x2;
          if (rot) {
            const float ang = pos * a.inv_freq[dim];
            const float c = round16(cosf(ang)), s = round16(sinf(ang));
            o1 = (f16)(round16(x1 * c) + round16(-x2 * s));
            o2 = (f16)(round16(x2 * c) + round16(x1 * s));
          }
          dst[dim] = o1;
          dst[dim + a.d / 2] = o2;
        }
      }
    }
  }

  if constexpr (KEEP) {
    // this tile's r and sums are complete device-wide; the workgroup of the
    // last tile normalises all rows (every wave a share) and leaves the
    // ticket at zero
    int last = 0;
    if (w == 0) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane == 0)
        last = __hip_atomic_fetch_add(a.grid_ticket, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == a.tiles - 1;
      last = __builtin_amdgcn_readfirstlane(last);
      if (last && lane == 0)
        __hip_atomic_store(a.grid_ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!broadcast(last, 1)) return;
    norm_tail(a, w, WAVES, lane);
  }
}

constexpr size_t kFusedTicketBytes = 64 * 1024;  // tickets for up to 16383 tiles
constexpr int kGridTicket = kFusedTicketBytes / sizeof(int) - 1;  // the launch-wide ticket

// Workgroups per tile when the tiles alone leave the chip short of ~192
// workgroups (split-K across workgroups, at least 512 keys each), or 1.  Every
// split adds a partial-tile round trip and a ticket before the epilogue; on
// the Qwen2.5-1.5B decode step (q/k/v 128 tiles, o and down 96) a target of
// 192 workgroups measured best: 512 -> 192 raised B = 1 from ~510 to ~544
// tok/s, and no split at all (one workgroup per tile) fell to ~489.
constexpr int kSplitTargetWgs = 192;
int ks_for(int tiles, int K) {
  int ks = (kSplitTargetWgs + tiles - 1) / tiles;
  const int max_ks = K / 512 > 0 ? K / 512 : 1;
  ks = ks < max_ks ? ks : max_ks;
  return ks > 1 ? ks : 1;
}


}  // namespace

// Workspace of the fused projections for these sizes: split-K tickets at
// offset 0 (fixed region, shared by every shape) and the partial tiles.
extern "C" size_t fe_gemm_fused_workspace_size(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return kFusedTicketBytes;
  const int tiles = (N + 15) / 16;
  const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  return kFusedTicketBytes + (size_t)tiles * ks_for(tiles, K) * mt * kWave * 16;
}

namespace {

// Waves per workgroup: enough to put ~2048 waves in flight when there are few
// tiles, and at least 32 keys per wave.  With many tiles (gate/up: 1120, the
// LM head: 9496) one wave per workgroup streaming all of K measured fastest
// (B = 1: 4 waves 544, 2 waves 554, 1 wave 568 tok/s): a wave's pipeline ramp
// and drain are paid once per longer stream, and no LDS reduction is needed.
constexpr int kManyTilesWaves = 1;
int waves_for(int tiles, int K) {
  int waves = tiles <= 160 ? 16 : (tiles <= 512 ? 8 : kManyTilesWaves);
  while (waves > 1 && (int64_t)(waves - 1) * 32 >= K) waves /= 2;
  return waves;
}

template <int EPI, bool NORM>
int launch_fused(FusedArgs a, int tiles, void* workspace, size_t workspace_bytes,
                 hipStream_t stream) {
  a.tiles = tiles;
  a.ks_count = ks_for(tiles, a.K);
  if (a.ks_count > 1 || EPI == kEpiResidNorm) {
    const size_t need = fe_gemm_fused_workspace_size(a.M, a.N, a.K);
    if (workspace == nullptr || workspace_bytes < need ||
        (reinterpret_cast<uintptr_t>(workspace) & 255))
      return FE_ERR_WORKSPACE;
    a.tickets = (int*)workspace;
    a.part = (f32x4*)((char*)workspace + kFusedTicketBytes);
    a.grid_ticket = a.tickets + kGridTicket;
  }
  int kslice_wg = (a.K + a.ks_count - 1) / a.ks_count;
  a.kslice_wg = (kslice_wg + 31) / 32 * 32;
  // split workgroups: 4 waves (1, 2, 8 and 16 measured slower)
  int waves = a.ks_count > 1 ? 4 : waves_for(tiles, a.K);
  if (a.M > 16 && waves > 8) waves = 8;  // two row tiles: the register budget of 8 waves
  if (a.M > 32 && waves > 4) waves = 4;  // four row tiles: at most 4 waves
  int kslice = (a.kslice_wg + waves - 1) / waves;
  a.kslice = (kslice + 31) / 32 * 32;
  const dim3 grid((unsigned)((int64_t)tiles * a.ks_count));
#define FE_FUSED(MT, WV)                                                                       \
  hipLaunchKernelGGL((gemm_fused_kernel<MT, WV, EPI, NORM>), grid, dim3((WV) * kWave), 0, \
                     stream, a)
  if (a.M <= 16) {
    if (waves == 16) FE_FUSED(1, 16);
    else if (waves == 8) FE_FUSED(1, 8);
    else if (waves == 2) FE_FUSED(1, 2);
    else if (waves == 1) FE_FUSED(1, 1);
    else FE_FUSED(1, 4);
  } else if (a.M <= 32) {
    if (waves == 8) FE_FUSED(2, 8);
    else if (waves == 2) FE_FUSED(2, 2);
    else if (waves == 1) FE_FUSED(2, 1);
    else FE_FUSED(2, 4);
  } else {
    if (waves == 1) FE_FUSED(4, 1);
    else if (waves == 2) FE_FUSED(4, 2);
    else FE_FUSED(4, 4);
  }
#undef FE_FUSED
  return FE_LAUNCH_STATUS();
}

// Common checks and the operand / prologue fields.
int fill_common(FusedArgs& a, const void* x, const float* x_ss, int ss_tiles, const void* norm_w,
                float eps, int M, int K, const void* W, int N) {
  FE_CHECK_ARG(M >= 0 && K > 0 && N > 0);
  if (M > 64 || K % 32 != 0) return FE_ERR_UNSUPPORTED;
  // 32-bit buffer offsets into W and x
  FE_CHECK_ARG((int64_t)N * K * 2 < ((int64_t)1 << 31) && (int64_t)M * K * 2 < ((int64_t)1 << 31));
  FE_CHECK_ARG(x && W);
  // x and W are read with 16-byte loads
  FE_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W)) & 15) == 0);
  FE_CHECK_ARG(x_ss == nullptr || (ss_tiles > 0 && ss_tiles <= 4 * kMaxSsPerLane && norm_w != nullptr));
  a = FusedArgs{};
  a.W = (const f16*)W;
  a.N = N;
  a.K = K;
  a.M = M;
  a.x = (const f16*)x;
  a.x_ss = x_ss;
  a.ss_tiles = ss_tiles;
  a.norm_w = (const f16*)norm_w;
  a.eps = eps;
  return FE_OK;
}

}  // namespace

extern "C" int fe_gemm_f16(const void* x, const float* x_ss, int ss_tiles, const void* norm_w,
                           float eps, int M, int K, const void* W, int N, const void* bias,
                           void* out, void* workspace, size_t workspace_bytes,
                           fe_stream_t stream) {
  FusedArgs a;
  const int rc = fill_common(a, x, x_ss, ss_tiles, norm_w, eps, M, K, W, N);
  if (rc != FE_OK || M == 0) return rc;
  FE_CHECK_ARG(out != nullptr);
  a.bias = (const f16*)bias;
  a.out = (f16*)out;
  const int tiles = (N + 15) / 16;
  return x_ss ? launch_fused<kEpiF16, true>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream)
              : launch_fused<kEpiF16, false>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int fe_gemm_resid(const void* x, int M, int K, const void* W, int N,
                             const void* residual, void* out, float* out_ss, void* workspace,
                             size_t workspace_bytes, fe_stream_t stream) {
  FusedArgs a;
  const int rc = fill_common(a, x, nullptr, 0, nullptr, 0.f, M, K, W, N);
  if (rc != FE_OK || M == 0) return rc;
  FE_CHECK_ARG(residual && out && out_ss);
  FE_CHECK_ARG(out != residual && out != x);  // the header: out aliases nothing read
  a.residual = (const f16*)residual;
  a.out = (f16*)out;
  a.out_ss = out_ss;
  return launch_fused<kEpiResid, false>(a, (N + 15) / 16, workspace, workspace_bytes,
                                        (hipStream_t)stream);
}

extern "C" int fe_gemm_resid_rmsnorm(const void* x, int M, int K, const void* W, int N,
                                     const void* residual, void* out, float* out_ss,
                                     const void* norm_w, float eps, void* norm_out,
                                     void* workspace, size_t workspace_bytes,
                                     fe_stream_t stream) {
  FusedArgs a;
  const int rc = fill_common(a, x, nullptr, 0, nullptr, 0.f, M, K, W, N);
  if (rc != FE_OK || M == 0) return rc;
  FE_CHECK_ARG(residual && out && out_ss && norm_w && norm_out);
  // out, out_ss and norm_out alias nothing the call reads, nor each other
  FE_CHECK_ARG(out != residual && out != x && norm_out != out && norm_out != residual &&
               norm_out != x);
  if (N % 16 != 0 || N > kWave * 8 * kTailChunks || N / 16 > kWave * kTailSs)
    return FE_ERR_UNSUPPORTED;
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  FE_CHECK_ARG(al16(out) && al16(norm_w) && al16(norm_out));
  a.residual = (const f16*)residual;
  a.out = (f16*)out;
  a.out_ss = out_ss;
  a.tail_w = (const f16*)norm_w;
  a.tail_eps = eps;
  a.tail_out = (f16*)norm_out;
  return launch_fused<kEpiResidNorm, false>(a, N / 16, workspace, workspace_bytes,
                                            (hipStream_t)stream);
}

extern "C" int fe_gemm_silu(const void* x, const float* x_ss, int ss_tiles, const void* norm_w,
                            float eps, int M, int K, const void* W, int N, void* out,
                            void* workspace, size_t workspace_bytes, fe_stream_t stream) {
  FusedArgs a;
  const int rc = fill_common(a, x, x_ss, ss_tiles, norm_w, eps, M, K, W, N);
  if (rc != FE_OK || M == 0) return rc;
  FE_CHECK_ARG(out != nullptr && N % 2 == 0);
  a.out = (f16*)out;
  const int tiles = (N / 2 + 7) / 8;
  return x_ss ? launch_fused<kEpiSilu, true>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream)
              : launch_fused<kEpiSilu, false>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int fe_gemm_rope(const void* x, const float* x_ss, int ss_tiles, const void* norm_w,
                            float eps, int M, int K, const void* W, const void* bias,
                            const int64_t* positions, const float* inv_freq, int num_q_heads,
                            int kv_heads, int head_dim, void* q_out, void* k_out, void* v_out,
                            void* workspace, size_t workspace_bytes, fe_stream_t stream) {
  FE_CHECK_ARG(num_q_heads > 0 && kv_heads > 0 && head_dim > 0);
  if (head_dim % 16 != 0) return FE_ERR_UNSUPPORTED;
  const int N = (num_q_heads + 2 * kv_heads) * head_dim;
  FusedArgs a;
  const int rc = fill_common(a, x, x_ss, ss_tiles, norm_w, eps, M, K, W, N);
  if (rc != FE_OK || M == 0) return rc;
  FE_CHECK_ARG(positions && inv_freq && q_out && k_out && v_out);
  a.bias = (const f16*)bias;
  a.out = (f16*)q_out;
  a.k_out = (f16*)k_out;
  a.v_out = (f16*)v_out;
  a.positions = positions;
  a.inv_freq = inv_freq;
  a.hq = num_q_heads;
  a.hkv = kv_heads;
  a.d = head_dim;
  const int tiles = N / 16;
  return x_ss ? launch_fused<kEpiRope, true>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream)
              : launch_fused<kEpiRope, false>(a, tiles, workspace, workspace_bytes, (hipStream_t)stream);
}
