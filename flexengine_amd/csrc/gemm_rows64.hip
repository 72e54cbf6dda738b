// Decode-step projections for 33..64 rows (the batch-64 decode step) on gfx950:
// out [M][N] = fp16(x [M][K] @ W^T + bias), W in PyTorch Linear layout [N][K].
//
// The fused projections of gemm_fused.hip give every lane its own x rows in
// registers; at 64 rows each wave would then re-read all of x for every weight
// tile (4x the weight bytes through the caches).  Here the four waves of a
// workgroup take four different 16-row weight tiles over the same K range, and
// each 128-key chunk of x (up to 64 rows, 16 KiB) is staged once in LDS and read
// by all four: x travels once per workgroup, the weights once in total.
//
// Per 128-key step a wave multiplies its tile (the A operand of
// v_mfma_f32_16x16x16_f16, lane (g, n): weight row n, 16 bytes at k0 + 32j + 8g
// straight from HBM, two register stages) with the MT x tiles read from LDS
// (B operand, lane (g, n): x row mt*16 + n, same keys).  The next step's weight
// and x loads are in flight while a step computes; one barrier per step hands
// the x buffer over.  When the weight tiles alone leave the chip short of ~256
// workgroups, K is split across workgroups; each writes its fp32 partial tile
// with device-coherent stores and takes a per-tile ticket, and the last adds
// the partials in split order (deterministic) and writes the fp16 result.
// Replaces the library GEMMs (torch.nn.functional.linear -> hipBLASLt) of the
// batch-64 decode step (src/flexengine/inference/models/qwen2.py:152-154,
// 183-186 through the HF modules).
#include "fe_common.h"

using namespace fe;

namespace {

constexpr int kStep = 128;                // keys per pipeline step
constexpr int kTilesPerWg = 4;            // one 16-row weight tile per wave
constexpr int kThreadsR = kTilesPerWg * kWave;
constexpr int kXPitch = kStep + 8;        // halves per staged x row: 16 bytes of padding
constexpr int kTargetWgs = 256;           // split K until about this many workgroups
constexpr size_t kTicketBytesR = 64 * 1024;  // per-tile tickets (up to 16384 tiles)
constexpr int kSc1 = 16;                  // buffer-instruction cache policy: sc1

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct RowsArgs {
  const f16* W;      // [N][K]
  const f16* x;      // [M][K]
  const f16* bias;   // [N] or null
  f16* out;          // [M][N]
  int N, K, M;
  int groups;        // workgroups per K split (ceil(tiles / kTilesPerWg))
  int ks_count;      // K splits
  int kslice;        // keys per split (a multiple of 32)
  f32x4* part;       // [tiles][ks_count][MT][64] lane-layout partial tiles
  int* tickets;      // [tiles], zero between calls
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

template <int MT>
__global__ __launch_bounds__(kThreadsR) void gemm_rows64_kernel(const RowsArgs a) {
  __shared__ __align__(16) f16 xs[2][MT * 16][kXPitch];
  constexpr int XCH = MT * 16 * (kStep / 8) / kThreadsR;  // 16-byte x chunks per thread
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int group = blockIdx.x % a.groups;
  const int ks = blockIdx.x / a.groups;
  const int tile = group * kTilesPerWg + w;
  const int tiles = (a.N + 15) / 16;
  const int M = a.M;
  const int k_begin = ks * a.kslice;
  const int k_end = min(a.K, k_begin + a.kslice);

  // weight row tile*16 + n; rows past N (and tiles past the last) read zeros
  const uint32_t wbytes = (uint32_t)a.N * a.K * 2;
  const __amdgpu_buffer_rsrc_t rw = rsrc(a.W, wbytes);
  const int row = tile * 16 + n;
  const uint32_t w_off = row < a.N ? (uint32_t)(row * a.K * 2 + g * 16) : wbytes;
  // x rows past M read zeros (the descriptor ends at row M)
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (uint32_t)M * a.K * 2);

  f16x8 wa[4], wb[4], xr[XCH];
  auto load_w = [&](f16x8 (&wr)[4], int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      wr[j] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(rw, w_off, (uint32_t)(k0 + 32 * j) * 2, 0));
  };
  // thread t stages chunks t, t + 256, ...: x row c / 16, keys (c % 16) * 8 .. +7
  auto load_x = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
      const int idx = threadIdx.x + c * kThreadsR;
      const int xrow = idx >> 4;
      const int col = (idx & 15) * 8;
      const uint32_t off =
          xrow < M && k0 + col < a.K ? (uint32_t)(xrow * a.K + k0 + col) * 2 : (uint32_t)M * a.K * 2;
      xr[c] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  };
  auto store_x = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
      const int idx = threadIdx.x + c * kThreadsR;
      *reinterpret_cast<f16x8*>(&xs[buf][idx >> 4][(idx & 15) * 8]) = xr[c];
    }
  };

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // nj: 32-key groups of the step below k_end (the last step of a split may be short)
  auto compute = [&](const f16x8 (&wr)[4], int buf, int nj) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nj) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f16x8 xv = *reinterpret_cast<const f16x8*>(&xs[buf][mt * 16 + n][32 * j + 8 * g]);
          acc[mt] = mfma16(lo4(wr[j]), lo4(xv), acc[mt]);
          acc[mt] = mfma16(hi4(wr[j]), hi4(xv), acc[mt]);
        }
      }
    }
  };

  // every wave runs the same number of steps and barriers (k_begin, k_end are
  // uniform over the workgroup)
  int k0 = k_begin;
  int buf = 0;
  if (k0 < k_end) {
    load_w(wa, k0);
    load_x(k0);
    store_x(0);
  }
  __syncthreads();
  while (k0 < k_end) {
    const int nj = min(4, (k_end - k0) / 32);
    const int kn = k0 + kStep;
    const bool more = kn < k_end;
    if (more) {
      load_w(wb, kn);
      load_x(kn);
    }
    compute(wa, buf, nj);
    if (more) store_x(buf ^ 1);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) wa[j] = wb[j];
    k0 = kn;
    buf ^= 1;
  }
  if (tile >= tiles) return;

  // ---- split-K: the last workgroup of the tile adds the partials in split order ----
  if (a.ks_count > 1) {
    const __amdgpu_buffer_rsrc_t rp = rsrc(a.part + (int64_t)tile * a.ks_count * MT * kWave,
                                           (uint32_t)a.ks_count * MT * kWave * 16);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt]), rp,
                                             (uint32_t)(((ks * MT + mt) * kWave + lane) * 16), 0,
                                             kSc1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // partial complete device-wide
    int last = 0;
    if (lane == 0)
      last = __hip_atomic_fetch_add(a.tickets + tile, 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == a.ks_count - 1;
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    if (lane == 0)
      __hip_atomic_store(a.tickets + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // MB splits' partials in flight at once (a load-add loop would wait out one
    // round trip per split), added in split order
    constexpr int MB = 16 / MT;
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

  // ---- epilogue: lane (g, n) holds out[m = mt*16 + n][tile row 4g + i] ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + n;
    if (m >= M) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = tile * 16 + 4 * g + i;
      if (r >= a.N) continue;
      float v = acc[mt][i];
      if (a.bias) v += (float)a.bias[r];
      a.out[(int64_t)m * a.N + r] = (f16)v;
    }
  }
}

// K splits for `groups` workgroups per split: about kTargetWgs workgroups, at
// least two steps (256 keys) per split.
int ks_for_rows(int groups, int K) {
  int ks = (kTargetWgs + groups - 1) / groups;
  const int max_ks = K / 256 > 0 ? K / 256 : 1;
  ks = ks < max_ks ? ks : max_ks;
  return ks > 1 ? ks : 1;
}

}  // namespace

extern "C" size_t fe_gemm_rows64_workspace_size(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return kTicketBytesR;
  const int tiles = (N + 15) / 16;
  const int groups = (tiles + kTilesPerWg - 1) / kTilesPerWg;
  const int mt = (M + 15) / 16;
  return kTicketBytesR + (size_t)tiles * ks_for_rows(groups, K) * mt * kWave * 16;
}

extern "C" int fe_gemm_rows64(const void* x, int M, int K, const void* W, int N,
                              const void* bias, void* out, void* workspace,
                              size_t workspace_bytes, fe_stream_t stream) {
  FE_CHECK_ARG(M >= 0 && K > 0 && N > 0);
  if (M > 64 || K % 32 != 0) return FE_ERR_UNSUPPORTED;
  // 32-bit buffer offsets into W and x
  FE_CHECK_ARG((int64_t)N * K * 2 < ((int64_t)1 << 31) && (int64_t)M * K * 2 < ((int64_t)1 << 31));
  if (M == 0) return FE_OK;
  FE_CHECK_ARG(x && W && out);
  FE_CHECK_ARG(out != x);
  // x and W are read with 16-byte loads
  FE_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W)) & 15) == 0);
  const int tiles = (N + 15) / 16;
  if (tiles > (int)(kTicketBytesR / sizeof(int))) return FE_ERR_UNSUPPORTED;
  RowsArgs a;
  a.W = (const f16*)W;
  a.x = (const f16*)x;
  a.bias = (const f16*)bias;
  a.out = (f16*)out;
  a.N = N;
  a.K = K;
  a.M = M;
  a.groups = (tiles + kTilesPerWg - 1) / kTilesPerWg;
  a.ks_count = ks_for_rows(a.groups, K);
  const int kslice = (K + a.ks_count - 1) / a.ks_count;
  a.kslice = (kslice + 31) / 32 * 32;
  a.part = nullptr;
  a.tickets = nullptr;
  if (a.ks_count > 1) {
    const size_t need = fe_gemm_rows64_workspace_size(M, N, K);
    if (workspace == nullptr || workspace_bytes < need ||
        (reinterpret_cast<uintptr_t>(workspace) & 255))
      return FE_ERR_WORKSPACE;
    a.tickets = (int*)workspace;
    a.part = (f32x4*)((char*)workspace + kTicketBytesR);
  }
  const dim3 grid((unsigned)((int64_t)a.groups * a.ks_count));
  const hipStream_t s = (hipStream_t)stream;
  const int mt = (M + 15) / 16;
  if (mt == 1) hipLaunchKernelGGL(gemm_rows64_kernel<1>, grid, dim3(kThreadsR), 0, s, a);
  else if (mt == 2) hipLaunchKernelGGL(gemm_rows64_kernel<2>, grid, dim3(kThreadsR), 0, s, a);
  else if (mt == 3) hipLaunchKernelGGL(gemm_rows64_kernel<3>, grid, dim3(kThreadsR), 0, s, a);
  else hipLaunchKernelGGL(gemm_rows64_kernel<4>, grid, dim3(kThreadsR), 0, s, a);
  return FE_LAUNCH_STATUS();
}
