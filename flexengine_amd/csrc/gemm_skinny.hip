// Skinny GEMM for decode-sized batches on gfx950: part[ks][m][o] =
// sum_{k in slice ks} x[m][k] * W[o][k], for M <= 32 rows of x and a weight
// W[N][K] in the PyTorch Linear layout.  Decode steps of a 1.5B model read
// ~3 GB of weights per token batch, so these products are HBM-bound weight
// streams; the library GEMMs reach ~1.3 TB/s at M = 1..8 (measured), this
// kernel streams the weights near the HBM roofline.
//
// Work: one wave per (16 output rows, K slice).  The 16 weight rows are the A
// operand of v_mfma_f32_16x16x16_f16 straight from HBM (lane (g, n) loads row
// n, 16 bytes at k0 + 32j + 8g: a wave reads 16 rows x 256 contiguous bytes per
// step), x supplies the B operand the same way (lane (g, n): row m = n of x).
// Lane (g, n) accumulates out[m = n][o = 16 tile + 4g + i].  K is cut into
// 4*S slices so that small N still gives thousands of waves; the four waves of
// a workgroup take four consecutive slices of the same 16 rows and add their
// results through LDS, so S fp32 partials are written (no atomics,
// deterministic) and the consumer kernel sums them (model_ops.hip).
#include "fe_common.h"

using namespace fe;

namespace {

constexpr int kGemmThreads = 256;
constexpr int kGemmWaves = kGemmThreads / kWave;
constexpr int kStepK = 128;  // k per pipeline step (4 MFMA k-groups of 32)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

__device__ __forceinline__ f16x8 ld(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

template <int MT>
struct Step {
  f16x8 w[4];
  f16x8 x[MT][4];
};

template <int MT>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
void gemm_skinny_kernel(const f16* __restrict__ x, int M, int K, const f16* __restrict__ W, int N,
                        float* __restrict__ part, int KS, int kslice) {
  const int lane = lane_id();
  const int g = lane >> 4;
  const int n = lane & 15;
  const int tiles = (N + 15) / 16;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x % tiles;
  const int ks = blockIdx.x / tiles;        // partial written by this workgroup
  const int k_begin = (ks * kGemmWaves + w) * kslice;
  const int k_end = min(K, k_begin + kslice);
  const int row0 = tile * 16;
  const int rows = min(16, N - row0);
  // descriptors: weight rows row0.. (rows past N read as zeros), all of x
  const __amdgpu_buffer_rsrc_t rw = rsrc(W + (int64_t)row0 * K, (uint32_t)rows * K * 2);
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, (uint32_t)M * K * 2);
  const uint32_t w_off = (uint32_t)(n * K * 2 + g * 16);
  uint32_t x_off[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) x_off[mt] = (uint32_t)((mt * 16 + n) * K * 2 + g * 16);

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto load = [&](Step<MT>& s, int k0) __attribute__((always_inline)) {
    // k0 past k_end: the loads stay inside the descriptors and are never used
#pragma unroll
    for (int j = 0; j < 4; ++j) s.w[j] = ld(rw, w_off, (uint32_t)(k0 + 32 * j) * 2);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) s.x[mt][j] = ld(rx, x_off[mt], (uint32_t)(k0 + 32 * j) * 2);
  };
  auto compute = [&](const Step<MT>& s, int nj) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nj) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt] = mfma16(lo4(s.w[j]), lo4(s.x[mt][j]), acc[mt]);
          acc[mt] = mfma16(hi4(s.w[j]), hi4(s.x[mt][j]), acc[mt]);
        }
      }
    }
  };

  // two register stages: step t+1's loads are in flight while step t is computed
  Step<MT> sa, sb;
  int k0 = k_begin;
  if (k0 < k_end) load(sa, k0);
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
    if (k0 >= k_end) break;
  }

  // the four waves' results for these 16 rows are added through LDS
  __shared__ f32x4 red[kGemmWaves - 1][MT][kWave];
  if (w > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[w - 1][mt][lane] = acc[mt];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int v = 0; v < kGemmWaves - 1; ++v)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] += red[v][mt][lane];
  // lane (g, n): out[m = mt*16 + n][o = row0 + 4g + i]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + n;
    if (m < M) {
      float* dst = part + ((int64_t)ks * M + m) * N + row0 + 4 * g;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * g + i < rows) dst[i] = acc[mt][i];
    }
  }
}

}  // namespace

// Number of fp32 partials fe_gemm_skinny writes for an N x K weight (the
// partial buffer holds splits * M * N floats); K is cut into 4 * splits slices.
extern "C" int fe_gemm_skinny_splits(int N, int K) {
  if (N <= 0 || K <= 0) return 0;
  const int tiles = (N + 15) / 16;
  // about 512 workgroups (2048 waves, eight per CU), slices of at least 128 keys
  int s = (512 + tiles - 1) / tiles;
  const int max_s = K / (kStepK * kGemmWaves) > 0 ? K / (kStepK * kGemmWaves) : 1;
  s = s < max_s ? s : max_s;
  return s > 0 ? s : 1;
}

extern "C" int fe_gemm_skinny(const void* x, int M, int K, const void* W, int N, float* partials,
                              int splits, fe_stream_t stream) {
  FE_CHECK_ARG(M >= 0 && K > 0 && N > 0 && splits > 0);
  if (M > 32 || K % 32 != 0) return FE_ERR_UNSUPPORTED;
  // 32-bit buffer offsets
  FE_CHECK_ARG((int64_t)16 * K * 2 < ((int64_t)1 << 31) && (int64_t)M * K * 2 < ((int64_t)1 << 31));
  if (M == 0) return FE_OK;
  FE_CHECK_ARG(x && W && partials);
  // x and W are read with 16-byte loads
  FE_CHECK_ARG(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W)) & 15) == 0);
  // 4 * splits slices of kslice keys (a multiple of 32); trailing slices may be
  // empty (their waves add zeros)
  const int slices = splits * kGemmWaves;
  int kslice = (K + slices - 1) / slices;
  kslice = (kslice + 31) / 32 * 32;
  FE_CHECK_ARG((int64_t)(splits - 1) * kGemmWaves * kslice < K);  // every partial holds keys
  const int tiles = (N + 15) / 16;
  const dim3 grid((unsigned)((int64_t)tiles * splits));
  if (M <= 16)
    hipLaunchKernelGGL(gemm_skinny_kernel<1>, grid, dim3(kGemmThreads), 0, (hipStream_t)stream,
                       (const f16*)x, M, K, (const f16*)W, N, partials, splits, kslice);
  else
    hipLaunchKernelGGL(gemm_skinny_kernel<2>, grid, dim3(kGemmThreads), 0, (hipStream_t)stream,
                       (const f16*)x, M, K, (const f16*)W, N, partials, splits, kslice);
  return FE_LAUNCH_STATUS();
}
