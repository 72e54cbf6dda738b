// Element-wise kernels of the decoder layer around the attention: fused
// residual add + RMSNorm, RoPE on the fused q/k/v projection, SiLU-gated
// product.  Each replaces a chain of ~5-15 small PyTorch kernels per call
// (src/flexengine/inference/models/qwen2.py:67-77,97-102,129-130 and the HF
// Qwen2RMSNorm / Qwen2MLP they call), which on a graph-replayed decode step
// cost more GPU time than the layer's GEMMs.
//
// Rounding follows the PyTorch fp16 semantics of those chains -- every
// element-wise op computes in fp32 and rounds its result to fp16 -- so the
// fused results match the unfused ones up to the last-ulp differences of the
// transcendental functions.
#include "fe_common.h"

using namespace fe;

// No multiply-add contraction in this file: PyTorch rounds every product and
// every sum of these chains separately (a fused multiply-add skips a rounding).
#pragma clang fp contract(off)

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormMaxPerThread = 32;  // hidden sizes up to 8192

__device__ __forceinline__ float round16(float x) { return (float)(f16)x; }

// An input matrix [rows][cols] given either as fp16 rows (splits == 0, with a
// row stride in elements) or as the fp32 partial products of fe_gemm_skinny
// (splits > 0: [splits][rows][cols], summed here, plus an optional fp16 bias),
// rounded to fp16 like a library GEMM's output.
struct Src {
  const void* p;
  int64_t stride;
  int splits;
  const f16* bias;
  __device__ __forceinline__ float at(int row, int rows, int col, int cols) const {
    if (splits == 0) return (float)static_cast<const f16*>(p)[(int64_t)row * stride + col];
    const float* f = static_cast<const float*>(p);
    float acc = 0.f;
#pragma unroll 4  // four partial loads in flight per round trip; added in split order
    for (int k = 0; k < splits; ++k) acc += f[((int64_t)k * rows + row) * cols + col];
    if (bias) acc += (float)bias[col];
    return round16(acc);
  }
};

// One workgroup per row.  r = x (+ residual), rounded to fp16 (the residual
// stream's dtype); residual_out = r; out = weight * fp16(r * rsqrt(mean(r^2) + eps))
// (transformers' Qwen2RMSNorm: the normalised value is cast to fp16 before
// the weight multiply).  A decode step runs this on a handful of rows, so it
// is pure latency: every global load of a thread (its x partials, residual and
// weight elements) is issued before the first one is waited for.
constexpr int kNormMaxSplits = 8;

template <int PER>  // elements per thread: hidden <= PER * kNormThreads
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    Src x, const f16* __restrict__ residual, f16* __restrict__ residual_out,
    const f16* __restrict__ weight, f16* __restrict__ out, int rows, int hidden, float eps) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)row * hidden;
  float v[PER], wv[PER];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid + j * kNormThreads;
    const bool ok = e < hidden;
    const int ec = ok ? e : hidden - 1;
    float a;
    if (x.splits == 0) {
      a = (float)static_cast<const f16*>(x.p)[(int64_t)row * x.stride + ec];
    } else {
      const float* f = static_cast<const float*>(x.p);
      float part[kNormMaxSplits];
#pragma unroll
      for (int k = 0; k < kNormMaxSplits; ++k)
        part[k] = k < x.splits ? f[((int64_t)k * rows + row) * hidden + ec] : 0.f;
      a = 0.f;
#pragma unroll
      for (int k = 0; k < kNormMaxSplits; ++k) a += part[k];
      for (int k = kNormMaxSplits; k < x.splits; ++k) a += f[((int64_t)k * rows + row) * hidden + ec];
      a = round16(a);
    }
    const float rsd = residual ? (float)residual[base + ec] : 0.f;
    wv[j] = (float)weight[ec];
    const f16 r = (f16)(a + rsd);
    if (ok && residual_out) residual_out[base + e] = r;
    v[j] = ok ? (float)r : 0.f;
    ss += v[j] * v[j];
  }
  __shared__ float part_ss[kNormThreads / kWave];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
  if (lane_id() == 0) part_ss[tid / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) tot += part_ss[w];
  const float inv = rsqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = tid + j * kNormThreads;
    if (e < hidden) out[base + e] = (f16)(wv[j] * round16(v[j] * inv));
  }
}

// The same RMSNorm for fp16 rows (no partials), one wave per row: each lane
// holds NCH 16-byte chunks of the row (hidden <= 512 * NCH), so the whole row
// is one batch of loads and the sum of squares one cross-lane reduction -- no
// LDS, no barrier.  Four rows per 256-thread workgroup.
template <int NCH>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(
    const f16* __restrict__ x, const f16* residual, f16* residual_out,  // may alias (in place)
    const f16* __restrict__ weight, f16* __restrict__ out, int rows, int hidden, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t base = (int64_t)row * hidden;
  f16x8 xv[NCH], rv[NCH], wv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e0 = (c * kWave + lane) * 8;
    const bool ok = e0 < hidden;
    xv[c] = ok ? ld16(x + base + e0) : f16x8{};
    rv[c] = ok && residual ? ld16(residual + base + e0) : f16x8{};
    wv[c] = ok ? ld16(weight + e0) : f16x8{};
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f16 r = residual ? (f16)((float)xv[c][e] + (float)rv[c][e]) : xv[c][e];
      xv[c][e] = r;
      ss += (float)r * (float)r;
    }
    const int e0 = (c * kWave + lane) * 8;
    if (residual_out && e0 < hidden) st16(residual_out + base + e0, xv[c]);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
  const float inv = rsqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e0 = (c * kWave + lane) * 8;
    if (e0 >= hidden) continue;
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (f16)((float)wv[c][e] * round16((float)xv[c][e] * inv));
    st16(out + base + e0, o);
  }
}

// RoPE (rotate_half form) on the q and k heads of a fused projection row
// [q: Hq*D | k: Hkv*D | v: Hkv*D]; v is copied.  One thread per (row, head,
// pair i < D/2): angle = pos * inv_freq[i] in fp32, c = fp16(cos), s = fp16(sin),
//   out[i]       = fp16(fp16(x[i] * c)       + fp16(-x[i + D/2] * s))
//   out[i + D/2] = fp16(fp16(x[i + D/2] * c) + fp16( x[i] * s))
__global__ void rope_qkv_kernel(Src qkv, const int64_t* __restrict__ positions,
                                const float* __restrict__ inv_freq, f16* __restrict__ q_out,
                                f16* __restrict__ k_out, f16* __restrict__ v_out, int rows, int hq,
                                int hkv, int d) {
  const int half = d / 2;
  const int heads = hq + 2 * hkv;
  const int64_t total = (int64_t)rows * heads * half;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(t % half);
    const int hh = (int)((t / half) % heads);
    const int row = (int)(t / ((int64_t)half * heads));
    const int cols = heads * d;
    const f16 x1 = (f16)qkv.at(row, rows, hh * d + i, cols);
    const f16 x2 = (f16)qkv.at(row, rows, hh * d + i + half, cols);
    if (hh >= hq + hkv) {
      f16* dst = v_out + ((int64_t)row * hkv + (hh - hq - hkv)) * d;
      dst[i] = x1;
      dst[i + half] = x2;
      continue;
    }
    const float ang = (float)positions[row] * inv_freq[i];
    const float c = round16(cosf(ang)), s = round16(sinf(ang));
    const float a = (float)x1, b = (float)x2;
    const f16 o1 = (f16)(round16(a * c) + round16(-b * s));
    const f16 o2 = (f16)(round16(b * c) + round16(a * s));
    f16* dst = hh < hq ? q_out + ((int64_t)row * hq + hh) * d
                       : k_out + ((int64_t)row * hkv + (hh - hq)) * d;
    dst[i] = o1;
    dst[i + half] = o2;
  }
}

// out = fp16(fp16(silu(g)) * u) over a fused [gate | up] row.
__global__ void silu_mul_kernel(Src gate_up, f16* __restrict__ out, int rows, int inter) {
  const int64_t total = (int64_t)rows * inter;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(t / inter);
    const int e = (int)(t % inter);
    const float g = gate_up.at(row, rows, e, 2 * inter);
    const float s = round16(g / (1.f + expf(-g)));
    out[t] = (f16)(s * gate_up.at(row, rows, inter + e, 2 * inter));
  }
}

inline int grid_for(int64_t work, int threads) {
  const int64_t blocks = (work + threads - 1) / threads;
  return (int)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace

extern "C" int fe_rmsnorm(const void* x, int x_splits, const void* residual, void* residual_out,
                          const void* weight, void* out, int rows, int hidden, float eps,
                          fe_stream_t stream) {
  FE_CHECK_ARG(rows >= 0 && hidden > 0 && x_splits >= 0);
  if (hidden > kNormThreads * kNormMaxPerThread) return FE_ERR_UNSUPPORTED;
  if (rows == 0) return FE_OK;
  FE_CHECK_ARG(x && weight && out);
  const auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (x_splits == 0 && hidden % 8 == 0 && al(x) && al(residual) && al(residual_out) &&
      al(weight) && al(out)) {
    const int nch = (hidden + 511) / 512;
    const dim3 grid((rows + 3) / 4);
#define FE_NORM_WAVE(N)                                                                        \
  hipLaunchKernelGGL(rmsnorm_wave_kernel<N>, grid, dim3(256), 0, (hipStream_t)stream,           \
                     (const f16*)x, (const f16*)residual, (f16*)residual_out, (const f16*)weight, \
                     (f16*)out, rows, hidden, eps)
    if (nch <= 1) FE_NORM_WAVE(1);
    else if (nch <= 2) FE_NORM_WAVE(2);
    else if (nch <= 3) FE_NORM_WAVE(3);
    else if (nch <= 4) FE_NORM_WAVE(4);
    else if (nch <= 8) FE_NORM_WAVE(8);
    else FE_NORM_WAVE(16);
#undef FE_NORM_WAVE
    return FE_LAUNCH_STATUS();
  }
  const Src src{x, hidden, x_splits, nullptr};
  const int per = (hidden + kNormThreads - 1) / kNormThreads;
#define FE_NORM_LAUNCH(P)                                                                        \
  hipLaunchKernelGGL(rmsnorm_kernel<P>, dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream, \
                     src, (const f16*)residual, (f16*)residual_out, (const f16*)weight,         \
                     (f16*)out, rows, hidden, eps)
  if (per <= 2) FE_NORM_LAUNCH(2);
  else if (per <= 4) FE_NORM_LAUNCH(4);
  else if (per <= 8) FE_NORM_LAUNCH(8);
  else if (per <= 16) FE_NORM_LAUNCH(16);
  else FE_NORM_LAUNCH(32);
#undef FE_NORM_LAUNCH
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_rope_qkv(const void* qkv, int64_t row_stride, int qkv_splits, const void* bias,
                           const int64_t* positions, const float* inv_freq, void* q_out,
                           void* k_out, void* v_out, int rows, int num_q_heads, int kv_heads,
                           int head_dim, fe_stream_t stream) {
  FE_CHECK_ARG(rows >= 0 && num_q_heads > 0 && kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0);
  FE_CHECK_ARG(qkv_splits >= 0);
  FE_CHECK_ARG(qkv_splits > 0 || row_stride >= (int64_t)(num_q_heads + 2 * kv_heads) * head_dim);
  if (rows == 0) return FE_OK;
  FE_CHECK_ARG(qkv && positions && inv_freq && q_out && k_out && v_out);
  const int64_t work = (int64_t)rows * (num_q_heads + 2 * kv_heads) * (head_dim / 2);
  hipLaunchKernelGGL(rope_qkv_kernel, dim3(grid_for(work, 256)), dim3(256), 0, (hipStream_t)stream,
                     Src{qkv, row_stride, qkv_splits, (const f16*)bias}, positions, inv_freq,
                     (f16*)q_out, (f16*)k_out, (f16*)v_out, rows, num_q_heads, kv_heads, head_dim);
  return FE_LAUNCH_STATUS();
}

extern "C" int fe_silu_mul(const void* gate_up, int64_t row_stride, int splits, void* out, int rows,
                           int inter, fe_stream_t stream) {
  FE_CHECK_ARG(rows >= 0 && inter > 0 && splits >= 0);
  FE_CHECK_ARG(splits > 0 || row_stride >= 2 * (int64_t)inter);
  if (rows == 0) return FE_OK;
  FE_CHECK_ARG(gate_up && out);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for((int64_t)rows * inter, 256)), dim3(256), 0,
                     (hipStream_t)stream, Src{gate_up, row_stride, splits, nullptr}, (f16*)out, rows,
                     inter);
  return FE_LAUNCH_STATUS();
}
