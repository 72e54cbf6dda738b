// Attention for the shapes the matrix-core kernels do not take: head_dim other
// than 64 and 128 (1 .. 512), and decode groups of 17 .. 32 query heads per KV
// head.  The reference's Triton decode takes any head_dim (BLOCK_D =
// next_power_of_2 and a dim mask, src/flexengine/inference/kernels/
// paged_attention.py:106,112,152), and its own synthetic-model test runs
// head_dim 8 (tests/unit/test_synthetic_qwen.py:55); these shapes keep that
// envelope.
//
// One workgroup (four waves) per item: a decode row's key split, or a tile of
// up to TQ consecutive prefill tokens (causal: token i of a sequence with c
// cached keys reads keys 0 .. c + i), for one KV head.  The item's R = tokens
// x G query rows sit in LDS as fp32, scaled to base 2.  Keys are walked in
// chunks of CK: the workgroup stages the chunk's K and V rows in LDS in their
// own element type with coalesced 16-byte loads (element loads when head_dim
// is not a multiple of the vector or the rows are not 16-byte aligned); the
// score pass puts one key on each lane (a wave holds 64 / CK segments of CK
// lanes, each segment a subset of the rows), reads the key's row 8 dims at a
// time against every row of its subset, and keeps each row's running maximum
// and sum in the segment's registers (online softmax, cross-lane reductions
// within the segment); the probabilities and rescale factors go to LDS; the
// product pass gives each thread 4 consecutive output dims of a row (and a
// share of the chunk's keys when the rows are few) and accumulates p * V in
// registers.  fp32 arithmetic throughout; fp16, bf16 and fp32 data.
//
// A decode split covers keys [s * span, (s + 1) * span) of its row, span a
// multiple of CK; with more than one split per row each split writes its
// normalised output and base-2 LSE to the caller's workspace and
// generic_merge_kernel folds them.  The decode's optional page write (k_new /
// v_new at key L - 1) is done by the split holding that key, which stages the
// new row from k_new / v_new directly.
#include <hip/hip_runtime.h>

#include "attn_core.h"
#include "flexengine_amd.h"

using namespace fe;

namespace {

#ifndef GEN_WAVES
#define GEN_WAVES 2
#endif
constexpr int kGThreads = 256;
constexpr int kGWaves = kGThreads / kWave;
constexpr int kGMaxRows = 64;     // query rows of one item (tokens x group)
constexpr int kGRowStep = 4;      // rows scored per pass over a key's row
constexpr int kGMaxQuads = 4;     // output quads per thread: rows x padded dims <= 4096
constexpr int kGPre = 4;          // prefetched 16-byte K (and V) vectors per thread: a row holds <= 4 x (256 / CK)
constexpr int kGMaxSplits = 32;   // decode key splits per row

struct GArgs {
  const void* q;
  int64_t q_stride;  // elements from one query token (or decode row) to the next
  void* out;
  int64_t out_stride;
  const void* k_new;  // decode page write (null: none)
  const void* v_new;
  int64_t new_stride;
  void* k_pool;
  void* v_pool;
  const int32_t* tables;
  int W;
  const int32_t* ctx;    // decode: [B] context lengths; prefill: [S]
  const int32_t* q_off;  // prefill: [S + 1] chunk offsets; null for the decode
  int S;                 // prefill: sequences
  int total;             // decode: rows; prefill: tokens
  int Hq, Hkv, G, D, DP, BS, bs_log2, NB;
  int TQ;                // tokens per prefill tile (1 for the decode)
  int splits;            // decode key splits per row
  float* part_o;         // [B * Hq][splits][D] when splits > 1
  float* part_lse;       // [B * Hq][splits]
  int vec;               // 16-byte global loads of K / V / new rows
  float scale_log2;
};

// s_waitcnt operand: lgkmcnt 0 (this wave's LDS operations done), vmcnt and
// expcnt at their maxima (not waited for)
constexpr int kWaitLgkm0 = 0xC07F;

// The workgroup's LDS handoff with this wave's global loads left in flight
// (__syncthreads()'s release fence would wait for them): the wave's LDS
// reads and writes complete, then the barrier; the compiler fences keep every
// LDS access on its side.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <class E>
constexpr int kElemBytes = kIsF32<E> ? 4 : 2;
template <class E>
constexpr int kVecElems = 16 / kElemBytes<E>;  // elements per 16-byte vector

template <class E>
__device__ __forceinline__ float ld_el(const void* base, int64_t i) {
  if constexpr (kIsF32<E>)
    return reinterpret_cast<const float*>(base)[i];
  else if constexpr (__is_same(E, Bf16))
    return (float)__builtin_bit_cast(__bf16, reinterpret_cast<const f16*>(base)[i]);
  else
    return (float)reinterpret_cast<const f16*>(base)[i];
}

template <class E>
__device__ __forceinline__ float el16(f16 v) {
  if constexpr (__is_same(E, Bf16))
    return (float)__builtin_bit_cast(__bf16, v);
  else
    return (float)v;
}

// 8 consecutive LDS elements of type E as floats (16-bit: one 16-byte read;
// fp32: two)
template <class E>
__device__ __forceinline__ void lds8(const unsigned char* p, float (&x)[8]) {
  if constexpr (kIsF32<E>) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
  } else {
    const f16x8 v = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = el16<E>(v[i]);
  }
}

// 4 consecutive LDS elements of type E as floats
template <class E>
__device__ __forceinline__ f32x4 lds4(const unsigned char* p) {
  if constexpr (kIsF32<E>) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const f16x4 v = *reinterpret_cast<const f16x4*>(p);
    return f32x4{el16<E>(v[0]), el16<E>(v[1]), el16<E>(v[2]), el16<E>(v[3])};
  }
}

// LDS layout of one workgroup (byte offsets), from the item's most rows R and
// padded dims DP: q [R][DP] fp32 | K [CK][DP elements + 16 bytes] | V [CK][DP]
// | p [R][CK] fp32 | rescale [R] | (max, sum) [R][2].  The K / V region holds
// the product pass's per-part partials at the end (4 KB; the p region starts
// after whichever is larger).
struct GLds {
  int q, k, v, p, al, ml, bytes, kst;
};
template <class E, int CK>
__host__ __device__ inline GLds glds(int R, int DP) {
  GLds l;
  l.kst = DP * kElemBytes<E> + 16;
  l.q = 0;
  l.k = R * DP * 4;
  l.v = l.k + CK * l.kst;
  const int kv_end = l.v + CK * DP * kElemBytes<E>;
  const int part_end = l.k + kGThreads * 16;
  l.p = kv_end > part_end ? kv_end : part_end;
  l.al = l.p + R * CK * 4;
  l.ml = l.al + R * 4;
  l.bytes = l.ml + R * 8;
  return l;
}

// One segment of an item: ntok query tokens from flattened index t0 (decode:
// the row), attending table row `trow` causally with key limits lim0,
// lim0 + 1, ... (decode: all L) over keys [k_lo, k_hi).  new_key (or -1) is
// staged from k_new / v_new.  Output: query head hq of token t at
// t * out_stride + hq * D, or the split's slot.
template <class E, int CK>
__device__ __forceinline__ void generic_segment(const GArgs& a, unsigned char* lds, int h,
                                                int trow, int t0,
                                int ntok, int lim0, int k_lo, int k_hi, int new_key, int split) {
  constexpr int NSEG = kWave / CK;
  constexpr int EB = kElemBytes<E>;
  constexpr int VW = kVecElems<E>;
  const int G = a.G, D = a.D, DP = a.DP;
  const int R = ntok * G;
  const GLds L = glds<E, CK>(a.TQ * G, DP);
  float* const qs = reinterpret_cast<float*>(lds + L.q);
  unsigned char* const ks = lds + L.k;
  unsigned char* const vs = lds + L.v;
  float* const ps = reinterpret_cast<float*>(lds + L.p);
  float* const al = reinterpret_cast<float*>(lds + L.al);
  float* const ml = reinterpret_cast<float*>(lds + L.ml);
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = tid / kWave;
  const int j = lane % CK;    // this lane's key in the chunk (score pass)
  const int seg = lane / CK;  // this lane's rows: w + 4 * (seg + NSEG * i)
  // lane segments per wave hold rows in slots 0 .. nslots - 1 (wave-uniform)
  const int nslots = (R + kGWaves * NSEG - 1) / (kGWaves * NSEG);
  const int64_t rs = (int64_t)a.Hkv * D;  // pool elements from one key row to the next
  // the K / V sources as locals (a select between two fields of `a` would
  // address the argument block in memory)
  const unsigned char* const kpool = reinterpret_cast<const unsigned char*>(a.k_pool);
  const unsigned char* const vpool = reinterpret_cast<const unsigned char*>(a.v_pool);
  const unsigned char* const knew = reinterpret_cast<const unsigned char*>(a.k_new);
  const unsigned char* const vnew = reinterpret_cast<const unsigned char*>(a.v_new);
  const int64_t new_off = (int64_t)trow * a.new_stride + (int64_t)h * D;

  // ---- the rows' queries, scaled, padded with zeros ----
  for (int i = tid; i < R * DP; i += kGThreads) {
    const int r = i / DP, d = i - r * DP;
    const int tok = r / G, g = r - tok * G;
    qs[i] = d < D ? ld_el<E>(a.q, (int64_t)(t0 + tok) * a.q_stride + (int64_t)(h * G + g) * D + d) *
                        a.scale_log2
                  : 0.f;
  }
  // ---- the product pass's ownership: NQ quads of 4 dims ----
  const int QPR = DP / 4;  // quads per row
  const int NQ = R * QPR;
  // fewer quads than threads: thread t takes quad t % NQ and key part t / NQ;
  // quad q has cnt(q) = (255 - q) / NQ + 1 parts, part p taking keys p,
  // p + cnt(q), ...
  const bool many = NQ >= kGThreads;
  const int my_q = many ? tid : tid % NQ;
  const int part = many ? 0 : tid / NQ;
  const int my_cnt = many ? 1 : (kGThreads - 1 - my_q) / NQ + 1;
  f32x4 acc[kGMaxQuads];
#pragma unroll
  for (int i = 0; i < kGMaxQuads; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r = tid; r < R; r += kGThreads) {
    ml[2 * r] = kNegInf;
    ml[2 * r + 1] = 0.f;
  }
  __syncthreads();

  // 16-byte vectors: TPK threads per key row, thread tid moving vectors
  // tid % TPK + TPK u of key tid / TPK (one table lookup and one address per
  // thread); the next chunk's are loaded into registers while the current one
  // is scored
  constexpr int TPK = kGThreads / CK;
  const int vpr = D / VW;
  const int my_kj = tid / TPK;
  const int my_v0 = tid % TPK;
  f32x4 kr[kGPre], vr[kGPre];
  auto fetch = [&](int c0) __attribute__((always_inline)) {
    const int k = c0 + my_kj;
    if (k < k_hi) {
      const bool nw = k == new_key;
      const int blk = clamp_block(a.tables[(int64_t)trow * a.W + (k >> a.bs_log2)], a.NB);
      const int64_t off =
          ((nw ? new_off : ((int64_t)blk * a.BS + (k & (a.BS - 1))) * rs + (int64_t)h * D) +
           (int64_t)my_v0 * VW) * EB;
      const unsigned char* const kb = (nw ? knew : kpool) + off;
      const unsigned char* const vb = (nw ? vnew : vpool) + off;
#pragma unroll
      for (int u = 0; u < kGPre; ++u) {
        if (my_v0 + TPK * u < vpr) {
          kr[u] = *reinterpret_cast<const f32x4*>(kb + TPK * 16 * u);
          vr[u] = *reinterpret_cast<const f32x4*>(vb + TPK * 16 * u);
        }
      }
    }
  };
  if (a.vec && k_lo < k_hi) fetch(k_lo);

  for (int c0 = k_lo; c0 < k_hi; c0 += CK) {
    const int nk = min(CK, k_hi - c0);
    // ---- stage the chunk's K and V rows ----
    if (a.vec) {
      if (my_kj < nk) {
        unsigned char* const kd = ks + my_kj * L.kst + my_v0 * 16;
        unsigned char* const vd = vs + (my_kj * DP + my_v0 * VW) * EB;
#pragma unroll
        for (int u = 0; u < kGPre; ++u) {
          if (my_v0 + TPK * u < vpr) {
            *reinterpret_cast<f32x4*>(kd + TPK * 16 * u) = kr[u];
            *reinterpret_cast<f32x4*>(vd + TPK * 16 * u) = vr[u];
          }
        }
      }
      if (DP > D) {  // fp32 rows of 8k + 4 dims: zero the last 4 of the padding
        for (int kj = tid; kj < nk; kj += kGThreads) {
          *reinterpret_cast<f32x4*>(ks + kj * L.kst + D * EB) = f32x4{0.f, 0.f, 0.f, 0.f};
          *reinterpret_cast<f32x4*>(vs + (kj * DP + D) * EB) = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    } else {
      for (int i = tid; i < nk * DP; i += kGThreads) {
        const int kj = i / DP, d = i - kj * DP;
        const int k = c0 + kj;
        const bool nw = k == new_key;
        const int blk = clamp_block(a.tables[(int64_t)trow * a.W + (k >> a.bs_log2)], a.NB);
        const unsigned char* const kb = nw ? knew : kpool;
        const unsigned char* const vb = nw ? vnew : vpool;
        const int64_t off =
            nw ? new_off : ((int64_t)blk * a.BS + (k & (a.BS - 1))) * rs + (int64_t)h * D;
        unsigned char* kd = ks + kj * L.kst + d * EB;
        unsigned char* vd = vs + (kj * DP + d) * EB;
        if constexpr (kIsF32<E>) {
          *reinterpret_cast<float*>(kd) = d < D ? reinterpret_cast<const float*>(kb)[off + d] : 0.f;
          *reinterpret_cast<float*>(vd) = d < D ? reinterpret_cast<const float*>(vb)[off + d] : 0.f;
        } else {
          *reinterpret_cast<uint16_t*>(kd) =
              d < D ? reinterpret_cast<const uint16_t*>(kb)[off + d] : (uint16_t)0;
          *reinterpret_cast<uint16_t*>(vd) =
              d < D ? reinterpret_cast<const uint16_t*>(vb)[off + d] : (uint16_t)0;
        }
      }
    }
    __syncthreads();
    if (a.vec && c0 + CK < k_hi) fetch(c0 + CK);

    // ---- scores and the online softmax: lane = key j, rows of this segment,
    //      kGRowStep at a time; a row's running (max, sum) lives in LDS, read by
    //      the segment's lanes and written back by its lane 0 ----
    {
      const unsigned char* krow = ks + j * L.kst;
      for (int i0 = 0; i0 < nslots; i0 += kGRowStep) {  // wave-uniform
        // the step's rows (a row past R reads row 0 and is discarded): no
        // branches in the dot products, so a step's LDS reads issue together
        const float* qrow[kGRowStep];
#pragma unroll
        for (int u = 0; u < kGRowStep; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          qrow[u] = qs + (i0 + u < nslots && r < R ? r : 0) * DP;
        }
        float s[kGRowStep];
#pragma unroll
        for (int u = 0; u < kGRowStep; ++u) s[u] = 0.f;
#pragma unroll 1
        for (int d = 0; d < DP; d += 8) {
          float kx[8];
          lds8<E>(krow + d * EB, kx);
#pragma unroll
          for (int u = 0; u < kGRowStep; ++u) {
            const f32x4 qa = *reinterpret_cast<const f32x4*>(qrow[u] + d);
            const f32x4 qb = *reinterpret_cast<const f32x4*>(qrow[u] + d + 4);
            float t = s[u];
            t += qa[0] * kx[0];
            t += qa[1] * kx[1];
            t += qa[2] * kx[2];
            t += qa[3] * kx[3];
            t += qb[0] * kx[4];
            t += qb[1] * kx[5];
            t += qb[2] * kx[6];
            t += qb[3] * kx[7];
            s[u] = t;
          }
        }
        // the online softmax of the step's rows, their reductions interleaved;
        // every lane joins them, and rows past R (slots past nslots among them)
        // have nothing valid and write nothing
        float mo[kGRowStep], mn[kGRowStep], lo[kGRowStep], pv[kGRowStep];
#pragma unroll
        for (int u = 0; u < kGRowStep; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          const bool valid = r < R && j < nk && c0 + j < lim0 + r / G;
          const int rr = r < R ? r : 0;
          mo[u] = ml[2 * rr];
          lo[u] = ml[2 * rr + 1];
          s[u] = valid ? s[u] : kNegInf;
          mn[u] = s[u];
        }
#pragma unroll
        for (int m = CK / 2; m >= 1; m >>= 1) {
#pragma unroll
          for (int u = 0; u < kGRowStep; ++u) mn[u] = fmaxf(mn[u], shfl_xor_f(mn[u], m));
        }
#pragma unroll
        for (int u = 0; u < kGRowStep; ++u) {
          mn[u] = fmaxf(mo[u], mn[u]);
          pv[u] = s[u] == kNegInf ? 0.f : exp2f(s[u] - mn[u]);
          s[u] = pv[u];
        }
#pragma unroll
        for (int m = CK / 2; m >= 1; m >>= 1) {
#pragma unroll
          for (int u = 0; u < kGRowStep; ++u) s[u] += shfl_xor_f(s[u], m);
        }
#pragma unroll
        for (int u = 0; u < kGRowStep; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          const float alpha = mo[u] == kNegInf ? 0.f : exp2f(mo[u] - mn[u]);
          if (r < R) {
            ps[r * CK + j] = pv[u];
            if (j == 0) {
              al[r] = alpha;
              ml[2 * r] = mn[u];
              ml[2 * r + 1] = lo[u] * alpha + s[u];
            }
          }
        }
      }
    }
    lds_barrier();

    // ---- products: quads (row r, dims 4x .. 4x + 3) ----
    if (many) {
      // up to four quads per thread (tid + 256 i), every key; the quads' chains
      // are interleaved key by key
      const float* pr[kGMaxQuads];
      const unsigned char* vc[kGMaxQuads];
#pragma unroll
      for (int i = 0; i < kGMaxQuads; ++i) {
        const int qd = tid + kGThreads * i;
        const int qc = qd < NQ ? qd : 0;  // past NQ: quad 0 again, discarded
        const int r = qc / QPR, x = qc - r * QPR;
        acc[i] *= al[r];
        pr[i] = ps + r * CK;
        vc[i] = vs + x * 4 * EB;
      }
#pragma unroll 2
      for (int kj = 0; kj < nk; ++kj) {
#pragma unroll
        for (int i = 0; i < kGMaxQuads; ++i)
          acc[i] += pr[i][kj] * lds4<E>(vc[i] + kj * DP * EB);
      }
    } else {
      // one quad, keys part, part + cnt, ... four per step with their LDS
      // reads issued together
      const int r = my_q / QPR, x = my_q - r * QPR;
      f32x4 o = acc[0] * al[r];
      const float* pr = ps + r * CK;
      const unsigned char* vcol = vs + x * 4 * EB;
      const int vstep = my_cnt * DP * EB;
      f32x4 o1 = f32x4{0.f, 0.f, 0.f, 0.f};
      int kj = part;
      for (; kj + 3 * my_cnt < nk; kj += 4 * my_cnt) {
        const unsigned char* v0 = vcol + kj * DP * EB;
        const float p0 = pr[kj], p1 = pr[kj + my_cnt], p2 = pr[kj + 2 * my_cnt],
                    p3 = pr[kj + 3 * my_cnt];
        const f32x4 w0 = lds4<E>(v0), w1 = lds4<E>(v0 + vstep), w2 = lds4<E>(v0 + 2 * vstep),
                    w3 = lds4<E>(v0 + 3 * vstep);
        o += p0 * w0;
        o1 += p1 * w1;
        o += p2 * w2;
        o1 += p3 * w3;
      }
      for (; kj < nk; kj += my_cnt) o += pr[kj] * lds4<E>(vcol + kj * DP * EB);
      acc[0] = o + o1;
    }
    lds_barrier();
  }

  // ---- the key parts summed ----
  f32x4* const parts = reinterpret_cast<f32x4*>(lds + L.k);  // [part][NQ] when NQ < 256
  if (!many) parts[tid] = acc[0];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kGMaxQuads; ++i) {
    const int qd = many ? tid + kGThreads * i : (i == 0 ? tid : NQ);
    if (qd < NQ) {
      f32x4 o = acc[i];
      if (!many) {
        o = parts[qd];
        const int cnt = (kGThreads - 1 - qd) / NQ + 1;
        for (int p2 = 1; p2 < cnt; ++p2) o += parts[p2 * NQ + qd];
      }
      const int r = qd / QPR, x = qd - r * QPR;
      const int tok = r / G, g = r - tok * G;
      const float mr = ml[2 * r], lr = ml[2 * r + 1];
      const float inv = lr > 0.f ? 1.f / lr : 0.f;
      const int hq = h * G + g;
      if (a.splits > 1) {
        const int64_t slot = ((int64_t)(t0 + tok) * a.Hq + hq) * a.splits + split;
        float* po = a.part_o + slot * D;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * x + e < D) po[4 * x + e] = o[e] * inv;
        if (x == 0) a.part_lse[slot] = lr > 0.f ? mr + log2f(lr) : kNegInf;
      } else {
        const int64_t orow = (int64_t)(t0 + tok) * a.out_stride + (int64_t)hq * D;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * x + e < D)
            store_out1<E>(reinterpret_cast<f16*>(a.out), orow + 4 * x + e, o[e] * inv);
      }
    }
  }
  __syncthreads();  // the next segment reuses the LDS
}

template <class E, int CK>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(GEN_WAVES, GEN_WAVES)))
void generic_attn_kernel(const GArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int max_len = a.W * a.BS;
  if (a.q_off == nullptr) {
    // ---- decode: item = (row b, KV head h, split s) ----
    const int s = blockIdx.x % a.splits;
    const int bh = blockIdx.x / a.splits;
    const int h = bh % a.Hkv, b = bh / a.Hkv;
    const int L = min(clamp_len(a.ctx[b]), max_len);
    const int per = (L + a.splits - 1) / a.splits;
    const int span = (per + CK - 1) / CK * CK;
    const int k_lo = min(s * span, L), k_hi = min(k_lo + span, L);
    const int new_key = a.k_new != nullptr && L > 0 ? L - 1 : -1;
    if (new_key >= k_lo && new_key < k_hi) {
      // the page write, by the split that holds the new key
      const int blk = clamp_block(a.tables[(int64_t)b * a.W + (new_key >> a.bs_log2)], a.NB);
      const int64_t dst =
          ((int64_t)blk * a.BS + (new_key & (a.BS - 1))) * a.Hkv * a.D + (int64_t)h * a.D;
      const int64_t src = (int64_t)b * a.new_stride + (int64_t)h * a.D;
      for (int d = threadIdx.x; d < a.D; d += kGThreads) {
        if constexpr (kIsF32<E>) {
          reinterpret_cast<uint32_t*>(a.k_pool)[dst + d] =
              reinterpret_cast<const uint32_t*>(a.k_new)[src + d];
          reinterpret_cast<uint32_t*>(a.v_pool)[dst + d] =
              reinterpret_cast<const uint32_t*>(a.v_new)[src + d];
        } else {
          reinterpret_cast<uint16_t*>(a.k_pool)[dst + d] =
              reinterpret_cast<const uint16_t*>(a.k_new)[src + d];
          reinterpret_cast<uint16_t*>(a.v_pool)[dst + d] =
              reinterpret_cast<const uint16_t*>(a.v_new)[src + d];
        }
      }
    }
    generic_segment<E, CK>(a, lds, h, b, b, 1, L, k_lo, k_hi, new_key, s);
    return;
  }
  // ---- prefill: item = (tile of TQ flattened tokens, KV head h); the tile's
  //      tokens are walked sequence by sequence ----
  const int h = blockIdx.x % a.Hkv;
  const int tile = blockIdx.x / a.Hkv;
  const int t_end = min((tile + 1) * a.TQ, a.total);
  for (int t0 = tile * a.TQ; t0 < t_end;) {
    int lo = 0, hi = a.S;  // the last sequence s with q_off[s] <= t0
    while (hi - lo > 1) {
      const int mid = (lo + hi) / 2;
      if (a.q_off[mid] <= t0) lo = mid; else hi = mid;
    }
    const int q0 = a.q_off[lo], q1 = a.q_off[lo + 1];
    if (t0 < q0 || t0 >= q1) {
      // tokens outside every chunk: zeros
      const int GD = a.G * a.D;
      for (int i = threadIdx.x; i < (t_end - t0) * GD; i += kGThreads) {
        const int tok = i / GD, e = i - tok * GD;
        store_out1<E>(reinterpret_cast<f16*>(a.out),
                      (int64_t)(t0 + tok) * a.out_stride + (int64_t)h * GD + e, 0.f);
      }
      break;
    }
    const int seg_end = min(t_end, q1);
    const int ctx = clamp_len(a.ctx[lo]);
    const int n = q1 - q0;
    const int cached = ctx >= n ? ctx - n : 0;
    const int lim0 = cached + (t0 - q0) + 1;
    const int k_hi = min(lim0 + (seg_end - t0) - 1, max_len);
    generic_segment<E, CK>(a, lds, h, lo, t0, seg_end - t0, lim0, 0, k_hi, -1, 0);
    t0 = seg_end;
  }
}

// Decode splits folded: row r = (b, query head), its splits' normalised
// outputs weighted by 2^(lse_s - max).
template <class E>
__global__ __launch_bounds__(kWave) void generic_merge_kernel(const GArgs a) {
  const int r = blockIdx.x;  // b * Hq + hq
  const int S = a.splits;
  const float* lse = a.part_lse + (int64_t)r * S;
  float M = kNegInf;
  for (int s = 0; s < S; ++s) M = fmaxf(M, lse[s]);
  float wgt[kGMaxSplits];
  float den = 0.f;
#pragma unroll
  for (int s = 0; s < kGMaxSplits; ++s) {
    const float ls = lse[s < S ? s : 0];
    wgt[s] = s < S && ls != kNegInf ? exp2f(ls - M) : 0.f;
    den += wgt[s];
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const int b = r / a.Hq, hq = r - b * a.Hq;
  const float* po = a.part_o + (int64_t)r * S * a.D;
  for (int d = threadIdx.x; d < a.D; d += kWave) {
    float num = 0.f;
#pragma unroll
    for (int s = 0; s < kGMaxSplits; ++s)
      if (wgt[s] > 0.f) num += wgt[s] * po[(int64_t)s * a.D + d];
    store_out1<E>(reinterpret_cast<f16*>(a.out), (int64_t)b * a.out_stride + (int64_t)hq * a.D + d,
                  num * inv);
  }
}

template <class E, int CK>
int launch_ck(const GArgs& a, hipStream_t stream) {
  const GLds L = glds<E, CK>(a.TQ * a.G, a.DP);
  const int64_t items = a.q_off == nullptr
                            ? (int64_t)a.total * a.Hkv * a.splits
                            : (int64_t)((a.total + a.TQ - 1) / a.TQ) * a.Hkv;
  if (items >= ((int64_t)1 << 31)) return FE_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((generic_attn_kernel<E, CK>), dim3((unsigned)items), dim3(kGThreads),
                     (size_t)L.bytes, stream, a);
  if (a.q_off == nullptr && a.splits > 1)
    hipLaunchKernelGGL((generic_merge_kernel<E>), dim3((unsigned)((int64_t)a.total * a.Hq)),
                       dim3(kWave), 0, stream, a);
  return FE_LAUNCH_STATUS();
}

// Keys per chunk: about 34 KB of K and V staging at most
template <class E>
int launch_e(const GArgs& a, hipStream_t stream) {
  const int row_bytes = a.DP * kElemBytes<E>;
  if (row_bytes <= 256) return launch_ck<E, 64>(a, stream);
  if (row_bytes <= 512) return launch_ck<E, 32>(a, stream);
  if (row_bytes <= 1024) return launch_ck<E, 16>(a, stream);
  return launch_ck<E, 8>(a, stream);
}

}  // namespace

namespace fe {

int generic_padded_dims(int d) { return (d + 7) / 8 * 8; }

bool generic_shape(int hq, int hkv, int d) {
  if (hkv <= 0 || hq % hkv != 0 || d <= 0 || d > kGenericMaxHeadDim) return false;
  const int G = hq / hkv;
  return G <= kGenericMaxGroup && (int64_t)G * generic_padded_dims(d) <= kGenericMaxElems;
}

int generic_attention(const GenericAttn& g, hipStream_t stream) {
  if (!generic_shape(g.hq, g.hkv, g.d)) return FE_ERR_UNSUPPORTED;
  if (g.rows == 0) return FE_OK;
  GArgs a{};
  a.q = g.q;
  a.q_stride = g.q_stride;
  a.out = g.out;
  a.out_stride = g.out_stride;
  a.k_new = g.k_new;
  a.v_new = g.v_new;
  a.new_stride = g.new_stride;
  a.k_pool = g.k_pool;
  a.v_pool = g.v_pool;
  a.tables = g.tables;
  a.W = g.table_stride;
  a.ctx = g.ctx;
  a.q_off = g.q_offsets;
  a.S = g.num_seqs;
  a.total = g.rows;
  a.Hq = g.hq;
  a.Hkv = g.hkv;
  a.G = g.hq / g.hkv;
  a.D = g.d;
  a.DP = generic_padded_dims(g.d);
  a.BS = g.bs;
  a.bs_log2 = 0;
  while ((1 << a.bs_log2) < g.bs) ++a.bs_log2;
  a.NB = g.num_blocks;
  a.scale_log2 = g.scale * kLog2e;
  // prefill tiles: rows (tokens x group) <= 64 and rows x padded dims <= 4096
  a.TQ = 1;
  if (g.q_offsets != nullptr) {
    int tq = kGMaxRows / a.G;
    const int by_elems = kGenericMaxElems / (a.G * a.DP);
    if (by_elems < tq) tq = by_elems;
    a.TQ = tq < 1 ? 1 : (tq > 16 ? 16 : tq);
  }
  a.splits = g.q_offsets == nullptr && g.splits > 1 ? g.splits : 1;
  if (a.splits > kGMaxSplits) return FE_ERR_UNSUPPORTED;
  if (a.splits > 1 && (g.part_o == nullptr || g.part_lse == nullptr)) return FE_ERR_WORKSPACE;
  a.part_o = g.part_o;
  a.part_lse = g.part_lse;
  // 16-byte loads: rows a whole number of vectors apart, 16-byte aligned bases
  const int vw = g.elem == 2 ? 4 : 8;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  a.vec = g.d % vw == 0 && al16(g.k_pool) && al16(g.v_pool) &&
          (g.k_new == nullptr || (al16(g.k_new) && al16(g.v_new) && g.new_stride % vw == 0));
  if (g.elem == 2) return launch_e<F32>(a, stream);
  if (g.elem == 1) return launch_e<Bf16>(a, stream);
  return launch_e<Fp16>(a, stream);
}

}  // namespace fe
