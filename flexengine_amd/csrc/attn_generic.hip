// Attention for the shapes the matrix-core kernels do not take: head_dim other
// than 64 and 128 (1 .. 512), and decode groups of 17 .. 128 query heads per KV
// head (group x head_dim <= 8192).  The reference's Triton decode takes any head_dim (BLOCK_D =
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

#include <type_traits>

#include "attn_core.h"
#include "flexengine_amd.h"

using namespace fe;

namespace {

#ifndef GEN_WAVES
#define GEN_WAVES 3
#endif
constexpr int kGThreads = 256;
constexpr int kGWaves = kGThreads / kWave;
constexpr int kGMaxRows = 64;     // query rows of a prefill tile (tokens x group; one token at least)
constexpr int kGRowStep = 4;      // rows scored per pass over a key's row
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

// sum_i a[i] * b[i] + c over 8 16-bit elements, four fp32 dot products of pairs
// (v_dot2_f32_f16 / v_dot2_f32_bf16)
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
template <class E>
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float c) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2_t x = h2_t{a[2 * i], a[2 * i + 1]};
    const h2_t y = h2_t{b[2 * i], b[2 * i + 1]};
    if constexpr (__is_same(E, Bf16))
      c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, x), __builtin_bit_cast(b2_t, y), c,
                                          false);
    else
      c = __builtin_amdgcn_fdot2(x, y, c, false);
  }
  return c;
}

// c + a.x * b.x + a.y * b.y for a pair of 16-bit elements in one dword each
template <class E>
__device__ __forceinline__ float dot2w(uint32_t a, uint32_t b, float c) {
  if constexpr (__is_same(E, Bf16))
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, a), __builtin_bit_cast(b2_t, b), c,
                                           false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

// o + p * V over one unit of the product pass, for 4 consecutive dims at
// vcol: fp32, key m (p an fp32, V rows of DP floats); 16-bit, keys 2m and
// 2m + 1 (p a pair of E, V pair rows of 2 DP elements, dim-major within a
// pair, so a dword holds both keys' element of one dim)
template <class E>
__device__ __forceinline__ f32x4 pv_unit(const unsigned char* prow, const unsigned char* vcol,
                                         int m, int DP, f32x4 o) {
  if constexpr (kIsF32<E>) {
    const float p = reinterpret_cast<const float*>(prow)[m];
    return o + p * *reinterpret_cast<const f32x4*>(vcol + m * DP * 4);
  } else {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const uint32_t pp = reinterpret_cast<const uint32_t*>(prow)[m];
    const u32x4 v = *reinterpret_cast<const u32x4*>(vcol + m * DP * 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = dot2w<E>(pp, v[e], o[e]);
    return o;
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

// v[u] combined (op) over the CK lanes of this lane's segment, for RS values
// at once, every lane of the segment getting the result: DPP row operations
// within 16 lanes (quad swaps, then the 8- and 16-lane mirrors), across the
// four rows of the wave with readlane (CK = 64), or xor shuffles (CK = 32).
template <int CK, int RS, class Op>
__device__ __forceinline__ void seg_reduce(float (&v)[RS], Op op) {
  auto dppf = [](auto ctrl, float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value,
                                           0xF, 0xF, false));
  };
  if constexpr (CK == 32) {
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
#pragma unroll
      for (int u = 0; u < RS; ++u) v[u] = op(v[u], shfl_xor_f(v[u], m));
    }
  } else {
#pragma unroll
    for (int u = 0; u < RS; ++u)
      v[u] = op(v[u], dppf(std::integral_constant<int, dpp::kQuadXor1>{}, v[u]));
#pragma unroll
    for (int u = 0; u < RS; ++u)
      v[u] = op(v[u], dppf(std::integral_constant<int, dpp::kQuadXor2>{}, v[u]));
#pragma unroll
    for (int u = 0; u < RS; ++u)
      v[u] = op(v[u], dppf(std::integral_constant<int, dpp::kRowHalfMirror>{}, v[u]));
    if constexpr (CK >= 16) {
#pragma unroll
      for (int u = 0; u < RS; ++u)
        v[u] = op(v[u], dppf(std::integral_constant<int, dpp::kRowMirror>{}, v[u]));
    }
    if constexpr (CK == 64) {
      auto rl = [](float x, int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
      };
#pragma unroll
      for (int u = 0; u < RS; ++u)
        v[u] = op(op(rl(v[u], 0), rl(v[u], 16)), op(rl(v[u], 32), rl(v[u], 48)));
    }
  }
}

// LDS layout of one workgroup (byte offsets), from the item's most rows R and
// padded dims DP: q [R][DP] fp32 (16-bit types: their own type) | K [CK][DP
// elements + 16 bytes] | V [CK][DP] (16-bit types: by key pairs) | p [R][CK]
// fp32 (16-bit types: their own type) | rescale [R] | (max, sum) [R][2] |
// the product pass's accumulators.
struct GLds {
  int q, k, v, p, al, ml, acc, bytes, kst;
};
template <class E, int CK>
__host__ __device__ inline GLds glds(int R, int DP) {
  GLds l;
  l.kst = DP * kElemBytes<E> + 16;
  l.q = 0;
  l.k = R * DP * 4;
  l.v = l.k + CK * l.kst;
  l.p = l.v + CK * DP * kElemBytes<E>;
  l.al = l.p + R * CK * 4;
  l.ml = l.al + R * 4;
  l.acc = (l.ml + R * 8 + 15) & ~15;
  // the product pass's accumulators: a quad's (or a quad part's) f32x4 each,
  // max(256, R * DP / 4) of them
  const int nacc = R * DP / 4 > kGThreads ? R * DP / 4 : kGThreads;
  l.bytes = l.acc + nacc * 16;
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
  f16* const ps16 = reinterpret_cast<f16*>(lds + L.p);  // 16-bit types: p in E
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

  // 16-byte vectors: TPP threads per key pair (keys 2m, 2m + 1 of the chunk),
  // thread tid moving vectors tid % TPP + TPP u of both keys of pair tid / TPP
  // (one address per key; a pair shares its block unless the block size is
  // 1), so the 16-bit V pairs interleave in registers; the next chunk's are
  // loaded into registers while the current one is scored
  constexpr int TPP = 2 * kGThreads / CK;
  constexpr int UP = kGPre / 2;  // vectors of each key per thread
  const int vpr = D / VW;
  const int my_pm = tid / TPP;
  const int my_v0 = tid % TPP;
  f32x4 kr[2][UP], vr[2][UP];
  // the block ids of this thread's keys in the next chunk to fetch, loaded one
  // fetch ahead (a fetch is then one round trip, not a table lookup and a load)
  const int32_t* const trow_ids = a.tables + (int64_t)trow * a.W;
  auto block_of = [&](int k) __attribute__((always_inline)) {
    return k < k_hi ? trow_ids[k >> a.bs_log2] : 0;
  };
  int blk_next[2] = {0, 0};
  auto next_ids = [&](int c0) __attribute__((always_inline)) {
    blk_next[0] = block_of(c0 + 2 * my_pm);
    blk_next[1] = a.bs_log2 == 0 ? block_of(c0 + 2 * my_pm + 1) : blk_next[0];
  };
  auto fetch = [&](int c0) __attribute__((always_inline)) {
    const int blk[2] = {clamp_block(blk_next[0], a.NB), clamp_block(blk_next[1], a.NB)};
    next_ids(c0 + CK);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int k = c0 + 2 * my_pm + e;
#pragma unroll
      for (int u = 0; u < UP; ++u) vr[e][u] = f32x4{0.f, 0.f, 0.f, 0.f};  // keys past the range
      if (k < k_hi) {
        const bool nw = k == new_key;
        const int64_t off =
            ((nw ? new_off : ((int64_t)blk[e] * a.BS + (k & (a.BS - 1))) * rs + (int64_t)h * D) +
             (int64_t)my_v0 * VW) * EB;
        const unsigned char* const kb = (nw ? knew : kpool) + off;
        const unsigned char* const vb = (nw ? vnew : vpool) + off;
#pragma unroll
        for (int u = 0; u < UP; ++u) {
          if (my_v0 + TPP * u < vpr) {
            kr[e][u] = *reinterpret_cast<const f32x4*>(kb + TPP * 16 * u);
            vr[e][u] = *reinterpret_cast<const f32x4*>(vb + TPP * 16 * u);
          }
        }
      }
    }
  };
  // the first chunk's loads go out before the queries'
  if (a.vec && k_lo < k_hi) {
    next_ids(k_lo);
    fetch(k_lo);
  }

  // ---- the rows' queries, padded with zeros: fp32 scaled to base 2, or the
  //      16-bit values as they are (their scores are scaled instead) ----
  uint16_t* const qs16 = reinterpret_cast<uint16_t*>(lds + L.q);
  for (int i = tid; i < R * DP; i += kGThreads) {
    const int r = i / DP, d = i - r * DP;
    const int tok = r / G, g = r - tok * G;
    const int64_t qi = (int64_t)(t0 + tok) * a.q_stride + (int64_t)(h * G + g) * D + d;
    if constexpr (kIsF32<E>)
      qs[i] = d < D ? reinterpret_cast<const float*>(a.q)[qi] * a.scale_log2 : 0.f;
    else
      qs16[i] = d < D ? reinterpret_cast<const uint16_t*>(a.q)[qi] : (uint16_t)0;
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
  // accumulators in LDS: quad tid + 256 i (NQ >= 256), or quad my_q's part
  // `part` at tid (= part * NQ + my_q)
  f32x4* const accl = reinterpret_cast<f32x4*>(lds + L.acc);
  const int nacc = many ? NQ : kGThreads;
  for (int i = tid; i < nacc; i += kGThreads) accl[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r = tid; r < R; r += kGThreads) {
    ml[2 * r] = kNegInf;
    ml[2 * r + 1] = 0.f;
  }
  __syncthreads();

  for (int c0 = k_lo; c0 < k_hi; c0 += CK) {
    const int nk = min(CK, k_hi - c0);
    // ---- stage the chunk's K and V rows ----
    if (a.vec) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int kj = 2 * my_pm + e;
        if (kj < nk) {
          unsigned char* const kd = ks + kj * L.kst + my_v0 * 16;
#pragma unroll
          for (int u = 0; u < UP; ++u)
            if (my_v0 + TPP * u < vpr) *reinterpret_cast<f32x4*>(kd + TPP * 16 * u) = kr[e][u];
          if constexpr (kIsF32<E>) {
            unsigned char* const vd = vs + (kj * DP + my_v0 * VW) * EB;
#pragma unroll
            for (int u = 0; u < UP; ++u)
              if (my_v0 + TPP * u < vpr) *reinterpret_cast<f32x4*>(vd + TPP * 16 * u) = vr[e][u];
          }
        }
      }
      if constexpr (!kIsF32<E>) {
        // V by key pairs, dims interleaved (a key past the range is zeros)
        if (2 * my_pm < nk) {
          unsigned char* const vd = vs + my_pm * 4 * DP + my_v0 * 32;
#pragma unroll
          for (int u = 0; u < UP; ++u) {
            if (my_v0 + TPP * u < vpr) {
              const f16x8 a0 = __builtin_bit_cast(f16x8, vr[0][u]);
              const f16x8 b0 = __builtin_bit_cast(f16x8, vr[1][u]);
              *reinterpret_cast<f16x8*>(vd + TPP * 32 * u) =
                  __builtin_shufflevector(a0, b0, 0, 8, 1, 9, 2, 10, 3, 11);
              *reinterpret_cast<f16x8*>(vd + TPP * 32 * u + 16) =
                  __builtin_shufflevector(a0, b0, 4, 12, 5, 13, 6, 14, 7, 15);
            }
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
      // (16-bit: keys up to the next even count, the odd tail's partner zero)
      const int nkv = kIsF32<E> ? nk : (nk + 1) & ~1;
      for (int i = tid; i < nkv * DP; i += kGThreads) {
        const int kj = i / DP, d = i - kj * DP;
        // the odd tail's partner (kj == nk) is zeros: its table entry may lie past
        // the row, so it looks up the chunk's first key instead
        const int k = c0 + (kj < nk ? kj : 0);
        const bool nw = k == new_key;
        const int blk = clamp_block(a.tables[(int64_t)trow * a.W + (k >> a.bs_log2)], a.NB);
        const unsigned char* const kb = nw ? knew : kpool;
        const unsigned char* const vb = nw ? vnew : vpool;
        const int64_t off =
            nw ? new_off : ((int64_t)blk * a.BS + (k & (a.BS - 1))) * rs + (int64_t)h * D;
        const bool in = d < D && kj < nk;
        unsigned char* kd = ks + kj * L.kst + d * EB;
        if constexpr (kIsF32<E>) {
          unsigned char* vd = vs + (kj * DP + d) * EB;
          *reinterpret_cast<float*>(kd) = in ? reinterpret_cast<const float*>(kb)[off + d] : 0.f;
          *reinterpret_cast<float*>(vd) = in ? reinterpret_cast<const float*>(vb)[off + d] : 0.f;
        } else {
          unsigned char* vd = vs + (kj >> 1) * 4 * DP + d * 4 + (kj & 1) * 2;
          *reinterpret_cast<uint16_t*>(kd) =
              in ? reinterpret_cast<const uint16_t*>(kb)[off + d] : (uint16_t)0;
          *reinterpret_cast<uint16_t*>(vd) =
              in ? reinterpret_cast<const uint16_t*>(vb)[off + d] : (uint16_t)0;
        }
      }
    }
    __syncthreads();
    if (a.vec && c0 + CK < k_hi) fetch(c0 + CK);

    // ---- scores and the online softmax: lane = key j, rows of this segment,
    //      RS at a time (RS = 1 or 2 when the wave holds only that many); a
    //      row's running (max, sum) lives in LDS, read by the segment's lanes
    //      and written back by its lane 0 ----
    {
      const unsigned char* krow = ks + j * L.kst;
      auto rows_step = [&](auto rs_c, int i0) __attribute__((always_inline)) {
        constexpr int RS = decltype(rs_c)::value;
        // the step's rows (a row past R reads row 0 and is discarded): no
        // branches in the dot products, so a step's LDS reads issue together
        int qoff[RS];
#pragma unroll
        for (int u = 0; u < RS; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          qoff[u] = (r < R ? r : 0) * DP;
        }
        float s[RS];
#pragma unroll
        for (int u = 0; u < RS; ++u) s[u] = 0.f;
        for (int d = 0; d < DP; d += 8) {
          if constexpr (kIsF32<E>) {
            float kx[8];
            lds8<E>(krow + d * EB, kx);
#pragma unroll
            for (int u = 0; u < RS; ++u) {
              const f32x4 qa = *reinterpret_cast<const f32x4*>(qs + qoff[u] + d);
              const f32x4 qb = *reinterpret_cast<const f32x4*>(qs + qoff[u] + d + 4);
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
          } else {
            // 16-bit q and K as they are: fp32 dot products of element pairs
            const f16x8 kv = *reinterpret_cast<const f16x8*>(krow + d * 2);
#pragma unroll
            for (int u = 0; u < RS; ++u) {
              const f16x8 qv = *reinterpret_cast<const f16x8*>(qs16 + qoff[u] + d);
              s[u] = dot8<E>(qv, kv, s[u]);
            }
          }
        }
        // the online softmax of the step's rows, their reductions interleaved;
        // every lane joins them, and rows past R have nothing valid and write
        // nothing
        float mo[RS], mn[RS], lo[RS], pv[RS];
#pragma unroll
        for (int u = 0; u < RS; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          const bool valid = r < R && j < nk && c0 + j < lim0 + r / G;
          const int rr = r < R ? r : 0;
          mo[u] = ml[2 * rr];
          lo[u] = ml[2 * rr + 1];
          s[u] = valid ? (kIsF32<E> ? s[u] : s[u] * a.scale_log2) : kNegInf;
          mn[u] = s[u];
        }
        seg_reduce<CK, RS>(mn, [](float x, float y) { return fmaxf(x, y); });
#pragma unroll
        for (int u = 0; u < RS; ++u) {
          mn[u] = fmaxf(mo[u], mn[u]);
          pv[u] = s[u] == kNegInf ? 0.f : exp2f(s[u] - mn[u]);
          s[u] = pv[u];
        }
        seg_reduce<CK, RS>(s, [](float x, float y) { return x + y; });
#pragma unroll
        for (int u = 0; u < RS; ++u) {
          const int r = w + kGWaves * (seg + NSEG * (i0 + u));
          const float alpha = mo[u] == kNegInf ? 0.f : exp2f(mo[u] - mn[u]);
          if (r < R) {
            if constexpr (kIsF32<E>)
              ps[r * CK + j] = pv[u];
            else
              ps16[r * CK + j] = to16<E>(pv[u]);
            if (j == 0) {
              al[r] = alpha;
              ml[2 * r] = mn[u];
              ml[2 * r + 1] = lo[u] * alpha + s[u];
            }
          }
        }
      };
      if (nslots == 1) {  // wave-uniform
        rows_step(std::integral_constant<int, 1>{}, 0);
      } else if (nslots == 2) {
        rows_step(std::integral_constant<int, 2>{}, 0);
      } else {
        for (int i0 = 0; i0 < nslots; i0 += kGRowStep)
          rows_step(std::integral_constant<int, kGRowStep>{}, i0);
      }
    }
    lds_barrier();

    // ---- products: quads (row r, dims 4x .. 4x + 3) over the chunk's units
    //      (fp32: keys; 16-bit: key pairs) ----
    const int nu = kIsF32<E> ? nk : (nk + 1) >> 1;
    const unsigned char* const pbase = lds + L.p;
    constexpr int PRB = kIsF32<E> ? 4 * CK : 2 * CK;  // bytes of a row's probabilities
    // quads tid, tid + 256, ... (NQ >= 256: every unit), or quad my_q's units
    // part, part + cnt, ...; four units per step with their LDS reads issued
    // together
    for (int idx = tid; idx < nacc; idx += kGThreads) {
      const int qd = many ? idx : my_q;
      const int m0 = many ? 0 : part;
      const int cnt = many ? 1 : my_cnt;
      const int r = qd / QPR, x = qd - r * QPR;
      f32x4 o = accl[idx] * al[r];
      f32x4 o1 = f32x4{0.f, 0.f, 0.f, 0.f};
      const unsigned char* const pr = pbase + r * PRB;
      const unsigned char* const vcol = vs + x * 16;
      int m = m0;
      for (; m + 3 * cnt < nu; m += 4 * cnt) {
        o = pv_unit<E>(pr, vcol, m, DP, o);
        o1 = pv_unit<E>(pr, vcol, m + cnt, DP, o1);
        o = pv_unit<E>(pr, vcol, m + 2 * cnt, DP, o);
        o1 = pv_unit<E>(pr, vcol, m + 3 * cnt, DP, o1);
      }
      for (; m < nu; m += cnt) o = pv_unit<E>(pr, vcol, m, DP, o);
      accl[idx] = o + o1;
    }
    lds_barrier();
  }

  // ---- the key parts summed (the accumulators of part p of quad q at
  //      p * NQ + q) ----
  __syncthreads();
  for (int qd = tid; qd < NQ; qd += kGThreads) {
    {
      f32x4 o = accl[qd];
      if (!many) {
        const int cnt = (kGThreads - 1 - qd) / NQ + 1;
        for (int p2 = 1; p2 < cnt; ++p2) o += accl[p2 * NQ + qd];
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

template <class E, int CK, bool PREFILL>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(GEN_WAVES, GEN_WAVES)))
void generic_attn_kernel(const GArgs a) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int max_len = a.W * a.BS;
  if constexpr (!PREFILL) {
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

// Decode splits folded: one wave per row r = (b, query head), lane s holding
// split s's weight 2^(lse_s - max); each lane then sums dims lane, lane + 64, ...
// over the splits.
constexpr int kGMergeRows = 4;  // rows (waves) per merge workgroup
template <class E>
__global__ __launch_bounds__(kWave * kGMergeRows) void generic_merge_kernel(const GArgs a) {
  const int lane = lane_id();
  const int r = blockIdx.x * kGMergeRows + threadIdx.x / kWave;  // b * Hq + hq
  if (r >= a.total * a.Hq) return;                             // wave-uniform
  const int S = a.splits;
  const float ls = lane < S ? a.part_lse[(int64_t)r * S + lane] : kNegInf;
  float M = ls;
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) M = fmaxf(M, shfl_xor_f(M, m));
  const float wl = ls == kNegInf ? 0.f : exp2f(ls - M);
  float den = wl;
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) den += shfl_xor_f(den, m);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const int b = r / a.Hq, hq = r - b * a.Hq;
  const float* po = a.part_o + (int64_t)r * S * a.D;
  auto wsplit = [&](int s) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), s));
  };
  for (int d = lane; d < a.D; d += kWave) {
    float num = 0.f;
    int s = 0;
    for (; s + 8 <= S; s += 8) {  // eight loads in flight
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = po[(int64_t)(s + i) * a.D + d];
#pragma unroll
      for (int i = 0; i < 8; ++i) num += wsplit(s + i) * v[i];
    }
    for (; s < S; ++s) num += wsplit(s) * po[(int64_t)s * a.D + d];
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
  if (a.q_off == nullptr)
    hipLaunchKernelGGL((generic_attn_kernel<E, CK, false>), dim3((unsigned)items),
                       dim3(kGThreads), (size_t)L.bytes, stream, a);
  else
    hipLaunchKernelGGL((generic_attn_kernel<E, CK, true>), dim3((unsigned)items),
                       dim3(kGThreads), (size_t)L.bytes, stream, a);
  if (a.q_off == nullptr && a.splits > 1) {
    const int64_t rows = (int64_t)a.total * a.Hq;
    hipLaunchKernelGGL((generic_merge_kernel<E>),
                       dim3((unsigned)((rows + kGMergeRows - 1) / kGMergeRows)),
                       dim3(kWave * kGMergeRows), 0, stream, a);
  }
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
