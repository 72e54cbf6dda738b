// Shared device helpers for the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flexengine_amd_model.h"

namespace fe {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---- wave-level helpers (wave64) -------------------------------------------

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ int readlane_i(int v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

// splitmix64's finaliser (S. Vigna, public domain); the host folds the fields a
// step plan is tied to through it, so a planned launch checks its plan with one
// two-word compare (plan_key)
inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
inline uint64_t plan_key(const uint64_t* f, int n) {
  uint64_t h = 0;
  for (int i = 0; i < n; ++i) h = mix64(h ^ f[i]);
  return h;
}

// the two 32-bit halves of an address (plan descriptors record their inputs' addresses)
__device__ __forceinline__ int lo32(const void* p) { return (int)(uint32_t)(uintptr_t)p; }
__device__ __forceinline__ int hi32(const void* p) { return (int)(uint32_t)((uintptr_t)p >> 32); }

// Cross-lane integer reductions and scans on DPP row operations (VALU, a few
// cycles each) instead of LDS-routed shuffles: within each row of 16 lanes,
// then across the four rows with readlane.
namespace dpp {
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141; // lane i <- 7-i within each 8 lanes
constexpr int kRowMirror = 0x140;     // lane i <- 15-i within each row
constexpr int kRowShr = 0x110;        // + n: lane i <- i-n within the row
template <int CTRL>
__device__ __forceinline__ int mov(int v) {
  // bound_ctrl: a source outside the row reads as 0
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
}  // namespace dpp

// Sum over all 64 lanes (wave-uniform result).
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp::mov<dpp::kQuadXor1>(v);
  v += dpp::mov<dpp::kQuadXor2>(v);
  v += dpp::mov<dpp::kRowHalfMirror>(v);
  v += dpp::mov<dpp::kRowMirror>(v);
  return (readlane_i(v, 0) + readlane_i(v, 16)) + (readlane_i(v, 32) + readlane_i(v, 48));
}

// Inclusive prefix sum across the 64 lanes.
__device__ __forceinline__ int wave_scan_incl_i(int v) {
  v += dpp::mov<dpp::kRowShr + 1>(v);
  v += dpp::mov<dpp::kRowShr + 2>(v);
  v += dpp::mov<dpp::kRowShr + 4>(v);
  v += dpp::mov<dpp::kRowShr + 8>(v);
  const int r0 = readlane_i(v, 15);
  const int r1 = r0 + readlane_i(v, 31);
  const int r2 = r1 + readlane_i(v, 47);
  const int lane = lane_id();
  return v + (lane < 16 ? 0 : (lane < 32 ? r0 : (lane < 48 ? r1 : r2)));
}

// ---- 16-byte global accesses ------------------------------------------------

// Cache policies of the K/V page loads (buffer-instruction aux bits).
// kPagePolicy (default caching) for kernels that read whole contexts: one page
// can be read by many rows of a launch (a prefix cache maps a shared prefix into
// every member's block table), and the L2 / Infinity Cache then serve the
// repeats -- at B = 256 with 8 groups of 32 rows sharing 2048 tokens, 110 us per
// decode step vs 162 us with non-temporal loads; read-once batches are
// unaffected (B = 64: 20.8 us either way).
// kStreamPolicy = nt (non-temporal, bit 1) for the cascade's suffix pass, whose
// pages are private to one row and read once: 83 vs 89 us at the same shape.
constexpr int kPagePolicy = 0;
constexpr int kStreamPolicy = 2;

// 2^x with the hardware instruction alone (v_exp_f32, ~1 ulp): exp2f adds a
// range reduction per call so that results below 2^-126 stay denormal instead
// of flushing to zero.  The softmax probabilities need no such values (they
// become fp16 operands, whose smallest subnormal is 2^-24) and the reduction
// cost about 4 VALU instructions per score in the prefill loop.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f16x8 ld16(const f16* p) {
  return *reinterpret_cast<const f16x8*>(p);
}
__device__ __forceinline__ void st16(f16* p, f16x8 v) {
  *reinterpret_cast<f16x8*>(p) = v;
}

// ---- MFMA wrappers ------------------------------------------------------------
// v_mfma_f32_16x16x16_f16.  Operand layout for lane l (g = l/16, n = l%16):
//   A: A[row n][k-slots of group g] (4 halves)   B: B[k-slots of group g][col n]
//   C: C[row 4g+i][col n], i = 0..3
// A and B use the same k-slots for a given (g, register), so any assignment of
// reduction indices to slots is valid as long as both operands follow it.
__device__ __forceinline__ f32x4 mfma16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// ---- 16-bit element types of the attention kernels ----------------------------
// K, V, q and outputs are fp16 (Fp16) or bf16 (Bf16).  Either way they live in
// 16-bit registers as raw bits (the f16x4 / f16x8 storage types): the loads,
// LDS staging, transposing reads and page writes do not look at the values.
// Only the MFMA that consumes them and the conversions from fp32 depend on the
// type.
struct Fp16 {};
struct Bf16 {};
// fp32 pools, q and outputs (the decode's F32Core; products on
// v_mfma_f32_16x16x4_f32, no rounding anywhere but the fp32 arithmetic's own)
struct F32 {};
template <class E>
constexpr bool kIsF32 = __is_same(E, F32);
// v_mfma_f32_16x16x4_f32: lane l (g = l/16, n = l%16) holds A[row n][k = g] and
// B[k = g][col n]; C as for the 16-bit MFMAs (C[row 4g+i][col n]).
__device__ __forceinline__ f32x4 mfma4_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// 16x16x16 MFMA (k = 16) on 16-bit operands of type E
template <class E>
__device__ __forceinline__ f32x4 mma16(f16x4 a, f16x4 b, f32x4 c) {
  if constexpr (__is_same(E, Bf16))
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a),
                                                     __builtin_bit_cast(s16x4_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// 16x16x32 MFMA (k = 32, gfx950) on 16-bit operands of type E
template <class E>
__device__ __forceinline__ f32x4 mma32(f16x8 a, f16x8 b, f32x4 c) {
  if constexpr (__is_same(E, Bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// fp32 -> the 16-bit bits of type E (round to nearest even)
template <class E>
__device__ __forceinline__ f16 to16(float x) {
  if constexpr (__is_same(E, Bf16))
    return __builtin_bit_cast(f16, (__bf16)x);
  else
    return (f16)x;
}
template <class E>
__device__ __forceinline__ f16x4 to16x4(float a, float b, float c, float d) {
  return f16x4{to16<E>(a), to16<E>(b), to16<E>(c), to16<E>(d)};
}
template <class E>
__device__ __forceinline__ f16x4 to16x4(f32x4 v) {
  return to16x4<E>(v[0], v[1], v[2], v[3]);
}
// Outputs idx .. idx+3 of element type E from fp32: `out` is the kernels'
// 16-bit-typed output pointer, which for F32 holds floats (idx counts elements)
template <class E>
__device__ __forceinline__ void store_out4(f16* out, int64_t idx, f32x4 v) {
  if constexpr (kIsF32<E>)
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + idx) = v;
  else
    *reinterpret_cast<f16x4*>(out + idx) = to16x4<E>(v);
}
// One output element of type E set to x
template <class E>
__device__ __forceinline__ void store_out1(f16* out, int64_t idx, float x) {
  if constexpr (kIsF32<E>)
    reinterpret_cast<float*>(out)[idx] = x;
  else
    out[idx] = to16<E>(x);
}

__device__ __forceinline__ f16x4 lo4(f16x8 v) { return f16x4{v[0], v[1], v[2], v[3]}; }
__device__ __forceinline__ f16x4 hi4(f16x8 v) { return f16x4{v[4], v[5], v[6], v[7]}; }

// ---- split-K partition ---------------------------------------------------------
// The keys of every sequence are cut into 64-token "quads" (one 16-token tile
// per wave of a 256-thread workgroup).  All sequences share one chunk size,
// chosen on the device from the live context lengths so that the whole batch
// yields about `target` pieces per KV head:
//   quads_b = ceil(L_b / 64), chunk = max(1, ceil(sum_b quads_b / target)),
//   splits_b = ceil(quads_b / chunk).
// Pieces are numbered sequence-major; piece ids run over [0, sum_b splits_b) <=
// target + batch.  find_piece is evaluated by a whole wave and returns
// wave-uniform values.
//
// With a shared-prefix (cascade) decode, sequence b's keys before tok0[b] are
// attended elsewhere, and only its suffix [tok0[b], L_b) is partitioned here
// (quads_b counts the suffix).  tok0 == nullptr means tok0[b] = 0.

__device__ __forceinline__ int clamp_len(int L) { return L > 0 ? L : 0; }

// Context length as the kernels see it: negative -> 0, and never more than
// the block table can address (max_len = table width * block size).
__device__ __forceinline__ int seq_len(const int32_t* ctx, int b, int max_len) {
  const int L = clamp_len(ctx[b]);
  return L < max_len ? L : max_len;
}

// Maximum over all 64 lanes (wave-uniform result).
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp::mov<dpp::kQuadXor1>(v));
  v = max(v, dpp::mov<dpp::kQuadXor2>(v));
  v = max(v, dpp::mov<dpp::kRowHalfMirror>(v));
  v = max(v, dpp::mov<dpp::kRowMirror>(v));
  return max(max(readlane_i(v, 0), readlane_i(v, 16)), max(readlane_i(v, 32), readlane_i(v, 48)));
}

// Chunk size in quads.  Besides ~target pieces in total, no sequence is cut
// into more than kMaxPieces pieces, which bounds the merge of one sequence to
// four rounds of 16 partials, and no piece holds fewer than kMinChunk quads
// unless its sequence is shorter: at small batches, pieces of a quad or two
// spend more on their merge than they gain in parallelism.
constexpr int kMaxPieces = 64;
#ifndef FE_MIN_CHUNK
#define FE_MIN_CHUNK 3
#endif
constexpr int kMinChunk = FE_MIN_CHUNK;

// First key of sequence b's suffix (0 without a shared prefix); <= its length.
__device__ __forceinline__ int suffix_start(const int32_t* tok0, int b, int L) {
  if (tok0 == nullptr) return 0;
  const int t = tok0[b];
  return t > 0 ? (t < L ? t : L) : 0;
}

struct Piece {
  int b;         // sequence
  int id;        // piece id, sequence-major: the slot of its partial in a merge
  int split;     // index of this piece within the sequence
  int nsplit;    // pieces of this sequence
  int L;         // context length of the sequence
  int tok0;      // first key of the sequence's suffix (> 0: a shared prefix precedes it)
  int tok_begin; // first key position of the piece
  int tok_end;   // one past the last key position of the piece
};

// Finds the piece that workgroup slot `item` runs; false when item is past the
// last piece, in which case `total` receives the number of pieces.
//
// Pieces are numbered sequence-major (sequence b's pieces are ids first_b ..
// first_b + nsplit_b - 1, the slots of its merge) but handed out largest
// first: slots 0.. take every piece of exactly `chunk` quads, then come the
// sequences' remainders of at least chunk/2 quads, then the smaller ones.
// Workgroups start in slot order as compute units free up, so the short
// pieces fill the gaps left by compute units that finished early (the HBM
// service a CU receives varies by several microseconds over a launch), and
// the launch ends more evenly than in sequence order.
//
// Three passes over the sequences (quad totals -> chunk; piece counts per
// class; the search); the lengths of the first 64 sequences are loaded once
// and kept in registers, so a batch of up to 64 costs one round trip to
// memory.
__device__ __forceinline__ bool find_piece(const int32_t* ctx, const int32_t* tok0, int B,
                                           int max_len, int target, int item, Piece& pc,
                                           int& total) {
  const int lane = lane_id();
  int L0 = 0, s0 = 0;
  if (lane < B) {
    L0 = seq_len(ctx, lane, max_len);
    s0 = suffix_start(tok0, lane, L0);
  }
  const int nq0 = (L0 - s0 + 63) >> 6;
  int sum = wave_sum_i(nq0), longest = wave_max_i(nq0);
  for (int base = kWave; base < B; base += kWave) {
    const int b = base + lane;
    int nq = 0;
    if (b < B) {
      const int L = seq_len(ctx, b, max_len);
      nq = (L - suffix_start(tok0, b, L) + 63) >> 6;
    }
    sum += wave_sum_i(nq);
    const int m = wave_max_i(nq);
    longest = longest > m ? longest : m;
  }
  // the shuffle reductions leave the same value in every lane; readfirstlane
  // tells the compiler they are wave-uniform, so every bound and address
  // derived from them stays in scalar registers
  sum = __builtin_amdgcn_readfirstlane(sum);
  longest = __builtin_amdgcn_readfirstlane(longest);
  int chunk = (sum + target - 1) / target;
  const int floor_chunk = (longest + kMaxPieces - 1) / kMaxPieces;
  chunk = chunk > floor_chunk ? chunk : floor_chunk;
  chunk = chunk > kMinChunk ? chunk : kMinChunk;

  // quads of sequence base + lane (0 past the batch)
  auto quads = [&](int base, int& L, int& t0) __attribute__((always_inline)) {
    const int b = base + lane;
    if (base == 0) {
      L = L0;
      t0 = s0;
    } else {
      L = b < B ? seq_len(ctx, b, max_len) : 0;
      t0 = b < B ? suffix_start(tok0, b, L) : 0;
    }
    return (L - t0 + 63) >> 6;
  };
  // size class of a sequence's last piece: 0 none, 1 at least chunk/2 quads, 2 smaller
  auto rem_class = [&](int nq) __attribute__((always_inline)) {
    const int r = nq % chunk;
    return r == 0 ? 0 : (2 * r >= chunk ? 1 : 2);
  };

  int nfull = 0, nbig = 0;
  for (int base = 0; base < B; base += kWave) {
    int L, t0;
    const int nq = quads(base, L, t0);
    nfull += wave_sum_i(nq / chunk);
    nbig += wave_sum_i(rem_class(nq) == 1 ? 1 : 0);
  }
  nfull = __builtin_amdgcn_readfirstlane(nfull);
  nbig = __builtin_amdgcn_readfirstlane(nbig);
  const int cls = item < nfull ? 0 : (item < nfull + nbig ? 1 : 2);
  const int idx = item - (cls == 0 ? 0 : (cls == 1 ? nfull : nfull + nbig));

  int carry = 0, carry_id = 0;
  for (int base = 0; base < B; base += kWave) {
    const int b = base + lane;
    int L, t0;
    const int nq = quads(base, L, t0);
    const int nf = nq / chunk;
    const int rc = rem_class(nq);
    const int ns = nf + (rc != 0 ? 1 : 0);
    const int cnt = cls == 0 ? nf : (rc == cls ? 1 : 0);
    const int incl = wave_scan_incl_i(cnt) + carry;
    const int excl = incl - cnt;
    const int incl_id = wave_scan_incl_i(ns) + carry_id;
    const unsigned long long hit = __ballot(b < B && idx >= excl && idx < incl);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      pc.b = base + src;
      pc.L = readlane_i(L, src);
      pc.tok0 = readlane_i(t0, src);
      pc.nsplit = readlane_i(ns, src);
      pc.split = cls == 0 ? idx - readlane_i(excl, src) : readlane_i(nf, src);
      pc.id = readlane_i(incl_id, src) - pc.nsplit + pc.split;
      pc.tok_begin = pc.tok0 + pc.split * chunk * 64;
      const int e = pc.tok0 + (pc.split + 1) * chunk * 64;
      pc.tok_end = e < pc.L ? e : pc.L;
      return true;
    }
    carry = readlane_i(incl, kWave - 1);
    carry_id = readlane_i(incl_id, kWave - 1);
  }
  total = carry_id;
  return false;
}

// ---- shared-prefix (cascade) decode: the prefix half, launched by
// fe_paged_decode_shared_prefix (paged_decode.hip) and implemented with the
// prefill kernel (prefill.hip).  Group s is the decode rows group_offsets[s]
// .. group_offsets[s+1]-1; they share the first prefix_len[s] keys (whole
// blocks) of row group_offsets[s]'s table.  Output per (row, query head):
// the attention over the shared keys as fp32 (normalised) plus its base-2
// LSE, and tok0[b] for every row: the first key its own decode attends (the
// prefix end, or 0 when the row does not share a prefix). ----
// Most slots of a shared-prefix result (CascadePrefix::splits).
constexpr int kMaxPrefixSlots = 4;
struct CascadePrefix {
  const void* q;
  int64_t q_stride;
  const void* k_pool;
  const void* v_pool;
  int num_blocks;
  const int32_t* tables;
  int table_stride;
  const int32_t* ctx;
  const int32_t* group_offsets;
  const int32_t* prefix_len;
  int num_groups, batch, hq, hkv, d, bs;
  float scale;
  float* pre_o;      // [batch * hq][d]
  float* pre_lse;    // [batch * hq]
  int32_t* tok0;     // [batch]
  void* scratch;     // key-split partials, cascade_prefix_scratch_bytes
  bool bf16;         // q and the pools are bfloat16 (fp16 otherwise)
  bool f32;          // q and the pools are float32
  // set by cascade_prefix_launch: the prefix result the decode launch folds
  // into every row with a shared prefix -- `splits` slots per query-head row
  // r (row-major: the slots of a row are adjacent), slot s a normalised
  // output at out_o + (r * splits + s) * d and its base-2 LSE at
  // out_lse[r * splits + s]
  float* out_o;
  float* out_lse;
  int splits;
};
__attribute__((visibility("hidden"))) size_t cascade_prefix_scratch_bytes(int num_groups,
                                                                          int batch, int hq,
                                                                          int hkv, int d);
__attribute__((visibility("hidden"))) int cascade_prefix_launch(CascadePrefix& c,
                                                                hipStream_t stream);

// ---- generic attention (attn_generic.hip): the shapes the matrix-core kernels
// do not take -- head_dim other than 64 / 128, or more than 16 query heads per
// KV head.  A decode row attends keys 0 .. ctx[row] - 1 of table row `row`,
// cut into `splits` key ranges (more than one: normalised partial outputs and
// base-2 LSEs in part_o [rows * hq][splits][d] / part_lse [rows * hq][splits],
// folded by a second launch); a prefill token (q_offsets != null) of sequence
// s attends keys 0 .. cached + its index, cached = ctx[s] - n_s (0 when
// ctx[s] < n_s).  Rows with no keys give zeros. ----
constexpr int kGenericMaxHeadDim = 512;
constexpr int kGenericMaxGroup = 128;   // query heads per KV head
constexpr int kGenericMaxElems = 8192;  // group size * head_dim (padded to 8): LDS of an item
struct GenericAttn {
  const void* q;
  int64_t q_stride;    // elements between consecutive query rows
  void* out;
  int64_t out_stride;  // elements between consecutive output rows
  const void* k_new;   // decode page write at key ctx[row] - 1 (null: none)
  const void* v_new;
  int64_t new_stride;
  void* k_pool;
  void* v_pool;
  int num_blocks;
  const int32_t* tables;
  int table_stride;
  const int32_t* ctx;
  const int32_t* q_offsets;  // prefill: [num_seqs + 1]; null for a decode
  int num_seqs;
  int rows;  // decode: batch; prefill: total_q
  int hq, hkv, d, bs;
  float scale;
  int elem;  // 0 fp16, 1 bf16, 2 fp32
  int splits;  // decode key splits per row (<= 32)
  float* part_o;
  float* part_lse;
};
// head_dim rounded up to a multiple of 8 (the kernel's LDS rows)
__attribute__((visibility("hidden"))) int generic_padded_dims(int d);

// head_dim as the 16-bit matrix-core decode and prefill compute it: a multiple
// of 8 below 256 other than 64 / 128 runs padded to the next of 64 / 128 / 256
// (the dims past head_dim zeros in q and K, never read from the pools nor
// written to the output)
inline int mfma_padded_head_dim(int d) {
  if (d % 8 != 0 || d >= 256) return d;
  return d <= 64 ? 64 : (d <= 128 ? 128 : 256);
}
__attribute__((visibility("hidden"))) bool generic_shape(int hq, int hkv, int d);
__attribute__((visibility("hidden"))) int generic_attention(const GenericAttn& g,
                                                            hipStream_t stream);

}  // namespace fe

#define FE_CHECK_ARG(cond)                 \
  do {                                     \
    if (!(cond)) return FE_ERR_INVALID_ARGUMENT; \
  } while (0)

#define FE_LAUNCH_STATUS() ((int)hipGetLastError())
