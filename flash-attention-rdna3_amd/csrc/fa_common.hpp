// fa_common.hpp - device building blocks shared by the gfx950 attention kernels.
//
// Matrix-core conventions (CDNA4, wave64).  For a 32x32 MFMA accumulator the
// element i (0..15) held by lane l sits at
//     row = 8*(i/4) + 4*(l/32) + (i%4),   col = l%32.
// An A operand (32 x K) gives lane l row l%32 and E consecutive k-slots of
// half l/32; a B operand (K x 32) gives lane l column l%32 and the same
// k-slots.  Because the hardware pairs A and B k-slots identically, any
// bijection between k-slots and the contracted index may be used as long as
// A and B agree; the kernels rely on that to feed an accumulator straight
// back as a B operand (the contracted index then follows the accumulator's
// row map).
//
// 16-bit inputs use v_mfma_f32_32x32x16_{f16,bf16} (KSTEP 16, E 8),
// fp32 inputs use v_mfma_f32_32x32x2_f32 (KSTEP 2, E 1).
#pragma once

#include <climits>
#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fa_mi355x.h"

namespace fa {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 b16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

struct f16_t {};   // tag: IEEE half
struct bf16_t {};  // tag: bfloat16
struct f32_t {};   // tag: fp32

// ---------------------------------------------------------------------------
// Element traits: storage type, conversions, MFMA operand type and instruction.
// ---------------------------------------------------------------------------
template <typename Tag> struct Elem;

template <> struct Elem<f16_t> {
  using S = uint16_t;            // storage
  using Op = s16x8;              // MFMA operand (8 elements)
  static constexpr int KSTEP = 16;
  static constexpr int E = 8;    // k-slots per lane per MFMA
  static constexpr int CE = 8;   // elements per 16-byte chunk
  __device__ static inline float to_f(S x) { return (float)__builtin_bit_cast(_Float16, x); }
  __device__ static inline S from_f(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h16x8, a),
                                                  __builtin_bit_cast(h16x8, b), c, 0, 0, 0);
  }
};

template <> struct Elem<bf16_t> {
  using S = uint16_t;
  using Op = s16x8;
  static constexpr int KSTEP = 16;
  static constexpr int E = 8;
  static constexpr int CE = 8;
  __device__ static inline float to_f(S x) { return __uint_as_float(((uint32_t)x) << 16); }
  __device__ static inline S from_f(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b16x8, a),
                                                   __builtin_bit_cast(b16x8, b), c, 0, 0, 0);
  }
};

template <> struct Elem<f32_t> {
  using S = float;
  using Op = float;
  static constexpr int KSTEP = 2;
  static constexpr int E = 1;
  static constexpr int CE = 4;
  __device__ static inline float to_f(S x) { return x; }
  __device__ static inline S from_f(float x) { return x; }
  __device__ static inline f32x16 mma(Op a, Op b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

__device__ inline f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row of element i of a 32x32 accumulator for lane half h.
__device__ constexpr inline int acc_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// ---------------------------------------------------------------------------
// Operand loads.  E elements at `p` (16 bytes for 16-bit types, 4 for fp32).
// ---------------------------------------------------------------------------
template <typename Tag>
__device__ inline typename Elem<Tag>::Op load_op(const typename Elem<Tag>::S* p) {
  if constexpr (Elem<Tag>::E == 8) {
    return *reinterpret_cast<const s16x8*>(p);
  } else {
    return *p;
  }
}

template <typename Tag>
__device__ inline typename Elem<Tag>::Op zero_op() {
  if constexpr (Elem<Tag>::E == 8) {
    s16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    return z;
  } else {
    return 0.f;
  }
}

// Pack accumulator elements [8*j .. 8*j+7] (16-bit) or element j (fp32) of a
// 32x32 fp32 tile into a B operand whose k-slots follow the tile's row map.
template <typename Tag>
__device__ inline typename Elem<Tag>::Op pack_op(const f32x16& acc, int j) {
  using EL = Elem<Tag>;
  if constexpr (EL::E == 8) {
    s16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (short)EL::from_f(acc[8 * j + e]);
    return r;
  } else {
    return acc[j];
  }
}

// A operand read from a transposed LDS tile T[row][col] (col contiguous) where
// the k-slots follow an accumulator row map: slot e of lane half h reads
// column base + acc_row(8*j + e, h) (16-bit) or base + acc_row(j, h) (fp32).
template <typename Tag>
__device__ inline typename Elem<Tag>::Op lds_op_rowmap(const typename Elem<Tag>::S* row, int j, int h) {
  using EL = Elem<Tag>;
  if constexpr (EL::E == 8) {
    // slots 0..3 -> cols 16*(j/2)... see acc_row: for i = 8*(j%2) + e,
    // acc_row = 16*(j%2) + 8*(e/4) + 4h + (e%4) within the 32-row block j/2.
    const int base = 32 * (j >> 1) + 16 * (j & 1) + 4 * h;
    s16x4 lo = *reinterpret_cast<const s16x4*>(row + base);
    s16x4 hi = *reinterpret_cast<const s16x4*>(row + base + 8);
    s16x8 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return r;
  } else {
    const int blk = j >> 4, i = j & 15;
    return row[32 * blk + acc_row(i, h)];
  }
}

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt/lgkmcnt fields left at "no wait").
// Used once after the register operands loaded before a main loop, so the
// compiler's wait analysis knows they are resident on every path into the
// loop and does not drain the in-flight prefetches at the first MFMA.
__device__ inline void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// ---------------------------------------------------------------------------
// Cross-lane helpers (wave64).
// ---------------------------------------------------------------------------
// x combined with its partner lane 32 apart (sum / max over the two wave
// halves), without an LDS round trip: v_permlane32_swap exchanges the upper
// half of its first operand with the lower half of its second, so with both
// operands = x the pair holds x's lower half twice (r[0]) and its upper half
// twice (r[1]), and r[0] op r[1] is the combined value in every lane.
__device__ inline float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy
// as 1, 2, 3", SC'11).  Counter = 64-bit element offset, key = 64-bit seed.
// Returns a uniform float in [0, 1) from the first output word.
// ---------------------------------------------------------------------------
__device__ inline float philox_uniform(uint64_t seed, uint64_t offset) {
  uint32_t c0 = (uint32_t)offset, c1 = (uint32_t)(offset >> 32), c2 = 0u, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0 = __umulhi(M0, c0), lo0 = M0 * c0;
    uint32_t hi1 = __umulhi(M1, c2), lo1 = M1 * c2;
    uint32_t n0 = hi1 ^ c1 ^ k0;
    uint32_t n1 = lo1;
    uint32_t n2 = hi0 ^ c3 ^ k1;
    uint32_t n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += W0; k1 += W1;
  }
  return (float)(c0 >> 8) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------------------
// Score modifiers, applied in the log2 domain in the reference order
// scale -> softcap -> bias -> ALiBi -> mask (reference _common.py:276-308).
// ---------------------------------------------------------------------------
struct Mods {
  float scale_log2;   // softmax_scale * log2(e)
  float cap2;         // softcap * log2(e), 0 = off
  float cap_k;        // 2 log2(e) * softmax_scale / softcap: exp2 argument of e^{2y}
  float cap2_m2;      // -2 * cap2
  const void* bias;   // already offset to (batch, head); NULL = off
  int bias_f32;       // bias element type: 1 fp32, 0 q dtype
  int bias_bf16;      // q dtype is bf16 (only meaningful when !bias_f32)
  int64_t bias_sm, bias_sn;
  float alibi_log2;   // slope * log2(e), 0 = off
  int has_alibi;
  int causal, wl, wr; // window sides (-1 = unbounded)
  int off;            // seqlen_k - seqlen_q (bottom-right alignment)
  int seqlen_k;
  float drop_p;       // 0 = off
  float drop_scale;   // 1 / (1 - p)
  uint64_t drop_seed;
  uint64_t drop_base; // ((b*Hq + h) * Sq) for the element offset
  int64_t drop_sk;    // Sk of the dense problem
};

// Softcapped log2-domain score x = cap2 * tanh(s * scale / cap) of the raw dot
// product s, and tcap = tanh(s * scale / cap) (for the backward), from
// tanh(y) = 1 - 2 / (1 + e^{2y}): one hardware exp2 and one reciprocal.
// Saturates to +-1 without a sign split (e^{2y} -> inf gives 1, -> 0 gives
// -1); the absolute error of tcap is a few 2^-24, which is what the
// exp2 of the softmax sees (x's error is cap2 times that).
// In terms of r = 1 / (1 + e^{2y}): x = cap2 - 2 cap2 r, tcap = 1 - 2r and
// (1 - tcap^2) / 4 = r - r^2.  x falls as r grows; a hidden score (x = -inf)
// is r = +inf.
__device__ inline float softcap_r(const Mods& md, float s) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(s * md.cap_k));
}
__device__ inline float softcap_score(const Mods& md, float s, float& tcap) {
  const float r = softcap_r(md, s);
  tcap = __builtin_fmaf(-2.f, r, 1.f);
  return __builtin_fmaf(md.cap2_m2, r, md.cap2);
}

// A visibility interval [lo, hi] of positions base + k, held relative to
// base so the per-score test compares the compile-time offset k against two
// registers (no per-score address arithmetic).  Bounds are clamped to
// +-2^30 first, so the subtraction cannot overflow.
struct Span {
  int lo, hi;
};
__device__ inline Span make_span(int lo, int hi, int base) {
  constexpr int kBig = 1 << 30;
  return Span{max(lo, -kBig) - base, min(hi, kBig) - base};
}
__device__ inline bool in_span(const Span& s, int k) { return (k >= s.lo) & (k <= s.hi); }

// Visible keys of row m form [lo, hi] (empty when hi < lo).  The mode flags
// are wave-uniform, so the bounds are scalar selects.
__device__ inline void key_bounds(const Mods& md, int m, int& lo, int& hi) {
  const int qp = m + md.off;
  hi = min(md.seqlen_k - 1, min(md.causal ? qp : INT_MAX, md.wr >= 0 ? qp + md.wr : INT_MAX));
  lo = md.wl >= 0 ? qp - md.wl : INT_MIN;
}

// Visible query rows of key n form [lo, hi] (empty when hi < lo): the
// transpose of key_bounds.
__device__ inline void row_bounds(const Mods& md, int n, int& lo, int& hi) {
  constexpr int kBig = 1 << 30;
  lo = max(md.causal ? n : -kBig, md.wr >= 0 ? n - md.wr : -kBig) - md.off;
  hi = (md.wl >= 0 ? n + md.wl : kBig) - md.off;
  if (n >= md.seqlen_k) { lo = kBig; hi = -kBig; }
}

__device__ inline bool keep_pos(const Mods& md, int m, int n) {
  int lo, hi;
  key_bounds(md, m, lo, hi);
  return (n <= hi) & (n >= lo);
}

__device__ inline float load_bias(const Mods& md, int m, int n) {
  const int64_t o = (int64_t)m * md.bias_sm + (int64_t)n * md.bias_sn;
  if (md.bias_f32) return reinterpret_cast<const float*>(md.bias)[o];
  uint16_t b = reinterpret_cast<const uint16_t*>(md.bias)[o];
  return md.bias_bf16 ? Elem<bf16_t>::to_f(b) : Elem<f16_t>::to_f(b);
}

// Full modifier chain on one raw dot product s (no mask).  Returns the log2
// domain score and, through tcap, tanh(.) of the softcap (for the backward).
template <bool MODS>
__device__ inline float score(const Mods& md, float s, int m, int n, float& tcap) {
  float x = s * md.scale_log2;
  tcap = 0.f;
  if constexpr (MODS) {
    if (md.cap2 > 0.f) {
      x = softcap_score(md, s, tcap);
    }
    if (md.bias) x += load_bias(md, m, n) * kLog2e;
    if (md.has_alibi) x -= md.alibi_log2 * fabsf((float)(n - m - md.off));
  }
  return x;
}

// Bias element of kind K: 1 fp32, 2 fp16, 3 bf16.
template <int K>
__device__ inline float load_bias_k(const Mods& md, int m, int n) {
  const int64_t o = (int64_t)m * md.bias_sm + (int64_t)n * md.bias_sn;
  if constexpr (K == 1) return reinterpret_cast<const float*>(md.bias)[o];
  const uint16_t b = reinterpret_cast<const uint16_t*>(md.bias)[o];
  if constexpr (K == 3) return Elem<bf16_t>::to_f(b);
  return Elem<f16_t>::to_f(b);
}

// score() with the modifier set fixed at compile time (no per-score tests).
// BIASK: 0 no bias, else the kind of load_bias_k.
template <bool CAP, int BIASK, bool ALIBI>
__device__ inline float score_m(const Mods& md, float s, int m, int n, float& tcap) {
  float x = s * md.scale_log2;
  tcap = 0.f;
  if constexpr (CAP) {
    x = softcap_score(md, s, tcap);
  }
  if constexpr (BIASK != 0) x += load_bias_k<BIASK>(md, m, n) * kLog2e;
  if constexpr (ALIBI) x -= md.alibi_log2 * fabsf((float)(n - m - md.off));
  return x;
}

// Calls f(cap, bias_kind, alibi) with std::integral_constant flags for the
// modifiers `md` enables: the per-tile unswitch of score_m.
template <typename F>
__device__ inline void dispatch_mods(const Mods& md, F&& f) {
  using T = std::true_type;
  using N = std::false_type;
  auto with_bias = [&](auto cap, auto al) {
    if (md.bias == nullptr) f(cap, std::integral_constant<int, 0>{}, al);
    else if (md.bias_f32) f(cap, std::integral_constant<int, 1>{}, al);
    else if (md.bias_bf16) f(cap, std::integral_constant<int, 3>{}, al);
    else f(cap, std::integral_constant<int, 2>{}, al);
  };
  const bool cap = md.cap2 > 0.f, al = md.has_alibi != 0;
  if (cap) { if (al) with_bias(T{}, T{}); else with_bias(T{}, N{}); }
  else { if (al) with_bias(N{}, T{}); else with_bias(N{}, N{}); }
}

__device__ inline bool dropout_keep(const Mods& md, int m, int n) {
  const uint64_t o = (md.drop_base + (uint64_t)m) * (uint64_t)md.drop_sk + (uint64_t)n;
  return philox_uniform(md.drop_seed, o) > md.drop_p;
}

// Visibility of a (rows [m0, m0+mr), keys [n0, n0+nr)) rectangle under the
// position masks: 0 = fully hidden, 1 = partially, 2 = fully visible.
__device__ inline int rect_visibility(const Mods& md, int m0, int mr, int n0, int nr) {
  const int n1 = n0 + nr - 1;
  const int q0 = m0 + md.off, q1 = m0 + mr - 1 + md.off;
  if (n0 >= md.seqlen_k) return 0;
  if (md.causal && n0 > q1) return 0;
  if (md.wl >= 0 && n1 < q0 - md.wl) return 0;
  if (md.wr >= 0 && n0 > q1 + md.wr) return 0;
  bool full = n1 < md.seqlen_k;
  if (md.causal) full = full && (n1 <= q0);
  if (md.wl >= 0) full = full && (n0 >= q1 - md.wl);
  if (md.wr >= 0) full = full && (n1 <= q0 + md.wr);
  return full ? 2 : 1;
}

// Tile visibility from per-block bounds computed once.  For a fixed block of
// query rows (positions q = m + off in [q0, q1]) a key tile [n0, n1] is
// visible (1) when it meets [lo_any, hi_any] and fully visible (2) when it
// lies inside [lo_all, hi_all]; same result as rect_visibility, with the
// mode tests hoisted out of the tile loop.
struct VisBounds {
  int lo_any, hi_any, lo_all, hi_all;
};

__device__ inline VisBounds row_block_bounds(const Mods& md, int m0, int mr) {
  VisBounds v;
  if (mr <= 0) {
    v.lo_any = INT_MAX; v.hi_any = INT_MIN; v.lo_all = INT_MAX; v.hi_all = INT_MIN;
    return v;
  }
  const int q0 = m0 + md.off, q1 = m0 + mr - 1 + md.off;
  v.lo_any = md.wl >= 0 ? q0 - md.wl : INT_MIN;
  v.hi_any = min(md.seqlen_k - 1, min(md.causal ? q1 : INT_MAX, md.wr >= 0 ? q1 + md.wr : INT_MAX));
  v.lo_all = md.wl >= 0 ? q1 - md.wl : INT_MIN;
  v.hi_all = min(md.seqlen_k - 1, min(md.causal ? q0 : INT_MAX, md.wr >= 0 ? q0 + md.wr : INT_MAX));
  return v;
}

// The transposed case: fixed keys [n0, n1], query tiles varying.  Bounds are
// on the query position q = m + off.
__device__ inline VisBounds key_block_bounds(const Mods& md, int n0, int nc) {
  VisBounds v;
  const int n1 = n0 + nc - 1;
  if (nc <= 0 || n0 >= md.seqlen_k) {
    v.lo_any = INT_MAX; v.hi_any = INT_MIN; v.lo_all = INT_MAX; v.hi_all = INT_MIN;
    return v;
  }
  v.lo_any = max(md.causal ? n0 : INT_MIN, md.wr >= 0 ? n0 - md.wr : INT_MIN);
  v.hi_any = md.wl >= 0 ? n1 + md.wl : INT_MAX;
  const bool keys_ok = n1 < md.seqlen_k;
  v.lo_all = keys_ok ? max(md.causal ? n1 : INT_MIN, md.wr >= 0 ? n1 - md.wr : INT_MIN) : INT_MAX;
  v.hi_all = keys_ok ? (md.wl >= 0 ? n0 + md.wl : INT_MAX) : INT_MIN;
  return v;
}

// 0 / 1 / 2 for the interval [a0, a1] against the bounds.
__device__ inline int bounds_vis(const VisBounds& v, int a0, int a1) {
  const bool any = (a1 >= v.lo_any) & (a0 <= v.hi_any);
  const bool all = (a0 >= v.lo_all) & (a1 <= v.hi_all);
  return any ? (all ? 2 : 1) : 0;
}

// Bounded varlen interval (reference varlen.py:21-27).
__device__ inline void bounded_seq(const int32_t* cu, int b, int total, int& start, int& len) {
  int s = cu[b], e = cu[b + 1];
  s = min(max(s, 0), total);
  e = min(max(e, 0), total);
  start = s;
  len = max(e - s, 0);
}

// Modifier state of (batch b, query head hq) for a problem whose sequence
// lengths (after varlen bounding) are sq x sk.
__device__ inline Mods make_mods(const fa_fwd_params& p, int b, int hq, int sq, int sk) {
  Mods md;
  md.scale_log2 = p.softmax_scale * kLog2e;
  md.cap2 = p.softcap * kLog2e;
  md.cap_k = p.softcap > 0.f ? 2.f * kLog2e * p.softmax_scale / p.softcap : 0.f;
  md.cap2_m2 = -2.f * md.cap2;
  md.bias = nullptr;
  md.bias_f32 = p.bias_dtype == FA_DTYPE_F32;
  md.bias_bf16 = p.dtype == FA_DTYPE_BF16;
  md.bias_sm = p.bias_stride[2];
  md.bias_sn = p.bias_stride[3];
  if (p.bias) {
    const int64_t o = b * p.bias_stride[0] + hq * p.bias_stride[1];
    md.bias = md.bias_f32 ? (const void*)(reinterpret_cast<const float*>(p.bias) + o)
                          : (const void*)(reinterpret_cast<const uint16_t*>(p.bias) + o);
  }
  md.has_alibi = p.alibi_slopes != nullptr;
  md.alibi_log2 = md.has_alibi ? p.alibi_slopes[hq] * kLog2e : 0.f;
  md.causal = p.causal;
  md.wl = p.window_left;
  md.wr = p.window_right;
  md.off = sk - sq;
  md.seqlen_k = sk;
  md.drop_p = p.dropout_p;
  md.drop_scale = p.dropout_p > 0.f ? 1.f / (1.f - p.dropout_p) : 1.f;
  md.drop_seed = p.dropout_seed;
  md.drop_base = ((uint64_t)b * p.heads_q + hq) * (uint64_t)p.seqlen_q;
  md.drop_sk = p.seqlen_k;
  return md;
}

// Linear workgroup id remapped so that consecutive logical ids land on the
// same XCD (the hardware deals workgroups round-robin over 8 XCDs, each with
// its own L2).  Only applied when the grid is a multiple of 8.
__device__ inline int xcd_swizzle(int id, int n) {
  if ((n & 7) != 0) return id;
  return (id & 7) * (n >> 3) + (id >> 3);
}

}  // namespace fa
