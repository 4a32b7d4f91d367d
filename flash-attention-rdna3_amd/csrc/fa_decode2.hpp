// fa_decode2.hpp - streaming decode kernel (16-bit, D <= 128), contiguous or
// paged cache.  Same results as decode_kernel (reference kernels/decode.py:9-125,
// kernels/paged.py:16-89); organised for HBM throughput on gfx950:
//
//  * K rows load straight into registers in the MFMA operand layout; V rows
//    load into registers as raw 16-byte pieces (each instruction reads four
//    whole 256-byte rows) and go to a per-wave swizzled LDS tile just before
//    use, from which the P.V MFMA reads them transposed.
//  * Every wave streams its own 32-key chunks through NBUF private slots
//    (128 VGPRs of slots: 32 KiB in flight per wave) and synchronises only with itself
//    (s_waitcnt), so the workgroup never stalls on a barrier in the key loop.
//  * Scores use v_mfma_f32_16x16x32: the packed GQA rows (group heads x Sq,
//    usually 4) occupy 16 MFMA columns instead of 32.  P^T feeds the P.V MFMA
//    from its accumulator; V^T comes from the row-major LDS tile through
//    ds_read_b64_tr_b16.
//  * The 4 wave states are merged in LDS, so one partial per workgroup (or
//    the final row, with a single split) reaches HBM.
#pragma once

#include "fa_internal.hpp"
#include "fa_tiles.hpp"

// Workgroups of 8 waves (two per SIMD, a smaller chunk-slot budget each) for
// fp8 caches and for 4- / 8-key pages: there the per-chunk work (fp8
// conversion, per-lane page choice), not the bytes in flight, bounds the
// kernel, and a second wave per SIMD overlaps it (measured 8-10 % faster for
// fp8, 7-14 % for small pages; 4 waves stay faster for 16-bit caches in
// pages of >= 16 keys or contiguous).
namespace fa {

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <typename Tag> __device__ inline f32x4v mma16(s16x8 a, s16x8 b, f32x4v c);
template <> __device__ inline f32x4v mma16<f16_t>(s16x8 a, s16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, a), __builtin_bit_cast(h16x8, b), c, 0, 0, 0);
}
template <> __device__ inline f32x4v mma16<bf16_t>(s16x8 a, s16x8 b, f32x4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b16x8, a), __builtin_bit_cast(b16x8, b), c, 0, 0, 0);
}


template <int D, bool KV8 = false, bool SMALLPG = false>
struct Dec2Cfg {
  static constexpr bool WIDE = KV8 || SMALLPG;       // 8 waves, 64-VGPR slot budget
  static constexpr int NW = WIDE ? 8 : 4;
  static constexpr int NT = 64 * NW;
  static constexpr int CK = 32;                      // keys per chunk
  static constexpr int CPR = D / 8;                  // 16-byte chunks per row
  static constexpr int TILE = CK * D;                // elements of a V tile
  static constexpr int NSTEP = D / 32;               // 16x16x32 k-steps
  static constexpr int NDB = D / 16;                 // 16-wide blocks of O^T
  static constexpr int KLOADS = 2 * NSTEP;           // K dwordx4 loads per chunk per lane
  static constexpr int VLOADS = CK * CPR / 64;       // V dwordx4 loads per chunk per lane
  static constexpr int PER = KLOADS + VLOADS;        // vector-memory ops per chunk
  // Chunk slots per wave (each slot is 4*PER VGPRs per lane): 128 VGPRs of
  // slots for 16-bit caches, 64 for fp8 caches (SLOT_VGPRS8).
  static constexpr int SLOT_VGPRS = 128;
  // fp8 cache: 16-byte loads of 16 elements.  K steps go in pairs (KP) when
  // NSTEP is even (else one 8-byte load per step); V rows in 16-element
  // pieces (VN loads per chunk per lane).
  static constexpr bool KP = KV8 && NSTEP % 2 == 0;
  static constexpr int KN = KP ? NSTEP / 2 : NSTEP;   // K loads per key block
  static constexpr int VN = KV8 ? CK * (D / 16) / 64 : VLOADS;
  static constexpr int SLOT_REGS = KV8 ? 2 * KN * (KP ? 4 : 2) + 4 * VN : 4 * PER;
  static constexpr int SLOT_VGPRS8 = 64;
  static constexpr int NBUF = (KV8 ? SLOT_VGPRS8 : WIDE ? 64 : SLOT_VGPRS) / SLOT_REGS;
  static constexpr int WAVE_ELEMS = TILE;            // one private V tile per wave
  static constexpr int LOOP_BYTES = NW * WAVE_ELEMS * 2;
  static constexpr int OLD = 17;                     // merge buffer row stride (floats)
  static constexpr int MERGE_BYTES = NW * D * OLD * 4 + 2 * NW * 16 * 4 + 16;  // + ticket flag
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
};

// PAGE: 0 contiguous cache; 1 paged with block_size >= 16 (a 32-key chunk
// spans at most two pages, whose ids are wave-uniform scalar loads); 2 paged
// with block_size 4 or 8 (up to eight pages per chunk, one id per 4 keys).
//
// Pipeline: each wave owns NBUF chunk slots of registers.  Slot j holds chunk
// k = NBUF*i + j: K in the MFMA A layout (lane row l%16, 8 dims per k-step)
// and V as the raw 16-byte pieces of the chunk's rows.  A chunk's V goes to
// the wave's private swizzled LDS tile just before use and is read back
// transposed.  Every slot is refilled right after it is consumed,
// unconditionally (slots past the wave's last chunk load a readable stand-in
// row), so NBUF-1 chunks stay in flight while one is computed.  All loads are
// ordinary vector loads into registers: the compiler's per-register vmcnt
// tracking then waits exactly for the slot being used.  (Asynchronous LDS DMA
// in this loop makes it drain every load at the loop head instead.)
// KV8: the cache holds fp8 (OCP e4m3) K and V.
template <typename Tag, int D, int PAGE, bool KV8 = false>
__global__ __launch_bounds__((KV8 || PAGE == 2) ? 512 : 256) void decode2_kernel(DecodeArgs a) {
  static_assert(PAGE >= 0 && PAGE <= 2, "decode2 handles contiguous caches and pages of >= 4 keys");
  constexpr bool PAGED = PAGE != 0;
  using C = Dec2Cfg<D, KV8, PAGE == 2>;
  using EL = Elem<Tag>;
  using S = uint16_t;
  using KE = typename std::conditional<KV8, uint8_t, S>::type;  // cache element
  // Registers of one K / V load (see Dec2Cfg: KP, KN, VN).
  using KRaw = typename std::conditional<KV8, typename std::conditional<C::KP, u32x4, u32x2>::type, s16x8>::type;
  using VRaw = typename std::conditional<KV8, u32x4, s16x8>::type;
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, l16 = lane & 15;
  const int group = a.heads_q / a.heads_kv;
  const int rows = group * a.seqlen_q;
  // Grid (heads_kv * row blocks * slots, batch or 1), KV heads fastest: the
  // KV heads of one key range are adjacent in dispatch order, so a paged
  // cache's pages (all KV heads of a token row side by side) are read by
  // neighbouring workgroups at about the same time (measured 4 % faster on
  // paged caches).
  const int nrb = (rows + 15) / 16;
  const int hk = blockIdx.x % a.heads_kv;
  const int rb = (blockIdx.x / a.heads_kv) % nrb;
  const int slot = blockIdx.x / (a.heads_kv * nrb);
  auto seq_len = [&](int bb) {
    return a.lens ? min(max(a.lens[bb * a.lens_stride] + a.lens_add, 0), a.max_len) : a.max_len;
  };
  // One segment: chunks [c0, c0 + cnt) of sequence b.  With nctr == 1 the
  // segment is the whole sequence and writes the output rows; otherwise it
  // is one of nctr partials, stored at partial slot `pslot`, and the last of
  // them to arrive merges slots pfirst + k * pstep, k < nctr.
  auto segment = [&](const int b, const int len, const int c0, const int cnt, const int nctr, const int pslot,
                     const int pfirst, const int pstep) {
  // This lane's packed query column (group head, query row).
  const int r = rb * 16 + l16;
  const bool rvalid = r < rows;
  const int gq = rvalid ? r / a.seqlen_q : 0;
  const int mq = rvalid ? r - gq * a.seqlen_q : 0;
  const int hq = hk * group + gq;
  // Last key this lane's query row sees (bottom-right causal), or all.
  const int klim = a.causal ? len - a.seqlen_q + mq : INT_MAX;
  // Q operand: loaded after the first chunk's loads are issued (one round
  // trip to memory for both), waited for at its first use.
  s16x8 qop[C::NSTEP];
  auto load_q = [&]() {
    const S* qrow = reinterpret_cast<const S*>(a.q) + b * a.q_stride[0] + hq * a.q_stride[1] + mq * a.q_stride[2];
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      // With paired fp8 K loads, lane group g4 covers the 16 dims
      // 64*(s/2) + 16*g4 of a step pair (a permutation of the contracted
      // index, applied to Q and K alike).
      const int d0 = C::KP ? 64 * (s / 2) + 16 * g4 + 8 * (s % 2) : 8 * (4 * s + g4);
      qop[s] = load_op<Tag>(qrow + d0);
    }
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) qop[s] = rvalid ? qop[s] : zero_op<Tag>();
  };

  const KE* kbase = reinterpret_cast<const KE*>(a.k);
  const KE* vbase = reinterpret_cast<const KE*>(a.v);
  if constexpr (!PAGED) {
    kbase += b * a.k_stride[0] + hk * a.k_stride[1];
    vbase += b * a.v_stride[0] + hk * a.v_stride[1];
  } else {
    kbase += hk * a.k_stride[2];
    vbase += hk * a.v_stride[2];
  }
  const int bs_mask = (1 << a.block_shift) - 1;
  S* wbase = reinterpret_cast<S*>(smem_raw) + wave * C::WAVE_ELEMS;

  // Page ids are read through the constant address space so the compiler
  // issues scalar loads (lgkmcnt): a vector load would enter the vmcnt
  // sequence the pipeline counts on.
  typedef const __attribute__((address_space(4))) int32_t const_i32;
  const_i32* btab = (const_i32*)a.block_table;
  const int64_t bt_row = (int64_t)b * a.bt_stride[0];
  // Page ids of the (at most two) pages holding rows [0,16) and [16,32) of a
  // chunk (uniform across the wave).
  auto chunk_pages = [&](int c, int& pg0, int& pg1) {
    const int n0 = c * C::CK;
    const int last = (a.max_len - 1) >> a.block_shift;
    pg0 = btab[bt_row + (int64_t)min(n0 >> a.block_shift, last) * a.bt_stride[1]];
    pg1 = btab[bt_row + (int64_t)min((n0 + 16) >> a.block_shift, last) * a.bt_stride[1]];
  };
  // PAGE 2: ids of the pages holding rows [4i, 4i + 4) of a chunk.
  struct Pages8 { int p0, p1, p2, p3, p4, p5, p6, p7; };
  auto chunk_pages8 = [&](int c, Pages8& pg) {
    const int n0 = c * C::CK;
    const int last = (a.max_len - 1) >> a.block_shift;
    auto id = [&](int i) { return btab[bt_row + (int64_t)min((n0 + 4 * i) >> a.block_shift, last) * a.bt_stride[1]]; };
    pg = Pages8{id(0), id(1), id(2), id(3), id(4), id(5), id(6), id(7)};
  };
  // The page of chunk row r (a per-lane choice among uniform ids, as selects).
  auto page8 = [&](const Pages8& pg, int r) -> int {
    const int g = r >> 2;
    const int p01 = (g & 1) ? pg.p1 : pg.p0, p23 = (g & 1) ? pg.p3 : pg.p2;
    const int p45 = (g & 1) ? pg.p5 : pg.p4, p67 = (g & 1) ? pg.p7 : pg.p6;
    const int p03 = (g & 2) ? p23 : p01, p47 = (g & 2) ? p67 : p45;
    return (g & 4) ? p47 : p03;
  };
  // Element offset of key n's row from the per-(b, hk) base, or -1 if absent
  // (branch-free).
  auto key_off = [&](int n, int pg0, int pg1, const Pages8& p8, const int64_t* st) -> int64_t {
    bool ok = n < len;
    int64_t off;
    if constexpr (PAGE == 0) {
      off = (int64_t)n * st[2];
    } else {
      const int phys = PAGE == 2 ? page8(p8, n & 31) : ((n & 31) < 16) ? pg0 : pg1;
      ok = ok && phys >= 0 && phys < a.num_blocks;
      off = (int64_t)phys * st[0] + (int64_t)(n & bs_mask) * st[1];
    }
    return ok ? off : -1;
  };

  // Contiguous 16-bit caches are read with nontemporal loads (each byte is
  // read once): measured 3-4 us faster on config 3, while paged caches ran
  // 1.5-2 us slower with them, so those keep plain loads.
  auto ld16 = [](const auto* p) {
    if constexpr (PAGE == 0 && !KV8) return __builtin_nontemporal_load(p);
    else return *p;
  };
  // Chunk slot j: K registers kr[j], V registers vr[j].  `live` false loads
  // the stand-in row 0 (nothing of it is used).
  KRaw kr[C::NBUF][2][C::KN];
  VRaw vreg[C::NBUF][C::VN];
  auto issue_chunk = [&](int c, bool live, KRaw (&kd)[2][C::KN], VRaw (&vd)[C::VN]) {
    const int n0 = c * C::CK;
    int pg0 = 0, pg1 = 0;
    Pages8 p8{};
    if constexpr (PAGE == 1) chunk_pages(c, pg0, pg1);
    if constexpr (PAGE == 2) chunk_pages8(c, p8);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      int64_t ko = key_off(n0 + 16 * kb + l16, pg0, pg1, p8, a.k_stride);
      ko = (ko < 0 || !live) ? 0 : ko;
#pragma unroll
      for (int s = 0; s < C::KN; ++s) {
        if constexpr (C::KP) kd[kb][s] = *reinterpret_cast<const u32x4*>(kbase + ko + 64 * s + 16 * g4);
        else if constexpr (KV8) kd[kb][s] = *reinterpret_cast<const u32x2*>(kbase + ko + 8 * (4 * s + g4));
        else kd[kb][s] = ld16(reinterpret_cast<const s16x8*>(kbase + ko + 8 * (4 * s + g4)));
      }
    }
    // V: 8-element (16-bit) or 16-element (fp8) pieces of the chunk's rows.
    constexpr int PPR = KV8 ? D / 16 : C::CPR;  // pieces per row
#pragma unroll
    for (int i = 0; i < C::VN; ++i) {
      const int slot = 64 * i + lane;
      const int row = slot / PPR;
      int64_t vo = key_off(n0 + row, pg0, pg1, p8, a.v_stride);
      vo = (vo < 0 || !live) ? 0 : vo;
      vd[i] = ld16(reinterpret_cast<const VRaw*>(vbase + vo + (slot % PPR) * (KV8 ? 16 : 8)));
    }
  };
  // Bit k of the result: key n0 + k of the chunk is visible.
  auto chunk_mask = [&](int c) -> uint32_t {
    int pg0 = 0, pg1 = 0;
    Pages8 p8{};
    if constexpr (PAGE == 1) chunk_pages(c, pg0, pg1);
    if constexpr (PAGE == 2) chunk_pages8(c, p8);
    const int n = c * C::CK + (lane & 31);
    const bool ok = key_off(n, pg0, pg1, p8, a.k_stride) >= 0;
    return (uint32_t)__builtin_amdgcn_ballot_w64(ok && lane < 32);
  };

  float m_i = kNegInf, l_i = 0.f;
  f32x4v acc[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) acc[i] = f32x4v{0.f, 0.f, 0.f, 0.f};

  S* const Vs = wbase;
  // K operand of step s of key block kb.
  auto k_op = [&](const KRaw (&kd)[2][C::KN], int kb, int s) -> s16x8 {
    if constexpr (C::KP) {
      const u32x4 w = kd[kb][s / 2];
      return fp8x8_to_op<Tag>(s % 2 ? u32x2{w[2], w[3]} : u32x2{w[0], w[1]});
    } else if constexpr (KV8) {
      return fp8x8_to_op<Tag>(kd[kb][s]);
    } else {
      return kd[kb][s];
    }
  };
  auto compute_chunk = [&](int c, const KRaw (&kd)[2][C::KN], const VRaw (&vd)[C::VN]) {
    const uint32_t vmask = chunk_mask(c);
    // V rows -> this wave's LDS tile (swizzled); the previous chunk's reads of
    // the tile precede these writes in the wave's LDS order.
#pragma unroll
    for (int i = 0; i < C::VN; ++i) {
      const int slot = 64 * i + lane;
      if constexpr (KV8) {
        const int row = slot / (D / 16), col = (slot % (D / 16)) * 16;
        *reinterpret_cast<s16x8*>(Vs + swz_off<D>(row, col)) = fp8x8_to_op<Tag>(u32x2{vd[i][0], vd[i][1]});
        *reinterpret_cast<s16x8*>(Vs + swz_off<D>(row, col + 8)) = fp8x8_to_op<Tag>(u32x2{vd[i][2], vd[i][3]});
      } else {
        *reinterpret_cast<s16x8*>(Vs + swz_off<D>(slot / C::CPR, (slot % C::CPR) * 8)) = vd[i];
      }
    }
    f32x4v sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s) sacc[kb] = mma16<Tag>(k_op(kd, kb, s), qop[s], sacc[kb]);
    }
    float tmax = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 16 * kb + 4 * g4 + i;
        const float x =
            (((vmask >> key) & 1u) && c * C::CK + key <= klim) ? sacc[kb][i] * a.scale_log2 : kNegInf;
        sacc[kb][i] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_i, tmax);
    const float m_use = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
    float rsum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pv = __builtin_amdgcn_exp2f(sacc[kb][i] - m_use);
        sacc[kb][i] = pv;
        rsum += pv;
      }
    rsum += __shfl_xor(rsum, 16, 64);
    rsum += __shfl_xor(rsum, 32, 64);
    l_i = l_i * alpha + rsum;
    m_i = m_new;
    s16x8 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pb[i] = (short)EL::from_f(sacc[0][i]);
      pb[4 + i] = (short)EL::from_f(sacc[1][i]);
    }
    // V^T operand: group g4 holds keys 4*g4 + e and 16 + 4*g4 + e of column
    // block db (ds_read_b64_tr_b16 lane semantics as in tr_op_rowmap).  Rows
    // r and r + 16 share the swizzle.
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const int trow = 4 * g4 + ((lane & 15) >> 2);
    s16x4 vr[2 * C::NDB];
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      S* p = const_cast<S*>(Vs) + swz_off<D>(trow, 16 * db + 4 * (lane & 3));
      const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)p);
      const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p + 16 * D));
      vr[2 * db] = s16x4{lo[0], lo[1], lo[2], lo[3]};
      vr[2 * db + 1] = s16x4{hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      const s16x4 lo = vr[2 * db], hi = vr[2 * db + 1];
      const s16x8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      acc[db] *= alpha;
      acc[db] = mma16<Tag>(va, pb, acc[db]);
    }
  };

  // Chunks of this wave: c0 + wave + NW*k, k < mine.
  const int mine = cnt > wave ? (cnt - wave + C::NW - 1) / C::NW : 0;
  const int groups = (mine + C::NBUF - 1) / C::NBUF;
#pragma unroll
  for (int j = 0; j < C::NBUF; ++j) {
    issue_chunk(c0 + wave + C::NW * j, j < mine, kr[j], vreg[j]);
    if (j == 0) load_q();
  }
  // Steady state: every slot is refilled after use.
  for (int gi = 0; gi + 1 < groups; ++gi) {
#pragma unroll
    for (int j = 0; j < C::NBUF; ++j) {
      const int k = gi * C::NBUF + j;
      compute_chunk(c0 + wave + C::NW * k, kr[j], vreg[j]);
      const int kn = k + C::NBUF;
      issue_chunk(c0 + wave + C::NW * kn, kn < mine, kr[j], vreg[j]);
    }
  }
  // Last group: everything it needs is in flight.
  if (groups > 0) {
#pragma unroll
    for (int j = 0; j < C::NBUF; ++j) {
      const int k = (groups - 1) * C::NBUF + j;
      if (k < mine) compute_chunk(c0 + wave + C::NW * k, kr[j], vreg[j]);
    }
  }

  // Merge the wave states through LDS.
  __syncthreads();
  float* ow = reinterpret_cast<float*>(smem_raw);
  float* mw = ow + C::NW * D * C::OLD;
  float* lw = mw + C::NW * 16;
#pragma unroll
  for (int db = 0; db < C::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) ow[(wave * D + 16 * db + 4 * g4 + i) * C::OLD + l16] = acc[db][i];
  if (g4 == 0) {
    mw[wave * 16 + l16] = m_i;
    lw[wave * 16 + l16] = l_i;
  }
  __syncthreads();
  for (int idx = tid; idx < 16 * D; idx += C::NT) {
    const int cc = idx / D, d = idx - (idx / D) * D;
    const int row = rb * 16 + cc;
    if (row >= rows) continue;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < C::NW; ++w) M = fmaxf(M, mw[w * 16 + cc]);
    const float Mu = (M == kNegInf) ? 0.f : M;
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < C::NW; ++w) {
      const float sc = __builtin_amdgcn_exp2f(mw[w * 16 + cc] - Mu);
      L += lw[w * 16 + cc] * sc;
      o += ow[(w * D + d) * C::OLD + cc] * sc;
    }
    const float Ls = (L == 0.f) ? 1.f : L;
    o = o / Ls * a.out_scale;  // out_scale: v_scale of an fp8 cache, else 1
    const int gg = row / a.seqlen_q, mm = row - gg * a.seqlen_q;
    const int hh = hk * group + gg;
    if (nctr == 1) {
      S* op = reinterpret_cast<S*>(a.out) + b * a.out_stride[0] + hh * a.out_stride[1] + mm * a.out_stride[2];
      op[d] = EL::from_f(o);
    } else {
      const int64_t prow = ((int64_t)pslot * a.heads_q + hh) * a.seqlen_q + mm;
      const float lse = (M == kNegInf || L == 0.f) ? kNegInf : (M + __log2f(L)) * kLn2;
      if (a.tickets) {
        // Agent-scope stores are written through to the device's coherence
        // point (the XCDs' L2s are not coherent with each other), so the
        // merging workgroup, on any XCD, reads them with agent-scope loads.
        __hip_atomic_store(a.ws_o + prow * a.head_dim + d, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) __hip_atomic_store(a.ws_lse + prow, lse, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        a.ws_o[prow * a.head_dim + d] = o;
        if (d == 0) a.ws_lse[prow] = lse;
      }
    }
  }
  if (nctr == 1 || a.tickets == nullptr) return;

  // Fused merge of the splits: every workgroup of this (batch, KV head, row
  // block) publishes its partial and takes a ticket; the one that draws the
  // last ticket resets it to zero for the next call and merges all partials
  // in split order.  Publication: the partials above were stored at agent
  // scope (write-through, acknowledged once visible device-wide), and each
  // wave waits for those acknowledgements (vmcnt 0) before the barrier that
  // precedes the ticket, so no L2 write-back or invalidate is needed (an
  // agent-scope release / acquire fence pair costs about 20 us per call
  // here).  No workgroup waits for another, so nothing can stall on a
  // missing arrival.
  wait_vm_all();
  __syncthreads();
  int* flag = reinterpret_cast<int*>(lw + C::NW * 16);
  if (tid == 0) {
    uint32_t* t = a.tickets + ((int64_t)b * a.heads_kv + hk) * nrb + rb;
    const uint32_t prev = __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == (uint32_t)(nctr - 1);
    if (last) __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last ? 1 : 0;
  }
  __syncthreads();
  if (*flag == 0) return;
  // Merge: TPR threads per row, each owning DPT consecutive dims.  Per chunk
  // of 8 contributors a thread issues all its loads at once (their LSEs and
  // DPT-float pieces of their partial rows, agent-scope buffer loads), then
  // folds them in contributor order with a running max (natural-log
  // domain): one memory round trip per chunk.
  constexpr int TPR = C::NT / 16;
  constexpr int DPT = D / TPR;  // 8 / 4 / 2 / 1 floats
  static_assert(DPT >= 1 && DPT * TPR == D, "merge layout");
  constexpr int SC1 = 16;       // cache policy: agent scope (coherent across XCDs)
  const int cc = tid / TPR, d0 = (tid % TPR) * DPT;
  const int row = rb * 16 + cc;
  if (row >= rows) return;
  const int gg = row / a.seqlen_q, mm = row - gg * a.seqlen_q;
  const int hh = hk * group + gg;
  const int64_t plane = (int64_t)a.heads_q * a.seqlen_q;
  const int64_t prow = (int64_t)hh * a.seqlen_q + mm;
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(a.ws_lse, (short)0, 0x7FFFFFFF, 0x00020000);
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(a.ws_o, (short)0, 0x7FFFFFFF, 0x00020000);
  float M = kNegInf, den = 0.f, num[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) num[e] = 0.f;
  for (int k0 = 0; k0 < nctr; k0 += 8) {
    float ls[8], part[8][DPT];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t srow = (int64_t)(pfirst + min(k0 + u, nctr - 1) * pstep) * plane + prow;
      ls[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, (int)(srow * 4), 0, SC1));
      const int off = (int)((srow * D + d0) * 4);
      if constexpr (DPT >= 4) {
#pragma unroll
        for (int q = 0; q < DPT / 4; ++q) {
          // (bit_cast the whole result: subscripting the builtin's vector
          // directly compiles to one dword load splatted to all four.)
          const f32x4v w = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(ro, off + 16 * q, 0, SC1));
#pragma unroll
          for (int e = 0; e < 4; ++e) part[u][4 * q + e] = w[e];
        }
      } else if constexpr (DPT == 2) {
        typedef float f32x2v __attribute__((ext_vector_type(2)));
        const f32x2v w = __builtin_bit_cast(f32x2v, __builtin_amdgcn_raw_buffer_load_b64(ro, off, 0, SC1));
        part[u][0] = w[0];
        part[u][1] = w[1];
      } else {
        part[u][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ro, off, 0, SC1));
      }
    }
    float mc = M;
#pragma unroll
    for (int u = 0; u < 8; ++u) mc = fmaxf(mc, k0 + u < nctr ? ls[u] : kNegInf);
    const float mu = (mc == kNegInf) ? 0.f : mc;
    const float sc = (M == kNegInf) ? 0.f : __expf(M - mu);
    den *= sc;
#pragma unroll
    for (int e = 0; e < DPT; ++e) num[e] *= sc;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float w = (k0 + u < nctr && ls[u] != kNegInf) ? __expf(ls[u] - mu) : 0.f;
      den += w;
#pragma unroll
      for (int e = 0; e < DPT; ++e) num[e] += w * part[u][e];
    }
    M = mc;
  }
  const float inv = 1.f / (den == 0.f ? 1.f : den);
  S* op = reinterpret_cast<S*>(a.out) + b * a.out_stride[0] + hh * a.out_stride[1] + mm * a.out_stride[2] + d0;
#pragma unroll
  for (int e = 0; e < DPT; ++e) op[e] = EL::from_f(num[e] * inv);
  };  // segment

  // Which segment this workgroup runs.
  int sb, slen, sc0, scnt, snctr, spslot, spfirst, spstep;
  if (a.balanced) {
    // Balanced: the workgroups of one (KV head, row block) are shared out
    // over the sequences in proportion to their chunk counts, so a long
    // sequence among short ones is split finely and the CUs of short
    // sequences do not idle.  With G = num_splits * batch the target count,
    // sequence b gets g_b = max(1, floor(n_b * G / T)) workgroups (T = total
    // chunks; equal lengths give exactly num_splits each) and an even share
    // of its chunks per workgroup.  The sum stays within G + batch, the
    // workgroups launched per (KV head, row block); those past the last
    // sequence's share exit.  Sequence b's partial slots are the
    // consecutive workgroup slots [P_b, P_b + g_b).
    const int G = a.num_splits * a.batch;
    const int len_l = lane < a.batch ? seq_len(lane) : 0;
    const int nch_l = (len_l + C::CK - 1) / C::CK;
    int tot = nch_l;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
    const int gb = lane < a.batch ? max(1, tot > 0 ? (int)((int64_t)nch_l * G / tot) : 0) : 0;
    int incl = gb;  // inclusive prefix sum over lanes (sequences)
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o, 64);
      incl += lane >= o ? y : 0;
    }
    // b = number of sequences whose share ends at or before this slot.
    const int b = __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < a.batch && incl <= slot));
    if (b >= a.batch) return;
    const int g_b = __builtin_amdgcn_readlane(gb, b);
    const int p_b = __builtin_amdgcn_readlane(incl, b) - g_b;
    const int n = __builtin_amdgcn_readlane(nch_l, b);
    const int j = slot - p_b;
    const int per = n / g_b, extra = n % g_b;
    sb = b;
    slen = __builtin_amdgcn_readlane(len_l, b);
    sc0 = j * per + min(j, extra);
    scnt = per + (j < extra ? 1 : 0);
    snctr = g_b;
    spslot = slot;
    spfirst = p_b;
    spstep = 1;
  } else {
    // Per sequence: split `slot` of sequence blockIdx.y takes an even share
    // of its chunks; the partial slots of sequence b are s * batch + b.
    const int b = blockIdx.y;
    slen = seq_len(b);
    const int nch = (slen + C::CK - 1) / C::CK;
    const int per = nch / a.num_splits, extra = nch % a.num_splits;
    sb = b;
    sc0 = slot * per + min(slot, extra);
    scnt = per + (slot < extra ? 1 : 0);
    snctr = a.num_splits;
    spslot = slot * a.batch + b;
    spfirst = b;
    spstep = a.batch;
  }
  segment(sb, slen, sc0, scnt, snctr, spslot, spfirst, spstep);
}

// One wave per output row: out = sum_s w_s O_s / sum_s w_s with
// w_s = exp(lse_s - max_s lse_s).  Lane s reads lse_s (splits <= 64), the
// weights come from a wave reduction, then each lane sums its D/64 dims over
// all splits with the loads of up to 8 splits in flight at once.
template <typename Tag, int D>
__global__ __launch_bounds__(256) void decode_combine2_kernel(DecodeArgs a) {
  using EL = Elem<Tag>;
  constexpr int DPL = D / 64 > 0 ? D / 64 : 1;  // dims per lane (lanes >= D idle when D < 64)
  const int rows = a.batch * a.heads_q * a.seqlen_q;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t plane = rows;
  const int ns = a.num_splits;
  const float ls = lane < ns ? a.ws_lse[lane * plane + row] : kNegInf;
  float M = ls;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  const float Mu = (M == kNegInf) ? 0.f : M;
  const float w = (ls == kNegInf) ? 0.f : __expf(ls - Mu);
  float den = w;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  const int d0 = lane * DPL;
  const bool active = d0 < D;
  float num[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) num[e] = 0.f;
  const float* src = a.ws_o + (int64_t)row * D + (active ? d0 : 0);
  for (int s0 = 0; s0 < ns; s0 += 8) {
    float part[8][DPL];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int s = min(s0 + u, ns - 1);
#pragma unroll
      for (int e = 0; e < DPL; ++e) part[u][e] = src[(int64_t)s * plane * D + e];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float ws = __shfl(w, min(s0 + u, 63), 64);
      const float wu = (s0 + u < ns) ? ws : 0.f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) num[e] += wu * part[u][e];
    }
  }
  if (!active) return;
  const float inv = 1.f / (den == 0.f ? 1.f : den);
  const int mm = row % a.seqlen_q;
  const int hh = (row / a.seqlen_q) % a.heads_q;
  const int bb = row / (a.seqlen_q * a.heads_q);
  uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + bb * a.out_stride[0] + hh * a.out_stride[1] + mm * a.out_stride[2];
#pragma unroll
  for (int e = 0; e < DPL; ++e) op[d0 + e] = EL::from_f(num[e] * inv);
}

}  // namespace fa
