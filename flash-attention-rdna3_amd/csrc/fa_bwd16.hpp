// fa_bwd16.hpp - dK/dV and dQ kernels specialised for 16-bit inputs, D <= 128.
//
// Same math as bwd_dkdv_kernel / bwd_dq_kernel (reference
// kernels/backward.py:49-322, _common.py:347-508), with the gfx950 layout of
// fa_fwd16.hpp:
//  * every LDS tile is row-major with an XOR chunk swizzle; operands that
//    contract over the tile row (dO^T, Q^T for dK/dV; K^T for dQ) are read
//    with ds_read_b64_tr_b16 from the same row-major tile that feeds the
//    row-contracting MFMAs, so each tile is loaded and stored once;
//  * blocks strictly inside the visible region skip the per-score masking;
//  * LSE is staged as lse*log2(e), with +inf for rows that must contribute
//    nothing (past the sequence end, or no visible key), so
//    P = exp2(s*c - lse2) is 0 there without a select.
#pragma once

#include <type_traits>

#include "fa_internal.hpp"
#include "fa_tiles.hpp"

namespace fa {

__device__ inline float lse2_of(float lse) { return lse == kNegInf ? __builtin_inff() : lse * kLog2e; }

// Elements of the dS scratch before sequence b's regions.  WAVE: called by
// a whole wave (every lane active); for varlen, lane i then sums the regions
// of sequences i, i + 64, ... below b (one round trip per 64 sequences) and a
// wave reduction adds the lanes; otherwise one thread walks them in turn.
// (A batch of 400 sequences: walking them one by one took the dK/dV pass
// 3.36 ms and dQ 1.88 ms, against 0.61 and 0.37 ms with the wave sum.)
template <bool WAVE>
__device__ inline int64_t ds_seq_base(const fa_bwd_params& p, int b, int sq, int sk) {
  const fa_fwd_params& f = p.fwd;
  if (!f.cu_seqlens_q) return (int64_t)b * f.heads_q * ds_region_elems(sq, sk);
  const int lane = WAVE ? (int)(threadIdx.x & 63) : 0;
  const int step = WAVE ? 64 : 1;
  int64_t acc = 0;
  for (int i = lane; i - lane < b; i += step) {
    if (i < b) {
      int s0, l0, s1, l1;
      bounded_seq(f.cu_seqlens_q, i, f.total_q, s0, l0);
      bounded_seq(f.cu_seqlens_k, i, f.total_k, s1, l1);
      acc += ds_region_elems(l0, l1);
    }
  }
  if constexpr (WAVE) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
  }
  return acc * f.heads_q;
}

// Start (elements) of the dS region of query head hq of a sequence whose
// regions start at `base`, or -1 when it would not fit (varlen lengths
// inconsistent with max_seqlen / total): then nothing is stored there or
// read from it.
__device__ inline int64_t ds_region_at(const fa_bwd_params& p, int64_t base, int hq, int sq, int sk) {
  const int64_t start = base + (int64_t)hq * ds_region_elems(sq, sk);
  const int64_t cap = (p.ds_workspace_bytes - 1024) / 2;
  return (start + ds_region_elems(sq, sk) <= cap) ? start : -1;
}


// ---------------------------------------------------------------------------
// dK / dV: each wave owns 32 keys (lane axis of S = Q K^T).
// ---------------------------------------------------------------------------
// A workgroup owns BN = 128 keys (32 per wave of a half) and splits their
// query range in two: waves 0-3 walk the first half of the query steps,
// waves 4-7 the second, each half through its own double-buffered Q / dO
// stages.  The K and V operands of the 128 keys are parked once in LDS (they
// are shared by the two waves that own the same keys), which keeps a wave
// under 256 VGPRs so the 8-wave workgroup runs at two waves per SIMD.  The
// two dK / dV partial sums are added through LDS at the end in a fixed order.
template <int D>
struct Dkdv16Cfg {
  static constexpr int NQ = 4;                          // key quarters (waves per half)
  static constexpr int NW = 2 * NQ;
  static constexpr int NT = 64 * NW;
  static constexpr int NTH = 64 * NQ;
  static constexpr int BN = 32 * NQ;
  static constexpr int BMQ = 32;
  static constexpr int QT = BMQ * D;                    // elements per Q / dO tile
  static constexpr int STAGE_BYTES = 2 * QT * 2 + 2 * BMQ * 4;
  static constexpr int HALF_BYTES = 2 * STAGE_BYTES;
  static constexpr int PARK_BYTES = 2 * BN * D * 2;     // K then V, [key quarter][32][D]
  static constexpr int LOOP_BYTES = 2 * HALF_BYTES + PARK_BYTES;
  static constexpr int MERGE_BYTES = NQ * 2 * (D / 32) * 16 * 64 * 4;
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
  static constexpr int NSTEP = D / 16;
  static constexpr int NPV = BMQ / 16;
  static constexpr int NDB = D / 32;
};

template <typename Tag, int D, int MODE>
__global__ __launch_bounds__(512, 1) void dkdv16_kernel(fa_bwd_params p, int num_n_blocks) {
  using C = Dkdv16Cfg<D>;
  using EL = Elem<Tag>;
  using S = uint16_t;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const fa_fwd_params& f = p.fwd;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qhalf = wave8 / C::NQ;        // which half of the query steps
  const int wave = wave8 % C::NQ;         // key quarter
  const int htid = tid % C::NTH;
  const int h = lane >> 5, l32 = lane & 31;
  const int bhk_count = f.batch * f.heads_kv;
  // Low key blocks first: under causal masking they see the most query rows.
  const int nblk = blockIdx.x / bhk_count;
  const int bhk = blockIdx.x - nblk * bhk_count;
  const int b = bhk / f.heads_kv, hk = bhk - b * f.heads_kv;
  const int group = f.heads_q / f.heads_kv;

  int q_start = 0, sq = f.seqlen_q, k_start = 0, sk = f.seqlen_k;
  if (f.cu_seqlens_q) {
    bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
    bounded_seq(f.cu_seqlens_k, b, f.total_k, k_start, sk);
  }
  const int n0 = nblk * C::BN;
  if (n0 >= sk || num_n_blocks <= 0) return;

  const S* kbase = reinterpret_cast<const S*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] +
                   (int64_t)k_start * f.k_stride[2];
  const S* vbase = reinterpret_cast<const S*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] +
                   (int64_t)k_start * f.v_stride[2];
  const int n0w = n0 + 32 * wave;
  const int ncols = min(32, sk - n0w);
  const int n = n0w + l32;
  const bool nvalid = n < sk;

  // Park this key quarter's K / V operands (the lane layout of the MFMA B
  // operand) in LDS; the first barrier of the query loop publishes them.
  S* const klds = reinterpret_cast<S*>(smem_raw + 2 * C::HALF_BYTES) + wave * 32 * D;
  S* const vlds = klds + C::BN * D;
  // The parked tiles are this wave's 32 key rows, row-major and swizzled:
  // they go HBM -> LDS by DMA (rows past the sequence end read as zeros) in
  // the same round trip as the first Q / dO stage.
  if (qhalf == 0) {
    DmaSwzTile<32, D, 64> pk, pv;
    pk.init(f.k_stride[2], lane);
    pv.init(f.v_stride[2], lane);
    pk.load(rows_rsrc_words<D>(kbase + (int64_t)n0w * f.k_stride[2], f.k_stride[2], ncols), lds_addr(klds), 0);
    pv.load(rows_rsrc_words<D>(vbase + (int64_t)n0w * f.v_stride[2], f.v_stride[2], ncols), lds_addr(vlds), 0);
  }

  f32x16 dk[C::NDB], dv[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) { dk[i] = zero16(); dv[i] = zero16(); }

  // Q / dO tiles go HBM -> LDS directly when the tile is a whole number of
  // 16-byte chunks per thread of a half (D >= 64); otherwise through registers.
  constexpr bool DMA = (C::BMQ * D / 8) % C::NTH == 0;
  using RegTile = BufSwzTile<C::BMQ, D, C::NTH>;
  using DTile = DmaSwzTile<C::BMQ, (DMA ? D : 64), C::NTH>;
  RegTile qt, gt;
  DTile qd, gd;
  if constexpr (DMA) {
    qd.init(f.q_stride[2], htid);
    gd.init(p.dout_stride[2], htid);
  } else {
    qt.init(f.q_stride[2], htid);
    gt.init(p.dout_stride[2], htid);
  }
  unsigned char* const hsmem = smem_raw + qhalf * C::HALF_BYTES;
  const uint32_t lds0 = lds_addr(hsmem);
  const int nlast = min(n0 + C::BN, sk) - 1;

  const int64_t ds_base = p.ds_workspace != nullptr ? ds_seq_base<true>(p, b, sq, sk) : 0;
  for (int g = 0; g < group; ++g) {
    const int hq = hk * group + g;
    const Mods md = make_mods(f, b, hq, sq, sk);
    const float c = md.scale_log2;
    const S* qbase = reinterpret_cast<const S*>(f.q) + b * f.q_stride[0] + hq * f.q_stride[1] +
                     (int64_t)q_start * f.q_stride[2];
    const S* gbase = reinterpret_cast<const S*>(p.dout) + b * p.dout_stride[0] + hq * p.dout_stride[1] +
                     (int64_t)q_start * p.dout_stride[2];
    const float* lbase = f.lse + b * f.lse_stride[0] + hq * f.lse_stride[1] + (int64_t)q_start * f.lse_stride[2];
    const float* dbase = p.delta + b * p.delta_stride[0] + hq * p.delta_stride[1] +
                         (int64_t)q_start * p.delta_stride[2];
    const int64_t qs = f.q_stride[2], gs = p.dout_stride[2];

    int mlo = 0, mhi = sq;
    if (f.causal) mlo = max(mlo, n0 - md.off);
    if (f.window_right >= 0) mlo = max(mlo, n0 - md.off - f.window_right);
    if (f.window_left >= 0) mhi = min(mhi, nlast - md.off + f.window_left + 1);
    mlo = max(mlo, 0) / C::BMQ * C::BMQ;
    const int nsteps = mhi > mlo ? (mhi - mlo + C::BMQ - 1) / C::BMQ : 0;
    // Query steps [0, nh0) go to half 0, [nh0, nsteps) to half 1; both
    // halves run nh0 iterations so their barriers line up.
    const int nh0 = (nsteps + 1) / 2;
    const int my_first = qhalf == 0 ? 0 : nh0;
    const int my_count = qhalf == 0 ? nh0 : nsteps - nh0;

    float lreg = 0.f, dreg = 0.f;  // this thread's lse2 / delta for the next stage
    auto load_stage = [&](int m0, int st) {
      const int rows = min(C::BMQ, sq - m0);
      if constexpr (DMA) {
        const uint32_t base = lds0 + (uint32_t)(st * C::STAGE_BYTES);
        qd.load(rows_rsrc_words<D>(qbase + (int64_t)m0 * qs, qs, rows), base, wave);
        gd.load(rows_rsrc_words<D>(gbase + (int64_t)m0 * gs, gs, rows), base + C::QT * 2u, wave);
      } else {
        qt.load(rows_rsrc<D>(qbase + (int64_t)m0 * qs, qs, rows));
        gt.load(rows_rsrc<D>(gbase + (int64_t)m0 * gs, gs, rows));
      }
      if (htid < C::BMQ) {
        const int m = min(m0 + htid, sq - 1);
        lreg = lbase[(int64_t)m * f.lse_stride[2]];
        dreg = dbase[(int64_t)m * p.delta_stride[2]];
      }
    };
    auto store_stage = [&](int st, int m0) {
      unsigned char* base = hsmem + st * C::STAGE_BYTES;
      S* sp = reinterpret_cast<S*>(base);
      if constexpr (!DMA) {
        qt.store(sp, htid);
        gt.store(sp + C::QT, htid);
      }
      if (htid < C::BMQ) {
        float* lf = reinterpret_cast<float*>(base + 2 * C::QT * 2);
        const float l2v = (m0 + htid < sq) ? lse2_of(lreg) : __builtin_inff();
        // MODE 0 seeds the score accumulators with -lse2/c and -delta (the
        // MFMAs then produce s - lse2/c and dP - delta directly); the other
        // modes need the raw scores and keep lse2 / delta.
        // MODE 3 keeps cap2 - lse2: exp2(x - lse2) is then one FMA on the
        // softcap's r away (x = cap2 - 2 cap2 r).
        lf[htid] = (MODE == 0) ? -l2v / md.scale_log2 : (MODE == 3) ? md.cap2 - l2v : l2v;
        lf[C::BMQ + htid] = (MODE != 2) ? -dreg : dreg;
      }
    };

    // dS row of this lane's key in the score-gradient scratch, read back by
    // dqs16_kernel (ds_on: this query head's dS is stored; wave-uniform).
    // Lanes past the last key write to the scratch's slack instead, so every
    // wave of a storing step issues the same stores (the end-of-step wait
    // below counts them).
    bool ds_on = false;
    S* dsn = nullptr;
    S* ds_dump = nullptr;
    if (p.ds_workspace != nullptr) {
      const int64_t region = ds_region_at(p, ds_base, hq, sq, sk);
      ds_on = region >= 0;
      S* const ws = reinterpret_cast<S*>(p.ds_workspace);
      // row n % 64 of the key block's tiles; + (query block) * tile
      //   + (query sub-tile) * sub-tile + q % 32
      dsn = ws + (ds_on ? region : 0) + (int64_t)(n / kDsTileKeys) * ds_qblocks(sq) * kDsTileElems +
            (n % kDsTileKeys) * kDsSubQueries;
      ds_dump = ws + (p.ds_workspace_bytes - 1024) / 2;
    }
    const VisBounds kvb = key_block_bounds(md, n0w, ncols);
    // Visible rows of this lane's key, relative to the row of slot 0.
    int rlo, rhi;
    row_bounds(md, n, rlo, rhi);
    if (my_count > 0) {
      const int m_first = mlo + my_first * C::BMQ;
      load_stage(m_first, 0);
      store_stage(0, m_first);
    }
    wait_vm_all();
    __syncthreads();
    for (int t = 0; t < nh0; ++t) {
      const int m0 = mlo + (my_first + t) * C::BMQ;
      const int st = t & 1;
      if (t + 1 < my_count) load_stage(m0 + C::BMQ, st ^ 1);

      const int vis = t < my_count ? bounds_vis(kvb, m0 + md.off, min(m0 + C::BMQ, sq) - 1 + md.off) : 0;
      if (vis) {
        const unsigned char* base = hsmem + st * C::STAGE_BYTES;
        const S* Qs = reinterpret_cast<const S*>(base);
        const S* Gs = Qs + C::QT;
        const float* L2 = reinterpret_cast<const float*>(base + 2 * C::QT * 2);
        const float* DL = L2 + C::BMQ;

        f32x16 sacc, pacc;
        float dl[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(L2 + 8 * q4 + 4 * h);
          const f32x4 d = *reinterpret_cast<const f32x4*>(DL + 8 * q4 + 4 * h);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // The dP accumulator starts at -delta except under dropout (whose
            // dP is scaled per score first); the score accumulator starts at
            // -lse2/c in MODE 0, where no modifier needs the raw score.
            if constexpr (MODE == 0) sacc[4 * q4 + r] = a[r];
            if constexpr (MODE != 2) pacc[4 * q4 + r] = d[r];
            else dl[4 * q4 + r] = d[r];
          }
        }
        if constexpr (MODE != 0) sacc = zero16();
        if constexpr (MODE == 2) pacc = zero16();
#pragma unroll
        for (int s = 0; s < C::NSTEP; ++s) {
          sacc = EL::mma(swz_op<D>(Qs, l32, 2 * s + h), swz_op<D>(klds, l32, 2 * s + h), sacc);
          pacc = EL::mma(swz_op<D>(Gs, l32, 2 * s + h), swz_op<D>(vlds, l32, 2 * s + h), pacc);
        }
        // The LDS operand reads of the score MFMAs go two MFMAs ahead (the
        // four-ahead schedule spilled VGPRs: measured config 5's MODE 3
        // dK/dV 766 -> 718 us, config 2's MODE 0 88.4 -> 87.9 us).
        if constexpr (MODE == 0 || MODE == 3) sched_read_ahead<2 * C::NSTEP, 2, 2, 8>();
        // The fully visible case (no modifiers) is its own straight-line
        // body: a per-element choice would become one branch per score.
        // MASK: the block is partly visible (vis == 1); fully visible blocks
        // skip the per-score visibility test.
        const Span rs = make_span(rlo, rhi, m0 + 4 * h);
        auto scores = [&](auto plain_t, auto cap_t, auto bias_t, auto alibi_t, auto mask_t) {
          (void)plain_t;  // the dK/dV body has no separate plain path
          constexpr bool CAP = decltype(cap_t)::value;
          constexpr bool MASK = decltype(mask_t)::value;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float pv, tc = 0.f, capq = 0.f;
            if constexpr (MODE == 0) {
              // sacc = s - lse2/c, pacc = dP - delta (seeded accumulators).
              pv = __builtin_amdgcn_exp2f(sacc[i] * c);
              if constexpr (MASK) pv = in_span(rs, acc_row(i, 0)) ? pv : 0.f;
            } else if constexpr (MODE == 3) {
              // L2 holds cap2 - lse2; capq = (1 - tanh^2) / 4 (the 4 is
              // applied to dK at the end).
              const float r = softcap_r(md, sacc[i]);
              pv = __builtin_amdgcn_exp2f(__builtin_fmaf(md.cap2_m2, r, L2[8 * (i / 4) + 4 * h + (i % 4)]));
              capq = __builtin_fmaf(-r, r, r);
              if constexpr (MASK) pv = in_span(rs, acc_row(i, 0)) ? pv : 0.f;
            } else {
              const int m = m0 + acc_row(i, h);
              const float x = score_m<CAP, decltype(bias_t)::value, decltype(alibi_t)::value>(md, sacc[i], m, n, tc);
              // lse2 of this score's row, read here rather than held across
              // the stage (register pressure of the modifier variants).
              const float l2i = L2[8 * (i / 4) + 4 * h + (i % 4)];
              pv = __builtin_amdgcn_exp2f(x - l2i);
              if constexpr (MASK) pv = in_span(rs, acc_row(i, 0)) ? pv : 0.f;
            }
            float dp = pacc[i], pd = pv;
            if constexpr (MODE == 2) {
              if (md.drop_p > 0.f) {
                const bool keep = dropout_keep(md, m0 + acc_row(i, h), n);
                pd = keep ? pv * md.drop_scale : 0.f;
                dp = keep ? dp * md.drop_scale : 0.f;
              }
            }
            float ds = (MODE != 2) ? pv * dp : pv * (dp - dl[i]);
            if constexpr (MODE == 3) ds *= capq;
            else if constexpr (CAP) ds *= (1.f - tc * tc);
            sacc[i] = pd;
            pacc[i] = ds;
          }
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        if constexpr (MODE == 3) {
          // softcap only
          if (vis == 1) scores(F_{}, T_{}, std::integral_constant<int, 0>{}, F_{}, T_{});
          else scores(F_{}, T_{}, std::integral_constant<int, 0>{}, F_{}, F_{});
        } else if constexpr (MODE >= 1) {
          if (vis == 1) dispatch_mods(md, [&](auto a, auto b_, auto c_) { scores(F_{}, a, b_, c_, T_{}); });
          else dispatch_mods(md, [&](auto a, auto b_, auto c_) { scores(F_{}, a, b_, c_, F_{}); });
        } else {
          if (vis == 2) scores(T_{}, F_{}, std::integral_constant<int, 0>{}, F_{}, F_{});
          else scores(F_{}, F_{}, std::integral_constant<int, 0>{}, F_{}, T_{});
        }
        s16x8 pb[C::NPV], sb[C::NPV];
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) {
          pb[j] = pack_op<Tag>(sacc, j);
          sb[j] = pack_op<Tag>(pacc, j);
        }
#pragma unroll
        for (int j = 0; j < C::NPV; ++j)
#pragma unroll
          for (int db = 0; db < C::NDB; ++db) {
            dv[db] = EL::mma(tr_op_rowmap<D>(Gs, 0, 32 * db, j, lane), pb[j], dv[db]);
            dk[db] = EL::mma(tr_op_rowmap<D>(Qs, 0, 32 * db, j, lane), sb[j], dk[db]);
          }
        // Two ahead here too (config 2's dK/dV 90.3 -> 89.1 us against four).
        if constexpr (MODE == 0) sched_read_ahead<2 * C::NPV * C::NDB, 2, 2>();
        if (t + 1 < my_count) store_stage(st ^ 1, m0 + C::BMQ);
        if (ds_on) {
          // Operand j of lane half h holds rows 16j + 4h + e and
          // 16j + 8 + 4h + e (e < 4) of this lane's key.  One permlane32
          // swap per dword gives half h rows 16h .. 16h + 15 (operand 0 of
          // half 1 trades with operand 1 of half 0): 32 contiguous bytes of
          // the dS row, two 16-byte stores.  Issued after the stage's
          // register loads are consumed (a wait for those would also wait
          // for these stores).
          static_assert(C::NPV == 2, "one 32-row query step per dS store");
          u32x4 w0 = __builtin_bit_cast(u32x4, sb[0]), w1 = __builtin_bit_cast(u32x4, sb[1]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const auto r = __builtin_amdgcn_permlane32_swap(w0[i], w1[i], false, false);
            w0[i] = r[0];
            w1[i] = r[1];
          }
          static_assert(C::BMQ == kDsSubQueries, "a query step is one dS sub-tile");
          S* const at = !nvalid ? ds_dump
                                : dsn + (int64_t)(m0 / kDsTileQueries) * kDsTileElems +
                                      (m0 % kDsTileQueries) / kDsSubQueries * kDsSubElems + 16 * h;
          // Plain (temporal) stores: measured dQ 42.0 -> 39.4 us at config
          // 2 against nontemporal stores, dK/dV unchanged (a 143 MB dS
          // stream can stay in the 256 MiB memory-side cache for the dQ
          // pass).
          *reinterpret_cast<u32x4*>(at) = u32x4{w0[0], w0[1], w1[0], w1[1]};
          *reinterpret_cast<u32x4*>(at + 8) = u32x4{w0[2], w0[3], w1[2], w1[3]};
        }
      } else if (t + 1 < my_count) {
        store_stage(st ^ 1, m0 + C::BMQ);
      }
      // The next stage's loads must have landed; this step's dS stores,
      // issued after them, may still be in flight (vector memory operations
      // complete in issue order, so vmcnt <= #stores covers the loads).
      if (ds_on && vis) wait_vm<2>();
      else wait_vm_all();
      __syncthreads();
    }
  }

  // dK / dV = first query half + second query half, added in that order.
  {
    float* ow = reinterpret_cast<float*>(smem_raw);
    __syncthreads();  // the parked operands and stages are dead from here
    if (qhalf == 1) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        park_acc(ow + ((wave * 2 + 0) * C::NDB + db) * 1024, lane, dk[db]);
        park_acc(ow + ((wave * 2 + 1) * C::NDB + db) * 1024, lane, dv[db]);
      }
    }
    __syncthreads();
    if (qhalf == 1) return;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      dk[db] += unpark_acc(ow + ((wave * 2 + 0) * C::NDB + db) * 1024, lane);
      dv[db] += unpark_acc(ow + ((wave * 2 + 1) * C::NDB + db) * 1024, lane);
    }
  }

  // Whole-row dK / dV stores through this wave's two LDS blocks of the
  // merge above (read back already).
  S* dkr0 = reinterpret_cast<S*>(p.dk) + b * p.dk_stride[0] + hk * p.dk_stride[1] +
            (int64_t)(k_start + n0w) * p.dk_stride[2];
  S* dvr0 = reinterpret_cast<S*>(p.dv) + b * p.dv_stride[0] + hk * p.dv_stride[1] +
            (int64_t)(k_start + n0w) * p.dv_stride[2];
  const float sc = f.softmax_scale * (MODE == 3 ? 4.f : 1.f);
  unsigned char* const wblk = smem_raw + wave * 2 * C::NDB * 4096;
  store_rows_staged<Tag, D>(dk, sc, reinterpret_cast<uint16_t*>(wblk), dkr0, p.dk_stride[2], ncols, lane);
  store_rows_staged<Tag, D>(dv, 1.f, reinterpret_cast<uint16_t*>(wblk + C::NDB * 4096), dvr0, p.dv_stride[2],
                            ncols, lane);
}

// ---------------------------------------------------------------------------
// dQ: each wave owns 32 queries (lane axis of S^T = K Q^T).
// ---------------------------------------------------------------------------
template <int D>
struct Dq16Cfg {
  // 128 query rows (a row quarter of 32 per wave) with the key range split in
  // two halves of 4 waves each, merged through LDS (same layout and reasons
  // as the forward kernel).
  static constexpr int NQ = 4;
  static constexpr int NW = 2 * NQ;
  static constexpr int NT = 64 * NW;
  static constexpr int NTH = 64 * NQ;
  static constexpr int BM = 32 * NQ;
  static constexpr int BN = (D <= 64) ? 64 : 32;
  static constexpr int KT = BN * D;
  static constexpr int STAGE = 2 * KT;  // K, V
  static constexpr int HALF = 2 * STAGE;
  static constexpr int LOOP_BYTES = 2 * HALF * 2;
  static constexpr int MERGE_BYTES = NQ * (D / 32) * 16 * 64 * 4;
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
  static constexpr int NSTEP = D / 16;
  static constexpr int NKB = BN / 32;
  static constexpr int NPV = BN / 16;
  static constexpr int NDB = D / 32;
};

// One 128-row query block (mb_rev counts from the last block) of (sequence,
// query head) bh; fuse_delta computes delta here.
template <typename Tag, int D, int MODE>
__device__ inline void dq16_block(const fa_bwd_params& p, int num_m_blocks, int mb_rev, int bh, int fuse_delta) {
  using C = Dq16Cfg<D>;
  using EL = Elem<Tag>;
  using S = uint16_t;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  S* smem = reinterpret_cast<S*>(smem_raw);
  const fa_fwd_params& f = p.fwd;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int khalf = wave8 / C::NQ;
  const int wave = wave8 % C::NQ;
  const int htid = tid % C::NTH;
  const int h = lane >> 5, l32 = lane & 31;
  const int b = bh / f.heads_q, hq = bh - b * f.heads_q;
  const int hk = hq / (f.heads_q / f.heads_kv);
  const int mblk = num_m_blocks - 1 - mb_rev;  // heaviest causal blocks first

  int q_start = 0, sq = f.seqlen_q, k_start = 0, sk = f.seqlen_k;
  if (f.cu_seqlens_q) {
    bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
    bounded_seq(f.cu_seqlens_k, b, f.total_k, k_start, sk);
  }
  const int m0 = mblk * C::BM;
  if (m0 >= sq) return;

  const S* kbase = reinterpret_cast<const S*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] +
                   (int64_t)k_start * f.k_stride[2];
  const S* vbase = reinterpret_cast<const S*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] +
                   (int64_t)k_start * f.v_stride[2];
  const int64_t ks = f.k_stride[2], vs = f.v_stride[2];
  const Mods md = make_mods(f, b, hq, sq, sk);
  const float c = md.scale_log2;

  const int mlast = min(m0 + C::BM, sq) - 1;
  int lo = 0, hi = sk;
  if (f.causal) hi = min(hi, mlast + md.off + 1);
  if (f.window_right >= 0) hi = min(hi, mlast + md.off + f.window_right + 1);
  if (f.window_left >= 0) lo = max(0, m0 + md.off - f.window_left);
  lo = lo / C::BN * C::BN;
  const int ntiles = hi > lo ? (hi - lo + C::BN - 1) / C::BN : 0;

  const int m0w = m0 + 32 * wave;
  const int mrows = min(32, sq - m0w);
  const int m = m0w + l32;
  const bool mvalid = m < sq;
  s16x8 qop[C::NSTEP], gop[C::NSTEP];
  float lse2 = __builtin_inff(), dlt = 0.f;

  f32x16 dq[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dq[i] = zero16();

  constexpr bool DMA = (C::BN * D / 8) % C::NTH == 0;
  BufSwzTile<C::BN, D, C::NTH> kt, vt;
  DmaSwzTile<C::BN, (DMA ? D : 64), C::NTH> kd, vd;
  if constexpr (DMA) {
    kd.init(ks, htid);
    vd.init(vs, htid);
  } else {
    kt.init(ks, htid);
    vt.init(vs, htid);
  }
  const int nh0 = (ntiles + 1) / 2;
  const int my_first = khalf == 0 ? 0 : nh0;
  const int my_count = khalf == 0 ? nh0 : ntiles - nh0;
  S* const hsmem = smem + khalf * C::HALF;
  const uint32_t lds0 = lds_addr(hsmem);
  auto load_stage = [&](int n0, int st) {
    const int rows = min(C::BN, sk - n0);
    if constexpr (DMA) {
      const uint32_t base = lds0 + (uint32_t)(st * C::STAGE) * 2u;
      kd.load(rows_rsrc_words<D>(kbase + (int64_t)n0 * ks, ks, rows), base, wave);
      vd.load(rows_rsrc_words<D>(vbase + (int64_t)n0 * vs, vs, rows), base + C::KT * 2u, wave);
    } else {
      kt.load(rows_rsrc<D>(kbase + (int64_t)n0 * ks, ks, rows));
      vt.load(rows_rsrc<D>(vbase + (int64_t)n0 * vs, vs, rows));
    }
  };
  auto store_stage = [&](int st) {
    if constexpr (!DMA) {
      S* base = hsmem + st * C::STAGE;
      kt.store(base, htid);
      vt.store(base + C::KT, htid);
    }
  };

  const VisBounds qvb = row_block_bounds(md, m0w, mrows);
  if (my_count > 0) {
    load_stage(lo + my_first * C::BN, 0);
    store_stage(0);
  }
  // The row operands load after the first K / V stage is issued: one round
  // trip to memory for both.
  {
    const int mm = mvalid ? m : 0;
    const S* qr = reinterpret_cast<const S*>(f.q) + b * f.q_stride[0] + hq * f.q_stride[1] +
                  (int64_t)(q_start + mm) * f.q_stride[2] + 8 * h;
    const S* gr = reinterpret_cast<const S*>(p.dout) + b * p.dout_stride[0] + hq * p.dout_stride[1] +
                  (int64_t)(q_start + mm) * p.dout_stride[2] + 8 * h;
    // With fuse_delta, O is loaded in the same chunks as dO (issued with the
    // operand loads, one round trip) for delta = rowsum(O * dO).
    const S* orow = reinterpret_cast<const S*>(fuse_delta ? f.out : f.q) +
                    (fuse_delta ? b * f.out_stride[0] + hq * f.out_stride[1] + (int64_t)(q_start + mm) * f.out_stride[2]
                                : b * f.q_stride[0] + hq * f.q_stride[1] + (int64_t)(q_start + mm) * f.q_stride[2]) +
                    8 * h;
    s16x8 oop[C::NSTEP];
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      qop[s] = load_op<Tag>(qr + 16 * s);
      gop[s] = load_op<Tag>(gr + 16 * s);
      oop[s] = load_op<Tag>(orow + 16 * s);
    }
    const float l = f.lse[b * f.lse_stride[0] + hq * f.lse_stride[1] + (int64_t)(q_start + mm) * f.lse_stride[2]];
    float* const drow = p.delta + b * p.delta_stride[0] + hq * p.delta_stride[1] + (int64_t)(q_start + mm) * p.delta_stride[2];
    float d;
    if (fuse_delta) {
      // delta = rowsum(O * dO) for this lane's row, from the same 16-byte
      // chunks the dO operand holds (reference backward.py:18-46); written
      // for the dK/dV kernel, which runs after this one.
      wait_vm_all();
      float acc = 0.f;
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += EL::to_f((uint16_t)oop[s][e]) * EL::to_f((uint16_t)gop[s][e]);
      d = half_sum(acc);
      if (mvalid && khalf == 0 && h == 0) *drow = d;
    } else {
      d = *drow;
    }
    wait_vm_all();
    if (mvalid) {
      lse2 = lse2_of(l);
      dlt = d;
    } else {
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s) { qop[s] = zero_op<Tag>(); gop[s] = zero_op<Tag>(); }
    }
  }

  // Visible keys of this lane's row, and the constants of the score loop:
  // cap2 - lse2 (MODE 3: exp2(x - lse2) is one FMA on the softcap's r) and
  // the dP accumulator seed (-delta in MODES 1 and 3, so the MFMAs produce
  // dP - delta).
  int klo, khi;
  key_bounds(md, m, klo, khi);
  const float capl = md.cap2 - lse2;
  f32x16 dseed;
#pragma unroll
  for (int i = 0; i < 16; ++i) dseed[i] = (MODE == 1 || MODE == 3) ? -dlt : 0.f;

  wait_vm_all();
  __syncthreads();
  for (int t = 0; t < nh0; ++t) {
    const int n0 = lo + (my_first + t) * C::BN;
    const int st = t & 1;
    if (t + 1 < my_count) load_stage(n0 + C::BN, st ^ 1);
    const int vis = t < my_count ? bounds_vis(qvb, n0, n0 + C::BN - 1) : 0;
    if (vis) {
      const S* Ks = hsmem + st * C::STAGE;
      const S* Vs = Ks + C::KT;
      f32x16 sacc[C::NKB], pacc[C::NKB];
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) { sacc[kb2] = zero16(); pacc[kb2] = dseed; }
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s)
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
          sacc[kb2] = EL::mma(swz_op<D>(Ks, kb2 * 32 + l32, 2 * s + h), qop[s], sacc[kb2]);
          pacc[kb2] = EL::mma(swz_op<D>(Vs, kb2 * 32 + l32, 2 * s + h), gop[s], pacc[kb2]);
        }
      if constexpr (MODE == 0) sched_read_ahead<2 * C::NSTEP * C::NKB, 4>();
      // MASK: the tile is partly visible (vis == 1); fully visible tiles
      // skip the per-score visibility test.
      const Span ks = make_span(klo, khi, n0 + 4 * h);
      auto scores = [&](auto plain_t, auto cap_t, auto bias_t, auto alibi_t, auto mask_t) {
        constexpr bool plain = decltype(plain_t)::value;
        constexpr bool CAP = decltype(cap_t)::value;
        constexpr bool MASK = decltype(mask_t)::value;
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            float pv, tc = 0.f, capq = 0.f;
            const int nn = n0 + kb2 * 32 + acc_row(i, h);
            if constexpr (plain) {
              pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb2][i], c, -lse2));
            } else if constexpr (MODE == 3) {
              // capq = (1 - tanh^2) / 4 (the 4 is applied to dQ at the end)
              const float r = softcap_r(md, sacc[kb2][i]);
              pv = __builtin_amdgcn_exp2f(__builtin_fmaf(md.cap2_m2, r, capl));
              capq = __builtin_fmaf(-r, r, r);
              if constexpr (MASK) pv = in_span(ks, kb2 * 32 + acc_row(i, 0)) ? pv : 0.f;
            } else {
              const float x = score_m<CAP, decltype(bias_t)::value, decltype(alibi_t)::value>(md, sacc[kb2][i], m, nn, tc);
              pv = __builtin_amdgcn_exp2f(x - lse2);
              if constexpr (MASK) pv = in_span(ks, kb2 * 32 + acc_row(i, 0)) ? pv : 0.f;
            }
            float dp = pacc[kb2][i];
            float ds;
            if constexpr (MODE == 1 || MODE == 3) {
              ds = pv * dp;  // dp - delta: the accumulator was seeded with -delta
            } else {
              // (MODE 0 keeps a zero seed: the seed's registers, live across
              // the loop, cost it more than the subtraction, measured)
              if constexpr (MODE == 2) {
                if (md.drop_p > 0.f) dp = dropout_keep(md, m, nn) ? dp * md.drop_scale : 0.f;
              }
              ds = pv * (dp - dlt);
            }
            if constexpr (MODE == 3) ds *= capq;
            else if constexpr (CAP) ds *= (1.f - tc * tc);
            sacc[kb2][i] = ds;
          }
      };
      using T_ = std::true_type;
      using F_ = std::false_type;
      if constexpr (MODE == 3) {
        // softcap only
        if (vis == 1) scores(F_{}, T_{}, std::integral_constant<int, 0>{}, F_{}, T_{});
        else scores(F_{}, T_{}, std::integral_constant<int, 0>{}, F_{}, F_{});
      } else if constexpr (MODE >= 1) {
        if (vis == 1) dispatch_mods(md, [&](auto a, auto b_, auto c_) { scores(F_{}, a, b_, c_, T_{}); });
        else dispatch_mods(md, [&](auto a, auto b_, auto c_) { scores(F_{}, a, b_, c_, F_{}); });
      } else {
        if (vis == 2) scores(T_{}, F_{}, std::integral_constant<int, 0>{}, F_{}, F_{});
        else scores(F_{}, F_{}, std::integral_constant<int, 0>{}, F_{}, T_{});
      }
      s16x8 sb[C::NPV];
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) sb[j] = pack_op<Tag>(sacc[j >> 1], j & 1);
#pragma unroll
      for (int j = 0; j < C::NPV; ++j)
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) dq[db] = EL::mma(tr_op_rowmap<D>(Ks, 0, 32 * db, j, lane), sb[j], dq[db]);
      if constexpr (MODE == 0) sched_read_ahead<C::NPV * C::NDB, 4, 2>();
    }
    if (t + 1 < my_count) store_stage(st ^ 1);
    wait_vm_all();
    __syncthreads();
  }

  // dQ = dQ(first key half) + dQ(second key half), summed in that order.
  {
    float* ow = reinterpret_cast<float*>(smem_raw);
    if (khalf == 1) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) park_acc(ow + (wave * C::NDB + db) * 1024, lane, dq[db]);
    }
    __syncthreads();
    if (khalf == 1) return;
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) dq[db] += unpark_acc(ow + (wave * C::NDB + db) * 1024, lane);
  }

  if (!mvalid) return;
  S* dqr = reinterpret_cast<S*>(p.dq) + b * p.dq_stride[0] + hq * p.dq_stride[1] +
           (int64_t)(q_start + m) * p.dq_stride[2];
  const float sc = f.softmax_scale * (MODE == 3 ? 4.f : 1.f);
#pragma unroll
  for (int db = 0; db < C::NDB; ++db)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      s16x4 w;
#pragma unroll
      for (int r = 0; r < 4; ++r) w[r] = (short)EL::from_f(dq[db][4 * gq + r] * sc);
      *reinterpret_cast<s16x4*>(dqr + db * 32 + 8 * gq + 4 * h) = w;
    }
}


// flags: bit 0 computes delta in this kernel (fused).  Bit 1 is the
// fallback pass after dQ from stored dS: one workgroup per sequence, which
// returns at once unless some head's dS region did not fit the scratch
// (varlen lengths beyond what max_seqlen / total promised; a region's end
// grows with the head index, so the last head decides); the heads that did
// not fit get the recomputed dQ of all their query blocks here.
template <typename Tag, int D, int MODE>
__global__ __launch_bounds__(512, 1) void dq16_kernel(fa_bwd_params p, int num_m_blocks, int flags) {
  const fa_fwd_params& f = p.fwd;
  if (flags & 2) {
    const int b = blockIdx.x;
    int q_start = 0, sq = f.seqlen_q, k_start = 0, sk = f.seqlen_k;
    if (f.cu_seqlens_q) {
      bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
      bounded_seq(f.cu_seqlens_k, b, f.total_k, k_start, sk);
    }
    const int64_t base = ds_seq_base<true>(p, b, sq, sk);
    if (ds_region_at(p, base, f.heads_q - 1, sq, sk) >= 0) return;
    for (int hq = 0; hq < f.heads_q; ++hq) {
      if (ds_region_at(p, base, hq, sq, sk) >= 0) continue;
      for (int mb_rev = 0; mb_rev < num_m_blocks; ++mb_rev) {
        dq16_block<Tag, D, MODE>(p, num_m_blocks, mb_rev, b * f.heads_q + hq, 0);
        __syncthreads();  // every wave is back here; the next block reuses LDS
      }
    }
    return;
  }
  const int bh_count = f.batch * f.heads_q;
  const int mb_rev = blockIdx.x / bh_count;
  dq16_block<Tag, D, MODE>(p, num_m_blocks, mb_rev, blockIdx.x - mb_rev * bh_count, flags & 1);
}

// ---------------------------------------------------------------------------
// dQ from stored dS: dQ = scale * dS K.  The dK/dV pass stores the 16-bit dS
// it forms (the operand of its dK product) in key-major rows of the scratch;
// this kernel is the one remaining matrix product, block-sparse over the
// visible tiles, in place of dq16_kernel's recomputation of S and dP.
// A workgroup owns 128 query rows (32 per wave of a half) and splits their
// key tiles in two halves of 4 waves, like dq16_kernel.  Per 64-key tile the
// K rows and the dS rows of the tile's keys (128 queries each) go HBM -> LDS
// by DMA; both MFMA operands are transposing LDS reads (the contracted index,
// keys, runs along the tile rows of both).
// ---------------------------------------------------------------------------
// Two configurations of the same kernel:
//  * OCC = 1 (few workgroups per CU over the launch, e.g. one causal batch):
//    32-key steps through a 4-stage ring per key half (96 KiB of dS and K in
//    flight per CU), one workgroup per CU;
//  * OCC = 2, D = 128 (many workgroups per CU, e.g. a packed varlen batch): 16-key
//    steps through a 4-stage ring (64 KiB of LDS), two workgroups per CU, so
//    one workgroup's prologue (its first loads) and epilogue (the half merge
//    and dQ store) overlap the other's steady state.
// Measured at config 2 (512 workgroups) 43 us with OCC = 1 against 50 us;
// at config 5 (4608 workgroups) 310 us with OCC = 2 against 369 us.
template <int D, int OCC>
struct Dqs16Cfg {
  static constexpr int NQ = 4;
  static constexpr int NW = 2 * NQ;
  static constexpr int NT = 64 * NW;
  static constexpr int NTH = 64 * NQ;
  static constexpr int BM = 32 * NQ;
  // keys per step (part of a dS tile); 16-key stages need D >= 128 to fill
  // whole 16-byte chunks per thread
  static constexpr int BN = (OCC == 2 && D >= 128) ? 16 : 32;
  static constexpr int NSTG = 4;                   // ring of stages per key half
  static constexpr int KT = BN * D;                // K rows (elements)
  static constexpr int ST = BN * BM;               // dS rows: BN keys x BM queries
  static constexpr int STAGE = KT + ST;
  static constexpr int HALF = NSTG * STAGE;
  static constexpr int LOOP_BYTES = 2 * HALF * 2;
  static constexpr int MERGE_BYTES = NQ * (D / 32) * 16 * 64 * 4;
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
  static constexpr int NPV = BN / 16;
  static constexpr int NDB = D / 32;
  // DMA instructions per thread per stage (the end-of-step wait counts them)
  static constexpr int LOADS = (KT / 8) / NTH + (ST / 8) / NTH;
  static_assert(BM == kDsTileQueries && kDsTileKeys % BN == 0, "a dQ step reads whole rows of one dS tile");
  static_assert(OCC == 1 || 2 * LDS_BYTES <= 160 * 1024, "two workgroups must fit one CU's LDS");
};

// One work item (query block `item / (B * Hq)` from the heavy end of
// (batch, head) `item % (B * Hq)`); `end_barrier` as in fwd16_item.
template <typename Tag, int D, int OCC, bool VARLEN>
__device__ __forceinline__ void dqs16_item(const fa_bwd_params& p, int num_m_blocks, float dq_scale, bool ds_nt,
                                           int item, unsigned char* smem_raw, bool end_barrier) {
  using C = Dqs16Cfg<D, OCC>;
  using EL = Elem<Tag>;
  using S = uint16_t;
  S* smem = reinterpret_cast<S*>(smem_raw);
  const fa_fwd_params& f = p.fwd;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int khalf = wave8 / C::NQ;
  const int wave = wave8 % C::NQ;
  const int htid = tid % C::NTH;
  const int h = lane >> 5, l32 = lane & 31;
  const int bh_count = f.batch * f.heads_q;
  const int mb_rev = item / bh_count;
  const int bh = item - mb_rev * bh_count;
  const int b = bh / f.heads_q, hq = bh - b * f.heads_q;
  const int hk = hq / (f.heads_q / f.heads_kv);
  const int mblk = num_m_blocks - 1 - mb_rev;  // heaviest causal blocks first

  int q_start = 0, sq = f.seqlen_q, k_start = 0, sk = f.seqlen_k;
  if constexpr (VARLEN) {
    bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
    bounded_seq(f.cu_seqlens_k, b, f.total_k, k_start, sk);
  }
  const int m0 = mblk * C::BM;
  if (m0 >= sq) return;
  // The dense form is a separate instantiation without the wave sum:
  // compiled in, it cost config 2's dQ 3-4 us.
  const int64_t base = VARLEN ? ds_seq_base<true>(p, b, sq, sk) : (int64_t)b * f.heads_q * ds_region_elems(sq, sk);
  const int64_t region = ds_region_at(p, base, hq, sq, sk);
  const int64_t qblocks = ds_qblocks(sq);

  const S* kbase = reinterpret_cast<const S*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] +
                   (int64_t)k_start * f.k_stride[2];
  // dS tiles of this query block: key block kb at dsbase + kb * qblocks * tile
  const S* dsbase = reinterpret_cast<const S*>(p.ds_workspace) + (region < 0 ? 0 : region) +
                    (int64_t)mblk * kDsTileElems;
  const int64_t ks = f.k_stride[2];
  const Mods md = make_mods(f, b, hq, sq, sk);

  const int mlast = min(m0 + C::BM, sq) - 1;
  int lo = 0, hi = sk;
  if (f.causal) hi = min(hi, mlast + md.off + 1);
  if (f.window_right >= 0) hi = min(hi, mlast + md.off + f.window_right + 1);
  if (f.window_left >= 0) lo = max(0, m0 + md.off - f.window_left);
  // The key range is split between the halves at a 32-key boundary in both
  // configurations, and each 16-key MFMA slice starts at a multiple of 16:
  // dQ sums the same products in the same order whichever step size runs,
  // so a sequence's dQ does not depend on the launch it is part of.
  constexpr int SPLIT = 32, SPS = SPLIT / C::BN;  // steps per split unit
  // The step bounds are the same for every lane but derive from per-lane
  // loads (cu_seqlens): kept in scalar registers so the step loop's control
  // and waits stay scalar instead of exec-mask branches.
  lo = __builtin_amdgcn_readfirstlane(lo / SPLIT * SPLIT);
  hi = __builtin_amdgcn_readfirstlane(hi);
  const int nsplit = __builtin_amdgcn_readfirstlane((hi > lo && region >= 0) ? (hi - lo + SPLIT - 1) / SPLIT : 0);

  const int m0w = m0 + 32 * wave;
  const int mrows = min(32, sq - m0w);
  const int m = m0w + l32;

  f32x16 dq[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dq[i] = zero16();

  DmaSwzTile<C::BN, D, C::NTH> kd;
  DmaSwzTile<C::BN, C::BM, C::NTH> sd;
  kd.init(ks, htid);
  sd.template init_blocked<kDsSubQueries / 8>(kDsSubElems * 2, htid);
  // Both halves run nh0 steps so their barriers line up; a step whose keys
  // start at or past hi is never loaded (its rows could lie past the end).
  const int half0 = (nsplit + 1) / 2;
  const int nh0 = half0 * SPS;
  const int my_first = khalf == 0 ? 0 : nh0;
  const int my_end = min(lo + SPLIT * (khalf == 0 ? half0 : nsplit), hi);
  const int my_count =
      __builtin_amdgcn_readfirstlane(max(0, (my_end - (lo + my_first * C::BN) + C::BN - 1) / C::BN));
  S* const hsmem = smem + khalf * C::HALF;
  const uint32_t lds0 = lds_addr(hsmem);
  // Stage st holds step t with t % NSTG == st; NSTG - 1 steps are in flight
  // while one is computed.
  auto load_stage = [&](int n0, int st) {
    const int rows = min(C::BN, sk - n0);
    const uint32_t base = lds0 + (uint32_t)(st * C::STAGE) * 2u;
    kd.load(rows_rsrc_words<D>(kbase + (int64_t)n0 * ks, ks, rows), base, wave);
    // The tile's 4 query sub-tiles hold rows of 32 queries; the window is
    // the whole tile (rows past the last key are garbage there and are
    // zeroed by the visibility mask of the partly visible step).
    const int r0 = n0 % kDsTileKeys;  // first key row of the step within the tile
    const S* dtile = dsbase + (int64_t)(n0 / kDsTileKeys) * qblocks * kDsTileElems + r0 * kDsSubQueries;
    const i32x4 drs = rsrc_words(dtile, (kDsTileElems - r0 * kDsSubQueries) * 2);
    if (ds_nt) sd.load_nt(drs, base + C::KT * 2u, wave);
    else sd.load(drs, base + C::KT * 2u, wave);
  };

  // Visible keys of this lane's row: partly visible tiles zero the dS of
  // hidden pairs, which the dK/dV pass may not have written.
  int klo, khi;
  key_bounds(md, m, klo, khi);
  const VisBounds qvb = row_block_bounds(md, m0w, mrows);
#pragma unroll
  for (int i = 0; i < C::NSTG - 1; ++i)
    if (i < my_count) load_stage(lo + (my_first + i) * C::BN, i);
  for (int t = 0; t < nh0; ++t) {
    const int n0 = lo + (my_first + t) * C::BN;
    const int st = t % C::NSTG;
    // Step t's loads have landed once at most the later steps' loads are
    // outstanding (vector memory operations complete in issue order).
    const int later = min(my_count - 1 - t, C::NSTG - 2);
    if (later >= 2) wait_vm<2 * C::LOADS>();
    else if (later == 1) wait_vm<C::LOADS>();
    else wait_vm_all();
    __syncthreads();
    // The stage refilled here was last read in step t - 1, before the barrier.
    if (t + C::NSTG - 1 < my_count) load_stage(n0 + (C::NSTG - 1) * C::BN, (t + C::NSTG - 1) % C::NSTG);
    const int vis = __builtin_amdgcn_readfirstlane(t < my_count ? bounds_vis(qvb, n0, n0 + C::BN - 1) : 0);
    if (vis) {
      const S* Ks = hsmem + st * C::STAGE;
      const S* Ss = Ks + C::KT;
      s16x8 sb[C::NPV];
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) sb[j] = tr_op_rowmap<C::BM>(Ss, 0, 32 * wave, j, lane);
      if (vis == 1) {
        // Element e of operand j holds key 32 (j/2) + 16 (j%2) + 4h + e%4
        // (+ 8 for e >= 4), the row map of tr_op_rowmap.
        const Span ks2 = make_span(klo, khi, n0 + 4 * h);
#pragma unroll
        for (int j = 0; j < C::NPV; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (!in_span(ks2, 32 * (j >> 1) + 16 * (j & 1) + 8 * (e >> 2) + (e & 3))) sb[j][e] = 0;
      }
#pragma unroll
      for (int j = 0; j < C::NPV; ++j)
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) dq[db] = EL::mma(tr_op_rowmap<D>(Ks, 0, 32 * db, j, lane), sb[j], dq[db]);
      sched_read_ahead<C::NPV * C::NDB, 4, 2>();
    }
  }
  __syncthreads();

  // dQ = dQ(first key half) + dQ(second key half), summed in that order.
  {
    float* ow = reinterpret_cast<float*>(smem_raw);
    if (khalf == 1) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) park_acc(ow + (wave * C::NDB + db) * 1024, lane, dq[db]);
    }
    __syncthreads();
    if (khalf == 1) {
      if (end_barrier) __syncthreads();
      return;
    }
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) dq[db] += unpark_acc(ow + (wave * C::NDB + db) * 1024, lane);
  }

  // Whole-row dQ stores through this wave's LDS block of the merge above.
  S* dqr0 = reinterpret_cast<S*>(p.dq) + b * p.dq_stride[0] + hq * p.dq_stride[1] +
            (int64_t)(q_start + m0w) * p.dq_stride[2];
  store_rows_staged<Tag, D>(dq, dq_scale, reinterpret_cast<uint16_t*>(smem_raw + wave * C::NDB * 4096), dqr0,
                            p.dq_stride[2], mrows, lane);
  if (end_barrier) __syncthreads();
}

// PAIR: workgroup (j, b·Hq) runs query block j from the heavy end, then
// from the light end, of the same (batch, head), like fwd16_kernel.
// ds_nt: read dS with nontemporal loads (scratch too large for the 256 MiB
// memory-side cache, so the dS lines only displace reused K rows from L2).
// VARLEN: cu_seqlens_q / cu_seqlens_k are set (the host picks the form).
template <typename Tag, int D, int OCC, bool PAIR, bool VARLEN>
__global__ __launch_bounds__(512, OCC) void dqs16_kernel(fa_bwd_params p, int num_m_blocks, float dq_scale, int ds_nt) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  if constexpr (!PAIR) {
    dqs16_item<Tag, D, OCC, VARLEN>(p, num_m_blocks, dq_scale, ds_nt != 0, blockIdx.x, smem_raw, false);
  } else {
    const int bh_count = p.fwd.batch * p.fwd.heads_q;
    const int j = blockIdx.x / bh_count;
    const int bh = blockIdx.x - j * bh_count;
    const int j2 = num_m_blocks - 1 - j;
    dqs16_item<Tag, D, OCC, VARLEN>(p, num_m_blocks, dq_scale, ds_nt != 0, j * bh_count + bh, smem_raw, j2 != j);
    if (j2 != j) dqs16_item<Tag, D, OCC, VARLEN>(p, num_m_blocks, dq_scale, ds_nt != 0, j2 * bh_count + bh, smem_raw, false);
  }
}

}  // namespace fa
