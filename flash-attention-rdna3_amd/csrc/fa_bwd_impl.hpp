#pragma once
#include <type_traits>
// Kernel templates of fa_bwd; instantiated per dtype by fa_bwd_<dtype>.hip.
// fa_bwd.hip - FlashAttention-2 backward for gfx950: delta, dK/dV, dQ.
//
// Same math as the reference's `_attention_bwd_preprocess`,
// `_attention_bwd_dkdv`, `_attention_bwd_dq` and their varlen twins
// (fa_rdna3/kernels/backward.py:18-322, varlen.py:152-421, inner loops
// _common.py:347-508): P is recomputed from the stored LSE,
//     P = exp2(x - lse*log2e),  dV += P_d^T dO,  dP = dO V^T,
//     dS = P (dP_d - delta) [* (1 - tanh^2) under softcap],
//     dK = scale * dS^T Q,      dQ = scale * dS K,
// with delta = rowsum(O * dO) and P_d / dP_d the dropout-masked, 1/(1-p)
// scaled copies.  No atomics: dK/dV and dQ are separate kernels and a GQA
// group is summed inside the dK/dV workgroup, so gradients are deterministic.
//
// MI355X layout.
//  * dK/dV: each wave owns 32 KEYS, which sit on the lane axis of
//    S = Q K^T (queries x keys).  K and V are B operands held in registers;
//    Q and dO stream through LDS per 32-row query block in both row-major
//    form (A operands of S and dP) and transposed form (A operands of
//    dK^T += Q^T dS and dV^T += dO^T P_d).  P_d and dS go straight from the
//    accumulators into B operands.
//  * dQ: each wave owns 32 QUERIES (lane axis of S^T = K Q^T, as in the
//    forward); K, V and K^T are staged in LDS and shared by the 4 waves,
//    Q and dO are register B operands, dS^T feeds dQ^T += K^T dS^T directly.
#include "fa_internal.hpp"
#include "fa_tiles.hpp"
#include "fa_bwd16.hpp"

namespace fa {


// ---------------------------------------------------------------------------
// delta[m] = sum_d O[m][d] * dO[m][d]   (fp32 accumulate)
// ---------------------------------------------------------------------------
// Rows per thread of the delta pass: four 16-byte chunks of O and of dO in
// flight per thread (one row of D = 512 f16, four rows of D = 128 f16).
template <typename Tag, int D>
constexpr int delta_rows_per_thread() {
  constexpr int chunks = (D / Elem<Tag>::CE + 15) / 16;
  return chunks >= 4 ? 1 : 4 / chunks;
}

// heads_fast: grid (heads_q, row blocks, batch) instead of (row blocks,
// batch * heads_q), for O / dO whose heads sit side by side within a row
// (packed varlen and (B, S, H, D) layouts): the workgroups in flight then
// read whole rows of all heads together instead of 256-byte pieces of one
// head spread a row stride apart.
template <typename Tag, int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(fa_bwd_params p, int heads_fast) {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  constexpr int CE = EL::CE, CPR = D / CE;
  constexpr int LPR = 16;  // lanes per row
  // Each thread covers R rows 16 apart and issues all of their loads before
  // the products, so a wave keeps R times more bytes in flight than a
  // one-row pass.
  constexpr int R = delta_rows_per_thread<Tag, D>();
  const fa_fwd_params& f = p.fwd;
  int b, hq, rb;
  if (heads_fast) {
    hq = blockIdx.x, rb = blockIdx.y, b = blockIdx.z;
  } else {
    const int bh = blockIdx.y;
    b = bh / f.heads_q, hq = bh - b * f.heads_q, rb = blockIdx.x;
  }
  int q_start = 0, sq = f.seqlen_q;
  if (f.cu_seqlens_q) bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
  const int mrow = rb * (16 * R) + (threadIdx.x >> 4);
  if (rb * (16 * R) >= sq) return;
  const int sub = threadIdx.x & 15;
  const S* obase = reinterpret_cast<const S*>(f.out) + b * f.out_stride[0] + hq * f.out_stride[1];
  const S* gbase = reinterpret_cast<const S*>(p.dout) + b * p.dout_stride[0] + hq * p.dout_stride[1];
  constexpr int NC = (CPR + LPR - 1) / LPR;  // chunks per lane per row
  uint4 a[R][NC], g[R][NC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int m = min(mrow + 16 * r, sq - 1);
    const S* o = obase + (int64_t)(q_start + m) * f.out_stride[2];
    const S* d = gbase + (int64_t)(q_start + m) * p.dout_stride[2];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int c = sub + i * LPR;
      if (c < CPR) {
        // O is read once (nontemporal: config 5 delta 68 -> 60 us); dO
        // stays cached for the dK/dV pass that reads it next.
        a[r][i] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(o + c * CE)));
        g[r][i] = *reinterpret_cast<const uint4*>(d + c * CE);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      if (sub + i * LPR < CPR) {
        const S* av = reinterpret_cast<const S*>(&a[r][i]);
        const S* bv = reinterpret_cast<const S*>(&g[r][i]);
#pragma unroll
        for (int e = 0; e < CE; ++e) acc += EL::to_f(av[e]) * EL::to_f(bv[e]);
      }
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) acc += __shfl_xor(acc, w, 64);
    const int m = mrow + 16 * r;
    if (m < sq && sub == 0)
      p.delta[b * p.delta_stride[0] + hq * p.delta_stride[1] + (int64_t)(q_start + m) * p.delta_stride[2]] = acc;
  }
}

// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------
template <typename Tag, int D>
struct DkdvCfg {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int NW = 4;
  static constexpr int NT = 64 * NW;
  static constexpr int BN = 32 * NW;  // keys per workgroup
  static constexpr int BMQ = 32;      // query rows per inner step
  static constexpr int DO = (D <= 128) ? D : ((sizeof(S) == 4 && D == 512) ? 64 : 128);
  static constexpr bool KVREG = (sizeof(S) == 2) ? (D <= 128) : (D <= 64);
  static constexpr int QLD = D + EL::CE;     // Q / dO row-major tiles
  static constexpr int TLD = BMQ + EL::CE;   // Q^T / dO^T tiles
  static constexpr int QTILE = BMQ * QLD;
  static constexpr int TTILE = DO * TLD;
  // stage: Q, dO, Q^T, dO^T (elements of S) then lse2, delta (floats)
  static constexpr int STAGE_ELEMS = 2 * QTILE + 2 * TTILE;
  static constexpr int STAGE_BYTES = STAGE_ELEMS * (int)sizeof(S) + 2 * BMQ * 4;
  static constexpr int NSTAGE = (2 * STAGE_BYTES <= 160 * 1024) ? 2 : 1;
  static constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;
  static constexpr int NSTEP = D / EL::KSTEP;
  static constexpr int NMB = BMQ / 32;
  static constexpr int NPV = BMQ / (2 * EL::E);
  static constexpr int NDB = DO / 32;
};

template <typename Tag, int D, int MODE>
__global__ __launch_bounds__(256) void bwd_dkdv_kernel(fa_bwd_params p, int num_n_blocks) {
  using C = DkdvCfg<Tag, D>;
  using EL = Elem<Tag>;
  using S = typename EL::S;
  using Op = typename EL::Op;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const fa_fwd_params& f = p.fwd;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;
  const int ndc = D / C::DO;
  const int bhk_count = f.batch * f.heads_kv;
  const int id = blockIdx.x;
  const int nb_rev = id / (bhk_count * ndc);
  const int rest = id - nb_rev * bhk_count * ndc;
  const int bhk = rest / ndc, dc = rest - (rest / ndc) * ndc;
  const int b = bhk / f.heads_kv, hk = bhk - b * f.heads_kv;
  const int group = f.heads_q / f.heads_kv;
  const int nblk = num_n_blocks - 1 - nb_rev;

  int q_start = 0, sq = f.seqlen_q, k_start = 0, sk = f.seqlen_k;
  if (f.cu_seqlens_q) {
    bounded_seq(f.cu_seqlens_q, b, f.total_q, q_start, sq);
    bounded_seq(f.cu_seqlens_k, b, f.total_k, k_start, sk);
  }
  const int n0 = nblk * C::BN;
  if (n0 >= sk) return;

  const S* kbase = reinterpret_cast<const S*>(f.k) + b * f.k_stride[0] + hk * f.k_stride[1] +
                   (int64_t)k_start * f.k_stride[2];
  const S* vbase = reinterpret_cast<const S*>(f.v) + b * f.v_stride[0] + hk * f.v_stride[1] +
                   (int64_t)k_start * f.v_stride[2];

  const int n0w = n0 + 32 * wave;
  const int ncols = min(32, sk - n0w);  // <= 0: the wave only helps load
  const int n = n0w + l32;
  const bool nvalid = n < sk;
  const S* krow = kbase + (int64_t)(nvalid ? n : 0) * f.k_stride[2] + EL::E * h;
  const S* vrow = vbase + (int64_t)(nvalid ? n : 0) * f.v_stride[2] + EL::E * h;
  Op kop[C::KVREG ? C::NSTEP : 1], vop[C::KVREG ? C::NSTEP : 1];
  if constexpr (C::KVREG) {
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      kop[s] = nvalid ? load_op<Tag>(krow + EL::KSTEP * s) : zero_op<Tag>();
      vop[s] = nvalid ? load_op<Tag>(vrow + EL::KSTEP * s) : zero_op<Tag>();
    }
    wait_vm_all();
  }

  f32x16 dk[C::NDB], dv[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) { dk[i] = zero16(); dv[i] = zero16(); }

  RowTile<Tag, C::BMQ, D, C::NT> qt, gt;
  TransTile<Tag, C::BMQ, C::DO, C::NT> qtt, gtt;

  const int nlast = min(n0 + C::BN, sk) - 1;
  for (int g = 0; g < group; ++g) {
    const int hq = hk * group + g;
    const Mods md = make_mods(f, b, hq, sq, sk);
    const S* qbase = reinterpret_cast<const S*>(f.q) + b * f.q_stride[0] + hq * f.q_stride[1] +
                     (int64_t)q_start * f.q_stride[2];
    const S* gbase = reinterpret_cast<const S*>(p.dout) + b * p.dout_stride[0] + hq * p.dout_stride[1] +
                     (int64_t)q_start * p.dout_stride[2];
    const float* lbase = f.lse + b * f.lse_stride[0] + hq * f.lse_stride[1] + (int64_t)q_start * f.lse_stride[2];
    const float* dbase = p.delta + b * p.delta_stride[0] + hq * p.delta_stride[1] +
                         (int64_t)q_start * p.delta_stride[2];
    const int64_t qs = f.q_stride[2], gs = p.dout_stride[2];

    // Query rows that can see this key block (reference backward.py:110-136).
    int mlo = 0, mhi = sq;
    if (f.causal) mlo = max(mlo, n0 - md.off);
    if (f.window_right >= 0) mlo = max(mlo, n0 - md.off - f.window_right);
    if (f.window_left >= 0) mhi = min(mhi, nlast - md.off + f.window_left + 1);
    mlo = max(mlo, 0) / C::BMQ * C::BMQ;
    const int nsteps = mhi > mlo ? (mhi - mlo + C::BMQ - 1) / C::BMQ : 0;

    auto load_stage = [&](int m0) {
      qt.load([&](int r) -> const S* { int m = m0 + r; return m < sq ? qbase + (int64_t)m * qs : nullptr; }, qbase, tid);
      gt.load([&](int r) -> const S* { int m = m0 + r; return m < sq ? gbase + (int64_t)m * gs : nullptr; }, gbase, tid);
      qtt.load([&](int r) -> const S* {
        int m = m0 + r; return m < sq ? qbase + (int64_t)m * qs + dc * C::DO : nullptr; }, qbase + dc * C::DO, tid);
      gtt.load([&](int r) -> const S* {
        int m = m0 + r; return m < sq ? gbase + (int64_t)m * gs + dc * C::DO : nullptr; }, gbase + dc * C::DO, tid);
    };
    auto store_stage = [&](int st, int m0) {
      unsigned char* base = smem_raw + st * C::STAGE_BYTES;
      S* sp = reinterpret_cast<S*>(base);
      qt.store(sp, C::QLD, tid);
      gt.store(sp + C::QTILE, C::QLD, tid);
      qtt.store(sp + 2 * C::QTILE, C::TLD, tid);
      gtt.store(sp + 2 * C::QTILE + C::TTILE, C::TLD, tid);
      float* lf = reinterpret_cast<float*>(base + C::STAGE_ELEMS * sizeof(S));
      if (tid < C::BMQ) {
        const int m = m0 + tid;
        float l = kNegInf, dl = 0.f;
        if (m < sq) {
          l = lbase[(int64_t)m * f.lse_stride[2]];
          dl = dbase[(int64_t)m * p.delta_stride[2]];
        }
        lf[tid] = (l == kNegInf) ? kNegInf : l * kLog2e;
        lf[C::BMQ + tid] = dl;
      }
    };

    if (nsteps > 0) {
      load_stage(mlo);
      store_stage(0, mlo);
    }
    __syncthreads();
    for (int t = 0; t < nsteps; ++t) {
      const int m0 = mlo + t * C::BMQ;
      const int st = (C::NSTAGE == 2) ? (t & 1) : 0;
      if (C::NSTAGE == 2 && t + 1 < nsteps) load_stage(m0 + C::BMQ);

      const int vis = ncols > 0 ? rect_visibility(md, m0, min(C::BMQ, sq - m0), n0w, ncols) : 0;
      if (vis) {
        const unsigned char* base = smem_raw + st * C::STAGE_BYTES;
        const S* Qs = reinterpret_cast<const S*>(base);
        const S* Gs = Qs + C::QTILE;
        const S* QTs = Qs + 2 * C::QTILE;
        const S* GTs = QTs + C::TTILE;
        const float* L2 = reinterpret_cast<const float*>(base + C::STAGE_ELEMS * sizeof(S));
        const float* DL = L2 + C::BMQ;

        f32x16 sacc[C::NMB], pacc[C::NMB];
#pragma unroll
        for (int mb = 0; mb < C::NMB; ++mb) {
          sacc[mb] = zero16();
          pacc[mb] = zero16();
          const S* qr = Qs + (mb * 32 + l32) * C::QLD + EL::E * h;
          const S* gr = Gs + (mb * 32 + l32) * C::QLD + EL::E * h;
#pragma unroll
          for (int s = 0; s < C::NSTEP; ++s) {
            Op kb_, vb_;
            if constexpr (C::KVREG) { kb_ = kop[s]; vb_ = vop[s]; }
            else {
              kb_ = nvalid ? load_op<Tag>(krow + EL::KSTEP * s) : zero_op<Tag>();
              vb_ = nvalid ? load_op<Tag>(vrow + EL::KSTEP * s) : zero_op<Tag>();
            }
            sacc[mb] = EL::mma(load_op<Tag>(qr + EL::KSTEP * s), kb_, sacc[mb]);
            pacc[mb] = EL::mma(load_op<Tag>(gr + EL::KSTEP * s), vb_, pacc[mb]);
          }
        }
        // P_d -> sacc, dS -> pacc.
#pragma unroll
        for (int mb = 0; mb < C::NMB; ++mb) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int ml = mb * 32 + acc_row(i, h);
            const int m = m0 + ml;
            float tc;
            const float x = score<(MODE >= 1)>(md, sacc[mb][i], m, n, tc);
            const float l2 = L2[ml];
            float pv = (l2 == kNegInf) ? 0.f : exp2f(x - l2);
            if (vis == 1 && !keep_pos(md, m, n)) pv = 0.f;
            float dp = pacc[mb][i];
            float pd = pv;
            if constexpr (MODE == 2) {
              if (md.drop_p > 0.f) {
                const bool keep = dropout_keep(md, m, n);
                pd = keep ? pv * md.drop_scale : 0.f;
                dp = keep ? dp * md.drop_scale : 0.f;
              }
            }
            float ds = pv * (dp - DL[ml]);
            if constexpr (MODE >= 1) {
              if (md.cap2 > 0.f) ds *= (1.f - tc * tc);
            }
            sacc[mb][i] = pd;
            pacc[mb][i] = ds;
          }
        }
        constexpr int J = 16 / EL::E;
        Op pb[C::NPV], sb[C::NPV];
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) {
          pb[j] = pack_op<Tag>(sacc[j / J], j % J);
          sb[j] = pack_op<Tag>(pacc[j / J], j % J);
        }
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
          const S* gtr = GTs + (db * 32 + l32) * C::TLD;
          const S* qtr = QTs + (db * 32 + l32) * C::TLD;
#pragma unroll
          for (int j = 0; j < C::NPV; ++j) {
            dv[db] = EL::mma(lds_op_rowmap<Tag>(gtr, j, h), pb[j], dv[db]);
            dk[db] = EL::mma(lds_op_rowmap<Tag>(qtr, j, h), sb[j], dk[db]);
          }
        }
      }
      if (C::NSTAGE == 2) {
        if (t + 1 < nsteps) store_stage(st ^ 1, m0 + C::BMQ);
        __syncthreads();
      } else {
        __syncthreads();
        if (t + 1 < nsteps) {
          load_stage(m0 + C::BMQ);
          store_stage(0, m0 + C::BMQ);
        }
        __syncthreads();
      }
    }
  }

  if (!nvalid) return;
  S* dkr = reinterpret_cast<S*>(p.dk) + b * p.dk_stride[0] + hk * p.dk_stride[1] +
           (int64_t)(k_start + n) * p.dk_stride[2] + dc * C::DO;
  S* dvr = reinterpret_cast<S*>(p.dv) + b * p.dv_stride[0] + hk * p.dv_stride[1] +
           (int64_t)(k_start + n) * p.dv_stride[2] + dc * C::DO;
  const float sc = f.softmax_scale;
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) {
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d = db * 32 + 8 * gq + 4 * h;
      if constexpr (sizeof(S) == 2) {
        s16x4 wk, wv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          wk[r] = (short)EL::from_f(dk[db][4 * gq + r] * sc);
          wv[r] = (short)EL::from_f(dv[db][4 * gq + r]);
        }
        *reinterpret_cast<s16x4*>(dkr + d) = wk;
        *reinterpret_cast<s16x4*>(dvr + d) = wv;
      } else {
        f32x4 wk, wv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          wk[r] = dk[db][4 * gq + r] * sc;
          wv[r] = dv[db][4 * gq + r];
        }
        *reinterpret_cast<f32x4*>(dkr + d) = wk;
        *reinterpret_cast<f32x4*>(dvr + d) = wv;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <typename Tag, int D>
struct DqCfg {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int NW = 4;
  static constexpr int NT = 64 * NW;
  static constexpr int BM = 32 * NW;
  static constexpr int BN = (D <= 64) ? 64 : 32;
  static constexpr int DO = (D <= 128) ? D : ((sizeof(S) == 4 && D == 512) ? 64 : 128);
  static constexpr bool QREG = (sizeof(S) == 2) ? (D <= 128) : (D <= 64);
  static constexpr int KLD = D + EL::CE;
  static constexpr int TLD = BN + EL::CE;
  static constexpr int KTILE = BN * KLD;
  static constexpr int TTILE = DO * TLD;
  static constexpr int STAGE = 2 * KTILE + TTILE;  // K, V, K^T
  static constexpr int STAGE_BYTES = STAGE * (int)sizeof(S);
  static constexpr int NSTAGE = (2 * STAGE_BYTES <= 160 * 1024) ? 2 : 1;
  static constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;
  static constexpr int NSTEP = D / EL::KSTEP;
  static constexpr int NKB = BN / 32;
  static constexpr int NPV = BN / (2 * EL::E);
  static constexpr int NDB = DO / 32;
};

template <typename Tag, int D, int MODE>
__global__ __launch_bounds__(256) void bwd_dq_kernel(fa_bwd_params p, int num_m_blocks) {
  using C = DqCfg<Tag, D>;
  using EL = Elem<Tag>;
  using S = typename EL::S;
  using Op = typename EL::Op;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  S* smem = reinterpret_cast<S*>(smem_raw);
  const fa_fwd_params& f = p.fwd;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;
  const int ndc = D / C::DO;
  const int bh_count = f.batch * f.heads_q;
  const int id = blockIdx.x;
  const int mb_rev = id / (bh_count * ndc);
  const int rest = id - mb_rev * bh_count * ndc;
  const int bh = rest / ndc, dc = rest - (rest / ndc) * ndc;
  const int b = bh / f.heads_q, hq = bh - b * f.heads_q;
  const int hk = hq / (f.heads_q / f.heads_kv);
  const int mblk = num_m_blocks - 1 - mb_rev;

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
  const S* qrow = reinterpret_cast<const S*>(f.q) + b * f.q_stride[0] + hq * f.q_stride[1] +
                  (int64_t)(q_start + (mvalid ? m : 0)) * f.q_stride[2] + EL::E * h;
  const S* grow = reinterpret_cast<const S*>(p.dout) + b * p.dout_stride[0] + hq * p.dout_stride[1] +
                  (int64_t)(q_start + (mvalid ? m : 0)) * p.dout_stride[2] + EL::E * h;
  Op qop[C::QREG ? C::NSTEP : 1], gop[C::QREG ? C::NSTEP : 1];
  if constexpr (C::QREG) {
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) {
      qop[s] = mvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
      gop[s] = mvalid ? load_op<Tag>(grow + EL::KSTEP * s) : zero_op<Tag>();
    }
  }
  float lse2 = kNegInf, dlt = 0.f;
  if (mvalid) {
    const float l = f.lse[b * f.lse_stride[0] + hq * f.lse_stride[1] + (int64_t)(q_start + m) * f.lse_stride[2]];
    lse2 = (l == kNegInf) ? kNegInf : l * kLog2e;
    dlt = p.delta[b * p.delta_stride[0] + hq * p.delta_stride[1] + (int64_t)(q_start + m) * p.delta_stride[2]];
  }
  wait_vm_all();

  f32x16 dq[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) dq[i] = zero16();

  RowTile<Tag, C::BN, D, C::NT> kt, vt;
  TransTile<Tag, C::BN, C::DO, C::NT> ktt;
  auto load_stage = [&](int n0) {
    kt.load([&](int r) -> const S* { int nn = n0 + r; return nn < sk ? kbase + (int64_t)nn * ks : nullptr; }, kbase, tid);
    vt.load([&](int r) -> const S* { int nn = n0 + r; return nn < sk ? vbase + (int64_t)nn * vs : nullptr; }, vbase, tid);
    ktt.load([&](int r) -> const S* {
      int nn = n0 + r; return nn < sk ? kbase + (int64_t)nn * ks + dc * C::DO : nullptr; }, kbase + dc * C::DO, tid);
  };
  auto store_stage = [&](int st) {
    S* base = smem + st * C::STAGE;
    kt.store(base, C::KLD, tid);
    vt.store(base + C::KTILE, C::KLD, tid);
    ktt.store(base + 2 * C::KTILE, C::TLD, tid);
  };

  if (ntiles > 0) {
    load_stage(lo);
    store_stage(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = lo + t * C::BN;
    const int st = (C::NSTAGE == 2) ? (t & 1) : 0;
    if (C::NSTAGE == 2 && t + 1 < ntiles) load_stage(n0 + C::BN);
    const int vis = mrows > 0 ? rect_visibility(md, m0w, mrows, n0, C::BN) : 0;
    if (vis) {
      const S* Ks = smem + st * C::STAGE;
      const S* Vs = Ks + C::KTILE;
      const S* KTs = Ks + 2 * C::KTILE;
      f32x16 sacc[C::NKB], pacc[C::NKB];
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
        sacc[kb2] = zero16();
        pacc[kb2] = zero16();
        const S* kr = Ks + (kb2 * 32 + l32) * C::KLD + EL::E * h;
        const S* vr = Vs + (kb2 * 32 + l32) * C::KLD + EL::E * h;
#pragma unroll
        for (int s = 0; s < C::NSTEP; ++s) {
          Op qb_, gb_;
          if constexpr (C::QREG) { qb_ = qop[s]; gb_ = gop[s]; }
          else {
            qb_ = mvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
            gb_ = mvalid ? load_op<Tag>(grow + EL::KSTEP * s) : zero_op<Tag>();
          }
          sacc[kb2] = EL::mma(load_op<Tag>(kr + EL::KSTEP * s), qb_, sacc[kb2]);
          pacc[kb2] = EL::mma(load_op<Tag>(vr + EL::KSTEP * s), gb_, pacc[kb2]);
        }
      }
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int nn = n0 + kb2 * 32 + acc_row(i, h);
          float tc;
          const float x = score<(MODE >= 1)>(md, sacc[kb2][i], m, nn, tc);
          float pv = (lse2 == kNegInf) ? 0.f : exp2f(x - lse2);
          if (vis == 1 && !keep_pos(md, m, nn)) pv = 0.f;
          float dp = pacc[kb2][i];
          if constexpr (MODE == 2) {
            if (md.drop_p > 0.f) dp = dropout_keep(md, m, nn) ? dp * md.drop_scale : 0.f;
          }
          float ds = pv * (dp - dlt);
          if constexpr (MODE >= 1) {
            if (md.cap2 > 0.f) ds *= (1.f - tc * tc);
          }
          sacc[kb2][i] = ds;
        }
      }
      constexpr int J = 16 / EL::E;
      Op sb[C::NPV];
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) sb[j] = pack_op<Tag>(sacc[j / J], j % J);
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const S* ktr = KTs + (db * 32 + l32) * C::TLD;
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) dq[db] = EL::mma(lds_op_rowmap<Tag>(ktr, j, h), sb[j], dq[db]);
      }
    }
    if (C::NSTAGE == 2) {
      if (t + 1 < ntiles) store_stage(st ^ 1);
      __syncthreads();
    } else {
      __syncthreads();
      if (t + 1 < ntiles) {
        load_stage(n0 + C::BN);
        store_stage(0);
      }
      __syncthreads();
    }
  }

  if (!mvalid) return;
  S* dqr = reinterpret_cast<S*>(p.dq) + b * p.dq_stride[0] + hq * p.dq_stride[1] +
           (int64_t)(q_start + m) * p.dq_stride[2] + dc * C::DO;
  const float sc = f.softmax_scale;
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) {
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d = db * 32 + 8 * gq + 4 * h;
      if constexpr (sizeof(S) == 2) {
        s16x4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = (short)EL::from_f(dq[db][4 * gq + r] * sc);
        *reinterpret_cast<s16x4*>(dqr + d) = w;
      } else {
        f32x4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = dq[db][4 * gq + r] * sc;
        *reinterpret_cast<f32x4*>(dqr + d) = w;
      }
    }
  }
}

// ---------------------------------------------------------------------------
template <typename Tag, int D, int MODE>
static hipError_t run_bwd_dkdv16(const fa_bwd_params& p, hipStream_t stream) {
  using C = Dkdv16Cfg<D>;
  auto kern = dkdv16_kernel<Tag, D, MODE>;
  hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
  if (e != hipSuccess) return e;
  const int nnb = (p.fwd.seqlen_k + C::BN - 1) / C::BN;
  const long grid = (long)nnb * p.fwd.batch * p.fwd.heads_kv;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nnb);
  return hipGetLastError();
}

template <typename Tag, int D, int OCC, bool PAIR = false, bool VARLEN = false>
static hipError_t launch_dqs16(const fa_bwd_params& p, long grid, int nmb, float dq_scale, int ds_nt,
                               hipStream_t stream) {
  using C = Dqs16Cfg<D, OCC>;
  auto kern = dqs16_kernel<Tag, D, OCC, PAIR, VARLEN>;
  hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nmb, dq_scale, ds_nt);
  return hipGetLastError();
}

template <typename Tag, int D, int MODE>
static hipError_t run_bwd(const fa_bwd_params& p, int phases, hipStream_t stream) {
  const fa_fwd_params& f = p.fwd;
  constexpr bool FAST = !std::is_same<Tag, f32_t>::value && D <= 128;
  bool fast_ok = false;
  if constexpr (FAST)
    fast_ok = buf_rows_ok(f.q_stride[2], Dkdv16Cfg<D>::BMQ) && buf_rows_ok(p.dout_stride[2], Dkdv16Cfg<D>::BMQ) &&
              buf_rows_ok(f.k_stride[2], Dq16Cfg<D>::BN) && buf_rows_ok(f.v_stride[2], Dq16Cfg<D>::BN);
  // With score-gradient scratch the dK/dV kernel stores dS and dQ = dS K
  // runs after it (dqs16_kernel); without it, the full 16-bit backward
  // computes delta inside the dQ kernel, which then runs first.  Otherwise
  // delta has its own kernel.
  bool use_ds = false;
  if constexpr (FAST && D >= 64) {
    const size_t need = bwd_ds_bytes(p);
    use_ds = fast_ok && p.ds_workspace != nullptr && need > 0 && p.ds_workspace_bytes >= (int64_t)need;
  }
  // Scratch too small for every head at once: dK/dV and dQ run in two
  // chunks of KV heads (with their query heads), each reusing the scratch,
  // after one delta pass over all heads, when bwd_ds_chunk_heads allows it.
  // Only whole backwards (both passes in one call) are chunked, and only
  // without the per-head modifiers (MODE 0: causal / window; MODE 3:
  // softcap), whose head index would otherwise shift.
  if constexpr (FAST && D >= 64 && (MODE == 0 || MODE == 3)) {
    if (fast_ok && !use_ds && p.ds_workspace != nullptr && (phases & 6) == 6) {
      const int per = bwd_ds_chunk_heads(p, p.ds_workspace_bytes);
      if (per > 0) {
        if (phases & 1) {
          constexpr int rows = 16 * delta_rows_per_thread<Tag, D>();
          const int nrb = (f.seqlen_q + rows - 1) / rows;
          const int heads_fast = (f.out_stride[1] < f.out_stride[2] && p.dout_stride[1] < p.dout_stride[2] &&
                                  nrb <= 65535 && f.batch <= 65535) ? 1 : 0;
          const dim3 grid = heads_fast ? dim3(f.heads_q, nrb, f.batch) : dim3(nrb, f.batch * f.heads_q);
          hipLaunchKernelGGL((bwd_delta_kernel<Tag, D>), grid, dim3(256), 0, stream, p, heads_fast);
          hipError_t e = hipGetLastError();
          if (e != hipSuccess) return e;
        }
        const int group = f.heads_q / f.heads_kv;
        for (int kv0 = 0; kv0 < f.heads_kv; kv0 += per) {
          const int n = std::min(per, f.heads_kv - kv0);
          const int64_t h0 = (int64_t)kv0 * group;
          fa_bwd_params c = p;
          auto shift = [](const void* ptr, int64_t elems) {
            return static_cast<const void*>(static_cast<const uint16_t*>(ptr) + elems);
          };
          c.fwd.q = shift(f.q, h0 * f.q_stride[1]);
          c.fwd.k = shift(f.k, kv0 * f.k_stride[1]);
          c.fwd.v = shift(f.v, kv0 * f.v_stride[1]);
          c.fwd.out = const_cast<void*>(shift(f.out, h0 * f.out_stride[1]));
          c.fwd.lse = f.lse + h0 * f.lse_stride[1];
          c.dout = shift(p.dout, h0 * p.dout_stride[1]);
          c.delta = p.delta + h0 * p.delta_stride[1];
          c.dq = const_cast<void*>(shift(p.dq, h0 * p.dq_stride[1]));
          c.dk = const_cast<void*>(shift(p.dk, kv0 * p.dk_stride[1]));
          c.dv = const_cast<void*>(shift(p.dv, kv0 * p.dv_stride[1]));
          c.fwd.heads_kv = n;
          c.fwd.heads_q = n * group;
          hipError_t e = run_bwd<Tag, D, MODE>(c, 6, stream);
          if (e != hipSuccess) return e;
        }
        return hipSuccess;
      }
    }
  }
  const bool fused_delta = fast_ok && !use_ds && (phases & 1) && (phases & 4);
  if ((phases & 1) && !fused_delta) {
    constexpr int rows = 16 * delta_rows_per_thread<Tag, D>();
    const int nrb = (f.seqlen_q + rows - 1) / rows;
    const int heads_fast = (f.out_stride[1] < f.out_stride[2] && p.dout_stride[1] < p.dout_stride[2] &&
                            nrb <= 65535 && f.batch <= 65535) ? 1 : 0;
    const dim3 grid = heads_fast ? dim3(f.heads_q, nrb, f.batch) : dim3(nrb, f.batch * f.heads_q);
    hipLaunchKernelGGL((bwd_delta_kernel<Tag, D>), grid, dim3(256), 0, stream, p, heads_fast);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if constexpr (FAST) {
  if (fast_ok) {
    if constexpr (D >= 64) {
    if ((phases & 4) && use_ds) {
      // dQ from the dS the dK/dV pass stored: runs after it.
      if (phases & 2) {
        hipError_t e = run_bwd_dkdv16<Tag, D, MODE>(p, stream);
        if (e != hipSuccess) return e;
        phases &= ~2;
      }
      const int nmb = (f.seqlen_q + Dqs16Cfg<D, 1>::BM - 1) / Dqs16Cfg<D, 1>::BM;
      const long grid = (long)nmb * f.batch * f.heads_q;
      // MODE 3 stores dS / 4 (its softcap factor is (1 - tanh^2) / 4).
      const float dq_scale = f.softmax_scale * (MODE == 3 ? 4.f : 1.f);
      // A scratch bound above twice the 256 MiB memory-side cache: the dS
      // comes from HBM either way, and nontemporal loads keep it out of L2
      // (config 5, 3.0 GB bound: dQ 303.5 -> 295.2 us).  Below it the plain
      // loads hit the dS the dK/dV pass left in that cache (config 2, 268 MB
      // bound: 36 against 39 us with nontemporal loads).
      const int ds_nt = bwd_ds_bytes(p) > (size_t(512) << 20) ? 1 : 0;
      // Two workgroups per CU (D = 128) once the launch spans more than
      // three rounds of one workgroup per CU; below that, heavy and light
      // query blocks of a head paired in one workgroup when the pairs still
      // give every CU one (config 2: dQ 37.8 -> 36.9 us, same results).
      auto launch_all = [&](auto varlen_t) -> hipError_t {
        constexpr bool VL = decltype(varlen_t)::value;
        if constexpr (D >= 128) {
          const long cus = device_cu_count();
          const long pairs = (long)((nmb + 1) / 2) * f.batch * f.heads_q;
          if (grid > 3L * cus) return launch_dqs16<Tag, D, 2, false, VL>(p, grid, nmb, dq_scale, ds_nt, stream);
          if (pairs >= cus) return launch_dqs16<Tag, D, 1, true, VL>(p, pairs, nmb, dq_scale, ds_nt, stream);
        }
        return launch_dqs16<Tag, D, 1, false, VL>(p, grid, nmb, dq_scale, ds_nt, stream);
      };
      hipError_t e = f.cu_seqlens_q ? launch_all(std::true_type{}) : launch_all(std::false_type{});
      if (e != hipSuccess) return e;
      // Varlen: a sequence longer than max_seqlen / total promised has no
      // room in the scratch; dQ from dS left its heads alone and they get
      // the recomputed dQ here (one workgroup per sequence, which returns at
      // once when its last head's region fit, and so all of them).  Dense
      // scratch is sized exactly, so no such head exists.
      if (f.cu_seqlens_q) {
        using CQ = Dq16Cfg<D>;
        auto kq = dq16_kernel<Tag, D, MODE>;
        e = allow_lds((const void*)kq, CQ::LDS_BYTES);
        if (e != hipSuccess) return e;
        const int nq = (f.seqlen_q + CQ::BM - 1) / CQ::BM;
        hipLaunchKernelGGL(kq, dim3((unsigned)f.batch), dim3(CQ::NT), CQ::LDS_BYTES, stream, p, nq, 2);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
    }
    }
    if ((phases & 4) && !use_ds) {
      using C = Dq16Cfg<D>;
      auto kern = dq16_kernel<Tag, D, MODE>;
      hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
      if (e != hipSuccess) return e;
      const int nmb = (f.seqlen_q + C::BM - 1) / C::BM;
      const long grid = (long)nmb * f.batch * f.heads_q;
      hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nmb, fused_delta ? 1 : 0);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if (phases & 2) {
      // Without dS scratch the kernel must not store dS (ds_workspace is
      // only honoured when its size was checked above).
      fa_bwd_params q = p;
      if (!use_ds) q.ds_workspace = nullptr;
      hipError_t e = run_bwd_dkdv16<Tag, D, MODE>(q, stream);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  }
  constexpr int GMODE = MODE == 3 ? 1 : MODE;  // no softcap-only generic variant
  if (phases & 2) {
    using C = DkdvCfg<Tag, D>;
    auto kern = bwd_dkdv_kernel<Tag, D, GMODE>;
    hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
    if (e != hipSuccess) return e;
    const int nnb = (f.seqlen_k + C::BN - 1) / C::BN;
    const long grid = (long)nnb * f.batch * f.heads_kv * (D / C::DO);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nnb);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (phases & 4) {
    using C = DqCfg<Tag, D>;
    auto kern = bwd_dq_kernel<Tag, D, GMODE>;
    hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
    if (e != hipSuccess) return e;
    const int nmb = (f.seqlen_q + C::BM - 1) / C::BM;
    const long grid = (long)nmb * f.batch * f.heads_q * (D / C::DO);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nmb);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <typename Tag, int MODE>
static hipError_t bwd_by_dim(const fa_bwd_params& p, int ph, hipStream_t s) {
  switch (p.fwd.head_dim) {
    case 32: return run_bwd<Tag, 32, MODE>(p, ph, s);
    case 64: return run_bwd<Tag, 64, MODE>(p, ph, s);
    case 128: return run_bwd<Tag, 128, MODE>(p, ph, s);
    case 256: return run_bwd<Tag, 256, MODE>(p, ph, s);
    case 512: return run_bwd<Tag, 512, MODE>(p, ph, s);
  }
  return hipErrorInvalidValue;
}

template <typename Tag>
hipError_t bwd_by_mods(const fa_bwd_params& p, int ph, hipStream_t s) {
  const fa_fwd_params& f = p.fwd;
  if (f.dropout_p > 0.f) return bwd_by_dim<Tag, 2>(p, ph, s);
  if constexpr (!std::is_same<Tag, f32_t>::value)
    if (f.softcap > 0.f && !f.bias && !f.alibi_slopes) return bwd_by_dim<Tag, 3>(p, ph, s);
  if (f.softcap > 0.f || f.bias || f.alibi_slopes) return bwd_by_dim<Tag, 1>(p, ph, s);
  return bwd_by_dim<Tag, 0>(p, ph, s);
}

}  // namespace fa
