#pragma once
// Kernel templates of fa_fwd; instantiated per dtype by fa_fwd_<dtype>.hip.
// fa_fwd.hip - FlashAttention-2 forward (dense and packed varlen) for gfx950.
//
// Follows the algorithm of the reference's `_attention_forward` /
// `_attention_forward_varlen` (fa_rdna3/kernels/forward.py:28-164,
// varlen.py:41-149, inner loop _common.py:233-345): exp2 online softmax over
// key tiles, output normalised by the row sum, LSE = m*ln2 + ln(l).
//
// MI355X layout.  A workgroup is 4 waves; each wave owns 32 query rows, so a
// workgroup covers BM = 128 rows of one (batch, head).  Scores are computed
// TRANSPOSED, S^T = K Q^T (keys x queries), with v_mfma_f32_32x32x16: the
// query then lives on the lane (column) axis, so the row max / row sum of the
// softmax are a per-lane reduction over registers plus a single swap with the
// lane 32 apart, and the rescale of O^T = V^T P^T is a per-lane scalar.  Q^T is
// the B operand and stays in registers for the whole kernel; K (row-major) and
// V^T (transposed on the way into LDS) are double-buffered in LDS and shared
// by the 4 waves; P^T goes from the accumulator straight back into the B
// operand of the P.V MFMA without touching LDS.
//
// Work order: the m-block index is the slowest-varying grid coordinate and is
// walked from the last block down, so under causal masking the longest
// workgroups are dispatched first.
#include <type_traits>

#include "fa_internal.hpp"
#include "fa_tiles.hpp"
#include "fa_fwd16.hpp"

namespace fa {


template <typename Tag, int D>
struct FwdCfg {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int NW = 4;
  static constexpr int NT = 64 * NW;
  static constexpr int BM = 32 * NW;
  static constexpr int BN = (D <= 128) ? 64 : 32;
  // Output columns per workgroup: D > 128 splits O^T over the grid (each
  // split recomputes the scores) to bound the accumulator registers.
  static constexpr int DO = (D <= 128) ? D : ((sizeof(S) == 4 && D == 512) ? 64 : 128);
  static constexpr bool QREG = (sizeof(S) == 2) ? (D <= 256) : (D <= 128);
  static constexpr int KLD = D + EL::CE;   // K tile row stride (elements)
  static constexpr int VLD = BN + EL::CE;  // V^T tile row stride
  static constexpr int KTILE = BN * KLD;
  static constexpr int VTILE = DO * VLD;
  static constexpr int STAGE = KTILE + VTILE;
  static constexpr int LDS_BYTES = 2 * STAGE * (int)sizeof(S);
  static constexpr int NSTEP = D / EL::KSTEP;   // MFMA k-steps over D
  static constexpr int NKB = BN / 32;           // 32-key accumulator blocks
  static constexpr int NPV = BN / (2 * EL::E);  // P.V MFMAs per d-block
  static constexpr int NDB = DO / 32;           // 32-wide output blocks
};

template <typename Tag, int D, int MODE>
__global__ __launch_bounds__(256) void fwd_kernel(fa_fwd_params p, int num_m_blocks) {
  using C = FwdCfg<Tag, D>;
  using EL = Elem<Tag>;
  using S = typename EL::S;
  using Op = typename EL::Op;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  S* smem = reinterpret_cast<S*>(smem_raw);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;

  const int ndc = D / C::DO;
  const int bh_count = p.batch * p.heads_q;
  const int id = blockIdx.x;
  const int mb_rev = id / (bh_count * ndc);
  const int rest = id - mb_rev * bh_count * ndc;
  const int bh = rest / ndc, dc = rest - (rest / ndc) * ndc;
  const int b = bh / p.heads_q, hq = bh - b * p.heads_q;
  const int hk = hq / (p.heads_q / p.heads_kv);
  const int mblk = num_m_blocks - 1 - mb_rev;

  int q_start = 0, sq = p.seqlen_q, k_start = 0, sk = p.seqlen_k;
  if (p.cu_seqlens_q) {
    bounded_seq(p.cu_seqlens_q, b, p.total_q, q_start, sq);
    bounded_seq(p.cu_seqlens_k, b, p.total_k, k_start, sk);
  }
  const int m0 = mblk * C::BM;
  if (m0 >= sq) return;  // uniform: past the end of a short varlen sequence

  const S* qb = reinterpret_cast<const S*>(p.q) + b * p.q_stride[0] + hq * p.q_stride[1] +
                (int64_t)q_start * p.q_stride[2];
  const S* kb = reinterpret_cast<const S*>(p.k) + b * p.k_stride[0] + hk * p.k_stride[1] +
                (int64_t)k_start * p.k_stride[2];
  const S* vb = reinterpret_cast<const S*>(p.v) + b * p.v_stride[0] + hk * p.v_stride[1] +
                (int64_t)k_start * p.v_stride[2] + dc * C::DO;
  S* ob = reinterpret_cast<S*>(p.out) + b * p.out_stride[0] + hq * p.out_stride[1] +
          (int64_t)q_start * p.out_stride[2];
  float* lb = p.lse + b * p.lse_stride[0] + hq * p.lse_stride[1] + (int64_t)q_start * p.lse_stride[2];
  const int64_t qs = p.q_stride[2], ks = p.k_stride[2], vs = p.v_stride[2];

  const Mods md = make_mods(p, b, hq, sq, sk);

  // Key range of the workgroup (reference forward.py:92-127, tightened to the
  // rows that exist).
  const int mlast = min(m0 + C::BM, sq) - 1;
  int lo = 0, hi = sk;
  if (p.causal) hi = min(hi, mlast + md.off + 1);
  if (p.window_right >= 0) hi = min(hi, mlast + md.off + p.window_right + 1);
  if (p.window_left >= 0) lo = max(0, m0 + md.off - p.window_left);
  lo = lo / C::BN * C::BN;
  const int ntiles = hi > lo ? (hi - lo + C::BN - 1) / C::BN : 0;

  // This wave's query rows.
  const int m0w = m0 + 32 * wave;
  const int mrows = min(32, sq - m0w);  // <= 0: the wave only helps load
  const int m = m0w + l32;
  const bool mvalid = m < sq;

  Op qop[C::QREG ? C::NSTEP : 1];
  const S* qrow = qb + (int64_t)(mvalid ? m : 0) * qs + EL::E * h;
  if constexpr (C::QREG) {
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s)
      qop[s] = mvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
    wait_vm_all();
  }

  float m_i = kNegInf, l_i = 0.f;
  f32x16 acc[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) acc[i] = zero16();

  RowTile<Tag, C::BN, D, C::NT> kt;
  TransTile<Tag, C::BN, C::DO, C::NT> vt;

  auto load_tiles = [&](int n0) {
    kt.load([&](int r) -> const S* { int n = n0 + r; return n < sk ? kb + (int64_t)n * ks : nullptr; }, kb, tid);
    vt.load([&](int r) -> const S* { int n = n0 + r; return n < sk ? vb + (int64_t)n * vs : nullptr; }, vb, tid);
  };
  auto store_tiles = [&](int stage) {
    S* base = smem + stage * C::STAGE;
    kt.store(base, C::KLD, tid);
    vt.store(base + C::KTILE, C::VLD, tid);
  };

  if (ntiles > 0) {
    load_tiles(lo);
    store_tiles(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int n0 = lo + t * C::BN;
    const int stage = t & 1;
    if (t + 1 < ntiles) load_tiles(n0 + C::BN);

    const int vis = mrows > 0 ? rect_visibility(md, m0w, mrows, n0, C::BN) : 0;
    if (vis) {
      const S* Ks = smem + stage * C::STAGE;
      const S* Vs = Ks + C::KTILE;
      f32x16 sacc[C::NKB];
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
        sacc[kb2] = zero16();
        const S* krow = Ks + (kb2 * 32 + l32) * C::KLD + EL::E * h;
#pragma unroll
        for (int s = 0; s < C::NSTEP; ++s) {
          Op a = load_op<Tag>(krow + EL::KSTEP * s);
          Op bq;
          if constexpr (C::QREG) bq = qop[s];
          else bq = mvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
          sacc[kb2] = EL::mma(a, bq, sacc[kb2]);
        }
      }
      // Scores in the log2 domain, masked, and the tile max per query.
      float tmax = kNegInf;
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int n = n0 + kb2 * 32 + acc_row(i, h);
          float tc;
          float x = score<(MODE >= 1)>(md, sacc[kb2][i], m, n, tc);
          if (vis == 1 && !keep_pos(md, m, n)) x = kNegInf;
          sacc[kb2][i] = x;
          tmax = fmaxf(tmax, x);
        }
      }
      tmax = half_max(tmax);
      const float m_new = fmaxf(m_i, tmax);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;  // safe softmax
      const float alpha = exp2f(m_i - m_use);
      float rsum = 0.f;
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = exp2f(sacc[kb2][i] - m_use);
          sacc[kb2][i] = pv;
          rsum += pv;
        }
      }
      rsum = half_sum(rsum);
      l_i = l_i * alpha + rsum;
      m_i = m_new;
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) acc[db] *= alpha;
      if constexpr (MODE == 2) {
        if (md.drop_p > 0.f) {
#pragma unroll
          for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int n = n0 + kb2 * 32 + acc_row(i, h);
              sacc[kb2][i] = dropout_keep(md, m, n) ? sacc[kb2][i] * md.drop_scale : 0.f;
            }
        }
      }
      // O^T += V^T P^T.  bf16 keeps only 8 mantissa bits, so P is fed as
      // hi + lo bf16 parts (two MFMAs on the same V^T operand); the product
      // then carries P to ~2^-17 and the output error is dominated by the
      // final rounding of O.
      constexpr bool PSPLIT = std::is_same<Tag, bf16_t>::value;
      Op pb[C::NPV], pl[PSPLIT ? C::NPV : 1];
      constexpr int J = 16 / EL::E;  // MFMAs per 32-key accumulator block
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) pb[j] = pack_op<Tag>(sacc[j / J], j % J);
      if constexpr (PSPLIT) {
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) sacc[kb2][i] -= EL::to_f(EL::from_f(sacc[kb2][i]));
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) pl[j] = pack_op<Tag>(sacc[j / J], j % J);
      }
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        const S* vrow = Vs + (db * 32 + l32) * C::VLD;
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) {
          const Op a = lds_op_rowmap<Tag>(vrow, j, h);
          acc[db] = EL::mma(a, pb[j], acc[db]);
          if constexpr (PSPLIT) acc[db] = EL::mma(a, pl[j], acc[db]);
        }
      }
    }

    if (t + 1 < ntiles) store_tiles(stage ^ 1);
    __syncthreads();
  }

  if (!mvalid) return;
  const float l_safe = (l_i == 0.f) ? 1.f : l_i;
  const float inv = 1.f / l_safe;
  S* orow = ob + (int64_t)m * p.out_stride[2] + dc * C::DO;
#pragma unroll
  for (int db = 0; db < C::NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = db * 32 + 8 * g + 4 * h;
      if constexpr (sizeof(S) == 2) {
        s16x4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = (short)EL::from_f(acc[db][4 * g + r] * inv);
        *reinterpret_cast<s16x4*>(orow + d) = w;
      } else {
        f32x4 w;
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = acc[db][4 * g + r] * inv;
        *reinterpret_cast<f32x4*>(orow + d) = w;
      }
    }
  }
  if (h == 0 && dc == 0)
    lb[(int64_t)m * p.lse_stride[2]] = (m_i == kNegInf) ? kNegInf : (m_i + __log2f(l_safe)) * kLn2;
}

template <typename Tag, int D, int MODE, int NH, bool PAIR = false>
static hipError_t launch_fwd16(const fa_fwd_params& p, long grid, int nmb, hipStream_t stream) {
  using C = Fwd16Cfg<D, NH>;
  auto kern = fwd16_kernel<Tag, D, MODE, NH, PAIR>;
  hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nmb);
  return hipGetLastError();
}

template <typename Tag, int D, int MODE>
static hipError_t run_fwd(const fa_fwd_params& p, hipStream_t stream) {
  if constexpr (!std::is_same<Tag, f32_t>::value && D <= 128) {
    using C = Fwd16Cfg<D>;
    if (buf_rows_ok(p.k_stride[2], C::BN) && buf_rows_ok(p.v_stride[2], C::BN)) {
    const int nmb = (p.seqlen_q + C::BM - 1) / C::BM;
    const long grid = (long)nmb * p.batch * p.heads_q;
    if (grid <= 0) return hipSuccess;
    // One key half, two workgroups per CU, for packed varlen batches and for
    // dense grids of more than eight rounds of one 8-wave workgroup per CU.
    // (Varlen always: a sequence's output then does not depend on the batch
    // it is packed with.  The two forms sum the key tiles in different
    // orders, so they agree to rounding, not bit for bit.)
    if (p.cu_seqlens_q || grid > 8L * device_cu_count())
      return launch_fwd16<Tag, D, MODE, 1>(p, grid, nmb, stream);
    // Heavy and light row blocks of a head paired in one workgroup, when
    // the pairs still give every CU a workgroup (config 2: 256 pairs):
    // forward 52.5 -> 51.4 us, same results bit for bit.
    const long pairs = (long)((nmb + 1) / 2) * p.batch * p.heads_q;
    if (pairs >= device_cu_count()) return launch_fwd16<Tag, D, MODE, 2, true>(p, pairs, nmb, stream);
    return launch_fwd16<Tag, D, MODE, 2>(p, grid, nmb, stream);
    }
  }
  // The generic kernel has no softcap-only variant (MODE 3 is MODE 1 there).
  constexpr int GMODE = MODE == 3 ? 1 : MODE;
  using C = FwdCfg<Tag, D>;
  auto kern = fwd_kernel<Tag, D, GMODE>;
  hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
  if (e != hipSuccess) return e;
  const int nmb = (p.seqlen_q + C::BM - 1) / C::BM;
  const long grid = (long)nmb * p.batch * p.heads_q * (D / C::DO);
  if (grid <= 0) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, stream, p, nmb);
  return hipGetLastError();
}

template <typename Tag, int MODE>
static hipError_t fwd_by_dim(const fa_fwd_params& p, hipStream_t s) {
  switch (p.head_dim) {
    case 32: return run_fwd<Tag, 32, MODE>(p, s);
    case 64: return run_fwd<Tag, 64, MODE>(p, s);
    case 128: return run_fwd<Tag, 128, MODE>(p, s);
    case 256: return run_fwd<Tag, 256, MODE>(p, s);
    case 512: return run_fwd<Tag, 512, MODE>(p, s);
  }
  return hipErrorInvalidValue;
}

template <typename Tag>
hipError_t fwd_by_mods(const fa_fwd_params& p, hipStream_t s) {
  // 0: plain, 1: softcap / bias / ALiBi, 2: also dropout (Philox per score),
  // 3: softcap without bias or ALiBi (16-bit kernels; one score variant).
  if (p.dropout_p > 0.f) return fwd_by_dim<Tag, 2>(p, s);
  if constexpr (!std::is_same<Tag, f32_t>::value)
    if (p.softcap > 0.f && !p.bias && !p.alibi_slopes) return fwd_by_dim<Tag, 3>(p, s);
  if (p.softcap > 0.f || p.bias || p.alibi_slopes) return fwd_by_dim<Tag, 1>(p, s);
  return fwd_by_dim<Tag, 0>(p, s);
}

}  // namespace fa
