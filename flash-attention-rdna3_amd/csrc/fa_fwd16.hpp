// fa_fwd16.hpp - forward kernel specialised for 16-bit inputs and D <= 128.
//
// Same algorithm and results as fwd_kernel (exp2 online softmax,
// LSE = m*ln2 + ln l; reference kernels/forward.py:28-164 and
// _common.py:233-345), organised for throughput on gfx950:
//  * K and V tiles sit row-major in LDS with an XOR chunk swizzle (no
//    padding, conflict-free reads); S^T = K Q^T reads K with ds_read_b128 and
//    O^T += V^T P^T reads V^T straight from the row-major tile with
//    ds_read_b64_tr_b16, so nothing is transposed through registers;
//  * tiles strictly inside the visible region take an unmasked path whose
//    per-score work is one FMA + one exp2 + max/sum;
//  * the running max is updated lazily: P = exp2(s*c - m) is accepted while
//    the tile max stays within 2^8 of m, and O, l are rescaled (wave-wide)
//    only when some row's max grows past that, so the O^T rescale leaves the
//    steady-state loop.  The result is identical up to rounding: O and l are
//    both expressed relative to the same m, and the final O / l and
//    lse = (m + log2 l) * ln2 do not depend on which m was used.
#pragma once

#include <type_traits>

#include "fa_internal.hpp"
#include "fa_tiles.hpp"

namespace fa {

// A workgroup owns BM = 128 query rows (4 row quarters of 32, one per wave)
// and splits their key range in two: waves 0-3 stream the first half of the
// key tiles, waves 4-7 the second, each half through its own double-buffered
// K/V tiles.  The two partial states (O, m, l) of a row are merged through
// LDS at the end.  One 8-wave workgroup fills a CU at two waves per SIMD, so
// a heavy causal block runs at full CU throughput instead of sharing the CU
// with a light one and then running alone.
//
// NH = 1 is the same kernel with one key half: 4 waves walk all key tiles of
// the 128 rows and no merge is needed.  Its 64 KiB of LDS and 4 waves let two
// workgroups share a CU, so one workgroup's prologue (Q and first tiles) and
// epilogue (output store) overlap the other's steady state.  It is launched
// when the grid spans many rounds of workgroups (a packed varlen batch),
// where that per-workgroup cost adds up; a short causal batch keeps NH = 2,
// whose key split lets a heavy block use the whole CU.
template <int D, int NH = 2>
struct Fwd16Cfg {
  static constexpr int NQ = 4;                 // row quarters (waves per half)
  static constexpr int NW = NH * NQ;
  static constexpr int NT = 64 * NW;
  static constexpr int NTH = 64 * NQ;          // threads per key half
  static constexpr int BM = 32 * NQ;
  static constexpr int BN = 64;
  static constexpr int KTILE = BN * D;  // elements (K), then V
  static constexpr int STAGE = 2 * KTILE;
  static constexpr int HALF = 2 * STAGE;       // two stages per key half
  static constexpr int MERGE_BYTES = NH == 1 ? 0 : NQ * (D / 32) * 16 * 64 * 4 + 2 * NQ * 64 * 4;
  static constexpr int LOOP_BYTES = NH * HALF * 2;
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
  static constexpr int NSTEP = D / 16;
  static constexpr int NKB = BN / 32;
  static constexpr int NPV = BN / 16;
  static constexpr int NDB = D / 32;
};

// Largest growth of the running max (log2 domain) absorbed without rescaling.
constexpr float kLazyRescale = 8.0f;

// One work item: the 128 query rows of row block (num_m_blocks - 1 - mb_rev)
// of (batch, head) bh, item = mb_rev * B * Hq + bh.  `end_barrier`: the
// workgroup runs another item after this one, so every wave passes a
// barrier once this item's LDS use (merge, staged stores) is over.
template <typename Tag, int D, int MODE, int NH>
__device__ __forceinline__ void fwd16_item(const fa_fwd_params& p, int num_m_blocks, int item,
                                           unsigned char* smem_raw, bool end_barrier) {
  using C = Fwd16Cfg<D, NH>;
  using EL = Elem<Tag>;
  using S = uint16_t;
  S* smem = reinterpret_cast<S*>(smem_raw);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave8 = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int khalf = wave8 / C::NQ;        // which half of the key tiles
  const int wave = wave8 % C::NQ;         // row quarter
  const int htid = tid % C::NTH;          // thread index within the key half
  const int h = lane >> 5, l32 = lane & 31;

  const int bh_count = p.batch * p.heads_q;
  const int mb_rev = item / bh_count;
  const int bh = item - mb_rev * bh_count;
  const int b = bh / p.heads_q, hq = bh - b * p.heads_q;
  const int hk = hq / (p.heads_q / p.heads_kv);
  const int mblk = num_m_blocks - 1 - mb_rev;  // heaviest causal blocks first

  int q_start = 0, sq = p.seqlen_q, k_start = 0, sk = p.seqlen_k;
  if (p.cu_seqlens_q) {
    bounded_seq(p.cu_seqlens_q, b, p.total_q, q_start, sq);
    bounded_seq(p.cu_seqlens_k, b, p.total_k, k_start, sk);
  }
  const int m0 = mblk * C::BM;
  if (m0 >= sq) return;

  const S* qb = reinterpret_cast<const S*>(p.q) + b * p.q_stride[0] + hq * p.q_stride[1] +
                (int64_t)q_start * p.q_stride[2];
  const S* kb = reinterpret_cast<const S*>(p.k) + b * p.k_stride[0] + hk * p.k_stride[1] +
                (int64_t)k_start * p.k_stride[2];
  const S* vb = reinterpret_cast<const S*>(p.v) + b * p.v_stride[0] + hk * p.v_stride[1] +
                (int64_t)k_start * p.v_stride[2];
  const int64_t qs = p.q_stride[2], ks = p.k_stride[2], vs = p.v_stride[2];
  const Mods md = make_mods(p, b, hq, sq, sk);
  const float c = md.scale_log2;

  const int mlast = min(m0 + C::BM, sq) - 1;
  int lo = 0, hi = sk;
  if (p.causal) hi = min(hi, mlast + md.off + 1);
  if (p.window_right >= 0) hi = min(hi, mlast + md.off + p.window_right + 1);
  if (p.window_left >= 0) lo = max(0, m0 + md.off - p.window_left);
  lo = lo / C::BN * C::BN;
  const int ntiles = hi > lo ? (hi - lo + C::BN - 1) / C::BN : 0;

  const int m0w = m0 + 32 * wave;
  const int mrows = min(32, sq - m0w);
  const int m = m0w + l32;
  const bool mvalid = m < sq;

  s16x8 qop[C::NSTEP];

  float m_i = kNegInf, l_i = 0.f;
  f32x16 acc[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) acc[i] = zero16();

  DmaSwzTile<C::BN, D, C::NTH> kt, vt;
  kt.init(ks, htid);
  vt.init(vs, htid);
  // Both halves run nh0 steps so their barriers line up.
  const int nh0 = NH == 1 ? ntiles : (ntiles + 1) / 2;
  // Half 0 takes the even key tiles, half 1 the odd ones: the two masked
  // diagonal tiles of a causal block then fall into the same step instead of
  // two steps in which half 0 waits for half 1.
  const int my_first = khalf;
  constexpr int TSTEP = NH;
  const int my_count = NH == 1 ? ntiles : khalf == 0 ? nh0 : ntiles - nh0;
  const uint32_t lds0 = lds_addr(smem) + (uint32_t)(khalf * C::HALF) * 2u;
  // Tile sources advance by BN rows per load (scalar pointer arithmetic).
  int n_next = lo + my_first * C::BN;
  const S* k_next = kb + (int64_t)n_next * ks;
  const S* v_next = vb + (int64_t)n_next * vs;
  auto load_tiles = [&](int stage) {
    const int rows = min(C::BN, sk - n_next);
    const uint32_t base = lds0 + (uint32_t)(stage * C::STAGE) * 2u;
    kt.load(rows_rsrc_words<D>(k_next, ks, rows), base, wave);
    vt.load(rows_rsrc_words<D>(v_next, vs, rows), base + C::KTILE * 2u, wave);
    n_next += TSTEP * C::BN;
    k_next += (int64_t)(TSTEP * C::BN) * ks;
    v_next += (int64_t)(TSTEP * C::BN) * vs;
  };
  const VisBounds vbnd = row_block_bounds(md, m0w, mrows);

  // The first tiles' DMA and the Q loads share one round trip to memory.
  if (my_count > 0) load_tiles(0);
  {
    const S* qrow = qb + (int64_t)(mvalid ? m : 0) * qs + 8 * h;
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) qop[s] = load_op<Tag>(qrow + 16 * s);
    wait_vm_all();
    if (!mvalid) {
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s) qop[s] = zero_op<Tag>();
    }
  }
  __syncthreads();

  for (int t = 0; t < nh0; ++t) {
    const int n0 = lo + (my_first + TSTEP * t) * C::BN;
    const int stage = t & 1;
    const int vis = t < my_count ? bounds_vis(vbnd, n0, n0 + C::BN - 1) : 0;
    if (!vis && t + 1 < my_count) load_tiles(stage ^ 1);
    if (vis) {
      const S* Ks = smem + khalf * C::HALF + stage * C::STAGE;
      const S* Vs = Ks + C::KTILE;
      f32x16 sacc[C::NKB];
#pragma unroll
      for (int kb2 = 0; kb2 < C::NKB; ++kb2) sacc[kb2] = zero16();
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s)
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
          sacc[kb2] = EL::mma(swz_op<D>(Ks, kb2 * 32 + l32, 2 * s + h), qop[s], sacc[kb2]);
      sched_read_ahead<C::NSTEP * C::NKB, 4>();
      // The next tile's loads go out while the score MFMAs drain (issuing
      // them before the MFMAs would hold the MFMAs back behind the queue).
      if (t + 1 < my_count) load_tiles(stage ^ 1);

      // Scores -> log2 domain (masked or modified when needed), tile max.
      float tmax = kNegInf;
      const bool plain = (MODE == 0) && vis == 2 && c > 0.f;
      if (plain) {
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sacc[kb2][i]);
        tmax *= c;  // the plain path is only taken for c > 0
      } else {
        // This lane's visible keys (its row is fixed): one interval per tile.
        int klo = INT_MIN, khi = INT_MAX;
        if (vis == 1) key_bounds(md, m, klo, khi);
        const Span ks = make_span(klo, khi, n0 + 4 * h);
        // MASK: the tile is partly visible (vis == 1); a fully visible tile
        // with modifiers skips the per-score interval test.
        auto masked_scores = [&](auto cap_t, auto bias_t, auto alibi_t, auto mask_t) {
#pragma unroll
          for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int n = n0 + kb2 * 32 + acc_row(i, h);
              float tc;
              float x = score_m<decltype(cap_t)::value, decltype(bias_t)::value, decltype(alibi_t)::value>(
                  md, sacc[kb2][i], m, n, tc);
              if constexpr (decltype(mask_t)::value) x = in_span(ks, kb2 * 32 + acc_row(i, 0)) ? x : kNegInf;
              sacc[kb2][i] = x;
              tmax = fmaxf(tmax, x);
            }
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        if constexpr (MODE == 3) {
          // Softcap only.  The tile keeps the softcap's r (x = cap2 - 2 cap2 r
          // falls as r grows, a hidden score is r = +inf): the row max comes
          // from the least r and exp2(x - m) is one FMA on r.
          float rmin = __builtin_inff();
          auto rscores = [&](auto mask_t) {
#pragma unroll
            for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                float r = softcap_r(md, sacc[kb2][i]);
                if constexpr (decltype(mask_t)::value) r = in_span(ks, kb2 * 32 + acc_row(i, 0)) ? r : __builtin_inff();
                sacc[kb2][i] = r;
                rmin = fminf(rmin, r);
              }
          };
          if (vis == 1) rscores(T_{});
          else rscores(F_{});
          tmax = __builtin_fmaf(md.cap2_m2, rmin, md.cap2);
        } else if constexpr (MODE == 1) {
          if (vis == 1) dispatch_mods(md, [&](auto a, auto b_, auto c_) { masked_scores(a, b_, c_, T_{}); });
          else dispatch_mods(md, [&](auto a, auto b_, auto c_) { masked_scores(a, b_, c_, F_{}); });
        } else if constexpr (MODE == 2) {
          // (one variant: the dropout kernel has no registers to spare)
          dispatch_mods(md, [&](auto a, auto b_, auto c_) { masked_scores(a, b_, c_, T_{}); });
        } else {
          masked_scores(F_{}, std::integral_constant<int, 0>{}, F_{}, T_{});
        }
      }
      tmax = half_max(tmax);
      // Lazy rescale, decided for the whole wave.
      if (__builtin_amdgcn_ballot_w64(tmax > m_i + kLazyRescale)) {
        const float m_new = fmaxf(m_i, tmax);
        const float alpha = (m_new == kNegInf) ? 1.f : __builtin_amdgcn_exp2f(m_i - m_new);
        l_i *= alpha;
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) acc[db] *= alpha;
        m_i = m_new;
      }
      const float m_use = (m_i == kNegInf) ? 0.f : m_i;
      float rsum = 0.f;
      if (plain) {
        const float mc = -m_use;
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb2][i], c, mc));
            sacc[kb2][i] = pv;
            rsum += pv;
          }
      } else if constexpr (MODE == 3) {
        const float cm = md.cap2 - m_use;
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(md.cap2_m2, sacc[kb2][i], cm));
            sacc[kb2][i] = pv;
            rsum += pv;
          }
      } else {
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = __builtin_amdgcn_exp2f(sacc[kb2][i] - m_use);
            sacc[kb2][i] = pv;
            rsum += pv;
          }
      }
      rsum = half_sum(rsum);
      l_i += rsum;
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
      // O^T += V^T P^T (bf16: P as hi + lo parts, see fwd_kernel).
      constexpr bool PSPLIT = std::is_same<Tag, bf16_t>::value;
      s16x8 pb[C::NPV], pl[PSPLIT ? C::NPV : 1];
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) pb[j] = pack_op<Tag>(sacc[j >> 1], j & 1);
      if constexpr (PSPLIT) {
#pragma unroll
        for (int kb2 = 0; kb2 < C::NKB; ++kb2)
#pragma unroll
          for (int i = 0; i < 16; ++i) sacc[kb2][i] -= EL::to_f(EL::from_f(sacc[kb2][i]));
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) pl[j] = pack_op<Tag>(sacc[j >> 1], j & 1);
      }
#pragma unroll
      for (int j = 0; j < C::NPV; ++j)
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
          const s16x8 a = tr_op_rowmap<D>(Vs, 0, 32 * db, j, lane);
          acc[db] = EL::mma(a, pb[j], acc[db]);
          if constexpr (PSPLIT) acc[db] = EL::mma(a, pl[j], acc[db]);
        }
      if constexpr (!PSPLIT) sched_read_ahead<C::NPV * C::NDB, 4, 2>();
    }

    wait_vm_all();
    __syncthreads();
  }

  // Merge the two key halves: half 1 parks (O^T, m, l) in LDS, half 0 folds
  // them into its own state.  Both are relative to their own running max.
  if constexpr (NH == 2) {
    float* ow = reinterpret_cast<float*>(smem_raw);
    float* mw = ow + C::NQ * C::NDB * 16 * 64;
    float* lw = mw + C::NQ * 64;
    if (khalf == 1) {
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) park_acc(ow + (wave * C::NDB + db) * 1024, lane, acc[db]);
      mw[wave * 64 + lane] = m_i;
      lw[wave * 64 + lane] = l_i;
    }
    __syncthreads();
    if (khalf == 1) {
      if (end_barrier) __syncthreads();
      return;
    }
    const float mb2 = mw[wave * 64 + lane], lb2 = lw[wave * 64 + lane];
    const float mn = fmaxf(m_i, mb2);
    const float mu = (mn == kNegInf) ? 0.f : mn;
    const float sa = __builtin_amdgcn_exp2f(m_i - mu), sb = __builtin_amdgcn_exp2f(mb2 - mu);
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) {
      const f32x16 o2 = unpark_acc(ow + (wave * C::NDB + db) * 1024, lane);
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[db][i] = acc[db][i] * sa + o2[i] * sb;
    }
    l_i = l_i * sa + lb2 * sb;
    m_i = mn;
  }

  const float l_safe = (l_i == 0.f) ? 1.f : l_i;
  const float inv = 1.f / l_safe;
  // Whole-row output stores through this wave's LDS block: with NH = 2 the
  // block this wave's merge partner parked into (read above), with NH = 1 a
  // stage buffer (every tile read ended at the loop's last barrier).
  S* orow0 = reinterpret_cast<S*>(p.out) + b * p.out_stride[0] + hq * p.out_stride[1] +
             (int64_t)(q_start + m0w) * p.out_stride[2];
  store_rows_staged<Tag, D>(acc, inv, reinterpret_cast<uint16_t*>(smem_raw + wave * C::NDB * 4096), orow0,
                            p.out_stride[2], mrows, lane);
  if (mvalid && h == 0) {
    float* lb = p.lse + b * p.lse_stride[0] + hq * p.lse_stride[1] + (int64_t)(q_start + m) * p.lse_stride[2];
    *lb = (m_i == kNegInf || l_i == 0.f) ? kNegInf : (m_i + __log2f(l_safe)) * kLn2;
  }
  if (end_barrier) __syncthreads();
}

// PAIR: workgroup (j, bh) runs row block j from the heavy end, then row
// block j from the light end, of the same (batch, head): under causal
// masking the two carry the same number of key tiles together, and both
// read the same head's K / V, which the workgroup's XCD then holds in L2.
template <typename Tag, int D, int MODE, int NH, bool PAIR>
__global__ __launch_bounds__(256 * NH, 3 - NH) void fwd16_kernel(fa_fwd_params p, int num_m_blocks) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  if constexpr (!PAIR) {
    fwd16_item<Tag, D, MODE, NH>(p, num_m_blocks, blockIdx.x, smem_raw, false);
  } else {
    const int bh_count = p.batch * p.heads_q;
    const int j = blockIdx.x / bh_count;
    const int bh = blockIdx.x - j * bh_count;
    const int j2 = num_m_blocks - 1 - j;
    fwd16_item<Tag, D, MODE, NH>(p, num_m_blocks, j * bh_count + bh, smem_raw, j2 != j);
    if (j2 != j) fwd16_item<Tag, D, MODE, NH>(p, num_m_blocks, j2 * bh_count + bh, smem_raw, false);
  }
}

}  // namespace fa
