// fa_decode.hip - split-K decode and paged-KV decode for gfx950.
//
// Same results as the reference's `_attention_split` + `_attention_combine`
// (fa_rdna3/kernels/decode.py:9-125) and `_attention_decode_paged`
// (fa_rdna3/kernels/paged.py:16-89): every (sequence, query row) gets
// softmax(q K^T * scale) V over its visible keys, computed per key split as a
// normalised partial O plus a natural-log LSE, then merged with weights
// exp(lse_s - max_s lse) (empty splits, lse = -inf, weigh nothing; an all-empty
// row is zero).  Paged lookups clamp the context to the block-table capacity
// and treat physical ids outside [0, num_blocks) as absent keys
// (reference paged.py:37-38, :58-59).
//
// MI355X layout.  Decode is HBM-bound, so the kernel is organised around
// reading each K/V byte once:
//  * a workgroup owns one (batch, KV head, split) and packs the whole GQA
//    group (group heads x Sq query rows) onto the 32 lanes of the MFMA
//    column axis, so K/V of a KV head are never re-read per query head (the
//    reference re-reads them Hq/Hkv times);
//  * its 4 waves walk interleaved 32-key chunks, each through a wave-private
//    LDS slot (K row-major, V transposed) with the next chunk's 16-byte
//    coalesced loads in flight while the current chunk is computed;
//  * the 4 wave states (max, sum, O^T) are merged in LDS at the end, so one
//    partial per workgroup reaches HBM.  With a single split the merged row
//    is written straight to `out` and no combine kernel runs.
#include <hip/hip_ext.h>

#include <mutex>

#include "fa_internal.hpp"
#include "fa_tiles.hpp"

namespace fa {

struct DecodeArgs {
  const void* q;
  int64_t q_stride[4];  // batch, head, row, dim
  void* out;
  int64_t out_stride[4];
  const void* k;
  const void* v;
  // Contiguous cache: key n of (b, hk) at base + b*s0 + hk*s1 + n*s2.
  // Paged cache:      key n at base + phys*s0 + (n % bs)*s1 + hk*s2,
  //                   phys = block_table[b*bt0 + (n / bs)*bt1].
  int64_t k_stride[3];
  int64_t v_stride[3];
  const int32_t* block_table;
  int64_t bt_stride[2];
  int32_t num_blocks;
  int32_t block_shift;  // log2(block_size)
  const int32_t* lens;  // NULL: every sequence has max_len keys
  int64_t lens_stride;
  int32_t lens_add;     // added to lens[b] before clamping
  int32_t max_len;      // Sk, or max_blocks * block_size when paged
  int32_t batch, heads_q, heads_kv, seqlen_q, head_dim;
  float scale_log2;
  int32_t num_splits;
  int32_t causal;       // bottom-right per sequence: row i sees keys <= len - Sq + i
  int32_t kv8;          // fp8 (OCP e4m3) K/V cache
  float out_scale;      // multiplies the output (v_scale of an fp8 cache); 1 otherwise
  float* ws_o;          // [splits][B][Hq][Sq][D] fp32
  float* ws_lse;        // [splits][B][Hq][Sq] fp32
  uint32_t* tickets;    // NULL: a second launch merges the splits; else per
                        // (b, hk, row block) arrival counters, zero between calls
  int32_t balanced;     // streaming kernel: share num_splits * batch workgroups
                        // out over the sequences by length (needs tickets)
};

}  // namespace fa

#include "fa_decode2.hpp"

namespace fa {

template <typename Tag, int D>
struct DecCfg {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  static constexpr int NW = (D >= 512) ? 2 : 4;  // 4 wave slots of D=512 exceed 160 KiB
  static constexpr int NT = 64 * NW;
  static constexpr int CH = 32;  // keys per wave chunk
  static constexpr int DO = (D <= 128) ? D : 128;
  static constexpr bool QREG = D <= 128;
  static constexpr int KLD = D + EL::CE;
  static constexpr int VLD = CH + EL::CE;
  static constexpr int KT = CH * KLD;
  static constexpr int VT = DO * VLD;
  static constexpr int WAVE_ELEMS = KT + VT;
  static constexpr int LOOP_BYTES = NW * WAVE_ELEMS * (int)sizeof(S);
  static constexpr int OLD = 33;  // merge buffer row stride (floats)
  static constexpr int MERGE_BYTES = NW * DO * OLD * 4 + 2 * NW * 32 * 4;
  static constexpr int LDS_BYTES = LOOP_BYTES > MERGE_BYTES ? LOOP_BYTES : MERGE_BYTES;
  static constexpr int NSTEP = D / EL::KSTEP;
  static constexpr int NPV = CH / (2 * EL::E);
  static constexpr int NDB = DO / 32;
};

// Partial slots: num_splits per sequence, plus one per sequence for the
// balanced partition (its per-sequence shares are rounded up to at least one
// workgroup each).
size_t decode_workspace_bytes(int batch, int heads_q, int seqlen_q, int head_dim, int num_splits) {
  const size_t rows = (size_t)(num_splits + 1) * batch * heads_q * seqlen_q;
  size_t bytes = rows * (size_t)head_dim * 4 + rows * 4;
  return (bytes + 255) / 256 * 256;
}

// KV8: the cache holds fp8 (OCP e4m3) K and V, converted as the tiles load.
template <typename Tag, int D, bool PAGED, bool KV8 = false>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  using C = DecCfg<Tag, D>;
  using EL = Elem<Tag>;
  using S = typename EL::S;
  using KE = typename std::conditional<KV8, uint8_t, S>::type;  // cache element
  using Op = typename EL::Op;
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int h = lane >> 5, l32 = lane & 31;
  const int split = blockIdx.x;
  const int group = a.heads_q / a.heads_kv;
  const int rows = group * a.seqlen_q;
  const int nrb = (rows + 31) / 32;
  const int y = blockIdx.y;
  const int rb = y % nrb;
  const int bhk = y / nrb;
  const int b = bhk / a.heads_kv, hk = bhk - b * a.heads_kv;
  const int dc = blockIdx.z;

  int len = a.max_len;
  if (a.lens) len = min(max(a.lens[b * a.lens_stride] + a.lens_add, 0), a.max_len);
  const int nch = (len + C::CH - 1) / C::CH;
  const int per = nch / a.num_splits, extra = nch % a.num_splits;
  const int c0 = split * per + min(split, extra);
  const int cnt = per + (split < extra ? 1 : 0);

  // This lane's packed query row.
  const int r = rb * 32 + l32;
  const bool rvalid = r < rows;
  const int g = rvalid ? r / a.seqlen_q : 0;
  const int mq = rvalid ? r - g * a.seqlen_q : 0;
  const int hq = hk * group + g;
  const S* qrow = reinterpret_cast<const S*>(a.q) + b * a.q_stride[0] + hq * a.q_stride[1] +
                  mq * a.q_stride[2] + EL::E * h;
  // Last key this lane's query row sees (bottom-right causal), or all.
  const int klim = a.causal ? len - a.seqlen_q + mq : INT_MAX;
  Op qop[C::QREG ? C::NSTEP : 1];
  if constexpr (C::QREG) {
#pragma unroll
    for (int s = 0; s < C::NSTEP; ++s) qop[s] = rvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
    wait_vm_all();
  }

  const KE* kbase = reinterpret_cast<const KE*>(a.k);
  const KE* vbase = reinterpret_cast<const KE*>(a.v);
  if constexpr (!PAGED) {
    kbase += b * a.k_stride[0] + hk * a.k_stride[1];
    vbase += b * a.v_stride[0] + hk * a.v_stride[1];
  } else {
    kbase += hk * a.k_stride[2];
    vbase += hk * a.v_stride[2];
  }
  // Offset (elements) of key n's row, or -1 when the key is absent.
  auto key_off = [&](int n, const int64_t* st) -> int64_t {
    if (n >= len) return -1;
    if constexpr (!PAGED) {
      return (int64_t)n * st[2];
    } else {
      const int blk = n >> a.block_shift, pos = n & ((1 << a.block_shift) - 1);
      const int phys = a.block_table[b * a.bt_stride[0] + blk * a.bt_stride[1]];
      if (phys < 0 || phys >= a.num_blocks) return -1;
      return (int64_t)phys * st[0] + (int64_t)pos * st[1];
    }
  };

  S* ks = reinterpret_cast<S*>(smem_raw) + wave * C::WAVE_ELEMS;
  S* vs = ks + C::KT;
  RowTile<Tag, C::CH, D, 64, KV8> kt;
  TransTile<Tag, C::CH, C::DO, 64, KV8> vt;
  uint32_t valid_next = 0, valid_cur = 0;
  auto load_chunk = [&](int c) {
    const int n0 = c * C::CH;
    kt.load([&](int rr) -> const KE* {
      const int64_t o = key_off(n0 + rr, a.k_stride); return o < 0 ? nullptr : kbase + o; }, kbase, lane);
    vt.load([&](int rr) -> const KE* {
      const int64_t o = key_off(n0 + rr, a.v_stride); return o < 0 ? nullptr : vbase + o + dc * C::DO; }, vbase + dc * C::DO, lane);
    valid_next = (uint32_t)__ballot(l32 == lane && key_off(n0 + l32, a.k_stride) >= 0);
  };

  float m_i = kNegInf, l_i = 0.f;
  f32x16 acc[C::NDB];
#pragma unroll
  for (int i = 0; i < C::NDB; ++i) acc[i] = zero16();

  const int rounds = (cnt + C::NW - 1) / C::NW;
  int my = wave;  // chunk index (relative to c0) of this wave in the current round
  if (rounds > 0 && my < cnt) load_chunk(c0 + my);
  for (int it = 0; it < rounds; ++it) {
    const bool have = my < cnt;
    if (have) {
      kt.store(ks, C::KLD, lane);
      vt.store(vs, C::VLD, lane);
      valid_cur = valid_next;
    }
    __syncthreads();
    const int nxt = my + C::NW;
    if (it + 1 < rounds && nxt < cnt) load_chunk(c0 + nxt);
    if (have) {
      f32x16 sacc = zero16();
      const S* krow = ks + l32 * C::KLD + EL::E * h;
#pragma unroll
      for (int s = 0; s < C::NSTEP; ++s) {
        Op bq;
        if constexpr (C::QREG) bq = qop[s];
        else bq = rvalid ? load_op<Tag>(qrow + EL::KSTEP * s) : zero_op<Tag>();
        sacc = EL::mma(load_op<Tag>(krow + EL::KSTEP * s), bq, sacc);
      }
      float tmax = kNegInf;
      const int n0c = (c0 + my) * C::CH;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kr = acc_row(i, h);
        const float x = (((valid_cur >> kr) & 1u) && n0c + kr <= klim) ? sacc[i] * a.scale_log2 : kNegInf;
        sacc[i] = x;
        tmax = fmaxf(tmax, x);
      }
      tmax = half_max(tmax);
      const float m_new = fmaxf(m_i, tmax);
      const float m_use = (m_new == kNegInf) ? 0.f : m_new;
      const float alpha = exp2f(m_i - m_use);
      float rsum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = exp2f(sacc[i] - m_use);
        sacc[i] = pv;
        rsum += pv;
      }
      rsum = half_sum(rsum);
      l_i = l_i * alpha + rsum;
      m_i = m_new;
      constexpr int J = 16 / EL::E;
      Op pb[C::NPV];
#pragma unroll
      for (int j = 0; j < C::NPV; ++j) pb[j] = pack_op<Tag>(sacc, j % J);
#pragma unroll
      for (int db = 0; db < C::NDB; ++db) {
        acc[db] *= alpha;
        const S* vrow = vs + (db * 32 + l32) * C::VLD;
#pragma unroll
        for (int j = 0; j < C::NPV; ++j) acc[db] = EL::mma(lds_op_rowmap<Tag>(vrow, j, h), pb[j], acc[db]);
      }
    }
    __syncthreads();
    my = nxt;
  }

  // Merge the 4 wave states of each row through LDS.
  float* ow = reinterpret_cast<float*>(smem_raw);
  float* mw = ow + C::NW * C::DO * C::OLD;
  float* lw = mw + C::NW * 32;
#pragma unroll
  for (int db = 0; db < C::NDB; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) ow[(wave * C::DO + db * 32 + acc_row(i, h)) * C::OLD + l32] = acc[db][i];
  if (h == 0) {
    mw[wave * 32 + l32] = m_i;
    lw[wave * 32 + l32] = l_i;
  }
  __syncthreads();

  for (int idx = tid; idx < 32 * C::DO; idx += C::NT) {
    const int rr = idx / C::DO, d = idx - (idx / C::DO) * C::DO;
    const int row = rb * 32 + rr;
    if (row >= rows) continue;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < C::NW; ++w) M = fmaxf(M, mw[w * 32 + rr]);
    const float Mu = (M == kNegInf) ? 0.f : M;
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < C::NW; ++w) {
      const float sc = exp2f(mw[w * 32 + rr] - Mu);
      L += lw[w * 32 + rr] * sc;
      o += ow[(w * C::DO + d) * C::OLD + rr] * sc;
    }
    const float Ls = (L == 0.f) ? 1.f : L;
    o = o / Ls * a.out_scale;  // out_scale: v_scale of an fp8 cache, else 1
    const int gg = row / a.seqlen_q, mm = row - gg * a.seqlen_q;
    const int hh = hk * group + gg;
    const int dd = dc * C::DO + d;
    if (a.num_splits == 1) {
      S* op = reinterpret_cast<S*>(a.out) + b * a.out_stride[0] + hh * a.out_stride[1] + mm * a.out_stride[2];
      op[dd] = EL::from_f(o);
    } else {
      const int64_t prow = (((int64_t)split * a.batch + b) * a.heads_q + hh) * a.seqlen_q + mm;
      a.ws_o[prow * a.head_dim + dd] = o;
      if (dc == 0 && d == 0) a.ws_lse[prow] = (M == kNegInf || L == 0.f) ? kNegInf : (M + __log2f(L)) * kLn2;
    }
  }
}

// out[row] = sum_s w_s O_s / sum_s w_s,  w_s = exp(lse_s - max lse) (0 for -inf).
template <typename Tag>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeArgs a) {
  using EL = Elem<Tag>;
  using S = typename EL::S;
  const int rows = a.batch * a.heads_q * a.seqlen_q;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t plane = (int64_t)rows;
  float M = kNegInf;
  for (int s = 0; s < a.num_splits; ++s) M = fmaxf(M, a.ws_lse[s * plane + row]);
  const float Mu = (M == kNegInf) ? 0.f : M;
  const int mm = row % a.seqlen_q;
  const int hh = (row / a.seqlen_q) % a.heads_q;
  const int bb = row / (a.seqlen_q * a.heads_q);
  S* op = reinterpret_cast<S*>(a.out) + bb * a.out_stride[0] + hh * a.out_stride[1] + mm * a.out_stride[2];
  for (int d = lane; d < a.head_dim; d += 64) {
    float num = 0.f, den = 0.f;
    for (int s = 0; s < a.num_splits; ++s) {
      const float l = a.ws_lse[s * plane + row];
      const float w = (l == kNegInf) ? 0.f : __expf(l - Mu);
      den += w;
      num += w * a.ws_o[(s * plane + row) * a.head_dim + d];
    }
    op[d] = EL::from_f(num / (den == 0.f ? 1.f : den));
  }
}

// When set, the launch that ends a decode call completes this event (the
// kernel's own completion signal, no extra queue packet) and clears it; a
// call whose last launch does not take it leaves it set for the caller to
// record.  Used by fa_decode_splitk_noalloc to order its calls.
static thread_local hipEvent_t t_stop_event = nullptr;

template <typename Tag, int D, bool PAGED>
static hipError_t run_decode(DecodeArgs a, hipStream_t stream) {
  // Paged caches with blocks under 4 keys take the generic kernel (a chunk
  // would need more page ids than the streaming kernel keeps in scalars).
  if constexpr (D <= 128) {
    if (!PAGED || a.block_shift >= 2) {
      const int group = a.heads_q / a.heads_kv;
      const int nrb = (group * a.seqlen_q + 15) / 16;
      // Balanced partition over all sequences when the merge is fused and the
      // sequence lengths fit one wave's prefix scan.
      // The in-launch merge addresses the workspace with 32-bit offsets.
      if (decode_workspace_bytes(a.batch, a.heads_q, a.seqlen_q, D, a.num_splits) >= ((size_t)1 << 31))
        a.tickets = nullptr;
      a.balanced = (a.tickets != nullptr && a.batch <= 64) ? 1 : 0;
      dim3 grid = a.balanced ? dim3(a.heads_kv * nrb * (a.num_splits + 1) * a.batch, 1)
                             : dim3(a.heads_kv * nrb * a.num_splits, a.batch);
      constexpr int PG1 = PAGED ? 1 : 0, PG2 = PAGED ? 2 : 0;
      const bool small = PAGED && a.block_shift < 4;
      auto launch2 = [&](auto kv8_t, auto pg_t) -> hipError_t {
        constexpr bool K8 = decltype(kv8_t)::value;
        constexpr int PG = decltype(pg_t)::value;
        using C = Dec2Cfg<D, K8, PG == 2>;
        auto kern = decode2_kernel<Tag, D, PG, K8>;
        hipError_t err = allow_lds((const void*)kern, C::LDS_BYTES);
        if (err != hipSuccess) return err;
        // With the merge in this launch (tickets), it is the call's last.
        if (t_stop_event && a.tickets) {
          hipExtLaunchKernelGGL(kern, grid, dim3(C::NT), C::LDS_BYTES, stream, nullptr, t_stop_event, 0u, a);
          t_stop_event = nullptr;
        } else {
          hipLaunchKernelGGL(kern, grid, dim3(C::NT), C::LDS_BYTES, stream, a);
        }
        return hipGetLastError();
      };
      using P1 = std::integral_constant<int, PG1>;
      using P2 = std::integral_constant<int, PG2>;
      hipError_t e = a.kv8 ? (small ? launch2(std::true_type{}, P2{}) : launch2(std::true_type{}, P1{}))
                           : (small ? launch2(std::false_type{}, P2{}) : launch2(std::false_type{}, P1{}));
      if (e != hipSuccess || a.num_splits == 1 || a.tickets) return e;
      const int rows = a.batch * a.heads_q * a.seqlen_q;
      hipLaunchKernelGGL((decode_combine2_kernel<Tag, D>), dim3((rows + 3) / 4), dim3(256), 0, stream, a);
      return hipGetLastError();
    }
  }
  using C = DecCfg<Tag, D>;
  auto kern = a.kv8 ? decode_kernel<Tag, D, PAGED, true> : decode_kernel<Tag, D, PAGED>;
  hipError_t e = allow_lds((const void*)kern, C::LDS_BYTES);
  if (e != hipSuccess) return e;
  const int group = a.heads_q / a.heads_kv;
  const int nrb = (group * a.seqlen_q + 31) / 32;
  dim3 grid(a.num_splits, a.batch * a.heads_kv * nrb, D / C::DO);
  hipLaunchKernelGGL(kern, grid, dim3(C::NT), C::LDS_BYTES, stream, a);
  e = hipGetLastError();
  if (e != hipSuccess || a.num_splits == 1) return e;
  const int rows = a.batch * a.heads_q * a.seqlen_q;
  hipLaunchKernelGGL((decode_combine_kernel<Tag>), dim3((rows + 3) / 4), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <typename Tag, bool PAGED>
static hipError_t decode_by_dim(const DecodeArgs& a, hipStream_t s) {
  switch (a.head_dim) {
    case 32: return run_decode<Tag, 32, PAGED>(a, s);
    case 64: return run_decode<Tag, 64, PAGED>(a, s);
    case 128: return run_decode<Tag, 128, PAGED>(a, s);
    case 256: return run_decode<Tag, 256, PAGED>(a, s);
    case 512: return run_decode<Tag, 512, PAGED>(a, s);
  }
  return hipErrorInvalidValue;
}

template <bool PAGED>
static hipError_t decode_dispatch(int dtype, const DecodeArgs& a, hipStream_t s) {
  if (dtype == FA_DTYPE_F16) return decode_by_dim<f16_t, PAGED>(a, s);
  if (dtype == FA_DTYPE_BF16) return decode_by_dim<bf16_t, PAGED>(a, s);
  return hipErrorInvalidValue;
}

static void split_workspace(DecodeArgs& a, void* ws) {
  const size_t rows = (size_t)(a.num_splits + 1) * a.batch * a.heads_q * a.seqlen_q;
  a.ws_o = reinterpret_cast<float*>(ws);
  a.ws_lse = a.ws_o + rows * a.head_dim;
}

hipError_t launch_decode(const fa_decode_params& p, hipStream_t s) {
  DecodeArgs a{};
  a.q = p.q;
  for (int i = 0; i < 4; ++i) { a.q_stride[i] = p.q_stride[i]; a.out_stride[i] = p.out_stride[i]; }
  a.out = p.out;
  a.k = p.k;
  a.v = p.v;
  for (int i = 0; i < 3; ++i) { a.k_stride[i] = p.k_stride[i]; a.v_stride[i] = p.v_stride[i]; }
  a.lens = p.cache_seqlens;
  a.lens_stride = p.cache_seqlens_stride;
  a.lens_add = p.cache_seqlens_add;
  a.max_len = p.seqlen_k;
  a.batch = p.batch;
  a.heads_q = p.heads_q;
  a.heads_kv = p.heads_kv;
  a.seqlen_q = p.seqlen_q;
  a.head_dim = p.head_dim;
  a.kv8 = p.kv_fp8 ? 1 : 0;
  // An fp8 cache holds K / k_scale and V / v_scale: k_scale joins the logit
  // scale, v_scale multiplies the output.
  a.scale_log2 = p.softmax_scale * (a.kv8 ? p.k_scale : 1.f) * kLog2e;
  a.out_scale = a.kv8 ? p.v_scale : 1.f;
  a.num_splits = p.num_splits;
  a.causal = p.causal ? 1 : 0;
  split_workspace(a, p.workspace);
  a.tickets = p.tickets;
  return decode_dispatch<false>(p.dtype, a, s);
}

// ---------------------------------------------------------------------------
// Static scratch of fa_decode_splitk_noalloc: the arrival counters first
// (zero at load, left zero by every call), then the split workspace.  Host
// code never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): each device's address is looked up once
// with hipGetSymbolAddress, with that device current, and kept per device.
// ---------------------------------------------------------------------------
constexpr size_t kNoallocTicketBytes = (size_t)FA_NOALLOC_TICKETS * 4;
static __device__ __align__(256) unsigned char scratch[kNoallocTicketBytes + FA_NOALLOC_WORKSPACE_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_ptr[kMaxDevices] = {};

hipError_t scratch_for_current_device(unsigned char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = static_cast<unsigned char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}
}  // namespace

// Calls on one device are ordered by the order they are made on the host:
// each call records `done` on its stream, and a call on another stream first
// waits for the previous call's `done`.  So two streams (or host threads)
// no longer race on the shared scratch; the mutex keeps the record and the
// launch of one call together.  Under graph capture there is no wait or
// record (a captured wait on an event from outside the capture is an error):
// replays of a captured call must not overlap other calls on that device.
namespace {
struct NoallocOrder {
  hipStream_t last = nullptr;
  hipEvent_t done = nullptr;  // created on the device's first call outside capture
};
std::mutex g_order_mu;
NoallocOrder g_order[kMaxDevices];
}  // namespace

hipError_t launch_decode_noalloc(const fa_decode_params& p, hipStream_t s) {
  unsigned char* base = nullptr;
  hipError_t e = scratch_for_current_device(&base);
  if (e != hipSuccess) return e;
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess) return e;
  const bool capturing = cs != hipStreamCaptureStatusNone;
  fa_decode_params q = p;
  q.tickets = reinterpret_cast<uint32_t*>(base);
  q.workspace = base + kNoallocTicketBytes;
  std::lock_guard<std::mutex> lock(g_order_mu);
  NoallocOrder& o = g_order[dev];
  if (!capturing && o.done && o.last != s) {
    e = hipStreamWaitEvent(s, o.done, 0);
    if (e != hipSuccess) return e;
  }
  if (capturing) return launch_decode(q, s);
  if (!o.done) {
    e = hipEventCreateWithFlags(&o.done, hipEventDisableTiming);
    if (e != hipSuccess) {
      o.done = nullptr;
      return e;
    }
  }
  // The single-launch path completes `done` with its kernel; the others
  // leave t_stop_event set and `done` is recorded after them.
  t_stop_event = o.done;
  e = launch_decode(q, s);
  const bool taken = t_stop_event == nullptr;
  t_stop_event = nullptr;
  if (e != hipSuccess) return e;
  if (!taken) {
    e = hipEventRecord(o.done, s);
    if (e != hipSuccess) return e;
  }
  o.last = s;
  return hipSuccess;
}

hipError_t launch_paged(const fa_paged_params& p, hipStream_t s) {
  DecodeArgs a{};
  a.q = p.q;
  for (int i = 0; i < 4; ++i) { a.q_stride[i] = p.q_stride[i]; a.out_stride[i] = p.out_stride[i]; }
  a.out = p.out;
  a.k = p.k_cache;
  a.v = p.v_cache;
  for (int i = 0; i < 3; ++i) { a.k_stride[i] = p.k_stride[i]; a.v_stride[i] = p.v_stride[i]; }
  a.block_table = p.block_table;
  a.bt_stride[0] = p.block_table_stride[0];
  a.bt_stride[1] = p.block_table_stride[1];
  a.num_blocks = p.num_blocks;
  int shift = 0;
  while ((1 << shift) < p.block_size) ++shift;
  a.block_shift = shift;
  a.lens = p.context_lens;
  a.lens_stride = p.context_lens_stride;
  a.max_len = p.max_blocks * p.block_size;
  a.batch = p.batch;
  a.heads_q = p.heads_q;
  a.heads_kv = p.heads_kv;
  a.seqlen_q = p.seqlen_q;
  a.head_dim = p.head_dim;
  a.scale_log2 = p.softmax_scale * kLog2e;
  a.num_splits = p.num_splits;
  a.causal = p.causal ? 1 : 0;
  a.kv8 = p.kv_fp8 ? 1 : 0;
  a.scale_log2 = p.softmax_scale * (a.kv8 ? p.k_scale : 1.f) * kLog2e;
  a.out_scale = a.kv8 ? p.v_scale : 1.f;
  split_workspace(a, p.workspace);
  a.tickets = p.tickets;
  return decode_dispatch<true>(p.dtype, a, s);
}


// ---------------------------------------------------------------------------
// KV-cache append (cache update of the kv-cache entry point): one 16-byte
// piece of a new K and V row per thread, written at row cache_seqlens[b] + s.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kv_append_kernel(fa_append_params p, int64_t pieces) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= pieces) return;
  const int cpr = p.head_dim / 8;  // 16-byte pieces per row
  const int c = (int)(i % cpr);
  int64_t row = i / cpr;
  const int s = (int)(row % p.seqlen_new);
  row /= p.seqlen_new;
  const int h = (int)(row % p.heads_kv);
  const int b = (int)(row / p.heads_kv);
  const int pos = p.cache_seqlens[b * p.cache_seqlens_stride] + s;
  if (pos < 0 || pos >= p.seqlen_cache) return;
  const uint16_t* kn = reinterpret_cast<const uint16_t*>(p.k_new) + b * p.k_new_stride[0] + h * p.k_new_stride[1] +
                       (int64_t)s * p.k_new_stride[2] + 8 * c;
  const uint16_t* vn = reinterpret_cast<const uint16_t*>(p.v_new) + b * p.v_new_stride[0] + h * p.v_new_stride[1] +
                       (int64_t)s * p.v_new_stride[2] + 8 * c;
  uint16_t* kc = reinterpret_cast<uint16_t*>(p.k_cache) + b * p.k_cache_stride[0] + h * p.k_cache_stride[1] +
                 (int64_t)pos * p.k_cache_stride[2] + 8 * c;
  uint16_t* vc = reinterpret_cast<uint16_t*>(p.v_cache) + b * p.v_cache_stride[0] + h * p.v_cache_stride[1] +
                 (int64_t)pos * p.v_cache_stride[2] + 8 * c;
  *reinterpret_cast<uint4*>(kc) = *reinterpret_cast<const uint4*>(kn);
  *reinterpret_cast<uint4*>(vc) = *reinterpret_cast<const uint4*>(vn);
}

hipError_t launch_append(const fa_append_params& p, hipStream_t stream) {
  const int64_t pieces = (int64_t)p.batch * p.heads_kv * p.seqlen_new * (p.head_dim / 8);
  if (pieces == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, p, pieces);
  return hipGetLastError();
}

}  // namespace fa
