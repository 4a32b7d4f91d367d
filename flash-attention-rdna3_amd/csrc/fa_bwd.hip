// Dtype dispatch of the bwd kernels (instantiated in fa_bwd_{f16,bf16,f32}.hip).
#include "fa_internal.hpp"
#include "fa_common.hpp"

namespace fa {

template <typename Tag>
hipError_t bwd_by_mods(const fa_bwd_params& p, int ph, hipStream_t s);

size_t bwd_ds_bytes(const fa_bwd_params& p) {
  const fa_fwd_params& f = p.fwd;
  if (f.dtype == FA_DTYPE_F32 || f.head_dim > 128 || f.head_dim < 64) return 0;
  if (f.batch <= 0 || f.heads_q <= 0 || f.seqlen_q <= 0 || f.seqlen_k <= 0) return 0;
  int64_t elems;
  if (f.cu_seqlens_q) {
    if (f.batch > kDsMaxVarlenBatch || f.total_q < 0) return 0;
    // sum_b kblocks(Sk_b) * qblocks(Sq_b)
    //   <= kblocks(max_seqlen_k) * (total_q / 128 + batch)
    const int64_t kb = ((int64_t)f.seqlen_k + kDsTileKeys - 1) / kDsTileKeys;
    elems = (int64_t)f.heads_q * kb * ((int64_t)f.total_q / kDsTileQueries + f.batch) * kDsTileElems;
  } else {
    elems = (int64_t)f.batch * f.heads_q * ds_region_elems(f.seqlen_q, f.seqlen_k);
  }
  return (size_t)elems * 2 + 1024;
}

size_t bwd_ds_chunk_bytes(const fa_bwd_params& p, int kv_heads) {
  const fa_fwd_params& f = p.fwd;
  if (f.bias || f.alibi_slopes || f.dropout_p > 0.f) return 0;
  if (f.heads_kv <= 0 || kv_heads <= 0 || kv_heads > f.heads_kv) return 0;
  const size_t full = bwd_ds_bytes(p);
  if (full == 0) return 0;
  // The bound is linear in the number of heads (plus the 1 KiB slack).
  return (full - 1024) / f.heads_kv * kv_heads + 1024;
}

// Two chunks of near-equal size, each with at least 1 GiB of dS: measured on
// MI355X, two such chunks run as fast as the whole scratch (B=1, H=32,
// S=16384 causal: 9.71 against 9.75 ms), while three or more, or smaller
// chunks, lose to recomputing dQ (the same step with three chunks 10.09 ms,
// recompute 10.08 ms; config 2 in two chunks of 134 MB 244 against 210 us).
int bwd_ds_chunk_heads(const fa_bwd_params& p, int64_t ws) {
  const fa_fwd_params& f = p.fwd;
  if (f.heads_kv < 2) return 0;
  const size_t full = bwd_ds_bytes(p);
  if (full == 0 || ws >= (int64_t)full) return 0;
  const int per = (f.heads_kv + 1) / 2;
  const size_t chunk = bwd_ds_chunk_bytes(p, per);
  if (chunk == 0 || (int64_t)chunk - 1024 < kDsMinChunkBytes || ws < (int64_t)chunk) return 0;
  return per;
}

hipError_t launch_bwd(const fa_bwd_params& p, int ph, hipStream_t s) {
  switch (p.fwd.dtype) {
    case FA_DTYPE_F16: return bwd_by_mods<f16_t>(p, ph, s);
    case FA_DTYPE_BF16: return bwd_by_mods<bf16_t>(p, ph, s);
    case FA_DTYPE_F32: return bwd_by_mods<f32_t>(p, ph, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
