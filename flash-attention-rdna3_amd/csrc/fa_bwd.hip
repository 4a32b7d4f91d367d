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

hipError_t launch_bwd(const fa_bwd_params& p, int ph, hipStream_t s) {
  switch (p.fwd.dtype) {
    case FA_DTYPE_F16: return bwd_by_mods<f16_t>(p, ph, s);
    case FA_DTYPE_BF16: return bwd_by_mods<bf16_t>(p, ph, s);
    case FA_DTYPE_F32: return bwd_by_mods<f32_t>(p, ph, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
