// Dtype dispatch of the bwd kernels (instantiated in fa_bwd_{f16,bf16,f32}.hip).
#include "fa_internal.hpp"
#include "fa_common.hpp"

namespace fa {

template <typename Tag>
hipError_t bwd_by_mods(const fa_bwd_params& p, int ph, hipStream_t s);

hipError_t launch_bwd(const fa_bwd_params& p, int ph, hipStream_t s) {
  switch (p.fwd.dtype) {
    case FA_DTYPE_F16: return bwd_by_mods<f16_t>(p, ph, s);
    case FA_DTYPE_BF16: return bwd_by_mods<bf16_t>(p, ph, s);
    case FA_DTYPE_F32: return bwd_by_mods<f32_t>(p, ph, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
