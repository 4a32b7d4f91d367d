// Dtype dispatch of the fwd kernels (instantiated in fa_fwd_{f16,bf16,f32}.hip).
#include "fa_internal.hpp"
#include "fa_common.hpp"

namespace fa {

template <typename Tag>
hipError_t fwd_by_mods(const fa_fwd_params& p, hipStream_t s);

hipError_t launch_fwd(const fa_fwd_params& p, hipStream_t s) {
  switch (p.dtype) {
    case FA_DTYPE_F16: return fwd_by_mods<f16_t>(p, s);
    case FA_DTYPE_BF16: return fwd_by_mods<bf16_t>(p, s);
    case FA_DTYPE_F32: return fwd_by_mods<f32_t>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace fa
