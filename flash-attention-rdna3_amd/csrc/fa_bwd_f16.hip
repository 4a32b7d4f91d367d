// Instantiates the bwd kernels for f16.
#include "fa_bwd_impl.hpp"

namespace fa {
template hipError_t bwd_by_mods<f16_t>(const fa_bwd_params& p, int ph, hipStream_t s);
}  // namespace fa

