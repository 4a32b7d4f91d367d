// Instantiates the fwd kernels for f16.
#include "fa_fwd_impl.hpp"

namespace fa {
template hipError_t fwd_by_mods<f16_t>(const fa_fwd_params& p, hipStream_t s);
}  // namespace fa

