#include "fa_internal.hpp"
namespace fa {
hipError_t launch_decode(const fa_decode_params&, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_paged(const fa_paged_params&, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_tiny(const fa_tiny_params&, hipStream_t) { return hipErrorInvalidValue; }
size_t decode_workspace_bytes(int, int, int, int, int) { return 0; }
}
