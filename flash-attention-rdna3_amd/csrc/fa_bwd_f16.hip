// Instantiates the bwd kernels for f16.
#include "fa_bwd_impl.hpp"

namespace fa {
template hipError_t bwd_by_mods<f16_t>(const fa_bwd_params& p, int ph, hipStream_t s);
}  // namespace fa

#ifdef FA_TRACE_WG
// Copies (and optionally clears) this translation unit's workgroup trace.
extern "C" int fa_debug_trace_bwd_f16(void* dst, size_t bytes, int clear) {
  if (dst && hipMemcpyFromSymbol(dst, HIP_SYMBOL(fa::g_fa_trace), bytes, 0, hipMemcpyDeviceToHost) != hipSuccess) return 1;
  if (clear) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(fa::g_fa_trace)) != hipSuccess) return 2;
    if (hipMemset(p, 0, sizeof(fa::g_fa_trace)) != hipSuccess) return 3;
  }
  return 0;
}
#endif
