// fa_hbm_read.hip - streaming-read probe: the HBM read rate a plain
// hand-written kernel reaches on this GPU for a given byte count.  It is the
// ceiling the HBM-bound decode kernels are compared against (their work is a
// one-pass read of the visible K/V bytes), not part of the attention path.
//
// Every variant reads each 16-byte piece of [src, src + bytes) exactly once
// with dwordx4 loads, keeps U loads per lane in flight before it uses any of
// them, folds them into one XOR per lane and stores that only when it equals
// a value the data never produce, so the loads cannot be elided and almost
// nothing is written.  Three grid shapes:
//   * one pass: workgroup i reads the contiguous span [i * NT * U, (i + 1) * NT * U)
//     pieces, and the hardware hands spans to CUs as workgroups finish;
//   * grid-stride: a fixed number of workgroups per CU walk the spans in a
//     grid-stride loop (all of them advance through the buffer together);
//   * contiguous slices: a fixed number of workgroups per CU each walk their
//     own contiguous slice (one long stream per workgroup, as the split-K
//     decode reads its key ranges).
// Plain or nontemporal loads.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "fa_internal.hpp"

namespace fa {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int NT, int U, bool NTL, int PERSIST>
__global__ __launch_bounds__(NT) void hbm_read_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                      uint32_t* __restrict__ sink) {
  constexpr int64_t SPAN = (int64_t)NT * U;
  const int64_t nspan = (n16 + SPAN - 1) / SPAN;
  uint32_t acc = 0;
  // PERSIST 2: workgroup i walks its own contiguous slice of the spans.
  const int64_t per = (nspan + gridDim.x - 1) / gridDim.x;
  const int64_t sp0 = PERSIST == 2 ? blockIdx.x * per : blockIdx.x;
  const int64_t sp1 = PERSIST == 2 ? (sp0 + per < nspan ? sp0 + per : nspan) : nspan;
  for (int64_t sp = sp0; sp < sp1; sp += PERSIST == 1 ? gridDim.x : PERSIST == 2 ? 1 : nspan) {
    const int64_t base = sp * SPAN + threadIdx.x;
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * NT;
      const int64_t j = i < n16 ? i : n16 - 1;  // tail lanes re-read the last piece
      if constexpr (NTL) v[u] = __builtin_nontemporal_load(src + j);
      else v[u] = src[j];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == 0x9E3779B9u) sink[threadIdx.x] = acc;
}

struct ReadVariant {
  const void* fn;
  int nt, u;
  int persist;  // 0 one pass, 1 grid-stride (8 per CU), 2 contiguous slices (persist_wg per CU)
  int per_cu;
  const char* name;
};

#define FA_RV(NT, U, NTL, P, C) \
  { (const void*)hbm_read_kernel<NT, U, NTL, P>, NT, U, P, C, #NT " threads, " #U " x 16 B per lane in flight, " \
    #NTL " nontemporal, grid mode " #P " (0 one pass, 1 grid-stride, 2 contiguous slices), " #C " per CU" }
static const ReadVariant kReadVariants[] = {
    FA_RV(256, 8, false, 0, 0),  FA_RV(256, 16, false, 0, 0), FA_RV(512, 8, false, 0, 0),
    FA_RV(512, 16, false, 0, 0), FA_RV(1024, 8, false, 0, 0), FA_RV(256, 8, true, 0, 0),
    FA_RV(256, 16, true, 0, 0),  FA_RV(512, 8, true, 0, 0),   FA_RV(256, 8, false, 1, 8),
    FA_RV(256, 16, false, 1, 8), FA_RV(512, 8, false, 1, 8),  FA_RV(256, 16, true, 1, 8),
    FA_RV(256, 8, true, 2, 1),   FA_RV(256, 8, true, 2, 2),   FA_RV(256, 8, true, 2, 8),
    FA_RV(256, 16, true, 2, 1),
};
#undef FA_RV
constexpr int kNumReadVariants = sizeof(kReadVariants) / sizeof(kReadVariants[0]);

}  // namespace fa

extern "C" {

int fa_hbm_read_probe_count(void) { return fa::kNumReadVariants; }

const char* fa_hbm_read_probe_name(int variant) {
  return (variant >= 0 && variant < fa::kNumReadVariants) ? fa::kReadVariants[variant].name : "";
}

int fa_hbm_read_probe(const void* src, size_t bytes, void* sink, int variant, void* stream) {
  if (!src || !sink || bytes < 16 || bytes % 16 != 0 || (uintptr_t)src % 16 != 0) return 1;
  if (variant < 0 || variant >= fa::kNumReadVariants) return 1;
  const fa::ReadVariant& rv = fa::kReadVariants[variant];
  const int64_t n16 = (int64_t)(bytes / 16);
  const int64_t span = (int64_t)rv.nt * rv.u;
  const int64_t nspan = (n16 + span - 1) / span;
  const int64_t grid = rv.persist ? std::min<int64_t>(nspan, rv.per_cu * (int64_t)fa::device_cu_count()) : nspan;
  if (grid > 0x7FFFFFFF) return 1;
  const fa::u32x4_t* s = reinterpret_cast<const fa::u32x4_t*>(src);
  uint32_t* k = reinterpret_cast<uint32_t*>(sink);
  void* args[] = {(void*)&s, (void*)&n16, (void*)&k};
  const hipError_t e = hipLaunchKernel(rv.fn, dim3((unsigned)grid), dim3(rv.nt), args, 0, (hipStream_t)stream);
  return e == hipSuccess ? 0 : 3;
}

}  // extern "C"
