// fa_internal.hpp - host-side launchers behind the C ABI (fa_api.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/fa_mi355x.h"

namespace fa {

// Buffer-addressed tiles use 32-bit byte offsets inside a window of `rows`
// rows: the fast kernels need rows * stride * 2 < 2^31.
inline bool buf_rows_ok(int64_t stride_elems, int rows) {
  return stride_elems >= 0 && stride_elems * 2 * (int64_t)rows < (int64_t(1) << 31);
}

// Each launcher validates nothing beyond what it needs to pick a kernel
// instantiation; fa_api.cpp has already checked the arguments.  They return
// hipSuccess, hipErrorInvalidValue for an unsupported configuration, or the
// launch error.
hipError_t launch_fwd(const fa_fwd_params& p, hipStream_t stream);
// phases: bit 0 delta, bit 1 dK/dV, bit 2 dQ.
hipError_t launch_bwd(const fa_bwd_params& p, int phases, hipStream_t stream);
hipError_t launch_decode(const fa_decode_params& p, hipStream_t stream);
// launch_decode with the library's static per-device scratch as workspace and
// tickets (sizes already checked against FA_NOALLOC_*).
hipError_t launch_decode_noalloc(const fa_decode_params& p, hipStream_t stream);
hipError_t launch_paged(const fa_paged_params& p, hipStream_t stream);
hipError_t launch_tiny(const fa_tiny_params& p, hipStream_t stream);
hipError_t launch_append(const fa_append_params& p, hipStream_t stream);

size_t decode_workspace_bytes(int batch, int heads_q, int seqlen_q, int head_dim, int num_splits);

// Score-gradient scratch of the 16-bit backward: per (sequence, query head)
// a region of tiles of 64 keys x 128 queries (16 KiB of 16-bit dS), tile
// (key block kb, query block qb) at kb * ds_qblocks(Sq) + qb; the regions of
// a varlen batch are packed in sequence order.  Inside a tile, queries come
// in 4 sub-tiles of 32 (4 KiB each, key-major rows of 32 queries): element
// (key n, query q) at (q / 32) * 2048 + n * 32 + q % 32.  A dK/dV step (32
// queries) then writes whole 64-byte rows, 2 KiB contiguous per wave, and a
// dQ step reads one tile's 16 contiguous KiB.  The scratch ends
// in 1 KiB of slack where lanes past the last key of a dK/dV wave write.
constexpr int kDsMaxVarlenBatch = 512;
constexpr int kDsTileKeys = 64, kDsTileQueries = 128, kDsTileElems = kDsTileKeys * kDsTileQueries;
constexpr int kDsSubQueries = 32, kDsSubElems = kDsTileKeys * kDsSubQueries;
__host__ __device__ inline int64_t ds_qblocks(int sq) { return ((int64_t)sq + kDsTileQueries - 1) / kDsTileQueries; }
__host__ __device__ inline int64_t ds_region_elems(int sq, int sk) {
  return ((int64_t)sk + kDsTileKeys - 1) / kDsTileKeys * ds_qblocks(sq) * kDsTileElems;
}
size_t bwd_ds_bytes(const fa_bwd_params& p);
// dS scratch for `kv_heads` KV heads (with their query heads) of p, or 0
// when the backward cannot run in KV-head chunks: the per-head modifiers
// (bias, ALiBi, dropout) are indexed by the head, so only problems without
// them are chunked.
size_t bwd_ds_chunk_bytes(const fa_bwd_params& p, int kv_heads);
// KV heads per chunk when a backward with `ws` bytes of dS scratch runs in
// chunks, or 0 when it does not (the whole dS fits, or the problem cannot
// be chunked, or chunking would not pay: it is used only for two chunks of
// at least 1 GiB of dS each).
int bwd_ds_chunk_heads(const fa_bwd_params& p, int64_t ws);
constexpr int64_t kDsMinChunkBytes = int64_t(1) << 30;

// Raise a kernel's dynamic LDS limit once per process (gfx950: 160 KiB/CU).
hipError_t allow_lds(const void* kernel, int bytes);

// Compute units of the current device (cached per device).
int device_cu_count();

}  // namespace fa
