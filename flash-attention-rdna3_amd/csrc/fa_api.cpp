// fa_api.cpp - the extern "C" boundary declared in include/fa_mi355x.h.
//
// Checks what would let a kernel touch memory out of bounds, converts every
// failure into an fa_status plus a thread-local message, and never lets a C++
// exception or a HIP error escape as anything but a return code.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "fa_internal.hpp"

namespace {

thread_local std::string g_last_error = "no error";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FA_OK;
  if (e == hipErrorInvalidValue)
    return fail(FA_ERR_UNSUPPORTED, "%s: unsupported configuration", what);
  return fail(FA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A tensor whose rows are read with 16-byte vector loads: contiguous last
// dim, every row start 16-byte aligned.
bool rows_ok(const void* p, const int64_t* st, int nst, int esize) {
  if (!p || !aligned16(p)) return false;
  if (st[nst - 1] != 1) return false;
  for (int i = 0; i < nst - 1; ++i)
    if ((st[i] * esize) % 16 != 0) return false;
  return true;
}

int esize_of(int dtype) { return dtype == FA_DTYPE_F32 ? 4 : 2; }

bool dim_ok(int d) { return d == 32 || d == 64 || d == 128 || d == 256 || d == 512; }

int check_fwd(const fa_fwd_params& p, const char* who) {
  if (p.abi_version != FA_ABI_VERSION)
    return fail(FA_ERR_INVALID, "%s: abi_version %d != %d", who, p.abi_version, FA_ABI_VERSION);
  if (p.dtype < 0 || p.dtype > 2) return fail(FA_ERR_INVALID, "%s: bad dtype %d", who, p.dtype);
  if (!dim_ok(p.head_dim))
    return fail(FA_ERR_UNSUPPORTED, "%s: head_dim %d (kernels take 32/64/128/256/512)", who, p.head_dim);
  if (p.batch <= 0 || p.heads_q <= 0 || p.heads_kv <= 0 || p.heads_q % p.heads_kv != 0)
    return fail(FA_ERR_INVALID, "%s: bad batch/heads", who);
  if (p.seqlen_q <= 0 || p.seqlen_k <= 0) return fail(FA_ERR_INVALID, "%s: bad sequence lengths", who);
  const int es = esize_of(p.dtype);
  if (!rows_ok(p.q, p.q_stride, 4, es) || !rows_ok(p.k, p.k_stride, 4, es) ||
      !rows_ok(p.v, p.v_stride, 4, es) || !rows_ok(p.out, p.out_stride, 4, es))
    return fail(FA_ERR_INVALID, "%s: q/k/v/out need a unit last stride and 16-byte aligned rows", who);
  if (!p.lse) return fail(FA_ERR_INVALID, "%s: lse is NULL", who);
  if ((p.cu_seqlens_q == nullptr) != (p.cu_seqlens_k == nullptr))
    return fail(FA_ERR_INVALID, "%s: cu_seqlens_q and cu_seqlens_k must both be set", who);
  if (p.cu_seqlens_q && (p.total_q <= 0 || p.total_k <= 0))
    return fail(FA_ERR_INVALID, "%s: varlen totals must be positive", who);
  if (p.bias && p.bias_dtype != FA_DTYPE_F32 && p.bias_dtype != p.dtype)
    return fail(FA_ERR_INVALID, "%s: bias dtype must match q or be fp32", who);
  if (p.dropout_p < 0.f || p.dropout_p >= 1.f) return fail(FA_ERR_INVALID, "%s: dropout_p out of range", who);
  return FA_OK;
}

}  // namespace

namespace fa {

hipError_t allow_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::unordered_map<const void*, int> done;
  std::lock_guard<std::mutex> g(mu);
  auto it = done.find(kernel);
  if (it != done.end() && it->second >= bytes) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done[kernel] = bytes;
  return e;
}

int device_cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace fa

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_last_error_string(void) { return g_last_error.c_str(); }

size_t fa_params_size(int which) {
  switch (which) {
    case 0: return sizeof(fa_fwd_params);
    case 1: return sizeof(fa_bwd_params);
    case 2: return sizeof(fa_decode_params);
    case 3: return sizeof(fa_paged_params);
    case 4: return sizeof(fa_tiny_params);
    case 5: return sizeof(fa_append_params);
  }
  return 0;
}

size_t fa_decode_ticket_count(int batch, int heads_q, int seqlen_q) {
  if (batch <= 0 || heads_q <= 0 || seqlen_q <= 0) return 0;
  return (size_t)batch * heads_q * seqlen_q;
}

size_t fa_decode_workspace_bytes(int batch, int heads_q, int seqlen_q, int head_dim, int num_splits) {
  if (batch <= 0 || heads_q <= 0 || seqlen_q <= 0 || head_dim <= 0 || num_splits <= 0) return 0;
  return fa::decode_workspace_bytes(batch, heads_q, seqlen_q, head_dim, num_splits);
}

int fa_fwd(const fa_fwd_params* params, void* stream) {
  if (!params) return fail(FA_ERR_INVALID, "fa_fwd: params is NULL");
  int rc = check_fwd(*params, "fa_fwd");
  if (rc) return rc;
  return from_hip(fa::launch_fwd(*params, (hipStream_t)stream), "fa_fwd");
}

static int bwd_common(const fa_bwd_params* params, int phases, void* stream) {
  if (!params) return fail(FA_ERR_INVALID, "fa_bwd: params is NULL");
  int rc = check_fwd(params->fwd, "fa_bwd");
  if (rc) return rc;
  const fa_bwd_params& p = *params;
  const int es = esize_of(p.fwd.dtype);
  if (!rows_ok(p.dout, p.dout_stride, 4, es) || !rows_ok(p.dq, p.dq_stride, 4, es) ||
      !rows_ok(p.dk, p.dk_stride, 4, es) || !rows_ok(p.dv, p.dv_stride, 4, es))
    return fail(FA_ERR_INVALID, "fa_bwd: dout/dq/dk/dv need a unit last stride and 16-byte aligned rows");
  if (!p.delta) return fail(FA_ERR_INVALID, "fa_bwd: delta is NULL");
  return from_hip(fa::launch_bwd(p, phases, (hipStream_t)stream), "fa_bwd");
}

int fa_bwd(const fa_bwd_params* params, void* stream) { return bwd_common(params, 7, stream); }

size_t fa_bwd_workspace_bytes(const fa_bwd_params* params) {
  if (!params) return 0;
  return fa::bwd_ds_bytes(*params);
}

size_t fa_bwd_workspace_min_bytes(const fa_bwd_params* params) {
  if (!params) return 0;
  const size_t full = fa::bwd_ds_bytes(*params);
  const int per = (params->fwd.heads_kv + 1) / 2;
  const size_t half = params->fwd.heads_kv > 1 ? fa::bwd_ds_chunk_bytes(*params, per) : 0;
  return (half > 0 && fa::bwd_ds_chunk_heads(*params, (int64_t)half) == per) ? half : full;
}

// With dS scratch, phase 2 alone reads the dS that phase 1 stored there.
// Each phase-1 launch on a scratch records what it computed (the forward
// problem, dO, delta and the scratch size); phase 2 alone on that scratch
// must match the record, or it is refused instead of reading stale dS.
// (Memory reused by someone else between the two calls cannot be seen.)
namespace {
struct DsRecord {
  fa_fwd_params fwd;
  const void* dout;
  int64_t dout_stride[4];
  const float* delta;
  int64_t delta_stride[3];
  int64_t bytes;
};

std::mutex g_ds_mu;
std::unordered_map<const void*, DsRecord> g_ds_records;

DsRecord ds_record_of(const fa_bwd_params& p) {
  DsRecord r;
  std::memset(&r, 0, sizeof(r));
  r.fwd = p.fwd;
  r.dout = p.dout;
  std::memcpy(r.dout_stride, p.dout_stride, sizeof(r.dout_stride));
  r.delta = p.delta;
  std::memcpy(r.delta_stride, p.delta_stride, sizeof(r.delta_stride));
  r.bytes = p.ds_workspace_bytes;
  return r;
}

bool ds_scratch_used(const fa_bwd_params& p) {
  if (!p.ds_workspace) return false;
  const size_t need = fa::bwd_ds_bytes(p);
  return need > 0 && p.ds_workspace_bytes >= (int64_t)need;
}
}  // namespace

int fa_bwd_phase(const fa_bwd_params* params, int phase, void* stream) {
  if (phase < 0 || phase > 2) return fail(FA_ERR_INVALID, "fa_bwd_phase: phase %d not in 0..2", phase);
  if (params && phase == 2 && ds_scratch_used(*params)) {
    const DsRecord want = ds_record_of(*params);
    std::lock_guard<std::mutex> lock(g_ds_mu);
    const auto it = g_ds_records.find(params->ds_workspace);
    if (it == g_ds_records.end() || std::memcmp(&it->second, &want, sizeof(want)) != 0)
      return fail(FA_ERR_INVALID,
                  "fa_bwd_phase: phase 2 with ds_workspace reads the dS that phase 1 of the same problem "
                  "stores there; run phase 1 on this scratch first (or pass no ds_workspace to recompute dQ)");
  }
  const int rc = bwd_common(params, 1 << phase, stream);
  if (rc == FA_OK && phase == 1 && ds_scratch_used(*params)) {
    std::lock_guard<std::mutex> lock(g_ds_mu);
    g_ds_records[params->ds_workspace] = ds_record_of(*params);
  }
  return rc;
}

namespace {

// Checks of fa_decode_splitk and fa_decode_splitk_noalloc (the latter brings
// its own workspace and tickets, so it skips those two).
int check_decode(const fa_decode_params* params, const char* who, bool own_scratch) {
  if (!params) return fail(FA_ERR_INVALID, "%s: params is NULL", who);
  const fa_decode_params& p = *params;
  if (p.abi_version != FA_ABI_VERSION) return fail(FA_ERR_INVALID, "%s: abi_version mismatch", who);
  if (p.dtype != FA_DTYPE_F16 && p.dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_INVALID, "%s: dtype must be f16 or bf16", who);
  if (!dim_ok(p.head_dim)) return fail(FA_ERR_UNSUPPORTED, "%s: head_dim %d", who, p.head_dim);
  if (p.batch <= 0 || p.heads_q <= 0 || p.heads_kv <= 0 || p.heads_q % p.heads_kv || p.seqlen_q <= 0 ||
      p.seqlen_k <= 0)
    return fail(FA_ERR_INVALID, "%s: bad shape", who);
  if (p.num_splits < 1 || p.num_splits > 64) return fail(FA_ERR_INVALID, "%s: num_splits", who);
  if (p.kv_fp8 != 0 && p.kv_fp8 != 1) return fail(FA_ERR_INVALID, "%s: kv_fp8 must be 0 or 1", who);
  const int kes = p.kv_fp8 ? 1 : 2;
  if (!rows_ok(p.q, p.q_stride, 4, 2) || !rows_ok(p.k, p.k_stride, 4, kes) || !rows_ok(p.v, p.v_stride, 4, kes) ||
      !rows_ok(p.out, p.out_stride, 4, 2))
    return fail(FA_ERR_INVALID, "%s: q/k/v/out need a unit last stride and 16-byte aligned rows", who);
  if (!own_scratch) {
    if (!p.workspace || !aligned16(p.workspace)) return fail(FA_ERR_INVALID, "%s: workspace", who);
    if ((reinterpret_cast<uintptr_t>(p.tickets) & 3u) != 0) return fail(FA_ERR_INVALID, "%s: tickets", who);
  }
  if (p.causal != 0 && p.causal != 1) return fail(FA_ERR_INVALID, "%s: causal must be 0 or 1", who);
  return FA_OK;
}

}  // namespace

int fa_decode_splitk(const fa_decode_params* params, void* stream) {
  const int rc = check_decode(params, "fa_decode_splitk", false);
  if (rc != FA_OK) return rc;
  return from_hip(fa::launch_decode(*params, (hipStream_t)stream), "fa_decode_splitk");
}

int fa_decode_splitk_noalloc(const fa_decode_params* params, void* stream) {
  const int rc = check_decode(params, "fa_decode_splitk_noalloc", true);
  if (rc != FA_OK) return rc;
  const fa_decode_params& p = *params;
  const size_t ws = fa::decode_workspace_bytes(p.batch, p.heads_q, p.seqlen_q, p.head_dim, p.num_splits);
  const size_t nt = (size_t)p.batch * p.heads_q * p.seqlen_q;
  if (ws > FA_NOALLOC_WORKSPACE_BYTES || nt > FA_NOALLOC_TICKETS)
    return fail(FA_ERR_INVALID,
                "fa_decode_splitk_noalloc: needs %zu workspace bytes and %zu tickets; the static scratch holds "
                "%d and %d (use fa_decode_splitk with a caller workspace)",
                ws, nt, FA_NOALLOC_WORKSPACE_BYTES, FA_NOALLOC_TICKETS);
  return from_hip(fa::launch_decode_noalloc(p, (hipStream_t)stream), "fa_decode_splitk_noalloc");
}

int fa_decode_paged(const fa_paged_params* params, void* stream) {
  if (!params) return fail(FA_ERR_INVALID, "fa_decode_paged: params is NULL");
  const fa_paged_params& p = *params;
  if (p.abi_version != FA_ABI_VERSION) return fail(FA_ERR_INVALID, "fa_decode_paged: abi_version mismatch");
  if (p.dtype != FA_DTYPE_F16 && p.dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_INVALID, "fa_decode_paged: dtype must be f16 or bf16");
  if (!dim_ok(p.head_dim)) return fail(FA_ERR_UNSUPPORTED, "fa_decode_paged: head_dim %d", p.head_dim);
  if (p.batch <= 0 || p.heads_q <= 0 || p.heads_kv <= 0 || p.heads_q % p.heads_kv || p.num_blocks <= 0 ||
      p.max_blocks <= 0 || p.block_size <= 0 || p.block_size > 256 || (p.block_size & (p.block_size - 1)))
    return fail(FA_ERR_INVALID, "fa_decode_paged: bad shape");
  if (p.num_splits < 1 || p.num_splits > 64) return fail(FA_ERR_INVALID, "fa_decode_paged: num_splits");
  if (p.seqlen_q < 1) return fail(FA_ERR_INVALID, "fa_decode_paged: seqlen_q must be >= 1");
  if (p.causal != 0 && p.causal != 1) return fail(FA_ERR_INVALID, "fa_decode_paged: causal must be 0 or 1");
  if (p.kv_fp8 != 0 && p.kv_fp8 != 1) return fail(FA_ERR_INVALID, "fa_decode_paged: kv_fp8 must be 0 or 1");
  const int kes = p.kv_fp8 ? 1 : 2;
  if (!rows_ok(p.q, p.q_stride, 4, 2) || !rows_ok(p.k_cache, p.k_stride, 4, kes) ||
      !rows_ok(p.v_cache, p.v_stride, 4, kes) || !rows_ok(p.out, p.out_stride, 4, 2))
    return fail(FA_ERR_INVALID, "fa_decode_paged: q/caches/out need a unit last stride and 16-byte aligned rows");
  if (!p.block_table || !p.context_lens) return fail(FA_ERR_INVALID, "fa_decode_paged: metadata is NULL");
  if (!p.workspace || !aligned16(p.workspace)) return fail(FA_ERR_INVALID, "fa_decode_paged: workspace");
  if ((reinterpret_cast<uintptr_t>(p.tickets) & 3u) != 0) return fail(FA_ERR_INVALID, "fa_decode_paged: tickets");
  return from_hip(fa::launch_paged(p, (hipStream_t)stream), "fa_decode_paged");
}

int fa_tiny_fwd_f32(const fa_tiny_params* params, void* stream) {
  if (!params) return fail(FA_ERR_INVALID, "fa_tiny_fwd_f32: params is NULL");
  const fa_tiny_params& p = *params;
  if (p.abi_version != FA_ABI_VERSION) return fail(FA_ERR_INVALID, "fa_tiny_fwd_f32: abi_version mismatch");
  if (p.seqlen < 1 || p.seqlen > 32 || p.batch <= 0 || p.heads <= 0)
    return fail(FA_ERR_INVALID, "fa_tiny_fwd_f32: bad shape");
  if (!p.q || !p.k || !p.v || !p.out) return fail(FA_ERR_INVALID, "fa_tiny_fwd_f32: NULL tensor");
  return from_hip(fa::launch_tiny(p, (hipStream_t)stream), "fa_tiny_fwd_f32");
}

int fa_kvcache_append(const fa_append_params* params, void* stream) {
  if (!params) return fail(FA_ERR_INVALID, "fa_kvcache_append: params is NULL");
  const fa_append_params& p = *params;
  if (p.abi_version != FA_ABI_VERSION) return fail(FA_ERR_INVALID, "fa_kvcache_append: abi_version mismatch");
  if (p.dtype != FA_DTYPE_F16 && p.dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_INVALID, "fa_kvcache_append: dtype must be f16 or bf16");
  if (p.head_dim <= 0 || p.head_dim % 8)
    return fail(FA_ERR_UNSUPPORTED, "fa_kvcache_append: head_dim %d not a multiple of 8", p.head_dim);
  if (p.batch <= 0 || p.heads_kv <= 0 || p.seqlen_new < 0 || p.seqlen_cache <= 0)
    return fail(FA_ERR_INVALID, "fa_kvcache_append: bad shape");
  if (!p.cache_seqlens) return fail(FA_ERR_INVALID, "fa_kvcache_append: cache_seqlens is NULL");
  if (p.seqlen_new == 0) return FA_OK;
  if (!rows_ok(p.k_new, p.k_new_stride, 4, 2) || !rows_ok(p.v_new, p.v_new_stride, 4, 2) ||
      !rows_ok(p.k_cache, p.k_cache_stride, 4, 2) || !rows_ok(p.v_cache, p.v_cache_stride, 4, 2))
    return fail(FA_ERR_INVALID, "fa_kvcache_append: tensors need a unit last stride and 16-byte aligned rows");
  return from_hip(fa::launch_append(p, (hipStream_t)stream), "fa_kvcache_append");
}

}  // extern "C"
