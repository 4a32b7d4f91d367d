/*
 * fa_mi355x.h - C ABI of the MI355X (gfx950) FlashAttention-2 kernels.
 *
 * Every entry point replaces one group of Triton launch sites of the reference
 * (chelokot/flash-attention-rdna3, fa_rdna3/interface.py).  The boundary is
 * plain C: device pointers, element strides, sizes, scalars and an opaque
 * stream handle (a hipStream_t, or NULL for the null stream).  No torch types
 * cross it.
 *
 * Conventions
 *   - All strides are in ELEMENTS of the tensor they describe (not bytes), so
 *     arbitrary views (transposes, packed qkv, strided metadata) are accepted.
 *   - The caller owns every buffer, including LSE, delta and the decode split
 *     workspace; the library never allocates device memory and keeps no
 *     pointer after a call returns.
 *   - Calls are asynchronous on `stream` and never synchronise the host.
 *   - Every call returns FA_OK (0) or an fa_status code; a human-readable
 *     message for the last failure on the calling thread is available from
 *     fa_last_error_string().  Nothing throws across the ABI.
 *   - Argument contracts are checked by the host layer above (same messages as
 *     the reference's fa_rdna3/_validation.py); this layer re-checks only what
 *     would make a kernel read or write out of bounds (shape limits, dtype
 *     codes, head dims) and rejects it with FA_ERR_INVALID / FA_ERR_UNSUPPORTED.
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 4

typedef enum fa_dtype {
  FA_DTYPE_F16 = 0,
  FA_DTYPE_BF16 = 1,
  FA_DTYPE_F32 = 2
} fa_dtype;

typedef enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID = 1,     /* malformed arguments (null pointer, bad size) */
  FA_ERR_UNSUPPORTED = 2, /* valid but not implemented (head dim, dtype) */
  FA_ERR_LAUNCH = 3       /* hipGetLastError() reported a launch failure */
} fa_status;

/*
 * Forward attention with natural-log LSE, dense or packed-varlen.
 *
 * Replaces the `_attention_forward[grid](...)` launch of `_forward`
 * (interface.py:154-199, launch at :180) and the
 * `_attention_forward_varlen[grid](...)` launch of `_forward_varlen`
 * (interface.py:482-511, launch at :494).
 *
 * Dense:  q (B,Hq,Sq,D), k/v (B,Hkv,Sk,D), out like q, lse (B,Hq,Sq) fp32.
 * Varlen: cu_seqlens_q != NULL.  q (Tq,Hq,D) is described with
 *         q_stride = {0, stride(1), stride(0), stride(2)} (batch, head, row,
 *         dim); lse (Hq,Tq) with lse_stride = {0, stride(0), stride(1)}.
 *         Sequence b covers rows [cu_q[b], cu_q[b+1]) clamped to [0, total_q]
 *         (reference varlen.py:21-27); seqlen_q/seqlen_k carry max_seqlen.
 */
typedef struct fa_fwd_params {
  int32_t abi_version; /* must be FA_ABI_VERSION */
  int32_t dtype;       /* fa_dtype of q, k, v, out */
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  int64_t q_stride[4];   /* batch, head, row, dim */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t lse_stride[3]; /* batch, head, row */
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t seqlen_q; /* dense: Sq.  varlen: max_seqlen_q */
  int32_t seqlen_k; /* dense: Sk.  varlen: max_seqlen_k */
  int32_t head_dim; /* 32, 64, 128, 256 or 512 */
  const int32_t* cu_seqlens_q; /* NULL for dense */
  const int32_t* cu_seqlens_k;
  int32_t total_q;
  int32_t total_k;
  float softmax_scale;
  int32_t causal;       /* bottom-right aligned when Sq != Sk */
  int32_t window_left;  /* -1: unbounded */
  int32_t window_right; /* -1: unbounded */
  float softcap;        /* 0: off; else softcap*tanh(s/softcap) */
  const void* bias;     /* NULL or additive logit bias (B,Hq,Sq,Sk) view */
  int32_t bias_dtype;   /* fa_dtype of bias (q dtype or FA_DTYPE_F32) */
  int32_t reserved0;
  int64_t bias_stride[4]; /* broadcast dims carry stride 0 */
  const float* alibi_slopes; /* NULL or (Hq,) fp32 */
  float dropout_p;
  int32_t reserved1;
  uint64_t dropout_seed;
} fa_fwd_params;

/*
 * Backward: delta precompute, dK/dV and dQ in one call (three kernels on the
 * same stream, no atomics, deterministic).
 *
 * Replaces `_backward` (interface.py:202-277, launches at :226, :236, :258)
 * and `_backward_varlen` (interface.py:514-580, launches at :531, :541, :562).
 * `delta` is caller-provided scratch shaped like lse.  Gradients are written
 * in the dtype of q/k/v with their own strides.
 */
typedef struct fa_bwd_params {
  fa_fwd_params fwd; /* q, k, v, out, lse and every option of the forward */
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  float* delta;
  int64_t dout_stride[4];
  int64_t dq_stride[4];
  int64_t dk_stride[4];
  int64_t dv_stride[4];
  int64_t delta_stride[3];
  /* Optional score-gradient scratch (no counterpart in the reference, whose
   * dQ kernel recomputes the scores).  When non-NULL and at least
   * fa_bwd_workspace_bytes(params) bytes, the dK/dV pass stores the 16-bit
   * dS it already forms and dQ becomes the single product dS K, instead of
   * recomputing S and dP (two of its three matrix products).  A smaller
   * scratch of at least fa_bwd_workspace_min_bytes(params) makes fa_bwd run
   * dK/dV and dQ in two chunks of KV heads (large problems without bias,
   * ALiBi or dropout).  NULL, or less than that: dQ recomputes.
   * Results agree either way to the rounding of the accumulation order. */
  void* ds_workspace;
  int64_t ds_workspace_bytes;
} fa_bwd_params;

/*
 * Split-K decode with an LSE-weighted merge.
 *
 * Replaces `flash_attention_decode`'s two launches (interface.py:427-479,
 * `_attention_split` at :458 and `_attention_combine` at :471).
 * q (B,Hq,Sq,D), k/v (B,Hkv,Sk,D), out like q.  Non-causal as in the
 * reference.  When cache_seqlens != NULL, sequence b only attends keys
 * [0, len_b) with len_b = cache_seqlens[b] + cache_seqlens_add clamped to
 * [0, Sk]; a length of 0
 * yields a zero output row.  `causal` (no counterpart in the reference's
 * decode; used by the kv-cache entry point below) masks bottom-right per
 * sequence: query row i sees keys j <= len_b - Sq + i, and a row that sees
 * no key yields zeros.
 * `workspace` must hold fa_decode_workspace_bytes(...) bytes.
 */
typedef struct fa_decode_params {
  int32_t abi_version;
  int32_t dtype; /* FA_DTYPE_F16 or FA_DTYPE_BF16 */
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t seqlen_q;
  int32_t seqlen_k;
  int32_t head_dim;
  const int32_t* cache_seqlens; /* NULL: every sequence has Sk keys */
  int64_t cache_seqlens_stride;
  float softmax_scale;
  int32_t num_splits; /* 1..64 */
  void* workspace;
  int32_t causal; /* 0 or 1, see above */
  int32_t cache_seqlens_add; /* added to every cache_seqlens[b] before clamping
                                (rows just appended by fa_kvcache_append); 0 otherwise */
  int32_t kv_fp8;  /* 1: k and v are fp8 (OCP e4m3) holding K / k_scale and V / v_scale;
                      0: they have `dtype` and the scales are ignored */
  float k_scale;
  float v_scale;
  int32_t reserved0;
  uint32_t* tickets; /* NULL: the split partials are merged by a second launch.
                        Else fa_decode_ticket_count(...) uint32 arrival counters,
                        all zero before the call and left zero by it: the last
                        split of each (batch, KV head, 16-row block) merges the
                        partials in the same launch (head_dim <= 128 kernels;
                        the others keep the second launch).  Calls that share
                        one tickets array must not overlap in time. */
} fa_decode_params;

/*
 * Appends new keys / values to a contiguous KV cache in place:
 * k_cache[b, h, cache_seqlens[b] + s, :] = k_new[b, h, s, :] (same for v) for
 * s < Snew.  Rows that would land outside [0, Sc) are skipped.
 *
 * No counterpart in the reference (its decode takes a ready cache,
 * interface.py:427-479); it is the cache-update half of the
 * flash_attn_with_kvcache-style entry point (`flash_attention_with_kvcache`).
 * k_new/v_new (B,Hkv,Snew,D); k_cache/v_cache (B,Hkv,Sc,D); cache_seqlens
 * (B,) int32, not modified.  Unit last stride and 16-byte aligned rows.
 */
typedef struct fa_append_params {
  int32_t abi_version;
  int32_t dtype; /* FA_DTYPE_F16 or FA_DTYPE_BF16 */
  const void* k_new;
  const void* v_new;
  void* k_cache;
  void* v_cache;
  const int32_t* cache_seqlens;
  int64_t cache_seqlens_stride;
  int64_t k_new_stride[4];
  int64_t v_new_stride[4];
  int64_t k_cache_stride[4];
  int64_t v_cache_stride[4];
  int32_t batch;
  int32_t heads_kv;
  int32_t seqlen_new;
  int32_t seqlen_cache;
  int32_t head_dim;
  int32_t reserved0;
} fa_append_params;

/*
 * Paged-KV decode walking a block table (vLLM-style cache).
 *
 * Replaces `flash_attention_decode_paged`'s launches (interface.py:643-728,
 * `_attention_decode_paged` at :704 and `_attention_combine` at :720).
 * q (B,Hq,D) in the reference, here (B,Hq,Sq,D) with seqlen_q = Sq (1 for
 * the reference's case); k_cache/v_cache (num_blocks, block_size, Hkv, D);
 * block_table (B, max_blocks) int32; context_lens (B,) int32.  Context is
 * clamped to [0, max_blocks*block_size] and physical ids outside
 * [0, num_blocks) contribute nothing (reference paged.py:37-38, :58-59).
 * With Sq > 1 (speculative / chunked decode, no counterpart in the
 * reference) `causal` masks bottom-right per sequence as in
 * fa_decode_params.
 */
typedef struct fa_paged_params {
  int32_t abi_version;
  int32_t dtype; /* FA_DTYPE_F16 or FA_DTYPE_BF16 */
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* out;
  const int32_t* block_table;
  const int32_t* context_lens;
  int64_t q_stride[4];  /* batch, head, row, dim */
  int64_t k_stride[4];  /* block, position, head, dim */
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t block_table_stride[2];
  int64_t context_lens_stride;
  int32_t batch;
  int32_t heads_q;
  int32_t heads_kv;
  int32_t head_dim;
  int32_t num_blocks;
  int32_t block_size; /* power of two, 1..256 */
  int32_t max_blocks; /* columns of block_table */
  int32_t num_splits; /* 1..64 */
  float softmax_scale;
  int32_t seqlen_q; /* query rows per sequence, >= 1 */
  void* workspace; /* fa_decode_workspace_bytes(batch, heads_q, seqlen_q, head_dim, num_splits) */
  int32_t causal;  /* 0 or 1 */
  int32_t kv_fp8;  /* 1: caches are fp8 (OCP e4m3) holding K / k_scale and V / v_scale;
                      0: they have `dtype` */
  float k_scale;
  float v_scale;
  uint32_t* tickets; /* NULL: the split partials are merged by a second launch.
                        Else fa_decode_ticket_count(...) uint32 arrival counters,
                        all zero before the call and left zero by it: the last
                        split of each (batch, KV head, 16-row block) merges the
                        partials in the same launch (head_dim <= 128 kernels;
                        the others keep the second launch).  Calls that share
                        one tickets array must not overlap in time. */
} fa_paged_params;

/*
 * Short-sequence fp32 inference forward (D = 128, S <= 32, non-causal).
 * Replaces the `_attention_tiny_forward` launch (interface.py:84-104).
 */
typedef struct fa_tiny_params {
  int32_t abi_version;
  int32_t seqlen; /* 1..32, Sq == Sk */
  const float* q;
  const float* k;
  const float* v;
  float* out;
  const float* bias; /* NULL or fp32 (B,H,S,S) view */
  int64_t q_stride[4];
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t bias_stride[4];
  int32_t batch;
  int32_t heads;
  float softmax_scale;
  int32_t reserved0;
} fa_tiny_params;

/* Version of this header the library was built from (FA_ABI_VERSION). */
int fa_abi_version(void);

/* Message describing the last non-FA_OK return on the calling thread. */
const char* fa_last_error_string(void);

/* sizeof() of each params struct as compiled into the library, so a binding
 * can verify its own layout: which = 0 fwd, 1 bwd, 2 decode, 3 paged, 4 tiny,
 * 5 append. */
size_t fa_params_size(int which);

/* Bytes of scratch the split-K and paged decode need for `num_splits`. */
size_t fa_decode_workspace_bytes(int batch, int heads_q, int seqlen_q,
                                 int head_dim, int num_splits);

int fa_fwd(const fa_fwd_params* params, void* stream);
int fa_bwd(const fa_bwd_params* params, void* stream);
/* One stage of fa_bwd: 0 = delta, 1 = dK/dV, 2 = dQ (1 and 2 read delta).
 * No counterpart in the reference (its three backward launches are separate
 * Triton calls, interface.py:226/:236/:258); it exists so profilers and
 * benchmarks can time each backward kernel on its own.  With ds_workspace,
 * phase 2 reads the dS that phase 1 stored there: phase 2 is refused
 * (FA_ERR_INVALID) unless the last phase-1 call on that scratch had the same
 * forward problem, dout, delta and scratch size (memory reused by others in
 * between cannot be detected). */
int fa_bwd_phase(const fa_bwd_params* params, int phase, void* stream);
/* Bytes of ds_workspace the backward of `params` can use (0: the dS path
 * does not apply: fp32, head_dim other than 64 or 128, or more than 512
 * varlen sequences).
 * Dense: batch * heads_q * ceil(Sk / 64) * ceil(Sq / 128) * 16 KiB plus
 * 1 KiB; varlen, an upper bound from max_seqlen_k, total_q and batch.  With dS scratch, phase 2 of
 * fa_bwd_phase reads the dS that phase 1 stored. */
size_t fa_bwd_workspace_bytes(const fa_bwd_params* params);
/* No counterpart in the reference.  The smallest ds_workspace fa_bwd uses
 * the dS path with: for a problem it chunks, the dS of ceil(heads_kv / 2)
 * KV heads and their query heads (plus the 1 KiB slack), and fa_bwd then
 * runs dK/dV and dQ once per half of the KV heads.  It chunks only when
 * each half holds at least 1 GiB of dS and the problem has no bias, ALiBi
 * or dropout (their head index would shift); smaller or more chunks measured
 * slower than recomputing dQ.  Otherwise equal to fa_bwd_workspace_bytes
 * (0 when the dS path does not apply).  fa_bwd_phase uses the dS path only
 * with the full fa_bwd_workspace_bytes. */
size_t fa_bwd_workspace_min_bytes(const fa_bwd_params* params);
/* uint32 counters `tickets` needs: batch * heads_q * seqlen_q. */
size_t fa_decode_ticket_count(int batch, int heads_q, int seqlen_q);

int fa_decode_splitk(const fa_decode_params* params, void* stream);

/*
 * fa_decode_splitk without any caller scratch and without any allocation.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, and
 * harnesses that forbid hipMalloc.  `workspace` and `tickets` in params are
 * ignored.  The split partials and the merge's arrival counters live in a
 * static scratch array of FA_NOALLOC_WORKSPACE_BYTES + 4 * FA_NOALLOC_TICKETS
 * bytes, one per GPU, held until the process ends.  A call that would need
 * more (fa_decode_workspace_bytes(...) > FA_NOALLOC_WORKSPACE_BYTES, or
 * batch * heads_q * seqlen_q > FA_NOALLOC_TICKETS) fails with FA_ERR_INVALID.
 * Every call on one GPU shares that GPU's scratch.  Calls made outside graph
 * capture are ordered on the device in the order they are made on the host:
 * a call on another stream than the previous call's first waits for that
 * call (an event the library creates on the device's first call, completed
 * by the decode kernel itself; no device memory).  Under graph capture nothing is recorded or waited for, so graph
 * replays must not overlap other calls on the same GPU.  The counters start
 * at zero when the library loads and every call leaves them at zero.
 */
#define FA_NOALLOC_WORKSPACE_BYTES (32 * 1024 * 1024)
#define FA_NOALLOC_TICKETS 65536
int fa_decode_splitk_noalloc(const fa_decode_params* params, void* stream);
int fa_decode_paged(const fa_paged_params* params, void* stream);

/*
 * HBM streaming-read probe.  No counterpart in the reference: it is the
 * measurement the HBM-bound decode kernels are compared against.  Reads
 * every byte of [src, src + bytes) once with 16-byte loads (bytes a multiple
 * of 16, src 16-byte aligned) and writes at most a few bytes of `sink`
 * (>= 4 KiB of device memory).  `variant` in [0, fa_hbm_read_probe_count())
 * picks the block size, loads in flight per lane, plain or nontemporal loads,
 * and one-pass or persistent grid; fa_hbm_read_probe_name describes it.
 * Returns 0, or 1 for bad arguments, 3 for a launch failure.
 */
int fa_hbm_read_probe_count(void);
const char* fa_hbm_read_probe_name(int variant);
int fa_hbm_read_probe(const void* src, size_t bytes, void* sink, int variant, void* stream);
int fa_tiny_fwd_f32(const fa_tiny_params* params, void* stream);
int fa_kvcache_append(const fa_append_params* params, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
