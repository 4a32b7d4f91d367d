"""ctypes binding of the MI355X C ABI (``include/fa_mi355x.h``).

This module is the only place that touches ``libfa_mi355x.so``.  It mirrors
the header's parameter structs, checks at load time that their sizes match
what the library was compiled with, and turns a non-zero status into a
``RuntimeError`` carrying ``fa_last_error_string()``.  There is no fallback:
if the library is missing the import of any compute path fails loudly.
"""

import ctypes
import os
import threading

import torch

ABI_VERSION = 4
DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_LIB_NAME = "libfa_mi355x.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)
# PyTorch host glue of the dense forward / backward (csrc/fa_torch.cpp):
# registers the torch.ops.fa_mi355x operators on top of the C ABI.
_TORCH_LIB_NAME = "libfa_torch.so"
_TORCH_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _TORCH_LIB_NAME)

_i64_4 = ctypes.c_int64 * 4
_i64_3 = ctypes.c_int64 * 3
_i64_2 = ctypes.c_int64 * 2


class FwdParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("q_stride", _i64_4), ("k_stride", _i64_4), ("v_stride", _i64_4),
        ("out_stride", _i64_4), ("lse_stride", _i64_3),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p), ("cu_seqlens_k", ctypes.c_void_p),
        ("total_q", ctypes.c_int32), ("total_k", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("causal", ctypes.c_int32), ("window_left", ctypes.c_int32), ("window_right", ctypes.c_int32),
        ("softcap", ctypes.c_float),
        ("bias", ctypes.c_void_p), ("bias_dtype", ctypes.c_int32), ("reserved0", ctypes.c_int32),
        ("bias_stride", _i64_4),
        ("alibi_slopes", ctypes.c_void_p),
        ("dropout_p", ctypes.c_float), ("reserved1", ctypes.c_int32),
        ("dropout_seed", ctypes.c_uint64),
    ]


class BwdParams(ctypes.Structure):
    _fields_ = [
        ("fwd", FwdParams),
        ("dout", ctypes.c_void_p), ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p), ("delta", ctypes.c_void_p),
        ("dout_stride", _i64_4), ("dq_stride", _i64_4), ("dk_stride", _i64_4),
        ("dv_stride", _i64_4), ("delta_stride", _i64_3),
        ("ds_workspace", ctypes.c_void_p), ("ds_workspace_bytes", ctypes.c_int64),
    ]


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("q_stride", _i64_4), ("k_stride", _i64_4), ("v_stride", _i64_4), ("out_stride", _i64_4),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("cache_seqlens", ctypes.c_void_p), ("cache_seqlens_stride", ctypes.c_int64),
        ("softmax_scale", ctypes.c_float), ("num_splits", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("causal", ctypes.c_int32), ("cache_seqlens_add", ctypes.c_int32),
        ("kv_fp8", ctypes.c_int32), ("k_scale", ctypes.c_float), ("v_scale", ctypes.c_float),
        ("reserved0", ctypes.c_int32), ("tickets", ctypes.c_void_p),
    ]


class AppendParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("k_new", ctypes.c_void_p), ("v_new", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("cache_seqlens", ctypes.c_void_p), ("cache_seqlens_stride", ctypes.c_int64),
        ("k_new_stride", _i64_4), ("v_new_stride", _i64_4),
        ("k_cache_stride", _i64_4), ("v_cache_stride", _i64_4),
        ("batch", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("seqlen_new", ctypes.c_int32), ("seqlen_cache", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("reserved0", ctypes.c_int32),
    ]


class PagedParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("block_table", ctypes.c_void_p), ("context_lens", ctypes.c_void_p),
        ("q_stride", _i64_4), ("k_stride", _i64_4), ("v_stride", _i64_4), ("out_stride", _i64_4),
        ("block_table_stride", _i64_2), ("context_lens_stride", ctypes.c_int64),
        ("batch", ctypes.c_int32), ("heads_q", ctypes.c_int32), ("heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("num_blocks", ctypes.c_int32), ("block_size", ctypes.c_int32),
        ("max_blocks", ctypes.c_int32), ("num_splits", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("seqlen_q", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("causal", ctypes.c_int32), ("kv_fp8", ctypes.c_int32),
        ("k_scale", ctypes.c_float), ("v_scale", ctypes.c_float),
        ("tickets", ctypes.c_void_p),
    ]


class TinyParams(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32), ("seqlen", ctypes.c_int32),
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("bias", ctypes.c_void_p),
        ("q_stride", _i64_4), ("k_stride", _i64_4), ("v_stride", _i64_4),
        ("out_stride", _i64_4), ("bias_stride", _i64_4),
        ("batch", ctypes.c_int32), ("heads", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float), ("reserved0", ctypes.c_int32),
    ]


_STRUCTS = (FwdParams, BwdParams, DecodeParams, PagedParams, TinyParams, AppendParams)
EXPORTS = (
    "fa_abi_version", "fa_last_error_string", "fa_params_size", "fa_decode_workspace_bytes",
    "fa_decode_ticket_count",
    "fa_fwd", "fa_bwd", "fa_bwd_phase", "fa_bwd_workspace_bytes", "fa_bwd_workspace_min_bytes", "fa_decode_splitk", "fa_decode_splitk_noalloc", "fa_decode_paged",
    "fa_tiny_fwd_f32",
    "fa_kvcache_append",
    "fa_hbm_read_probe_count", "fa_hbm_read_probe_name", "fa_hbm_read_probe",
)

_lib = None
_lock = threading.Lock()


def library_path():
    return _LIB_PATH


def lib():
    """Load (once) and return the native library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"fa_rdna3 native library not found at {_LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__; __graft_entry__.build()'` or "
                "`make -C flash-attention-rdna3_amd/csrc`")
        handle = ctypes.CDLL(_LIB_PATH)
        handle.fa_abi_version.restype = ctypes.c_int
        handle.fa_last_error_string.restype = ctypes.c_char_p
        handle.fa_params_size.restype = ctypes.c_size_t
        handle.fa_params_size.argtypes = [ctypes.c_int]
        handle.fa_decode_workspace_bytes.restype = ctypes.c_size_t
        handle.fa_decode_workspace_bytes.argtypes = [ctypes.c_int] * 5
        handle.fa_bwd_workspace_bytes.restype = ctypes.c_size_t
        handle.fa_bwd_workspace_bytes.argtypes = [ctypes.c_void_p]
        handle.fa_bwd_workspace_min_bytes.restype = ctypes.c_size_t
        handle.fa_bwd_workspace_min_bytes.argtypes = [ctypes.c_void_p]
        handle.fa_decode_ticket_count.restype = ctypes.c_size_t
        handle.fa_decode_ticket_count.argtypes = [ctypes.c_int] * 3
        for name, struct in (("fa_fwd", FwdParams), ("fa_bwd", BwdParams),
                             ("fa_decode_splitk", DecodeParams), ("fa_decode_splitk_noalloc", DecodeParams),
                             ("fa_decode_paged", PagedParams),
                             ("fa_tiny_fwd_f32", TinyParams), ("fa_kvcache_append", AppendParams)):
            fn = getattr(handle, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.POINTER(struct), ctypes.c_void_p]
        handle.fa_bwd_phase.restype = ctypes.c_int
        handle.fa_hbm_read_probe_count.restype = ctypes.c_int
        handle.fa_hbm_read_probe_name.restype = ctypes.c_char_p
        handle.fa_hbm_read_probe_name.argtypes = [ctypes.c_int]
        handle.fa_hbm_read_probe.restype = ctypes.c_int
        handle.fa_hbm_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                             ctypes.c_void_p]
        handle.fa_bwd_phase.argtypes = [ctypes.POINTER(BwdParams), ctypes.c_int, ctypes.c_void_p]
        if handle.fa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{_LIB_NAME} ABI {handle.fa_abi_version()} != binding ABI {ABI_VERSION}")
        for which, struct in enumerate(_STRUCTS):
            if handle.fa_params_size(which) != ctypes.sizeof(struct):
                raise RuntimeError(
                    f"{struct.__name__} layout mismatch: library {handle.fa_params_size(which)} bytes, "
                    f"binding {ctypes.sizeof(struct)} bytes")
        if not os.path.exists(_TORCH_LIB_PATH):
            raise RuntimeError(
                f"fa_rdna3 torch host library not found at {_TORCH_LIB_PATH}; build it with "
                "`make -C flash-attention-rdna3_amd/csrc`")
        torch.ops.load_library(_TORCH_LIB_PATH)
        _lib = handle
        return _lib


def ops():
    """The ``torch.ops.fa_mi355x`` namespace (dense forward / backward and
    the differentiable ``attention``), loaded with the native library."""
    lib()
    return torch.ops.fa_mi355x


def _check(rc, what):
    if rc != 0:
        msg = lib().fa_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def _stream(tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def call(name, params, device_tensor):
    """Invoke an fa_* entry point on the current stream of the tensor's device."""
    fn = getattr(lib(), name)
    _check(fn(ctypes.byref(params), _stream(device_tensor)), name)


def call_bwd_phase(params, phase, device_tensor):
    _check(lib().fa_bwd_phase(ctypes.byref(params), int(phase), _stream(device_tensor)), "fa_bwd_phase")


def ds_scratch_limit():
    """Largest score-gradient (dS) scratch a backward allocates, in bytes
    (12 GiB by default).  A backward whose dS exceeds it runs in two chunks
    of KV heads when one chunk fits and the library chunks that problem
    (fa_bwd_workspace_min_bytes); otherwise dQ recomputes the scores instead
    of reading the stored dS.  0 means the dS path is off."""
    return int(ops().ds_scratch_limit())


def set_ds_scratch_limit(nbytes):
    """Set the dS scratch limit for every backward of this process (dense and
    varlen); returns the previous limit."""
    return int(ops().set_ds_scratch_limit(int(nbytes)))


def ds_scratch_bytes(full, half, limit):
    """Scratch bytes a backward takes under `limit`: the whole dS (`full`,
    fa_bwd_workspace_bytes), else one of the two KV-head chunks the library
    would run (`half`, fa_bwd_workspace_min_bytes, when smaller than
    `full`), else 0 (dQ then recomputes).  The C++ host path's rule."""
    if full <= 0:
        return 0
    if full <= limit:
        return full
    return half if 0 < half < full and half <= limit else 0


def attach_ds_scratch(params, device_tensor):
    """Give a filled BwdParams the dS scratch its backward can use (dQ as
    the single product dS K).  Returns the scratch tensor, which must stay
    alive until the launch is done, or None when the path does not apply."""
    full = int(lib().fa_bwd_workspace_bytes(ctypes.byref(params)))
    half = int(lib().fa_bwd_workspace_min_bytes(ctypes.byref(params)))
    need = ds_scratch_bytes(full, half, ds_scratch_limit())
    if need == 0:
        params.ds_workspace, params.ds_workspace_bytes = None, 0
        return None
    buf = torch.empty(need, dtype=torch.uint8, device=device_tensor.device)
    params.ds_workspace, params.ds_workspace_bytes = buf.data_ptr(), need
    return buf


def decode_workspace_bytes(batch, heads_q, seqlen_q, head_dim, num_splits):
    return int(lib().fa_decode_workspace_bytes(batch, heads_q, seqlen_q, head_dim, num_splits))


# The split-K / paged decode merges its split partials inside the split
# launch (last-arriving workgroup, arrival counters in `decode_tickets`).
# False selects the two-launch path (split kernel, then a merge kernel).
FUSED_SPLIT_MERGE = True

_tickets = {}


def decode_tickets(device_tensor, batch, heads_q, seqlen_q):
    """Address of zeroed uint32 arrival counters for one decode call on the
    current stream of the tensor's device, or None for the two-launch merge.

    The decode kernels leave every counter at zero, so one buffer per
    (device, stream) serves all calls issued in stream order; it grows when
    a call needs more counters than it holds.

    Under HIP graph capture no buffer is created: a capture only records the
    zero fill, so a buffer made then would hold undefined counters for
    every later eager call or other graph on that stream.  A call captured
    before its stream has a large enough buffer therefore takes the
    two-launch merge (None).  A buffer that a graph may have recorded is
    never freed: when a larger one replaces it, the old one is kept alive
    for the life of the process."""
    if not FUSED_SPLIT_MERGE:
        return None
    need = int(lib().fa_decode_ticket_count(batch, heads_q, seqlen_q))
    stream = torch.cuda.current_stream(device_tensor.device)
    key = (device_tensor.device.index, stream.cuda_stream)
    buf = _tickets.get(key)
    if buf is None or buf.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            return None
        size = max(need, 1024 if buf is None else 2 * buf.numel())
        if buf is not None:
            _retired_tickets.append(buf)
        buf = torch.zeros(size, dtype=torch.int32, device=device_tensor.device)
        _tickets[key] = buf
    return buf.data_ptr()


_retired_tickets = []


def kernel_ready(t):
    """Return ``t`` or a contiguous copy so rows satisfy the ABI's vector-load
    contract (unit last stride, 16-byte aligned row starts)."""
    esize = t.element_size()
    ok = t.stride(-1) == 1 or t.shape[-1] == 1
    ok = ok and t.data_ptr() % 16 == 0
    ok = ok and all((s * esize) % 16 == 0 for s, n in zip(t.stride()[:-1], t.shape[:-1]) if n > 1)
    if ok and t.stride(-1) == 1:
        return t
    return t.contiguous()


def strides(t, n=None):
    """Element strides of ``t`` for the ABI: size-1 dims (never stepped over)
    get stride 0, and the last dim is contiguous (see ``kernel_ready``)."""
    st = [s if sz > 1 else 0 for s, sz in zip(t.stride(), t.shape)]
    st[-1] = 1
    return st if n is None else st[:n]


def hbm_read_probe(src, sink, variant):
    """Read every byte of the device tensor ``src`` once with the streaming
    read probe ``variant`` on the current stream (``sink``: >= 4 KiB of
    device memory).  A measurement utility, not part of the attention path."""
    nbytes = src.numel() * src.element_size()
    _check(lib().fa_hbm_read_probe(src.data_ptr(), nbytes, sink.data_ptr(), int(variant), _stream(src)),
           "fa_hbm_read_probe")


def hbm_read_probe_variants():
    """Descriptions of the streaming read probe's variants, by index."""
    n = lib().fa_hbm_read_probe_count()
    return [lib().fa_hbm_read_probe_name(i).decode() for i in range(n)]
