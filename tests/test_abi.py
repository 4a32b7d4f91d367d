"""The C-ABI library loads on a CPU host, exports every entry point the
public header declares, and agrees with the ctypes binding on struct layouts
(no compute calls: those need a GPU)."""

import ctypes
import os
import re
import subprocess

import pytest

from fa_rdna3 import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa_mi355x.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(fa_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_exports():
    assert set(_declared_functions()) == set(_native.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _native.library_path()], capture_output=True, text=True)
    if out.returncode == 0:
        for name in _declared_functions():
            assert re.search(rf"\bT {name}\b", out.stdout), name


def test_abi_version_and_struct_layouts():
    lib = _native.lib()
    assert lib.fa_abi_version() == _native.ABI_VERSION
    for which, struct in enumerate(_native._STRUCTS):
        assert lib.fa_params_size(which) == ctypes.sizeof(struct), struct.__name__
    assert lib.fa_params_size(99) == 0


def test_workspace_size():
    # (splits + 1) * B * H * Sq * (D + 1) fp32, rounded up to 256 bytes: one
    # partial slot per split and sequence, plus one per sequence for the
    # length-proportional shares of the balanced partition
    n = _native.decode_workspace_bytes(4, 32, 1, 128, 8)
    assert n == (9 * 4 * 32 * 1 * 129 * 4 + 255) // 256 * 256
    assert _native.lib().fa_decode_ticket_count(4, 32, 3) == 4 * 32 * 3
    assert _native.decode_workspace_bytes(0, 32, 1, 128, 8) == 0


def test_null_params_are_rejected_without_touching_a_gpu():
    lib = _native.lib()
    assert lib.fa_fwd(None, None) == 1
    assert b"NULL" in lib.fa_last_error_string()
    assert lib.fa_bwd_phase(None, 5, None) == 1


def test_bad_arguments_are_rejected_before_launch():
    lib = _native.lib()
    p = _native.FwdParams()
    p.abi_version = 99
    assert lib.fa_fwd(ctypes.byref(p), None) == 1
    assert b"abi_version" in lib.fa_last_error_string()
    p.abi_version = _native.ABI_VERSION
    p.dtype, p.head_dim = 0, 48
    assert lib.fa_fwd(ctypes.byref(p), None) == 2
    assert b"head_dim" in lib.fa_last_error_string()
    p.head_dim, p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_k = 64, 1, 6, 4, 8, 8
    assert lib.fa_fwd(ctypes.byref(p), None) == 1
    t = _native.TinyParams()
    t.abi_version, t.seqlen = _native.ABI_VERSION, 33
    assert lib.fa_tiny_fwd_f32(ctypes.byref(t), None) == 1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(RuntimeError, match="native library not found"):
        _native.lib()


def test_bwd_ds_workspace_size():
    """fa_bwd_workspace_bytes: 64-key x 128-query tiles of 16-bit dS per
    (batch, query head) plus 1 KiB; 0 where the dS path does not apply."""
    lib = _native.lib()
    p = _native.BwdParams()
    p.fwd.abi_version, p.fwd.dtype = _native.ABI_VERSION, 0
    p.fwd.batch, p.fwd.heads_q, p.fwd.heads_kv = 2, 16, 16
    p.fwd.seqlen_q = p.fwd.seqlen_k = 2048
    p.fwd.head_dim = 128
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(p)) == 2 * 16 * 32 * 16 * 16384 + 1024
    p.fwd.seqlen_q, p.fwd.seqlen_k = 129, 65  # 2 query blocks x 2 key blocks
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(p)) == 2 * 16 * 4 * 16384 + 1024
    p.fwd.head_dim = 32
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(p)) == 0
    p.fwd.head_dim, p.fwd.dtype = 128, 2  # fp32
    assert lib.fa_bwd_workspace_bytes(ctypes.byref(p)) == 0
    assert lib.fa_bwd_workspace_bytes(None) == 0


def test_bwd_ds_workspace_min_size_and_chunk_rule():
    """fa_bwd_workspace_min_bytes: half the KV heads' share of the dS scratch
    (the bound is linear in the heads) plus the slack, when each half holds
    at least 1 GiB and the problem has no bias / ALiBi / dropout; the full
    size otherwise; 0 where the dS path does not apply.  ds_scratch_bytes
    picks the whole scratch, else one chunk's, else nothing."""
    lib = _native.lib()
    p = _native.BwdParams()
    p.fwd.abi_version, p.fwd.dtype = _native.ABI_VERSION, 0
    p.fwd.batch, p.fwd.heads_q, p.fwd.heads_kv = 1, 32, 32
    p.fwd.seqlen_q = p.fwd.seqlen_k = 16384
    p.fwd.head_dim = 128
    full = lib.fa_bwd_workspace_bytes(ctypes.byref(p))
    head = 256 * 128 * 16384  # 64-key x 128-query tiles of 16 KiB per head
    assert full == 32 * head + 1024
    half = lib.fa_bwd_workspace_min_bytes(ctypes.byref(p))
    assert half == 16 * head + 1024
    assert _native.ds_scratch_bytes(full, half, full) == full
    assert _native.ds_scratch_bytes(full, half, full - 1) == half
    assert _native.ds_scratch_bytes(full, half, half - 1) == 0
    p.fwd.heads_kv = 3  # odd KV head count: ceil(3 / 2) = 2 of 3 per chunk
    p.fwd.heads_q = 3
    assert lib.fa_bwd_workspace_min_bytes(ctypes.byref(p)) == 2 * head + 1024
    p.fwd.heads_q = p.fwd.heads_kv = 32
    p.fwd.dropout_p = 0.1
    assert lib.fa_bwd_workspace_min_bytes(ctypes.byref(p)) == full
    p.fwd.dropout_p = 0.0
    slopes = (ctypes.c_float * 32)()
    p.fwd.alibi_slopes = ctypes.addressof(slopes)
    assert lib.fa_bwd_workspace_min_bytes(ctypes.byref(p)) == full
    p.fwd.alibi_slopes = None
    # A half below 1 GiB of dS is not chunked: config 2 (268 MB in all).
    p.fwd.batch, p.fwd.heads_q, p.fwd.heads_kv, p.fwd.seqlen_q, p.fwd.seqlen_k = 2, 16, 16, 2048, 2048
    assert lib.fa_bwd_workspace_min_bytes(ctypes.byref(p)) == lib.fa_bwd_workspace_bytes(ctypes.byref(p))
    p.fwd.head_dim = 32
    assert lib.fa_bwd_workspace_min_bytes(ctypes.byref(p)) == 0
    assert lib.fa_bwd_workspace_min_bytes(None) == 0


def test_torch_host_library_registers_its_operators():
    """libfa_torch.so (the C++ host path of the dense forward / backward)
    loads with the C-ABI library and registers its operators; the dS
    scratch limit round-trips through it (no compute without a GPU)."""
    ops = _native.ops()
    for name in ("attention", "forward", "backward", "set_ds_scratch_limit", "ds_scratch_limit"):
        assert hasattr(ops, name), name
    saved = _native.set_ds_scratch_limit(12345)
    try:
        assert _native.ds_scratch_limit() == 12345
    finally:
        _native.set_ds_scratch_limit(saved)
    assert _native.ds_scratch_limit() == saved


def test_torch_host_operators_refuse_host_tensors():
    """The native operators hand bare pointers to the C ABI, so they refuse
    tensors that are not on a GPU before any launch (no GPU needed)."""
    import torch

    ops = _native.ops()
    q = torch.zeros(1, 1, 8, 64, dtype=torch.float16)
    args = (True, 0.125, -1, -1, 0.0, None, None, 0.0, 0)
    for fn in (ops.attention, ops.forward):
        with pytest.raises(Exception, match="GPU|CUDA|backend"):
            fn(q, q, q, *args)
    with pytest.raises(Exception, match="GPU|CUDA|backend"):
        ops.backward(q, q, q, q, q, torch.zeros(1, 1, 8), *args)


def test_bwd_phase2_on_unfilled_ds_scratch_is_refused():
    """With dS scratch, dQ alone (fa_bwd_phase 2) reads the dS that phase 1
    stored; on a scratch where phase 1 of that problem never ran it is
    refused before any launch (no GPU needed for the refusal)."""
    lib = _native.lib()
    p = _native.BwdParams()
    f = p.fwd
    f.abi_version, f.dtype = _native.ABI_VERSION, 0
    f.batch, f.heads_q, f.heads_kv, f.seqlen_q, f.seqlen_k, f.head_dim = 1, 2, 2, 256, 256, 128
    f.softmax_scale = 0.125
    base = 1 << 32
    f.q, f.k, f.v, f.out, f.lse = base, base + (1 << 24), base + (2 << 24), base + (3 << 24), base + (4 << 24)
    p.dout, p.dq, p.dk, p.dv, p.delta = (base + (i << 24) for i in range(5, 10))
    for name in ("q_stride", "k_stride", "v_stride", "out_stride"):
        getattr(f, name)[:] = [2 * 256 * 128, 256 * 128, 128, 1]
    for name in ("dout_stride", "dq_stride", "dk_stride", "dv_stride"):
        getattr(p, name)[:] = [2 * 256 * 128, 256 * 128, 128, 1]
    f.lse_stride[:] = [512, 256, 1]
    p.delta_stride[:] = [512, 256, 1]
    need = lib.fa_bwd_workspace_bytes(ctypes.byref(p))
    assert need > 0
    p.ds_workspace, p.ds_workspace_bytes = base + (12 << 24), need
    assert lib.fa_bwd_phase(ctypes.byref(p), 2, None) == 1
    assert b"phase 1" in lib.fa_last_error_string()


def test_hbm_read_probe_describes_its_variants_and_checks_arguments():
    """The read-ceiling probe exports a variant list and rejects bad
    arguments before any launch (no GPU needed for either)."""
    lib = _native.lib()
    names = _native.hbm_read_probe_variants()
    assert len(names) == lib.fa_hbm_read_probe_count() >= 12
    assert all("threads" in n for n in names)
    assert lib.fa_hbm_read_probe(None, 256, None, 0, None) == 1
    assert lib.fa_hbm_read_probe(1 << 32, 24, 1 << 33, 0, None) == 1   # size not a multiple of 16
    assert lib.fa_hbm_read_probe(1 << 32, 256, 1 << 33, -1, None) == 1
