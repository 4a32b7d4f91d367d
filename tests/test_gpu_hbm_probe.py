"""The streaming-read probe behind bench.py's `hbm_read_ceiling`: every
variant runs on a buffer that is not a multiple of its span (tail lanes
re-read the last piece), leaves the sink untouched (the data never produce
its magic value) and rejects bad arguments before any launch."""

import ctypes

import pytest
import torch

from fa_rdna3 import _native

pytestmark = pytest.mark.gpu


def test_every_variant_reads_and_leaves_the_sink_alone():
    names = _native.hbm_read_probe_variants()
    assert len(names) >= 12
    src = torch.arange((3 << 20) + 48, dtype=torch.int32, device="cuda")  # 12 MiB + 192 B
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    for vi in range(len(names)):
        _native.hbm_read_probe(src, sink, vi)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0


def test_bad_arguments_are_rejected():
    lib = _native.lib()
    src = torch.zeros(64, dtype=torch.int32, device="cuda")
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    assert lib.fa_hbm_read_probe(src.data_ptr(), 24, sink.data_ptr(), 0, None) == 1  # not a multiple of 16
    assert lib.fa_hbm_read_probe(src.data_ptr(), 256, sink.data_ptr(), 999, None) == 1
    assert lib.fa_hbm_read_probe(None, 256, sink.data_ptr(), 0, None) == 1
    assert lib.fa_hbm_read_probe_name(999) == b""
