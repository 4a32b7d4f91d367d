"""ComfyUI adapter (fa_rdna3/comfyui.py) without ComfyUI itself; the cases
follow the reference's tests/test_comfyui.py.  CPU tests swap the kernel
entry point for a recorder; the `gpu` ones compare with torch SDPA."""

import os
import subprocess
import sys

import pytest
import torch
import torch.nn.functional as F

import fa_rdna3.comfyui as comfyui
import fa_rdna3.sdpa as sdpa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "flash-attention-rdna3_amd")


def _never(*args, **kwargs):
    raise AssertionError("this path must not run")


def test_comfy_layout_is_split_into_heads_and_restored(monkeypatch):
    q, k, v = torch.randn(2, 5, 12), torch.randn(2, 7, 12), torch.randn(2, 7, 12)
    mask = torch.ones(5, 7, dtype=torch.bool)
    mask[:, -1] = False
    seen = {}
    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: True)

    def kernel(qh, kh, vh, **kw):
        seen.update(q=qh, k=kh, v=vh, bias=kw["bias"], scale=kw["softmax_scale"])
        return qh

    monkeypatch.setattr(comfyui, "flash_attention", kernel)
    out = comfyui.ComfyUIAttentionOverride()(_never, q, k, v, 3, mask=mask, scale=0.25)
    assert seen["q"].shape == (2, 3, 5, 4) and seen["k"].shape == (2, 3, 7, 4) and seen["v"].shape == (2, 3, 7, 4)
    assert seen["scale"] == 0.25
    assert seen["bias"].shape == (1, 5, 7)
    assert torch.all(seen["bias"][..., :-1] == 0) and torch.all(seen["bias"][..., -1] == float("-inf"))
    torch.testing.assert_close(out, seen["q"].transpose(1, 2).reshape(2, 5, 12))
    # the head split is a view of the caller's tensor, not a copy
    torch.testing.assert_close(seen["q"][:, 1], q[:, :, 4:8])


def test_head_layout_and_gqa_pass_through(monkeypatch):
    q, k = torch.randn(2, 4, 5, 8), torch.randn(2, 2, 7, 8)
    v = torch.randn_like(k)
    seen = {}
    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: True)

    def kernel(qh, kh, vh, **kw):
        seen["shapes"] = (qh.shape, kh.shape, vh.shape)
        return qh

    monkeypatch.setattr(comfyui, "flash_attention", kernel)
    out = comfyui.ComfyUIAttentionOverride()(_never, q, k, v, 4, skip_reshape=True,
                                             skip_output_reshape=True, enable_gqa=True)
    assert seen["shapes"] == (q.shape, k.shape, v.shape)
    assert out is q


def test_gqa_in_comfy_layout_needs_enable_gqa(monkeypatch):
    q, k = torch.randn(1, 6, 32), torch.randn(1, 9, 16)   # 4 query heads, 2 kv heads of 8
    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: True)
    monkeypatch.setattr(comfyui, "flash_attention", lambda qh, kh, vh, **kw: qh)
    fallback = lambda *a, **kw: "fallback"
    assert comfyui.ComfyUIAttentionOverride()(fallback, q, k, k, 4) == "fallback"
    out = comfyui.ComfyUIAttentionOverride()(fallback, q, k, k, 4, enable_gqa=True)
    assert out.shape == (1, 6, 32)


@pytest.mark.parametrize("case", ["heads_not_int", "width_not_divisible", "rank", "batch"])
def test_unsplittable_inputs_fall_back(monkeypatch, case):
    monkeypatch.setattr(comfyui, "flash_attention", _never)
    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: True)
    q = torch.randn(2, 4, 16)
    k = v = q
    heads = 2
    if case == "heads_not_int":
        heads = True
    elif case == "width_not_divisible":
        heads = 3
    elif case == "rank":
        q = k = v = torch.randn(2, 4, 16, 1)
    else:
        k = v = torch.randn(3, 4, 16)
    assert comfyui.ComfyUIAttentionOverride()(lambda *a, **kw: "fallback", q, k, v, heads) == "fallback"


def test_existing_override_keeps_precedence_and_gets_a_wrapped_fallback(monkeypatch):
    calls = []

    def existing(attention, *args, **kwargs):
        calls.append(attention)
        return attention(*args, **kwargs)

    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: False)
    original = lambda *a, **kw: "original"
    q = torch.randn(1, 4, 16)
    assert comfyui.ComfyUIAttentionOverride(existing)(original, q, q, q, 2) == "original"
    assert len(calls) == 1 and calls[0] is not original
    monkeypatch.setattr(comfyui, "flash_attention", _never)
    assert comfyui.ComfyUIAttentionOverride(lambda att, *a, **kw: "existing")(original, q, q, q, 2) == "existing"


def test_existing_override_can_delegate_to_the_kernels(monkeypatch):
    monkeypatch.setattr(comfyui, "_is_supported", lambda *a: True)
    monkeypatch.setattr(comfyui, "flash_attention", lambda qh, kh, vh, **kw: qh)

    def add_one(attention, q, k, v, heads, **kwargs):
        return attention(q + 1, k, v, heads, **kwargs)

    q = torch.zeros(1, 4, 16)
    out = comfyui.ComfyUIAttentionOverride(add_one)(_never, q, q, q, 2)
    torch.testing.assert_close(out, torch.ones_like(q))


def test_fp32_accumulation_requests_fall_back(monkeypatch):
    monkeypatch.setattr(comfyui, "flash_attention", _never)
    q = torch.randn(1, 4, 16, dtype=torch.float16)
    fb = lambda *a, **kw: "fallback"
    assert comfyui.ComfyUIAttentionOverride()(fb, q, q, q, 2, attn_precision=torch.float32) == "fallback"
    upcast = comfyui.ComfyUIAttentionOverride(precision_resolver=lambda p, d: torch.float32)
    assert upcast(fb, q, q, q, 2) == "fallback"
    assert comfyui.ComfyUIAttentionOverride()(fb, q, q, q, 2, low_precision_attention=False) == "fallback"


def test_fallback_runs_with_the_sdpa_dispatch_bypassed(monkeypatch):
    seen = []
    monkeypatch.setattr(comfyui, "flash_attention", _never)

    def comfy_attention(q, k, v, heads, **kwargs):
        seen.append(getattr(sdpa._dispatch_bypass_state, "depth", 0))
        return "fallback"

    q = torch.randn(1, 4, 16)
    comfyui.ComfyUIAttentionOverride()(comfy_attention, q, q, q, 2, low_precision_attention=False)
    assert seen == [1]
    assert getattr(sdpa._dispatch_bypass_state, "depth", 0) == 0


class FakeModel:
    def __init__(self, transformer_options=None):
        self.model_options = {"transformer_options": dict(transformer_options or {})}

    def clone(self):
        return FakeModel(self.model_options["transformer_options"])


def test_node_clones_composes_and_enables_sdpa_dispatch(monkeypatch):
    enabled = []
    previous = lambda *a, **kw: "previous"
    model = FakeModel({"optimized_attention_override": previous})
    monkeypatch.setattr(comfyui, "unsupported_reason", lambda: None)
    monkeypatch.setattr(comfyui, "enable_rdna3_flash_attention", lambda: enabled.append(True))
    monkeypatch.setattr(comfyui, "_get_comfyui_precision_resolver", lambda: (lambda p, d: p))
    patched, = comfyui.ApplyRDNA3FlashAttention().patch(model)
    override = patched.model_options["transformer_options"]["optimized_attention_override"]
    assert patched is not model
    assert model.model_options["transformer_options"]["optimized_attention_override"] is previous
    assert isinstance(override, comfyui.ComfyUIAttentionOverride) and override.previous_override is previous
    assert enabled == [True]
    # patching an already patched model reuses its override instead of nesting
    again, = comfyui.ApplyRDNA3FlashAttention().patch(patched)
    assert again.model_options["transformer_options"]["optimized_attention_override"] is override


def test_node_errors(monkeypatch):
    monkeypatch.setattr(comfyui, "unsupported_reason", lambda: "unsupported test GPU")
    with pytest.raises(RuntimeError, match="Cannot enable RDNA3 Flash Attention: unsupported test GPU"):
        comfyui.ApplyRDNA3FlashAttention().patch(FakeModel())
    monkeypatch.setattr(comfyui, "unsupported_reason", lambda: None)
    with pytest.raises(TypeError, match="optimized_attention_override must be callable"):
        comfyui.ApplyRDNA3FlashAttention().patch(FakeModel({"optimized_attention_override": object()}))


def test_node_registry():
    assert comfyui.NODE_CLASS_MAPPINGS == {"ApplyRDNA3FlashAttention": comfyui.ApplyRDNA3FlashAttention}
    assert comfyui.NODE_DISPLAY_NAME_MAPPINGS == {"ApplyRDNA3FlashAttention": "RDNA3 Flash Attention"}
    node = comfyui.ApplyRDNA3FlashAttention
    assert node.INPUT_TYPES() == {"required": {"model": ("MODEL",)}}
    assert (node.RETURN_TYPES, node.FUNCTION) == (("MODEL",), "patch")


def test_custom_node_entry_ignores_a_conflicting_top_level_package(tmp_path):
    stale = tmp_path / "fa_rdna3"
    stale.mkdir()
    (stale / "__init__.py").write_text("SOURCE = 'stale install'\n")
    script = f"""
import importlib.util, sys
spec = importlib.util.spec_from_file_location(
    "mi355x_custom_node", {os.path.join(PKG_DIR, "__init__.py")!r}, submodule_search_locations=[{PKG_DIR!r}])
module = importlib.util.module_from_spec(spec)
sys.modules["mi355x_custom_node"] = module
spec.loader.exec_module(module)
node = module.NODE_CLASS_MAPPINGS["ApplyRDNA3FlashAttention"]
assert node.__module__.startswith("mi355x_custom_node.fa_rdna3"), node.__module__
"""
    subprocess.run([sys.executable, "-c", script], cwd=tmp_path,
                   env={**os.environ, "PYTHONPATH": str(tmp_path)}, check=True, timeout=120)


@pytest.mark.gpu
def test_override_matches_sdpa_in_comfy_layout():
    torch.manual_seed(0)
    B, Sq, Sk, H, D = 2, 96, 137, 4, 64
    q = torch.randn(B, Sq, H * D, device="cuda", dtype=torch.float16)
    k = torch.randn(B, Sk, H * D, device="cuda", dtype=torch.float16)
    v = torch.randn_like(k)
    mask = torch.zeros(Sq, Sk, device="cuda")
    mask[:, -11:] = float("-inf")
    heads = lambda t: t.reshape(B, t.shape[1], H, D).transpose(1, 2)
    ref = F.scaled_dot_product_attention(heads(q), heads(k), heads(v), attn_mask=mask.unsqueeze(0))
    ref = ref.transpose(1, 2).reshape(B, Sq, H * D)
    out = comfyui.ComfyUIAttentionOverride()(_never, q, k, v, H, mask=mask)
    torch.testing.assert_close(out.float(), ref.float(), atol=3e-3, rtol=3e-3)


@pytest.mark.gpu
def test_override_matches_sdpa_in_head_layout_with_gqa():
    torch.manual_seed(1)
    q = torch.randn(1, 8, 128, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, 2, 192, 64, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    ref = F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
    out = comfyui.ComfyUIAttentionOverride()(_never, q, k, v, 8, skip_reshape=True, skip_output_reshape=True,
                                             enable_gqa=True)
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
def test_fallback_is_torch_sdpa_even_with_dispatch_enabled(monkeypatch):
    q = torch.randn(1, 2, 64, 32, device="cuda", dtype=torch.float16)
    k, v = torch.randn_like(q), torch.randn_like(q)
    ref = F.scaled_dot_product_attention(q, k, v)
    monkeypatch.setattr(sdpa, "flash_attention", _never)
    sdpa.enable_rdna3_flash_attention()
    try:
        out = comfyui.ComfyUIAttentionOverride()(
            lambda q_, k_, v_, h, **kw: F.scaled_dot_product_attention(q_, k_, v_), q, k, v, 2,
            skip_reshape=True, skip_output_reshape=True, low_precision_attention=False)
    finally:
        sdpa.disable_rdna3_flash_attention()
    torch.testing.assert_close(out, ref)
