"""CPU tests of the Hugging Face integration shim: what install wraps, that
uninstall restores it, the SDPA routing, the shape checks (no kernel runs)."""
import pytest
import torch

pytest.importorskip("transformers.models.qwen3_vl")

from tests._hf_tiny import tiny_model


def test_install_wraps_every_linear_and_norm_and_uninstall_restores():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from respect_amd.kernels import dispatch, patch
    m = tiny_model()
    before = {n: type(mod) for n, mod in m.named_modules()}
    n = patch.install(m, prompt_len=40)
    try:
        # 2 layers x (7 linears + 4 norms) + the final norm + lm_head
        assert n == 2 * 11 + 2
        assert patch.is_installed()
        assert isinstance(m.lm_head, patch.FixedLinear) and m.lm_head.out_dtype == "lm"
        assert isinstance(m.model.layers[0].self_attn.q_norm, patch.FixedNorm)
        assert isinstance(m.model.norm, patch.FixedNorm)
        assert dispatch.STATE["PL"] == 40
        assert ALL_ATTENTION_FUNCTIONS["sdpa"] is dispatch.unified_forward
        assert patch.install(m, 40) == n          # wrapping twice wraps nothing new
    finally:
        patch.uninstall(m)
    assert not patch.is_installed()
    assert {n: type(mod) for n, mod in m.named_modules()} == before
    assert dispatch.STATE["PL"] is None
    assert ALL_ATTENTION_FUNCTIONS["sdpa"] is dispatch.ORIG


def test_install_refuses_unsupported_weights():
    from respect_amd.kernels import patch
    m = tiny_model(hidden=192, ffn=512, heads=3, kv_heads=1)   # ragged shapes are built (any N, K)
    m.model.layers[0].self_attn.q_proj.float()                  # an fp32 weight is not
    before = {n: type(mod) for n, mod in m.named_modules()}
    with pytest.raises(ValueError, match="layers.0.self_attn.q_proj"):
        patch.install(m, 8)
    assert not patch.is_installed()
    assert {n: type(mod) for n, mod in m.named_modules()} == before


def test_dispatch_falls_back_without_prompt_length():
    from respect_amd.kernels import dispatch
    calls = []
    orig = dispatch.ORIG
    dispatch.ORIG = lambda *a, **k: calls.append(1) or ("orig", None)
    try:
        dispatch.STATE["PL"] = None
        q = torch.zeros(1, 4, 3, 64)
        assert dispatch.unified_forward(None, q, q, q, None)[0] == "orig"
        dispatch.STATE["PL"] = 2
        b2 = torch.zeros(2, 4, 3, 64)                             # batch 2
        assert dispatch.unified_forward(None, b2, b2, b2, None)[0] == "orig"
        assert dispatch.unified_forward(None, q, q, q, None, dropout=0.1)[0] == "orig"
        assert len(calls) == 3 and dispatch.STATS["fallback"] >= 3
    finally:
        dispatch.ORIG = orig
        dispatch.STATE["PL"] = None
