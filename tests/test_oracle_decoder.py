"""CPU pinning of the decoder oracle (oracle/decoder.py) on a tiny one-layer model:
the batched forward equals its own token-by-token forward through the KV dict
(slots, positions and the allow mask are wired consistently); the cache slot
layout does not matter; with one visible key the attention output is that
key's value, so q/k weights cannot change the logits."""
from types import SimpleNamespace

import numpy as np
import torch

from oracle.decoder import RefDecoder


def _model(seed=0, layers=1):
    g = torch.Generator().manual_seed(seed)
    cfg = SimpleNamespace(layers=layers, hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=256, vocab=64,
                          eps=1e-6, theta=1.0e6)
    r = lambda *s, std=0.05: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    n = lambda k: (1 + 0.02 * torch.randn(k, generator=g)).to(torch.bfloat16)
    qkv = (cfg.heads + 2 * cfg.kv_heads) * cfg.head_dim
    lay = [SimpleNamespace(in_norm=n(256), wqkv=r(qkv, 256), q_norm=n(64), k_norm=n(64), wo=r(256, 256),
                           post_norm=n(256), wgu=r(512, 256), wd=r(256, 256)) for _ in range(layers)]
    return SimpleNamespace(cfg=cfg, embed=r(64, 256, std=1.0), layers=lay, final_norm=n(256), lm_head=r(64, 256))


def test_batched_forward_equals_token_by_token():
    ref = RefDecoder(_model(layers=2))
    ids, T, S = [3, 17, 42, 8], 4, 8
    allow = torch.tril(torch.ones(T, S, dtype=torch.bool), diagonal=0)
    allow[:, T:] = False
    full, _ = ref.forward(ids, list(range(T)), list(range(100, 100 + T)), allow)
    kv = None
    for t in range(T):
        a = torch.zeros(1, S, dtype=torch.bool)
        a[0, :t + 1] = True
        one, kv = ref.forward([ids[t]], [t], [100 + t], a, kv)
        assert torch.allclose(one[0], full[t], rtol=0, atol=1e-5), t


def test_slot_layout_does_not_matter():
    ref = RefDecoder(_model(seed=1))
    ids, S = [5, 9, 11], 12
    a = torch.zeros(3, S, dtype=torch.bool)
    b = torch.zeros(3, S, dtype=torch.bool)
    sa, sb = [0, 1, 2], [7, 2, 10]
    for t in range(3):
        a[t, sa[:t + 1]] = True
        b[t, sb[:t + 1]] = True
    la, _ = ref.forward(ids, sa, [50, 51, 52], a)
    lb, _ = ref.forward(ids, sb, [50, 51, 52], b)
    assert torch.allclose(la, lb, rtol=0, atol=1e-5)


def test_single_visible_key_ignores_q_and_k_weights():
    m = _model(seed=2)
    ref = RefDecoder(m)
    a = torch.ones(1, 1, dtype=torch.bool)
    base, _ = ref.forward([7], [0], [3], a)
    H, D = 4, 64
    ref.layers[0]["wqkv"][:(H + 2) * D] = torch.randn((H + 2) * D, 256)   # q and k rows only
    other, _ = ref.forward([7], [0], [3], a)
    assert torch.equal(base, other)
    ref.layers[0]["wqkv"][(H + 2) * D:] *= 2                             # v rows do matter
    assert not torch.equal(base, ref.forward([7], [0], [3], a)[0])


# ---------------------------------------------------------------- against transformers' Qwen3-VL text decoder

def _from_hf(m):
    """RefDecoder's view of a transformers Qwen3-VL text model: [q | k | v] and
    [gate | up] weight rows stacked as the GPU decoder stores them."""
    lm, c = m.model, m.model.config
    layers = []
    for l in lm.layers:
        a, f = l.self_attn, l.mlp
        layers.append(SimpleNamespace(
            in_norm=l.input_layernorm.weight,
            wqkv=torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight]),
            q_norm=a.q_norm.weight, k_norm=a.k_norm.weight, wo=a.o_proj.weight,
            post_norm=l.post_attention_layernorm.weight,
            wgu=torch.cat([f.gate_proj.weight, f.up_proj.weight]), wd=f.down_proj.weight))
    cfg = SimpleNamespace(layers=len(layers), hidden=c.hidden_size, heads=c.num_attention_heads,
                          kv_heads=c.num_key_value_heads, head_dim=c.head_dim, ffn=c.intermediate_size,
                          vocab=c.vocab_size, eps=c.rms_norm_eps, theta=1.0e6)
    return SimpleNamespace(cfg=cfg, embed=lm.embed_tokens.weight, layers=layers, final_norm=lm.norm.weight,
                           lm_head=m.lm_head.weight)


def test_matches_transformers_qwen3_vl_and_slips_fail():
    """The oracle decoder against transformers' own Qwen3-VL text decoder (bf16 on the CPU,
    same weights, causal attention, rotary positions 7..7+T, the same in all M-RoPE axes):
    logits within 3 % of the largest |logit| (measured: 1.0 %; the difference is
    transformers' bf16 attention and bf16 logits against the oracle's float64 softmax and
    fp32 logits).  Planted slips -- RoPE sign, k/v rows swapped, gate/up swapped, q/k norm
    weights dropped, input/post norms swapped, a row not seeing its own slot -- each move
    the logits by 25 % or more."""
    import pytest
    pytest.importorskip("transformers.models.qwen3_vl")
    from tests._hf_tiny import tiny_model
    m = tiny_model(seed=0)
    with torch.no_grad():                  # norm weights 1 + N(0, 0.3): norm slips show
        for name, p in m.named_parameters():
            if p.dim() == 1:
                g = torch.Generator().manual_seed(len(name))
                p.copy_((1 + 0.3 * torch.randn(p.shape, generator=g)).to(p.dtype))
    T = 24
    ids = torch.randint(0, 1024, (1, T), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        hf = m(ids, position_ids=torch.arange(7, 7 + T)[None]).logits[0].float()
    allow = torch.tril(torch.ones(T, T, dtype=torch.bool))
    pos = list(range(7, 7 + T))

    def dist(view, positions=pos, mask=allow):
        out, _ = RefDecoder(view).forward(ids[0].tolist(), list(range(T)), positions, mask)
        return float((hf - out).abs().max() / hf.abs().max())

    assert dist(_from_hf(m)) <= 0.03
    H, HK, D = 4, 2, 64

    def planted(fn):
        v = _from_hf(m)
        for l in v.layers:
            fn(l)
        return v

    def swap_kv(l):
        q, k = H * D, HK * D
        l.wqkv = torch.cat([l.wqkv[:q], l.wqkv[q + k:], l.wqkv[q:q + k]])

    def swap_gu(l):
        F = l.wgu.shape[0] // 2
        l.wgu = torch.cat([l.wgu[F:], l.wgu[:F]])

    def drop_qk_norm(l):
        l.q_norm, l.k_norm = torch.ones_like(l.q_norm), torch.ones_like(l.k_norm)

    def swap_norms(l):
        l.in_norm, l.post_norm = l.post_norm, l.in_norm

    own_missing = torch.tril(torch.ones(T, T, dtype=torch.bool), diagonal=-1)
    own_missing[0, 0] = True
    slips = {"rope sign": dist(_from_hf(m), positions=[-p for p in pos]),
             "k/v swapped": dist(planted(swap_kv)), "gate/up swapped": dist(planted(swap_gu)),
             "q/k norm dropped": dist(planted(drop_qk_norm)), "norms swapped": dist(planted(swap_norms)),
             "own slot masked": dist(_from_hf(m), mask=own_missing)}
    for name, d in slips.items():
        assert d > 0.2, (name, d)
