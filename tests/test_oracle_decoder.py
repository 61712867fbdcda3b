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
