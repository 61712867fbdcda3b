"""GPU test of the Hugging Face integration shim on a tiny random Qwen3-VL text
decoder: with the kernels installed, every trie node's logits from one
verification forward equal bitwise those of the 1-token path that feeds the
node's root path one token at a time (the reference's output-preservation
property, respect/decoding/verify.py + sequential.py), and compact() leaves the
accepted path's KV bitwise equal to the 1-token path's."""
import numpy as np
import pytest
import torch

pytest.importorskip("transformers.models.qwen3_vl")

from tests._hf_tiny import tiny_model

pytestmark = pytest.mark.gpu


def _path(tree, i):
    p = []
    while i is not None:
        p.append(i)
        i = tree.nodes[i].parent
    return p[::-1]


def test_trie_verification_equals_one_token_path_bitwise():
    from transformers.cache_utils import DynamicCache
    from respect_amd.candidates.trie import build_trie
    from respect_amd.decoding.hf_kv import FixedKVBuffer, compact
    from respect_amd.decoding.hf_verify import forward_tokens_hf, verify_trie_hf
    from respect_amd.kernels import dispatch, patch

    m = tiny_model(device="cuda")
    cfg_vocab = m.lm_head.weight.shape[0]
    g = torch.Generator().manual_seed(1)
    P, CAP, base = 40, 64, 3
    prompt = torch.randint(0, cfg_vocab, (1, P), generator=g).cuda()
    pc = DynamicCache()
    with torch.no_grad():                       # Prefill on the stock kernels, as the reference does
        m(prompt, position_ids=torch.arange(P, device="cuda")[None], past_key_values=pc)
    bufs = [FixedKVBuffer(P, (CAP,)) for _ in range(2)]
    for b in bufs:
        b.allocate(pc)
        b.write_prefill(pc)
    committed = [11, 12, 13]
    tree = build_trie([[5, 6, 7, 8], [5, 6, 9], [10, 11, 12, 13, 14], [10, 15]])
    print(f"[hf shim] P={P} base={base} nodes={len(tree.nodes)}", flush=True)

    patch.install(m, P)
    try:
        k0, f0 = dispatch.STATS["kernel"], dispatch.STATS["fallback"]
        for b in bufs:                           # the same committed tokens in both buffers
            forward_tokens_hf(m, b.window(CAP), committed, P, P, P, CAP)
        trie_logits = verify_trie_hf(m, bufs[0].window(CAP), tree, P, base, CAP)
        assert dispatch.STATS["fallback"] == f0 and dispatch.STATS["kernel"] > k0
        assert trie_logits.dtype == torch.float32
        for i in range(len(tree.nodes)):
            path = _path(tree, i)
            ref = bufs[1].window(CAP)
            seq = forward_tokens_hf(m, ref, [tree.nodes[j].token for j in path], P + base, P + base, P, CAP)
            assert torch.equal(seq[-1], trie_logits[i]), f"node {i}"
        # accept the path of node 4 (tokens 5, 6, 9): its KV moves to consecutive slots
        acc = _path(tree, 4)
        compact(bufs[0].window(CAP), P, base, acc)
        forward_tokens_hf(m, bufs[1].window(CAP), [tree.nodes[j].token for j in acc], P + base, P + base, P, CAP)
        n = P + base + len(acc)
        for kb, kr in zip(bufs[0].base_k + bufs[0].base_v, bufs[1].base_k + bufs[1].base_v):
            assert torch.equal(kb[:, :, :n], kr[:, :, :n])
    finally:
        patch.uninstall(m)
