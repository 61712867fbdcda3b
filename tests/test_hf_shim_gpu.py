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


@pytest.mark.parametrize("shape", [{}, dict(hidden=200, ffn=520, vocab=1000)],
                         ids=["aligned", "ragged"])
def test_trie_verification_equals_one_token_path_bitwise(shape):
    """shape "ragged": hidden 200, FFN 520 and vocabulary 1000, so every linear layer and
    RMSNorm runs the any-shape kernels."""
    from transformers.cache_utils import DynamicCache
    from respect_amd.candidates.trie import build_trie
    from respect_amd.decoding.hf_kv import FixedKVBuffer, compact
    from respect_amd.decoding.hf_verify import forward_tokens_hf, verify_trie_hf
    from respect_amd.kernels import dispatch, patch

    m = tiny_model(device="cuda", **shape)
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


def _logits_pair(seed=1):
    """Trie logits of one tiny Qwen3-VL through the patched kernels (GPU) and through the
    stock transformers kernels (SDPA with the same 4-D mask, nn.Linear, the stock RMSNorm;
    bf16 on the CPU, where SDPA's masked math path is safe), from identical prompt KV."""
    import copy
    from types import SimpleNamespace
    from transformers.cache_utils import DynamicCache
    from respect_amd.candidates.trie import build_trie
    from respect_amd.decoding.hf_kv import FixedKVBuffer
    from respect_amd.decoding.hf_verify import forward_tokens_hf, verify_trie_hf
    from respect_amd.kernels import patch
    m = tiny_model(device="cuda")
    cpu_model = copy.deepcopy(m).to("cpu")
    vocab = m.lm_head.weight.shape[0]
    g = torch.Generator().manual_seed(seed)
    P, CAP, base = 40, 64, 3
    prompt = torch.randint(0, vocab, (1, P), generator=g).cuda()
    pc = DynamicCache()
    with torch.no_grad():
        m(prompt, position_ids=torch.arange(P, device="cuda")[None], past_key_values=pc)
    pc_cpu = SimpleNamespace(layers=[SimpleNamespace(keys=l.keys.cpu(), values=l.values.cpu()) for l in pc.layers])
    gpu_buf, cpu_buf = FixedKVBuffer(P, (CAP,)), FixedKVBuffer(P, (CAP,))
    gpu_buf.allocate(pc)
    gpu_buf.write_prefill(pc)
    cpu_buf.allocate(pc_cpu)
    cpu_buf.write_prefill(pc_cpu)
    tree = build_trie([[5, 6, 7, 8], [5, 6, 9], [10, 11, 12, 13, 14], [10, 15]])
    committed = [11, 12, 13]
    patch.install(m, P)
    try:
        forward_tokens_hf(m, gpu_buf.window(CAP), committed, P, P, P, CAP)
        ours = verify_trie_hf(m, gpu_buf.window(CAP), tree, P, base, CAP).float().cpu()
    finally:
        patch.uninstall(m)
    forward_tokens_hf(cpu_model, cpu_buf.window(CAP), committed, P, P, P, CAP)
    stock = verify_trie_hf(cpu_model, cpu_buf.window(CAP), tree, P, base, CAP).float()
    return ours, stock, (cpu_model, cpu_buf, tree, P, CAP, base)


def test_patched_trie_logits_match_stock_transformers():
    """Oracle parity of the shim: the patched forward (row-invariant linear, norm and trie
    attention) against the unpatched transformers forward of the same model on the same
    trie: logits within 2 % of the largest |logit| (the stock path rounds its vocabulary
    scores and its attention to bf16; measured well inside).  The same comparison with a
    mask that hides one ancestor from every node moves the logits far outside."""
    ours, stock, (cpu_model, cpu_buf, tree, P, CAP, base) = _logits_pair()
    d = float((ours - stock).abs().max() / stock.abs().max())
    print(f"[hf shim] patched vs stock: max |diff| / max |logit| = {d:.4f}", flush=True)
    assert d <= 0.02
    # planted slip on the stock side: node 4's parent hidden (it sees only the root and itself)
    from respect_amd.decoding.hf_verify import verify_trie_hf
    import respect_amd.decoding.hf_verify as HV
    real = HV.trie_ancestry
    try:
        def hide_parents(t):
            a = real(t).copy()
            for i, n in enumerate(t.nodes):
                if n.parent is not None:
                    a[i, n.parent] = False
            return a
        HV.trie_ancestry = hide_parents
        slipped = verify_trie_hf(cpu_model, cpu_buf.window(CAP), tree, P, base, CAP).float()
    finally:
        HV.trie_ancestry = real
    assert float((slipped - stock).abs().max() / stock.abs().max()) > 5 * max(d, 0.01)


@pytest.mark.parametrize("q_len,n_node", [(1, 1), (5, 12), (64, 64), (7, 200)])
def test_unified_forward_causal_branch_matches_stock_sdpa(q_len, n_node):
    """dispatch.unified_forward without a 4-D mask (dispatch.py:110-114 of the reference):
    query i sits at node slot n_node - q_len + i and sees the whole prompt and node slots
    up to its own.  Against transformers' stock SDPA given that mask explicitly (bf16 on the
    GPU): within 2^-7 of the largest |output|; against the kernel-tree restatement: within
    2 bf16 ulp per element (ulp at max(|x|, max|row| / 64))."""
    import numpy as np
    from oracle import attention as A, bf16
    from respect_amd.kernels import dispatch
    H, HK, D, PL = 8, 2, 128, 96
    g = torch.Generator().manual_seed(q_len * 1000 + n_node)
    q = torch.randn(1, H, q_len, D, generator=g).to(torch.bfloat16).cuda()
    k = (torch.randn(1, HK, PL + n_node, D, generator=g) / 4).to(torch.bfloat16).cuda()
    v = torch.randn(1, HK, PL + n_node, D, generator=g).to(torch.bfloat16).cuda()
    print(f"[dispatch causal] q_len={q_len} n_node={n_node}", flush=True)
    dispatch.install(PL)
    try:
        k0, f0 = dispatch.STATS["kernel"], dispatch.STATS["fallback"]
        y, w = dispatch.unified_forward(None, q, k, v, None)
        torch.cuda.synchronize()
        assert w is None and dispatch.STATS["kernel"] == k0 + 1 and dispatch.STATS["fallback"] == f0
    finally:
        dispatch.uninstall()
    assert y.shape == (1, q_len, H, D)
    rows = torch.arange(q_len, device="cuda")[:, None] + (n_node - q_len)
    allow = torch.ones(q_len, PL + n_node, dtype=torch.bool, device="cuda")
    allow[:, PL:] = torch.arange(n_node, device="cuda")[None, :] <= rows
    # stock SDPA on the CPU (its masked bf16 math path is safe there), same bf16 inputs
    mod = type("M", (), {"num_key_value_groups": H // HK, "is_causal": False, "training": False})()
    ref, _ = dispatch.ORIG(mod, q.cpu(), k.cpu(), v.cpu(), allow[None, None].cpu(), 0.0, None, False)
    d = float((y.float().cpu() - ref.float()).abs().max() / ref.float().abs().max())
    assert d <= 2 ** -7, d
    qn = q[0].float().cpu().numpy()
    kn = k[0].float().cpu().numpy()
    vn = v[0].float().cpu().numpy()
    msk = allow[:, PL:].cpu().numpy()
    t = A.attn_tree_c(qn, kn[:, :PL], vn[:, :PL], kn[:, PL:], vn[:, PL:], msk, D ** -0.5)
    o = y[0].transpose(0, 1).float().cpu().numpy()
    mag = np.maximum(np.abs(o), np.abs(t))
    ud = np.abs(o.astype(np.float64) - t) / bf16.ulp(np.maximum(mag, mag.max(axis=-1, keepdims=True) / 64))
    assert ud.max() <= 2, ud.max()
