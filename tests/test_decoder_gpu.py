"""The verification step on a small random decoder, end to end on the GPU.

Bar (the reference's output-preservation check, summary.json "tokens and
committed KV equal"): tokens accepted by trie verification, and the KV they
leave in the cache, are bitwise identical to token-by-token greedy decoding
with the same kernels; the verified logits of every accepted node equal the
1-token logits bit for bit.  A CPU float64/fp32 reference decoder
(oracle/decoder.py) checks the wiring of the forward within a loose bound.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CFG = dict(layers=2, hidden=512, heads=4, kv_heads=2, head_dim=128, ffn=1024, vocab=4096)
P = 100


@pytest.fixture(scope="module")
def model():
    from respect_amd.decoding.engine import Decoder, DecoderConfig
    return Decoder(DecoderConfig(**CFG), seed=1, std=0.05)


def _prompt(seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, CFG["vocab"], (P,), generator=g)


def _filled_cache(model, chunk=64):
    from respect_amd.decoding.kv_buffer import KVCache
    c = model.cfg
    cache = KVCache(c.layers, c.kv_heads, c.head_dim, P + 256)
    last = model.prefill(_prompt().cuda(), cache, chunk=chunk)
    return cache, last


def _trie(seq, rng, n_other=3, vocab=4096, length=24):
    from respect_amd.candidates.trie import build_trie
    seqs = [list(seq[:length])]
    for _ in range(n_other):
        p = int(rng.integers(1, min(17, length)))
        seqs.append(list(seq[:p]) + [int(t) for t in rng.integers(0, vocab, length - p)])
    return build_trie(seqs)


def test_prefill_is_deterministic(model):
    """Same chunking twice: the same bits.  A different chunking changes which
    keys a row sees as prompt (grouped tree) and which as nodes (slot-order
    fold), so only layer 0's K/V -- computed before any attention -- must
    agree across chunkings."""
    a, la = _filled_cache(model, chunk=64)
    b, lb = _filled_cache(model, chunk=64)
    c, _ = _filled_cache(model, chunk=100)
    for li in range(model.cfg.layers):
        assert torch.equal(a.k[li][:, :P], b.k[li][:, :P]) and torch.equal(a.v[li][:, :P], b.v[li][:, :P])
    assert torch.equal(la, lb)
    assert torch.equal(a.k[0][:, :P], c.k[0][:, :P]) and torch.equal(a.v[0][:, :P], c.v[0][:, :P])


def test_forward_wiring_matches_cpu_reference(model):
    from oracle.decoder import RefDecoder
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.sequential import forward_token
    cache, last = _filled_cache(model)
    ref = RefDecoder(model)
    ids = _prompt()
    S = P + 8
    allow = torch.tril(torch.ones(P, S, dtype=torch.bool))
    rl, kv = ref.forward(ids.tolist(), list(range(P)), list(range(P)), allow)
    got = last.cpu()
    assert (got - rl[-1:]).abs().max() <= 0.05 * rl.abs().max()
    tok = int(greedy_token(last).item())
    lg = forward_token(model, cache, tok, P, 0).cpu()
    allow1 = torch.zeros(1, S, dtype=torch.bool)
    allow1[0, :P + 1] = True
    r1, _ = ref.forward([tok], [P], [P], allow1, kv)
    assert (lg - r1).abs().max() <= 0.05 * r1.abs().max()


def test_trie_verification_equals_token_by_token(model):
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.respect import respect_step
    from respect_amd.decoding.sequential import forward_token
    from respect_amd.decoding.verify import verify_trie
    # token-by-token reference: 60 greedy tokens, their logits and KV
    ar, last = _filled_cache(model)
    t0 = int(greedy_token(last).item())
    G, logits_ar = [t0], []
    for c in range(60):
        lg = forward_token(model, ar, G[-1], P, c)
        logits_ar.append(lg)
        G.append(int(greedy_token(lg).item()))
    # trie verification from the same prompt KV
    sp, _ = _filled_cache(model)
    rng = np.random.default_rng(0)
    base, first = 0, t0
    for step, length in enumerate((24, 24, 4)):
        if length == 24:
            tree = _trie(G[base:], rng)
        else:  # the target's path leaves the trie after 4 tokens
            from respect_amd.candidates.trie import build_trie
            tree = build_trie([G[base:base + 4] + [(G[base + 4] + 1) % 4096] * 4,
                               G[base:base + 2] + [7, 7, 7, 7, 7, 7]])
        logits = verify_trie(model, sp, tree, P, base)
        acc, rec, path = respect_step(model, sp, tree, first, P, base, eos=-1)
        print(f"[respect] step {step}: base {base}, {len(tree.nodes)} nodes, accepted {len(acc)}", flush=True)
        assert acc == G[base:base + length] and rec == G[base + length]
        for j, node in enumerate(path):  # verified logits == 1-token logits, bitwise
            assert torch.equal(logits[node:node + 1], logits_ar[base + j])
        for li in range(model.cfg.layers):  # committed KV == token-by-token KV, bitwise
            s0, s1 = P + base, P + base + length
            assert torch.equal(sp.k[li][:, s0:s1], ar.k[li][:, s0:s1])
            assert torch.equal(sp.v[li][:, s0:s1], ar.v[li][:, s0:s1])
        base += length
        first = rec


def test_greedy_token_rules():
    from respect_amd.decoding.acceptance import greedy_token
    lg = torch.tensor([[0.0, 5.0, 5.0, 1.0], [9.0, 1.0, 2.0, 2.0], [1.0, float("nan"), 3.0, float("nan")]],
                      device="cuda")
    assert greedy_token(lg).tolist() == [1, 0, 1]
    assert greedy_token(lg, 0, 1).tolist() == [1, 2, 1]
    assert greedy_token(lg[:2], 1, 2).tolist() == [3, 0]
    big = torch.randn(3, 151936, device="cuda")
    big[1, 100000] = 1e9
    big[2, 7] = big[2, 150000] = 1e9
    assert greedy_token(big).tolist() == [int(big[0].argmax()), 100000, 7]
    # action-vocabulary range excluded (acceptance.py:11-17)
    assert greedy_token(big, 100000, 50001).tolist()[1:] == [int(torch.cat([big[1, :100000], big[1, 150001:]]).argmax()), 7]


def test_trie_mask_from_parents():
    from respect_amd.candidates.trie import build_trie, node_mask
    from respect_amd.decoding.verify import trie_mask
    tree = build_trie([(1, 2, 3, 4), (1, 2, 5), (6, 7), (1, 8, 9, 10, 11)])
    for base in (0, 5, 37):
        NN = max(32, -(-(base + len(tree.nodes)) // 32) * 32)
        msk, depth = trie_mask(tree, base, NN, "cuda")
        assert np.array_equal(msk.cpu().numpy().astype(bool), node_mask(tree, base, NN))
        assert depth.cpu().tolist() == tree.depths.tolist()


def test_step_inputs_from_device_descriptor():
    """rspx_step_inputs: node rows get their token, slot P + base + i, position
    P + base + depth and rspx_trie_mask's mask row; padding rows token 0, slot
    pad0 + i, position 0, slot 0 only; a descriptor that does not fit counts as
    an empty trie; out-of-range tokens become 0."""
    from respect_amd import _lib
    from respect_amd.candidates.trie import build_trie, node_mask
    L = _lib.lib()
    tree = build_trie([(1, 2, 3, 4), (1, 2, 5), (6, 7), (1, 8, 9, 10, 11)])
    n, T, P, pad0, vocab = len(tree.nodes), 16, 1000, 5000, 100
    s = _lib.stream_ptr(torch.device("cuda"))
    for base, NN in ((0, 32), (5, 32), (37, 64), (60, 64)):
        desc = np.zeros(2 + 2 * T, np.int32)
        desc[0], desc[1] = n, base
        desc[2:2 + n] = tree.tokens
        desc[2 + T:2 + T + n] = tree.parents
        desc[2 + 3] = 999            # out of the vocabulary: token 0
        d = torch.from_numpy(desc).cuda()
        ids, slots, pos = (torch.full((T,), -7, dtype=torch.int32, device="cuda") for _ in range(3))
        msk = torch.full((T, NN), 9, dtype=torch.uint8, device="cuda")
        _lib.check("rspx_step_inputs", L.rspx_step_inputs(d.data_ptr(), T, P, NN, pad0, vocab, ids.data_ptr(),
                                                          slots.data_ptr(), pos.data_ptr(), msk.data_ptr(), NN, s))
        torch.cuda.synchronize()
        fits = base + n <= NN
        print(f"[step_inputs] base {base} NN {NN} fits {fits}", flush=True)
        m = msk.cpu().numpy().astype(bool)
        if fits:
            exp_tok = tree.tokens.astype(np.int64).copy()
            exp_tok[3] = 0
            assert ids.cpu().tolist() == exp_tok.tolist() + [0] * (T - n)
            assert slots.cpu().tolist() == [P + base + i for i in range(n)] + [pad0 + i for i in range(n, T)]
            assert pos.cpu().tolist() == [P + base + int(x) for x in tree.depths] + [0] * (T - n)
            assert np.array_equal(m[:n], node_mask(tree, base, NN))
            pad_rows = m[n:]
        else:
            assert ids.cpu().tolist() == [0] * T and pos.cpu().tolist() == [0] * T
            assert slots.cpu().tolist() == [pad0 + i for i in range(T)]
            pad_rows = m
        assert pad_rows[:, 0].all() and not pad_rows[:, 1:].any()


def test_kv_compact_overlapping_moves():
    from respect_amd.decoding.kv_buffer import KVCache
    c = KVCache(3, 2, 128, 64)
    for t in c.k + c.v:
        t.copy_(torch.randn_like(t, dtype=torch.float32).to(torch.bfloat16))
    before = [t.clone() for t in c.k + c.v]
    path = [0, 2, 3, 7, 8]          # destination of one is the source of the next
    c.compact(10, path)
    for t, b in zip(c.k + c.v, before):
        exp = b.clone()
        exp[:, 10:15] = b[:, [10 + s for s in path]]
        assert torch.equal(t, exp)


def test_graph_replays_equal_eager(model):
    """Captured forwards (HIP graphs) give the eager bits on every replay, with
    eager work and synchronisations between replays, for tries of different
    sizes and offsets and for 1-token calls; the greedy choices taken inside
    the graphs equal greedy_token on the eager logits."""
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.sequential import forward_token, next_token
    from respect_amd.decoding.verify import verify_trie, verify_trie_greedy
    cache, last = _filled_cache(model)
    t0 = int(greedy_token(last).item())
    rng = np.random.default_rng(1)
    for rep, base in enumerate((0, 5, 40, 5)):
        seq = [t0] + [int(t) for t in rng.integers(0, 4096, 30)]
        tree = _trie(seq, rng) if rep % 2 == 0 else _trie(seq, rng, n_other=1, length=10)
        eager = verify_trie(model, cache, tree, P, base).clone()
        torch.cuda.synchronize()
        graphed = verify_trie(model, cache, tree, P, base, graph=True).clone()
        torch.cuda.synchronize()
        print(f"[graph] rep {rep} base {base} nodes {len(tree.nodes)}", flush=True)
        assert torch.equal(eager, graphed)
        assert verify_trie_greedy(model, cache, tree, P, base) == greedy_token(eager).tolist()
        e1 = forward_token(model, cache, seq[1], P, base).clone()
        g1 = forward_token(model, cache, seq[1], P, base, graph=True).clone()
        assert torch.equal(e1, g1)
        assert next_token(model, cache, seq[1], P, base) == int(greedy_token(e1).item())


def test_graphs_are_tied_to_their_cache(model):
    """A captured forward holds its cache's device pointers: dropping the cache drops its
    graphs, and a new cache (which may get the old one's id) captures its own."""
    import gc
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.sequential import forward_token
    model.release_graphs()
    cache, last = _filled_cache(model)
    t0 = int(greedy_token(last).item())
    g1 = model.graphed(cache, P, 1, 64)
    assert len(model._graphs) == 1 and model.graphed(cache, P, 1, 64) is g1
    del cache, last, g1
    gc.collect()
    assert len(model._graphs) == 0
    cache2, last2 = _filled_cache(model)
    eager = forward_token(model, cache2, t0, P, 0).clone()
    graphed = forward_token(model, cache2, t0, P, 0, graph=True).clone()
    assert torch.equal(eager, graphed)
    assert len(model._graphs) == 1 and model._graphs.get(cache2) is not None


def test_capacity_is_enforced(model):
    """Slots past the cache's capacity are refused on the host (eager paths) before any
    kernel is queued."""
    from respect_amd.decoding.sequential import forward_token
    cache, _ = _filled_cache(model)
    with pytest.raises(ValueError):
        forward_token(model, cache, 1, P, cache.cap - P)
    with pytest.raises(ValueError):
        model.prefill(torch.zeros(cache.cap + 1, dtype=torch.int64, device="cuda"), cache)


@pytest.mark.parametrize("graph", [False, True])
def test_attention_wait_that_gives_up_fails_the_step(model, graph):
    """An attention wait that gives up (0 polls through the test hook, so every kernel
    still exits normally) makes the verification step raise AttentionWaitError at the
    device-to-host copy it already makes, before the walk: no token is returned and the
    cache is not compacted.  The flag is cleared, and the next step on the same cache
    gives the clean step's tokens and KV bit for bit."""
    from respect_amd import _lib
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.respect import respect_step
    from respect_amd.kernels.attention import AttentionWaitError, status_word
    L = _lib.lib()
    ref_cache, last = _filled_cache(model)
    t0 = int(greedy_token(last).item())
    rng = np.random.default_rng(3)
    tree = _trie([t0] + [int(t) for t in rng.integers(0, 4096, 30)], rng)
    want = respect_step(model, ref_cache, tree, t0, P, 0, eos=-1, graph=graph)
    model.release_graphs()
    cache, _ = _filled_cache(model)
    compacted = []
    real_compact = cache.compact
    cache.compact = lambda *a: compacted.append(a)
    prev = L.rspx_trie_attn_set_spin_limit(0)
    print(f"[give-up step] graph={graph} nodes={len(tree.nodes)}", flush=True)
    try:
        with pytest.raises(AttentionWaitError):
            respect_step(model, cache, tree, t0, P, 0, eos=-1, graph=graph)
    finally:
        L.rspx_trie_attn_set_spin_limit(prev)
        cache.compact = real_compact
    assert compacted == []
    assert int(status_word(model.attn_ws_used).item()) == 0
    model.release_graphs()          # a graph captured under the lowered limit keeps it
    got = respect_step(model, cache, tree, t0, P, 0, eos=-1, graph=graph)
    assert got == want
    for li in range(model.cfg.layers):
        s1 = P + len(want[0])
        assert torch.equal(cache.k[li][:, :s1], ref_cache.k[li][:, :s1])
        assert torch.equal(cache.v[li][:, :s1], ref_cache.v[li][:, :s1])
    model.release_graphs()
