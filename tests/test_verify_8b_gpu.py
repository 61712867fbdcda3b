"""The full-size verification step (the 36-layer 8B-shape decoder: hidden 4096, 32 q /
8 kv heads, head_dim 128, FFN 12288 SwiGLU, vocabulary 151936, bf16 weights ~ N(0, 0.02),
random-initialised; a 3072-token prompt KV from random ids), end to end on the GPU.

Bar (the reference's output-preservation check, examples/decode.py:97-104 and
results/paper/summary.json "tokens and committed KV equal"): over several verification
steps -- 64-node tries of 4 candidates x 24 tokens, one candidate being the target's own
greedy continuation, then a trie of distractors only -- the accepted tokens, the
correction token and the KV they leave in all 36 layers are bitwise those of token-by-
token greedy decoding with the same kernels, and every accepted node's verified logits
equal its 1-token logits bit for bit.  Both paths run as captured HIP graphs (the
benchmark's configuration) and, for the logits, eagerly.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

P = 3072
STEPS = 3          # continuation tries, then one distractor-only trie


@pytest.fixture(scope="module")
def setup():
    from respect_amd.decoding.engine import Decoder, DecoderConfig
    from respect_amd.decoding.kv_buffer import KVCache
    from respect_amd.decoding.verify import node_slots
    cfg = DecoderConfig()
    print("[8b] random-initialising the 36-layer model", flush=True)
    model = Decoder(cfg, seed=0, std=0.02)
    prompt = torch.randint(0, cfg.vocab, (P,), generator=torch.Generator().manual_seed(0)).cuda()
    cap = P + node_slots(24 * (STEPS + 2), 64, 64) + 64
    caches, last = [], None
    for _ in range(2):
        c = KVCache(cfg.layers, cfg.kv_heads, cfg.head_dim, cap)
        last = model.prefill(prompt, c, chunk=512)
        caches.append(c)
    torch.cuda.synchronize()
    print("[8b] prompt KV built", flush=True)
    yield model, caches[0], caches[1], last
    model.release_graphs()


def _continuation_trie(cont, rng, vocab):
    from respect_amd.candidates.trie import build_trie
    for _ in range(10000):
        seqs = [list(cont[:24])]
        for _ in range(3):
            p = int(rng.integers(1, 17))
            seqs.append(list(cont[:p]) + [int(t) for t in rng.integers(0, vocab, 24 - p)])
        tree = build_trie(seqs)
        if len(tree.nodes) == 64:
            return tree
    return tree


def _distractor_trie(first, target_next, rng, vocab):
    """64 nodes under the root ``first`` whose children never carry the target's next token."""
    from respect_amd.candidates.trie import build_trie
    seqs = []
    while True:
        seqs.append([first] + [int(t) for t in rng.integers(0, vocab, 20)])
        seqs[-1][1] = seqs[-1][1] if seqs[-1][1] != target_next else (target_next + 1) % vocab
        tree = build_trie(seqs)
        if len(tree.nodes) >= 64:
            return build_trie(seqs[:-1] + [seqs[-1][:64 - len(build_trie(seqs[:-1]).nodes) + 1]])


def test_verify_steps_equal_one_token_decoding(setup):
    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.respect import respect_step
    from respect_amd.decoding.sequential import forward_token, next_token
    from respect_amd.decoding.verify import verify_trie
    model, ar, sp, last = setup
    vocab = model.cfg.vocab
    first = int(greedy_token(last).item())
    n_ar = 24 * STEPS + 2
    G = [first]
    for c in range(n_ar):                      # token-by-token reference (captured 1-token forwards)
        G.append(next_token(model, ar, G[-1], P, c))
    print(f"[8b] {n_ar} reference tokens decoded", flush=True)
    rng = np.random.default_rng(0)
    base, nxt = 0, first
    for step in range(STEPS + 1):
        distractor = step == STEPS
        tree = _distractor_trie(nxt, G[base + 1], rng, vocab) if distractor else _continuation_trie(G[base:], rng, vocab)
        assert len(tree.nodes) == 64
        if step == 1:                          # eager verification logits of this trie, before it is compacted
            logits = verify_trie(model, sp, tree, P, base).clone()
        acc, rec, path = respect_step(model, sp, tree, nxt, P, base, eos=-1, graph=True)
        print(f"[8b] step {step}: base {base}, accepted {len(acc)}{' (distractors)' if distractor else ''}",
              flush=True)
        assert acc == G[base:base + len(acc)] and rec == G[base + len(acc)], f"step {step}"
        assert len(acc) == (1 if distractor else 24)
        if step == 1:                          # verified logits of the accepted nodes == 1-token logits
            for j, node in enumerate(path):
                one = forward_token(model, ar, G[base + j], P, base + j).clone()
                assert torch.equal(logits[node:node + 1], one), f"node {node}"
        base += len(acc)
        nxt = rec
    for li in range(model.cfg.layers):
        assert torch.equal(sp.k[li][:, P:P + base], ar.k[li][:, P:P + base]), f"K layer {li}"
        assert torch.equal(sp.v[li][:, P:P + base], ar.v[li][:, P:P + base]), f"V layer {li}"
