"""Seeded synthetic workloads of the benchmark (GPU tensors, no files, no network).

Shapes follow the 8B decoder of the verification step: 32 query heads, 8 kv
heads, head_dim 128, prompt KV of 3072 tokens, tries merged from candidate
sequences that share random-length prefixes.
"""
from __future__ import annotations

import numpy as np
import torch

from .candidates.trie import Trie, build_trie, node_mask

VOCAB = 151936


def merged_trie(seed: int, n_seqs: int, length: int, pre_lo: int, pre_hi: int,
                target_nodes: int | None = None, vocab: int = VOCAB) -> Trie:
    """Sequence i copies a prefix (length uniform in [pre_lo, pre_hi]) of a random earlier
    sequence; redrawn until the merged trie has ``target_nodes`` nodes."""
    rng = np.random.default_rng(seed)
    for _ in range(10000):
        seqs = [rng.integers(0, vocab, length)]
        for i in range(1, n_seqs):
            src = seqs[int(rng.integers(0, i))]
            s = int(rng.integers(pre_lo, pre_hi + 1))
            new = rng.integers(0, vocab, length)
            new[:s] = src[:s]
            seqs.append(new)
        tree = build_trie(seqs)
        if target_nodes is None or len(tree.nodes) == target_nodes:
            return tree
    raise RuntimeError("no trie with the requested node count")


class AttnWorkload:
    """``sets`` independent input sets (rotated to keep the KV stream out of the
    last-level cache) for one trie-verification attention shape."""

    def __init__(self, H=32, HK=8, D=128, P=3072, tree: Trie | None = None, base=0,
                 kv_scale=128 ** -0.5, sets=1, seed=0, device="cuda"):
        self.tree = tree if tree is not None else merged_trie(seed, 4, 24, 0, 16, 64)
        self.H, self.HK, self.D, self.P, self.base = H, HK, D, P, base
        self.N = len(self.tree.nodes)
        self.NN = max(32, -(-(base + self.N) // 32) * 32)
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        bf = torch.bfloat16

        def rnd(*shape, scale=1.0):
            return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * scale).to(bf)

        self.sets = []
        for _ in range(sets):
            q = rnd(H, self.N, D)
            kp = rnd(HK, P, D, scale=kv_scale)
            vp = rnd(HK, P, D, scale=kv_scale)
            kn = torch.zeros(HK, self.NN, D, dtype=bf, device=device)
            vn = torch.zeros_like(kn)
            kn[:, :base + self.N] = rnd(HK, base + self.N, D, scale=kv_scale)
            vn[:, :base + self.N] = rnd(HK, base + self.N, D, scale=kv_scale)
            self.sets.append((q, kp, vp, kn, vn))
        self.msk = torch.from_numpy(node_mask(self.tree, base, self.NN)).to(device)
        self.sm_scale = D ** -0.5

    def algorithmic_bytes(self) -> int:
        """K+V of prefix and nodes, Q in, O out, int32 parent array."""
        H, HK, D, P, N = self.H, self.HK, self.D, self.P, self.N
        return 4 * HK * D * (P + N) + 4 * H * N * D + 4 * N

    def flops(self) -> int:
        return 4 * self.H * self.D * self.N * (self.P + self.N)
