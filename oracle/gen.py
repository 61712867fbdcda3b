"""Seeded synthetic inputs for the benchmark workloads (numpy, CPU).

All tensors are float32 arrays holding bf16 values (rounded RNE), so the same
bits can be handed to the GPU kernels and to the oracle.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bf16 import round_bf16
from .trie import Trie, build_trie, trie_ancestry

VOCAB = 151936


def merged_trie(rng: np.random.Generator, n_seqs: int, length: int, pre_lo: int, pre_hi: int,
                target_nodes: int | None = None, vocab: int = VOCAB, max_tries: int = 10000) -> Trie:
    """Merge ``n_seqs`` random token sequences; sequence i copies a random-length
    prefix (uniform in [pre_lo, pre_hi]) of a random earlier sequence.  With a
    target node count, draws are repeated until the trie has exactly that many nodes."""
    for _ in range(max_tries):
        seqs = [rng.integers(0, vocab, length)]
        for i in range(1, n_seqs):
            src = seqs[int(rng.integers(0, i))]
            s = int(rng.integers(pre_lo, pre_hi + 1))
            new = rng.integers(0, vocab, length)
            new[:s] = src[:s]
            seqs.append(new)
        tree = build_trie([tuple(int(t) for t in s) for s in seqs])
        if target_nodes is None or len(tree.nodes) == target_nodes:
            return tree
    raise RuntimeError("could not draw a trie with the requested node count")


def bf16_normal(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return round_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


@dataclass
class AttnCase:
    q: np.ndarray      # [H, M, D]
    kp: np.ndarray     # [HK, P, D]
    vp: np.ndarray
    kn: np.ndarray     # [HK, NN, D]
    vn: np.ndarray
    msk: np.ndarray    # [M, NN] bool
    tree: Trie | None
    base: int          # committed node slots before the trie
    sm_scale: float


def trie_mask(tree: Trie, base: int, NN: int, slots: np.ndarray | None = None) -> np.ndarray:
    """[n, NN] bool: committed slots [0, base) open to every node; node i open to its
    ancestors, which sit at node slots ``slots[j]`` (default base + j)."""
    n = len(tree.nodes)
    if slots is None:
        slots = base + np.arange(n)
    anc = trie_ancestry(tree)
    msk = np.zeros((n, NN), dtype=bool)
    msk[:, :base] = True
    for i in range(n):
        msk[i, slots[anc[i]]] = True
    return msk


def attn_case(seed: int, H: int, HK: int, D: int, P: int, n_seqs: int, length: int,
              pre_lo: int, pre_hi: int, target_nodes: int | None, kv_scale: float = 1.0,
              base: int = 0, nn_step: int = 32) -> AttnCase:
    rng = np.random.default_rng(seed)
    tree = merged_trie(rng, n_seqs, length, pre_lo, pre_hi, target_nodes)
    M = len(tree.nodes)
    NN = max(nn_step, -(-(base + M) // nn_step) * nn_step)
    q = bf16_normal(rng, (H, M, D))
    kp = bf16_normal(rng, (HK, P, D), kv_scale)
    vp = bf16_normal(rng, (HK, P, D), kv_scale)
    kn = np.zeros((HK, NN, D), np.float32)
    vn = np.zeros((HK, NN, D), np.float32)
    kn[:, :base + M] = bf16_normal(rng, (HK, base + M, D), kv_scale)
    vn[:, :base + M] = bf16_normal(rng, (HK, base + M, D), kv_scale)
    return AttnCase(q, kp, vp, kn, vn, trie_mask(tree, base, NN), tree, base, D ** -0.5)


def cfg1(seed: int = 1) -> AttnCase:
    """512-token KV, 8 q / 2 kv heads, head_dim 64; 16-node trie from 3 sequences of 8."""
    return attn_case(seed, 8, 2, 64, 512, 3, 8, 0, 8, 16)


def cfg2(seed: int = 2, base: int = 0) -> AttnCase:
    """8B shape: 32 q / 8 kv heads, head_dim 128, 3072-token KV ~ N(0,1)/sqrt(128);
    64-node trie from 4 sequences of 24 with shared prefixes uniform in [0, 16]."""
    return attn_case(seed, 32, 8, 128, 3072, 4, 24, 0, 16, 64, kv_scale=128 ** -0.5, base=base)


def path_case(case: AttnCase, node: int) -> AttnCase:
    """The 1-token decoding view of ``node``: one query row whose node segment holds the
    committed slots followed by the node's root path laid out contiguously."""
    tree = case.tree
    path, cur = [], node
    while cur is not None:
        path.append(cur)
        cur = tree.nodes[cur].parent
    path = path[::-1]
    b = case.base
    T = b + len(path)
    NN = max(32, -(-T // 32) * 32)
    HK, _, D = case.kn.shape
    kn = np.zeros((HK, NN, D), np.float32)
    vn = np.zeros((HK, NN, D), np.float32)
    kn[:, :b] = case.kn[:, :b]
    vn[:, :b] = case.vn[:, :b]
    kn[:, b:T] = case.kn[:, b + np.array(path)]
    vn[:, b:T] = case.vn[:, b + np.array(path)]
    msk = np.zeros((1, NN), dtype=bool)
    msk[0, :T] = True
    return AttnCase(case.q[:, node:node + 1].copy(), case.kp, case.vp, kn, vn, msk, None, b, case.sm_scale)
