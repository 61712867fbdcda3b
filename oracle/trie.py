"""Trie construction, ancestry and the acceptance walk -- restated for the oracle.

Follows respect/candidates/trie.py:31-64 (build_trie, trie_ancestry) and
respect/decoding/acceptance.py:11-46 (mask_action_vocab, greedy_token, walk).

Pinned by: the known answers of the reference's tests/test_trie.py:11-49
(merge order, parent-before-child, ancestry row of a sibling branch, walk until
mismatch, walk stops at EOS), restated in tests/test_oracle.py; plus brute-force
checks (ancestry row i == set of nodes on the root path of i, by walking
parents) on random tries.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Node:
    token: int
    parent: int | None
    depth: int
    children: dict = field(default_factory=dict)


@dataclass
class Trie:
    nodes: list
    roots: dict
    seqs: list

    @property
    def parents(self) -> np.ndarray:
        """int32 parent index per node, -1 for a root (the kernel's parent-array format)."""
        return np.array([-1 if n.parent is None else n.parent for n in self.nodes], dtype=np.int32)

    @property
    def depths(self) -> np.ndarray:
        return np.array([n.depth for n in self.nodes], dtype=np.int32)

    @property
    def tokens(self) -> np.ndarray:
        return np.array([n.token for n in self.nodes], dtype=np.int64)


def build_trie(seqs) -> Trie:
    """Insert the distinct non-empty sequences in order; a new node gets the next index.

    trie.py:31-48: duplicates are dropped keeping the first occurrence, and a
    node is created the first time a (parent, token) pair is seen, so every
    parent index is smaller than its children's.
    """
    kept, seen = [], set()
    for s in seqs:
        s = tuple(s)
        if len(s) == 0 or s in seen:
            continue
        seen.add(s)
        kept.append(s)
    nodes: list[Node] = []
    roots: dict = {}
    for s in kept:
        cur = None
        for depth, tok in enumerate(s):
            table = roots if cur is None else nodes[cur].children
            nxt = table.get(tok)
            if nxt is None:
                nxt = len(nodes)
                table[tok] = nxt
                nodes.append(Node(int(tok), cur, depth))
            cur = nxt
    return Trie(nodes, roots, kept)


def trie_ancestry(tree: Trie) -> np.ndarray:
    """Boolean [n, n]: row i is node i and its ancestors (trie.py:51-64)."""
    n = len(tree.nodes)
    anc = np.zeros((n, n), dtype=bool)
    for i, nd in enumerate(tree.nodes):
        if nd.parent is not None:
            anc[i] = anc[nd.parent]
        anc[i, i] = True
    return anc


def ancestry_from_parents(parents) -> np.ndarray:
    """Same matrix from a parent array (parents precede children)."""
    parents = np.asarray(parents)
    n = len(parents)
    anc = np.zeros((n, n), dtype=bool)
    for i in range(n):
        p = int(parents[i])
        if p >= 0:
            assert p < i, "parents must precede children"
            anc[i] = anc[p]
        anc[i, i] = True
    return anc


def root_paths(tree: Trie) -> list[list[int]]:
    """Node-index path from the root to every leaf, in insertion order of the leaves."""
    leaves = [i for i, nd in enumerate(tree.nodes) if not nd.children]
    out = []
    for leaf in leaves:
        path, cur = [], leaf
        while cur is not None:
            path.append(cur)
            cur = tree.nodes[cur].parent
        out.append(path[::-1])
    return out


def mask_action_vocab(logits: np.ndarray, offset: int, size: int) -> np.ndarray:
    """fp32 copy of the logits with [offset, offset+size) set to -inf (acceptance.py:11-18)."""
    out = np.array(logits, dtype=np.float32, copy=True)
    out[..., offset:offset + size] = -np.inf
    return out


def greedy_token(logits: np.ndarray, offset: int, size: int) -> np.ndarray:
    """Row-wise argmax after masking; ties go to the lowest index (acceptance.py:21-23)."""
    return np.argmax(mask_action_vocab(logits, offset, size), axis=-1)


def walk(tree: Trie, first: int, cap: int, eos: int, pick):
    """Accept trie tokens while they match the target's choice (acceptance.py:26-46).

    Starts at the root whose token is ``first``.  ``pick(accepted, node)`` gives
    the target's token after ``node``.  Stops at EOS, at a branch end, at the
    first mismatch, or after ``cap`` tokens.  Returns (path, accepted, correction).
    """
    path: list[int] = []
    acc: list[int] = []
    node = tree.roots.get(first)
    correction = first
    while node is not None and len(acc) < cap:
        nd = tree.nodes[node]
        path.append(node)
        acc.append(nd.token)
        if nd.token == eos:
            break
        correction = pick(acc, node)
        node = nd.children.get(correction)
    return path, acc, correction
