"""Prefix trie over candidate token sequences (respect/candidates/trie.py:16-64).

Nodes are numbered in insertion order, so a parent always precedes its
children; the attention kernel relies on this when it folds a node's allowed
slots in slot order.  ``parents`` is the flat int32 parent array (-1 for a
root) from which the ancestor mask of a verification call is built.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Iterable

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
        return np.fromiter((-1 if n.parent is None else n.parent for n in self.nodes), np.int32,
                           len(self.nodes))

    @property
    def depths(self) -> np.ndarray:
        return np.fromiter((n.depth for n in self.nodes), np.int32, len(self.nodes))

    @property
    def tokens(self) -> np.ndarray:
        return np.fromiter((n.token for n in self.nodes), np.int64, len(self.nodes))


def build_trie(seqs: Iterable) -> Trie:
    """Merge sequences sharing a prefix into one trie; repeated sequences are dropped."""
    unique: list = []
    seen: set = set()
    for s in seqs:
        s = tuple(int(t) for t in s)
        if s and s not in seen:
            seen.add(s)
            unique.append(s)
    nodes: list[Node] = []
    roots: dict = {}
    for s in unique:
        parent = None
        for depth, tok in enumerate(s):
            children = roots if parent is None else nodes[parent].children
            idx = children.get(tok)
            if idx is None:
                idx = children[tok] = len(nodes)
                nodes.append(Node(tok, parent, depth))
            parent = idx
    return Trie(nodes, roots, unique)


def trie_ancestry(tree: Trie) -> np.ndarray:
    """[n, n] bool, entry (i, j) True when node i may attend to node j (itself or an ancestor)."""
    return ancestry_from_parents(tree.parents)


def ancestry_from_parents(parents) -> np.ndarray:
    parents = np.asarray(parents, dtype=np.int64)
    n = parents.shape[0]
    allowed = np.zeros((n, n), dtype=np.bool_)
    for i in range(n):
        p = parents[i]
        if p >= 0:
            if p >= i:
                raise ValueError("trie parents must precede their children")
            allowed[i] = allowed[p]
        allowed[i, i] = True
    return allowed


def node_mask(tree: Trie, base: int, n_slots: int) -> np.ndarray:
    """[n, n_slots] bool mask of a verification call whose node segment holds ``base``
    committed slots (open to every node) followed by the trie nodes in order."""
    n = len(tree.nodes)
    if base + n > n_slots:
        raise ValueError("node segment too small for the committed slots and the trie")
    m = np.zeros((n, n_slots), dtype=np.bool_)
    m[:, :base] = True
    m[:, base:base + n] = trie_ancestry(tree)
    return m
