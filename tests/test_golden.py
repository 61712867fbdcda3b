"""The reference's own known answers (tests/golden/reference_kats.json) against
the oracle and against the product's host-side trie code."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle.trie as OT
import respect_amd.candidates.trie as PT

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
EOS = KATS["eos"]


@pytest.mark.parametrize("mod", [OT, PT], ids=["oracle", "product"])
def test_build_trie_kats(mod):
    for case in KATS["build_trie"]:
        t = mod.build_trie([tuple(s) for s in case["seqs"]])
        assert [n.token for n in t.nodes] == case["tokens"], case["ref"]
        assert len(t.seqs) == case["n_seqs"], case["ref"]


@pytest.mark.parametrize("mod", [OT, PT], ids=["oracle", "product"])
def test_ancestry_kats(mod):
    for case in KATS["ancestry"]:
        t = mod.build_trie([tuple(s) for s in case["seqs"]])
        a = mod.trie_ancestry(t)
        assert np.flatnonzero(a[case["node"]]).tolist() == case["allowed"], case["ref"]
        for i, n in enumerate(t.nodes):
            assert n.parent is None or n.parent < i


def _walks():
    from respect_amd.decoding import acceptance
    return {"oracle": (OT.build_trie, OT.walk), "product": (PT.build_trie, acceptance.walk)}


@pytest.mark.parametrize("which", ["oracle", "product"])
def test_walk_kats(which):
    build, walk = _walks()[which]
    for case in KATS["walk"]:
        t = build([tuple(s) for s in case["seqs"]])
        tgt = {int(k): v for k, v in case["target_after_node"].items()}
        path, acc, rec = walk(t, case["root"], case["cap"], EOS, lambda a, ch: tgt[ch])
        assert acc == case["accepted"], case["ref"]
        if "path" in case:
            assert path == case["path"] and rec == case["recovered"], case["ref"]


def test_product_walk_equals_oracle_walk_on_random_tries():
    """Random tries, targets and caps (including 0 and an EOS inside a branch): the
    product's walk and the oracle's independent restatement agree on every output."""
    from respect_amd.decoding import acceptance
    rng = np.random.default_rng(7)
    for _ in range(300):
        seqs = [tuple(int(x) for x in rng.integers(0, 6, int(rng.integers(1, 7)))) for _ in range(int(rng.integers(1, 5)))]
        if rng.random() < 0.3:
            s = list(seqs[0])
            s[int(rng.integers(0, len(s)))] = EOS
            seqs[0] = tuple(s)
        po, pp = OT.build_trie(seqs), PT.build_trie(seqs)
        tgt = {i: int(rng.integers(0, 6)) for i in range(len(po.nodes))}
        if rng.random() < 0.5:       # a target that follows the first sequence
            for i, n in enumerate(po.nodes):
                kids = list(n.children)
                if kids:
                    tgt[i] = kids[0]
        root, cap = int(seqs[0][0]), int(rng.integers(0, 8))
        a = OT.walk(po, root, cap, EOS, lambda acc, ch: tgt[ch])
        b = acceptance.walk(pp, root, cap, EOS, lambda acc, ch: tgt[ch])
        assert a == b, (seqs, tgt, cap)


def test_slot_layout_fixture_is_consistent():
    """tests/test_attention_gpu.py::test_slot_layout_invariance_reference_shapes reads its
    sizes from this fixture."""
    s = KATS["slot_layout"]
    slots_b = list(range(18)) + list(range(200, 208))
    assert len(slots_b) == s["n"] and max(slots_b) < s["NN"] and s["NN"] % 16 == 0
