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


def test_walk_kats():
    for case in KATS["walk"]:
        t = OT.build_trie([tuple(s) for s in case["seqs"]])
        tgt = {int(k): v for k, v in case["target_after_node"].items()}
        path, acc, rec = OT.walk(t, case["root"], case["cap"], EOS, lambda a, ch: tgt[ch])
        assert acc == case["accepted"], case["ref"]
        if "path" in case:
            assert path == case["path"] and rec == case["recovered"], case["ref"]


def test_slot_layout_fixture_is_consistent():
    """The GPU slot-layout test reads its sizes from this fixture."""
    s = KATS["slot_layout"]
    slots_b = list(range(18)) + list(range(200, 208))
    assert len(slots_b) == s["n"] and max(slots_b) < s["NN"] and s["NN"] % 16 == 0
