"""Host-side model of the one-launch attention's cross-workgroup protocol
(respect_amd/csrc/trie_attn.hip: count_partial, block_tail, fused_kernel,
fused2_kernel), run on the CPU under many random schedules.

Each workgroup (g, rb, q) of a row block of NG workgroups:
  1. stores its group partial, then counts it: cnt[rb] += 1;
  2. polls cnt[rb] until it reaches NG or a deadline passes (then it "gives
     up": its rows become NaN and the status word is set);
  3. merges, reading the NG partials of its block;
  4. adds 1 to done[rb]; the workgroup that brings done[rb] to NG resets
     cnt[rb] and done[rb] to zero.
fused2_kernel runs steps 1 for both of its row blocks before any step 2.

The scheduler holds at most `slots` workgroups resident (dispatch in
workgroup order, a slot freed when a workgroup ends) and interleaves the
resident ones at random.  Checked in every schedule:
  - safety: a workgroup that merges without giving up saw all NG partials of
    its block complete (no merge reads a partial before its count);
  - no counter is reset while a workgroup of its block can still read it;
  - the counters are zero when the grid ends (the next call starts clean),
    whether or not a wait gave up;
  - liveness: with the whole grid resident no wait gives up; with fewer slots
    than workgroups the deadline ends every wait, so the grid still drains.
"""
import random

import pytest


def run(NRB, NG, slots, two=False, deadline=200, seed=0):
    rng = random.Random(seed)
    cnt = [0] * NRB
    done = [0] * NRB
    stored = [set() for _ in range(NRB)]
    NRBW = (NRB + 1) // 2
    wgs = []
    for q in range(NG):
        for rbw in range(NRBW if two else NRB):
            blocks = [rbw, rbw + NRBW] if two and rbw + NRBW < NRB else [rbw]
            wgs.append({"q": q, "blocks": blocks})
    events = {"gave_up": 0, "merged": 0}

    def program(wg):
        for rb in wg["blocks"]:                      # prompt groups, then counts
            yield
            stored[rb].add(wg["q"])                  # partial complete (vmcnt 0, barrier)
            cnt[rb] += 1                             # count_partial
        for rb in wg["blocks"]:                      # block_tail
            polls, v = 0, 0
            while True:
                v = cnt[rb]
                if v >= NG or polls >= deadline:
                    break
                polls += 1
                yield
            if v >= NG:
                assert len(stored[rb]) == NG         # every partial of the block is complete
                events["merged"] += 1
            else:
                events["gave_up"] += 1
            yield
            assert cnt[rb] >= v                      # no reset while this workgroup reads
            done[rb] += 1
            if done[rb] == NG:
                cnt[rb] = 0
                done[rb] = 0
                stored[rb].clear()

    pending = list(wgs)
    resident = []
    while pending or resident:
        while pending and len(resident) < slots:     # in-order dispatch
            resident.append(program(pending.pop(0)))
        p = rng.randrange(len(resident))
        try:
            next(resident[p])
        except StopIteration:
            resident.pop(p)
    assert cnt == [0] * NRB and done == [0] * NRB
    return events


@pytest.mark.parametrize("NRB,NG,two", [(1, 32, False), (2, 16, False), (4, 8, False), (4, 8, True),
                                        (3, 8, True)])
def test_resident_grid_never_gives_up(NRB, NG, two):
    """8B-shape grids (256 workgroups = 8 kv heads x 32; one kv head modelled) all resident."""
    n = NG * (((NRB + 1) // 2) if two else NRB)
    for seed in range(40):
        ev = run(NRB, NG, slots=n, two=two, seed=seed)
        assert ev["gave_up"] == 0 and ev["merged"] == NRB * NG


@pytest.mark.parametrize("NRB,NG,two", [(2, 16, False), (4, 8, True)])
def test_partial_residency_drains_by_the_deadline(NRB, NG, two):
    """Fewer slots than workgroups (another process holding CUs): waits give up at the
    deadline, every workgroup still ends, and the counters are zero afterwards."""
    n = NG * (((NRB + 1) // 2) if two else NRB)
    gave = 0
    for seed in range(40):
        ev = run(NRB, NG, slots=n // 2, two=two, seed=seed)
        assert ev["gave_up"] + ev["merged"] == NRB * NG
        gave += ev["gave_up"]
    assert gave > 0


def test_model_catches_a_count_before_the_store():
    """A planted mistake in the model (counting before the partial is complete) is caught."""
    def bad_run():
        cnt, stored = [0], set()
        order = [("count", 0), ("count", 1), ("merge", 0), ("store", 0), ("store", 1)]
        for op, q in order:
            if op == "count":
                cnt[0] += 1
            elif op == "store":
                stored.add(q)
            elif cnt[0] >= 2:
                assert len(stored) == 2
    with pytest.raises(AssertionError):
        bad_run()
