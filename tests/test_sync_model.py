"""Host-side model of the one-launch attention's cross-workgroup protocol
(respect_amd/csrc/trie_attn.hip: count_partial, block_tail, fused_kernel,
fused2_kernel), run on the CPU under many random schedules.

Each workgroup (g, rb, q) of a row block of NG workgroups:
  0. reads the block's counter at its start (`old`, before its own add);
  1. stores its group partial, then adds its share to the block's counter --
     kCountUnit / NG, plus one for the first kCountUnit % NG workgroups, so a
     call moves every counter it uses by exactly kCountUnit;
  2. polls the counter until it is kCountUnit past base = old rounded down
     to a multiple of kCountUnit, or a deadline passes (then it "gives up":
     its rows become NaN and the status word is set);
  3. merges, reading the NG partials of its block.
Counters are never reset.  fused2_kernel runs step 1 for both of its row
blocks before any step 2 (the first block's add comes once the second block's
first loads have landed); with NG = 2, 4 or 8 each of its workgroups then
runs steps 2-3 for one of the two blocks only (workgroups q < NG / 2 the
first), otherwise for both.

The scheduler holds at most `slots` workgroups resident (dispatch in
workgroup order, a slot freed when a workgroup ends) and interleaves the
resident ones at random.  Calls run one after another, with different NG and
row-block counts sharing the counters.  Checked in every schedule:
  - safety: a workgroup that merges without giving up saw all NG partials of
    its block complete (no merge reads a partial before its count);
  - every counter a call uses moves by exactly kCountUnit, whether or not a
    wait gave up, so the next call (of any shape) starts from multiples of
    kCountUnit;
  - liveness: with the whole grid resident no wait gives up; with fewer slots
    than workgroups the deadline ends every wait, so the grid still drains.
"""
import random

import pytest

UNIT = 8   # kCountUnit = kGroupTarget


def share(q, NG):
    return UNIT // NG + (1 if q < UNIT % NG else 0)


def run(cnt, NRB, NG, slots, two=False, deadline=200, seed=0):
    """One call on the shared counters `cnt` (one per row block)."""
    assert 1 <= NG <= UNIT
    rng = random.Random(seed)
    start = list(cnt)
    assert all(c % UNIT == 0 for c in start)
    stored = [set() for _ in range(NRB)]
    NRBW = (NRB + 1) // 2
    wgs = []
    for q in range(NG):
        for rbw in range(NRBW if two else NRB):
            blocks = [rbw, rbw + NRBW] if two and rbw + NRBW < NRB else [rbw]
            wgs.append({"q": q, "blocks": blocks})
    events = {"gave_up": 0, "merged": 0}

    def program(wg):
        blocks = wg["blocks"]
        olds = [cnt[rb] for rb in blocks]            # counter_before, at the kernel's start
        if len(blocks) == 1:
            yield                                    # prompt groups
            stored[blocks[0]].add(wg["q"])           # partial complete (vmcnt 0, barrier)
            cnt[blocks[0]] += share(wg["q"], NG)     # count_partial
        else:
            yield                                    # first block's prompt groups
            stored[blocks[0]].add(wg["q"])           # its stores issued ...
            yield                                    # ... second block's round 0 landed (vmcnt 0)
            cnt[blocks[0]] += share(wg["q"], NG)     # first block's count
            yield                                    # rest of the second block
            stored[blocks[1]].add(wg["q"])
            cnt[blocks[1]] += share(wg["q"], NG)     # count_partial
        for rb, old in merge_plan(wg, olds):         # block_tail
            base = old - old % UNIT
            polls = 0
            while True:
                v = cnt[rb]
                if v - base >= UNIT or polls >= deadline:
                    break
                polls += 1
                yield
            if v - base >= UNIT:
                assert len(stored[rb]) == NG         # every partial of the block is complete
                events["merged"] += 1
            else:
                events["gave_up"] += 1
            yield

    def merge_plan(wg, olds):
        blocks = wg["blocks"]
        if len(blocks) == 2 and NG in (2, 4, 8):     # one block's rows per workgroup
            i = 0 if wg["q"] < NG // 2 else 1
            return [(blocks[i], olds[i])]
        return list(zip(blocks, olds))

    events["expected"] = sum(len(merge_plan(wg, [0, 0])) for wg in wgs)
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
    assert [c - s for c, s in zip(cnt, start)] == [UNIT] * NRB
    return events


def n_wgs(NRB, NG, two):
    return NG * (((NRB + 1) // 2) if two else NRB)


@pytest.mark.parametrize("NRB,NG,two", [(1, 8, False), (2, 8, False), (4, 8, False), (4, 8, True), (3, 6, True),
                                        (4, 3, False), (2, 5, False), (1, 1, False), (2, 7, True), (8, 4, True),
                                        (5, 2, True), (16, 8, True)])
def test_resident_grid_never_gives_up(NRB, NG, two):
    """Grids of every NG (the 8B shape: 4 row blocks x 8 groups per kv head) all resident."""
    for seed in range(30):
        cnt = [0] * NRB
        for call in range(3):
            ev = run(cnt, NRB, NG, slots=n_wgs(NRB, NG, two), two=two, seed=seed * 7 + call)
            assert ev["gave_up"] == 0 and ev["merged"] == ev["expected"]


def test_calls_of_different_shapes_share_the_counters():
    """A sequence of calls with different NG, row-block counts and one or two blocks per
    workgroup on one set of counters (a shared workspace): every call merges cleanly."""
    rng = random.Random(5)
    cnt = [0] * 8
    for call in range(60):
        NRB = rng.randint(1, 8)
        NG = rng.randint(1, UNIT)
        two = rng.random() < 0.3
        sub = cnt[:NRB]
        ev = run(sub, NRB, NG, slots=n_wgs(NRB, NG, two), two=two, seed=call)
        cnt[:NRB] = sub
        assert ev["gave_up"] == 0 and ev["merged"] == ev["expected"]
    assert all(c % UNIT == 0 for c in cnt)


@pytest.mark.parametrize("NRB,NG,two", [(2, 8, False), (4, 8, True), (3, 5, False)])
def test_partial_residency_drains_by_the_deadline(NRB, NG, two):
    """Fewer slots than workgroups (another process holding CUs): waits give up at the
    deadline, every workgroup still ends, each counter still moves by exactly one unit,
    and the next call, fully resident, merges cleanly."""
    gave = 0
    for seed in range(30):
        cnt = [0] * NRB
        ev = run(cnt, NRB, NG, slots=max(1, n_wgs(NRB, NG, two) // 2), two=two, seed=seed)
        assert ev["gave_up"] + ev["merged"] == ev["expected"]
        gave += ev["gave_up"]
        ev = run(cnt, NRB, NG, slots=n_wgs(NRB, NG, two), two=two, seed=seed + 100)
        assert ev["gave_up"] == 0
    assert gave > 0


def test_model_catches_planted_mistakes():
    """Planted mistakes in the model fail it: a count before the store, and shares that
    do not add up to the unit (the next call's base would be off)."""
    def count_before_store():
        cnt, stored = [0], set()
        for op, q in [("count", 0), ("count", 1), ("merge", 0), ("store", 0), ("store", 1)]:
            if op == "count":
                cnt[0] += UNIT // 2
            elif op == "store":
                stored.add(q)
            elif cnt[0] >= UNIT:
                assert len(stored) == 2
    with pytest.raises(AssertionError):
        count_before_store()
    global share
    good = share
    try:
        share = lambda q, NG: UNIT // NG      # drops the remainder: NG = 3 adds 6, not 8
        with pytest.raises(AssertionError):
            run([0], 1, 3, slots=3)
    finally:
        share = good
