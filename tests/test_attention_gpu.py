"""GPU parity and invariance tests of the trie-verification attention kernel.

Parity, three ways:
(1) per element, within 2 bf16 ulp of oracle.attention.attn_tree -- the CPU
    restatement of the kernel's own fixed reduction tree, itself pinned against
    float64 attention (tests/test_oracle.py) -- the ulp taken at
    max(|kernel|, |tree|, max|row| / 64).  The restatement
    (oracle/c/attn_tree.c, bit for bit the numpy attn_tree) models each MFMA
    as measured on MI355X and uses a correctly rounded exp2; the device's
    v_exp_f32 differs from that by one fp32 ulp on ~5 % of inputs and the MFMA
    model is exact on ~98.6 % (scores) / ~81 % (PV) of elements, so now and
    then a probability rounds to bf16 differently and moves its whole row by
    about an ulp at the row's scale -- an element 64x smaller than its row's
    largest then shows several of its own ulps (measured at cfg2: 99.989 % of
    elements bit-equal, max 1.0 ulp with the floor, 7 without);
(2) every output element within the deterministic error bound of the
    reference's rounding points around the float64 answer
    (oracle.attention.attn_error_bound: 2^-9 relative error of the bf16 prompt
    probabilities + fp32 slack + 1 bf16 ulp), the bound the restatement of the
    reference kernel (attn_hyb) itself satisfies;
(3) in bf16 ulps (at max(|exact|, rms/8)) at least as close to fp64 as the
    reference's own arithmetic (attn_hyb): the fraction within 2 ulp and the
    mean ulp error may not be worse.  attn_hyb's 128-key online softmax rounds
    p against a different running maximum than any split-K tree, so the kernel
    is not within 2 ulp of it everywhere (measured: 92-96 % of elements, at
    most 13-16 ulp); (1) is the per-element bar.

Invariance (bitwise, torch.equal): trie rows vs 1-token calls along each
root path, slot layouts, committed-token offsets, rows-per-wave settings.
"""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import bf16, gen

pytestmark = pytest.mark.gpu


def _dev(x, dtype=torch.bfloat16):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(dtype).cuda() if dtype is not None else t.cuda()


def _run(case, **kw):
    from respect_amd.kernels.attention import trie_attn
    print(f"[attn] H={case.q.shape[0]} M={case.q.shape[1]} D={case.q.shape[2]} "
          f"HK={case.kp.shape[0]} P={case.kp.shape[1]} NN={case.kn.shape[1]} {kw}", flush=True)
    out = trie_attn(_dev(case.q), _dev(case.kp), _dev(case.vp), _dev(case.kn), _dev(case.vn),
                    _dev(case.msk, None), case.sm_scale, **kw)
    torch.cuda.synchronize()
    return out


def _np(t):
    return t.float().cpu().numpy()


TREE_ULP = 2.0   # per-element bar against the kernel-tree restatement, in bf16 ulp


TREE_FLOOR = 64  # ulp taken at no less than max|row| / TREE_FLOOR


def _check_tree(case, o):
    """|kernel - attn_tree| <= 2 bf16 ulp of max(|kernel|, |attn_tree|, max|row| / 64),
    every element."""
    a = (case.q, case.kp, case.vp, case.kn, case.vn, case.msk, case.sm_scale)
    t = A.attn_tree_c(*a)
    mag = np.maximum(np.abs(o), np.abs(t))
    err = np.abs(o.astype(np.float64) - t)
    ud = err / bf16.ulp(np.maximum(mag, mag.max(axis=-1, keepdims=True) / TREE_FLOOR))
    raw = err / bf16.ulp(mag)
    print(f"  vs kernel tree: max {ud.max():.2f} ulp (no floor {raw.max():.1f}), "
          f"<=1 {(ud <= 1).mean():.5f}, equal {(o == t).mean():.5f}", flush=True)
    assert ud.max() <= TREE_ULP, f"max {ud.max():.2f} ulp at {np.unravel_index(ud.argmax(), ud.shape)}"


def _check_parity(case, out):
    a = (case.q, case.kp, case.vp, case.kn, case.vn, case.msk, case.sm_scale)
    o = _np(out)
    assert np.isfinite(o).all()
    _check_tree(case, o)
    e = A.attn_exact(*a)
    bound = A.attn_error_bound(*a)
    ratio = np.abs(o - e) / bound
    assert ratio.max() <= 1.0, f"max err/bound {ratio.max():.3f}"
    # ulp distances, measured at max(|exact|, rms/8) so near-zero outputs are not
    # judged by a vanishing ulp.  The reference's own arithmetic (the oracle) is
    # not within 2 ulp of fp64 everywhere (bf16 probabilities); the kernel must be
    # at least as close to fp64 as the oracle is.
    ref = A.attn_hyb(*a)
    rms = np.sqrt((e ** 2).mean())
    ud_k = bf16.ulp_diff(o, e, rms / 8)
    ud_r = bf16.ulp_diff(ref, e, rms / 8)
    ud_kr = bf16.ulp_diff(o, ref, rms / 8)
    print(f"  err/bound max {ratio.max():.3f} (oracle {(np.abs(ref - e) / bound).max():.3f}); "
          f"ulp vs fp64: <=2 {(ud_k <= 2).mean():.4f} (oracle {(ud_r <= 2).mean():.4f}) "
          f"mean {ud_k.mean():.3f} (oracle {ud_r.mean():.3f}); vs oracle: <=2 {(ud_kr <= 2).mean():.4f} "
          f"max {ud_kr.max():.2f} equal {(o == ref).mean():.4f}", flush=True)
    assert (ud_k <= 2).mean() >= (ud_r <= 2).mean() - 0.01
    assert ud_k.mean() <= 1.25 * ud_r.mean() + 0.05
    return o


def test_cfg1_parity():
    c = gen.cfg1()
    _check_parity(c, _run(c))


def test_cfg2_parity():
    c = gen.cfg2()
    _check_parity(c, _run(c))


def test_repeat_calls_are_bitwise_identical():
    c = gen.cfg2(seed=5)
    a = _run(c)
    for _ in range(3):
        assert torch.equal(_run(c), a)


def test_rows_per_wave_does_not_change_bits():
    """64 or 128 rows per prompt workgroup: a different work split, the same bits."""
    c = gen.cfg2(seed=3)
    assert torch.equal(_run(c, rows_per_wave=1), _run(c, rows_per_wave=2))


@pytest.mark.parametrize("cfg", ["cfg1", "cfg2"])
def test_trie_rows_equal_one_token_paths(cfg):
    """Output preservation at kernel level: row i of the trie call equals the 1-row call
    whose node segment is node i's root path laid out contiguously."""
    c = getattr(gen, cfg)()
    full = _run(c)
    for i in range(len(c.tree.nodes)):
        one = _run(gen.path_case(c, i))
        assert torch.equal(one[:, 0], full[:, i]), f"node {i}"


@pytest.mark.parametrize("base", [1, 7, 37, 100, 150, 200, 300])
def test_committed_offset_rows_equal_paths(base):
    """Trie placed after `base` committed slots (all rows see them); tile edges of the
    node segment fall mid-trie.  Each row equals its 1-token path call.  base 150 / 200 /
    300 put 224 / 288 / 384 slots in the node segment (V resident, V resident, streamed),
    their 1-token calls at most 192 / 224 / 352 (resident, V resident, streamed)."""
    c = gen.cfg2(seed=4, base=base)
    _check_parity(c, full := _run(c))
    rng = np.random.default_rng(base)
    for i in rng.choice(len(c.tree.nodes), 12, replace=False):
        one = _run(gen.path_case(c, int(i)))
        assert torch.equal(one[:, 0], full[:, int(i)]), f"node {i}"


# (nodes, sequences, length, shared prefix lo, hi): depth <= 32, exact node counts.
SWEEP_TRIES = ((1, 1, 1, 0, 0), (8, 2, 5, 2, 2), (32, 2, 20, 8, 8), (64, 4, 24, 0, 16), (128, 5, 32, 8, 8))


@pytest.mark.parametrize("P", [1024, 3072, 8192, 16384])
@pytest.mark.parametrize("tri", SWEEP_TRIES, ids=lambda t: f"n{t[0]}")
def test_invariance_sweep(P, tri):
    """8B shape over prompt lengths x trie sizes, the trie placed after a random number of
    committed slots (node-segment tile edges fall mid-trie): sampled rows (always the
    deepest) equal their 1-token path calls bitwise."""
    n, seqs, length, lo, hi = tri
    rng = np.random.default_rng(P + n)
    base = int(rng.integers(0, 48))
    c = gen.attn_case(P + n, 32, 8, 128, P, seqs, length, lo, hi, n, kv_scale=128 ** -0.5, base=base)
    full = _run(c)
    _check_tree(c, _np(full))
    depth = np.array([nd.depth for nd in c.tree.nodes])
    picks = {int(np.argmax(depth))} | {int(i) for i in rng.choice(n, min(n, 4), replace=False)}
    for i in sorted(picks):
        one = _run(gen.path_case(c, i))
        assert torch.equal(one[:, 0], full[:, i]), f"P={P} n={n} base={base} node {i}"


def _slot_layout_fixture():
    import json
    from pathlib import Path
    kats = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
    return kats["slot_layout"]


def test_slot_layout_invariance_reference_shapes():
    """tests/test_kernel_invariance.py:30-54 of the reference: 26 node values in slots
    0-25 vs 0-17 + 200-207, H=32, HK=8, D=128, NP=300, NN=224, 64 query rows (sizes read
    from tests/golden/reference_kats.json)."""
    fx = _slot_layout_fixture()
    rng = np.random.default_rng(0)
    H, HK, D, NP, n, NN, M = fx["H"], fx["HK"], fx["D"], fx["NP"], fx["n"], fx["NN"], fx["M"]
    assert n == 26 and NN == 224
    q = gen.bf16_normal(rng, (H, M, D))
    kp = gen.bf16_normal(rng, (HK, NP, D))
    vp = gen.bf16_normal(rng, (HK, NP, D))
    kk = gen.bf16_normal(rng, (HK, n, D))
    vv = gen.bf16_normal(rng, (HK, n, D))
    outs = []
    for slots in (list(range(n)), list(range(18)) + list(range(200, 208))):
        kn = np.zeros((HK, NN, D), np.float32)
        vn = np.zeros_like(kn)
        msk = np.zeros((M, NN), bool)
        kn[:, slots] = kk
        vn[:, slots] = vv
        msk[:, slots] = True
        case = gen.AttnCase(q, kp, vp, kn, vn, msk, None, 0, D ** -0.5)
        outs.append(_run(case))
        _check_parity(case, outs[-1])
    assert torch.equal(outs[0], outs[1])
    # random layouts as well (run_kernel_order.py checks 5)
    for seed in range(5):
        slots = sorted(np.random.default_rng(seed).choice(NN, n, replace=False).tolist())
        kn = np.zeros((HK, NN, D), np.float32)
        vn = np.zeros_like(kn)
        msk = np.zeros((M, NN), bool)
        kn[:, slots] = kk
        vn[:, slots] = vv
        msk[:, slots] = True
        assert torch.equal(_run(gen.AttnCase(q, kp, vp, kn, vn, msk, None, 0, D ** -0.5)), outs[0])


@pytest.mark.parametrize("P", [1, 31, 33, 3086, 5000])
def test_prompt_lengths(P):
    c = gen.attn_case(6, 32, 8, 128, P, 3, 10, 0, 5, None, kv_scale=128 ** -0.5)
    full = _run(c)
    _check_parity(c, full)
    for i in (0, len(c.tree.nodes) - 1):
        assert torch.equal(_run(gen.path_case(c, i))[:, 0], full[:, i])


@pytest.mark.parametrize("H,HK,D", [(8, 8, 64), (16, 8, 128), (32, 4, 128), (16, 2, 64), (32, 2, 128)])
def test_gqa_and_head_dims(H, HK, D):
    c = gen.attn_case(7, H, HK, D, 700, 3, 9, 0, 6, None)
    full = _run(c)
    _check_parity(c, full)
    i = len(c.tree.nodes) - 1
    assert torch.equal(_run(gen.path_case(c, i))[:, 0], full[:, i])


HEAD_DIM_CASES = {
    # resident node segments (at most 192 slots at D = 32, 64 at D = 256)
    "d32": lambda: gen.attn_case(7, 8, 2, 32, 700, 3, 9, 0, 6, None),
    "d256": lambda: gen.attn_case(8, 16, 8, 256, 900, 3, 10, 0, 6, None, kv_scale=256 ** -0.5),
    # streamed node segments
    "d32_b200": lambda: gen.attn_case(9, 8, 2, 32, 1500, 3, 12, 0, 6, None, base=200),
    "d256_b60": lambda: gen.attn_case(10, 16, 8, 256, 1200, 3, 12, 0, 6, None, kv_scale=256 ** -0.5, base=60),
    # 8B-like trie at D = 256 (512 prompt workgroups: two launches) and a
    # 128-node trie at D = 32 (two row tiles per wave)
    "d256_n64": lambda: gen.attn_case(11, 32, 8, 256, 3072, 4, 24, 0, 16, 64, kv_scale=256 ** -0.5),
    "d32_n128": lambda: gen.attn_case(12, 32, 8, 32, 3072, 8, 32, 0, 32, 128, kv_scale=32 ** -0.5),
}


@pytest.mark.parametrize("which", list(HEAD_DIM_CASES))
def test_head_dims_32_and_256(which):
    """head_dim 32 and 256 (the other sizes the reference's kernels take): per-element
    parity with the kernel-tree restatement and the fp64 bound, trie rows bitwise equal
    to their 1-token calls, and the same bits from one and two launches and (D = 32)
    from one and two row tiles per wave.  D = 256 runs one row tile per wave only."""
    from respect_amd import _lib
    c = HEAD_DIM_CASES[which]()
    H, M, D = c.q.shape
    print(f"[head_dim] {which} M={M} NN={c.kn.shape[1]}", flush=True)
    full = _run(c)
    _check_parity(c, full)
    n = len(c.tree.nodes)
    for i in sorted({0, n // 2, n - 1}):
        assert torch.equal(_run(gen.path_case(c, i))[:, 0], full[:, i])
    assert torch.equal(_run(c, launches=2), full)
    assert torch.equal(_run(c, launches=1), full)
    if D == 32:
        assert torch.equal(_run(c, rows_per_wave=1), full)
        assert torch.equal(_run(c, rows_per_wave=2), full)
    else:
        assert torch.equal(_run(c, rows_per_wave=1), full)
        with pytest.raises(_lib.RspxError):
            _run(c, rows_per_wave=2)


GQA_CASES = {
    # one q head per kv head (multi-head attention) and sixteen
    "gqa1": lambda: gen.attn_case(15, 8, 8, 128, 900, 3, 10, 0, 6, None, kv_scale=128 ** -0.5, base=20),
    "gqa16": lambda: gen.attn_case(16, 32, 2, 128, 1100, 3, 10, 0, 6, None, kv_scale=128 ** -0.5, base=50),
}


@pytest.mark.parametrize("which", list(GQA_CASES))
def test_gqa_1_and_16(which):
    """The outer q-heads-per-kv-head ratios the plan accepts: per-element parity with
    the kernel-tree restatement and the fp64 bound, trie rows bitwise equal to their
    1-token calls, and the same bits from one and two launches and from one and two
    row tiles per wave."""
    c = GQA_CASES[which]()
    H, M, D = c.q.shape
    print(f"[gqa] {which} H={H} HK={c.kp.shape[0]} M={M} NN={c.kn.shape[1]}", flush=True)
    full = _run(c)
    _check_parity(c, full)
    n = len(c.tree.nodes)
    for i in sorted({0, n // 2, n - 1}):
        assert torch.equal(_run(gen.path_case(c, i))[:, 0], full[:, i])
    assert torch.equal(_run(c, launches=2), full)
    assert torch.equal(_run(c, launches=1), full)
    assert torch.equal(_run(c, rows_per_wave=1), full)
    assert torch.equal(_run(c, rows_per_wave=2), full)


def test_no_node_slots_and_no_prompt():
    c = gen.cfg1()
    # NN = 0: prompt only
    c0 = gen.AttnCase(c.q, c.kp, c.vp, c.kn[:, :0], c.vn[:, :0], c.msk[:, :0], None, 0, c.sm_scale)
    _check_parity(c0, _run(c0))
    # P = 0: node segment only; every row allows its own slot
    cp = gen.AttnCase(c.q, c.kp[:, :0], c.vp[:, :0], c.kn, c.vn, c.msk, c.tree, 0, c.sm_scale)
    o = _np(_run(cp))
    e = A.attn_exact(cp.q, cp.kp, cp.vp, cp.kn, cp.vn, cp.msk, cp.sm_scale)
    assert np.abs(o - e).max() <= 2 * bf16.ulp(np.abs(e).max())


def test_large_trie_128_nodes_long_prompt():
    c = gen.attn_case(8, 32, 8, 128, 16384, 8, 32, 0, 32, 128, kv_scale=128 ** -0.5)
    full = _run(c)
    _check_parity(c, full)
    for i in np.random.default_rng(0).choice(128, 8, replace=False):
        assert torch.equal(_run(gen.path_case(c, int(i)))[:, 0], full[:, int(i)])


def test_drop_in_signature_and_errors():
    from respect_amd.kernels.attention import fused_attn_hyb
    c = gen.cfg1()
    args = [_dev(c.q), _dev(c.kp), _dev(c.vp), _dev(c.kn), _dev(c.vn), _dev(c.msk, None)]
    out = fused_attn_hyb(*args, BM=64, BN=128, BNB=16, num_warps=4, num_stages=1)
    assert out.shape == args[0].shape and out.dtype == torch.bfloat16
    assert torch.equal(out, _run(c))
    with pytest.raises(AssertionError):
        fused_attn_hyb(*args, BNB=24)
    with pytest.raises(TypeError):
        fused_attn_hyb(args[0].float(), *args[1:])
    # non-contiguous views are accepted (copied where the layout needs it)
    qt = args[0].transpose(0, 1).contiguous().transpose(0, 1)
    assert torch.equal(fused_attn_hyb(qt, *args[1:]), out)


def _status(case, ws):
    from respect_amd import _lib
    H, M, D = case.q.shape
    HK, P, _ = case.kp.shape
    return _lib.lib().rspx_trie_attn_status(ws.data_ptr(), H, HK, M, P, D, _lib.stream_ptr(ws.device))


@pytest.mark.parametrize("which", ["cfg1", "cfg2", "base37", "base100", "n64b40", "long", "gqa2", "d64",
                                   "d64b90", "n128b70", "n72", "n100b30", "n192p512", "n256p512", "n512p256"])
def test_one_and_two_launches_equal(which):
    """The one-kernel path (prompt groups, node partials and merge with workgroups
    waiting on per-row-block counters) and the two-kernel path give the same
    bits; the counters are back at zero after each call (repeat calls on one
    workspace stay equal) and no wait ran out.  base100 / n64b40 / d64b90 put
    65-128 slots in the node segment (two chunks, loaded whole by both paths); long /
    n128b70 have 512 rows per kv head, two row blocks per workgroup in one launch;
    n72 / n100b30 (288 / 400 rows, 5 / 7 row blocks) leave the last workgroups of
    that launch a single block.  n192p512 / n256p512 / n512p256 take the two-block
    launch with 4 / 4 / 2 key groups, where each workgroup merges 2 x 64 / NG
    consecutive rows of one block (a resident, a V-resident and a streamed node
    segment; 32 and 64 merge rows need two and four node batches)."""
    from respect_amd import _lib
    c = {"cfg1": gen.cfg1, "cfg2": gen.cfg2, "base37": lambda: gen.cfg2(seed=4, base=37),
         "base100": lambda: gen.cfg2(seed=4, base=100),
         "n64b40": lambda: gen.attn_case(11, 32, 8, 128, 3072, 4, 24, 0, 16, 64, kv_scale=128 ** -0.5, base=40),
         "long": lambda: gen.attn_case(8, 32, 8, 128, 16384, 8, 32, 0, 32, 128, kv_scale=128 ** -0.5),
         "gqa2": lambda: gen.attn_case(7, 16, 8, 128, 700, 3, 9, 0, 6, None),
         "d64": lambda: gen.attn_case(7, 16, 2, 64, 3086, 3, 9, 0, 6, None),
         "d64b90": lambda: gen.attn_case(7, 16, 2, 64, 3086, 3, 9, 0, 6, None, base=90),
         "n128b70": lambda: gen.attn_case(10, 32, 8, 128, 3072, 8, 32, 0, 32, 128, kv_scale=128 ** -0.5,
                                          base=70),
         "n72": lambda: gen.attn_case(14, 32, 8, 128, 3072, 4, 24, 0, 16, 72, kv_scale=128 ** -0.5),
         "n100b30": lambda: gen.attn_case(13, 32, 8, 128, 3072, 6, 24, 0, 16, 100, kv_scale=128 ** -0.5,
                                          base=30),
         "n192p512": lambda: gen.attn_case(16, 32, 8, 128, 512, 12, 16, 0, 0, 192, kv_scale=128 ** -0.5),
         "n256p512": lambda: gen.attn_case(17, 32, 8, 128, 512, 16, 16, 0, 0, 256, kv_scale=128 ** -0.5),
         "n512p256": lambda: gen.attn_case(18, 32, 8, 128, 256, 16, 32, 0, 0, 512, kv_scale=128 ** -0.5)}[which]()
    print(f"[one/two launches] {which} NN={c.kn.shape[1]}", flush=True)
    H, M, D = c.q.shape
    HK, P, _ = c.kp.shape
    need = _lib.lib().rspx_trie_attn_workspace_bytes(H, HK, M, P, D)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    two = _run(c, launches=2, workspace=ws)
    ones = [_run(c, launches=1, workspace=ws) for _ in range(3)]
    auto = _run(c, workspace=ws)
    assert _status(c, ws) == 0
    for o in ones + [auto]:
        assert torch.equal(o, two)
    for rpw in (1, 2):
        assert torch.equal(_run(c, launches=1, rows_per_wave=rpw, workspace=ws), two)
    assert _status(c, ws) == 0


@pytest.mark.parametrize("shape", ["8b", "d64"])
def test_one_and_two_pass_node_segments_equal(shape):
    """The same trie and committed slots in a node segment of 128 and 192 slots (two and
    three chunks of K and V resident), of 256 slots (the extra slots masked out; V resident,
    scores from K fragments loaded into registers), of 384 slots (streamed: a score pass
    whose scores stay in LDS, then V gathered by rank) and of 1024 / 512 slots (streamed past
    the kept-score limit: the scores recomputed from K gathered by rank) give the same
    bits, through one and two launches."""
    args = {"8b": (11, 32, 8, 128, 3072, 4, 24, 0, 16, 64), "d64": (7, 16, 2, 64, 3086, 3, 9, 0, 6, None)}[shape]
    kw = {"kv_scale": 128 ** -0.5} if shape == "8b" else {}
    base = 40 if shape == "8b" else 90
    short = gen.attn_case(*args, base=base, **kw)
    assert 64 < short.kn.shape[1] <= 128
    ref = _run(short, launches=2)
    for step in (192, 256, 384, 1024 if shape == "8b" else 512):
        long = gen.attn_case(*args, base=base, nn_step=step, **kw)
        assert long.kn.shape[1] == step and np.array_equal(long.msk[:, :short.kn.shape[1]], short.msk)
        for launches in (1, 2):
            assert torch.equal(_run(long, launches=launches), ref), f"NN={step} launches={launches}"
    assert torch.equal(_run(short, launches=1), ref)


def test_one_launch_workspace_shared_by_shapes():
    """One workspace used by calls of different shapes in turn (as the decoder's
    verify and 1-token calls share one): the counters sit where no call writes
    partials, so every call still equals its two-kernel result."""
    from respect_amd import _lib
    cases = [gen.cfg2(seed=9), gen.cfg1(), gen.attn_case(3, 32, 8, 128, 5000, 2, 4, 0, 1, None),
             gen.cfg2(seed=9, base=100)]
    need = max(_lib.lib().rspx_trie_attn_workspace_bytes(c.q.shape[0], c.kp.shape[0], c.q.shape[1],
                                                         c.kp.shape[1], c.q.shape[2]) for c in cases)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    want = [_run(c, launches=2) for c in cases]
    for _ in range(2):
        for c, w in zip(cases, want):
            assert torch.equal(_run(c, launches=1, workspace=ws), w)
    assert _status(cases[0], ws) == 0


@pytest.mark.parametrize("which", ["cfg2", "cfg1", "n128", "one"])
def test_wait_that_gives_up_poisons_its_rows(which):
    """One-launch path with the counter wait forced to give up at once (the spin limit
    lowered through the test hook, so every workgroup still exits normally): every row
    whose merge could not wait is NaN in every element -- the failure reaches the
    output without a host synchronisation -- and the status flag is raised.  With the
    default limit restored the same workspace gives the two-launch bits again (the
    counters were left at zero)."""
    from respect_amd import _lib
    c = {"cfg2": lambda: gen.cfg2(seed=6), "cfg1": gen.cfg1,
         # 512 rows per kv head: two row blocks per workgroup in the one-launch path
         "n128": lambda: gen.attn_case(9, 32, 8, 128, 3072, 8, 32, 0, 32, 128, kv_scale=128 ** -0.5),
         # one query row (4 rows per kv head, one row tile per wave)
         "one": lambda: gen.path_case(gen.cfg2(seed=6), 5)}[which]()
    H, M, D = c.q.shape
    HK, P, _ = c.kp.shape
    L = _lib.lib()
    ws = torch.zeros(L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D), dtype=torch.uint8, device="cuda")
    ref = _run(c, launches=2)
    prev = L.rspx_trie_attn_set_spin_limit(0)
    try:
        bad = _run(c, launches=1, workspace=ws)
    finally:
        L.rspx_trie_attn_set_spin_limit(prev)
    assert _status(c, ws) == 1
    assert _status(c, ws) == 0          # the query clears what it reports
    # a limit of 0 polls gives up in every workgroup: every row is NaN in every element
    assert torch.isnan(bad.float()).all()
    good = _run(c, launches=1, workspace=ws)
    assert torch.equal(good, ref)
    assert _status(c, ws) == 0


@pytest.mark.parametrize("which", ["cfg2", "n128b70", "one", "d64"])
def test_tiled_output_is_the_strided_output(which):
    """out with som = RSPX_TILED (the [M, H D] matrix in the tiled activation layout)
    holds the strided call's values bit for bit, through one and two launches; rows
    past M of the last 64-row block are not written."""
    from _tiled import from_tiled
    c = {"cfg2": gen.cfg2, "one": lambda: gen.path_case(gen.cfg2(), 10),
         "d64": lambda: gen.attn_case(7, 16, 2, 64, 3086, 3, 9, 0, 6, None),
         "n128b70": lambda: gen.attn_case(10, 32, 8, 128, 3072, 8, 32, 0, 32, 128, kv_scale=128 ** -0.5,
                                          base=70)}[which]()
    H, M, D = c.q.shape
    print(f"[tiled out] {which} H={H} M={M} D={D}", flush=True)
    ref = _run(c)                                           # [H, M, D]
    want = ref.permute(1, 0, 2).reshape(M, H * D)
    n = -(-M // 64) * 64 * H * D
    for launches in (0, 1, 2):
        buf = torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")
        _run(c, out=buf, out_tiled=True, launches=launches)
        assert torch.equal(from_tiled(buf, M, H * D), want)
        assert torch.isnan(buf.float()).sum().item() == (-(-M // 64) * 64 - M) * H * D


def test_tiled_output_rejects_a_head_stride_other_than_d():
    """som = RSPX_TILED names the [M, H D] layout, whose head stride is D: any other soh is
    RSPX_EINVAL and nothing is launched."""
    from respect_amd import _lib
    c = gen.cfg1()
    H, M, D = c.q.shape
    HK, P, _ = c.kp.shape
    NN = c.kn.shape[1]
    L = _lib.lib()
    q, kp, vp, kn, vn = (_dev(a) for a in (c.q, c.kp, c.vp, c.kn, c.vn))
    msk = _dev(c.msk, None)
    out = torch.full((-(-M // 64) * 64 * H * D,), 7.0, dtype=torch.bfloat16, device="cuda")
    ws = torch.zeros(L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D), dtype=torch.uint8, device="cuda")
    args = (q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), kp.stride(0), kp.stride(1),
            vp.data_ptr(), vp.stride(0), vp.stride(1), kn.data_ptr(), kn.stride(0), kn.stride(1),
            vn.data_ptr(), vn.stride(0), vn.stride(1), msk.data_ptr(), msk.stride(0), msk.stride(1), out.data_ptr())
    tail = (H, HK, M, P, NN, D, c.sm_scale, ws.data_ptr(), ws.numel(), 0, _lib.stream_ptr(q.device))
    assert L.rspx_trie_attn(*args, 2 * D, _lib.RSPX_TILED, *tail) == -1   # RSPX_EINVAL
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
    assert L.rspx_trie_attn(*args, D, _lib.RSPX_TILED, *tail) == 0
