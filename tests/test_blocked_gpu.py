"""The tile-wise ("blocked") attention -- the negative control of the reference's
slot-layout experiment (respect/kernels/reference_blocked.py, scripts/run_kernel_order.py)
-- on the GPU.

Parity: every element within the error bound of its own rounding points around float64
attention (oracle.attention.attn_error_bound with node_p_bf16: bf16 probabilities in every
PV product), the bound the oracle's restatement attn_blocked satisfies.  The experiment:
the same 26 node values in slots 0-25 and in slots 0-17 + 200-207 (the reference's
tests/test_kernel_invariance.py:30-54 shapes) change the blocked kernel's output and leave
the trie kernel's bits unchanged (the reference reports a 2.4414e-04 maximum difference
for its blocked kernel on its real inputs, docs/method_details.md:176)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import gen

pytestmark = pytest.mark.gpu


def _dev(x, dtype=torch.bfloat16):
    t = torch.from_numpy(np.ascontiguousarray(x))
    return t.to(dtype).cuda() if dtype is not None else t.cuda()


def _blocked(case, BN=64):
    from respect_amd.kernels.reference_blocked import fused_attn
    print(f"[blocked] H={case.q.shape[0]} M={case.q.shape[1]} D={case.q.shape[2]} P={case.kp.shape[1]} "
          f"NN={case.kn.shape[1]} BN={BN}", flush=True)
    out = fused_attn(_dev(case.q), _dev(case.kp), _dev(case.vp), _dev(case.kn), _dev(case.vn),
                     _dev(case.msk, None), case.sm_scale, BN=BN)
    torch.cuda.synchronize()
    return out


def _check(case, out, BN=64):
    a = (case.q, case.kp, case.vp, case.kn, case.vn, case.msk, case.sm_scale)
    o = out.float().cpu().numpy()
    assert np.isfinite(o).all()
    e = A.attn_exact(*a)
    bound = A.attn_error_bound(*a, node_p_bf16=True)
    r = np.abs(o - e) / bound
    ref = A.attn_blocked(*a, BN=BN)
    print(f"  err/bound max {r.max():.3f} (oracle attn_blocked {(np.abs(ref - e) / bound).max():.3f})", flush=True)
    assert r.max() <= 1.0


@pytest.mark.parametrize("which,BN", [("cfg1", 64), ("cfg2", 64), ("cfg2", 32), ("cfg2", 128), ("base40", 64),
                                      ("d32", 64), ("d256", 32), ("d256", 128)])
def test_blocked_parity(which, BN):
    """Every head_dim the reference's fused_attn accepts (reference_blocked.py:89)."""
    c = {"cfg1": gen.cfg1, "cfg2": gen.cfg2, "base40": lambda: gen.cfg2(seed=4, base=40),
         "d32": lambda: gen.attn_case(7, 8, 2, 32, 700, 3, 10, 0, 8, 24),
         "d256": lambda: gen.attn_case(8, 8, 4, 256, 900, 3, 12, 0, 8, 32, kv_scale=256 ** -0.5)}[which]()
    _check(c, _blocked(c, BN), BN)


def _layout_cases():
    fx = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())["slot_layout"]
    rng = np.random.default_rng(0)
    H, HK, D, NP, n, NN, M = fx["H"], fx["HK"], fx["D"], fx["NP"], fx["n"], fx["NN"], fx["M"]
    q = gen.bf16_normal(rng, (H, M, D))
    kp = gen.bf16_normal(rng, (HK, NP, D))
    vp = gen.bf16_normal(rng, (HK, NP, D))
    kk = gen.bf16_normal(rng, (HK, n, D))
    vv = gen.bf16_normal(rng, (HK, n, D))
    cases = []
    for slots in (list(range(n)), list(range(18)) + list(range(200, 208))):
        kn = np.zeros((HK, NN, D), np.float32)
        vn = np.zeros_like(kn)
        msk = np.zeros((M, NN), bool)
        kn[:, slots] = kk
        vn[:, slots] = vv
        msk[:, slots] = True
        cases.append(gen.AttnCase(q, kp, vp, kn, vn, msk, None, 0, D ** -0.5))
    return cases


def test_slot_layout_experiment():
    """Blocked kernel: the layout changes the output; trie kernel: bitwise equal."""
    from respect_amd.kernels.attention import trie_attn
    a, b = _layout_cases()
    ba, bb = _blocked(a), _blocked(b)
    _check(a, ba)
    _check(b, bb)
    diff = float((ba.float() - bb.float()).abs().max())
    print(f"[slot layout] blocked kernel max |diff| between layouts: {diff:.4e}", flush=True)
    assert diff > 0
    run = lambda c: trie_attn(_dev(c.q), _dev(c.kp), _dev(c.vp), _dev(c.kn), _dev(c.vn), _dev(c.msk, None),
                              c.sm_scale)
    assert torch.equal(run(a), run(b))
    # the oracle's restatement of the blocked kernel also depends on the layout
    oa = A.attn_blocked(a.q, a.kp, a.vp, a.kn, a.vn, a.msk, a.sm_scale)
    ob = A.attn_blocked(b.q, b.kp, b.vp, b.kn, b.vn, b.msk, b.sm_scale)
    assert not np.array_equal(oa, ob)


def test_blocked_signature_and_errors():
    from respect_amd import _lib
    from respect_amd.kernels.reference_blocked import fused_attn
    c = gen.cfg1()
    args = [_dev(c.q), _dev(c.kp), _dev(c.vp), _dev(c.kn), _dev(c.vn), _dev(c.msk, None)]
    out = fused_attn(*args, sm_scale=None, BM=64, BN=64, num_warps=4, num_stages=2)
    assert out.shape == args[0].shape and out.dtype == torch.bfloat16
    assert torch.equal(out, fused_attn(*args))                 # deterministic
    with pytest.raises(_lib.RspxError):
        fused_attn(*args, BN=48)
    with pytest.raises(AssertionError):
        fused_attn(args[0][:5], *args[1:])                     # H = 5 not a multiple of HK = 2
