"""rspx_trie_attn_noalloc (the entry point that allocates nothing, its scratch a static
device array) against rspx_trie_attn with a caller workspace, through the C ABI: bitwise
equal on two calls in a row, the second smaller than the first, and sizes beyond the
static scratch refused with RSPX_EWORKSPACE before any launch; its timeout flag read and
cleared without a workspace pointer."""
import numpy as np
import pytest
import torch

from oracle import gen

pytestmark = pytest.mark.gpu


def _tensors(case):
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).cuda()
    return (t(case.q), t(case.kp), t(case.vp), t(case.kn), t(case.vn),
            torch.from_numpy(np.ascontiguousarray(case.msk)).to(torch.uint8).cuda())


def _args(q, kp, vp, kn, vn, msk, out):
    return (q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), kp.stride(0), kp.stride(1),
            vp.data_ptr(), vp.stride(0), vp.stride(1), kn.data_ptr(), kn.stride(0), kn.stride(1),
            vn.data_ptr(), vn.stride(0), vn.stride(1), msk.data_ptr(), msk.stride(0), msk.stride(1),
            out.data_ptr(), out.stride(0), out.stride(1))


def _shape(q, kp, kn):
    H, M, D = q.shape
    return H, kp.shape[0], M, kp.shape[1], kn.shape[1], D


def test_noalloc_equals_workspace_entry_point():
    from respect_amd import _lib
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    cases = [("cfg2", gen.cfg2(seed=2)), ("cfg1", gen.cfg1(seed=3))]      # the second call is smaller
    for name, c in cases:
        q, kp, vp, kn, vn, msk = _tensors(c)
        H, HK, M, P, NN, D = _shape(q, kp, kn)
        print(f"[noalloc] {name} H={H} HK={HK} M={M} P={P} NN={NN} D={D}", flush=True)
        ws = torch.zeros(L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D), dtype=torch.uint8, device="cuda")
        ref = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert L.rspx_trie_attn(*_args(q, kp, vp, kn, vn, msk, ref), H, HK, M, P, NN, D, D ** -0.5,
                                ws.data_ptr(), ws.numel(), 0, s) == 0
        assert L.rspx_trie_attn_noalloc(*_args(q, kp, vp, kn, vn, msk, got), H, HK, M, P, NN, D, D ** -0.5,
                                        0, s) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, ref), name
        # and once more on the same static scratch (its counters were left at zero)
        got2 = torch.full_like(q, float("nan"))
        assert L.rspx_trie_attn_noalloc(*_args(q, kp, vp, kn, vn, msk, got2), H, HK, M, P, NN, D, D ** -0.5,
                                        0, s) == 0
        torch.cuda.synchronize()
        assert torch.equal(got2, ref), name


def test_noalloc_wait_that_gives_up_is_reported_and_cleared():
    """The static scratch's timeout flag: read and cleared by rspx_trie_attn_status(NULL, ...)
    (no workspace pointer); a call whose waits give up (0 polls, forced from the host so every
    kernel exits normally) is reported once, and the next call on the same scratch is clean."""
    from respect_amd import _lib
    L = _lib.lib()
    s = _lib.stream_ptr(torch.device("cuda"))
    c = gen.cfg1(seed=5)
    q, kp, vp, kn, vn, msk = _tensors(c)
    H, HK, M, P, NN, D = _shape(q, kp, kn)
    print(f"[noalloc give-up] H={H} HK={HK} M={M} P={P} NN={NN} D={D}", flush=True)
    assert L.rspx_trie_attn_status(None, H, HK, M, P, D, s) == 0
    ref = torch.empty_like(q)
    assert L.rspx_trie_attn_noalloc(*_args(q, kp, vp, kn, vn, msk, ref), H, HK, M, P, NN, D, D ** -0.5, 0, s) == 0
    bad = torch.empty_like(q)
    prev = L.rspx_trie_attn_set_spin_limit(0)
    try:
        assert L.rspx_trie_attn_noalloc(*_args(q, kp, vp, kn, vn, msk, bad), H, HK, M, P, NN, D, D ** -0.5,
                                        0, s) == 0
    finally:
        L.rspx_trie_attn_set_spin_limit(prev)
    assert L.rspx_trie_attn_status(None, H, HK, M, P, D, s) == 1
    assert L.rspx_trie_attn_status(None, H, HK, M, P, D, s) == 0
    assert torch.isnan(bad.float()).all()
    good = torch.empty_like(q)
    assert L.rspx_trie_attn_noalloc(*_args(q, kp, vp, kn, vn, msk, good), H, HK, M, P, NN, D, D ** -0.5, 0, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(good, ref)
    assert L.rspx_trie_attn_status(None, H, HK, M, P, D, s) == 0


def test_noalloc_refuses_sizes_beyond_its_scratch():
    from respect_amd import _lib
    L = _lib.lib()
    H, HK, M, P, D = 32, 8, 1024, 3072, 128
    assert L.rspx_trie_attn_workspace_bytes(H, HK, M, P, D) > 32 << 20
    p = 1 << 20          # stand-in pointer: the call returns before any use
    rc = L.rspx_trie_attn_noalloc(p, M * D, D, p, P * D, D, p, P * D, D, p, 64 * D, D, p, 64 * D, D, p, 64, 1,
                                  p, M * D, D, H, HK, M, P, 64, D, D ** -0.5, 0, None)
    assert rc == -3
