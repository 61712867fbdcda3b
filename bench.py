#!/usr/bin/env python3
"""Benchmark of the deterministic trie-verification kernels on one MI355X.

Default workload (the headline): trie-verification attention at the 8B decoder
shape -- 32 query heads, 8 kv heads, head_dim 128, bf16, 3072-token prompt KV,
64-node trie merged from 4 candidate sequences of 24 tokens whose shared
prefixes are uniform in [0, 16].  A step is one attention call over one input
set; 32 input sets (445 MB) rotate so the KV stream comes from HBM, not from
the 256 MB last-level cache.

Timing: W untimed warm-up calls, then K calls enqueued behind a GPU sleep so the
host never starves the queue; two HIP events on the launch stream bracket the K
back-to-back calls.  ms_per_step = GPU time of the K calls / K, and
roofline.achieved = algorithmic bytes per call / that time.  cpu_baseline times the reference
math on the host cores on one input set: fp32 masked SDPA in PyTorch on up to 16 threads,
and beside it the literal logical-order fold on one thread.

Prints ONE JSON line.  Only one GPU is used: --gpus N with N > 1 exits.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "trie-verify attn µs + % HBM peak (64 nodes, KV 3072, 8B shape); committed tok/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(launchers, steps: int, warmup: int) -> float:
    """Run launchers round-robin; return the average GPU time per launch in ms.

    Two HIP events on the launch stream bracket the K timed launches; a GPU
    sleep queued first keeps the device busy while the host enqueues them, so
    the region holds back-to-back kernels and no host gaps.
    """
    import torch
    n = len(launchers)
    for i in range(warmup):
        launchers[i % n]()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(max(steps, 1) * 20e-6 * 2.4e9) + 10_000_000)
    start.record()
    for i in range(steps):   # the rotation continues after the warm-up's sets
        launchers[(warmup + i) % n]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


CPU_SHARE = 16   # host CPUs allotted to one GPU's job on a shared multi-GPU host (its OMP_NUM_THREADS)


def cpu_counts() -> dict:
    """The host's logical CPU count, how many this process may run on (affinity) and
    the thread count the CPU baseline uses: the affinity count, at most the host's
    CPU share per GPU (CPU_SHARE; the rest of the host belongs to other GPUs' jobs)."""
    total = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        aff = total
    return {"os_cpu_count": total, "affinity_cpus": aff, "threads": max(1, min(CPU_SHARE, aff))}


def cpu_threads() -> int:
    return cpu_counts()["threads"]


def cpu_baseline_attn(wl, budget_s: float = 20.0) -> dict:
    """The reference math on the host cores, on input set 0 of the same workload.

    (i) the headline figure: vectorised fp32 masked SDPA in PyTorch (torch's CPU
        scaled_dot_product_attention, the prompt keys open to every row, node slots
        by the mask; GQA by repeating K/V), torch.set_num_threads(cpu_threads());
        3 warm-ups, then the median of up to 20 calls within the budget;
    (ii) beside it: the literal logical-order fold of respect/kernels/attention.py:36-71
        (the numpy oracle attn_hyb), one thread, median of a few calls.
    """
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import attention as A
    q, kp, vp, kn, vn = (t.float().cpu() for t in wl.sets[0])
    msk = wl.msk.cpu().bool()
    H, M, D = q.shape
    rep = H // kp.shape[0]
    K = torch.cat([kp, kn], 1).repeat_interleave(rep, 0).contiguous()
    V = torch.cat([vp, vn], 1).repeat_interleave(rep, 0).contiguous()
    allow = torch.cat([torch.ones(M, kp.shape[1], dtype=torch.bool), msk], 1)
    threads = cpu_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        def sdpa():
            return torch.nn.functional.scaled_dot_product_attention(q, K, V, attn_mask=allow, scale=wl.sm_scale)
        for _ in range(3):
            sdpa()
        times, t_end = [], time.perf_counter() + budget_s / 2
        while len(times) < 20 and (time.perf_counter() < t_end or len(times) < 3):
            t0 = time.perf_counter()
            sdpa()
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    med = statistics.median(times)
    qn, kpn, vpn, knn, vnn = (t.numpy() for t in (q, kp, vp, kn, vn))
    fold = []
    with threadpool_limits(limits=1):
        t_end = time.perf_counter() + budget_s / 2
        while len(fold) < 3 and (time.perf_counter() < t_end or not fold):
            t0 = time.perf_counter()
            A.attn_hyb(qn, kpn, vpn, knn, vnn, msk.numpy(), wl.sm_scale)
            fold.append(time.perf_counter() - t0)
    cc = cpu_counts()
    return {"value": round(med * 1e6, 1), "unit": "us per call", "cores": threads, "kind": "port",
            "os_cpu_count": cc["os_cpu_count"], "affinity_cpus": cc["affinity_cpus"],
            "sample": f"{len(times)} full calls of the 8B-shape 64-node attention on input set 0: fp32 masked "
                      f"SDPA in PyTorch on {threads} host threads (median)",
            "literal_fold": {"value": round(statistics.median(fold) * 1e6, 1), "unit": "us per call", "cores": 1,
                             "sample": f"{len(fold)} calls of the numpy logical-order fold of "
                                       "respect/kernels/attention.py:36-71 (one thread; median)"}}


def bench_attn(args) -> dict:
    import torch

    from respect_amd.kernels.attention import make_launcher
    from respect_amd.workloads import AttnWorkload

    _log("building 8B-shape attention workload")
    wl = AttnWorkload(sets=args.sets, seed=0)
    launchers, keep = [], []
    for (q, kp, vp, kn, vn) in wl.sets:
        launch, out = make_launcher(q, kp, vp, kn, vn, wl.msk, wl.sm_scale)
        launchers.append(launch)
        keep.append(out)
    _log(f"N={wl.N} nodes, NN={wl.NN}, P={wl.P}; timing {args.steps} steps after {args.warmup} warm-up")
    ms_step = time_launches(launchers, args.steps, args.warmup)
    kern_ms = ms_step
    nbytes = wl.algorithmic_bytes()
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    tflops = wl.flops() / (kern_ms * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": round(ms_step * 1e3, 3),
        "unit": "us per trie-verify attention call",
        "higher_is_better": False,
        "ms_per_step": ms_step,
        "hbm_frac_of_peak": round(achieved / HBM_PEAK_GBS, 4),
        "mfma_frac_of_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
        "dtype": "bf16",
        "config": {"workload": "trie-verification attention, 8B shape: 32 q / 8 kv heads, head_dim 128, "
                               "3072-token prompt KV, 64-node trie (4 seqs x 24, shared prefix U[0,16])",
                   "nodes": wl.N, "prompt_len": wl.P, "node_slots": wl.NN, "input_sets": len(wl.sets),
                   "algorithmic_bytes_per_call": nbytes, "flops_per_call": wl.flops()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "rspx::fused_kernel<128,2> (one launch per call)"},
    }
    if not args.no_cpu:
        _log("timing CPU baseline (oracle)")
        res["cpu_baseline"] = cpu_baseline_attn(wl, args.cpu_budget)
    return res


# One call is one fused_kernel launch when its grid fits on the device at once,
# else prompt_kernel then node_merge_kernel.
ATTN_KERNELS = ("rspx::fused_kernel", "rspx::prompt_kernel", "rspx::node_merge_kernel")
COPY_KERNEL = "__amd_rocclr_copyBuffer"
PROBE_COPY_BYTES = 1 << 28   # the probe's device copy: 256 MiB read + 256 MiB written


def traffic_probe(args) -> int:
    """Child run under rocprofv3 --pmc: 6 attention calls and one 256 MiB device copy."""
    import torch

    from respect_amd.kernels.attention import make_launcher
    from respect_amd.workloads import AttnWorkload
    wl = AttnWorkload(sets=2, seed=0)
    launchers = [make_launcher(*st, wl.msk, wl.sm_scale)[0] for st in wl.sets]
    for i in range(6):
        launchers[i % 2]()
    src = torch.ones(PROBE_COPY_BYTES // 2, device="cuda", dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    return 0


def counter_probe(args) -> int:
    """Child run for rocprofv3 --pmc (MFMA counters): per dispatch, in this order, three
    attention calls at 8B heads with a 3072-token prompt KV and tries of 16, 64 and 128
    nodes, then the 64-row linear layers of one 8B decoder layer (q/k/v [6144, 4096],
    o [4096, 4096], gate/up [24576, 4096], down [4096, 12288]) once each, with x and the
    weights in the tiled layouts the decoder step uses."""
    import torch

    from respect_amd import _lib
    from respect_amd.kernels.attention import make_launcher
    from respect_amd.kernels.gemm import tile_weight
    from respect_amd.workloads import AttnWorkload, merged_trie
    for n, seqs, length, lo, hi in ((16, 2, 10, 4, 4), (64, 4, 24, 0, 16), (128, 5, 32, 8, 8)):
        wl = AttnWorkload(P=3072, tree=merged_trie(7, seqs, length, lo, hi, n), sets=1, seed=n)
        launch, _ = make_launcher(*wl.sets[0], wl.msk, wl.sm_scale)
        launch()
        torch.cuda.synchronize()
        _log(f"counter probe: attention, {n} nodes")
    L = _lib.lib()
    dev = torch.device("cuda")
    s = _lib.stream_ptr(dev)
    x = torch.randn(64 * 12288, device=dev).to(torch.bfloat16)   # tiled [64, K] for K <= 12288
    T = _lib.RSPX_TILED
    for N, K in ((6144, 4096), (4096, 4096), (24576, 4096), (4096, 12288)):
        w = tile_weight((0.02 * torch.randn(N, K, device=dev)).to(torch.bfloat16))
        y = torch.empty(64, N, device=dev, dtype=torch.bfloat16)
        ws = torch.zeros(max(16, L.rspx_linear_workspace_bytes(64, N, K)), dtype=torch.uint8, device=dev)
        torch.cuda.synchronize()
        _lib.check("rspx_linear", L.rspx_linear(x.data_ptr(), T, w.data_ptr(), T, y.data_ptr(), N, 64, N, K, 0,
                                                ws.data_ptr(), ws.numel(), s))
        torch.cuda.synchronize()
        _log(f"counter probe: linear 64 x [{N}, {K}]")
    return 0


def measure_traffic(timeout_s: float = 180.0):
    """Memory traffic per attention call from two rocprofv3 PMC passes over a child
    run of this script (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled
    by what the counter reads for the child's 256 MiB device copy.  Runs before this
    process touches the GPU.  Returns None if rocprofv3 is missing or a pass fails."""
    import csv
    import shutil
    import signal
    import subprocess
    import tempfile
    exe = shutil.which("rocprofv3")
    if exe is None:
        return None
    per_kernel: dict = {}
    scale: dict = {}
    with tempfile.TemporaryDirectory() as td:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", td, "-o", counter,
                   "--", sys.executable, str(ROOT / "bench.py"), "--traffic-probe"]
            _log(f"traffic pass {counter}")
            proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                                    start_new_session=True)
            try:
                rc = proc.wait(timeout=timeout_s)
            except subprocess.TimeoutExpired:
                os.killpg(proc.pid, signal.SIGKILL)
                proc.wait()
                _log(f"traffic pass {counter} timed out")
                return None
            path = Path(td) / f"{counter}_counter_collection.csv"
            if rc != 0 or not path.exists():
                _log(f"traffic pass {counter} failed (rc={rc})")
                return None
            vals: dict = {}
            with open(path) as f:
                for row in csv.DictReader(f):
                    vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
            copy_kib = max(vals.get(COPY_KERNEL, [0.0]))
            if copy_kib <= 0:
                return None
            scale[counter] = PROBE_COPY_BYTES / 1024 / copy_kib
            for name, v in vals.items():
                for k in ATTN_KERNELS:
                    if k in name:
                        per_kernel.setdefault(k, {})[counter] = statistics.median(v) * 1024 * scale[counter]
    per_kernel = {k: v for k, v in per_kernel.items() if len(v) == 2}
    if not per_kernel:
        return None
    total = sum(v["FETCH_SIZE"] + v["WRITE_SIZE"] for v in per_kernel.values())
    return {"bytes": total, "scale": scale,
            "by_kernel": {k: {"fetch": round(v["FETCH_SIZE"]), "write": round(v["WRITE_SIZE"])}
                          for k, v in per_kernel.items()}}


def _launcher(fn, *args):
    """Bind a C entry point and its arguments into a zero-argument launch."""
    from respect_amd import _lib

    def launch():
        rc = fn(*args)
        if rc != 0:
            _lib.check(fn.__name__, rc)
    return launch


def bench_norm_rope(args) -> dict:
    """RMSNorm [64, 4096] + q/k RMSNorm-and-RoPE (q [64,32,128], k [64,8,128]),
    positions = 3072 + trie depth; bf16.  One launch per step (rspx_rmsnorm_qk_norm_rope);
    the two separate launches are timed beside it."""
    import torch

    from respect_amd import _lib
    from respect_amd.system.fused import rope_tables
    L = _lib.lib()
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    T, HID, HQ, HK, D = 64, 4096, 32, 8, 128
    sets = 256
    w = (1 + 0.02 * torch.randn(HID, generator=g, device=dev)).to(torch.bfloat16)
    wq = (1 + 0.02 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    wk = (1 + 0.02 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    depth = torch.randint(0, 24, (T,), generator=g, device=dev)
    cos, sin = rope_tables(3072 + depth, D, 1.0e6, device=dev)
    s = _lib.stream_ptr(dev)
    norm_l, qk_l, one_l, keep = [], [], [], []
    for _ in range(sets):
        x = torch.randn(T, HID, generator=g, device=dev).to(torch.bfloat16)
        q = torch.randn(T, HQ, D, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(T, HK, D, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty_like(x)
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        keep += [x, q, k, y, qo, ko]
        norm_l.append(_launcher(L.rspx_rmsnorm, x.data_ptr(), HID, w.data_ptr(), y.data_ptr(), HID, T, HID, 1e-6, s))
        qk_l.append(_launcher(L.rspx_qk_norm_rope, q.data_ptr(), HQ * D, D, k.data_ptr(), HK * D, D, wq.data_ptr(),
                              wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), D, qo.data_ptr(), ko.data_ptr(),
                              T, HQ, HK, D, 1e-6, s))
        one_l.append(_launcher(L.rspx_rmsnorm_qk_norm_rope, x.data_ptr(), HID, w.data_ptr(), y.data_ptr(), HID, T,
                               HID, 1e-6, q.data_ptr(), HQ * D, D, k.data_ptr(), HK * D, D, wq.data_ptr(),
                               wk.data_ptr(), cos.data_ptr(), sin.data_ptr(), D, qo.data_ptr(), ko.data_ptr(),
                               T, HQ, HK, D, 1e-6, s))
    tn = time_launches(norm_l, args.steps, args.warmup) * 1e-3
    tq = time_launches(qk_l, args.steps, args.warmup) * 1e-3
    t1 = time_launches(one_l, args.steps, args.warmup) * 1e-3
    bytes_norm = 2 * T * HID * 2 + HID * 2
    bytes_rope = (T * HQ * D + T * HK * D) * 2 * 2 + 2 * T * D * 2
    return {"workload": "RMSNorm [64,4096] + q/k RMSNorm+RoPE q[64,32,128] k[64,8,128], theta 1e6, bf16",
            "us_per_step": round(t1 * 1e6, 3), "launches": 1,
            "two_launches_us": round((tn + tq) * 1e6, 3),
            "rmsnorm_us": round(tn * 1e6, 3), "rmsnorm_GBps": round(bytes_norm / tn / 1e9, 1),
            "qk_norm_rope_us": round(tq * 1e6, 3), "qk_norm_rope_GBps": round(bytes_rope / tq / 1e9, 1),
            "algorithmic_bytes": bytes_norm + bytes_rope,
            "hbm_frac_of_peak": round((bytes_norm + bytes_rope) / t1 / 1e9 / HBM_PEAK_GBS, 4)}


def bench_swiglu(args) -> dict:
    """SwiGLU on a packed gate/up [64, 2 x 12288] -> [64, 12288], bf16."""
    import torch

    from respect_amd import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    T, F = 64, 12288
    sets = 64
    s = _lib.stream_ptr(dev)
    ls, keep = [], []
    for _ in range(sets):
        gu = torch.randn(T, 2 * F, generator=g, device=dev).to(torch.bfloat16)
        y = torch.empty(T, F, device=dev, dtype=torch.bfloat16)
        keep += [gu, y]
        ls.append(_launcher(L.rspx_silu_mul, gu.data_ptr(), 2 * F, gu.data_ptr() + 2 * F, 2 * F, y.data_ptr(), F,
                            T, F, s))
    t = time_launches(ls, args.steps, args.warmup) * 1e-3
    nbytes = T * F * 2 * 3
    return {"workload": "SwiGLU gate/up [64, 2x12288] -> [64, 12288], bf16", "us_per_step": round(t * 1e6, 3),
            "algorithmic_bytes": nbytes, "GBps": round(nbytes / t / 1e9, 1),
            "hbm_frac_of_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


def bench_prefill(args) -> dict:
    """Prefill / Flow element-wise kernels on [4096, 4096] bf16 rows (rotating sets beyond the
    MALL): add_sq, square, norm_apply (the kernel halves of rmsnorm / norm_from), and the
    vision RoPE on [4096, 16, 80]."""
    import torch

    from respect_amd import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    M, N, sets = 4096, 4096, 6
    s = _lib.stream_ptr(dev)
    bf, f32 = torch.bfloat16, torch.float32
    out, keep = {}, []

    def rec(name, launchers, nbytes):
        t = time_launches(launchers, args.steps // 2, args.warmup) * 1e-3
        out[name] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                     "hbm_frac_of_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}

    ls_add, ls_sq, ls_norm = [], [], []
    for _ in range(sets):
        r = torch.randn(M, N, generator=g, device=dev).to(bf)
        h = torch.randn(M, N, generator=g, device=dev).to(bf)
        x = torch.empty(M, N, device=dev, dtype=bf)
        sq = torch.empty(M, N, device=dev, dtype=f32)
        var = torch.rand(M, generator=g, device=dev) + 0.5
        w = (1 + 0.02 * torch.randn(N, generator=g, device=dev)).to(bf)
        y = torch.empty(M, N, device=dev, dtype=bf)
        keep += [r, h, x, sq, var, w, y]
        ls_add.append(_launcher(L.rspx_add_sq, r.data_ptr(), N, h.data_ptr(), N, x.data_ptr(), N, sq.data_ptr(), N,
                                M, N, s))
        ls_sq.append(_launcher(L.rspx_square, r.data_ptr(), N, sq.data_ptr(), N, M, N, s))
        ls_norm.append(_launcher(L.rspx_norm_apply, r.data_ptr(), N, var.data_ptr(), w.data_ptr(), y.data_ptr(), N,
                                 M, N, 1e-6, s))
    rec("add_sq", ls_add, M * N * (2 + 2 + 2 + 4))
    rec("square", ls_sq, M * N * (2 + 4))
    rec("norm_apply", ls_norm, M * N * (2 + 2) + M * 4 + N * 2)
    Lv, NH, D = 4096, 16, 80
    ls_rope = []
    for _ in range(sets):
        xv = torch.randn(Lv, NH, D, generator=g, device=dev).to(bf)
        cs = torch.randn(Lv, D, generator=g, device=dev)
        sn = torch.randn(Lv, D, generator=g, device=dev)
        yv = torch.empty(Lv, NH, D, device=dev, dtype=bf)
        keep += [xv, cs, sn, yv]
        ls_rope.append(_launcher(L.rspx_rope_vision, xv.data_ptr(), NH * D, D, cs.data_ptr(), sn.data_ptr(), D,
                                 yv.data_ptr(), Lv, NH, D, s))
    rec("rope_vision", ls_rope, Lv * NH * D * 4 + Lv * D * 8)
    out["workload"] = "rows [4096, 4096] bf16 (fp32 squares); vision RoPE x [4096, 16, 80], fp32 cos/sin"
    return out


def _target_trie(cont, rng, n_seqs=4, length=24, target_nodes=64, vocab=151936):
    """Trie of ``n_seqs`` candidates of ``length`` tokens rooted at cont[0]: one is
    the target's own greedy continuation ``cont``, the others share a prefix of
    it (length uniform in [1, 16]) and continue randomly; redrawn until the trie
    has ``target_nodes`` nodes."""
    from respect_amd.candidates.trie import build_trie
    for _ in range(10000):
        seqs = [list(cont[:length])]
        for _ in range(n_seqs - 1):
            p = int(rng.integers(1, 17))
            seqs.append(list(cont[:p]) + [int(t) for t in rng.integers(0, vocab, length - p)])
        tree = build_trie(seqs)
        if len(tree.nodes) == target_nodes:
            return tree
    return tree


def _distractor_trie(first, target_next, rng, nodes=64, vocab=151936):
    """``nodes`` nodes under the root ``first`` (sequences of 21 tokens, the last one cut to
    fit), none of whose children carries ``target_next``."""
    from respect_amd.candidates.trie import build_trie
    seqs = []
    while True:
        s = [first] + [int(t) for t in rng.integers(0, vocab, 20)]
        if s[1] == target_next:
            s[1] = (target_next + 1) % vocab
        have = len(build_trie(seqs).nodes) if seqs else 0
        grown = build_trie(seqs + [s])
        if len(grown.nodes) >= nodes:
            return build_trie(seqs + [s[:nodes - have + (1 if seqs else 0)]])
        seqs.append(s)


def bench_decoder(args) -> dict:
    """One speculative verification step of a random-init 36-layer 8B-shape GQA
    decoder (hidden 4096, 32 q / 8 kv heads, head_dim 128, FFN 12288 SwiGLU,
    vocab 151936, bf16 weights ~ N(0, 0.02)) over a 3072-token prompt KV built
    from random ids: a 64-node trie is verified in one forward, walked with the
    target's greedy choices, and the accepted path's KV compacted; then the
    same tokens are decoded one forward per token.  Tokens and committed KV
    must match bitwise; committed tok/s = accepted tokens / verification time.  The
    same number of distractor-only steps (tries that never continue past their root:
    one accepted token per step) is reported beside it."""
    import numpy as np
    import torch

    from respect_amd.decoding.acceptance import greedy_token
    from respect_amd.decoding.engine import Decoder, DecoderConfig
    from respect_amd.decoding.kv_buffer import KVCache
    from respect_amd.decoding.respect import respect_step
    from respect_amd.decoding.sequential import next_token

    cfg = DecoderConfig()
    P, steps = 3072, args.decoder_steps
    _log("decoder: random-initialising the 36-layer 8B-shape model")
    model = Decoder(cfg, seed=0, std=0.02)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab, (P,), generator=g).cuda()
    from respect_amd.decoding.verify import node_slots
    max_base = 24 * (steps + 2)
    nn_max = node_slots(max_base, 64, 64)
    cap = P + nn_max + 64                     # + scratch slots of the 64-row graphs
    caches = []
    t0 = time.perf_counter()
    for _ in range(2):
        c = KVCache(cfg.layers, cfg.kv_heads, cfg.head_dim, cap)
        last = model.prefill(prompt, c, chunk=512)
        caches.append(c)
    torch.cuda.synchronize()
    _log(f"decoder: prompt KV of {P} tokens built twice in {time.perf_counter() - t0:.1f} s")
    ar, sp = caches
    # HIP graphs of the forwards the run will replay (node segments padded to 64).
    t0 = time.perf_counter()
    for NN in range(64, nn_max + 1, 64):
        model.graphed(ar, P, 1, NN)
        model.graphed(sp, P, 64, NN)
    torch.cuda.synchronize()
    _log(f"decoder: {sum(len(v) for v in model._graphs.values())} forwards captured in {time.perf_counter() - t0:.1f} s")
    # Token-by-token greedy reference: the tokens the tries are built from.
    first = int(greedy_token(last).item())
    n_ar = 24 * (steps + 1) + steps + 2
    G = [first]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for c in range(n_ar):
        G.append(next_token(model, ar, G[-1], P, c))
    torch.cuda.synchronize()
    ar_ms = (time.perf_counter() - t0) / n_ar * 1e3
    _log(f"decoder: {n_ar} tokens decoded one by one, {ar_ms:.2f} ms per token")
    rng = np.random.default_rng(0)
    base, nxt, accepted, times, nodes, ok = 0, first, 0, [], [], True
    for step in range(steps + 1):          # step 0 is the warm-up
        tree = _target_trie(G[base:], rng)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        acc, rec, path = respect_step(model, sp, tree, nxt, P, base, eos=-1, graph=True)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t1
        ok &= acc == G[base:base + len(acc)] and rec == G[base + len(acc)]
        if step > 0:
            times.append(dt)
            accepted += len(acc)
            nodes.append(len(tree.nodes))
        base += len(acc)
        nxt = rec
    # Distractor-only tries: 64 nodes under the root whose children never carry the
    # target's next token, so each step accepts one token (the worst case).
    d_times, d_acc = [], 0
    for step in range(steps):
        tree = _distractor_trie(nxt, G[base + 1], rng)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        acc, rec, path = respect_step(model, sp, tree, nxt, P, base, eos=-1, graph=True)
        torch.cuda.synchronize()
        d_times.append(time.perf_counter() - t1)
        ok &= acc == G[base:base + len(acc)] and rec == G[base + len(acc)]
        d_acc += len(acc)
        base += len(acc)
        nxt = rec
    kv_equal = all(torch.equal(sp.k[i][:, P:P + base], ar.k[i][:, P:P + base]) and
                   torch.equal(sp.v[i][:, P:P + base], ar.v[i][:, P:P + base]) for i in range(cfg.layers))
    step_s = sum(times) / len(times)
    wbytes = cfg.weight_bytes()
    return {"workload": "speculative verification step, random-init 36-layer 8B-shape GQA decoder "
                        "(hidden 4096, 32q/8kv, hd128, FFN 12288, vocab 151936), 3072-token prompt KV, "
                        "64-node trie of 4 candidates x 24 tokens (one is the target's greedy continuation)",
            "steps": len(times), "trie_nodes": nodes, "ms_per_verify_step": round(step_s * 1e3, 3),
            "accepted_per_step": accepted / len(times),
            "committed_tok_s": round(accepted / sum(times), 1),
            "distractor_only": {"steps": len(d_times), "accepted_per_step": d_acc / max(1, len(d_times)),
                                "ms_per_verify_step": round(sum(d_times) / max(1, len(d_times)) * 1e3, 3),
                                "committed_tok_s": round(d_acc / max(sum(d_times), 1e-9), 1),
                                "trie": "64 nodes under the root, no child carries the target's next token"},
            "ar_ms_per_token": round(ar_ms, 3), "ar_tok_s": round(1e3 / ar_ms, 1),
            "weight_GBps_verify": round(wbytes / step_s / 1e9, 1),
            "tokens_equal_1token_decoding": bool(ok), "committed_kv_bitwise_equal": bool(kv_equal),
            "launch": "HIP graphs (one captured forward per node-segment width), both paths"}


# Trie shapes of the invariance sweep: (nodes, sequences, length, shared prefix lo, hi);
# depth <= 32, node counts exact.
SWEEP_TRIES = ((1, 1, 1, 0, 0), (8, 2, 5, 2, 2), (32, 2, 20, 8, 8), (64, 4, 24, 0, 16), (128, 5, 32, 8, 8))
SWEEP_PROMPTS = (1024, 3072, 8192, 16384)


def bench_sweep(args) -> dict:
    """µs per call and fraction of HBM peak of the 8B-shape attention over prompt lengths and
    trie sizes (rotating input sets beyond the last-level cache, as the headline line)."""
    from respect_amd.kernels.attention import make_launcher
    from respect_amd.workloads import AttnWorkload, merged_trie

    points = []
    for P in SWEEP_PROMPTS:
        for (n, seqs, length, lo, hi) in SWEEP_TRIES:
            per_set = 4 * 8 * 128 * P
            sets = int(min(64, max(2, -(-300_000_000 // per_set))))
            tree = merged_trie(7, seqs, length, lo, hi, n)
            wl = AttnWorkload(P=P, tree=tree, sets=sets, seed=P + n)
            launchers, keep = [], []
            for (q, kp, vp, kn, vn) in wl.sets:
                launch, out = make_launcher(q, kp, vp, kn, vn, wl.msk, wl.sm_scale)
                launchers.append(launch)
                keep.append(out)
            ms = time_launches(launchers, 100, 10)
            gbs = wl.algorithmic_bytes() / (ms * 1e-3) / 1e9
            pt = {"prompt_len": P, "nodes": n, "us": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                  "hbm_frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
            if n >= 16:
                pt["mfma_frac_of_peak"] = round(wl.flops() / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)
            points.append(pt)
            del wl, launchers, keep
    return {"workload": "8B-shape attention (32 q / 8 kv heads, head_dim 128), prompt lengths x trie sizes",
            "points": points}


COMMITTED = (0, 24, 48, 72, 200, 500)


def bench_committed(args) -> dict:
    """The 8B-shape call with committed slots before the 64-node trie in the node segment
    (the verify step's attention after earlier steps): µs per call for each count."""
    from respect_amd.kernels.attention import make_launcher
    from respect_amd.workloads import AttnWorkload

    points = []
    for base in COMMITTED:
        wl = AttnWorkload(sets=16, seed=base, base=base)
        launchers, keep = [], []
        for (q, kp, vp, kn, vn) in wl.sets:
            launch, out = make_launcher(q, kp, vp, kn, vn, wl.msk, wl.sm_scale)
            launchers.append(launch)
            keep.append(out)
        ms = time_launches(launchers, 100, 10)
        points.append({"committed": base, "node_slots": wl.NN, "us": round(ms * 1e3, 2)})
        del wl, launchers, keep
    return {"workload": "8B-shape attention, 3072-token prompt KV, 64-node trie after N committed node slots "
                        "(16 rotating input sets)", "points": points}


def bench_floor(args) -> dict:
    """What the 8B-shape attention launch costs before any arithmetic (bench_floor.so, a
    bench-only library built from bench_floor.hip):
    its grid (256 x 512 threads, 147 KB LDS) empty; streaming each workgroup's K/V share
    with every load in flight (196 KB per workgroup, each byte read by 4 row blocks, as the
    attention reads it; and 49 KB unique shares); and the attention's own 2-round
    direct-to-LDS load schedule without arithmetic.  32 rotating K/V sets (403 MB)."""
    import ctypes

    import torch

    from respect_amd import _lib
    so = Path(__file__).resolve().with_name("bench_floor.so")
    if not so.exists():
        raise RuntimeError("bench_floor.so is not built (__graft_entry__.build() builds it)")
    fl = ctypes.CDLL(str(so))
    fl.rspx_bench_floor_launch.restype = ctypes.c_int
    fl.rspx_bench_floor_launch.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    sets = [(torch.randn(8, 3072, 128, generator=g, device=dev).to(torch.bfloat16),
             torch.randn(8, 3072, 128, generator=g, device=dev).to(torch.bfloat16)) for _ in range(32)]
    out = torch.zeros(256 * 512, dtype=torch.int32, device=dev)
    s = _lib.stream_ptr(dev)
    res = {}
    for which, name in ((0, "empty_grid_us"), (1, "stream_196KB_per_wg_us"), (2, "stream_49KB_unique_us"),
                        (3, "ring_schedule_us")):
        ls = [_launcher(fl.rspx_bench_floor_launch, which, ctypes.c_void_p(k.data_ptr()),
                        ctypes.c_void_p(v.data_ptr()), 8, 3072, 128, ctypes.c_void_p(out.data_ptr()), s)
              for k, v in sets]
        res[name] = round(time_launches(ls, args.steps, args.warmup) * 1e3, 2)
    res["workload"] = ("the attention's 8B-shape grid over K/V [8, 3072, 128] bf16: empty, streaming, "
                       "and its own load schedule without arithmetic")
    return res


def bench_copy(args) -> dict:
    """Device-to-device copy of a 1 GiB bf16 buffer (torch's copy kernel): the
    measured HBM ceiling the kernels above are compared with, and the known-size
    kernel that scales rocprofv3's FETCH_SIZE/WRITE_SIZE counters."""
    import torch
    n = 1 << 29
    src = torch.ones(n, device="cuda", dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    t = time_launches([lambda: dst.copy_(src)], max(args.steps // 10, 10), 3) * 1e-3
    nbytes = 2 * n * 2
    return {"workload": "device copy of 1 GiB (read 1 GiB + write 1 GiB)", "us_per_step": round(t * 1e6, 1),
            "GBps": round(nbytes / t / 1e9, 1), "hbm_frac_of_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


PHASES = ("round 0 landed", "round 0 computed", "round 1 landed", "round 1 computed", "round 2 landed",
          "round 2 computed", "node loads issued, quarter (m, l) exchanged", "scaled quarters written",
          "quarter sums read", "node chunk into LDS", "partial stored and counted", "node partials",
          "counter wait", "merge", "merge rows stored (end)")


def phase_trace(args) -> int:
    """The one-launch attention's phase timeline at the headline shape, from the trace build
    (librespect_amd_trace.so, ``python -m respect_amd.build --phase-trace``): every wave
    records s_memrealtime (100 MHz) at 16 marks; after back-to-back calls over rotating
    input sets, the last call's marks are read back.  Per workgroup a phase ends when its
    last wave passes the mark; printed: the median over workgroups of each phase's length
    and of each mark's time after the earliest start."""
    import ctypes

    import numpy as np
    import torch

    from respect_amd import _lib
    trace_so = _lib.LIB_PATH.with_name("librespect_amd_trace.so")
    if not trace_so.exists():
        print("librespect_amd_trace.so is not built: python -m respect_amd.build --phase-trace", file=sys.stderr)
        return 2
    _lib.LIB_PATH = trace_so
    L = _lib.lib()
    L.rspx_trie_attn_phase_trace.restype = ctypes.c_int
    L.rspx_trie_attn_phase_trace.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    from respect_amd.kernels.attention import make_launcher
    from respect_amd.workloads import AttnWorkload
    committed = args.trace_committed
    wl = AttnWorkload(sets=args.sets, seed=committed, base=committed) if committed else AttnWorkload(sets=args.sets, seed=0)
    launchers = [make_launcher(*st, wl.msk, wl.sm_scale)[0] for st in wl.sets]
    for i in range(40):
        launchers[i % len(launchers)]()
    torch.cuda.synchronize()
    WGS, WAVES, MARKS = 1024, 8, 16
    buf = np.zeros(WGS * WAVES * MARKS, dtype=np.uint64)
    _lib.check("rspx_trie_attn_phase_trace", L.rspx_trie_attn_phase_trace(buf.ctypes.data, buf.size))
    nwg = 256
    t = buf.reshape(WGS, WAVES, MARKS)[:nwg].astype(np.int64)
    t0 = t[:, :, 0].min()
    ends = t.max(axis=1) - t0                     # [wg, mark]: last wave past the mark
    starts = t[:, :, 0].min(axis=1) - t0
    span = (ends[:, 15].max() - starts.min()) * 10 / 1000
    rows = []
    prev = starts
    for k in range(1, MARKS):
        d = (ends[:, k] - prev) * 10 / 1000       # 100 MHz ticks -> us
        rows.append({"phase": PHASES[k - 1], "median_us": round(float(np.median(d)), 2),
                     "max_us": round(float(d.max()), 2), "ends_at_us": round(float(np.median(ends[:, k])) / 100, 2)})
        prev = ends[:, k]
    out = {"workload": "8B-shape attention, 64-node trie, KV 3072"
                       + (f", after {committed} committed node slots" if committed else "")
                       + ": the last of 40 back-to-back calls",
           "workgroups": nwg, "start_spread_us": round(float(starts.max() - starts.min()) / 100, 2),
           "first_start_to_last_end_us": round(float(span), 2),
           "wg_length_median_us": round(float(np.median(ends[:, 15] - starts)) / 100, 2), "phases": rows}
    print(json.dumps(out), flush=True)
    for r in rows:
        print(f"  {r['phase']:<28} {r['median_us']:6.2f} us  (max {r['max_us']:6.2f}, ends at {r['ends_at_us']:6.2f})")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sets", type=int, default=32, help="rotating input sets")
    ap.add_argument("--workload", default="attn", choices=["attn"])
    ap.add_argument("--no-extra", action="store_true", help="skip the norm/RoPE and SwiGLU lines")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 PMC passes")
    ap.add_argument("--no-decoder", action="store_true", help="skip the 36-layer verification-step line")
    ap.add_argument("--decoder-steps", type=int, default=4, help="timed verification steps")
    ap.add_argument("--traffic-probe", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--phase-trace", action="store_true",
                    help="phase timeline of the headline call from the trace build (librespect_amd_trace.so)")
    ap.add_argument("--trace-committed", type=int, default=0,
                    help="with --phase-trace: that many committed node slots before the trie (extra.attn_committed)")
    ap.add_argument("--counter-probe", action="store_true",
                    help="a few attention and linear-layer dispatches for rocprofv3 --pmc (MFMA counters)")
    args = ap.parse_args()
    if args.traffic_probe:
        return traffic_probe(args)
    if args.counter_probe:
        return counter_probe(args)
    if args.phase_trace:
        return phase_trace(args)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the verification kernels run on a single MI355X "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        return 2
    t0 = time.time()
    traffic = None if args.no_traffic else measure_traffic()
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    res = bench_attn(args)
    if traffic is not None:
        res["roofline"]["traffic"] = round(traffic["bytes"])
        res["roofline"]["kernel"] = " + ".join(f"{k}<128,...>" for k in traffic["by_kernel"]) + " (one call)"
        res["roofline"]["traffic_detail"] = {
            "source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, scaled by a 256 MiB device copy",
            "scale": {k: round(v, 4) for k, v in traffic["scale"].items()}, "by_kernel": traffic["by_kernel"]}
    if not args.no_extra:
        _log("timing RMSNorm + q/k norm+RoPE and SwiGLU")
        res["extra"] = {"norm_rope": bench_norm_rope(args), "swiglu": bench_swiglu(args),
                        "copy": bench_copy(args)}
        _log("timing the attention launch floor")
        res["extra"]["attn_floor"] = bench_floor(args)
        _log("timing the Prefill / Flow element-wise kernels")
        res["extra"]["prefill"] = bench_prefill(args)
        _log("timing the attention sweep (prompt lengths x trie sizes)")
        res["extra"]["attn_sweep"] = bench_sweep(args)
        _log("timing the call with committed node slots")
        res["extra"]["attn_committed"] = bench_committed(args)
    if not args.no_decoder:
        dec = bench_decoder(args)
        res["committed_tok_s"] = dec["committed_tok_s"]
        res.setdefault("extra", {})["verify_step"] = dec
    res.update({"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "scaling": "weak",
                "vs_baseline": None, "data": "synthetic (seeded torch.randn / numpy tries)"})
    res["wall_s"] = round(time.time() - t0, 2)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
