"""Build the gfx950 shared library ``librespect_amd.so`` in-tree with hipcc.

The library is one C-ABI ``.so`` (no torch types in any signature) compiled from
every ``respect_amd/csrc/*.hip`` file.  It is written next to this file so that
it travels with the source tree; ``python -m respect_amd.build`` rebuilds it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "librespect_amd.so"
ARCH = "gfx950"

# -ffp-contract=off: every FMA in the kernels is explicit, so an expression
# compiles to the same instructions wherever it is inlined (bitwise invariance).
# The packed-fp32 feature is switched off: only scalar fp32 VALU instructions.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",
    # MFMA results in ordinary VGPRs: the softmax reads the QK scores and the
    # rare rescale touches the accumulators, so AGPR round trips cost more
    # than they save.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-result",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build respect_amd")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


TRACE_LIB = PKG / "librespect_amd_trace.so"


def build(verbose: bool = False, jobs: int = 8, trace: bool = False) -> Path:
    """Compile every kernel source and link ``librespect_amd.so`` (always rebuilds).
    ``trace``: the measurement variant ``librespect_amd_trace.so`` instead, built with
    -DRSPX_PHASE_TRACE (the one-launch attention records per-wave phase timestamps,
    read back by rspx_trie_attn_phase_trace; ``bench.py --phase-trace``)."""
    srcs = sources()
    lib_out = TRACE_LIB if trace else LIB
    flags = [*HIPCC_FLAGS, "-DRSPX_PHASE_TRACE"] if trace else HIPCC_FLAGS
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="rspx_build_") as td:
        objs, procs = [], []
        for src in srcs:
            obj = Path(td) / (src.stem + ".o")
            cmd = [cc, *flags, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
            while sum(p.poll() is None for _, p in procs) >= jobs:
                procs[0][1].wait()
        for src, p in procs:
            out, _ = p.communicate()
            msgs = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
            if p.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(msgs))
            if verbose and msgs:
                print("\n".join(msgs))
        tmp = lib_out.with_suffix(".so.tmp")
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
        os.replace(tmp, lib_out)
    return lib_out


def build_bench_floor(verbose: bool = False) -> Path:
    """Compile ``bench_floor.hip`` (repository root; bench-only launch-floor probes,
    not part of the product ABI) into ``bench_floor.so`` beside it."""
    src = ROOT / "bench_floor.hip"
    out = ROOT / "bench_floor.so"
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-shared", "-o", str(tmp), str(src)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on bench_floor.hip:\n" + r.stdout + r.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    if "--phase-trace" in sys.argv:
        print(build(verbose="-v" in sys.argv, trace=True))
    else:
        print(build(verbose="-v" in sys.argv))
        print(build_bench_floor(verbose="-v" in sys.argv))
