"""Writes tests/golden/mfma_16x16x32_bf16.npz: inputs and MI355X outputs of
v_mfma_f32_16x16x32_bf16 (tests/golden/mfma_probe.hip, one MFMA per wave) on operands
shaped like the attention kernel's -- scores (q, k ~ N(0,1) bf16, a running fp32 sum)
and PV (v ~ N(0,1), p = 2^U(-25, 8) in bf16, a running fp32 sum).  Run on an MI355X:

    hipcc --offload-arch=gfx950 -O2 -shared -fPIC -o /tmp/mfma_probe.so tests/golden/mfma_probe.hip
    python tests/golden/make_mfma_fixture.py /tmp/mfma_probe.so
"""
import ctypes
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import bf16  # noqa: E402

N = 32   # problems (of 256 outputs) per kind


def main(so: str) -> None:
    lib = ctypes.CDLL(so)
    rng = np.random.default_rng(1)
    kinds = {
        "qk": (bf16.round_bf16(rng.standard_normal((N, 16, 32)).astype(np.float32)),
               bf16.round_bf16(rng.standard_normal((N, 32, 16)).astype(np.float32)),
               (rng.standard_normal((N, 16, 16)) * 5).astype(np.float32)),
        "pv": (bf16.round_bf16(rng.standard_normal((N, 16, 32)).astype(np.float32)),
               bf16.round_bf16(np.exp2(rng.uniform(-25, 8, (N, 32, 16))).astype(np.float32)),
               (rng.standard_normal((N, 16, 16)) * 50).astype(np.float32)),
    }
    out = {}
    for name, (a, b, c) in kinds.items():
        ab = torch.from_numpy(bf16.to_bits(a).view(np.int16)).cuda()
        bb = torch.from_numpy(bf16.to_bits(b).view(np.int16)).cuda()
        ct = torch.from_numpy(c).cuda()
        dt = torch.empty_like(ct)
        rc = lib.mfma_probe_launch(ctypes.c_void_p(ab.data_ptr()), ctypes.c_void_p(bb.data_ptr()),
                                   ctypes.c_void_p(ct.data_ptr()), ctypes.c_void_p(dt.data_ptr()), N, None)
        assert rc == 0
        torch.cuda.synchronize()
        out[f"{name}_a"] = bf16.to_bits(a)
        out[f"{name}_b"] = bf16.to_bits(b)
        out[f"{name}_c"] = c
        out[f"{name}_d"] = dt.cpu().numpy()
    np.savez_compressed(ROOT / "tests" / "golden" / "mfma_16x16x32_bf16.npz", **out)
    print("wrote", ROOT / "tests" / "golden" / "mfma_16x16x32_bf16.npz")


if __name__ == "__main__":
    main(sys.argv[1])
