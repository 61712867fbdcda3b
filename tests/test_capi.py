"""The C-ABI library loads, exports every symbol the header declares, and rejects bad
arguments with its documented codes before touching the GPU (CPU-only test)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "respect_amd.h").read_text()
    return sorted(set(re.findall(r"\b(rspx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from respect_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("librespect_amd.so not built")
    return _lib.lib()


def test_header_symbols_exported(lib):
    names = _declared()
    assert "rspx_trie_attn" in names
    raw = ctypes.CDLL(str(ROOT / "respect_amd" / "librespect_amd.so"))
    for n in names:
        assert hasattr(raw, n), n


def test_python_binding_covers_header():
    from respect_amd import _lib
    assert set(_declared()) <= set(_lib.SIGNATURES)


def test_version_and_errors(lib):
    assert b"gfx950" in lib.rspx_version()
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.rspx_strerror(code)


def _attn(lib, H=32, HK=8, M=4, P=64, NN=32, D=128, ws=1 << 30, ptr=16, stride=128):
    p = ptr
    return lib.rspx_trie_attn(p, stride * M, stride, p, stride * P, stride, p, stride * P, stride,
                              p, stride * NN, stride, p, stride * NN, stride, p, NN, 1,
                              p, stride * M, stride, H, HK, M, P, NN, D, 0.088,
                              p, ws, 0, None)


def test_attn_argument_errors(lib):
    assert _attn(lib, H=12, HK=8) == -1          # H not a multiple of HK
    assert _attn(lib, D=96) == -2                 # head_dim not built
    assert _attn(lib, H=24, HK=8) == -2           # GQA 3
    assert _attn(lib, ws=16) == -3                # workspace too small
    assert _attn(lib, ptr=8) == -4                # misaligned pointer
    assert _attn(lib, stride=100) == -4           # stride not a multiple of 8
    assert _attn(lib, M=0) == 0                   # nothing to do, no launch
    assert _attn(lib, NN=4104) == -1              # node segment beyond NMAX = 4096
    assert _attn(lib, M=17000, P=3072, ws=1 << 40) == -2   # group partials past 2^31 bytes
    assert lib.rspx_trie_attn_workspace_bytes(32, 8, 64, 3072, 128) > 65536
    assert lib.rspx_trie_attn_workspace_bytes(32, 8, 64, 3072, 96) < 0


def test_step_inputs_argument_checks(lib):
    p = 1 << 20           # stand-in pointer: every call below returns before using it
    assert lib.rspx_step_inputs(p, -1, 0, 32, 0, 10, p, p, p, p, 32, None) == -1     # T < 0
    assert lib.rspx_step_inputs(p, 4, 0, 0, 0, 10, p, p, p, p, 32, None) == -1       # NN < 1
    assert lib.rspx_step_inputs(p, 4, 0, 32, 0, 10, p, p, p, p, 16, None) == -1      # mask row stride < NN
    assert lib.rspx_step_inputs(p, 4, 0, 32, 0, 0, p, p, p, p, 32, None) == -1       # empty vocabulary
    assert lib.rspx_step_inputs(None, 4, 0, 32, 0, 10, p, p, p, p, 32, None) == -1   # no descriptor
    assert lib.rspx_step_inputs(p, 0, 0, 32, 0, 10, p, p, p, p, 32, None) == 0       # nothing to do
