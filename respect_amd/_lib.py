"""ctypes binding of ``librespect_amd.so`` (the C ABI declared in include/respect_amd.h).

torch is imported before the library is opened: the library then binds to the
HIP runtime torch already loaded (same SONAME), so torch's streams and device
pointers are valid handles for it.  There is no fallback: if the library is not
built, every kernel call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library will share)

LIB_PATH = Path(__file__).resolve().with_name("librespect_amd.so")

# Row stride value naming the tiled activation layout of x / y and the tiled
# weight layout of w (RSPX_TILED of include/respect_amd.h).
RSPX_TILED = -1

_c_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/respect_amd.h
SIGNATURES: dict[str, tuple] = {
    "rspx_strerror": (ctypes.c_char_p, [_i32]),
    "rspx_version": (ctypes.c_char_p, []),
    "rspx_trie_attn_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32]),
    "rspx_trie_attn": (_i32, [
        _c_p, _i64, _i64,          # q
        _c_p, _i64, _i64,          # kp
        _c_p, _i64, _i64,          # vp
        _c_p, _i64, _i64,          # kn
        _c_p, _i64, _i64,          # vn
        _c_p, _i64, _i64,          # msk
        _c_p, _i64, _i64,          # out
        _i32, _i32, _i32, _i32, _i32, _i32, _f32,   # H HK M P NN D scale
        _c_p, _i64, _i32,          # workspace, bytes, rows_per_wave
        _c_p,                      # stream
    ]),
    "rspx_trie_attn_launches": (_i32, [
        _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64,
        _c_p, _i64, _i64, _c_p, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _i32, _f32, _c_p, _i64, _i32, _i32, _c_p]),
    "rspx_trie_attn_status": (_i32, [_c_p, _i32, _i32, _i32, _i32, _i32, _c_p]),
    "rspx_trie_attn_set_spin_limit": (_i32, [_i32]),
    "rspx_blocked_attn": (_i32, [
        _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64,
        _c_p, _i64, _i64, _c_p, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _c_p]),
    "rspx_trie_attn_noalloc": (_i32, [
        _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _i64, _i64,
        _c_p, _i64, _i64, _c_p, _i64, _i64,
        _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _c_p]),
    "rspx_square": (_i32, [_c_p, _i64, _c_p, _i64, _i32, _i32, _c_p]),
    "rspx_add_sq": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _i64, _c_p, _i64, _i32, _i32, _c_p]),
    "rspx_norm_apply": (_i32, [_c_p, _i64, _c_p, _c_p, _c_p, _i64, _i32, _i32, _f32, _c_p]),
    "rspx_rope_vision": (_i32, [_c_p, _i64, _i64, _c_p, _c_p, _i64, _c_p, _i32, _i32, _i32, _c_p]),
    "rspx_rmsnorm": (_i32, [_c_p, _i64, _c_p, _c_p, _i64, _i32, _i32, _f32, _c_p]),
    "rspx_rope": (_i32, [_c_p, _i64, _i64, _i64, _c_p, _c_p, _i64, _i64, _c_p, _i32, _i32, _i32, _i32, _c_p]),
    "rspx_qk_norm_rope": (_i32, [_c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p,
                                 _i32, _i32, _i32, _i32, _f32, _c_p]),
    "rspx_rmsnorm_qk_norm_rope": (_i32, [_c_p, _i64, _c_p, _c_p, _i64, _i32, _i32, _f32,
                                         _c_p, _i64, _i64, _c_p, _i64, _i64, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _c_p,
                                         _i32, _i32, _i32, _i32, _f32, _c_p]),
    "rspx_silu_mul": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _i64, _i32, _i32, _c_p]),
    "rspx_linear_splits": (_i32, [_i32, _i32]),
    "rspx_linear_workspace_bytes": (_i64, [_i32, _i32, _i32]),
    "rspx_linear": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _i64, _i32, _i32, _i32, _i32, _c_p, _i64, _c_p]),
    "rspx_add_rmsnorm": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _c_p, _i64, _c_p, _i64, _i32, _i32, _f32, _c_p]),
    "rspx_qkv_rope_cache": (_i32, [_c_p, _i64, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i32, _c_p, _i64, _i64, _c_p, _i64,
                                   _i64, _c_p, _i32, _i32, _i32, _i32, _f32, _c_p]),
    "rspx_trie_mask": (_i32, [_c_p, _i32, _i32, _i32, _i32, _c_p, _i64, _c_p, _c_p]),
    "rspx_step_inputs": (_i32, [_c_p, _i32, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p, _c_p, _i64, _c_p]),
    "rspx_kv_compact": (_i32, [_c_p, _i32, _i32, _i32, _i64, _i64, _i32, _i32, _c_p, _i32, _c_p]),
    "rspx_argmax_workspace_bytes": (_i64, [_i32, _i32]),
    "rspx_argmax_rows": (_i32, [_c_p, _i64, _i32, _i32, _i32, _i32, _c_p, _c_p, _i64, _c_p]),
    "rspx_linear_partials": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _i32, _i32, _i32, _c_p]),
    "rspx_linear_silu": (_i32, [_c_p, _i64, _c_p, _i64, _c_p, _i64, _i32, _i32, _i32, _c_p]),
    "rspx_linear_tiled_weight_elems": (_i64, [_i32, _i32]),
    "rspx_linear_tile_weight": (_i32, [_c_p, _i64, _i32, _i32, _c_p, _c_p]),
    "rspx_add_rmsnorm_partials": (_i32, [_c_p, _i64, _c_p, _i32, _c_p, _c_p, _i64, _c_p, _i64, _i32, _i32, _f32,
                                         _c_p]),
    "rspx_qkv_rope_cache_partials": (_i32, [_c_p, _i32, _c_p, _c_p, _c_p, _c_p, _i64, _c_p, _i32, _c_p, _i64, _i64, _c_p,
                                            _i64, _i64, _c_p, _i32, _i32, _i32, _i32, _f32, _c_p]),
}

_lib = None


class RspxError(RuntimeError):
    """A nonzero status returned by the C ABI."""

    def __init__(self, fn: str, code: int):
        self.code = code
        super().__init__(f"{fn} failed: {strerror(code)} ({code})")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m respect_amd.build` (hipcc, gfx950)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def strerror(code: int) -> str:
    return lib().rspx_strerror(code).decode()


def check(fn: str, code: int) -> None:
    if code != 0:
        raise RspxError(fn, code)


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_WORKSPACES: dict = {}


def current_workspace(device: torch.device, tag: str = "attn") -> torch.Tensor | None:
    """The current stream's scratch of ``tag`` if one was made, else None."""
    stream = torch.cuda.current_stream(device)
    return _WORKSPACES.get((device.index, stream.cuda_stream, tag))


def workspace(device: torch.device, nbytes: int, tag: str = "attn") -> torch.Tensor:
    """Per-(device, stream, tag) scratch of at least ``nbytes`` bytes, grown on demand.

    Keyed by stream so that calls on different streams never share it; calls on
    one stream are ordered, so reuse is safe.
    """
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream, tag)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 256, 0 if ws is None else 2 * ws.numel())
        ws = torch.zeros(size, dtype=torch.uint8, device=device)  # the attention's sync words start at zero
        _WORKSPACES[key] = ws
    return ws
