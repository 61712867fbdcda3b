"""The tiled activation layout of include/respect_amd.h (row stride RSPX_TILED)
as torch reshapes, for the tests: element (m, k) of A[M, K] sits at
((((m // 64) * (K // 32) + k // 32) * 4 + (m % 64) // 16) * 64 + m % 16 + 16 * ((k % 32) // 8)) * 8 + k % 8."""
import torch


def tiled_index(m: int, k: int, K: int) -> int:
    """The header's formula, written out."""
    return ((((m // 64) * (K // 32) + k // 32) * 4 + (m % 64) // 16) * 64 + m % 16 + 16 * ((k % 32) // 8)) * 8 + k % 8


def tiled_rows(M: int) -> int:
    return -(-M // 64) * 64


def to_tiled(a: torch.Tensor, fill: float = 0.0) -> torch.Tensor:
    """a [M, K] -> flat tiled buffer of tiled_rows(M) * K elements (rows past M = fill)."""
    M, K = a.shape
    R = tiled_rows(M)
    p = torch.full((R, K), fill, dtype=a.dtype, device=a.device)
    p[:M] = a
    return p.view(R // 64, 4, 16, K // 32, 4, 8).permute(0, 3, 1, 4, 2, 5).contiguous().view(-1)


def from_tiled(flat: torch.Tensor, M: int, K: int) -> torch.Tensor:
    """Inverse of to_tiled: the [M, K] rows of a tiled buffer."""
    R = tiled_rows(M)
    return flat[:R * K].view(R // 64, K // 32, 4, 4, 16, 8).permute(0, 2, 4, 1, 3, 5).reshape(R, K)[:M]
