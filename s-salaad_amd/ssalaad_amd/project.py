"""Sparse projections of the compression loop on the GPU.

`project_S(M, n_keep, block_p, block_q)` replaces ssalaad/inference/egar.py:296-317
(`_project_S`): keep the `n_keep` blocks of largest Frobenius norm of M, as fp32,
zeros elsewhere. It runs `ssl_block_topk` (block sums of squares, a radix select
of the n_keep largest, the masked copy). Equal norms are taken in ascending
row-major block order (torch.topk leaves that order unspecified).

`project_S_nm(R, nm_n, nm_m)` replaces egar.py:284-292 (`_project_S_nm`): in
each run of nm_m consecutive entries of a row keep the nm_n of largest
magnitude, R.float() · mask. It runs `ssl_project_nm` (one thread per group).
Equal magnitudes go to the lower index.
"""

from __future__ import annotations

import torch

from . import _lib


def block_topk(M: torch.Tensor, n_keep: int, block_p: int, block_q: int):
    """(kept fp32 matrix, keep mask [rb, cb] bool, block sums of squares [rb, cb] fp32)."""
    if M.dim() != 2:
        raise ValueError("M must be 2-D")
    if M.device.type != "cuda":
        raise ValueError("the block projection runs on a ROCm GPU device; move M there first")
    n, m = M.shape
    if block_p <= 0 or block_q <= 0 or n % block_p or m % block_q:
        raise RuntimeError(
            f"shape '[{n // max(block_p, 1)}, {block_p}, {m // max(block_q, 1)}, {block_q}]' is "
            f"invalid for input of size {n * m}"
        )
    dt = _lib.dtype_code(M.dtype)
    if M.stride(-1) != 1:
        M = M.contiguous()
    rb, cb = n // block_p, m // block_q
    dev = M.device
    norms = torch.empty(max(rb * cb, 1), dtype=torch.float32, device=dev)
    keep = torch.empty(max(rb * cb, 1), dtype=torch.uint8, device=dev)
    out = torch.empty(n, m, dtype=torch.float32, device=dev)
    if rb * cb > 0:
        lib = _lib.load()
        ws_bytes = lib.ssl_block_topk_workspace_size(rb * cb)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = lib.ssl_block_topk(
                M.data_ptr(), M.stride(0), rb, cb, block_p, block_q, dt, int(n_keep),
                norms.data_ptr(), keep.data_ptr(), out.data_ptr(), out.stride(0),
                ws.data_ptr(), ws_bytes, _lib.stream_ptr(dev),
            )
        _lib.check(rc, "ssl_block_topk")
    # the kernels write keep bytes of exactly 0 and 1: a bool view, no copy
    return (out, keep[: rb * cb].view(rb, cb).view(torch.bool), norms[: rb * cb].view(rb, cb))


def project_S(M: torch.Tensor, n_keep: int, block_p: int, block_q: int) -> torch.Tensor:
    """Keep the ``n_keep`` blocks of largest Frobenius norm (egar.py:296-317)."""
    return block_topk(M, n_keep, block_p, block_q)[0]


def project_nm(R: torch.Tensor, nm_n: int, nm_m: int):
    """(R.float() · mask, keep mask [n, m] bool) of egar.py:284-292."""
    if R.dim() != 2:
        raise ValueError("R must be 2-D")
    if R.device.type != "cuda":
        raise ValueError("the N:M projection runs on a ROCm GPU device; move R there first")
    n, m = R.shape
    if nm_m <= 0 or m % nm_m:
        # the reference's R.float().view(n, m // nm_m, nm_m)
        raise RuntimeError(
            f"shape '[{n}, {m // max(nm_m, 1)}, {nm_m}]' is invalid for input of size {n * m}"
        )
    if not 0 <= nm_n <= nm_m:
        raise RuntimeError("selected index k out of range")  # topk(nm_n) over nm_m entries
    if R.stride(-1) != 1:
        R = R.contiguous()
    out = torch.empty(n, m, dtype=torch.float32, device=R.device)
    keep = torch.empty(n, m, dtype=torch.uint8, device=R.device)
    if n * m:
        lib = _lib.load()
        with torch.cuda.device(R.device):
            rc = lib.ssl_project_nm(R.data_ptr(), R.stride(0), n, m, int(nm_n), int(nm_m),
                                    _lib.dtype_code(R.dtype), out.data_ptr(), out.stride(0),
                                    keep.data_ptr(), keep.stride(0), _lib.stream_ptr(R.device))
        _lib.check(rc, "ssl_project_nm")
    return out, keep.view(torch.bool)  # keep bytes of exactly 0 and 1


def project_S_nm(R: torch.Tensor, nm_n: int, nm_m: int) -> torch.Tensor:
    """Keep the nm_n largest entries in each consecutive group of nm_m (egar.py:284-292)."""
    return project_nm(R, nm_n, nm_m)[0]
