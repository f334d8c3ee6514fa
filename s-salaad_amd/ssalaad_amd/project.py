"""Sparse projection of the compression loop on the GPU.

`project_S(M, n_keep, block_p, block_q)` replaces ssalaad/inference/egar.py:296-317
(`_project_S`): keep the `n_keep` blocks of largest Frobenius norm of M, as fp32,
zeros elsewhere. It runs `ssl_block_topk` (block sums of squares, a radix select
of the n_keep largest, the masked copy). Equal norms are taken in ascending
row-major block order (torch.topk leaves that order unspecified).
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
        with torch.cuda.device(dev):
            rc = lib.ssl_block_topk(
                M.data_ptr(), M.stride(0), rb, cb, block_p, block_q, dt, int(n_keep),
                norms.data_ptr(), keep.data_ptr(), out.data_ptr(), out.stride(0),
                _lib.stream_ptr(dev),
            )
        _lib.check(rc, "ssl_block_topk")
    return (out, keep[: rb * cb].view(rb, cb).bool(), norms[: rb * cb].view(rb, cb))


def project_S(M: torch.Tensor, n_keep: int, block_p: int, block_q: int) -> torch.Tensor:
    """Keep the ``n_keep`` blocks of largest Frobenius norm (egar.py:296-317)."""
    return block_topk(M, n_keep, block_p, block_q)[0]
