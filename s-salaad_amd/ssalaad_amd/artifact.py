"""BSR encoding on the GPU (mirror of ssalaad/efficient/artifact.py:7-37).

`dense_to_bsr` keeps the reference's contract — dense (n, m) in, a
torch.sparse_bsr_tensor with int64 crow/col and (nnz, p, q) values out, a block
kept iff its L1 sum is > 0, blocks in row-major order, ValueError when the shape
is not divisible by the block — but computes the structure with the device
encoder of libssalaad_amd.so. `encode_for_kernels` returns the module's kernel
view directly (int32 crow/col, (nnz, q, p) values, active block-rows), the
conversion of ls_linear.py:89-97 fused into the same pass.
"""

from __future__ import annotations

import torch

from . import _lib


def factor_from_svd(U: torch.Tensor, sigma: torch.Tensor, Vh: torch.Tensor, rank: int):
    """Rank-``rank`` factors of ``U diag(sigma) Vh`` with sqrt(sigma) in each (artifact.py:7-17)."""
    r = min(rank, sigma.shape[0])
    sqrt_sigma = sigma[:r].sqrt()
    return (U[:, :r] * sqrt_sigma, sqrt_sigma.unsqueeze(1) * Vh[:r, :])


def _encode(S: torch.Tensor, block_p: int, block_q: int, want_bsr: bool, want_t: bool):
    if S.dim() != 2:
        raise ValueError("S must be 2-D")
    (n, m) = S.shape
    if n % block_p or m % block_q:
        raise ValueError(f"shape ({n}, {m}) not divisible by block ({block_p}, {block_q})")
    if S.device.type != "cuda":
        raise ValueError("the BSR encoder runs on a ROCm GPU device; move S there first")
    dt = _lib.dtype_code(S.dtype)
    if S.stride(-1) != 1:
        S = S.contiguous()
    NB, NBK = n // block_p, m // block_q
    dev = S.device
    lib = _lib.load()
    flags = torch.empty(max(NB * NBK, 1), dtype=torch.uint8, device=dev)
    crow = torch.empty(NB + 1, dtype=torch.int32, device=dev)
    active = torch.empty(max(NB, 1), dtype=torch.int32, device=dev)
    totals = torch.zeros(2, dtype=torch.int32, device=dev)
    stream = _lib.stream_ptr(dev)
    with torch.cuda.device(dev):
        rc = lib.ssl_bsr_encode_count(
            S.data_ptr(), S.stride(0), NB, NBK, block_p, block_q, dt, flags.data_ptr(),
            crow.data_ptr(), active.data_ptr(), totals.data_ptr(), stream,
        )
        _lib.check(rc, "ssl_bsr_encode_count")
        nnz, n_active = (int(v) for v in totals.cpu().tolist())
        col = torch.empty(max(nnz, 1), dtype=torch.int32, device=dev)
        vb = torch.empty((nnz, block_p, block_q), dtype=S.dtype, device=dev) if want_bsr else None
        vt = torch.empty((nnz, block_q, block_p), dtype=S.dtype, device=dev) if want_t else None
        rc = lib.ssl_bsr_encode_fill(
            S.data_ptr(), S.stride(0), NB, NBK, block_p, block_q, dt, flags.data_ptr(),
            crow.data_ptr(), col.data_ptr(), _lib.ptr(vb), _lib.ptr(vt), stream,
        )
        _lib.check(rc, "ssl_bsr_encode_fill")
    return crow, col[:nnz], vb, vt, active[:n_active]


def dense_to_bsr(S: torch.Tensor, block_p: int, block_q: int) -> torch.Tensor:
    """Dense (n, m) -> torch.sparse_bsr_tensor, as artifact.py:20-37."""
    crow, col, vb, _, _ = _encode(S, block_p, block_q, True, False)
    return torch.sparse_bsr_tensor(
        crow.to(torch.int64), col.to(torch.int64), vb, size=tuple(S.shape)
    )


def encode_for_kernels(S: torch.Tensor, block_p: int, block_q: int):
    """Dense (n, m) -> (crow int32, col int32, values (nnz, q, p), active_rows int32)."""
    crow, col, _, vt, active = _encode(S, block_p, block_q, False, True)
    return crow, col, vt, active
