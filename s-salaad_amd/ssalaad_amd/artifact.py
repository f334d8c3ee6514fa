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


NM_BLOCK = 32  # 2:4 blocks: 32 input × 32 output features


def nm24_pack(S: torch.Tensor) -> dict:
    """2:4-sparse dense S [n, m] (16-bit, on the GPU) → the kernels' packed blocks.

    At most two of every four consecutive entries of a row (input features
    4g .. 4g + 3) may be non-zero (the pattern ssalaad/inference/egar.py:285-293
    produces). The matrix is cut into 32×32 blocks (zero padded at the edges);
    blocks with a non-zero are stored row-major in the layout `ssl_nm24_block_bytes`
    documents: the two kept values of every group and their positions. Groups
    with fewer than two non-zeros keep zeros at unused positions.
    Returns {crow, col, active_rows (int32), blocks (uint8 [nnz, 1280]), NB, NBK}.
    """
    if S.dim() != 2:
        raise ValueError("S must be 2-D")
    if S.device.type != "cuda":
        raise ValueError("the 2:4 packer runs on a ROCm GPU device; move S there first")
    if S.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("2:4 S needs 16-bit values (bf16 or fp16)")
    return _nm24_pack(S)


def nm24_prefill_layout(blocks: torch.Tensor) -> torch.Tensor:
    """Packed 2:4 blocks (uint8 [nnz, ssl_nm24_block_bytes()]) → the same blocks
    in the layout the prefill row kernel reads (uint8 [nnz,
    ssl_nm24_prefill_block_bytes()], include/ssalaad_amd.h): per output column
    j, its 16 kept values in order, then one uint32 of position nibbles per
    column (i0 | i1 << 2 for each group, group 4h + q at bit 16h + 4q)."""
    nnz = blocks.shape[0]
    vals = blocks[:, :1024].contiguous().view(torch.int16).view(nnz, 16, 16, 2)   # [c][i][s]
    v = vals.permute(0, 1, 3, 2).reshape(nnz, 32, 16)                             # [j = 2c + s][i]
    ib = blocks[:, 1024:1280].view(nnz, 16, 8, 2).permute(0, 1, 3, 2).reshape(nnz, 32, 2, 4)
    shifts = torch.tensor([0, 4, 8, 12], dtype=torch.int32, device=blocks.device)
    idx16 = (ib.to(torch.int32) << shifts).sum(dim=-1)                            # [j][h]
    idx = torch.stack([idx16[..., 0] & 0xFF, idx16[..., 0] >> 8,
                       idx16[..., 1] & 0xFF, idx16[..., 1] >> 8], dim=-1)         # little-endian
    return torch.cat([v.contiguous().view(torch.uint8).view(nnz, 1024),
                      idx.to(torch.uint8).view(nnz, 128)], dim=1).contiguous()


def _nm24_pack(S: torch.Tensor) -> dict:
    n, m = S.shape
    if m % 4:
        raise ValueError(f"in_features {m} is not a multiple of 4 (2:4 groups)")
    P = NM_BLOCK
    NB, NBK = -(-n // P), -(-m // P)
    Sp = torch.zeros(NB * P, NBK * P, dtype=S.dtype, device=S.device)
    Sp[:n, :m] = S
    G = NBK * P // 4
    Sg = Sp.view(NB * P, G, 4)
    nz = Sg != 0
    if bool((nz.sum(-1) > 2).any()):
        raise ValueError("S is not 2:4: a group of four input features holds more than two non-zeros")
    # the (up to) two non-zero positions of each group, lowest first; empty
    # slots take other positions, whose values are zero
    key = nz.to(torch.int32) * (8 - torch.arange(4, device=S.device, dtype=torch.int32)) + (
        3 - torch.arange(4, device=S.device, dtype=torch.int32))
    idx = key.topk(2, dim=-1).indices.sort(dim=-1).values           # [rows, G, 2], i0 < i1
    vals = torch.gather(Sg, -1, idx)                                 # [rows, G, 2]
    ib = (idx[..., 0] | (idx[..., 1] << 2)).to(torch.uint8)          # [rows, G]
    # blocks: [by][bc] → values [c][i = 2·grp + slot][s], index [c][grp][s]
    v = vals.view(NB, 16, 2, NBK, 8, 2).permute(0, 3, 1, 4, 5, 2).reshape(NB, NBK, 512)
    x = ib.view(NB, 16, 2, NBK, 8).permute(0, 3, 1, 4, 2).reshape(NB, NBK, 256)
    blocks = torch.cat([v.contiguous().view(torch.uint8).view(NB, NBK, 1024), x], dim=-1)
    keep = nz.view(NB, P, NBK, 8, 4).any(dim=4).any(dim=3).any(dim=1)  # [NB, NBK]
    counts = keep.sum(dim=1)
    crow = torch.zeros(NB + 1, dtype=torch.int32, device=S.device)
    crow[1:] = counts.cumsum(0).to(torch.int32)
    col = keep.nonzero(as_tuple=False)[:, 1].to(torch.int32)
    active = (counts > 0).nonzero(as_tuple=False).squeeze(-1).to(torch.int32)
    return dict(crow=crow, col=col, active_rows=active, blocks=blocks[keep].contiguous(), NB=NB,
                NBK=NBK)
