"""Block shapes the kernels run, and the exact re-blocking into them.

The streaming kernel's tile is P ∈ {16, 32, 48, 64} output features wide and
walks a block's Q input features as K slabs, Q any multiple of 16 up to 256.
The reference GPU module accepts any block whose sides are multiples of 16
(ssalaad/efficient/ls_linear.py:114-117). A (q, p)-stored block with p > 64 or
q > 256 is therefore cut into (Q, P) sub-blocks: block-row `by` becomes the
p / P kernel rows by·(p/P) + h, each holding, for every block of the row, its
q / Q sub-blocks in column order (column col·(q/Q) + j). The sub-blocks tile
the block exactly, so the product is the same sum with the same terms; only
the order in which fp32 partial sums are added changes. Output columns are
unchanged (kernel row r covers columns r·P … r·P + P − 1 = by·p + h·P …).

The tiled kernels of many-token calls run square 16/32/64 blocks only; a call
with other blocks (16×32, 48-wide, fp32 64×64, cut wide blocks) runs on the
same matrix cut into the widest square blocks that tile its blocks exactly.
"""

from __future__ import annotations

import numpy as np
import torch

KERNEL_P = (64, 48, 32, 16)   # tile widths, widest first
MAX_Q = 256


def kernel_block_shape(p: int, q: int) -> tuple[int, int]:
    """(P, Q) the kernels run a (p, q) block as: the widest tile dividing p,
    and q itself up to MAX_Q, else its largest multiple-of-16 divisor ≤ MAX_Q."""
    P = next(w for w in KERNEL_P if p % w == 0)
    Q = q if q <= MAX_Q else max(d for d in range(16, MAX_Q + 1, 16) if q % d == 0)
    return P, Q


def prefill_square(P: int, Q: int, elem_bytes: int) -> bool:
    """Whether the tiled many-token kernels run (Q, P) blocks as they are:
    square 16, 32 or 64 (fp32: 16 or 32)."""
    return P == Q and P in (16, 32, 64) and not (elem_bytes == 4 and P == 64)


def square_block(P: int, Q: int, elem_bytes: int) -> int:
    """The widest square block the tiled kernels run (64, 32 or 16; fp32: 32
    or 16) that tiles a (Q, P) block exactly; a many-token call with other
    blocks runs on this re-blocked view of the same matrix."""
    for s in (64, 32, 16):
        if P % s == 0 and Q % s == 0 and not (elem_bytes == 4 and s == 64):
            return s
    return 0


def reblock(crow_h: np.ndarray, col_h: np.ndarray, values: torch.Tensor, p: int, q: int,
            P: int, Q: int):
    """Return (crow', col', values') of the same matrix in (Q, P) blocks:
    crow'/col' int32 NumPy arrays, values' (nnz', Q, P) on values' device."""
    fp, fq = p // P, q // Q
    NB = crow_h.shape[0] - 1
    counts = np.diff(crow_h.astype(np.int64))
    # new rows (by, h): every block of row by, in order, for each h
    order_k = []
    order_h = []
    for by in range(NB):
        ks = np.arange(crow_h[by], crow_h[by + 1])
        for h in range(fp):
            order_k.append(ks)
            order_h.append(np.full(ks.shape, h))
    k_idx = np.concatenate(order_k) if order_k else np.zeros(0, np.int64)
    h_idx = np.concatenate(order_h) if order_h else np.zeros(0, np.int64)
    new_counts = np.repeat(counts, fp) * fq
    crow2 = np.concatenate([[0], np.cumsum(new_counts)]).astype(np.int32)
    col2 = ((col_h.astype(np.int64)[k_idx] * fq)[:, None] + np.arange(fq)[None]).reshape(-1)
    nnz = values.shape[0]
    v5 = values.reshape(nnz, fq, Q, fp, P).permute(0, 3, 1, 2, 4)   # (k, h, j, Q, P)
    dev = values.device
    vals2 = v5[torch.from_numpy(k_idx).to(dev), torch.from_numpy(h_idx).to(dev)]
    return crow2, col2.astype(np.int32), vals2.reshape(-1, Q, P).contiguous()


def reblock_rows(rows: np.ndarray, fp: int) -> np.ndarray:
    """Kernel rows of the listed block-rows (each becomes fp consecutive rows)."""
    rows = np.asarray(rows, dtype=np.int64)
    return (rows[:, None] * fp + np.arange(fp)[None]).reshape(-1).astype(np.int32)
