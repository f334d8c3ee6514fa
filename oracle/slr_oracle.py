"""CPU oracle for the sparse-plus-low-rank (SLR) linear hot path.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and never
as the thing measured or shipped. The product path (ssalaad_amd) never calls it.

It restates, in NumPy (float64 unless stated), what the reference computes:

  dense_to_bsr          ssalaad/efficient/artifact.py:20-37
  module_buffers        ssalaad/efficient/ls_linear.py:86-97
  bsr_addmm_inplace     ssalaad/tilelang_sparse/addmm_inplace.py:59-82 and
                        ssalaad/cpu_sparse/bsr_addmm_avx2.cpp:67-140
  slr_linear            ssalaad/efficient/ls_linear.py:38-44,124-137,155-164
  slr_linear_ref_rounding  the bf16 rounding points of ls_linear.py:131-137
                        (F.linear outputs in bf16, fp32 accumulation of the
                        sparse term from the bf16 output, bias add in bf16)
  factor_from_svd       ssalaad/efficient/artifact.py:7-17
  project_blocks        ssalaad/inference/egar.py:296-317 (_project_S): keep the
                        n_keep blocks of largest Frobenius norm (fp32 input,
                        equal norms taken in ascending row-major block order)
  project_nm            ssalaad/inference/egar.py:284-292 (_project_S_nm): in
                        each run of nm_m consecutive entries of a row keep the
                        nm_n of largest magnitude; out = R.float() · mask

How each function is pinned (tests/test_oracle.py):
  * dense_to_bsr        vs torch.Tensor.to_sparse_bsr (the library routine the
                        reference's own test uses, tests/test_ssalaad.py:307-317)
                        plus the NaN/negative-zero special cases of the L1 rule;
  * bsr_addmm_inplace   vs the reference AVX2 kernel compiled from its source
                        (oracle/_ref, golden fixtures under tests/golden), vs the
                        closed form x @ S.T (tests/test_ssalaad.py:320-327), vs a
                        pure-Python loop on tiny inputs, and the untouched-rows
                        invariant (tests/test_ssalaad.py:330-337);
  * slr_linear          vs x @ (A @ B + S).T + b with S densified independently
                        (the bundle test's formula, tests/test_ssalaad.py:229-259);
  * slr_linear_ref_rounding  vs slr_linear within bf16 tolerance and exactly
                        equal on inputs whose every intermediate is representable;
  * factor_from_svd     A @ B reconstructs a rank-r matrix; rank 0 gives empty
                        factors (tests/test_ssalaad.py:276-283).
  * project_blocks      the reference's own case (tests/test_ssalaad.py:215-221),
                        the selection torch.topk makes on tie-free inputs (the
                        routine _project_S calls), brute force over every subset
                        on tiny inputs, and the clamping of n_keep (egar.py:304-306).
                        Which of several EQUAL norms survive is parity unpinned:
                        torch.topk does not specify it; the oracle and the GPU
                        take the lowest block index.
  * project_nm          vs the routine _project_S_nm calls (torch.topk over
                        |R| in groups, then scatter and multiply) on tie-free
                        inputs, brute force over every subset of tiny groups,
                        the closed forms nm_n = nm_m (R·1) and nm_n = 0 (R·0,
                        so −0 and NaN survive as the multiply leaves them), and
                        the reference's 2:4 case. Which of EQUAL magnitudes
                        survive is parity unpinned (torch.topk leaves it
                        unspecified); the oracle and the GPU take the lower
                        index. A NaN counts as the largest magnitude.
"""

from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------- bfloat16 --


def bf16_round(a) -> np.ndarray:
    """Round float values to the nearest bfloat16 (ties to even); float32 result."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    out = (r.astype(np.uint32) << 16).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out.reshape(f.shape)


def bf16_bits(a) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float values."""
    f = np.ascontiguousarray(bf16_round(a))
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


# ---------------------------------------------------------------- structure --


def dense_to_bsr(S: np.ndarray, block_p: int, block_q: int):
    """Dense (n, m) -> (crow int64 [NB+1], col int64 [nnz], values [nnz, p, q]).

    artifact.py:20-37: blocks are taken row-major; a block is kept iff the sum of
    the absolute values over it is > 0 (NaN sums compare false, so a block holding
    a NaN is dropped); crow is the cumulative count per block-row.
    """
    S = np.asarray(S)
    n, m = S.shape
    if n % block_p or m % block_q:
        raise ValueError(f"shape ({n}, {m}) not divisible by block ({block_p}, {block_q})")
    rb, cb = n // block_p, m // block_q
    blocks = S.reshape(rb, block_p, cb, block_q).transpose(0, 2, 1, 3)
    with np.errstate(invalid="ignore", over="ignore"):
        l1 = np.abs(blocks.astype(np.float64)).reshape(rb, cb, -1).sum(axis=-1)
        mask = l1 > 0
    crow = np.zeros(rb + 1, dtype=np.int64)
    crow[1:] = np.cumsum(mask.sum(axis=1))
    rows, cols = np.nonzero(mask)  # row-major order
    values = np.ascontiguousarray(blocks[rows, cols])
    return crow, cols.astype(np.int64), values


def module_buffers(crow, col, values):
    """BSR -> the kernel view of ls_linear.py:89-97.

    Returns (crow int32, col int32, values transposed to (nnz, q, p), active
    block-rows int32 ascending).
    """
    crow = np.asarray(crow)
    crow32 = crow.astype(np.int32)
    col32 = np.asarray(col).astype(np.int32)
    values_t = np.ascontiguousarray(np.asarray(values).transpose(0, 2, 1))
    active = np.nonzero(crow[1:] - crow[:-1])[0].astype(np.int32)
    return crow32, col32, values_t, active


def bsr_to_dense(crow, col, values, n: int, m: int) -> np.ndarray:
    """(crow, col, values (nnz, p, q)) -> dense (n, m) float64: block k of
    block-row by (crow[by] <= k < crow[by+1]) lands at rows by·p.., columns
    col[k]·q.. (the BSR layout of torch.sparse_bsr_tensor). n and m are
    multiples of p and q."""
    values = np.asarray(values, dtype=np.float64)
    crow = np.asarray(crow, dtype=np.int64)
    p, q = values.shape[1], values.shape[2]
    NB, NBK = n // p, m // q
    rows = np.repeat(np.arange(len(crow) - 1), np.diff(crow))
    S4 = np.zeros((NB, NBK, p, q), dtype=np.float64)
    S4[rows, np.asarray(col, dtype=np.int64)] = values
    return np.ascontiguousarray(S4.transpose(0, 2, 1, 3)).reshape(n, m)


# -------------------------------------------------------------- arithmetic --


def bsr_addmm_inplace(out, x, crow, col, values_t, active_rows) -> np.ndarray:
    """out[:, by·p:(by+1)·p] += Σ_blocks x[:, col·q:(col+1)·q] @ values_t[blk].

    addmm_inplace.py:69-82: one accumulator per active block-row, initialised
    from out, blocks walked in col order, written back; block-rows not listed in
    active_rows are left untouched (tests/test_ssalaad.py:330-337). Computed in
    float64 and returned as float64 (the caller rounds to its dtype).
    """
    out = np.array(out, dtype=np.float64, copy=True)
    x = np.asarray(x, dtype=np.float64)
    values_t = np.asarray(values_t, dtype=np.float64)
    q, p = values_t.shape[1], values_t.shape[2]
    for by in np.asarray(active_rows):
        by = int(by)
        acc = out[:, by * p : (by + 1) * p].copy()
        for ji in range(int(crow[by]), int(crow[by + 1])):
            c = int(col[ji])
            acc += x[:, c * q : (c + 1) * q] @ values_t[ji]
        out[:, by * p : (by + 1) * p] = acc
    return out


def slr_linear(x, A, B, S_dense, bias=None) -> np.ndarray:
    """Closed form y = x·Bᵀ·Aᵀ + x·Sᵀ + b in float64 (ls_linear.py:38-44,155-164)."""
    x = np.asarray(x, dtype=np.float64)
    y = (x @ np.asarray(B, dtype=np.float64).T) @ np.asarray(A, dtype=np.float64).T
    y = y + x @ np.asarray(S_dense, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def slr_linear_bsr(x, A, B, crow, col, values_t, active_rows, bias=None) -> np.ndarray:
    """The same closed form, with the sparse term taken from the kernel buffers."""
    x = np.asarray(x, dtype=np.float64)
    y = (x @ np.asarray(B, dtype=np.float64).T) @ np.asarray(A, dtype=np.float64).T
    y = bsr_addmm_inplace(y, x, crow, col, values_t, active_rows)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def slr_linear_ref_rounding(x, A, B, crow, col, values_t, active_rows, bias=None) -> np.ndarray:
    """bf16 emulation of the reference's rounding points (ls_linear.py:131-137).

    latent = bf16(x·Bᵀ); y = bf16(latent·Aᵀ); y = bf16(fp32(y) + Σ blocks) (the
    BSR op accumulates from out in fp32, addmm_inplace.py:72-82); y = bf16(y + b).
    Products are accumulated in float64 before each rounding (the library GEMM's
    own summation order is not specified by the reference).
    """
    x = np.asarray(x, dtype=np.float64)
    t = bf16_round(x @ np.asarray(B, dtype=np.float64).T).astype(np.float64)
    y = bf16_round(t @ np.asarray(A, dtype=np.float64).T).astype(np.float64)
    y = bf16_round(bsr_addmm_inplace(y, x, crow, col, values_t, active_rows)).astype(np.float64)
    if bias is not None:
        y = bf16_round(y + np.asarray(bias, dtype=np.float64)).astype(np.float64)
    return y


def factor_from_svd(U, sigma, Vh, rank: int):
    """artifact.py:7-17: A = U[:, :r]·√σ, B = √σ·Vh[:r] with r = min(rank, len(σ))."""
    r = min(rank, len(sigma))
    s = np.sqrt(np.asarray(sigma[:r], dtype=np.float64))
    return np.asarray(U)[:, :r] * s, s[:, None] * np.asarray(Vh)[:r, :]


# ---------------------------------------------------------------- metrics --


def project_blocks(M, n_keep: int, block_p: int, block_q: int):
    """(kept fp32 matrix, keep mask [rb, cb]) of egar.py:296-317.

    The block norms are sums of squares of the fp32 values, accumulated in
    float64 here (the reference sums in fp32; the selections agree unless two
    norms at the threshold are closer than fp32 rounding). NaN norms count as
    the largest. Equal norms: ascending row-major block order.
    """
    Mf = np.asarray(M, dtype=np.float32)
    n, m = Mf.shape
    rb, cb = n // block_p, m // block_q
    n_keep = min(max(int(n_keep), 0), rb * cb)
    keep = np.zeros(rb * cb, dtype=bool)
    if n_keep > 0:
        blk = Mf.astype(np.float64).reshape(rb, block_p, cb, block_q)
        norms = (blk * blk).sum(axis=(1, 3)).reshape(-1)
        key = np.where(np.isnan(norms), np.inf, norms)
        nan_first = np.isnan(norms)
        # sort by (NaN first, then larger norm first, then lower index first)
        order = np.lexsort((np.arange(rb * cb), -key, ~nan_first))
        keep[order[:n_keep]] = True
    keep = keep.reshape(rb, cb)
    mask = np.repeat(np.repeat(keep, block_p, axis=0), block_q, axis=1)
    return np.where(mask, Mf, np.float32(0)).astype(np.float32), keep


def project_nm(R, nm_n: int, nm_m: int):
    """(R.float()·mask, mask) of egar.py:284-292: in each run of nm_m
    consecutive entries along a row, the nm_n of largest |R| are kept (mask 1).
    NaN magnitudes count as the largest; equal magnitudes: lower index first.
    Dropped entries are R·0 as the reference's multiply leaves them (−0 for
    negative values, NaN for NaN and ±inf)."""
    Rf = np.asarray(R, dtype=np.float32)
    n, m = Rf.shape
    if nm_m <= 0 or m % nm_m:
        raise ValueError("m must be a multiple of nm_m")
    if not 0 <= nm_n <= nm_m:
        raise ValueError("nm_n must lie in [0, nm_m]")
    R3 = Rf.reshape(n, m // nm_m, nm_m)
    mag = np.abs(R3)
    key = np.where(np.isnan(mag), np.inf, mag).astype(np.float64)
    nan = np.isnan(mag)
    # rank of each entry in its group: entries that come before it in the
    # order (NaN first, then larger magnitude, then lower index)
    idx = np.arange(nm_m)
    before = (
        (nan[..., :, None] & ~nan[..., None, :])
        | ((nan[..., :, None] == nan[..., None, :])
           & ((key[..., :, None] > key[..., None, :])
              | ((key[..., :, None] == key[..., None, :]) & (idx[:, None] < idx[None, :]))))
    )  # before[..., k, j]: entry k precedes entry j
    rank = before.sum(axis=-2)
    mask = rank < nm_n
    out = (R3 * mask.astype(np.float32)).astype(np.float32)
    return out.reshape(n, m), mask.reshape(n, m)


def max_abs_normalised_error(y, y_ref) -> float:
    """max|y − y_ref| / max|y_ref| (0 when both are zero)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    den = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    num = float(np.max(np.abs(y - y_ref))) if y_ref.size else 0.0
    if den == 0.0:
        return num
    return num / den


# ---------------------------------------------------------- synthetic data --


def random_block_structure(NB: int, NBK: int, density: float, rng: np.random.Generator):
    """Exactly round(d·NB·NBK) distinct block slots, uniform, sorted row-major."""
    total = NB * NBK
    k = int(round(density * total))
    slots = np.sort(rng.permutation(total)[:k])
    return slots // NBK, slots % NBK


def zipf_block_structure(NB: int, NBK: int, density: float, rng: np.random.Generator, s: float = 1.2):
    """Per-row block counts ∝ rank^-s over a random permutation of the rows,
    water-filled to the mean density under the cap NBK; columns uniform per row."""
    target = int(round(density * NB * NBK))
    w = np.arange(1, NB + 1, dtype=np.float64) ** (-s)
    w = w[rng.permutation(NB)]
    counts = np.zeros(NB, dtype=np.int64)
    remaining = target
    free = np.ones(NB, dtype=bool)
    while remaining > 0 and free.any():
        share = w * free
        share = share / share.sum() * remaining
        add = np.minimum(np.floor(share).astype(np.int64), NBK - counts)
        if add.sum() == 0:
            # hand the remainder out one at a time, largest weight first
            order = np.argsort(-(w * free))
            for i in order:
                if remaining == 0:
                    break
                if counts[i] < NBK:
                    counts[i] += 1
                    remaining -= 1
            break
        counts += add
        remaining -= int(add.sum())
        free = counts < NBK
    rows, cols = [], []
    for by in range(NB):
        c = np.sort(rng.permutation(NBK)[: counts[by]])
        rows.append(np.full(len(c), by))
        cols.append(c)
    return np.concatenate(rows).astype(np.int64), np.concatenate(cols).astype(np.int64)


def structure_to_bsr(rows, cols, NB: int, values: np.ndarray):
    """Sorted (row, col) slots + values (nnz, p, q) -> (crow, col, values)."""
    crow = np.zeros(NB + 1, dtype=np.int64)
    np.add.at(crow, np.asarray(rows) + 1, 1)
    crow = np.cumsum(crow)
    return crow, np.asarray(cols, dtype=np.int64), values
