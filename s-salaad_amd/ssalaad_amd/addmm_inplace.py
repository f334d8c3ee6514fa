"""`torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_` on gfx950.

Drop-in for ssalaad/tilelang_sparse/addmm_inplace.py: same op name and schema
(:130-136), same fake (:139-141), same argument meaning (:88-110) — but the body
is the hand-written HIP streaming kernel of libssalaad_amd.so instead of a
TileLang/CUDA JIT kernel:

    out_inplace[:, by·p:(by+1)·p] += Σ_blocks x[:, col·q:(col+1)·q] · values[blk]

for each block-row `by` listed in `active_rows`; values are (nnz, q, p), p and q
any multiples of 16 (square or not), as the TileLang kernel takes them
(:59-63, :96-97). The accumulator starts from out in fp32 and is stored once in
out's dtype. Unlike the TileLang kernel, M needs no padding to a tile multiple.
Blocks wider than the kernels' tiles (p > 64, or q > 256) are cut exactly into
sub-blocks once per structure (_reblock.py).

The per-structure work plan (which workgroup sums which blocks) is built on the
host the first time a given crow/col/active_rows triple is seen and cached on the
crow tensor object (keyed by the tensors' versions); building it validates the structure
— monotone crow, col within range, active rows ascending — so the kernel never
reads outside the tensors it is given. That first call copies the structure to the
host (a synchronisation); `prepare_bsr_addmm` does it ahead of time, after which
calls with that structure, including calls under HIP graph capture, touch only
the device. A first call under capture raises (a copy to the host cannot be
captured) instead of failing inside the capture.
"""

from __future__ import annotations

import weakref

import numpy as np
import torch

from . import _lib, _reblock, _runtime

# Block sides the kernels take: multiples of 16 (tiles of 16, 32, 48 or 64
# output features natively, wider blocks cut into those).
BLOCK_MULTIPLE = 16
SUPPORTED_BLOCK_SIZES = (16, 32, 48, 64)

_TORCH_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def get_tuned_config(block_p: int, block_q: int) -> dict:
    """Row-multiple contract of addmm_inplace.py:36-38.

    The HIP kernel masks token rows itself, so callers need no row padding (BM=1).
    """
    return {"BM": 1, "WARP_TILE_M": 16, "WARP_TILE_N": 16}


class _StructPlan:
    __slots__ = ("versions", "col_ref", "act_ref", "plans", "NB_K")

    def __init__(self, versions, col, act, NB_K):
        self.versions = versions
        self.col_ref = weakref.ref(col)
        self.act_ref = weakref.ref(act)
        self.plans: dict[int, _runtime.DevicePlan] = {}
        self.NB_K = NB_K


_PLAN_ATTR = "_ssl_struct_plan"
_PREFILL_MIN_ROWS = 128  # ssl_prefill_min_rows(): fewer token rows always stream


def _validated_host_structure(crow, col, active_rows, nnz_values, NB_K):
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            "the first call with a BSR structure builds its work plan from a host copy of the "
            "structure, which a HIP graph cannot capture; call "
            "ssalaad_amd.prepare_bsr_addmm(crow_indices, col_indices, values, active_rows, "
            "in_features) once before capturing")
    crow_h = crow.detach().to("cpu", torch.int64).numpy()
    col_h = col.detach().to("cpu", torch.int64).numpy()
    act_h = active_rows.detach().to("cpu", torch.int64).numpy()
    NB = crow_h.shape[0] - 1
    if NB < 0 or crow_h[0] != 0 or np.any(np.diff(crow_h) < 0):
        raise ValueError("crow_indices must start at 0 and be non-decreasing")
    if crow_h[-1] != col_h.shape[0] or col_h.shape[0] != nnz_values:
        raise ValueError(
            f"crow_indices[-1]={int(crow_h[-1])}, col_indices ({col_h.shape[0]}) and "
            f"values ({nnz_values}) must agree on nnz"
        )
    if col_h.size and (col_h.min() < 0 or col_h.max() >= NB_K):
        raise ValueError(f"col_indices must lie in [0, {NB_K})")
    if act_h.size and (act_h.min() < 0 or act_h.max() >= NB or np.any(np.diff(act_h) <= 0)):
        raise ValueError("active_rows must be ascending block-row indices")
    return crow_h.astype(np.int32), act_h.astype(np.int32)


def _plan_for(crow, col, active_rows, values, NB_K, block_p, block_q, M, elem_bytes,
              prefill=None):
    versions = (crow._version, col._version, active_rows._version, col.data_ptr(),
                active_rows.data_ptr(), values.shape[0], NB_K)
    sp = getattr(crow, _PLAN_ATTR, None)
    if (
        sp is None
        or sp.versions != versions
        or sp.col_ref() is not col
        or sp.act_ref() is not active_rows
    ):
        sp = _StructPlan(versions, col, active_rows, NB_K)
        setattr(crow, _PLAN_ATTR, sp)
    target_key = 0 if M > 64 else 1
    plan = sp.plans.get(target_key)
    if plan is None:
        crow_h, act_h = _validated_host_structure(crow, col, active_rows, values.shape[0], NB_K)
        total = int(crow_h[-1]) * block_q
        target = _runtime.plan_target_cost(total, block_p, elem_bytes, M)
        col_h = col.detach().to("cpu").numpy().astype(np.int32)
        table, n_chunks, n_slots = _runtime.build_plan(crow_h, col_h, NB_K, act_h, block_q, 0,
                                                       target)
        plan = _runtime.DevicePlan(table, n_chunks, n_slots, crow.device)
        sp.plans[target_key] = plan
    pf = None
    lib = _lib.load()
    dt = _lib.SSL_BF16 if elem_bytes == 2 else _lib.SSL_F32
    if prefill is None:
        prefill = bool(lib.ssl_bsr_addmm_takes_prefill(M, plan.n_chunks, block_p, block_q, dt))
    if prefill and plan.n_chunks > 0:
        # the prefill kernel's groups list the planned rows (active rows with blocks)
        G = int(lib.ssl_prefill_group(M, plan.n_chunks, block_p, block_q))
        step_cols = int(lib.ssl_prefill_step_cols(dt))
        pf = sp.plans.get(("pf", G, step_cols))
        if pf is None:
            crow_h, _ = _validated_host_structure(crow, col, active_rows, values.shape[0], NB_K)
            col_h = col.detach().to("cpu").numpy().astype(np.int32)
            rows_h = plan.table.cpu().numpy()[: plan.n_chunks, 0].astype(np.int32)
            groups, steps, ng = _runtime.build_prefill_plan(crow_h, col_h, NB_K, rows_h, block_p, G,
                                                            step_cols)
            pf = _runtime.DevicePrefillPlan(groups, steps, ng, G, crow.device)
            sp.plans[("pf", G, step_cols)] = pf
    return plan, pf


_VIEW_ATTR = "_ssl_kernel_view"


def _kernel_view(crow, col, values, active_rows, p, q, P, Q, NB_K):
    """(crow, col, values, active_rows) of the same matrix in (Q, P) blocks (the
    blocks the kernels run, or the square ones of many-token calls), cached on
    the values tensor per block shape while every input keeps its identity
    and version. The structure is validated before it is cut."""
    key = tuple((t.data_ptr(), t._version) for t in (crow, col, values, active_rows))
    views = getattr(values, _VIEW_ATTR, None)
    if views is None:
        views = {}
        setattr(values, _VIEW_ATTR, views)
    hit = views.get((P, Q))
    if hit is not None and hit[0] == key:
        return hit[1]
    crow_h, act_h = _validated_host_structure(crow, col, active_rows, values.shape[0], NB_K)
    col_h = col.detach().to("cpu").numpy().astype(np.int32)
    crow2, col2, vals2 = _reblock.reblock(crow_h, col_h, values.contiguous(), p, q, P, Q)
    dev = values.device
    view = (torch.from_numpy(crow2).to(dev), torch.from_numpy(col2).to(dev), vals2,
            torch.from_numpy(_reblock.reblock_rows(act_h, p // P)).to(dev))
    views[(P, Q)] = (key, view)
    return view


_VPQ_ATTR = "_ssl_values_pq"


def _values_pq(values: torch.Tensor, vals: torch.Tensor) -> torch.Tensor:
    """The blocks in (nnz, p, q) order for the prefill kernel, cached on the
    values tensor while its data pointer and version stay the same."""
    key = (values.data_ptr(), values._version)
    hit = getattr(values, _VPQ_ATTR, None)
    if hit is not None and hit[0] == key:
        return hit[1]
    vpq = vals.transpose(1, 2).contiguous()
    setattr(values, _VPQ_ATTR, (key, vpq))
    return vpq


def _aligned_rows(t: torch.Tensor) -> bool:
    eb = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and (t.stride(0) * eb) % 16 == 0


def bsr_addmm_inplace_(
    out_inplace: torch.Tensor,
    x: torch.Tensor,
    crow_indices: torch.Tensor,
    col_indices: torch.Tensor,
    values: torch.Tensor,
    active_rows: torch.Tensor,
) -> None:
    """In place ``out_inplace += x @ S.T`` on the active block-rows of S."""
    if out_inplace.dtype not in _TORCH_DTYPES:
        raise TypeError(
            f"HIP BSR kernel supports float16/bfloat16/float32, got {out_inplace.dtype}"
        )
    if x.dtype != out_inplace.dtype or values.dtype != out_inplace.dtype:
        raise TypeError("out_inplace, x and values must share one dtype")
    for name, t in (("crow_indices", crow_indices), ("col_indices", col_indices),
                    ("active_rows", active_rows)):
        if t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32, got {t.dtype}")
        if t.dim() != 1:
            raise ValueError(f"{name} must be 1-D")
    if out_inplace.dim() != 2 or x.dim() != 2 or values.dim() != 3:
        raise ValueError("out_inplace and x must be 2-D and values (nnz, block_q, block_p)")
    devs = {t.device for t in (out_inplace, x, crow_indices, col_indices, values, active_rows)}
    if len(devs) != 1 or out_inplace.device.type != "cuda":
        raise ValueError("all tensors must be on one ROCm GPU device")
    # The op's own kernels never wait on another workgroup; an earlier fused
    # call on the device that gave up a wait makes its inputs unreliable.
    _runtime.check_status(out_inplace.device)
    block_q = int(values.shape[1])
    block_p = int(values.shape[2])
    if block_p % BLOCK_MULTIPLE or block_q % BLOCK_MULTIPLE or block_p == 0 or block_q == 0:
        raise ValueError(
            f"The HIP BSR kernel requires block dimensions divisible by {BLOCK_MULTIPLE}, "
            f"got {block_p}x{block_q}."
        )
    M, N = out_inplace.shape
    NB = int(crow_indices.shape[0]) - 1
    if x.shape[0] != M:
        raise ValueError(f"x has {x.shape[0]} rows, out_inplace has {M}")
    if N != NB * block_p:
        raise ValueError(f"out N={N} does not match crow ({NB} block-rows) x block_p={block_p}")
    K = int(x.shape[1])
    if K % block_q:
        raise ValueError(f"x K={K} must be divisible by block_q={block_q}")
    NB_K = K // block_q
    if M == 0 or values.shape[0] == 0 or active_rows.numel() == 0:
        return
    P, Q = _reblock.kernel_block_shape(block_p, block_q)
    eb = out_inplace.element_size()
    if M >= _PREFILL_MIN_ROWS and not _reblock.prefill_square(P, Q, eb):
        # many tokens: blocks the tiled kernels do not run as they are go to
        # the same matrix in square blocks when the tiled kernels take it there
        s = _reblock.square_block(P, Q, eb)
        rows = active_rows.numel() * (block_p // s) if s else 0
        if s and _lib.load().ssl_bsr_addmm_takes_prefill(M, rows, s, s,
                                                          _lib.dtype_code(out_inplace.dtype)):
            view = _kernel_view(crow_indices, col_indices, values, active_rows, block_p,
                                block_q, s, s, NB_K)
            return bsr_addmm_inplace_(out_inplace, x, *view)
    if (P, Q) != (block_p, block_q):
        view = _kernel_view(crow_indices, col_indices, values, active_rows, block_p, block_q, P,
                            Q, NB_K)
        return bsr_addmm_inplace_(out_inplace, x, *view)
    plan, pf = _plan_for(crow_indices, col_indices, active_rows, values, NB_K, block_p, block_q,
                         M, out_inplace.element_size())
    if plan.n_chunks == 0:
        return
    if not _aligned_rows(x):
        x = x.contiguous()
        if not _aligned_rows(x):
            x = x.clone(memory_format=torch.contiguous_format)
    vals = values if (values.is_contiguous() and values.data_ptr() % 16 == 0) else values.contiguous()
    col = col_indices.contiguous()
    target = out_inplace
    if not _aligned_rows(out_inplace):
        target = out_inplace.contiguous().clone()
    lib = _lib.load()
    dt = _lib.dtype_code(out_inplace.dtype)
    dev = out_inplace.device
    with torch.cuda.device(dev):
        ws = _runtime.workspace(dev, lib.ssl_bsr_addmm_workspace_size(M, NB, block_p, plan.n_slots))
        cnt = _runtime.counters(dev, lib.ssl_bsr_addmm_counter_count(M, NB))
        vals_pq = _values_pq(values, vals) if pf else None
        rc = lib.ssl_bsr_addmm_inplace(
            target.data_ptr(), target.stride(0), x.data_ptr(), x.stride(0), col.data_ptr(),
            vals.data_ptr(), vals.shape[0], plan.table.data_ptr(), plan.n_chunks, plan.n_slots,
            vals_pq.data_ptr() if pf else None,
            pf.groups.data_ptr() if pf else None, pf.steps.data_ptr() if pf else None,
            pf.n_groups if pf else 0, pf.group if pf else 0, M, N, K, NB,
            block_p, block_q, dt, cnt.data_ptr(), cnt.numel(), ws.data_ptr(), ws.numel(),
            _lib.stream_ptr(dev),
        )
    _lib.check(rc, "ssl_bsr_addmm_inplace")
    if target is not out_inplace:
        out_inplace.copy_(target)


def prepare_bsr_addmm(
    crow_indices: torch.Tensor,
    col_indices: torch.Tensor,
    values: torch.Tensor,
    active_rows: torch.Tensor,
    in_features: int,
) -> None:
    """Validate a BSR structure and build every per-structure object the op
    caches for it (the kernels' block view, the decode and many-token work
    plans, the prefill plan and the (nnz, p, q) copy of the values), so that
    later calls with these tensors, unchanged, copy nothing to the host and can
    be captured in a HIP graph. No counterpart in the reference, whose op has no
    host-side plan. Raises as the op would for a bad structure."""
    for name, t in (("crow_indices", crow_indices), ("col_indices", col_indices),
                    ("active_rows", active_rows)):
        if t.dtype != torch.int32 or t.dim() != 1:
            raise TypeError(f"{name} must be a 1-D int32 tensor")
    if values.dim() != 3 or values.dtype not in _TORCH_DTYPES:
        raise ValueError("values must be (nnz, block_q, block_p) in float16/bfloat16/float32")
    block_q, block_p = int(values.shape[1]), int(values.shape[2])
    if block_p % BLOCK_MULTIPLE or block_q % BLOCK_MULTIPLE or block_p == 0 or block_q == 0:
        raise ValueError(
            f"The HIP BSR kernel requires block dimensions divisible by {BLOCK_MULTIPLE}, "
            f"got {block_p}x{block_q}.")
    if in_features % block_q:
        raise ValueError(f"in_features={in_features} must be divisible by block_q={block_q}")
    NB_K = in_features // block_q
    if values.shape[0] == 0 or active_rows.numel() == 0:
        _validated_host_structure(crow_indices, col_indices, active_rows, values.shape[0], NB_K)
        return
    P, Q = _reblock.kernel_block_shape(block_p, block_q)
    eb = values.element_size()
    s = _reblock.square_block(P, Q, eb)
    if not _reblock.prefill_square(P, Q, eb) and s:
        # many-token calls run the square view: its plans too
        prepare_bsr_addmm(*_kernel_view(crow_indices, col_indices, values, active_rows,
                                        block_p, block_q, s, s, NB_K), in_features)
    if (P, Q) != (block_p, block_q):
        crow_indices, col_indices, values, active_rows = _kernel_view(
            crow_indices, col_indices, values, active_rows, block_p, block_q, P, Q, NB_K)
        block_p, block_q, NB_K = P, Q, in_features // Q
    dt = _lib.dtype_code(values.dtype)
    lib = _lib.load()
    can_prefill = bool(lib.ssl_bsr_addmm_takes_prefill(1 << 20, 1, block_p, block_q, dt))
    with torch.cuda.device(values.device):
        for M, pf_wanted in ((1, False), (1 << 20, can_prefill)):
            _, pf = _plan_for(crow_indices, col_indices, active_rows, values, NB_K, block_p,
                              block_q, M, eb, prefill=pf_wanted)
            if pf is not None:
                vals = values if (values.is_contiguous() and values.data_ptr() % 16 == 0) \
                    else values.contiguous()
                _values_pq(values, vals)


# Same library name, op name and schema as addmm_inplace.py:130-136, in a
# FRAGMENT of the "ssalaad" namespace.
_lib_frag = torch.library.Library("ssalaad", "FRAGMENT")
_lib_frag.define(
    "tilelang_bsr_addmm_inplace_dense_(Tensor(a!) out_inplace, Tensor x, "
    "Tensor crow_indices, Tensor col_indices, Tensor values, Tensor active_rows) -> ()"
)
_lib_frag.impl("tilelang_bsr_addmm_inplace_dense_", bsr_addmm_inplace_, "CUDA")


@torch.library.register_fake("ssalaad::tilelang_bsr_addmm_inplace_dense_")
def _fake(out_inplace, x, crow_indices, col_indices, values, active_rows) -> None:
    return None
