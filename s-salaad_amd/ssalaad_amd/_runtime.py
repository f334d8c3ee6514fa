"""Host runtime pieces shared by the op and the module: work plans and workspaces.

A work plan (built by the C ABI's ssl_plan_build) assigns the units of each
block-row — its sparse blocks, then its low-rank slices — to workgroup chunks.
Workspaces hold the kernels' completion counters, the low-rank latent and the
partial tiles of split rows. Counters are zero at rest (the kernels return them
to zero), so one zero-initialised workspace per (device, stream) is reused by
every call on that stream and grown when a call needs more.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

# Workgroups the decode plan aims for: two per compute unit of an MI355X.
_TARGET_WORKGROUPS = 512
# Smallest chunk worth a workgroup, in weight bytes.
_MIN_CHUNK_BYTES = 16384


def plan_target_cost(total_cost: int, block_p: int, elem_bytes: int, M: int) -> int:
    """Chunk cost target for a call with M token rows (0 = never split a row).

    Cost units are columns of a p-row block (q per sparse block, 32 per low-rank
    unit). With one token tile (M ≤ 64) rows are split so the chip has ~512
    workgroups; with several token tiles the tiles already provide parallelism.
    """
    if M > 64:
        return 0
    min_cost = max(1, _MIN_CHUNK_BYTES // (block_p * elem_bytes))
    return max(min_cost, -(-total_cost // _TARGET_WORKGROUPS))


def build_plan(
    crow_host: np.ndarray,
    rows_host: np.ndarray | None,
    block_q: int,
    lr_units: int,
    target_cost: int,
) -> tuple[np.ndarray, int, int]:
    """Return (table [n_chunks, 8] int32, n_chunks, n_slots) for a BSR structure."""
    lib = _lib.load()
    crow_host = np.ascontiguousarray(crow_host, dtype=np.int32)
    NB = crow_host.shape[0] - 1
    rows_p = None
    n_rows = 0
    if rows_host is not None:
        rows_host = np.ascontiguousarray(rows_host, dtype=np.int32)
        rows_p = rows_host.ctypes.data
        n_rows = rows_host.shape[0]
    n_chunks = ctypes.c_int64()
    n_slots = ctypes.c_int64()
    rc = lib.ssl_plan_build(
        crow_host.ctypes.data, NB, rows_p, n_rows, block_q, lr_units, target_cost,
        None, 0, ctypes.byref(n_chunks), ctypes.byref(n_slots),
    )
    _lib.check(rc, "ssl_plan_build")
    table = np.zeros((max(n_chunks.value, 1), _lib.PLAN_STRIDE), dtype=np.int32)
    rc = lib.ssl_plan_build(
        crow_host.ctypes.data, NB, rows_p, n_rows, block_q, lr_units, target_cost,
        table.ctypes.data, table.shape[0], ctypes.byref(n_chunks), ctypes.byref(n_slots),
    )
    _lib.check(rc, "ssl_plan_build")
    return table[: n_chunks.value], int(n_chunks.value), int(n_slots.value)


class DevicePlan:
    """A plan uploaded to one device."""

    __slots__ = ("table", "n_chunks", "n_slots")

    def __init__(self, table: np.ndarray, n_chunks: int, n_slots: int, device: torch.device):
        t = torch.from_numpy(table if n_chunks else np.zeros((1, _lib.PLAN_STRIDE), np.int32))
        self.table = t.to(device)
        self.n_chunks = n_chunks
        self.n_slots = n_slots


_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-initialised uint8 workspace of at least `nbytes` for the current stream.

    Calls ordered on one stream share it; the kernels leave its counters at zero.
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(int(nbytes), 1 << 20)
        if ws is not None:
            size = max(size, 2 * ws.numel())
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws
