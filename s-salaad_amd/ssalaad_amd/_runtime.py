"""Host runtime pieces shared by the op and the module: work plans and workspaces.

A work plan (built by the C ABI's ssl_plan_build) assigns the units of each
block-row — its sparse blocks, then its low-rank slices — to workgroup chunks.
Scratch comes in two pools per (device, stream), shared by every call ordered on
that stream and grown when a call needs more:
  * counters: int32, zero-initialised and used for nothing else; the kernels
    return every counter they touch to zero, so the pool is zero at rest;
  * workspace: bytes for the low-rank latent and the partial tiles of split
    rows; no initialisation needed.
A plan that feeds the fused kernel also owns its exchange area (see
DevicePlan.exchange): it advances monotonically and is never shared.

A buffer that is outgrown is retired, never freed: a HIP graph captured
earlier holds its raw address and replays into it, so every retired pool
buffer and exchange area lives as long as the process (the pools grow
geometrically, so the retired ones total less than the live one).

Every fused call reports a bounded wait that gave up in one status word per
device (`status_word`). The word lives in pinned, coherent host memory that the
kernels write through its device address, so the host reads it with a plain
load: every call of the modules, groups, chains and the op checks it first
(`check_status`) and raises once a give-up has landed, and the decode engine
checks it before each step.
"""

from __future__ import annotations

import ctypes
import weakref

import numpy as np
import torch

from . import _lib

# Weight bytes one workgroup streams before a row is split: a workgroup's 8
# waves keep about 256 KiB in flight, so a chunk costs one or two memory round
# trips. Rows of up to this size are never split and need no cross-workgroup
# combine; longer rows (skewed structures) are.
_CHUNK_BYTES = 512 * 1024


def plan_target_cost(total_cost: int, block_p: int, elem_bytes: int, M: int) -> int:
    """Chunk cost target for a call with M token rows (0 = never split a row).

    Cost units are columns of a p-row block (q per sparse block, 32 per low-rank
    unit), i.e. p·elem_bytes weight bytes each. With one token tile (M ≤ 64) a
    row longer than _CHUNK_BYTES is split; several token tiles already provide
    the parallelism, so rows stay whole.
    """
    if M > 64:
        return 0
    return max(1, _CHUNK_BYTES // (block_p * elem_bytes))


# Row balancing for decode-shaped calls whose rows are long enough that the
# longest one sets the launch time (see balanced_target). _BALANCE_LATENT_MIN
# is the number of latent K chunks the balancing leaves room for.
_BALANCE_MIN_ROW_BYTES = 128 * 1024
_BALANCE_LATENT_MIN = 4
# With 64-wide blocks (one workgroup per compute unit) the chunks may exceed
# the slots the latent leaves free by an eighth of the compute units: the
# latent's workgroups end well before the longest rows, and the chunks
# dispatched into their slots still finish first. LLaMA-7B FFN decode
# (11008×4096, 8 weight copies): 16.4 → 15.9 µs at 1 token row, 17.3-17.9 →
# 17.0-17.1 at 16 (4096×11008: 19.95 → 19.5 / unchanged); a quarter of the
# compute units: 19.4 / 22.3 µs, the late chunks become the stragglers.
_BALANCE_EXTRA_P64 = 8  # extra chunks: compute units / this
# Block sizes it applies to: at p = 32 (two workgroups per compute unit,
# shorter rows) the split rows' exchange costs more than the straggler. At
# p = 16 a row of small blocks streams slowly on one workgroup (a 4096-row
# call has 256 block-rows for 512 slots), so splitting pays even unskewed.
_BALANCE_P = (16, 64)
# Any block size: structures whose longest row exceeds this multiple of the mean
# and that the default target leaves whole (Zipf rows of 16×16 blocks at decode:
# 51 → 26 µs; rows the default already splits got slower when split further,
# the latent losing its K chunks to the extra row workgroups).
_BALANCE_SKEW = 1.5


def balanced_target(costs: np.ndarray, cost_bytes: int, slots: int, lat_tiles: int) -> int:
    """A chunk cost target that splits only the longest rows, into the
    workgroup slots the other rows and a minimal latent leave free (0 = none).

    costs: per-row cost; cost_bytes: weight bytes per cost unit; slots: row and
    latent workgroups resident at once; lat_tiles: latent workgroups per K chunk.
    """
    costs = costs[costs > 0]
    if costs.size == 0 or _BALANCE_LATENT_MIN <= 0:
        return 0
    if costs.max() * cost_bytes < _BALANCE_MIN_ROW_BYTES:
        return 0
    budget = slots - _BALANCE_LATENT_MIN * lat_tiles
    if budget <= costs.size:
        return 0
    lo, hi = int(costs.mean() // 2), int(costs.max())  # hi: no split
    while lo < hi:  # smallest target whose chunk count fits the budget
        mid = (lo + hi) // 2
        if int(np.ceil(costs / mid).sum()) <= budget:
            hi = mid
        else:
            lo = mid + 1
    return 0 if lo >= costs.max() else lo


def partial_split_plan(crow_host: np.ndarray, col_host: np.ndarray, NBK: int, block_q: int,
                       lr_units: int, n_split: int) -> tuple[np.ndarray, int, int]:
    """A plan whose last `n_split` block-rows are split in two and the others
    kept whole, for structures of equal rows (2:4 storage) where the free
    workgroup slots fit only some extra chunks. Each split row's finaliser
    still follows its other chunk, as the kernel requires."""
    crow_host = np.ascontiguousarray(crow_host, dtype=np.int32)
    NB = crow_host.shape[0] - 1
    costs = np.diff(crow_host).astype(np.int64) * block_q + lr_units * 32
    half = int(costs.max()) // 2 + 1
    ta, na, sa = build_plan(crow_host, col_host, NBK, np.arange(0, NB - n_split, dtype=np.int32),
                            block_q, lr_units, 0)
    tb, nb, sb = build_plan(crow_host, col_host, NBK, np.arange(NB - n_split, NB, dtype=np.int32),
                            block_q, lr_units, half)
    if sa:
        raise RuntimeError("an unsplit plan holds partial-sum slots")
    return np.concatenate([ta[:na], tb[:nb]]).astype(np.int32), na + nb, sb


def build_plan(
    crow_host: np.ndarray,
    col_host: np.ndarray,
    NBK: int,
    rows_host: np.ndarray | None,
    block_q: int,
    lr_units: int,
    target_cost: int,
) -> tuple[np.ndarray, int, int]:
    """Return (table [n_chunks, 8] int32, n_chunks, n_slots) for a BSR structure
    with NBK block-columns; the library checks crow, col and rows first."""
    lib = _lib.load()
    crow_host = np.ascontiguousarray(crow_host, dtype=np.int32)
    col_host = np.ascontiguousarray(col_host, dtype=np.int32)
    col_p = col_host.ctypes.data if col_host.size else None
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
        crow_host.ctypes.data, col_p, NB, NBK, rows_p, n_rows, block_q, lr_units, target_cost,
        None, 0, ctypes.byref(n_chunks), ctypes.byref(n_slots),
    )
    _lib.check(rc, "ssl_plan_build")
    table = np.zeros((max(n_chunks.value, 1), _lib.PLAN_STRIDE), dtype=np.int32)
    rc = lib.ssl_plan_build(
        crow_host.ctypes.data, col_p, NB, NBK, rows_p, n_rows, block_q, lr_units, target_cost,
        table.ctypes.data, table.shape[0], ctypes.byref(n_chunks), ctypes.byref(n_slots),
    )
    _lib.check(rc, "ssl_plan_build")
    return table[: n_chunks.value], int(n_chunks.value), int(n_slots.value)


def build_prefill_plan(
    crow_host: np.ndarray, col_host: np.ndarray, NBK: int, rows_host: np.ndarray | None,
    block_p: int, group: int, step_cols: int = 64
) -> tuple[np.ndarray, np.ndarray, int]:
    """Group table [n_groups, 2 + group] and step records of `step_cols`
    columns (64 for 16-bit activations, 32 for fp32: ssl_prefill_step_cols)
    [n_steps, ssl_prefill_step_ints(p, group, step_cols)] (int32) for the
    prefill row kernels (ssl_prefill_plan_build)."""
    lib = _lib.load()
    crow_host = np.ascontiguousarray(crow_host, dtype=np.int32)
    col_host = np.ascontiguousarray(col_host, dtype=np.int32)
    NB = crow_host.shape[0] - 1
    rows_p, n_rows = None, 0
    if rows_host is not None:
        rows_host = np.ascontiguousarray(rows_host, dtype=np.int32)
        rows_p, n_rows = rows_host.ctypes.data, rows_host.shape[0]
    stride = int(lib.ssl_prefill_step_ints(block_p, group, step_cols))
    if stride <= 0:
        raise ValueError(f"no prefill plan for block {block_p}, group {group} and "
                         f"{step_cols}-column steps")
    ng, ns = ctypes.c_int64(), ctypes.c_int64()
    args = (crow_host.ctypes.data, col_host.ctypes.data if col_host.size else None, NB, NBK,
            rows_p, n_rows, block_p, group, step_cols)
    rc = lib.ssl_prefill_plan_build(*args, None, 0, None, 0, ctypes.byref(ng), ctypes.byref(ns))
    _lib.check(rc, "ssl_prefill_plan_build")
    groups = np.zeros((max(ng.value, 1), 2 + group), dtype=np.int32)
    steps = np.zeros((max(ns.value, 1), stride), dtype=np.int32)
    rc = lib.ssl_prefill_plan_build(*args, groups.ctypes.data, groups.shape[0], steps.ctypes.data,
                                    steps.shape[0], ctypes.byref(ng), ctypes.byref(ns))
    _lib.check(rc, "ssl_prefill_plan_build")
    return groups, steps, int(ng.value)


def build_prefill_parts(groups: np.ndarray, n_groups: int, group: int):
    """The part table of a prefill plan's groups (ssl_prefill_parts_build):
    (records [n_parts, 8] int32, n_parts, split_parts), or None when the
    groups are even enough to run whole."""
    lib = _lib.load()
    groups = np.ascontiguousarray(groups, dtype=np.int32)
    n_parts, split = ctypes.c_int64(), ctypes.c_int64()
    args = (groups.ctypes.data, n_groups, group)
    rc = lib.ssl_prefill_parts_build(*args, None, 0, ctypes.byref(n_parts), ctypes.byref(split))
    _lib.check(rc, "ssl_prefill_parts_build")
    if n_parts.value == 0:
        return None
    table = np.zeros((n_parts.value, 8), dtype=np.int32)
    rc = lib.ssl_prefill_parts_build(*args, table.ctypes.data, table.shape[0],
                                     ctypes.byref(n_parts), ctypes.byref(split))
    _lib.check(rc, "ssl_prefill_parts_build")
    return table, int(n_parts.value), int(split.value)


class DevicePrefillPlan:
    """A prefill plan (group table, step records and, for a skewed structure,
    its part table) on one device."""

    __slots__ = ("groups", "steps", "n_groups", "group", "parts", "n_parts", "split_parts")

    def __init__(self, groups: np.ndarray, steps: np.ndarray, n_groups: int, group: int,
                 device: torch.device, parts=None):
        self.groups = torch.from_numpy(groups).to(device)
        self.steps = torch.from_numpy(steps).to(device)
        self.n_groups = n_groups
        self.group = group
        self.parts = self.n_parts = None
        self.split_parts = 0
        if parts is not None:
            table, self.n_parts, self.split_parts = parts
            self.parts = torch.from_numpy(table).to(device)


_PLANS: "weakref.WeakSet[DevicePlan]" = weakref.WeakSet()


class DevicePlan:
    """A plan uploaded to one device."""

    __slots__ = ("table", "n_chunks", "n_slots", "lr_wgs", "_exchange", "_retired",
                 "__weakref__")

    def __init__(self, table: np.ndarray, n_chunks: int, n_slots: int, device: torch.device):
        t = torch.from_numpy(table if n_chunks else np.zeros((1, _lib.PLAN_STRIDE), np.int32))
        self.table = t.to(device)
        self.n_chunks = n_chunks
        self.n_slots = n_slots
        # workgroups that read the latent: the chunks with low-rank units
        lr = (table[:n_chunks, 4] - table[:n_chunks, 3]) if n_chunks else np.zeros(0)
        self.lr_wgs = int((lr > 0).sum())
        self._exchange: torch.Tensor | None = None
        self._retired: list[torch.Tensor] = []
        _PLANS.add(self)

    def exchange(self, nbytes: int) -> torch.Tensor:
        """The plan's own exchange area (bytes), at least `nbytes`.

        It holds the plan's latent-handshake counters, which the kernels advance
        monotonically and never reset, so it belongs to this plan alone and
        calls with one plan are ordered on one stream. Growing replaces it with
        zeros, which is a valid state for the next call; the outgrown area is
        kept alive with the plan, since a graph captured earlier replays into it.
        """
        if self._exchange is None or self._exchange.numel() < nbytes:
            if self._exchange is not None:
                self._retired.append(self._exchange)
            self._exchange = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8,
                                         device=self.table.device)
        return self._exchange

    def wait_status(self) -> int:
        """1 if a workgroup of a call with this plan gave up waiting, else 0.

        Synchronises the device.
        """
        if self._exchange is None:
            return 0
        return int(self._exchange[:8].view(torch.int64)[0].item())


_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}
_COUNTERS: dict[tuple[int, int], torch.Tensor] = {}
# Outgrown pool buffers: kept for the life of the process (see the module doc).
_RETIRED: list[torch.Tensor] = []
_STATUS: dict[int, "StatusWord"] = {}


def _key(device: torch.device) -> tuple[int, int]:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return (idx, torch._C._cuda_getCurrentRawStream(idx))


def _grown(pool, key, n, dtype, device, minimum):
    buf = pool.get(key)
    if buf is None or buf.numel() < n:
        size = max(int(n), minimum)
        if buf is not None:
            size = max(size, 2 * buf.numel())
            _RETIRED.append(buf)
        buf = torch.zeros(size, dtype=dtype, device=device)
        pool[key] = buf
    return buf


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """uint8 workspace of at least `nbytes` for the current stream."""
    return _grown(_WORKSPACES, _key(device), nbytes, torch.uint8, device, 1 << 20)


def counters(device: torch.device, count: int) -> torch.Tensor:
    """int32 counters (zero at rest) of at least `count` for the current stream."""
    return _grown(_COUNTERS, _key(device), count, torch.int32, device, 1 << 14)


class StatusWord:
    """A device's wait-status word: one uint64 of pinned, coherent host memory
    (ssl_status_word_alloc) that the kernels set to 1 through `device_ptr`
    when a workgroup gives up a bounded wait. The host reads and clears it
    in place; it lives as long as the process."""

    __slots__ = ("host_ptr", "device_ptr", "_word")

    def __init__(self) -> None:
        host, dev = ctypes.c_void_p(), ctypes.c_void_p()
        rc = _lib.load().ssl_status_word_alloc(ctypes.byref(host), ctypes.byref(dev))
        _lib.check(rc, "ssl_status_word_alloc")
        self.host_ptr, self.device_ptr = host.value, dev.value
        self._word = ctypes.c_uint64.from_address(self.host_ptr)

    def read(self) -> int:
        """The word as it stands (no synchronisation: a give-up of a call still
        running shows once its store lands)."""
        return int(self._word.value)

    def clear(self) -> None:
        self._word.value = 0


def _index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def status_word(device: torch.device) -> StatusWord:
    """The device's wait-status word, which every fused call on it reports into
    (its output is unreliable once the word is set). Zero until then; only
    `reset_status` clears it."""
    idx = _index(device)
    w = _STATUS.get(idx)
    if w is None:
        with torch.cuda.device(idx):
            w = StatusWord()
        _STATUS[idx] = w
    return w


def check_status(device: torch.device) -> None:
    """Raise RuntimeError if a fused call on `device` gave up waiting (as far as
    the host can see now, without synchronising)."""
    w = _STATUS.get(_index(device))
    if w is not None and w.read() != 0:
        if w.read() >> 8:
            raise RuntimeError(
                f"a device bounds check of a fused SLR launch on cuda:{_index(device)} failed "
                f"(status word {w.read():#x}: bit 8 + code, see ssl_device_checks); call "
                "ssalaad_amd.clear_wait_status() before the next call")
        raise RuntimeError(
            f"a fused SLR launch on cuda:{_index(device)} gave up waiting for another "
            "workgroup (bounded wait), so outputs computed since then are unreliable; "
            "call ssalaad_amd.clear_wait_status() before the next call")


def read_status(device: torch.device) -> int:
    """The device's wait status once all its work has finished (synchronises)."""
    torch.cuda.synchronize(device)
    return status_word(device).read()


def reset_status(device: torch.device) -> None:
    """Clear the device's wait status after all its work has finished
    (synchronises, so no running call sets it again afterwards)."""
    torch.cuda.synchronize(device)
    status_word(device).clear()
