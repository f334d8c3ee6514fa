"""`LRSLinear` on gfx950: the low-rank + block-sparse linear as one fused HIP call.

Mirror of ssalaad/efficient/ls_linear.py. The factory keeps the reference's
signature (:227-239), dispatch on nnz (:247-253) and validation messages; the
module classes keep the reference's attributes (in_features, out_features, r,
block_p, block_q, S_nnz, kind) and buffers (A, B, bias, S_crow, S_col, S_values
(nnz, q, p), S_active_rows — :28-36, :86-97). The forward

    y = x · Bᵀ · Aᵀ + x · Sᵀ + b

is one call of `ssl_slr_forward` — one kernel launch that computes the latent
t = x·Bᵀ and streams t·Aᵀ, the sparse term and the bias into one epilogue —
instead of the reference's F.linear ×2 + BSR op + bias add (:124-137).

Block shapes: any block whose sides are multiples of 16, square or not, as
the reference's GPU class takes (:114-117). The kernels run p ∈ {16, 32, 48,
64} output features by up to 256 input features natively; wider blocks are cut
exactly into such sub-blocks once, in the module's kernel view (_reblock.py).

Differences from the reference, all extensions:
  * fp32 runs on the GPU too (the TileLang class requires fp16/bf16, :118-119);
  * out/in features that are not multiples of the block (e.g. FFN 5461) are
    accepted when S is given at the padded shape (ceil(n/p)·p, ceil(m/q)·q);
    the padding must be zero, and y is returned at the true width;
  * no CPU path: the library is the GPU kernels, so CPU tensors are rejected
    (the reference's AVX2 CPU class, :140-164, is the oracle's baseline instead);
  * N:M (2:4) S (nm_n=2, nm_m=4, :167-224) runs on the same fused kernel with
    S packed into 32×32 blocks of kept values and positions (16-bit only)
    instead of the semi-structured tensor of cuSPARSELt.
"""

from __future__ import annotations

import weakref

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, _reblock, _runtime

# The reference's CPU (AVX2) class takes these square blocks; CPU tensors with
# any other block get its message (there is no CPU path here at all).
CPU_BLOCK_SIZES = (8, 16, 32, 64)
_LR_ONLY_BLOCK = 64  # output tile width when S is all zero


def _round_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


class _KernelState:
    """Device-side view of a module's weights in the layout the kernels read.

    Buffers the kernels can read as they are (aligned, padded dims already
    multiples) are used in place; otherwise a zero-padded copy is made once.
    The state records which buffers (and which in-place version of each) it was
    built from; the module rebuilds it when any of them changes, e.g. after
    load_state_dict or an in-place copy into A.
    """

    def __init__(self, mod: "_LRSLinearBase", device: torch.device,
                 block: tuple[int, int] | None = None):
        dtype = mod.A.dtype
        self.key = mod._weights_key()
        self.device = device
        self.dtype_code = _lib.dtype_code(dtype)
        self.elem = torch.empty((), dtype=dtype).element_size()
        n, m, r = mod.out_features, mod.in_features, mod.r
        p, q = block if block is not None else mod._kernel_block
        self._mod = weakref.ref(mod)
        self._square: "_KernelState | None" = None
        self.p, self.q = p, q
        # kernel block-rows: a stored block-row of bp features is bp / p kernel rows
        bp = getattr(mod, "block_p", None) or p
        self.NB = -(-n // bp) * (bp // p)
        self.n_pad = self.NB * p
        self.r_pad = _round_up(max(r, 1), 64)
        self.m_pad = _round_up(max(m, 1), 64)
        self.m = m
        self.A = self._padded(mod.A, self.n_pad, self.r_pad)
        self.B = self._padded(mod.B, self.r_pad, self.m_pad)
        self.bias = None
        if mod.bias is not None:
            b = mod.bias.to(dtype)
            self.bias = b if (self.n_pad == n and b.is_contiguous()) else F.pad(b, (0, self.n_pad - n)).contiguous()
        self.s_format = 1 if getattr(mod, "kind", "") == "nm" else 0
        if self.s_format == 1:
            self.col = mod._nm_col
            self.values = mod._nm_blocks
            crow_h = mod._nm_crow.detach().to("cpu").numpy().astype(np.int32)
            self.col_h = mod._nm_col.detach().to("cpu").numpy().astype(np.int32)
            self.nblk_total = int(crow_h[-1])
        elif mod.S_nnz > 0:
            self.col = mod.S_col
            self.values = mod.S_values
            crow_h = mod.S_crow.detach().to("cpu").numpy().astype(np.int32)
            self.col_h = mod.S_col.detach().to("cpu").numpy().astype(np.int32)
            bp, bq = mod.block_p, mod.block_q
            if (bp, bq) != (p, q):  # cut into the (q, p) sub-blocks the kernels run
                crow_h, self.col_h, self.values = _reblock.reblock(
                    crow_h, self.col_h, mod.S_values, bp, bq, p, q)
                self.col = torch.from_numpy(self.col_h).to(device)
            self.nblk_total = int(crow_h[-1])
        else:
            self.col = torch.zeros(1, dtype=torch.int32, device=device)
            self.values = torch.zeros(16, dtype=dtype, device=device)
            crow_h = np.zeros(self.NB + 1, dtype=np.int32)
            self.col_h = np.zeros(0, dtype=np.int32)
            self.nblk_total = 0
        self.crow_h = crow_h
        self.lr_units = self.r_pad // 32
        self.block_q = q
        # kernel block-columns: a stored block-column of bq features is bq / q of them
        bq = getattr(mod, "block_q", None) or q
        self.NBK = -(-m // bq) * (bq // q)
        self._plans: dict[int, _runtime.DevicePlan] = {}
        # fused calls led by this state: (M, stream, linears) -> _LaunchCall
        self._calls: dict[tuple, "_LaunchCall"] = {}
        self._pf_plans: dict[int, _runtime.DevicePrefillPlan] = {}
        self._values_pq: torch.Tensor | None = None

    def _padded(self, t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
        if t.shape == (rows, cols) and t.is_contiguous() and t.data_ptr() % 16 == 0:
            return t
        out = torch.zeros(rows, cols, dtype=t.dtype, device=t.device)
        out[: t.shape[0], : t.shape[1]] = t
        return out

    def plan(self, M: int, launch: tuple[int, int] | None = None) -> _runtime.DevicePlan:
        """The work plan for calls of M token rows; `launch` = (block-rows, 16-rank
        latent tiles) of every linear sharing the launch (None: this one alone),
        which the 2:4 row split budgets the free workgroup slots against."""
        if launch is None:
            launch = (self.NB, self.r_pad // 16)
        key = (0 if M > 64 else 1, launch if self.s_format == 1 else None)
        pl = self._plans.get(key)
        if pl is None:
            total = self.nblk_total * self.block_q + self.NB * self.lr_units * 32
            target = _runtime.plan_target_cost(total, self.p, self.elem, M)
            costs = np.diff(self.crow_h).astype(np.int64) * self.block_q + self.lr_units * 32
            # a skewed structure whose longest row the default target leaves whole
            skewed = (costs.size > 0 and costs.max() > _runtime._BALANCE_SKEW * costs.mean()
                      and (target == 0 or costs.max() <= target))
            if key[0] == 1 and self.s_format == 0 and (self.p in _runtime._BALANCE_P or skewed):
                # split the longest rows into the workgroup slots left free
                n_cu = torch.cuda.get_device_properties(self.device).multi_processor_count
                per_cu = 2 if (self.p <= 32 and self.elem == 2) else 1
                extra = n_cu // _runtime._BALANCE_EXTRA_P64 if self.p == 64 else 0
                bal = _runtime.balanced_target(costs, self.p * self.elem, n_cu * per_cu + extra,
                                               self.r_pad // 16)
                if bal:
                    target = min(target, bal) if target else bal
            n_split = 0
            if key[0] == 1 and self.s_format == 1 and self.lr_units > 0:
                # 2:4 rows are all alike: split the last rows in two, as many as
                # the free slots take (the balancing budget above), when that
                # is at most half of them (7B FFN at one token tile: 344 rows,
                # 104 split; 24.5 -> 22.0 µs). The slots are those the whole
                # launch leaves free; this linear takes its share of them.
                n_cu = torch.cuda.get_device_properties(self.device).multi_processor_count
                rows, lat_tiles = launch
                free = (n_cu * 2 - _runtime._BALANCE_LATENT_MIN * lat_tiles) - rows
                if 0 < free <= rows // 2:
                    n_split = free * self.NB // rows
            if n_split:
                table, n_chunks, n_slots = _runtime.partial_split_plan(
                    self.crow_h, self.col_h, self.NBK, self.block_q, self.lr_units, n_split)
            else:
                table, n_chunks, n_slots = _runtime.build_plan(
                    self.crow_h, self.col_h, self.NBK, None, self.block_q, self.lr_units, target
                )
            pl = _runtime.DevicePlan(table, n_chunks, n_slots, self.device)
            self._plans[key] = pl
        return pl

    def takes_prefill(self, M: int, n_rows: int | None = None) -> bool:
        """Whether a fused call of M token rows over `n_rows` block-rows (this
        linear's alone by default) runs the prefill kernels; the library decides
        (ssl_slr_takes_prefill), so host and device agree."""
        rows = self.NB if n_rows is None else n_rows
        if self.s_format == 1:  # 2:4: the row kernel on v_smfmac
            return bool(_lib.load().ssl_nm24_takes_prefill(M, rows, self.dtype_code))
        return bool(_lib.load().ssl_slr_takes_prefill(M, rows, self.p, self.q, self.dtype_code))

    def prefill_plan(self, G: int) -> _runtime.DevicePrefillPlan:
        """The prefill row kernel's plan with G block-rows per workgroup."""
        pp = self._pf_plans.get(G)
        if pp is None:
            step_cols = int(_lib.load().ssl_prefill_step_cols(self.dtype_code))
            groups, steps, ng = _runtime.build_prefill_plan(self.crow_h, self.col_h, self.NBK,
                                                            None, self.p, G, step_cols)
            # block storage: long groups of a skewed structure run in parts
            parts = (_runtime.build_prefill_parts(groups, ng, G)
                     if self.s_format == 0 and ng > 0 else None)
            pp = _runtime.DevicePrefillPlan(groups, steps, ng, G, self.device, parts)
            self._pf_plans[G] = pp
        if self._values_pq is None and self.nblk_total > 0:
            if self.s_format == 1:
                # 2:4 blocks as the structured-sparse MFMA reads them
                from .artifact import nm24_prefill_layout

                self._values_pq = nm24_prefill_layout(self.values)
            else:
                # the prefill kernels read each block k-contiguous per output column
                self._values_pq = self.values.transpose(1, 2).contiguous()
        return pp

    def prefill_view(self) -> "_KernelState | None":
        """The same weights in the square blocks the tiled many-token kernels
        run, when this view's blocks are not such (non-square, 48-wide, fp32
        64×64, cut wide blocks): the blocks cut exactly into the widest square
        blocks that tile them (_reblock.square_block), built on first use.
        None when this view runs there as it is (or has no blocks)."""
        if (self.s_format != 0 or self.nblk_total == 0
                or _reblock.prefill_square(self.p, self.q, self.elem)):
            return None
        if self._square is None:
            mod = self._mod()
            s = _reblock.square_block(self.p, self.q, self.elem)
            if mod is None or s == 0:
                return None
            self._square = _KernelState(mod, self.device, block=(s, s))
        return self._square

    def rows(self, x: torch.Tensor) -> torch.Tensor:
        """x as [M, ·] with 16-byte aligned rows (copied into a padded buffer if not)."""
        x2 = x.reshape(-1, x.shape[-1])
        if x2.stride(-1) != 1 or x2.data_ptr() % 16 or (x2.stride(0) * self.elem) % 16:
            ld = _round_up(self.m, 16 // self.elem)
            buf = torch.zeros(x2.shape[0], ld, dtype=x2.dtype, device=x2.device)
            buf[:, : self.m] = x2
            x2 = buf
        return x2

    def forward(self, x: torch.Tensor, out_features: int) -> torch.Tensor:
        """y = x·Bᵀ·Aᵀ + x·Sᵀ + b in one fused launch."""
        return _launch([self], x, [out_features])[0]


def _launch_shares(states, stages) -> list[tuple[int, int] | None]:
    """Per state: (block-rows, latent tiles) of the launch it shares (its stage
    of `stages` member counts, or all of `states` when stages is None), or None
    for a linear alone."""
    counts = stages if stages is not None else [len(states)]
    out, i = [], 0
    for n in counts:
        part = states[i:i + n]
        share = (sum(st.NB for st in part), sum(st.r_pad // 16 for st in part)) if n > 1 else None
        out += [share] * n
        i += n
    return out


class _Descriptors:
    """The C-ABI member descriptors of a fused call of M token rows over
    `states`: plans, sizes and weight pointers are set once; `bind` points
    them at the stream's scratch pools and the plans' exchange areas, `rebind`
    repeats that only when one of those buffers was replaced (a pool that
    grew), and the caller fills in each member's `y`. `extra_counters` more
    int32 counters follow the members' (bind returns their address).
    `stages`: member counts of a chained launch's stages."""

    __slots__ = ("states", "M", "G", "plans", "ws_need", "cnt_need", "xch_need", "extra",
                 "members", "_ws", "_cnt", "_xch", "_extra_ptr")

    def __init__(self, states, M: int, G: int, extra_counters: int = 0,
                 stages: list[int] | None = None) -> None:
        lib = _lib.load()
        self.states, self.M, self.G, self.extra = list(states), M, G, extra_counters
        # the 2:4 row split budgets the slots of each launch (a grouped launch,
        # or a chained launch's stage) as a whole
        self.plans = [st.plan(M, launch) for st, launch in zip(states, _launch_shares(states, stages))]
        self.ws_need = [_round_up(lib.ssl_slr_workspace_size(M, st.NB, st.p, st.r_pad, st.m_pad,
                                                             pl.n_slots, st.dtype_code), 256)
                        for st, pl in zip(states, self.plans)]
        self.cnt_need = [int(lib.ssl_slr_counter_count(M, st.NB)) for st in states]
        self.xch_need = [int(lib.ssl_slr_exchange_size(M, st.r_pad, st.m_pad, st.dtype_code))
                         for st in states]
        self.members = (_lib.SlrMember * len(states))()
        for i, (st, pl) in enumerate(zip(states, self.plans)):
            mb = self.members[i]
            mb.A, mb.B, mb.bias = st.A.data_ptr(), st.B.data_ptr(), _lib.ptr(st.bias)
            mb.col, mb.values = st.col.data_ptr(), st.values.data_ptr()
            mb.plan, mb.n_chunks, mb.n_slots = pl.table.data_ptr(), pl.n_chunks, pl.n_slots
            mb.lr_wgs, mb.NB, mb.r_pad = pl.lr_wgs, st.NB, st.r_pad
            mb.n_counters = self.cnt_need[i]
            mb.workspace_bytes = self.ws_need[i]
            mb.nnz = st.nblk_total
            mb.s_format = st.s_format
            mb.ldy = st.n_pad
            if G:
                pp = st.prefill_plan(G)
                mb.pf_groups, mb.pf_steps = pp.groups.data_ptr(), pp.steps.data_ptr()
                mb.pf_n_groups, mb.pf_group = pp.n_groups, pp.group
                mb.values_pq = _lib.ptr(st._values_pq)
                if pp.parts is not None:
                    # the parts' partial tiles follow the call's own workspace
                    mb.pf_parts, mb.pf_n_parts = pp.parts.data_ptr(), pp.n_parts
                    mb.pf_split_parts = pp.split_parts
                    self.ws_need[i] += _round_up(
                        int(lib.ssl_prefill_parts_bytes(M, pp.split_parts)), 256)
                    mb.workspace_bytes = self.ws_need[i]
        self._ws = self._cnt = None
        self._xch: list = [None] * len(states)
        self._extra_ptr = 0

    def bind(self, dev: torch.device) -> int:
        ws = _runtime.workspace(dev, sum(self.ws_need))
        cnt = _runtime.counters(dev, sum(self.cnt_need) + self.extra)
        xch = [pl.exchange(nb) for pl, nb in zip(self.plans, self.xch_need)]
        if (ws is not self._ws or cnt is not self._cnt
                or any(a is not b for a, b in zip(xch, self._xch))):
            status = _runtime.status_word(dev).device_ptr
            ws_off = cnt_off = 0
            for i, mb in enumerate(self.members):
                mb.counters = cnt.data_ptr() + 4 * cnt_off
                mb.exchange, mb.exchange_bytes = xch[i].data_ptr(), xch[i].numel()
                mb.workspace = ws.data_ptr() + ws_off
                mb.status = status
                ws_off += self.ws_need[i]
                cnt_off += self.cnt_need[i]
            self._ws, self._cnt, self._xch = ws, cnt, xch
            self._extra_ptr = cnt.data_ptr() + 4 * cnt_off
        return self._extra_ptr


def _members(states: list["_KernelState"], ys: list[torch.Tensor], M: int, G: int,
             extra_counters: int = 0, stages: list[int] | None = None):
    """The C-ABI member descriptors of a fused call of M token rows writing
    `ys`, with workspaces and zero-at-rest counters from the stream's pools;
    `extra_counters` more int32 counters follow the members' (their address is
    returned too). `stages`: member counts of a chained launch's stages."""
    d = _Descriptors(states, M, G, extra_counters, stages)
    extra = d.bind(ys[0].device)
    for mb, y in zip(d.members, ys):
        mb.y, mb.ldy = y.data_ptr(), y.stride(0)
    return d.members, extra


def _outputs(states, ys, out_features, lead: tuple) -> list[torch.Tensor]:
    outs = []
    for st, y, n in zip(states, ys, out_features):
        if st.n_pad != n:
            y = y[:, :n]
        outs.append(y.reshape(*lead, n))
    return outs


_MAX_CALLS = 16  # cached launch descriptors per leading state
_PREFILL_MIN_ROWS = 128  # ssl_prefill_min_rows(): fewer token rows always stream


def _launch(states: list["_KernelState"], x: torch.Tensor, out_features: list[int]):
    """One fused launch computing every state's linear of the same x.

    The descriptors of a call (plans, sizes, weight pointers, prefill plans)
    are built once per (token count, stream, linears) and kept on the leading
    state, which is rebuilt whenever a module's weights change; a call fills
    in x and the outputs only."""
    dev = x.device
    _runtime.check_status(dev)
    st0 = states[0]
    orig = x.shape
    x2 = st0.rows(x)
    M = x2.shape[0]
    if M >= _PREFILL_MIN_ROWS:
        # many tokens with blocks the tiled kernels do not run as they are:
        # the square view, when the tiled kernels take the call there
        views = [st.prefill_view() for st in states]
        if views[0] is not None and all(v is not None for v in views):
            if views[0].takes_prefill(M, sum(v.NB for v in views)):
                states = views
                st0 = views[0]
    ys = [torch.empty(M, st.n_pad, dtype=x.dtype, device=dev) for st in states]
    if M > 0:
        lib = _lib.load()
        stream = _lib.stream_ptr(dev)
        key = (M, stream, tuple(map(id, states)))
        d = st0._calls.get(key)  # its states are held, so their ids are not reused
        if d is None or any(a is not b for a, b in zip(d.states, states)):
            G = 0
            rows = sum(st.NB for st in states)
            if st0.takes_prefill(M, rows):
                G = int(lib.ssl_prefill_group(M, rows, st0.p, st0.q))
            if len(st0._calls) >= _MAX_CALLS:
                st0._calls.clear()
            d = st0._calls[key] = _Descriptors(states, M, G)
        d.bind(dev)
        for mb, y in zip(d.members, ys):
            mb.y = y.data_ptr()
        rc = lib.ssl_slr_forward_group(x2.data_ptr(), x2.stride(0), M, st0.m, st0.m_pad, st0.p,
                                       st0.q, st0.dtype_code, d.members, len(states), stream)
        _lib.check(rc, "ssl_slr_forward_group")
    return _outputs(states, ys, out_features, orig[:-1])


def latent_wait_status(device: torch.device) -> int:
    """1 if a fused call on `device` had a workgroup give up waiting (its output
    tile is then unreliable), else 0: the device's status word, which every call
    of this package reports into, and the plans' own words (used by callers of
    the C ABI that pass no status word). Synchronises.
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    words = [pl.wait_status() for pl in list(_runtime._PLANS) if pl.table.device.index == idx]
    return max(words + [_runtime.read_status(torch.device("cuda", idx))])


def clear_wait_status(device: torch.device | None = None) -> None:
    """Clear the wait status of `device` (the current device by default) after
    its work has finished. Every module, group, chain and op call raises
    RuntimeError while the status is set: a workgroup of an earlier call gave
    up a bounded wait, so what was computed since then is unreliable.
    Synchronises."""
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    _runtime.reset_status(device)


class _LRSLinearBase(nn.Module):
    """Buffers and validation of ls_linear.py:7-44."""

    kind: str = ""
    _kernel_block: tuple[int, int] = (_LR_ONLY_BLOCK, _LR_ONLY_BLOCK)  # (P, Q) the kernels run

    def __init__(self, A, B, *, in_features, out_features, bias=None) -> None:
        super().__init__()
        (n, r) = A.shape
        (rB, m) = B.shape
        if rB != r:
            raise ValueError(f"A.shape[1]={r} must match B.shape[0]={rB}")
        if (n, m) != (out_features, in_features):
            raise ValueError(
                f"L = A·B shape ({n},{m}) must equal (out_features={out_features}, in_features={in_features})"
            )
        self.in_features = in_features
        self.out_features = out_features
        self.r = int(r)
        self.register_buffer("B", B.contiguous())
        self.register_buffer("A", A.contiguous())
        if bias is not None:
            self.register_buffer("bias", bias.contiguous())
        else:
            self.bias = None
        self._state: _KernelState | None = None

    def _apply(self, fn, recurse: bool = True):
        self._state = None  # weights moved or cast: rebuild the kernel view lazily
        return super()._apply(fn, recurse=recurse)

    def _weights_key(self) -> tuple:
        """Identity and in-place version of every buffer the kernel view is
        built from (the reference module reads its buffers on every forward;
        this lets an update after the first forward take effect too)."""
        return tuple((name, t.data_ptr(), t._version) for name, t in self._buffers.items()
                     if t is not None)

    def _kernel(self) -> _KernelState:
        st = self._state
        if st is None or st.device != self.A.device or st.key != self._weights_key():
            if self.A.device.type != "cuda":
                raise ValueError("The HIP SLR kernels need the module on a ROCm GPU device.")
            st = _KernelState(self, self.A.device)
            self._state = st
        return st

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != self.A.dtype:
            raise TypeError(f"input dtype {x.dtype} does not match the weights' {self.A.dtype}")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"input has {x.shape[-1]} features, expected {self.in_features}")
        if x.device != self.A.device:
            raise ValueError(f"input on {x.device}, weights on {self.A.device}")
        return self._kernel().forward(x, self.out_features)


class _LRSLinearLR(_LRSLinearBase):
    """S ≡ 0 (ls_linear.py:47-54): the same fused call with no sparse units."""

    kind = "lr_only"
    S_nnz = 0

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, rank={self.r}, S=zero (skipped), bias={self.bias is not None}"


class _LRSLinearLRBlockBase(_LRSLinearBase):
    """Block-sparse S in BSR layout (ls_linear.py:57-104)."""

    kind = "block_sparse"

    def __init__(self, A, B, S_sparse, *, in_features, out_features, bias, block_p, block_q) -> None:
        super().__init__(A, B, in_features=in_features, out_features=out_features, bias=bias)
        p, q = int(block_p), int(block_q)
        expected = {(out_features, in_features), (_round_up(out_features, p), _round_up(in_features, q))}
        if tuple(S_sparse.shape) not in expected:
            raise ValueError(
                f"S shape {tuple(S_sparse.shape)} must equal "
                f"(out_features, in_features)=({out_features},{in_features})"
            )
        self.block_p = p
        self.block_q = q
        self._kernel_block = _reblock.kernel_block_shape(p, q) if p % 16 == 0 and q % 16 == 0 else (p, q)
        self.S_nnz = int(S_sparse._nnz())
        crow = S_sparse.crow_indices()
        self.register_buffer("S_crow", crow.to(torch.int32).clone())
        self.register_buffer("S_col", S_sparse.col_indices().to(torch.int32).clone())
        self.register_buffer("S_values", S_sparse.values().transpose(1, 2).contiguous().clone())
        active = (crow[1:] - crow[:-1]).nonzero(as_tuple=False).squeeze(-1)
        self.register_buffer("S_active_rows", active.to(torch.int32).clone())
        self._check_structure(S_sparse.shape)

    def _check_structure(self, shape) -> None:
        """Host check of the BSR structure the kernels index with."""
        crow = self.S_crow.detach().cpu().numpy().astype(np.int64)
        col = self.S_col.detach().cpu().numpy().astype(np.int64)
        nbk = shape[1] // self.block_q
        if crow[0] != 0 or np.any(np.diff(crow) < 0) or crow[-1] != col.shape[0]:
            raise ValueError("S has an inconsistent BSR row pointer")
        if col.size and (col.min() < 0 or col.max() >= nbk):
            raise ValueError("S has block-column indices out of range")
        if self.S_values.shape[0] != col.shape[0]:
            raise ValueError("S values and column indices disagree on nnz")

    def extra_repr(self) -> str:
        return (
            f"in_features={self.in_features}, out_features={self.out_features}, "
            f"rank={self.r}, S_nnz={self.S_nnz}, "
            f"block=({self.block_p}×{self.block_q}), bias={self.bias is not None}"
        )


class _LRSLinearLRBlockHIP(_LRSLinearLRBlockBase):
    """Block-sparse S on the gfx950 streaming kernels (replaces ls_linear.py:107-137)."""

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        if self.S_values.device.type != "cuda":
            raise ValueError("The HIP block kernel requires a ROCm GPU device.")
        if self.block_p % 16 or self.block_q % 16:
            raise ValueError("The HIP block kernel requires block dimensions divisible by 16.")
        if self.S_values.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("The HIP block kernel requires fp16, bf16 or fp32.")


class _LRSLinearLRNMHIP(_LRSLinearBase):
    """2:4 (N:M) S on the gfx950 streaming kernel (replaces ls_linear.py:167-219).

    S is packed once into 32×32 blocks holding the two kept values of every
    group of four input features and their positions (artifact.nm24_pack); the
    kernel expands each block into MFMA fragments in registers, so a decode
    call streams about 5/8 of the dense block bytes. The fused launch adds
    t·Aᵀ and the bias as for block-sparse S. As in the reference's N:M class,
    the packed S is not part of the state dict (non-persistent buffers).
    """

    kind = "nm"

    def __init__(self, A, B, S_dense, *, in_features, out_features, bias) -> None:
        super().__init__(A, B, in_features=in_features, out_features=out_features, bias=bias)
        if tuple(S_dense.shape) != (out_features, in_features):
            raise ValueError(
                f"S shape {tuple(S_dense.shape)} must equal "
                f"(out_features, in_features)=({out_features},{in_features})"
            )
        from .artifact import NM_BLOCK, nm24_pack

        packed = nm24_pack(S_dense.to(A.dtype))
        self._kernel_block = (NM_BLOCK, NM_BLOCK)
        self.block_p = self.block_q = None
        self.S_nnz = int(packed["blocks"].shape[0]) * NM_BLOCK * NM_BLOCK // 2
        self.register_buffer("_nm_crow", packed["crow"], persistent=False)
        self.register_buffer("_nm_col", packed["col"], persistent=False)
        self.register_buffer("_nm_blocks", packed["blocks"], persistent=False)
        self._nm_dtype = A.dtype  # the dtype the packed values are stored in

    def _kernel(self) -> _KernelState:
        if self.A.dtype != self._nm_dtype:
            raise TypeError(
                f"the 2:4 blocks were packed as {self._nm_dtype}; rebuild the module to run in "
                f"{self.A.dtype}"
            )
        return super()._kernel()

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"rank={self.r}, S_nnz={self.S_nnz}, N:M 2:4 (32×32 packed blocks), "
                f"bias={self.bias is not None}")


def LRSLinear(
    A,
    B,
    S_sparse,
    *,
    in_features,
    out_features,
    bias=None,
    block_p=None,
    block_q=None,
    nm_n=None,
    nm_m=None,
):
    """Compute x @ (A @ B + S).T (+ bias) with the gfx950 kernels.

    Same signature and dispatch as ls_linear.py:227-285: S with no stored block
    gives the low-rank-only module; block-sparse S needs its block shape. There
    is no dense or CSR fallback, so a pattern the kernels cannot run is rejected.
    """
    if S_sparse.layout == torch.strided:
        nnz = int(torch.count_nonzero(S_sparse))
    else:
        nnz = S_sparse._nnz()
    kwargs = dict(in_features=in_features, out_features=out_features, bias=bias)
    if nnz == 0:
        return _LRSLinearLR(A, B, **kwargs)
    if nm_n is not None:
        if (nm_n, nm_m) != (2, 4) or not A.is_cuda:
            raise ValueError("N:M inference requires CUDA and a 2:4 mask.")
        if A.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("The HIP 2:4 kernel requires fp16 or bf16.")
        dense = S_sparse if S_sparse.layout == torch.strided else S_sparse.to_dense()
        return _LRSLinearLRNMHIP(A, B, dense.to(A.device), **kwargs)
    if block_p is None or block_q is None:
        raise ValueError("Sparse S needs a recorded block shape to pick a kernel.")
    if not A.is_cuda:
        # The reference sends CPU tensors to its AVX2 class (square 8/16/32/64
        # blocks, :265-273); this package has no CPU path at all.
        if block_p != block_q or block_p not in CPU_BLOCK_SIZES:
            raise ValueError(
                f"The AVX2 kernel supports square {CPU_BLOCK_SIZES} blocks, "
                f"got ({block_p}, {block_q}); this package runs none of them on the CPU."
            )
        raise ValueError("The HIP kernels need A, B and S on a ROCm GPU device.")
    if S_sparse.layout == torch.strided:
        from .artifact import dense_to_bsr

        S_sparse = dense_to_bsr(S_sparse, block_p, block_q)
    return _LRSLinearLRBlockHIP(A, B, S_sparse, block_p=block_p, block_q=block_q, **kwargs)


class LRSLinearGroup(nn.Module):
    """Up to four SLR linears that read the same input, computed in ONE launch.

    `LRSLinearGroup(q, k, v)(x)` returns `(q(x), k(x), v(x))`, each computed as
    its module computes it (same rounding points, same plans), in one fused
    kernel launch instead of one per module: the latent and row workgroups of
    every member share the device at once. The reference calls every module
    on its own (ssalaad/efficient/model.py:41-57); grouping a layer's q/k/v
    and gate/up projections is this library's launch-count reduction for
    decode. Members must share in_features, dtype, device and block size.
    """

    def __init__(self, *linears: _LRSLinearBase) -> None:
        super().__init__()
        if not 1 <= len(linears) <= _lib.MAX_GROUP:
            raise ValueError(f"a group takes 1 to {_lib.MAX_GROUP} linears, got {len(linears)}")
        for mod in linears:
            if not isinstance(mod, _LRSLinearBase):
                raise ValueError("group members must be LRSLinear modules of this library")
        first = linears[0]
        for mod in linears[1:]:
            if mod.in_features != first.in_features:
                raise ValueError("group members must share in_features (they read the same x)")
            if mod.A.dtype != first.A.dtype or mod.A.device != first.A.device:
                raise ValueError("group members must share dtype and device")
            if (getattr(mod, "kind", "") == "nm") != (getattr(first, "kind", "") == "nm"):
                raise ValueError("group members must share the sparse storage (2:4 or blocks)")
            if mod._kernel_block != first._kernel_block:
                raise ValueError(
                    f"group members must share the kernel block shape, got {first._kernel_block} "
                    f"and {mod._kernel_block}"
                )
        self.members = nn.ModuleList(linears)
        self.in_features = first.in_features

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, ...]:
        first = self.members[0]
        if x.dtype != first.A.dtype:
            raise TypeError(f"input dtype {x.dtype} does not match the weights' {first.A.dtype}")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"input has {x.shape[-1]} features, expected {self.in_features}")
        if x.device != first.A.device:
            raise ValueError(f"input on {x.device}, weights on {first.A.device}")
        states = [mod._kernel() for mod in self.members]
        return tuple(_launch(states, x, [mod.out_features for mod in self.members]))


class LRSLinearChain(nn.Module):
    """Dependent stages of SLR linears computed in ONE launch at decode sizes.

    `LRSLinearChain([[q, k, v], [o], [gate, up], [down]], sources=[q, o, gate])`
    computes stage 0's members of the input x, then every later stage's
    members of the output of its source (a member of an earlier stage), and
    returns every member's output, stage by stage:
    `((q(x), k(x), v(x)), (o(q(x)),), (gate(o(..)), up(o(..))), (down(gate(..)),))`.
    Each output is what the module computes for that input (same plans and
    rounding points); stage 0's equal the grouped launch's bit for bit, later
    stages sum the latent t = x·Bᵀ over in_features in another fp32 order.

    Calls the streaming kernel serves (decode sizes, 16-bit activations, square
    16/32/64 or 2:4 blocks) run as one chained launch (ssl_slr_forward_chain):
    a stage's workgroups load their weights while the stage before it
    finishes, and wait for its output inside the launch instead of at a kernel
    boundary. Other calls run the stages as grouped launches one after another.
    Up to 4 stages of up to 8 linears in all travel in the kernel arguments;
    longer chains (every layer of a model, up to 256 linears) use a descriptor
    table in device memory, uploaded on each call, and `prepare` builds one
    once for fixed buffers (graph capture, static decode loops).
    The reference calls every module on its own (ssalaad/efficient/model.py:41-57).
    """

    def __init__(self, stages, sources) -> None:
        super().__init__()
        stages = [list(st) for st in stages]
        sources = list(sources)
        if not stages:
            raise ValueError("a chain takes at least one stage")
        if len(sources) != len(stages) - 1:
            raise ValueError("every stage after the first needs one source module")
        n = sum(len(st) for st in stages)
        if not 1 <= n <= _lib.MAX_CHAIN_TABLE:
            raise ValueError(f"a chain takes 1 to {_lib.MAX_CHAIN_TABLE} linears, got {n}")
        if any(len(st) > _lib.MAX_GROUP for st in stages):
            raise ValueError(f"a stage takes 1 to {_lib.MAX_GROUP} linears")
        self.groups = nn.ModuleList(LRSLinearGroup(*st) for st in stages)
        first = stages[0][0]
        flat = [mod for st in stages for mod in st]
        for mod in flat:
            if mod.A.dtype != first.A.dtype or mod.A.device != first.A.device:
                raise ValueError("chain members must share dtype and device")
            if (getattr(mod, "kind", "") == "nm") != (getattr(first, "kind", "") == "nm"):
                raise ValueError("chain members must share the sparse storage (2:4 or blocks)")
            if mod._kernel_block != first._kernel_block:
                raise ValueError("chain members must share the kernel block shape")
        self._src: list[tuple[int, int]] = []
        used = set()
        for s, src in enumerate(sources, start=1):
            hit = [(si, mi) for si in range(s) for mi, mod in enumerate(stages[si]) if mod is src]
            if len(hit) != 1:
                raise ValueError(f"stage {s}'s source must be one member of an earlier stage")
            if hit[0] in used:
                raise ValueError(f"stage {s}'s source already feeds another stage")
            used.add(hit[0])
            if src.out_features != stages[s][0].in_features:
                raise ValueError(f"stage {s} reads {stages[s][0].in_features} features, its source "
                                 f"writes {src.out_features}")
            self._src.append(hit[0])
        self.in_features = first.in_features
        self._table_dev: torch.Tensor | None = None

    def _descriptors(self, states, x2: torch.Tensor, ys: list[torch.Tensor], M: int):
        """The C-ABI member and stage descriptors of a chained call writing ys."""
        lib = _lib.load()
        flat = [st for sts in states for st in sts]
        n_sync = int(lib.ssl_slr_chain_sync_count(M))
        # the stage words start 256-byte aligned (64 int32 of slack)
        members, sync = _members(flat, ys, M, 0, extra_counters=n_sync * (len(states) - 1) + 64,
                                 stages=[len(sts) for sts in states])
        sync = (sync + 255) // 256 * 256
        stages = (_lib.SlrStage * len(states))()
        frags: list[torch.Tensor] = []
        base = [0]
        for sts in states:
            base.append(base[-1] + len(sts))
        for s, sts in enumerate(states):
            sg = stages[s]
            sg.m, sg.m_pad = sts[0].m, sts[0].m_pad
            sg.first, sg.count = base[s], len(sts)
            if s == 0:
                sg.x, sg.ldx, sg.src = x2.data_ptr(), x2.stride(0), -1
            else:
                si, mi = self._src[s - 1]
                sg.src = base[si] + mi
                sg.sync, sg.n_sync = sync + 4 * n_sync * (s - 1), n_sync
                # room for the source's output in MFMA-fragment order (the
                # stage then reads whole 1 KiB units)
                src = states[si][mi]
                nbytes = int(lib.ssl_slr_chain_frag_bytes(M, src.NB * src.p))
                if nbytes > 0:
                    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=x2.device)
                    frags.append(buf)
                    sg.xf, sg.xf_bytes = (buf.data_ptr() + 255) // 256 * 256, nbytes
        return members, stages, base, frags

    def prepare(self, x: torch.Tensor) -> "PreparedChain":
        """The chain over the fixed input buffer `x`: its descriptor table is
        built and uploaded once, and every PreparedChain.run() recomputes every
        output from what x holds then, into the same output tensors (a decode
        loop with static buffers, or a HIP graph capture of run())."""
        return PreparedChain(self, x)

    def _chained(self, states, M: int) -> bool:
        st0 = states[0][0]
        if st0.elem != 2 or M <= 0:
            return False
        if st0.s_format == 0 and not (st0.p == st0.q and st0.p in (16, 32, 64)):
            return False
        return not any(sts[0].takes_prefill(M, sum(st.NB for st in sts)) for sts in states)

    def forward(self, x: torch.Tensor) -> tuple[tuple[torch.Tensor, ...], ...]:
        first = self.groups[0].members[0]
        if x.dtype != first.A.dtype:
            raise TypeError(f"input dtype {x.dtype} does not match the weights' {first.A.dtype}")
        if x.shape[-1] != self.in_features:
            raise ValueError(f"input has {x.shape[-1]} features, expected {self.in_features}")
        if x.device != first.A.device:
            raise ValueError(f"input on {x.device}, weights on {first.A.device}")
        _runtime.check_status(x.device)
        states = [[mod._kernel() for mod in grp.members] for grp in self.groups]
        outf = [[mod.out_features for mod in grp.members] for grp in self.groups]
        st0 = states[0][0]
        lead = x.shape[:-1]
        x2 = st0.rows(x)
        M = x2.shape[0]
        if not self._chained(states, M):
            outs: list[list[torch.Tensor]] = []
            for s, sts in enumerate(states):
                xin = x if s == 0 else outs[self._src[s - 1][0]][self._src[s - 1][1]]
                outs.append(_launch(sts, xin, outf[s]))
            return tuple(tuple(o) for o in outs)
        flat = [st for sts in states for st in sts]
        ys = [torch.empty(M, st.n_pad, dtype=x.dtype, device=x.device) for st in flat]
        members, stages, base, frags = self._descriptors(states, x2, ys, M)
        lib = _lib.load()
        st0 = states[0][0]
        if len(states) <= _lib.MAX_CHAIN_STAGES and len(flat) <= _lib.MAX_CHAIN:
            rc = lib.ssl_slr_forward_chain(M, st0.p, st0.q, st0.dtype_code, stages, len(states),
                                           members, len(flat), _lib.stream_ptr(x.device))
            _lib.check(rc, "ssl_slr_forward_chain")
        else:
            host = _ChainTable(x.device)
            host.build(M, st0, stages, len(states), members, len(flat))
            dev = self._table_dev
            if dev is None or dev.device != x.device or dev.numel() < host.nbytes:
                dev = self._table_dev = torch.empty(host.nbytes, dtype=torch.uint8, device=x.device)
            dev.copy_(host.array)  # from pageable memory: ordered before the launch
            host.launch(dev, x.device)
        outs = _outputs(flat, ys, [n for o in outf for n in o], tuple(lead))
        return tuple(tuple(outs[base[s]:base[s + 1]]) for s in range(len(states)))


class _ChainTable:
    """A chained launch's descriptor table in (16-byte aligned) host memory."""

    def __init__(self, device: torch.device) -> None:
        lib = _lib.load()
        self.nbytes = int(lib.ssl_slr_chain_table_bytes())
        self._buf = np.zeros(self.nbytes + 16, dtype=np.uint8)
        off = (-self._buf.ctypes.data) % 16
        self._np = self._buf[off:off + self.nbytes]
        self.array = torch.from_numpy(self._np)
        self.device = device

    def build(self, M, st0, stages, n_stages, members, n_members) -> None:
        rc = _lib.load().ssl_slr_chain_table_build(M, st0.p, st0.q, st0.dtype_code, stages,
                                                   n_stages, members, n_members,
                                                   self._np.ctypes.data, self.nbytes)
        _lib.check(rc, "ssl_slr_chain_table_build")

    def launch(self, dev: torch.Tensor, device: torch.device) -> None:
        rc = _lib.load().ssl_slr_chain_table_launch(self._np.ctypes.data, dev.data_ptr(),
                                                    _lib.stream_ptr(device))
        _lib.check(rc, "ssl_slr_chain_table_launch")


class PreparedChain:
    """An LRSLinearChain bound to a fixed input buffer and its own output
    buffers, with its descriptor table built and in device memory: run()
    launches the whole chain (one launch, whatever its number of stages) and
    returns the outputs, stage by stage, as the chain's forward would. Each
    run() overwrites the outputs of the previous one. The buffers' contents
    may change between runs; their addresses may not. The table holds the
    kernel views of the weights as prepare() found them: after a module's
    weights change, prepare again (run(check=True) raises if they did)."""

    def __init__(self, chain: LRSLinearChain, x: torch.Tensor) -> None:
        first = chain.groups[0].members[0]
        if x.dtype != first.A.dtype or x.device != first.A.device:
            raise ValueError("x must have the weights' dtype and device")
        if x.dim() != 2 or x.shape[-1] != chain.in_features:
            raise ValueError(f"x must be [M, {chain.in_features}]")
        if x.stride(-1) != 1 or x.data_ptr() % 16 or (x.stride(0) * x.element_size()) % 16:
            raise ValueError("x rows must be contiguous and 16-byte aligned")
        states = [[mod._kernel() for mod in grp.members] for grp in chain.groups]
        M = x.shape[0]
        if not chain._chained(states, M):
            raise ValueError(f"calls of {M} token rows run the stages one by one; prepare serves "
                             "the chained launch (decode sizes, 16-bit activations)")
        self.x = x
        self._keys = [[st.key for st in sts] for sts in states]
        self._chain = chain
        flat = [st for sts in states for st in sts]
        self._ys = [torch.empty(M, st.n_pad, dtype=x.dtype, device=x.device) for st in flat]
        members, stages, base, self._frags = chain._descriptors(states, x, self._ys, M)
        self._host = _ChainTable(x.device)
        self._host.build(M, states[0][0], stages, len(states), members, len(flat))
        self._dev = self._host.array.to(x.device)
        outf = [[mod.out_features for mod in grp.members] for grp in chain.groups]
        outs = _outputs(flat, self._ys, [n for o in outf for n in o], (M,))
        self.outputs = tuple(tuple(outs[base[s]:base[s + 1]]) for s in range(len(states)))
        self.n_stages, self.n_linears = len(states), len(flat)

    def run(self, check: bool = False) -> tuple[tuple[torch.Tensor, ...], ...]:
        _runtime.check_status(self.x.device)
        if check:
            keys = [[mod._weights_key() for mod in grp.members] for grp in self._chain.groups]
            if keys != self._keys:
                raise RuntimeError("the chain's weights changed since prepare(); prepare it again")
        self._host.launch(self._dev, self.x.device)
        return self.outputs
