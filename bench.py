"""Benchmark: decode throughput of the SLR linears of a LLaMA-1B-shaped stack.

Workload (default): 24 layers × {q, k, v, o: 2048×2048; gate, up: 5461×2048;
down: 2048×5461} sparse-plus-low-rank linears, bf16, rank 256, 32×32 BSR blocks
at 50% block density, seeded random weights, decode batch M = 16 tokens. One
step = one pass of a batch through all 168 linears (y = x·Bᵀ·Aᵀ + x·Sᵀ), i.e.
the projection work of one decode step. Weights (1.69 GB) exceed the 256 MB
last-level cache, so every step streams them from HBM.

Data flow: each layer's projections read what the previous one wrote, in
the order of a decoder layer: q, k, v read the layer input; o reads q's output
(attention's output in a model); gate and up read o's output (the normed
residual); down reads gate's output (silu(gate)·up); the next layer reads
down's output. So every projection waits for the one before it, as in decode.

Launches: one chained launch per layer (LRSLinearChain: the stages q,k,v |
o | gate,up | down, each waiting inside the launch for its input), 24 per
step. --stack: ONE launch for the 96 stages of all 24 layers (a prepared
chain with its descriptor table in device memory; measured a few percent
slower at 16 rows: later layers' workgroups, dispatched into whichever slots
free up, crowd the compute units of the running stage); --no-chain: the
stages as grouped launches (LRSLinearGroup), 4 per layer, 96 per step;
--no-group: one launch per linear, 168 per step. Calls the chained kernel does
not serve (the 2048-token prefill detail) run the stages as grouped launches.

Timing: the step is captured once in a HIP graph and replayed; W untimed
replays, then K replays bracketed by synchronize + HIP events on the replay
stream. value = M·K / elapsed (tokens/s).

roofline: every launch of the step is the fused kernel (latent, sparse blocks,
t·Aᵀ and epilogue; chained: a layer's four stages); its average launch
duration = the HIP-event time of the graph replays / launches per step (gaps
between launches included, so this slightly understates the kernel);
achieved = algorithmic bytes per launch / that duration.

cpu_baseline: the reference AVX2 BSR kernel (oracle/_ref, compiled from the
reference's own source) plus torch-CPU F.linear ×2 — the reference's CPU
forward, fp32 — timed on this host on a sample (one layer's 7 linears, repeated
for ~10 s) and scaled to the 24-layer step.

Other workloads (--workload, one JSON line each; the default above is the
headline):
  llama7b_ffn_decode   one 11008×4096 SLR linear (64×64 blocks at 50%, r 256,
                       bf16), --batch tokens (default 1), 8 weight copies
                       cycled in a HIP graph: GB/s of algorithmic bytes
  llama7b_ffn_prefill  the same linear at 2048 tokens (one launch: the latent
                       t = x·Bᵀ workgroups, then the row workgroups for
                       x·Sᵀ + t·Aᵀ + b): TFLOP/s
  llama7b_lr_prefill   the low-rank share of that linear alone (S = 0: the
                       two GEMMs x·Bᵀ and t·Aᵀ) at 2048 tokens: TFLOP/s, with
                       torch's two F.linear calls on the same tensors beside it
  skew_prefill         one point of the skew sweep (4096x11008, r 128, Zipf(1.2)
                       rows of --block blocks at --density, --batch tokens, 2048
                       by default): TFLOP/s
  llama7b_ffn_prefill_nm24  the 2:4 projection of llama7b_ffn_decode_nm24 at
                       2048 tokens: TFLOP/s of the dense-equivalent work
                       (x·Bᵀ, t·Aᵀ and the kept half of S)
  block_topk           the compression loop's block projection (project_S) of
                       an 11008×4096 fp32 matrix, 64×64 blocks (--block P for
                       P×P), half kept: GB/s of compulsory traffic
  dense_to_bsr         the encoder (encode_for_kernels: flags, row counts,
                       crow, col and (q, p) values) of an 11008×4096 bf16
                       matrix with half of its 64×64 blocks (--block P) zero:
                       GB/s of compulsory traffic (read the matrix, write the
                       kept blocks)
  project_nm           the compression loop's N:M projection (project_S_nm,
                       2:4) of an 11008×4096 fp32 matrix: GB/s of compulsory
                       traffic (read it, write fp32 and the keep bytes)
  llama7b_ffn_decode_nm24  the same projection with 2:4 S (two of every four
                       input features kept, N(0, 0.02)) instead of blocks:
                       GB/s of algorithmic bytes (values plus 4-bit
                       positions per group)
  llama60m_forward     the LLaMA-60M-shaped decoder (8 layers, hidden 512, 8
                       heads, FFN 1376, vocab 32000) with every q/k/v/o/gate/
                       up/down an SLR linear (rank dim/4, 32×32 blocks at 50%,
                       N(0, 0.02)), fp32 forward of 8 × 256 tokens: tok/s
  sweep                the LLaMA-7B layer set (11008x4096, 4096x11008, 4096x4096;
                       64x64 blocks at 30/50/70%; r 256; 1, 16, 256, 2048 tokens)
                       and the skew sweep (4096x11008, r 128, Zipf(1.2) rows at
                       10/50/90% mean density, blocks 16/32/64, 1 and 2048
                       tokens): one JSON line with every point in "points"
  llama1b_prefill      the default workload's 24-layer projection stack at 2048
                       tokens (one HIP graph of the 96 grouped launches): TFLOP/s
  llama1b_decode_step  the whole KV-cached decode step of the LLaMA-1B-shaped
                       model (the projection stack above, plus RMSNorm, rotary
                       embedding, attention over a 1024-token context of
                       synthetic keys/values, SiLU, residuals and a 32000-word
                       LM head), --batch sequences (default 16), one HIP graph
                       per step: tok/s, and GB/s of the step's compulsory
                       bytes (weights plus the keys and values read)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "s-salaad_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
# the dominant kernel of the default workload's launches, by launch mode
KERNEL_NAMES = {
    "stack": "slr_chain_tab_kernel<1, 32, 8, 1, 4, 0, true> (bf16, p 32, KE 8, MT 1, UNR 4, BSR, "
             "fragment-order stage inputs): one launch per step, 96 stages (24 layers × "
             "q,k,v | o | gate,up | down)",
    "chain": "slr_chain_kernel<1, 32, 8, 1, 4, 0, true> (bf16, p 32, KE 8, MT 1, UNR 4, BSR, "
             "fragment-order stage inputs): one launch per layer, stages q,k,v | o | gate,up | down",
    "groups": "slr_kernel<1, 32, 8, 1, 1, 4, 0> (bf16, p 32, KE 8, MT 1, fused, UNR 4, BSR)",
    "linears": "slr_kernel<1, 32, 8, 1, 1, 4, 0> (bf16, p 32, KE 8, MT 1, fused, UNR 4, BSR)",
}
METRIC = "SLR-linear GB/s & TFLOP/s (% roofline); decode tok/s at LLaMA-1B shape"


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------- workloads --


def llama1b_shapes():
    h, f = 2048, 5461
    return [("q", h, h), ("k", h, h), ("v", h, h), ("o", h, h), ("gate", f, h), ("up", f, h),
            ("down", h, f)]


def zipf_row_counts(NB: int, NBK: int, density: float, gen, s: float = 1.2):
    """Blocks per row ∝ rank^-s over a seeded permutation of the rows, water-filled
    to round(d·NB·NBK) blocks in all under the cap of NBK per row."""
    import torch

    target = int(round(density * NB * NBK))
    w = torch.arange(1, NB + 1, dtype=torch.float64) ** (-s)
    w = w[torch.randperm(NB, generator=gen)]
    counts = torch.zeros(NB, dtype=torch.int64)
    remaining = target
    while remaining > 0:
        free = counts < NBK
        if not bool(free.any()):
            break
        share = w * free
        add = torch.minimum((share / share.sum() * remaining).floor().long(), NBK - counts)
        if int(add.sum()) == 0:  # the remainder one at a time, largest weight first
            for i in torch.argsort(-share).tolist():
                if remaining == 0:
                    break
                if counts[i] < NBK:
                    counts[i] += 1
                    remaining -= 1
            break
        counts += add
        remaining -= int(add.sum())
    return counts


def make_linear(n, m, r, p, density, gen, dev, dtype, skew=False):
    """Random SLR linear with exactly round(d·NB·NBK) blocks: uniformly placed,
    or with Zipf(1.2) row counts (skew) and uniform columns within each row."""
    import torch

    from ssalaad_amd import LRSLinear

    NB, NBK = -(-n // p), -(-m // p)
    if skew:
        counts = zipf_row_counts(NB, NBK, density, gen)
        rows = torch.repeat_interleave(torch.arange(NB), counts)
        cols = torch.cat([torch.randperm(NBK, generator=gen)[: int(c)].sort().values
                          for c in counts])
        k = int(counts.sum())
    else:
        k = int(round(density * NB * NBK))
        slots = torch.randperm(NB * NBK, generator=gen, device="cpu")[:k].sort().values
        rows, cols = slots // NBK, slots % NBK
    crow = torch.zeros(NB + 1, dtype=torch.int64)
    crow[1:] = torch.bincount(rows, minlength=NB).cumsum(0)
    vals = (torch.randn(k, p, p, generator=gen, device="cpu") * 0.02).to(dtype)
    # zero the padding of ragged edge blocks
    if n % p:
        edge = rows == NB - 1
        vals[edge, n - (NB - 1) * p:, :] = 0
    if m % p:
        edge = cols == NBK - 1
        vals[edge, :, m - (NBK - 1) * p:] = 0
    S = torch.sparse_bsr_tensor(crow.to(dev), cols.to(dev), vals.to(dev), size=(NB * p, NBK * p))
    A = (torch.randn(n, r, generator=gen) * 0.02).to(dtype).to(dev)
    B = (torch.randn(r, m, generator=gen) * 0.02).to(dtype).to(dev)
    mod = LRSLinear(A, B, S, in_features=m, out_features=n, bias=None, block_p=p, block_q=p)
    return mod


def algorithmic_bytes(mod, M: int, e: int) -> dict:
    """Compulsory traffic of one call: x, y, A, B, S values, indices, bias."""
    n, m, r, p = mod.out_features, mod.in_features, mod.r, mod.block_p
    nnz, NB = mod.S_nnz, -(-n // p)
    idx = 4 * (nnz + 2 * NB + 1)
    bias = e * n if mod.bias is not None else 0
    total = e * M * (m + n) + e * r * (n + m) + e * nnz * p * p + idx + bias
    flops = 2 * M * r * (m + n) + 2 * M * nnz * p * p
    return dict(total=total, flops=flops)


# -------------------------------------------------------------- GPU leg --


def build_layers(args):
    """The LLaMA-1B projection stack: args.layers × 7 SLR linears (bf16, r 256,
    32×32 blocks at 50%), seeded."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(args.seed)
    t0 = time.time()
    layers = []
    for li in range(args.layers):
        layers.append([(name, make_linear(n, m, 256, 32, 0.5, gen, dev, torch.bfloat16))
                       for name, n, m in llama1b_shapes()])
    torch.cuda.synchronize()
    _log(f"[bench] built {args.layers}x7 SLR linears in {time.time() - t0:.1f}s")
    return layers


def run_gpu(args, layers=None, M=None, steps=None):
    """One step = every launch of the stack at M token rows (args.batch by
    default), replayed from a HIP graph unless --eager."""
    import torch

    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    e = 2
    M = args.batch if M is None else M
    steps = args.steps if steps is None else steps
    gen = torch.Generator().manual_seed(args.seed + 7)
    if layers is None:
        layers = build_layers(args)
    h, f = 2048, 5461
    x0 = torch.randn(M, h, generator=gen).to(dtype).to(dev)
    mods = [(name, mod) for layer in layers for name, mod in layer]
    bytes_ = [algorithmic_bytes(mod, M, e) for _, mod in mods]
    from ssalaad_amd import LRSLinearChain, LRSLinearGroup

    # per layer: q,k,v (layer input) | o (q's output) | gate,up (o's output) |
    # down (gate's output); the next layer reads down's output
    chains = []
    for layer in layers:
        d = dict(layer)
        chains.append(LRSLinearChain([[d["q"], d["k"], d["v"]], [d["o"]], [d["gate"], d["up"]],
                                      [d["down"]]], sources=[d["q"], d["o"], d["gate"]]))
    groups = [(LRSLinearGroup(*c.groups[0].members), c.groups[1].members[0],
               LRSLinearGroup(*c.groups[2].members), c.groups[3].members[0]) for c in chains]
    mode = ("linears" if args.no_group else "groups" if args.no_chain
            else "stack" if args.stack else "chain")
    stack = None
    if mode == "stack":
        stages, sources = [], []
        for li, c in enumerate(chains):
            if li > 0:
                sources.append(chains[li - 1].groups[3].members[0])
            stages += [list(g.members) for g in c.groups]
            sources += [c.groups[0].members[0], c.groups[1].members[0], c.groups[2].members[0]]
        stack = LRSLinearChain(stages, sources)
        st = [[m._kernel() for m in g.members] for g in stack.groups]
        if not stack._chained(st, M):
            mode = "groups"  # prefill sizes: the stages one by one

    def layer_fwd(li, x):
        """The layer's 7 outputs (q, k, v, o, gate, up, down)."""
        if mode in ("chain", "stack"):
            return [y for stage in chains[li](x) for y in stage]
        d = dict(layers[li])
        if mode == "groups":
            g_qkv, m_o, g_gu, m_d = groups[li]
            q, k, v = g_qkv(x)
            o = m_o(q)
            g, u = g_gu(o)
            return [q, k, v, o, g, u, m_d(g)]
        q, k, v = d["q"](x), d["k"](x), d["v"](x)
        o = d["o"](q)
        g, u = d["gate"](o), d["up"](o)
        return [q, k, v, o, g, u, d["down"](g)]

    def step():
        outs, x = [], x0
        for li in range(len(layers)):
            ys = layer_fwd(li, x)
            outs.append((x, ys))
            x = ys[-1]
        return outs

    if mode == "stack":
        prep = stack.prepare(x0)

        def step():  # noqa: F811  (the whole stack in one launch)
            return [y for stage in prep.run() for y in stage]

        n_launch = 1
    elif mode == "chain":
        st = [[m._kernel() for m in g.members] for g in chains[0].groups]
        n_launch = len(layers) * (1 if chains[0]._chained(st, M) else 4)
    else:
        n_launch = len(layers) * (4 if mode == "groups" else 7)

    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        keep = step()
    torch.cuda.synchronize()
    if args.eager:
        # launches issued one by one (hardware counters are collected per
        # dispatch, which graph replays do not expose)
        run = step
    else:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            keep = step()
        torch.cuda.synchronize()
        run = g.replay

    with torch.cuda.stream(s):
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record(s)
        for _ in range(steps):
            run()
        ev1.record(s)
        torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / steps
    n_lin = len(mods)
    total_bytes = sum(b["total"] for b in bytes_)
    total_flops = sum(b["flops"] for b in bytes_)
    avg_us = ms_step * 1e3 / n_launch
    achieved = total_bytes / n_launch / (avg_us * 1e-6) / 1e9
    res = dict(
        ms_step=ms_step,
        tok_s=M / (ms_step * 1e-3),
        step_tflops=total_flops / (ms_step * 1e-3) / 1e12,
        avg_launch_us=avg_us,
        achieved_gbs=achieved,
        bytes_per_launch=total_bytes / n_launch,
        total_bytes_per_step=total_bytes,
        n_linears=n_lin,
        n_launches=n_launch,
    )
    # a parity spot check of the timed graph: the whole stack (or its last
    # layer, from the input the graph gave it) recomputed eagerly
    if mode == "stack":
        ref = [y for stage in stack(x0) for y in stage]
        torch.cuda.synchronize()
        res["graph_matches_eager"] = all(bool(torch.equal(a, b)) for a, b in zip(keep, ref))
    else:
        x_last, ys_last = keep[-1]
        ref = layer_fwd(len(layers) - 1, x_last)
        torch.cuda.synchronize()
        res["graph_matches_eager"] = all(bool(torch.equal(a, b)) for a, b in zip(ys_last, ref))
    res["mode"] = mode
    from ssalaad_amd.ls_linear import latent_wait_status

    with torch.cuda.stream(s):
        res["status"] = latent_wait_status(dev)
    res["status"] = max(res["status"], latent_wait_status(dev))
    return res


def _time_graph(fns, reps):
    """Mean µs per call of `fns` (called in turn) replayed in a HIP graph."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for f in fns:
            f()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for f in fns:
                f()
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            g.replay()
        e1.record(s)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps / len(fns)


def _time_calls(fns, reps, eager: bool):
    """µs per call of `fns` called in turn: replayed in a HIP graph, or with
    --eager issued one by one (hardware counters are collected per dispatch)."""
    if not eager:
        return _time_graph(fns, reps)
    n = len(fns)
    return _time_eager(lambda: [f() for f in fns], max(1, reps // n)) / n


def _time_eager(fn, reps):
    import torch

    fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def eager_calls(layers, M: int, reps: int) -> dict:
    """The drop-in path's per-call cost: module calls made one by one from
    Python, as a Hugging Face forward makes them (LRSLinear.forward, eager),
    against the same calls replayed from a HIP graph. The calls cycle through
    the 24 layers' gate projections (5461×2048), so the weights stream from
    HBM. host_issue_us is the host's time to issue one call (no waiting)."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(M, 2048, generator=gen).to(torch.bfloat16).to(dev)
    fns = [lambda md=dict(layer)["gate"]: md(x) for layer in layers]
    graph_us = _time_graph(fns, reps)
    for f in fns:
        f()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    t0 = time.perf_counter()
    for _ in range(reps):
        for f in fns:
            f()
    host = time.perf_counter() - t0
    e1.record()
    torch.cuda.synchronize()
    calls = reps * len(fns)
    eager_us = e0.elapsed_time(e1) * 1e3 / calls
    return {"eager_call_us": round(eager_us, 3), "graph_call_us": round(graph_us, 3),
            "host_issue_us": round(host * 1e6 / calls, 3),
            "eager_overhead_us": round(eager_us - graph_us, 3)}


def run_workload(args) -> dict:
    """The non-default workloads (see the module docstring)."""
    import torch

    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(args.seed)
    n, m, r, p = 11008, 4096, 256, 64
    base = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "data": "synthetic", "cpu_baseline": None}
    if args.workload == "llama7b_ffn_decode":
        M = args.batch if args.batch_set else 1
        mods = [make_linear(n, m, r, p, 0.5, gen, dev, torch.bfloat16) for _ in range(8)]
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        sts = [md._kernel() for md in mods]
        us = _time_calls([lambda st=st: st.forward(x, n) for st in sts], args.steps, args.eager)
        b = algorithmic_bytes(mods[0], M, 2)["total"]
        gbs = b / us / 1e3
        return dict(base, metric="SLR-linear decode GB/s (LLaMA-7B FFN projection)",
                    value=round(gbs, 1), unit="GB/s", ms_per_step=round(us / 1e3, 5), dtype="bf16",
                    config={"workload": "llama7b_ffn_decode", "n": n, "m": m, "rank": r,
                            "block": p, "block_density": 0.5, "batch_tokens": M,
                            "weight_copies": 8, "parallelism": "single_gpu"},
                    roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "traffic": None, "algorithmic_bytes_per_launch": int(b),
                              "avg_launch_us": round(us, 3)})
    if args.workload == "llama7b_ffn_decode_nm24":
        from ssalaad_amd import LRSLinear

        M = args.batch if args.batch_set else 1
        mods = []
        for _ in range(8):  # --pair: four (gate, up) pairs in grouped launches
            grp = torch.rand(n, m // 4, 4, generator=gen).argsort(dim=-1).argsort(dim=-1) < 2
            S = (torch.randn(n, m, generator=gen) * 0.02 * grp.reshape(n, m)).to(torch.bfloat16)
            A = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
            B = (torch.randn(r, m, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
            mods.append(LRSLinear(A, B, S.to(dev), in_features=m, out_features=n, nm_n=2, nm_m=4))
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        b = 2 * M * (m + n) + 2 * r * (n + m) + 2 * (n * m // 2) + n * m // 8
        if args.pair:
            from ssalaad_amd import LRSLinearGroup

            grps = [LRSLinearGroup(mods[2 * i], mods[2 * i + 1]) for i in range(4)]
            us = _time_calls([lambda g=g: g(x) for g in grps], args.steps, args.eager)
            b = 2 * b - 2 * M * m  # two projections, one read of x
        else:
            sts = [md._kernel() for md in mods]
            us = _time_calls([lambda st=st: st.forward(x, n) for st in sts], args.steps, args.eager)
        gbs = b / us / 1e3
        return dict(base, metric="SLR-linear decode GB/s (LLaMA-7B FFN projection, 2:4 S)",
                    value=round(gbs, 1), unit="GB/s", ms_per_step=round(us / 1e3, 5), dtype="bf16",
                    config={"workload": "llama7b_ffn_decode_nm24", "n": n, "m": m, "rank": r,
                            "sparsity": "2:4", "batch_tokens": M, "weight_copies": 8,
                            "linears_per_launch": 2 if args.pair else 1,
                            "parallelism": "single_gpu"},
                    roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "traffic": None, "algorithmic_bytes_per_launch": int(b),
                              "stored_bytes_per_launch": int((2 if args.pair else 1) * (
                                  2 * r * (n + m) + (n // 32) * (m // 32) * 1280)),
                              "avg_launch_us": round(us, 3)})
    if args.workload == "llama7b_ffn_prefill":
        M = args.batch if args.batch_set else 2048
        mod = make_linear(n, m, r, p, 0.5, gen, dev, torch.bfloat16)
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        us = _time_eager(lambda: mod(x), args.steps)
        fl = algorithmic_bytes(mod, M, 2)["flops"]
        tf = fl / us / 1e6
        return dict(base, metric="SLR-linear prefill TFLOP/s (LLaMA-7B FFN projection)",
                    value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(us / 1e3, 5),
                    dtype="bf16",
                    config={"workload": "llama7b_ffn_prefill", "n": n, "m": m, "rank": r,
                            "block": p, "block_density": 0.5, "batch_tokens": M,
                            "parallelism": "single_gpu"},
                    roofline={"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "flops_per_call": int(fl), "low_rank_flops": 2 * M * r * (m + n)})
    if args.workload == "llama7b_lr_prefill":
        # The low-rank share of the same projection alone: S ≡ 0 gives the
        # low-rank-only module (ls_linear.py:47-54), whose call is the two GEMMs
        # t = x·Bᵀ, y = t·Aᵀ of ls_linear.py:131 in one launch. torch's own two
        # F.linear calls (the library GEMMs the reference makes there) are timed
        # on the same tensors beside it.
        import torch.nn.functional as F

        from ssalaad_amd import LRSLinear

        M = args.batch if args.batch_set else 2048
        A = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
        B = (torch.randn(r, m, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
        mod = LRSLinear(A, B, torch.zeros(n, m, dtype=torch.bfloat16, device=dev),
                        in_features=m, out_features=n)
        assert mod.kind == "lr_only"
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        us = _time_graph([lambda: mod(x)], args.steps)
        us_call = _time_eager(lambda: mod(x), args.steps)
        us_lib = _time_graph([lambda: F.linear(F.linear(x, B), A)], args.steps)
        fl = 2 * M * r * (m + n)
        tf = fl / us / 1e6
        byt = 2 * (M * (m + n) + r * (m + n))
        return dict(base, metric="SLR-linear prefill low-rank share TFLOP/s (LLaMA-7B FFN "
                    "projection, S = 0)",
                    value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(us / 1e3, 5),
                    dtype="bf16",
                    config={"workload": "llama7b_lr_prefill", "n": n, "m": m, "rank": r,
                            "batch_tokens": M, "parallelism": "single_gpu"},
                    roofline={"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "flops_per_call": int(fl), "compulsory_bytes": int(byt),
                              "hbm_frac_at_this_time": round(byt / us / 1e3 / HBM_PEAK_GBS, 4)},
                    details={"call_us_eager": round(us_call, 3), "kernel_us_graph": round(us, 3),
                             "torch_two_linears_us_graph": round(us_lib, 3),
                             "torch_two_linears_TFLOPs": round(fl / us_lib / 1e6, 1)})
    if args.workload == "skew_prefill":
        # one point of the skew sweep: 4096x11008, r 128, Zipf(1.2) rows of
        # --block blocks at --density mean density, --batch tokens (2048)
        M = args.batch if args.batch_set else 2048
        mod = make_linear(4096, 11008, 128, args.block, args.density, gen, dev, torch.bfloat16,
                          skew=True)
        x = torch.randn(M, 11008, generator=gen).to(torch.bfloat16).to(dev)
        us = _time_eager(lambda: mod(x), args.steps)
        fl = algorithmic_bytes(mod, M, 2)["flops"]
        tf = fl / us / 1e6
        return dict(base, metric="SLR-linear TFLOP/s, skewed (Zipf 1.2) block rows",
                    value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(us / 1e3, 5),
                    dtype="bf16",
                    config={"workload": "skew_prefill", "n": 4096, "m": 11008, "rank": 128,
                            "block": args.block, "mean_block_density": args.density,
                            "batch_tokens": M, "parallelism": "single_gpu"},
                    roofline={"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "flops_per_call": int(fl)})
    if args.workload == "llama7b_ffn_prefill_nm24":
        from ssalaad_amd import LRSLinear

        M = args.batch if args.batch_set else 2048
        grp = torch.rand(n, m // 4, 4, generator=gen).argsort(dim=-1).argsort(dim=-1) < 2
        S = (torch.randn(n, m, generator=gen) * 0.02 * grp.reshape(n, m)).to(torch.bfloat16)
        A = (torch.randn(n, r, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
        B = (torch.randn(r, m, generator=gen) * 0.02).to(torch.bfloat16).to(dev)
        mod = LRSLinear(A, B, S.to(dev), in_features=m, out_features=n, nm_n=2, nm_m=4)
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        us = _time_eager(lambda: mod(x), args.steps)
        fl = 2 * M * r * (m + n) + 2 * M * n * (m // 2)
        tf = fl / us / 1e6
        return dict(base, metric="SLR-linear prefill TFLOP/s (LLaMA-7B FFN projection, 2:4 S)",
                    value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(us / 1e3, 5),
                    dtype="bf16",
                    config={"workload": "llama7b_ffn_prefill_nm24", "n": n, "m": m, "rank": r,
                            "sparsity": "2:4", "batch_tokens": M, "parallelism": "single_gpu"},
                    roofline={"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "flops_per_call": int(fl), "low_rank_flops": 2 * M * r * (m + n)})
    if args.workload == "block_topk":
        import ssalaad_amd

        if args.block_set:
            p = args.block
            if n % p or m % p:
                raise SystemExit(f"--block {p} does not divide {n}x{m}")
        Mt = torch.randn(n, m, generator=gen).to(dev)
        keep = (n // p) * (m // p) // 2
        us = _time_eager(lambda: ssalaad_amd.block_topk(Mt, keep, p, p), args.steps)
        b = n * m * 4 * 3 + (n // p) * (m // p) * 5  # read twice, write fp32 once; norms + flags
        gbs = b / us / 1e3
        return dict(base, metric=f"block projection GB/s (project_S, 11008x4096 fp32, {p}x{p} blocks)",
                    value=round(gbs, 1), unit="GB/s", ms_per_step=round(us / 1e3, 5), dtype="f32",
                    config={"workload": "block_topk", "n": n, "m": m, "block": p,
                            "blocks_kept": keep, "parallelism": "single_gpu"},
                    roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "traffic": None, "bytes_per_call": int(b)})
    if args.workload == "dense_to_bsr":
        from ssalaad_amd.artifact import encode_for_kernels

        p = args.block if args.block_set else 64
        if n % p or m % p:
            raise SystemExit(f"--block {p} does not divide {n}x{m}")
        keep_blocks = torch.rand(n // p, m // p, generator=gen) < 0.5
        mask = keep_blocks.repeat_interleave(p, 0).repeat_interleave(p, 1)
        St = (torch.randn(n, m, generator=gen) * mask).to(torch.bfloat16).to(dev)
        kept = int(keep_blocks.sum())
        us = _time_eager(lambda: encode_for_kernels(St, p, p), args.steps)
        b = n * m * 2 + kept * p * p * 2 + kept * 4 + (n // p + 1) * 4
        gbs = b / us / 1e3
        return dict(base, metric=f"BSR encode GB/s (encode_for_kernels, 11008x4096 bf16, {p}x{p} blocks)",
                    value=round(gbs, 1), unit="GB/s", ms_per_step=round(us / 1e3, 5),
                    dtype="bf16",
                    config={"workload": "dense_to_bsr", "n": n, "m": m, "block": p,
                            "blocks_kept": kept, "parallelism": "single_gpu"},
                    roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "traffic": None, "bytes_per_call": int(b)})
    if args.workload == "project_nm":
        import ssalaad_amd

        Rt = torch.randn(n, m, generator=gen).to(dev)
        us = _time_eager(lambda: ssalaad_amd.project_nm(Rt, 2, 4), args.steps)
        b = n * m * (4 + 4 + 1)  # read fp32, write fp32 and the keep bytes
        gbs = b / us / 1e3
        return dict(base, metric="N:M projection GB/s (project_nm 2:4, 11008x4096 fp32)",
                    value=round(gbs, 1), unit="GB/s", ms_per_step=round(us / 1e3, 5), dtype="f32",
                    config={"workload": "project_nm", "n": n, "m": m, "nm": "2:4",
                            "parallelism": "single_gpu"},
                    roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                              "traffic": None, "bytes_per_call": int(b)})
    if args.workload == "llama60m_forward":
        from ssalaad_amd import LRSLinear
        from ssalaad_amd.bundle import build_model_from_config

        cfg = {"model_type": "llama", "hidden_size": 512, "intermediate_size": 1376,
               "num_hidden_layers": 8, "num_attention_heads": 8, "num_key_value_heads": 8,
               "vocab_size": 32000, "max_position_embeddings": 256, "rms_norm_eps": 1e-6,
               "hidden_act": "silu", "bos_token_id": 1, "eos_token_id": 2, "pad_token_id": 0,
               "tie_word_embeddings": False}
        torch.manual_seed(args.seed)
        model = build_model_from_config(cfg, attn_implementation="sdpa").eval()
        projs = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                 "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]
        total_bytes = 0
        for li in range(cfg["num_hidden_layers"]):
            for proj in projs:
                parent = model.get_submodule(f"model.layers.{li}.{proj.split('.')[0]}")
                old = getattr(parent, proj.split(".")[1])
                nn_, mm = old.out_features, old.in_features
                rr, pp = min(nn_, mm) // 4, 32
                NB, NBK = nn_ // pp, mm // pp
                k = NB * NBK // 2
                slots = torch.randperm(NB * NBK, generator=gen)[:k].sort().values
                crow = torch.zeros(NB + 1, dtype=torch.int64)
                crow[1:] = torch.bincount(slots // NBK, minlength=NB).cumsum(0)
                vals = torch.randn(k, pp, pp, generator=gen) * 0.02
                S = torch.sparse_bsr_tensor(crow.to(dev), (slots % NBK).to(dev), vals.to(dev),
                                            size=(nn_, mm))
                A = (torch.randn(nn_, rr, generator=gen) * 0.02).to(dev)
                B = (torch.randn(rr, mm, generator=gen) * 0.02).to(dev)
                mod = LRSLinear(A, B, S, in_features=mm, out_features=nn_, block_p=pp, block_q=pp)
                total_bytes += 4 * (rr * (nn_ + mm) + k * pp * pp)
                setattr(parent, proj.split(".")[1], mod)
        model = model.to(dev)
        ids = torch.randint(3, cfg["vocab_size"], (8, 256), generator=gen).to(dev)
        with torch.no_grad():
            us = _time_eager(lambda: model(input_ids=ids), max(3, args.steps // 5))
        tok_s = 8 * 256 / (us * 1e-6)
        return dict(base, metric="LLaMA-60M SLR forward tok/s (fp32, 8 x 256 tokens)",
                    value=round(tok_s, 1), unit="tok/s", ms_per_step=round(us / 1e3, 4), dtype="f32",
                    config={"workload": "llama60m_forward", "layers": 8, "hidden": 512, "ffn": 1376,
                            "heads": 8, "vocab": 32000, "rank": "dim/4", "block": 32,
                            "block_density": 0.5, "batch": 8, "seq_len": 256,
                            "slr_weight_bytes": total_bytes, "parallelism": "single_gpu"},
                    roofline=None)
    if args.workload == "llama1b_decode_step":
        return run_decode_step(args, base, gen, dev)
    if args.workload == "sweep":
        return run_sweep(args, base, gen, dev)
    if args.workload == "llama1b_prefill":
        M = args.batch if args.batch_set else 2048
        args.batch = M
        g = run_gpu(args)
        tf = g["step_tflops"]
        return dict(base, metric="LLaMA-1B projection stack prefill TFLOP/s (2048 tokens)",
                    value=round(tf, 1), unit="TFLOP/s", ms_per_step=round(g["ms_step"], 4),
                    dtype="bf16",
                    config={"workload": "llama1b_prefill", "layers": args.layers, "hidden": 2048,
                            "ffn": 5461, "rank": 256, "block": 32, "block_density": 0.5,
                            "batch_tokens": M, "launches_per_step": g["n_launches"],
                            "parallelism": "single_gpu"},
                    roofline={"bound": "mfma", "achieved": round(tf, 1), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "tok_s": round(g["tok_s"], 1)},
                    graph_matches_eager=g["graph_matches_eager"])
    raise SystemExit(f"unknown workload {args.workload}")


def run_sweep(args, base: dict, gen, dev) -> dict:
    """The LLaMA-7B layer-set and skew sweeps: one point per (shape, density,
    block, structure, tokens). Up to 256 tokens (HBM-bound) the weights are cycled
    over enough copies to exceed 600 MB in a HIP graph; 2048 tokens run eagerly
    on one copy (MFMA-bound). value = the 11008x4096, d 0.5, 1-token point."""
    import math

    import torch

    pts = []
    for (n, m) in ((11008, 4096), (4096, 11008), (4096, 4096)):
        for d in (0.3, 0.5, 0.7):
            for M in (1, 16, 256, 2048):
                pts.append(dict(set="llama7b", n=n, m=m, r=256, p=64, d=d, skew=False, M=M))
    for p in (16, 32, 64):
        for d in (0.1, 0.5, 0.9):
            for M in (1, 2048):
                pts.append(dict(set="skew", n=4096, m=11008, r=128, p=p, d=d, skew=True, M=M))
    out = []
    head = None
    for pt in pts:
        n, m, r, p, d, M = pt["n"], pt["m"], pt["r"], pt["p"], pt["d"], pt["M"]
        first = make_linear(n, m, r, p, d, gen, dev, torch.bfloat16, skew=pt["skew"])
        b = algorithmic_bytes(first, M, 2)
        wbytes = algorithmic_bytes(first, 0, 2)["total"]
        x = torch.randn(M, m, generator=gen).to(torch.bfloat16).to(dev)
        if M <= 256:
            copies = max(4, math.ceil(600e6 / wbytes))
            mods = [first] + [make_linear(n, m, r, p, d, gen, dev, torch.bfloat16, skew=pt["skew"])
                              for _ in range(copies - 1)]
            sts = [md._kernel() for md in mods]
            us = _time_graph([lambda st=st: st.forward(x, n) for st in sts],
                             max(20, args.steps // 2))
            del mods, sts
        else:
            copies = 1
            us = _time_eager(lambda: first(x), max(5, args.steps // 10))
        gbs = b["total"] / us / 1e3
        tf = b["flops"] / us / 1e6
        bound = "hbm" if M <= 256 else "mfma"
        frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tf / 2500.0
        rec = dict(pt, us=round(us, 3), gbs=round(gbs, 1), tflops=round(tf, 1), bound=bound,
                   frac=round(frac, 4), copies=copies, nnz=first.S_nnz)
        out.append(rec)
        if (pt["set"], n, m, d, M) == ("llama7b", 11008, 4096, 0.5, 1):
            head = rec
        _log(f"[sweep] {json.dumps(rec)}")
        del first, x
        torch.cuda.empty_cache()
    return dict(base, metric="SLR-linear sweep GB/s (LLaMA-7B set and skewed structures)",
                value=head["gbs"], unit="GB/s", ms_per_step=round(head["us"] / 1e3, 5),
                dtype="bf16",
                config={"workload": "sweep", "points": len(out), "parallelism": "single_gpu"},
                roofline={"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": head["frac"], "traffic": None},
                points=out)


def run_decode_step(args, base: dict, gen, dev) -> dict:
    """The LLaMA-1B-shaped decode step through DecodeEngine at a 1024-token context."""
    import torch
    from torch import nn

    from ssalaad_amd import DecodeEngine
    from ssalaad_amd.bundle import build_model_from_config

    B = args.batch if args.batch_set else 16
    ctx, vocab, h, f, layers = 1024, 32000, 2048, 5461, args.layers
    dtype = torch.bfloat16
    cfg = {"model_type": "llama", "hidden_size": h, "intermediate_size": f,
           "num_hidden_layers": layers, "num_attention_heads": 16, "num_key_value_heads": 16,
           "head_dim": 128, "vocab_size": vocab, "max_position_embeddings": ctx,
           "rms_norm_eps": 1e-5, "rope_theta": 500000.0, "hidden_act": "silu",
           "tie_word_embeddings": False}
    t0 = time.time()
    with torch.device("meta"):
        model = build_model_from_config(cfg, attn_implementation="sdpa")
    model = model.to_empty(device=dev).to(dtype)
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(torch.randn(vocab, h, generator=gen).to(dtype))
        model.lm_head.weight.copy_((torch.randn(vocab, h, generator=gen) * 0.02).to(dtype))
        for name, prm in model.named_parameters():
            if "norm" in name:
                prm.fill_(1.0)
    model.model.rotary_emb = type(model.model.rotary_emb)(config=model.config, device=dev)
    slr_bytes = 0
    for li in range(layers):
        lay = model.model.layers[li]
        for part, proj, (nm, n, m) in zip(
                ["self_attn"] * 4 + ["mlp"] * 3,
                ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"],
                llama1b_shapes()):
            mod = make_linear(n, m, 256, 32, 0.5, gen, dev, dtype)
            slr_bytes += algorithmic_bytes(mod, 0, 2)["total"]
            setattr(getattr(lay, part), proj, mod)
    model.eval()
    torch.cuda.synchronize()
    _log(f"[bench] built the {layers}-layer decode model in {time.time() - t0:.1f}s")
    eng = DecodeEngine(model, max_batch=B, max_context=ctx)
    with torch.no_grad():  # a full synthetic context: keys and values ~N(0, 1)
        for li in range(layers):
            eng.k_cache[li].copy_(torch.randn(eng.k_cache[li].shape, generator=gen).to(dtype))
            eng.v_cache[li].copy_(torch.randn(eng.v_cache[li].shape, generator=gen).to(dtype))
    tokens = torch.randint(0, vocab, (B,), generator=gen)
    positions = [ctx - 1] * B
    logits = eng.step(tokens, positions)  # eager run, then capture
    logits = eng.step(tokens, positions)
    torch.cuda.synchronize()
    finite = bool(torch.isfinite(logits).all())
    g, _ = eng._graphs[B]
    s = eng._stream
    with torch.cuda.stream(s):
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(args.steps):
            g.replay()
        e1.record(s)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    kv_bytes = layers * B * 2 * 16 * ctx * 128 * 2
    head_bytes = vocab * h * 2 + B * vocab * 2
    norm_bytes = (2 * layers + 1) * h * 2
    total = slr_bytes + kv_bytes + head_bytes + norm_bytes + B * h * 2
    gbs = total / (ms * 1e-3) / 1e9
    return dict(base, metric="LLaMA-1B decode step tok/s (KV cache, 1024-token context)",
                value=round(B / (ms * 1e-3), 1), unit="tok/s", ms_per_step=round(ms, 4),
                dtype="bf16",
                config={"workload": "llama1b_decode_step", "layers": layers, "hidden": h,
                        "ffn": f, "heads": 16, "kv_heads": 16, "head_dim": 128,
                        "vocab": vocab, "context": ctx, "batch_sequences": B, "rank": 256,
                        "block": 32, "block_density": 0.5, "parallelism": "single_gpu"},
                roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                          "step_bytes": int(total), "slr_weight_bytes": int(slr_bytes),
                          "kv_bytes": int(kv_bytes), "lm_head_bytes": int(head_bytes)},
                logits_finite=finite)


def copy_probe(mib: int, reps: int) -> None:
    """A plain device-to-device copy of `mib` MiB, `reps` times: the known-size
    kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the kernel's."""
    import torch

    dev = torch.device("cuda:0")
    a = torch.ones(mib << 18, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": mib << 20, "reps": reps}), flush=True)


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, calibrated on a plain copy)
    and the source revision the counters were measured at; None when absent."""
    out = {"bytes": None, "revision": None}
    path = ROOT / "profiles" / "slr_chain_kernel_llama1b_decode_counters.md"
    if not path.exists():
        return out
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            out["bytes"] = int(line.split(":", 1)[1].strip())
        elif line.startswith("measured_at_revision:"):
            out["revision"] = line.split(":", 1)[1].strip()
    return out


# -------------------------------------------------------------- CPU leg --


def cpu_model() -> str | None:
    """The host CPU's model name (lscpu, else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def run_cpu(args):
    """The reference CPU forward (AVX2 BSR kernel + F.linear ×2), fp32, one layer."""
    import numpy as np
    import torch
    import torch.nn.functional as F

    ref_dir = ROOT / "oracle" / "_ref"
    kind = "reference"
    sys.path.insert(0, str(ref_dir))
    try:
        import bsr_ref_avx2  # the reference kernel, built from its own source

        kernel = bsr_ref_avx2.bsr_addmm_avx2_
    except ImportError:
        kind = "port"
        import ctypes

        lib = ctypes.CDLL(str(ROOT / "oracle" / "liboracle.so"))
        f = lib.oracle_bsr_addmm_port
        f.restype = ctypes.c_int
        f.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int64] * 5 + [ctypes.c_int]

        def kernel(out, x, crow, col, vals, act):
            f(out.data_ptr(), x.data_ptr(), crow.data_ptr(), col.data_ptr(), vals.data_ptr(),
              act.data_ptr(), out.shape[0], x.shape[1], crow.numel() - 1, act.numel(),
              vals.shape[1], torch.get_num_threads())

    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        cores = min(cores, int(omp))
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(args.seed + 1)
    M, r, p, d = args.batch, 256, 32, 0.5
    lin = []
    for name, n, m in llama1b_shapes():
        NB, NBK = -(-n // p), -(-m // p)
        k = int(round(d * NB * NBK))
        slots = torch.randperm(NB * NBK, generator=gen)[:k].sort().values
        rows, cols = slots // NBK, slots % NBK
        crow = torch.zeros(NB + 1, dtype=torch.int32)
        crow[1:] = torch.bincount(rows, minlength=NB).cumsum(0).to(torch.int32)
        vals = torch.randn(k, p, p, generator=gen) * 0.02
        act = (crow[1:] - crow[:-1]).nonzero().squeeze(-1).to(torch.int32)
        A = torch.zeros(NB * p, r)
        A[:n] = torch.randn(n, r, generator=gen) * 0.02
        B = torch.zeros(r, NBK * p)
        B[:, :m] = torch.randn(r, m, generator=gen) * 0.02
        lin.append((name, A, B, crow, cols.to(torch.int32), vals, act, NBK * p))
    xs = {w: torch.randn(M, w, generator=gen) for w in {L[7] for L in lin}}

    def layer():
        for name, A, B, crow, col, vals, act, w in lin:
            y = F.linear(F.linear(xs[w], B), A).contiguous()
            kernel(y, xs[w], crow, col, vals, act)

    layer()
    t0 = time.perf_counter()
    layer()
    one = time.perf_counter() - t0
    reps = max(3, min(200, int(args.cpu_seconds / max(one, 1e-6))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
    t_layer = float(np.median(times))
    t_step = t_layer * args.layers
    return dict(
        value=M / t_step,
        unit="tok/s",
        cores=cores,
        cpu_model=cpu_model(),
        kind=kind,
        sample=(f"one layer's 7 linears (2048/5461-wide, r256, 32x32@50%), fp32, batch {M}, "
                f"median of {reps} runs = {t_layer * 1e3:.2f} ms, scaled x{args.layers} layers"),
    )


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-details", action="store_true",
                    help="time only the headline batch (skip M=1, M=4 and the 2048-token prefill)")
    ap.add_argument("--eager", action="store_true",
                    help="launch eagerly instead of replaying a HIP graph (default workload, "
                         "llama7b_ffn_decode and llama7b_ffn_decode_nm24)")
    ap.add_argument("--pair", action="store_true",
                    help="llama7b_ffn_decode_nm24: the projections in grouped pairs (gate, up)")
    ap.add_argument("--stack", action="store_true",
                    help="one chained launch for the whole stack instead of one per layer")
    ap.add_argument("--no-chain", action="store_true",
                    help="the four stages of a layer as grouped launches instead of one chained launch")
    ap.add_argument("--no-group", action="store_true",
                    help="one launch per linear instead of grouping q/k/v and gate/up")
    ap.add_argument("--block", type=int, default=None,
                    help="skew_prefill: block size (default 16); block_topk: square block size "
                         "(default 64)")
    ap.add_argument("--density", type=float, default=0.5, help="skew_prefill: mean block density")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter calibration)")
    ap.add_argument("--workload", default="llama1b_decode",
                    choices=["llama1b_decode", "llama7b_ffn_decode", "llama7b_ffn_prefill",
                             "llama7b_ffn_decode_nm24", "llama7b_ffn_prefill_nm24", "block_topk",
                             "dense_to_bsr", "project_nm",
                             "llama7b_lr_prefill", "skew_prefill",
                             "llama60m_forward",
                             "llama1b_decode_step", "sweep", "llama1b_prefill"])
    args = ap.parse_args()
    args.batch_set = args.batch is not None
    if args.batch is None:
        args.batch = 16
    args.block_set = args.block is not None
    if args.block is None:
        args.block = 16
    if args.copy_probe:
        copy_probe(args.copy_probe, max(1, args.steps))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported. The SLR linear "
              "shards by output block-rows with no exchange inside a layer, so one GPU's "
              "share at its real shape is what this benchmark measures.",
              file=sys.stderr)
        sys.exit(2)
    if args.workload != "llama1b_decode":
        line = run_workload(args)
        line["warmup"] = args.warmup
        print(json.dumps(line), flush=True)
        return
    _log("[bench] GPU leg")
    layers = build_layers(args)
    g = run_gpu(args, layers)
    _log(f"[bench] GPU: {g['ms_step']:.3f} ms/step, {g['tok_s']:.0f} tok/s")
    # the other decode batches and the 2048-token prefill of the same stack
    more = {}
    for M in (() if args.no_details else (1, 4)):
        gm = run_gpu(args, layers, M=M, steps=max(5, args.steps // 2))
        more[f"decode_M{M}"] = {
            "tok_s": round(gm["tok_s"], 1), "ms_per_step": round(gm["ms_step"], 4),
            "avg_launch_us": round(gm["avg_launch_us"], 3),
            "hbm_frac": round(gm["achieved_gbs"] / HBM_PEAK_GBS, 4)}
        _log(f"[bench] decode M={M}: {gm['ms_step']:.3f} ms/step")
    if not args.no_details and g["mode"] == "chain":
        # the same step as ONE chained launch over all 24 layers (the layers
        # chain directly here; a decoder runs attention and norms between them)
        import copy
        a1 = copy.copy(args)
        a1.stack = True
        gs = run_gpu(a1, layers, steps=max(5, args.steps // 2))
        more["stack_M16"] = {"tok_s": round(gs["tok_s"], 1), "ms_per_step": round(gs["ms_step"], 4),
                             "launches_per_step": gs["n_launches"]}
        _log(f"[bench] one launch for the stack: {gs['ms_step']:.3f} ms/step")
    for M in (() if args.no_details else (1, 16)):
        more[f"eager_gate_M{M}"] = eager_calls(layers, M, max(5, args.steps // 2))
        _log(f"[bench] eager gate calls M={M}: {more[f'eager_gate_M{M}']}")
    if not args.no_details:
        gp = run_gpu(args, layers, M=2048, steps=max(3, args.steps // 10))
        more["prefill_2048"] = {
            "tok_s": round(gp["tok_s"], 1), "ms_per_step": round(gp["ms_step"], 4),
            "TFLOPs": round(gp["step_tflops"], 2),
            "mfma_frac": round(gp["step_tflops"] / 2500.0, 4)}
        _log(f"[bench] prefill 2048: {gp['ms_step']:.3f} ms/step")
    del layers
    cpu = None
    if not args.no_cpu:
        _log("[bench] CPU baseline leg")
        cpu = run_cpu(args)
        _log(f"[bench] CPU: {cpu['value']:.1f} tok/s on {cpu['cores']} cores ({cpu['kind']})")
    # the counters were measured for the default launch mode's kernel
    traffic = measured_traffic() if g["mode"] == "chain" else {"bytes": None, "revision": None}
    line = {
        "metric": METRIC,
        "value": round(g["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "llama1b_slr_projections_decode",
            "layers": args.layers,
            "linears_per_step": g["n_linears"],
            "launches_per_step": g["n_launches"],
            "launch": g["mode"],
            "hidden": 2048,
            "ffn": 5461,
            "rank": 256,
            "block": 32,
            "block_density": 0.5,
            "batch_tokens": args.batch,
            "parallelism": "single_gpu",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(g["achieved_gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(g["achieved_gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic["bytes"],
            "traffic_revision": traffic["revision"],
            "kernel": KERNEL_NAMES[g["mode"]],
            "avg_launch_us": round(g["avg_launch_us"], 3),
            "algorithmic_bytes_per_launch": int(g["bytes_per_launch"]),
        },
        "cpu_baseline": cpu,
        "details": {
            **more,
            "step_TFLOPs": round(g["step_tflops"], 3),
            "bytes_per_step": int(g["total_bytes_per_step"]),
            "graph_matches_eager": g["graph_matches_eager"],
            "timing": "eager launches" if args.eager else "HIP graph replay",
            "latent_wait_status": g["status"],
        },
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
