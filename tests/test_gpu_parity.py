"""GPU parity of the HIP kernels against the oracle (through the C ABI).

Tolerances (max-abs normalised error, max|y−y_ref| / max|y_ref|):
  fp32  1e-5   bf16 / fp16  1e-2   structure (crow/col/active/values bits): exact.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "golden"))

from golden_inputs import CASES, make_case  # noqa: E402
from oracle import slr_oracle as orc  # noqa: E402
from slr_cases import (TOL, err, make_nm_module, make_problem, make_x, nm24_matrix,  # noqa: E402
                       oracle_y, round_to, sparse_bsr_tensor, to_dev)

import ssalaad_amd  # noqa: E402
from ssalaad_amd import LRSLinear, _lib, _runtime  # noqa: E402
from ssalaad_amd.ls_linear import latent_wait_status  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = np.load(ROOT / "tests" / "golden" / "bsr_addmm_avx2.npz")
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _op(out, x, crow, col, vt, act):
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(out, x, crow, col, vt, act)


# --------------------------------------------------- in-place BSR op --


@pytest.mark.parametrize("name", [c for c in CASES if not c.endswith("_b8") and "_b8_" not in c])
def test_op_matches_reference_kernel_golden_outputs(name, gpu_device):
    c = make_case(name)
    dev = gpu_device
    out = torch.from_numpy(c["out"].copy()).to(dev)
    args = [torch.from_numpy(c[k]).to(dev) for k in ("x", "crow", "col", "values_t", "active")]
    _op(out, *args)
    torch.cuda.synchronize()
    ref = GOLDEN[f"{name}__out"]
    got = out.cpu().numpy()
    assert orc.max_abs_normalised_error(got, ref) <= 1e-5
    # block-rows without blocks are bit-identical to the input
    p = c["block"]
    for by in range(len(c["crow"]) - 1):
        if by not in set(c["active"].tolist()):
            assert np.array_equal(got[:, by * p:(by + 1) * p], c["out"][:, by * p:(by + 1) * p])


def test_op_rejects_block_8(gpu_device):
    """Block sides must be multiples of 16, as for the TileLang kernel."""
    c = make_case("reftest_b8")
    out = torch.from_numpy(c["out"].copy()).to(gpu_device)
    args = [torch.from_numpy(c[k]).to(gpu_device) for k in ("x", "crow", "col", "values_t", "active")]
    with pytest.raises(ValueError, match="divisible by 16"):
        _op(out, *args)


def _op_case(dtype, p, M, skew, seed, dev):
    prob = make_problem(8 * p, 12 * p, 4, p, 0.1 if skew else 0.5, dtype, seed=seed, skew=skew)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=seed + 7)
    out0 = orc.bf16_round(np.random.default_rng(seed).standard_normal((M, prob["n"]))).astype(np.float64)
    out0 = torch.from_numpy(out0).to(dtype).double().numpy()
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    out = to_dev(out0, dtype, dev)
    _op(out, to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev), torch.from_numpy(col32).to(dev),
        to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    return out, want, out0, act, prob


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("M", [1, 3, 16, 17, 40, 64, 65, 200])
def test_op_matches_oracle(dtype, p, M, gpu_device):
    out, want, out0, act, prob = _op_case(dtype, p, M, False, 10 * p + M, gpu_device)
    assert err(out, want) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("p", [16, 64])
@pytest.mark.parametrize("M", [1, 16, 100])
def test_op_skewed_rows_and_untouched_rows(dtype, p, M, gpu_device):
    out, want, out0, act, prob = _op_case(dtype, p, M, True, 3 * p + M, gpu_device)
    assert err(out, want) <= TOL[dtype]
    got = out.double().cpu().numpy()
    inactive = sorted(set(range(prob["NB"])) - set(act.tolist()))
    for by in inactive:
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_op_with_every_block_its_own_chunk(dtype, gpu_device, monkeypatch):
    """Maximal row splitting: every block is a chunk, every row goes through the
    partial/counter combine. Two calls: the counters must be back at zero."""
    monkeypatch.setattr(_runtime, "_CHUNK_BYTES", 1)
    p, M = 32, 16
    prob = make_problem(6 * p, 20 * p, 4, p, 0.6, dtype, seed=99, skew=True)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=5)
    want = orc.bsr_addmm_inplace(np.zeros((M, prob["n"])), x, crow32, col32, vt, act)
    dev = gpu_device
    args = (to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev), torch.from_numpy(col32).to(dev),
            to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    outs = []
    for _ in range(2):
        out = torch.zeros(M, prob["n"], dtype=dtype, device=dev)
        _op(out, *args)
        outs.append(out)
    torch.cuda.synchronize()
    assert err(outs[0], want) <= TOL[dtype]
    assert torch.equal(outs[0], outs[1])


# ------------------------------------------------------- fused module --


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("M", [1, 16, 40])
def test_module_with_every_unit_its_own_chunk(dtype, M, gpu_device, monkeypatch):
    """Maximal splitting of the fused linear: every block and every low-rank unit
    is its own chunk, so each row is combined from many partials and every
    low-rank chunk waits for the latent."""
    monkeypatch.setattr(_runtime, "_CHUNK_BYTES", 1)
    prob = make_problem(256, 2048, 96, 32, 0.3, dtype, seed=M, skew=True)
    mod = _module(prob, gpu_device)
    x = make_x(prob, M)
    ys = [mod(to_dev(x, dtype, gpu_device)) for _ in range(2)]
    torch.cuda.synchronize()
    assert err(ys[0], oracle_y(prob, x)) <= TOL[dtype]
    assert torch.equal(ys[0], ys[1])
    assert latent_wait_status(gpu_device) == 0


def _module(prob, dev, bias=True):
    dt = prob["dtype"]
    S = sparse_bsr_tensor(prob, dev)
    return LRSLinear(
        to_dev(prob["A"], dt, dev), to_dev(prob["B"], dt, dev), S,
        in_features=prob["m"], out_features=prob["n"],
        bias=to_dev(prob["bias"], dt, dev) if (bias and prob["bias"] is not None) else None,
        block_p=prob["p"], block_q=prob["p"],
    )


def test_single_slr_linear_fp32_config(gpu_device):
    """fp32 512×512, rank 128, 32×32 blocks at 50%, x[256,512] ~ N(0,1), bias zeros."""
    prob = make_problem(512, 512, 128, 32, 0.5, torch.float32, seed=0)
    prob["bias"] = np.zeros(512)
    mod = _module(prob, gpu_device)
    x = np.random.default_rng(1).standard_normal((256, 512)).astype(np.float32).astype(np.float64)
    y = mod(to_dev(x, torch.float32, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (256, 512)
    assert err(y, oracle_y(prob, x)) <= 1e-5


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [(256, 192, 64, 32), (192, 256, 100, 16), (128, 128, 4, 64)])
@pytest.mark.parametrize("M", [1, 4, 16, 33, 64, 130])
def test_module_matches_oracle(dtype, shape, M, gpu_device):
    n, m, r, p = shape
    prob = make_problem(n, m, r, p, 0.5, dtype, seed=n + m + r + M)
    mod = _module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (M, n) and y.dtype == dtype
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("M", [1, 16, 70])
def test_module_ragged_features_and_no_bias(dtype, M, gpu_device):
    """out/in features that are not block multiples (zero-padded S), no bias."""
    prob = make_problem(100, 200, 24, 32, 0.5, dtype, seed=M, bias=False, pad=True)
    mod = _module(prob, gpu_device, bias=False)
    x = make_x(prob, M)
    xt = to_dev(x, dtype, gpu_device)
    y = mod(xt)
    torch.cuda.synchronize()
    assert y.shape == (M, 100)
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]
    # leading dims are kept (ls_linear.py:125-137)
    y3 = mod(xt.reshape(1, M, 200))
    assert y3.shape == (1, M, 100) and torch.equal(y3.reshape(M, 100), y)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_low_rank_only_module(dtype, gpu_device):
    rng = np.random.default_rng(3)
    n, m, r = 96, 80, 16
    A = orc.bf16_round(rng.standard_normal((n, r)) * 0.1).astype(np.float64)
    B = orc.bf16_round(rng.standard_normal((r, m)) * 0.1).astype(np.float64)
    b = orc.bf16_round(rng.standard_normal(n)).astype(np.float64)
    dev = gpu_device
    mod = LRSLinear(to_dev(A, dtype, dev), to_dev(B, dtype, dev), torch.zeros(n, m, device=dev),
                    in_features=m, out_features=n, bias=to_dev(b, dtype, dev))
    assert mod.kind == "lr_only"
    x = orc.bf16_round(rng.standard_normal((9, m))).astype(np.float64)
    y = mod(to_dev(x, dtype, dev))
    torch.cuda.synchronize()
    assert err(y, orc.slr_linear(x, A, B, np.zeros((n, m)), b)) <= TOL[dtype]


def test_module_is_deterministic_and_reuses_workspace(gpu_device):
    prob = make_problem(4096, 1024, 256, 64, 0.5, torch.bfloat16, seed=4, skew=True)
    mod = _module(prob, gpu_device)
    x = to_dev(make_x(prob, 16), torch.bfloat16, gpu_device)
    y1 = mod(x)
    y2 = mod(x)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("M", [1, 16])
def test_llama7b_ffn_shape_decode(M, gpu_device):
    """Full-size 11008×4096 bf16, rank 256, 64×64 blocks at 50%: split rows,
    latent split over in_features."""
    prob = make_problem(11008, 4096, 256, 64, 0.5, torch.bfloat16, seed=7)
    mod = _module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("density,skew", [(0.1, True), (0.9, False)], ids=["zipf10", "uniform90"])
def test_zipf_16x16_rows_split_for_decode(M, density, skew, gpu_device):
    """4096×11008 bf16, rank 128, rows of 16×16 blocks: Zipf(1.2) at 10% mean
    density (the full rows, 688 blocks, 352 KB) or uniform at 90% (every row
    about 620 blocks). The decode balancing splits rows across workgroups, and
    the result matches the oracle."""
    prob = make_problem(4096, 11008, 128, 16, density, torch.bfloat16, seed=11, skew=skew)
    mod = _module(prob, gpu_device)
    st = mod._kernel()
    assert st.plan(M).n_chunks > st.NB  # some rows were split
    x = make_x(prob, M)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


def test_repeated_calls_and_graph_replays_are_bit_identical(gpu_device):
    """The handshake words are monotonic and the counters return to zero, so
    call k + 1 must see exactly what call k saw: 100 eager calls and 100 graph
    replays of a q/k/v-like group and of a split-row 1B down projection all
    equal the first output bit for bit, and no wait gave up."""
    dtype = torch.bfloat16
    probs = _group_probs(dtype, [(256, 64, 0.5), (128, 96, 0.3), (192, 32, 0.7)], 320, 32, 77)
    grp = ssalaad_amd.LRSLinearGroup(*[_module(pr, gpu_device) for pr in probs])
    down = _module(make_problem(2048, 5461, 256, 32, 0.5, dtype, seed=5, pad=True), gpu_device)
    xg = to_dev(make_x(probs[0], 16), dtype, gpu_device)
    xd = to_dev(np.random.default_rng(3).standard_normal((16, 5461)), dtype, gpu_device)

    def step():
        return list(grp(xg)) + [down(xd)]

    first = [t.clone() for t in step()]
    for _ in range(100):
        outs = step()
        assert all(torch.equal(a, b) for a, b in zip(outs, first))
    s = torch.cuda.Stream(gpu_device)
    s.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = step()
    for _ in range(100):
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()  # eager work between replays
        assert all(torch.equal(a, b) for a, b in zip(outs, first))
    assert latent_wait_status(gpu_device) == 0


@pytest.mark.parametrize("p,q", [(64, 64), (32, 32), (128, 64)])
def test_prepared_op_is_captured_in_a_graph(p, q, gpu_device):
    """prepare_bsr_addmm builds the op's per-structure objects ahead of time;
    calls with that structure at a decode and a prefill size (and a block shape
    the kernels cut into sub-blocks) are then captured in one HIP graph without
    a host copy (the op raises if it would make one), and every replay, with
    eager work between, equals the eager op on the same tensors bit for bit.
    Calls on copies of the structure size the stream's scratch pools first, so
    the captured calls see only what prepare_bsr_addmm built."""
    dtype, dev = torch.bfloat16, gpu_device
    prob = make_problem(6 * p, 8 * q, 4, p, 0.5, dtype, seed=p + q, q=q)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    crow, col, act_t = (torch.from_numpy(a).to(dev) for a in (crow32, col32, act))
    vals = to_dev(vt, dtype, dev)
    ssalaad_amd.prepare_bsr_addmm(crow, col, vals, act_t, prob["m"])
    rng = np.random.default_rng(p * q)
    xs = [to_dev(make_x(prob, M, seed=M), dtype, dev) for M in (16, 256)]
    base = [to_dev(rng.standard_normal((M, prob["n"])), dtype, dev) for M in (16, 256)]
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):  # the stream's pools, through copies of the structure
        c2, k2, v2, a2 = crow.clone(), col.clone(), vals.clone(), act_t.clone()
        for b0, x in zip(base, xs):
            _op(b0.clone(), x, c2, k2, v2, a2)
    torch.cuda.synchronize()
    outs = [b.clone() for b in base]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for o, x in zip(outs, xs):
            _op(o, x, crow, col, vals, act_t)
    want = [b.clone() for b in base]
    with torch.cuda.stream(s):
        for o, x in zip(want, xs):
            _op(o, x, crow, col, vals, act_t)
    torch.cuda.synchronize()
    for w, x, M in zip(want, xs, (16, 256)):
        ref = orc.bsr_addmm_inplace(base[0 if M == 16 else 1].double().cpu().numpy(),
                                    x.double().cpu().numpy(), crow32, col32, vt, act)
        assert err(w, ref) <= TOL[dtype]
    for _ in range(3):
        for o, b in zip(outs, base):
            o.copy_(b)
        torch.cuda.synchronize()  # eager work between replays
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, w) for o, w in zip(outs, want))


def test_llama1b_down_proj_ragged_decode(gpu_device):
    """2048×5461 bf16 (in_features not a block multiple), 32×32 blocks, rank 256."""
    prob = make_problem(2048, 5461, 256, 32, 0.5, torch.bfloat16, seed=8, pad=True)
    mod = _module(prob, gpu_device)
    x = make_x(prob, 4)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


# ------------------------------------------------------ prefill path --
# Calls with ≥ 128 token rows and 16-bit activations take the LDS-tiled
# latent GEMM + row GEMM kernels.


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("M", [128, 300, 600, 1100])
def test_prefill_module_matches_oracle(dtype, p, M, gpu_device):
    prob = make_problem(4 * 64, 6 * 64, 128, p, 0.5, dtype, seed=p + M, skew=(p == 32))
    mod = _module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dtype, gpu_device))
    y2 = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (M, prob["n"])
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]
    assert torch.equal(y, y2)


@pytest.mark.parametrize("M", [128, 257, 600])
def test_prefill_ragged_features_no_bias(M, gpu_device):
    prob = make_problem(100, 200, 24, 32, 0.5, torch.bfloat16, seed=M, bias=False, pad=True)
    mod = _module(prob, gpu_device, bias=False)
    x = make_x(prob, M)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (M, 100)
    assert err(y, oracle_y(prob, x)) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 64])
@pytest.mark.parametrize("M", [128, 600])
def test_prefill_op_matches_oracle_and_keeps_inactive_rows(dtype, p, M, gpu_device):
    out, want, out0, act, prob = _op_case(dtype, p, M, True, 7 * p + M, gpu_device)
    assert err(out, want) <= TOL[dtype]
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


def test_prefill_group(gpu_device):
    probs = _group_probs(torch.bfloat16, [(256, 64, 0.5), (128, 96, 0.3), (192, 128, 0.7)], 320, 32, 9)
    grp = ssalaad_amd.LRSLinearGroup(*[_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], 700)  # above 512 rows: 32×32 blocks take the prefill kernels
    ys = grp(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= 1e-2


def test_prefill_llama7b_ffn_2048_tokens(gpu_device):
    """Full-size 11008×4096 bf16 at 2048 tokens; the oracle checks a spread of rows."""
    prob = make_problem(11008, 4096, 256, 64, 0.5, torch.bfloat16, seed=11)
    mod = _module(prob, gpu_device)
    x = make_x(prob, 2048)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    rows = np.r_[0:40, 1000:1030, 2000:2048]
    assert err(y[rows], oracle_y(prob, x[rows])) <= 1e-2


# ----------------------------------------------------- grouped launch --


def _group_probs(dtype, specs, m, p, seed):
    return [make_problem(n, m, r, p, d, dtype, seed=seed + i, skew=(i == 1))
            for i, (n, r, d) in enumerate(specs)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("M", [1, 5, 16, 40, 100])
def test_group_matches_oracle_per_member(dtype, M, gpu_device):
    """q/k/v-like members of different widths and ranks in one launch: each
    output equals its own oracle, and repeated calls are bit-identical."""
    probs = _group_probs(dtype, [(256, 64, 0.5), (128, 96, 0.3), (192, 32, 0.7)], 320, 32, 40 + M)
    mods = [_module(pr, gpu_device) for pr in probs]
    grp = ssalaad_amd.LRSLinearGroup(*mods)
    x = make_x(probs[0], M)
    xt = to_dev(x, dtype, gpu_device)
    ys = grp(xt)
    ys2 = grp(xt)
    torch.cuda.synchronize()
    assert len(ys) == 3
    for y, y2, pr in zip(ys, ys2, probs):
        assert y.shape == (M, pr["n"])
        assert err(y, oracle_y(pr, x)) <= TOL[dtype]
        assert torch.equal(y, y2)
    # members still work on their own, interleaved with the group
    y0 = mods[0](xt)
    torch.cuda.synchronize()
    assert err(y0, oracle_y(probs[0], x)) <= TOL[dtype]
    assert latent_wait_status(gpu_device) == 0


def test_group_with_low_rank_only_and_ragged_members(gpu_device):
    dev, dtype = gpu_device, torch.bfloat16
    prob = make_problem(100, 200, 24, 32, 0.5, dtype, seed=3, bias=False, pad=True)
    rng = np.random.default_rng(4)
    A = orc.bf16_round(rng.standard_normal((72, 16)) * 0.1).astype(np.float64)
    B = orc.bf16_round(rng.standard_normal((16, 200)) * 0.1).astype(np.float64)
    lr = LRSLinear(to_dev(A, dtype, dev), to_dev(B, dtype, dev), torch.zeros(72, 200, device=dev),
                   in_features=200, out_features=72)
    sl = _module(prob, dev, bias=False)
    x = make_x(prob, 7)
    with pytest.raises(ValueError, match="block shape"):
        ssalaad_amd.LRSLinearGroup(sl, lr)  # 32×32 blocks vs the low-rank-only tile
    grp = ssalaad_amd.LRSLinearGroup(sl, _module(prob, dev, bias=False))
    y1, y2 = grp(to_dev(x, dtype, dev).reshape(1, 7, 200))
    torch.cuda.synchronize()
    assert y1.shape == (1, 7, 100) and torch.equal(y1, y2)
    assert err(y1.reshape(7, 100), oracle_y(prob, x)) <= 1e-2
    y_lr = lr(to_dev(x, dtype, dev))
    assert err(y_lr, orc.slr_linear(x, A, B, np.zeros((72, 200)))) <= 1e-2


def test_group_rejects_mismatched_members(gpu_device):
    a = _module(make_problem(64, 96, 8, 32, 0.5, torch.bfloat16, seed=1), gpu_device)
    b = _module(make_problem(64, 128, 8, 32, 0.5, torch.bfloat16, seed=2), gpu_device)
    with pytest.raises(ValueError, match="in_features"):
        ssalaad_amd.LRSLinearGroup(a, b)
    with pytest.raises(ValueError, match="1 to 4"):
        ssalaad_amd.LRSLinearGroup(a, a, a, a, a)


@pytest.mark.parametrize("M", [1, 16])
def test_group_llama7b_attention_projections(M, gpu_device):
    """Full-size q, k, v (4096×4096 bf16, rank 256, 64×64 blocks at 50%) in one launch."""
    probs = _group_probs(torch.bfloat16, [(4096, 256, 0.5)] * 3, 4096, 64, 70 + M)
    grp = ssalaad_amd.LRSLinearGroup(*[_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], M)
    ys = grp(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= 1e-2


# --------------------------------------------- block projection (_project_S) --


def _separated(n, m, p, q, seed):
    """Random blocks whose Frobenius norms differ by ≥ 0.1% (no near ties)."""
    rng = np.random.default_rng(seed)
    rb, cb = n // p, m // q
    M = rng.standard_normal((n, m)).astype(np.float32)
    blk = M.reshape(rb, p, cb, q)
    norms = np.sqrt((blk.astype(np.float64) ** 2).sum(axis=(1, 3)))
    target = 1.0 + 1e-3 * rng.permutation(rb * cb).reshape(rb, cb)
    blk *= (target / norms)[:, None, :, None].astype(np.float32)
    return blk.reshape(n, m)


@pytest.fixture(params=[0, 2], ids=["select_auto", "select_many_groups"])
def select_path(request):
    """The block projection's select: the library's choice (one workgroup at
    these sizes) or forced onto the many-workgroup launches."""
    lib = _lib.load()
    _lib.check(lib.ssl_debug_set(_lib.DEBUG_TOPK_GROUPS, request.param), "ssl_debug_set")
    yield request.param
    _lib.check(lib.ssl_debug_set(_lib.DEBUG_TOPK_GROUPS, 0), "ssl_debug_set")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("shape", [(64, 96, 16, 16), (128, 128, 32, 32), (256, 512, 64, 64),
                                   (48, 40, 8, 4), (12, 20, 1, 1)])
def test_project_S_matches_oracle(dtype, shape, select_path, gpu_device):
    """Keep mask and kept values exact (the values are the input as fp32)."""
    n, m, p, q = shape
    M = _separated(n, m, p, q, seed=n * 7 + m)
    Md = torch.from_numpy(M).to(dtype)
    Mq = Md.float().numpy()                      # the input as the kernel sees it
    total = (n // p) * (m // q)
    blk = Mq.astype(np.float64).reshape(n // p, p, m // q, q)
    want_norms = (blk * blk).sum(axis=(1, 3))
    for n_keep in (-3, 0, 1, total // 2, total - 1, total, total + 5):
        out, keep, norms = ssalaad_amd.block_topk(Md.to(gpu_device), n_keep, p, q)
        torch.cuda.synchronize()
        want, want_keep = orc.project_blocks(Mq, n_keep, p, q)
        assert np.array_equal(keep.cpu().numpy(), want_keep), n_keep
        assert np.array_equal(out.cpu().numpy(), want), n_keep
        # fp32 sums of p·q squares against float64 ones
        np.testing.assert_allclose(norms.cpu().numpy(), want_norms, rtol=2e-6 * p * q ** 0.5)


def test_project_S_ties_nan_and_inf(select_path, gpu_device):
    M = np.ones((8, 12), np.float32)             # twelve equal 2×4 blocks (4 × 3)
    out = ssalaad_amd.project_S(torch.from_numpy(M).to(gpu_device), 5, 2, 4)
    keep = (out.cpu().numpy().reshape(4, 2, 3, 4) != 0).any(axis=(1, 3)).reshape(-1)
    assert np.flatnonzero(keep).tolist() == [0, 1, 2, 3, 4]   # lowest block index first
    M = _separated(16, 16, 4, 4, seed=11)
    M[5, 6] = np.nan
    M[13, 1] = np.inf
    for n_keep in (1, 2, 7):
        out, keep, _ = ssalaad_amd.block_topk(torch.from_numpy(M).to(gpu_device), n_keep, 4, 4)
        want, want_keep = orc.project_blocks(M, n_keep, 4, 4)
        assert np.array_equal(keep.cpu().numpy(), want_keep)
        got = out.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(np.nan_to_num(got, nan=7.0), np.nan_to_num(want, nan=7.0))


@pytest.mark.parametrize("n_keep_frac", [0.0, 0.3, 0.5, 0.9, 1.0])
@pytest.mark.parametrize("shape", [(1024, 1024, 2, 2), (2048, 1536, 4, 4), (300, 700, 1, 1)])
def test_project_S_ties_across_workgroups(shape, n_keep_frac, select_path, gpu_device):
    """Small-integer blocks: every norm is an exact integer in both fp32 and the
    oracle's float64, so thousands of blocks tie at the threshold, spread over
    the ranges of many select workgroups (up to 262144 blocks here). The kept
    ones are the lowest block indices among the tied, as in the oracle."""
    n, m, p, q = shape
    rng = np.random.default_rng(n + m + int(100 * n_keep_frac))
    M = rng.integers(-2, 3, size=(n, m)).astype(np.float32)
    M[rng.random((n, m)) < 0.3] = 0.0
    total = (n // p) * (m // q)
    n_keep = int(total * n_keep_frac)
    out, keep, norms = ssalaad_amd.block_topk(torch.from_numpy(M).to(gpu_device), n_keep, p, q)
    torch.cuda.synchronize()
    want, want_keep = orc.project_blocks(M, n_keep, p, q)
    assert np.array_equal(keep.cpu().numpy(), want_keep)
    assert np.array_equal(out.cpu().numpy(), want)
    blk = M.astype(np.float64).reshape(n // p, p, m // q, q)
    assert np.array_equal(norms.cpu().numpy(), (blk * blk).sum(axis=(1, 3)).astype(np.float32))


def test_project_S_many_groups_repeat_and_shrink(gpu_device):
    """Calls in a row on one stream reuse nothing of the last call's select:
    a large call, then a smaller one with a different threshold, then the large
    one again."""
    cases = [(2048, 2048, 2, 2, 0.4), (512, 768, 2, 2, 0.7), (2048, 2048, 2, 2, 0.4)]
    rng = np.random.default_rng(5)
    for n, m, p, q, frac in cases:
        M = rng.integers(-3, 4, size=(n, m)).astype(np.float32)
        total = (n // p) * (m // q)
        out, keep, _ = ssalaad_amd.block_topk(torch.from_numpy(M).to(gpu_device), int(total * frac), p, q)
        torch.cuda.synchronize()
        want, want_keep = orc.project_blocks(M, int(total * frac), p, q)
        assert np.array_equal(keep.cpu().numpy(), want_keep), (n, m)
        assert np.array_equal(out.cpu().numpy(), want), (n, m)


def test_project_S_rejects_bad_arguments(gpu_device):
    M = torch.ones(8, 8, device=gpu_device)
    with pytest.raises(RuntimeError, match="invalid for input"):
        ssalaad_amd.project_S(M, 1, 3, 4)
    with pytest.raises(ValueError, match="GPU"):
        ssalaad_amd.project_S(M.cpu(), 1, 4, 4)


def test_project_then_encode_gives_the_reference_structure(gpu_device):
    """The compression loop's path: project (fp32) → cast to bf16 → dense_to_bsr
    (egar.py:464, :552-553; artifact.py:20-37), structure and values bit-exact."""
    n, m, p = 512, 768, 32
    M = _separated(n, m, p, p, seed=21)
    M[32:64, 64:96] = 1e-41                      # fp32 subnormals: zero once cast to bf16
    total = (n // p) * (m // p)
    for n_keep in (total // 2, total):
        out = ssalaad_amd.project_S(torch.from_numpy(M).to(gpu_device), n_keep, p, p)
        S = ssalaad_amd.dense_to_bsr(out.to(torch.bfloat16), p, p)
        torch.cuda.synchronize()
        want_proj, _ = orc.project_blocks(M, n_keep, p, p)
        crow, col, vals = orc.dense_to_bsr(orc.bf16_round(want_proj), p, p)
        assert np.array_equal(S.crow_indices().cpu().numpy(), crow)
        assert np.array_equal(S.col_indices().cpu().numpy(), col)
        assert np.array_equal(S.values().float().cpu().numpy(), vals)
    assert crow[-1] == total - 1                 # the kept subnormal block is dropped


@pytest.mark.parametrize("p", [64, 16, 8])
def test_project_S_llama7b_ffn_shape(p, gpu_device):
    """11008×4096 fp32, p×p blocks (11008 to 704512 of them), half kept."""
    n, m = 11008, 4096
    M = _separated(n, m, p, p, seed=23)
    total = (n // p) * (m // p)
    out, keep, _ = ssalaad_amd.block_topk(torch.from_numpy(M).to(gpu_device), total // 2, p, p)
    torch.cuda.synchronize()
    want, want_keep = orc.project_blocks(M, total // 2, p, p)
    assert np.array_equal(keep.cpu().numpy(), want_keep)
    assert torch.equal(out.cpu(), torch.from_numpy(want))


# ------------------------------------------------------------ encoder --


def _special_matrix(n, m, p, q, dtype, seed):
    rng = np.random.default_rng(seed)
    S = np.zeros((n, m), dtype=np.float32)
    NB, NBK = n // p, m // q
    for s in rng.permutation(NB * NBK)[: (NB * NBK) // 2]:
        br, bc = divmod(int(s), NBK)
        S[br * p:(br + 1) * p, bc * q:(bc + 1) * q] = rng.standard_normal((p, q))
    # special blocks (if the grid has room): NaN, -0 only, inf, a lone subnormal
    specials = [(0, 0, np.nan), (0, 1, -0.0), (1, 0, np.inf), (1, 1, "sub")]
    for br, bc, v in specials:
        if br < NB and bc < NBK:
            blk = S[br * p:(br + 1) * p, bc * q:(bc + 1) * q]
            if v == "sub":
                blk[:] = 0
                blk[p - 1, q - 1] = {torch.float32: 1e-45, torch.bfloat16: 1e-40,
                                     torch.float16: 6e-8}[dtype]
            elif isinstance(v, float) and v == 0.0:
                blk[:] = -0.0
            else:
                blk[p // 2, q // 2] = v
    return torch.from_numpy(S).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("pq", [(16, 16), (32, 32), (64, 64), (16, 32), (32, 16), (64, 32), (8, 128)])
def test_encoder_structure_is_bit_exact(dtype, pq, gpu_device):
    p, q = pq
    S = _special_matrix(6 * p, 9 * q, p, q, dtype, seed=p + q)
    crow, col, vals = orc.dense_to_bsr(S.float().numpy(), p, q)
    crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
    bits = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[dtype]
    S_bits = S.view(bits).numpy()
    dev = gpu_device
    k_crow, k_col, k_vt, k_act = ssalaad_amd.encode_for_kernels(S.to(dev), p, q)
    bsr = ssalaad_amd.dense_to_bsr(S.to(dev), p, q)
    torch.cuda.synchronize()
    assert np.array_equal(k_crow.cpu().numpy(), crow32)
    assert np.array_equal(k_col.cpu().numpy(), col32)
    assert np.array_equal(k_act.cpu().numpy(), act)
    assert np.array_equal(bsr.crow_indices().cpu().numpy(), crow)
    assert np.array_equal(bsr.col_indices().cpu().numpy(), col)
    assert bsr.crow_indices().dtype == torch.int64
    # values copied bit for bit: gather the kept blocks' bits from S directly
    rows = np.repeat(np.arange(len(crow) - 1), np.diff(crow))
    want_bits = np.stack([S_bits[r * p:(r + 1) * p, c * q:(c + 1) * q] for r, c in zip(rows, col)]) \
        if len(col) else np.zeros((0, p, q), S_bits.dtype)
    assert np.array_equal(bsr.values().cpu().view(bits).numpy(), want_bits)
    assert np.array_equal(k_vt.cpu().view(bits).numpy(), want_bits.transpose(0, 2, 1))


def test_encoder_feeds_the_module(gpu_device):
    """Dense S handed to the factory goes through the device encoder."""
    prob = make_problem(128, 192, 16, 32, 0.4, torch.bfloat16, seed=2)
    dev = gpu_device
    from slr_cases import s_dense

    S = to_dev(s_dense(prob), torch.bfloat16, dev)
    mod = LRSLinear(to_dev(prob["A"], torch.bfloat16, dev), to_dev(prob["B"], torch.bfloat16, dev),
                    S, in_features=192, out_features=128, bias=to_dev(prob["bias"], torch.bfloat16, dev),
                    block_p=32, block_q=32)
    assert mod.S_nnz == len(prob["col"])
    x = make_x(prob, 5)
    y = mod(to_dev(x, torch.bfloat16, dev))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


def test_no_workgroup_gave_up_waiting_for_the_latent(gpu_device):
    """Runs after the module tests: every fused call found its latent ready."""
    prob = make_problem(4096, 1024, 256, 64, 0.5, torch.bfloat16, seed=6)
    mod = _module(prob, gpu_device)
    for M in (1, 16, 64, 200):
        mod(to_dev(make_x(prob, M), torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert latent_wait_status(gpu_device) == 0


# ------------------------------------------------------------ 2:4 (N:M) S --


_nm24 = nm24_matrix
_nm_module = make_nm_module


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", [(256, 192, 64), (100, 200, 24), (64, 4096, 256)])
@pytest.mark.parametrize("M", [1, 16, 33, 130])
def test_nm24_module_matches_oracle(dtype, shape, M, gpu_device):
    n, m, r = shape
    mod, (A, B, S, b) = _nm_module(n, m, r, dtype, gpu_device, seed=n + m + M)
    assert mod.kind == "nm" and "S_nm" not in dict(mod.named_buffers())
    x = np.random.default_rng(M).standard_normal((M, m))
    x = torch.from_numpy(x).to(dtype).double().numpy()
    xt = to_dev(x, dtype, gpu_device)
    y1, y2 = mod(xt), mod(xt)
    torch.cuda.synchronize()
    want = orc.slr_linear(x, A, B, S, b)
    assert y1.shape == (M, n)
    assert err(y1, want) <= TOL[dtype]
    assert torch.equal(y1, y2)
    assert latent_wait_status(gpu_device) == 0


def test_nm24_pack_round_trip_and_rules(gpu_device):
    from ssalaad_amd.artifact import nm24_pack

    S = _nm24(70, 100, 5, torch.bfloat16)
    S[32:64, 32:64] = 0                                        # an empty block is not stored
    pk = nm24_pack(to_dev(S, torch.bfloat16, gpu_device))
    crow, col = pk["crow"].cpu().numpy(), pk["col"].cpu().numpy()
    blocks = pk["blocks"].cpu()
    D = np.zeros((pk["NB"] * 32, pk["NBK"] * 32))
    for by in range(pk["NB"]):
        for k in range(crow[by], crow[by + 1]):
            vals = blocks[k, :1024].view(torch.bfloat16).float().numpy().reshape(16, 16, 2)
            ix = blocks[k, 1024:].numpy().reshape(16, 8, 2)
            for c in range(16):
                for s_ in range(2):
                    for grp in range(8):
                        i0, i1 = ix[c, grp, s_] & 3, ix[c, grp, s_] >> 2
                        assert i0 < i1
                        D[by * 32 + 2 * c + s_, col[k] * 32 + 4 * grp + i0] = vals[c, 2 * grp, s_]
                        D[by * 32 + 2 * c + s_, col[k] * 32 + 4 * grp + i1] = vals[c, 2 * grp + 1, s_]
    assert np.array_equal(D[:70, :100], S)
    assert crow[-1] == pk["NB"] * pk["NBK"] - 1
    bad = S.copy()
    bad[3, 0:3] = 1.0                                          # three non-zeros in one group
    with pytest.raises(ValueError, match="not 2:4"):
        nm24_pack(to_dev(bad, torch.bfloat16, gpu_device))
    A, B = torch.zeros(64, 8, device=gpu_device), torch.zeros(8, 64, device=gpu_device)
    with pytest.raises(ValueError, match="fp16 or bf16"):
        LRSLinear(A, B, torch.ones(64, 64, device=gpu_device), in_features=64, out_features=64,
                  nm_n=2, nm_m=4)


def test_nm24_group_and_mixing_rules(gpu_device):
    dtype = torch.bfloat16
    mods = [_nm_module(n, 160, r, dtype, gpu_device, seed=7 + n)[0] for n, r in ((96, 32), (64, 16))]
    grp = ssalaad_amd.LRSLinearGroup(*mods)
    x = to_dev(np.random.default_rng(9).standard_normal((5, 160)), dtype, gpu_device)
    ys = grp(x)
    torch.cuda.synchronize()
    for y, mod in zip(ys, mods):
        assert torch.equal(y, mod(x))
    blk = _module(make_problem(96, 160, 8, 32, 0.5, dtype, seed=3), gpu_device)
    with pytest.raises(ValueError, match="sparse storage"):
        ssalaad_amd.LRSLinearGroup(mods[0], blk)


@pytest.mark.parametrize("M", [1, 16])
def test_nm24_llama7b_gate_up_group_decode(M, gpu_device):
    """The 7B gate and up projections with 2:4 S in one grouped launch: the row
    split budgets the slots the whole launch leaves free (none here: 688
    block-rows for 512 slots), and both outputs match the oracle."""
    dtype = torch.bfloat16
    pairs = [_nm_module(11008, 4096, 256, dtype, gpu_device, seed=41 + i, bias=False) for i in range(2)]
    grp = ssalaad_amd.LRSLinearGroup(*[m for m, _ in pairs])
    x = round_to(np.random.default_rng(M).standard_normal((M, 4096)), dtype)
    ys = grp(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    states = [m._kernel() for m, _ in pairs]
    share = (sum(st.NB for st in states), sum(st.r_pad // 16 for st in states))
    for st in states:
        pl = st.plan(M, share)
        assert pl.n_chunks == st.NB  # no row split inside the group
    assert states[0].plan(M).n_chunks > states[0].NB  # alone, some rows split
    for y, (_, (A, B, S, b)) in zip(ys, pairs):
        assert err(y, orc.slr_linear(x, A, B, S, b)) <= TOL[dtype]
    assert latent_wait_status(gpu_device) == 0


def test_nm24_llama7b_ffn_shape_decode(gpu_device):
    """11008×4096 bf16, rank 256, 2:4 S: one fused launch per call, with some of
    the 344 equal rows split in two to fill the free workgroup slots."""
    mod, (A, B, S, b) = _nm_module(11008, 4096, 256, torch.bfloat16, gpu_device, seed=31, bias=False)
    st = mod._kernel()
    assert st.NB < st.plan(4).n_chunks < 2 * st.NB  # a partial split
    x = np.random.default_rng(2).standard_normal((4, 4096))
    x = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    y2 = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, orc.slr_linear(x, A, B, S, b)) <= 1e-2
    assert torch.equal(y, y2)
    assert latent_wait_status(gpu_device) == 0


# ------------------------------------------------- 2:4 at prefill sizes --
# From ssl_prefill_min_rows() token rows 2:4 calls run the prefill row kernel
# on v_smfmac_f32_16x16x64 (the weights' kept values and positions as the
# sparse A operand, x as B, tiles transposed to features × tokens); the
# latent and the low-rank steps are the dense MFMA steps of the same kernel.


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", [(256, 192, 64), (100, 200, 24), (320, 1024, 128)])
@pytest.mark.parametrize("tile_mode", [0, 1, 2, 3], ids=["auto", "narrow", "tall", "short"])
@pytest.mark.parametrize("M", [128, 600])
def test_nm24_prefill_matches_oracle(dtype, shape, tile_mode, M, gpu_device):
    n, m, r = shape
    lib = _lib.load()
    assert lib.ssl_nm24_takes_prefill(M, -(-n // 32), _lib.dtype_code(dtype)) == 1
    mod, (A, B, S, b) = _nm_module(n, m, r, dtype, gpu_device, seed=n + m + M + tile_mode)
    x = np.random.default_rng(M + 1).standard_normal((M, m))
    x = torch.from_numpy(x).to(dtype).double().numpy()
    xt = to_dev(x, dtype, gpu_device)
    _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, tile_mode), "ssl_debug_set")
    try:
        y1, y2 = mod(xt), mod(xt)
        torch.cuda.synchronize()
    finally:
        lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, 0)
    assert err(y1, orc.slr_linear(x, A, B, S, b)) <= TOL[dtype]
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("k", [2, 3])
def test_nm24_prefill_split_row_groups(k, gpu_device):
    """The 2:4 prefill kernel with its row groups' steps in k parts and the
    latent's in_features in chunks (test hook), narrow and short tiles."""
    lib = _lib.load()
    n, m, r, dtype = 320, 2048, 128, torch.bfloat16
    mod, (A, B, S, b) = _nm_module(n, m, r, dtype, gpu_device, seed=k)
    x = np.random.default_rng(k).standard_normal((300, m))
    x = torch.from_numpy(x).to(dtype).double().numpy()
    xt = to_dev(x, dtype, gpu_device)
    for tile in (1, 3):
        _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, tile), "ssl_debug_set")
        _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_SPLIT, k), "ssl_debug_set")
        try:
            y1, y2 = mod(xt), mod(xt)
            torch.cuda.synchronize()
        finally:
            lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, 0)
            lib.ssl_debug_set(_lib.DEBUG_PREFILL_SPLIT, 0)
        assert err(y1, orc.slr_linear(x, A, B, S, b)) <= TOL[dtype]
        assert torch.equal(y1, y2)


def test_nm24_prefill_grouped_launch(gpu_device):
    dtype = torch.bfloat16
    mods = [_nm_module(n, 320, r, dtype, gpu_device, seed=17 + n) for n, r in ((96, 32), (200, 64), (64, 16))]
    grp = ssalaad_amd.LRSLinearGroup(*[md for md, _ in mods])
    x = np.random.default_rng(19).standard_normal((300, 320))
    x = torch.from_numpy(x).to(dtype).double().numpy()
    ys = grp(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    for y, (_, (A, B, S, b)) in zip(ys, mods):
        assert err(y, orc.slr_linear(x, A, B, S, b)) <= 1e-2


def test_nm24_llama7b_ffn_shape_at_2048_tokens_every_row(gpu_device):
    """11008×4096 bf16, rank 256, 2:4 S, 2048 tokens: the structured-sparse row
    kernel, every output row against the oracle."""
    mod, (A, B, S, b) = _nm_module(11008, 4096, 256, torch.bfloat16, gpu_device, seed=41,
                                   bias=False)
    x = np.random.default_rng(5).standard_normal((2048, 4096))
    x = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, orc.slr_linear(x, A, B, S, b)) <= 1e-2
