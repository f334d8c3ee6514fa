"""The prefill row kernels (calls with many token rows, 16-bit activations),
every tile configuration checked against the oracle on every output row.

The row kernel has three tiles (token rows × output features, 64/p block-rows
per workgroup): "narrow" (128 × 64), "tall" (256 × 64) and "short" (64 × 64);
the library picks one per call. The test hook SSL_DEBUG_PREFILL_TILE
forces each tile on any shape, for the fused linear (PF_FUSED), the grouped
launch and the in-place op (PF_OP). The full-size cases at the end run every
tile at the benchmark shapes, checked on all rows.
The forward these compute is ssalaad/efficient/ls_linear.py:124-137 (the op:
ssalaad/tilelang_sparse/addmm_inplace.py:41-82).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slr_oracle as orc
from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, to_dev

import ssalaad_amd
from ssalaad_amd import _lib

pytestmark = pytest.mark.gpu

NARROW, TALL, SHORT = 1, 2, 3
MODES = [NARROW, TALL, SHORT]
MODE_IDS = ["narrow", "tall", "short"]
DT16 = [torch.bfloat16, torch.float16]


@pytest.fixture
def tile():
    """Force a prefill row tile for the test's calls; restores the default."""
    lib = _lib.load()

    def force(mode):
        _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, mode), "ssl_debug_set")

    yield force
    force(0)


def _group_of(M, rows, p):
    return int(_lib.load().ssl_prefill_group(M, rows, p, p))


@pytest.mark.parametrize("r", [40, 64, 130], ids=["r40", "r64", "r130"])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
def test_latent_tile_counters_return_to_zero(r, mode, tile, gpu_device):
    """The latent tile counters live in the call's zero-at-rest counters: the
    last waiter of each tile returns them to zero, with no clearing launch.
    One low-rank step (r_pad 64: fetches past the end repeat the step that
    waits) must count each wave once; three calls in a row, each exact, and
    the counters back at zero after each."""
    from ssalaad_amd import _runtime

    tile(mode)
    dtype = torch.bfloat16
    prob = make_problem(10 * 64, 7 * 64, r, 64, 0.5, dtype, seed=r + mode, bias=True)
    mod = make_module(prob, gpu_device)
    for M in (200, 333, 128):
        x_np = make_x(prob, M, seed=M)
        y = mod(to_dev(x_np, dtype, gpu_device))
        torch.cuda.synchronize()
        assert err(y, oracle_y(prob, x_np)) <= TOL[dtype], M
        assert all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
                   if idx == gpu_device.index), M


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("M", [600, 1030])
def test_forced_tiles_fused_linear(dtype, p, mode, M, tile, gpu_device):
    """Ragged block-row count, skewed rows,
    ragged token count: every row of every tile against the oracle."""
    tile(mode)
    prob = make_problem(13 * p + 64, 9 * 64, 128, p, 0.5, dtype, seed=p + M + mode, skew=True)
    rows = prob["NB"]
    assert _group_of(M, rows, p) == 64 // p
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
def test_forced_tiles_grouped_launch(dtype, p, mode, tile, gpu_device):
    tile(mode)
    specs = [(5 * p, 64, 0.5), (3 * p, 96, 0.3), (7 * p, 128, 0.7)]
    probs = [make_problem(n, 8 * p, r, p, d, dtype, seed=31 + i, skew=(i == 1))
             for i, (n, r, d) in enumerate(specs)]
    grp = ssalaad_amd.LRSLinearGroup(*[make_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], 700)
    ys = grp(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", DT16, ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
def test_forced_tiles_inplace_op(dtype, p, mode, tile, gpu_device):
    """PF_OP: out += x·Sᵀ on the active rows only; every other row keeps its bits."""
    tile(mode)
    M = 300
    prob = make_problem(13 * p, 10 * p, 4, p, 0.3, dtype, seed=5 * p + mode, skew=True)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=3)
    rng = np.random.default_rng(p)
    out0 = torch.from_numpy(rng.standard_normal((M, prob["n"]))).to(dtype).double().numpy()
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dtype, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    assert err(out, want) <= TOL[dtype]
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


@pytest.mark.parametrize("n,m,p,tiled", [(4096, 2048, 64, False), (6144, 2048, 64, True),
                                          (2048, 5461, 32, False), (4160, 1024, 32, True),
                                          (1024, 1024, 16, True)],
                         ids=["p64-64rows", "p64-96rows", "p32-64rows", "p32-130rows", "p16"])
def test_inplace_op_automatic_routing_at_128_rows(n, m, p, tiled, gpu_device):
    """The op's own stream-or-tile choice at one token tile pair (128 rows) on
    both sides of its grid boundary: out += x·Sᵀ on the active rows, every
    other row untouched. The side each case takes is asserted: the op plans
    its active rows that hold blocks, and on a 256-CU device one token tile
    streams when those rows' 64-feature groups number at most a quarter of
    the CUs (64 groups)."""
    if torch.cuda.get_device_properties(gpu_device).multi_processor_count != 256:
        pytest.skip("the sides checked are those of a 256-CU device")
    M, dtype = 128, torch.bfloat16
    prob = make_problem(n, m, 4, p, 0.5, dtype, seed=n + p, pad=True)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    planned = int(np.count_nonzero(np.diff(crow32)[act]))
    lib = _lib.load()
    assert bool(lib.ssl_bsr_addmm_takes_prefill(M, planned, p, p, _lib.SSL_BF16)) == tiled
    x = make_x(prob, M, seed=7)
    rng = np.random.default_rng(n)
    out0 = torch.from_numpy(rng.standard_normal((M, prob["NB"] * p))).to(dtype).double().numpy()
    xp = np.zeros((M, prob["NBK"] * p))
    xp[:, :m] = x
    want = orc.bsr_addmm_inplace(out0, xp, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dtype, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(xp, dtype, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    assert err(out, want) <= TOL[dtype]
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


# ------------------------------------------------------------ K parts --


@pytest.fixture
def split():
    """Force the K parts of fused prefill calls (1: none, 2-4: that many)."""
    lib = _lib.load()

    def force(k):
        _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_SPLIT, k), "ssl_debug_set")

    yield force
    force(0)


def _counters_at_rest(dev) -> bool:
    from ssalaad_amd import _runtime

    torch.cuda.synchronize()
    return all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("mode", [NARROW, SHORT], ids=["narrow", "short"])
@pytest.mark.parametrize("k", [2, 3, 4])
def test_split_row_groups_and_latent(dtype, p, mode, k, tile, split, gpu_device):
    """Every row group's sparse steps in k parts (the last also runs the
    low-rank steps) and the latent's in_features in chunks: the parts' fp32
    tiles summed in part order by the last to arrive. Skewed rows (groups with
    fewer sparse steps than parts), ragged token count, 5000 in_features (the
    latent in several chunks): every row against the oracle, twice, and the
    counters back at zero after each call."""
    if dtype == torch.float32 and p == 64:
        pytest.skip("fp32 prefill blocks are 16 or 32")
    tile(mode)
    split(k)
    prob = make_problem(11 * p + 64, 5000, 128, p, 0.5, dtype, seed=7 * p + k + mode, skew=True,
                        pad=True)
    mod = make_module(prob, gpu_device)
    for M in (333, 200):
        x = make_x(prob, M, seed=M)
        y = mod(to_dev(x, dtype, gpu_device))
        torch.cuda.synchronize()
        assert err(y, oracle_y(prob, x)) <= TOL[dtype], M
        assert _counters_at_rest(gpu_device), M


@pytest.mark.parametrize("k", [2, 4])
def test_split_grouped_launch(k, tile, split, gpu_device):
    """K parts in a grouped launch of three linears of different ranks and
    shapes (every member's row groups in k parts, each latent in its own
    chunks)."""
    tile(NARROW)
    split(k)
    dtype, p = torch.bfloat16, 32
    specs = [(5 * p, 64, 0.5), (3 * p, 192, 0.3), (7 * p, 128, 0.7)]
    probs = [make_problem(n, 40 * p, r, p, d, dtype, seed=41 + i, skew=(i == 1))
             for i, (n, r, d) in enumerate(specs)]
    grp = ssalaad_amd.LRSLinearGroup(*[make_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], 300)
    ys = grp(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= TOL[dtype]
    assert _counters_at_rest(gpu_device)


# -------------------------------------------- full size, library's choice --


@pytest.mark.parametrize("mode", [0] + MODES, ids=["auto"] + MODE_IDS)
def test_skewed_16x16_at_2048_tokens_every_row(mode, tile, gpu_device):
    """4096×11008 bf16, rank 128, 16×16 blocks with Zipf(1.2) rows at 50% mean
    density, 2048 tokens."""
    tile(mode)
    prob = make_problem(4096, 11008, 128, 16, 0.5, torch.bfloat16, seed=21, skew=True)
    assert _group_of(2048, prob["NB"], 16) == 4
    mod = make_module(prob, gpu_device)
    x = make_x(prob, 2048)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


@pytest.mark.parametrize("mode", [0] + MODES, ids=["auto"] + MODE_IDS)
def test_llama1b_gate_up_group_at_2048_tokens_every_row(mode, tile, gpu_device):
    """LLaMA-1B gate and up (5461×2048, 32×32 blocks at 50%, rank 256, FFN padded
    to 5472) in one grouped launch at 2048 tokens."""
    tile(mode)
    probs = [make_problem(5461, 2048, 256, 32, 0.5, torch.bfloat16, seed=40 + i, pad=True)
             for i in range(2)]
    assert _group_of(2048, 2 * probs[0]["NB"], 32) == 2
    grp = ssalaad_amd.LRSLinearGroup(*[make_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], 2048)
    ys = grp(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert y.shape == (2048, 5461)
        assert err(y, oracle_y(pr, x)) <= 1e-2


@pytest.mark.parametrize("mode", [0] + MODES, ids=["auto"] + MODE_IDS)
def test_llama7b_ffn_at_2048_tokens_every_row(mode, tile, gpu_device):
    """11008×4096 bf16, 64×64 blocks at 50%, rank 256, 2048 tokens, every row
    against the oracle."""
    tile(mode)
    prob = make_problem(11008, 4096, 256, 64, 0.5, torch.bfloat16, seed=11)
    assert _group_of(2048, prob["NB"], 64) == 1
    mod = make_module(prob, gpu_device)
    x = make_x(prob, 2048)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2


def test_llama7b_down_automatic_tile_and_parts_every_row(tile, split, gpu_device):
    """4096×11008 bf16 (64×64 blocks at 50%: 86 sparse steps a row group, a
    172-step latent), rank 256, on a 256-CU device. The library's own choice
    at each token count equals, bit for bit, the forced configuration it should
    take, and every row matches the oracle:
      512 rows: 256 row groups' worth of narrow tiles in 2 parts (512 parts;
                the latent is 1.5 times a group's steps), latent in chunks;
      640 rows: 320 groups' worth of narrow tiles whole (640 parts would stack
                three to a CU);
      768 rows: 384 groups' worth of narrow tiles whole (768 parts would
                stack three to a CU)."""
    if torch.cuda.get_device_properties(gpu_device).multi_processor_count != 256:
        pytest.skip("the choices checked are those of a 256-CU device")
    prob = make_problem(4096, 11008, 256, 64, 0.5, torch.bfloat16, seed=23)
    mod = make_module(prob, gpu_device)
    x = make_x(prob, 768, seed=3)
    want = oracle_y(prob, x)
    for M, forced_tile, forced_parts in ((512, NARROW, 2), (640, NARROW, 1), (768, NARROW, 1)):
        xt = to_dev(x[:M], torch.bfloat16, gpu_device)
        y_auto = mod(xt)
        tile(forced_tile)
        split(forced_parts)
        try:
            y_forced = mod(xt)
        finally:
            tile(0)
            split(0)
        torch.cuda.synchronize()
        assert torch.equal(y_auto, y_forced), M
        assert err(y_auto, want[:M]) <= 1e-2, M
        assert _counters_at_rest(gpu_device)


@pytest.mark.parametrize("n,m,p,M,tiled", [
    (2048, 2048, 32, 128, False),   # one token tile, 2048 output features: streams
    (2080, 2048, 32, 128, True),    # 65 block-rows: tiled
    (4096, 2048, 16, 128, True),    # 16×16 blocks, one token tile: tiled
    (4096, 2048, 16, 300, True),    # 16×16 blocks, ragged token tiles, K parts
    (4096, 3072, 64, 128, True),
], ids=["stream-2048x2048-p32", "tiled-2080-p32", "tiled-p16-128", "tiled-p16-300", "tiled-p64-128"])
def test_automatic_routing_at_its_boundaries_every_row(n, m, p, M, tiled, gpu_device):
    """The library's own stream-or-tile choice on both sides of its boundary
    (128 rows, 2048 output features), every row against the oracle."""
    lib = _lib.load()
    prob = make_problem(n, m, 128, p, 0.5, torch.bfloat16, seed=n + M)
    assert bool(lib.ssl_slr_takes_prefill(M, prob["NB"], p, p, _lib.SSL_BF16)) == tiled
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M, seed=M)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= 1e-2
    assert _counters_at_rest(gpu_device)


# ------------------------------------------------------------------- fp32 --
# fp32 calls run the same kernels with 32-column steps (128 bytes per tile
# row, v_mfma_f32_16x16x4f32); 16×16 and 32×32 blocks (64-wide blocks stream).
# The library sends them there when the grid fills the device; a forced tile
# sends any call of 128 rows or more.


@pytest.mark.parametrize("p", [16, 32])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
@pytest.mark.parametrize("M", [600, 1030])
def test_fp32_forced_tiles_fused_linear(p, mode, M, tile, gpu_device):
    tile(mode)
    dt = torch.float32
    prob = make_problem(13 * p + 64, 9 * 64 + 3 * p, 128, p, 0.5, dt, seed=p + M + mode, skew=True)
    assert _lib.load().ssl_slr_takes_prefill(M, prob["NB"], p, p, _lib.SSL_F32) == 1
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dt, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= TOL[dt]


@pytest.mark.parametrize("p", [16, 32])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
def test_fp32_ragged_features_and_grouped_launch(p, mode, tile, gpu_device):
    """n and m not multiples of the block (a ragged last block column is cut by
    in_features), three linears in one launch, 300 token rows."""
    tile(mode)
    dt = torch.float32
    specs = [(5 * p + 3, 96, 0.5), (3 * p, 64, 0.3), (7 * p - 5, 128, 0.7)]
    m = 8 * p - 7
    probs = [make_problem(n, m, r, p, d, dt, seed=71 + i, skew=(i == 1), pad=True)
             for i, (n, r, d) in enumerate(specs)]
    grp = ssalaad_amd.LRSLinearGroup(*[make_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], 300)
    ys = grp(to_dev(x, dt, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= TOL[dt]


@pytest.mark.parametrize("p", [16, 32])
@pytest.mark.parametrize("mode", MODES, ids=MODE_IDS)
def test_fp32_inplace_op(p, mode, tile, gpu_device):
    tile(mode)
    dt = torch.float32
    M = 300
    prob = make_problem(13 * p, 10 * p, 4, p, 0.3, dt, seed=7 * p + mode, skew=True)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=3)
    rng = np.random.default_rng(p)
    out0 = rng.standard_normal((M, prob["n"])).astype(np.float32).astype(np.float64)
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dt, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(x, dt, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, dt, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    assert err(out, want) <= TOL[dt]
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


def test_fp32_llama60m_gate_at_2048_tokens_every_row(gpu_device):
    """LLaMA-60M gate (1376×512, 32×32 blocks at 50%, rank 128), fp32, 2048
    tokens: the shape of config 2's projections."""
    dt = torch.float32
    prob = make_problem(1376, 512, 128, 32, 0.5, dt, seed=60)
    mod = make_module(prob, gpu_device)
    x = make_x(prob, 2048)
    y = mod(to_dev(x, dt, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= TOL[dt]


# ------------------------------------------------- skewed structures: parts --
# Zipf(1.2) rows: the prefill plan's longest groups run in parts of about the
# mean group's steps (ssl_prefill_parts_build), each part's fp32 tile summed in
# part order by the last to arrive. 64 groups at 1900-2048 tokens: the tall
# grid is one round of the device, so the parts run (narrow or short tiles).


@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("mode", [0, NARROW, SHORT], ids=["auto", "narrow", "short"])
@pytest.mark.parametrize("M", [2048, 1900])
def test_skewed_groups_run_in_parts(p, mode, M, tile, gpu_device):
    from ssalaad_amd import _runtime

    if mode:
        tile(mode)
    dtype = torch.bfloat16
    prob = make_problem(4096, 8192, 96, p, 0.1, dtype, seed=p + M, skew=True)
    mod = make_module(prob, gpu_device)
    st = mod._kernel()
    pp = st.prefill_plan(int(_lib.load().ssl_prefill_group(M, st.NB, p, p)))
    assert pp.parts is not None and pp.split_parts > 0
    x_np = make_x(prob, M, seed=M)
    print(f"[parts] p={p} tile={mode} M={M} parts={pp.n_parts} split={pp.split_parts}", flush=True)
    y1 = mod(to_dev(x_np, dtype, gpu_device))
    y2 = mod(to_dev(x_np, dtype, gpu_device))
    torch.cuda.synchronize()
    assert err(y1, oracle_y(prob, x_np)) <= TOL[dtype]
    assert torch.equal(y1, y2)
    assert all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == gpu_device.index)
