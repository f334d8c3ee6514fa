"""Host-side behaviour of the reference-mirroring Python layer (no GPU):
factory dispatch and validation messages, op registration and schema."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import ssalaad_amd
from ssalaad_amd import LRSLinear
from ssalaad_amd.ls_linear import _LRSLinearLR


def _block_sparse(n, m, block, coords, seed=0):
    g = torch.Generator().manual_seed(seed)
    S = torch.zeros(n, m)
    for br, bc in coords:
        S[br * block:(br + 1) * block, bc * block:(bc + 1) * block] = torch.randn(block, block, generator=g)
    return S


def test_block_kernel_rejects_unsupported_block_shape():
    """Mirror of tests/test_ssalaad.py:340-354: non-square blocks fail loudly."""
    torch.manual_seed(0)
    A, B = torch.randn(64, 8), torch.randn(8, 96)
    S = _block_sparse(64, 96, 8, [(0, 1), (1, 0)])
    with pytest.raises(ValueError, match="square"):
        LRSLinear(A, B, S.to_sparse_bsr(blocksize=(8, 8)), in_features=96, out_features=64,
                  block_p=8, block_q=16)


@pytest.mark.parametrize("block,message", [(8, "GPU"), (48, "square"), (16, "GPU")])
def test_cpu_tensors_get_the_reference_cpu_message_or_no_fallback(block, message):
    """CPU tensors: blocks the reference's AVX2 class refuses get its "square"
    message (ls_linear.py:265-273); the others find no CPU path here."""
    A, B = torch.randn(96, 4), torch.randn(4, 96)
    S = _block_sparse(96, 96, block, [(0, 0)])
    with pytest.raises(ValueError, match=message):
        LRSLinear(A, B, S.to_sparse_bsr(blocksize=(block, block)), in_features=96,
                  out_features=96, block_p=block, block_q=block)


def test_sparse_s_without_block_shape_is_rejected():
    A, B = torch.randn(32, 4), torch.randn(4, 32)
    S = _block_sparse(32, 32, 16, [(0, 0)])
    with pytest.raises(ValueError, match="block shape"):
        LRSLinear(A, B, S.to_sparse_bsr(blocksize=(16, 16)), in_features=32, out_features=32)


def test_cpu_tensors_have_no_fallback():
    A, B = torch.randn(32, 4), torch.randn(4, 32)
    S = _block_sparse(32, 32, 16, [(0, 0)])
    with pytest.raises(ValueError, match="GPU"):
        LRSLinear(A, B, S.to_sparse_bsr(blocksize=(16, 16)), in_features=32, out_features=32,
                  block_p=16, block_q=16)


def test_nm_needs_a_gpu_and_a_2_4_mask():
    """ls_linear.py:254-256: N:M runs on the GPU with a 2:4 mask only."""
    A, B = torch.randn(32, 4), torch.randn(4, 32)
    S = _block_sparse(32, 32, 16, [(0, 0)])
    with pytest.raises(ValueError, match="N:M inference requires CUDA and a 2:4 mask"):
        LRSLinear(A, B, S, in_features=32, out_features=32, nm_n=2, nm_m=4)
    with pytest.raises(ValueError, match="N:M inference requires CUDA and a 2:4 mask"):
        LRSLinear(A, B, S, in_features=32, out_features=32, nm_n=1, nm_m=4)


def test_zero_s_gives_the_low_rank_module():
    """ls_linear.py:252-253; also the module's shape validation (:20-27)."""
    A, B = torch.randn(32, 4), torch.randn(4, 48)
    mod = LRSLinear(A, B, torch.zeros(32, 48), in_features=48, out_features=32)
    assert isinstance(mod, _LRSLinearLR) and mod.kind == "lr_only" and mod.r == 4
    assert "S=zero" in mod.extra_repr()
    with pytest.raises(ValueError, match="must match"):
        LRSLinear(torch.randn(32, 4), torch.randn(5, 48), torch.zeros(32, 48), in_features=48,
                  out_features=32)
    with pytest.raises(ValueError, match="must equal"):
        LRSLinear(A, B, torch.zeros(32, 48), in_features=40, out_features=32)
    with pytest.raises(ValueError, match="GPU"):
        mod(torch.randn(2, 48))


def test_op_is_registered_with_the_reference_schema():
    op = torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_
    schema = str(op.default._schema)
    assert schema.startswith("ssalaad::tilelang_bsr_addmm_inplace_dense_(Tensor(a!) out_inplace, Tensor x, Tensor crow_indices, Tensor col_indices, Tensor values, Tensor active_rows) -> ()")
    assert ssalaad_amd.get_tuned_config(64, 64)["BM"] == 1


def test_op_fake_kernel_returns_none():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        out = torch.empty(4, 64)
        x = torch.empty(4, 64)
        crow = torch.empty(2, dtype=torch.int32)
        col = torch.empty(1, dtype=torch.int32)
        vals = torch.empty(1, 64, 64)
        act = torch.empty(1, dtype=torch.int32)
        assert torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(out, x, crow, col, vals, act) is None


def test_op_validates_arguments_on_cpu():
    out = torch.zeros(4, 64)
    x = torch.zeros(4, 64)
    crow = torch.tensor([0, 1], dtype=torch.int32)
    col = torch.tensor([0], dtype=torch.int32)
    vals = torch.zeros(1, 64, 64)
    act = torch.tensor([0], dtype=torch.int32)
    f = ssalaad_amd.bsr_addmm_inplace_
    with pytest.raises(TypeError):
        f(out.long(), x, crow, col, vals, act)
    with pytest.raises(TypeError):
        f(out, x.double(), crow, col, vals, act)
    with pytest.raises(TypeError):
        f(out, x, crow.long(), col, vals, act)
    with pytest.raises(ValueError, match="GPU"):
        f(out, x, crow, col, vals, act)


def test_factor_from_svd_mirror():
    """tests/test_ssalaad.py:276-283 on the mirrored helper (torch ops, any device)."""
    torch.manual_seed(0)
    matrix = torch.randn(16, 3) @ torch.randn(3, 32)
    svd = torch.linalg.svd(matrix, full_matrices=False)
    A, B = ssalaad_amd.factor_from_svd(*svd, 3)
    torch.testing.assert_close(A @ B, matrix, atol=1e-4, rtol=1e-4)
    A0, B0 = ssalaad_amd.factor_from_svd(*svd, 0)
    assert A0.shape == (16, 0) and B0.shape == (0, 32)


def test_encoder_front_end_checks_shape_first():
    with pytest.raises(ValueError, match="not divisible"):
        ssalaad_amd.dense_to_bsr(torch.zeros(10, 16), 4, 4)


def _tiny_llama():
    from ssalaad_amd.bundle import build_model_from_config

    return build_model_from_config({
        "model_type": "llama", "hidden_size": 64, "intermediate_size": 96, "num_hidden_layers": 1,
        "num_attention_heads": 4, "num_key_value_heads": 4, "vocab_size": 50,
        "max_position_embeddings": 16, "hidden_act": "silu"})


def test_generate_checks_arguments_like_the_reference():
    """generate.py:14-19: the same errors before any work."""
    from ssalaad_amd import generate

    model = _tiny_llama()
    with pytest.raises(ValueError, match="nonempty"):
        generate(model, torch.zeros(2, 0, dtype=torch.long), 1)
    with pytest.raises(ValueError, match="nonempty"):
        generate(model, torch.zeros(3, dtype=torch.long), 1)
    with pytest.raises(ValueError, match="nonnegative"):
        generate(model, torch.zeros(1, 4, dtype=torch.long), -1)
    with pytest.raises(ValueError, match="context length"):
        generate(model, torch.zeros(1, 10, dtype=torch.long), 7)


def test_decode_engine_has_no_cpu_path():
    from ssalaad_amd import DecodeEngine
    from ssalaad_amd.bundle import build_model_from_config

    model = build_model_from_config({
        "model_type": "llama", "hidden_size": 128, "intermediate_size": 64, "num_hidden_layers": 1,
        "num_attention_heads": 2, "num_key_value_heads": 2, "vocab_size": 50,
        "max_position_embeddings": 16, "hidden_act": "silu"})
    with pytest.raises(ValueError, match="ROCm GPU"):
        DecodeEngine(model, max_batch=1, max_context=4)


def test_decode_engine_rejects_head_widths_without_a_kernel():
    from ssalaad_amd import DecodeEngine
    from ssalaad_amd.bundle import build_model_from_config

    model = build_model_from_config({
        "model_type": "llama", "hidden_size": 96, "intermediate_size": 64, "num_hidden_layers": 1,
        "num_attention_heads": 2, "num_key_value_heads": 2, "vocab_size": 50,
        "max_position_embeddings": 16, "hidden_act": "silu"})
    with pytest.raises(NotImplementedError, match="head_dim 48"):
        DecodeEngine(model, max_batch=1, max_context=4)


def test_nm24_prefill_layout_decodes_to_the_same_matrix():
    """The 2:4 blocks in the prefill row kernel's layout (values per output
    column, position nibbles per group) hold exactly the packed matrix: decoded
    independently here from the layout include/ssalaad_amd.h documents."""
    import numpy as np

    from ssalaad_amd.artifact import _nm24_pack, nm24_prefill_layout

    g = torch.Generator().manual_seed(3)
    n, m = 70, 100
    count = torch.randint(0, 3, (n, m // 4), generator=g)
    order = torch.rand(n, m // 4, 4, generator=g).argsort(-1).argsort(-1)
    keep = order < count[..., None]
    S = (torch.randn(n, m // 4, 4, generator=g) * keep).reshape(n, m).to(torch.bfloat16)
    pk = _nm24_pack(S)
    pf = nm24_prefill_layout(pk["blocks"])
    assert pf.shape == (pk["blocks"].shape[0], ssalaad_amd._lib.load().ssl_nm24_prefill_block_bytes())
    crow, col = pk["crow"].numpy(), pk["col"].numpy()
    D = np.zeros((pk["NB"] * 32, pk["NBK"] * 32), np.float32)
    for by in range(pk["NB"]):
        for k in range(crow[by], crow[by + 1]):
            vals = pf[k, :1024].view(torch.bfloat16).float().numpy().reshape(32, 2, 8)
            idx = pf[k, 1024:].view(torch.int32).numpy().astype(np.int64) & 0xFFFFFFFF
            for j in range(32):
                for h in range(2):
                    for q in range(4):
                        nib = (int(idx[j]) >> (16 * h + 4 * q)) & 0xF
                        i0, i1 = nib & 3, nib >> 2
                        assert i0 < i1
                        kk = col[k] * 32 + 16 * h + 4 * q
                        D[by * 32 + j, kk + i0] += vals[j, h, 2 * q]
                        D[by * 32 + j, kk + i1] += vals[j, h, 2 * q + 1]
    assert np.array_equal(D[:n, :m], S.float().numpy())


def test_first_op_call_under_graph_capture_raises(monkeypatch):
    """The op's first call with a structure copies it to the host to build the
    plan; under HIP graph capture it raises instead, naming prepare_bsr_addmm."""
    import torch
    from ssalaad_amd import addmm_inplace

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    crow = torch.tensor([0, 1], dtype=torch.int32)
    col = torch.tensor([0], dtype=torch.int32)
    act = torch.tensor([0], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="prepare_bsr_addmm"):
        addmm_inplace._validated_host_structure(crow, col, act, 1, 1)


@pytest.mark.parametrize("p,q,elem,s", [(16, 32, 2, 16), (32, 16, 2, 16), (48, 48, 2, 16),
                                        (64, 32, 2, 32), (128, 320, 2, 32), (128, 512, 2, 64), (96, 96, 2, 16),
                                        (64, 64, 4, 32), (64, 192, 4, 32)])
def test_square_view_is_the_same_matrix(p, q, elem, s):
    """Many-token calls with blocks the tiled kernels do not run as they are use
    the widest square block that tiles them (fp32 at most 32): the re-blocked
    structure densifies to the same matrix, rows in order."""
    from oracle import slr_oracle as orc
    from ssalaad_amd import _reblock

    P, Q = _reblock.kernel_block_shape(p, q)
    assert not _reblock.prefill_square(P, Q, elem)
    assert _reblock.square_block(P, Q, elem) == s
    rng = np.random.default_rng(p + q)
    NB, NBK = 5, 4
    counts = np.array([2, 0, 4, 1, 3])
    crow = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    col = np.concatenate([np.sort(rng.permutation(NBK)[:c]) for c in counts]).astype(np.int32)
    vals = rng.standard_normal((int(crow[-1]), p, q))
    vt = torch.from_numpy(vals.transpose(0, 2, 1).copy())               # stored (nnz, q, p)
    crow2, col2, vt2 = _reblock.reblock(crow, col, vt, p, q, s, s)
    dense = orc.bsr_to_dense(crow, col, vals, NB * p, NBK * q)
    dense2 = orc.bsr_to_dense(crow2, col2, vt2.numpy().transpose(0, 2, 1), NB * p, NBK * q)
    np.testing.assert_array_equal(dense, dense2)
    assert crow2.shape[0] - 1 == NB * (p // s)
    assert np.all(np.diff(crow2) >= 0) and crow2[-1] == col2.shape[0]
    for r in range(NB * (p // s)):                                        # columns ascending
        assert np.all(np.diff(col2[crow2[r]:crow2[r + 1]]) > 0)
