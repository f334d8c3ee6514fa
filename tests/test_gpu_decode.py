"""KV-cached decode step on the GPU: kernels and engine against the oracle.

Kernel tests compare each decode kernel with the same operation written in
torch (transformers' own functions where they exist: LlamaRMSNorm,
apply_rotary_pos_emb, the rotary tables) or with a float64 softmax-attention
on the CPU. Engine tests run a small SLR-compressed LLaMA / Qwen3 through
DecodeEngine and compare its logits at every step with oracle/decode_oracle.py
(float64, pinned against transformers' full-sequence forward on the CPU).

Tolerances (max-abs normalised error):
  fp32  kernels and model logits 1e-5 (the SLR linear's fp32 bar; measured on
        MI355X: logits within 7e-7 of the oracle);
  16-bit kernels: bit-exact where torch rounds the same values at the same
        points (rotary embedding, residual add), else one rounding of the
        output (bf16 1e-2, fp16 2e-3);
  bf16 model logits: at most twice the error of the reference's own bf16
        forward on the same weights, measured in the same test. That forward
        (the Hugging Face model on the CPU in bf16 with each projection
        computed as the reference GPU module does, _ReferenceSLR) is itself
        1.2e-2 to 1.4e-2 from the float64 oracle on these models: it rounds to
        bf16 about ten times per layer, each worth up to 2^-9 relative. No
        bf16 implementation meets a 1e-2 bar on them, so the bar is set
        relative to the reference's own rounding, with 3e-2 as a ceiling.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_oracle as dor

pytestmark = pytest.mark.gpu

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _lib():
    from ssalaad_amd import _lib as L

    return L, L.load()


def _err(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


# --------------------------------------------------------------- kernels --


def _attention(q, kc, vc, pos, heads, kvh, hd, ctx, n_split=None):
    L, lib = _lib()
    B = q.shape[0]
    ns = n_split or lib.ssl_decode_attention_splits(B, heads, kvh, ctx)
    ws = torch.empty(lib.ssl_decode_attention_workspace_size(B, heads, hd, ns), dtype=torch.uint8,
                     device=q.device)
    cnt = torch.zeros(lib.ssl_decode_attention_counter_count(B, heads, kvh), dtype=torch.int32,
                      device=q.device)
    out = torch.full((B, heads * hd), float("nan"), dtype=q.dtype, device=q.device)
    rc = lib.ssl_decode_attention(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                  out.data_ptr(), out.stride(0), B, heads, kvh, hd, ctx,
                                  hd ** -0.5, ns, ws.data_ptr(), ws.numel(), cnt.data_ptr(),
                                  cnt.numel(), L.dtype_code(q.dtype), L.stream_ptr(q.device))
    L.check(rc, "ssl_decode_attention")
    torch.cuda.synchronize()
    assert (cnt == 0).all()  # every arrival counter is back at zero
    return out


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("heads,kvh", [(4, 4), (8, 2), (16, 1), (6, 2)])
@pytest.mark.parametrize("n_split", [None, 1, 7])
def test_attention_matches_float64_softmax(dt, hd, heads, kvh, n_split, gpu_device):
    dtype = DTYPES[dt]
    g = torch.Generator().manual_seed(hd + heads + (n_split or 0))
    B, ctx = 3, 300
    positions = [0, 63, 299] if n_split != 7 else [64, 1, 150]
    q = torch.randn(B, heads, hd, generator=g).to(dtype)
    kc = torch.randn(B, kvh, ctx, hd, generator=g).to(dtype)
    vc = torch.randn(B, kvh, ctx, hd, generator=g).to(dtype)
    pos = torch.tensor(positions, dtype=torch.int32)
    out = _attention(q.to(gpu_device), kc.to(gpu_device), vc.to(gpu_device), pos.to(gpu_device),
                     heads, kvh, hd, ctx, n_split)
    torch.cuda.synchronize()
    want = np.zeros((B, heads * hd))
    for b in range(B):
        want[b] = dor.attention(q[b].double().numpy(), kc[b, :, : positions[b] + 1].double().numpy(),
                                vc[b, :, : positions[b] + 1].double().numpy(), hd ** -0.5).reshape(-1)
    tol = {"f32": 1e-5, "bf16": 1e-2, "f16": 2e-3}[dt]
    assert _err(out.float().cpu(), want) <= tol


def test_attention_long_context_and_every_split_count(gpu_device):
    """A 4096-position context, bf16, MHA with 128-wide heads; every split count
    from 1 to 128 gives the same answer to fp32 rounding."""
    g = torch.Generator().manual_seed(5)
    B, H, hd, ctx = 2, 4, 128, 4096
    q = torch.randn(B, H, hd, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, H, ctx, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, H, ctx, hd, generator=g).to(torch.bfloat16)
    pos = torch.tensor([4095, 2049], dtype=torch.int32)
    qd, kd, vd, pd = (t.to(gpu_device) for t in (q, kc, vc, pos))
    want = np.zeros((B, H * hd))
    for b in range(B):
        L = int(pos[b]) + 1
        want[b] = dor.attention(q[b].double().numpy(), kc[b, :, :L].double().numpy(),
                                vc[b, :, :L].double().numpy(), hd ** -0.5).reshape(-1)
    for ns in (1, 2, 5, 16, 33, 64, 128):
        out = _attention(qd, kd, vd, pd, H, H, hd, ctx, ns).float().cpu()
        assert _err(out, want) <= 1e-2, ns


def test_add_rmsnorm_matches_llama_rmsnorm(gpu_device):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    L, lib = _lib()
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        g = torch.Generator().manual_seed(1)
        rows, hidden = 5, 2048 + 96
        h = torch.randn(rows, hidden, generator=g).to(dtype).to(gpu_device)
        d = torch.randn(rows, hidden, generator=g).to(dtype).to(gpu_device)
        norm = LlamaRMSNorm(hidden, eps=1e-5).to(gpu_device, dtype)
        with torch.no_grad():
            norm.weight.copy_(1 + 0.2 * torch.randn(hidden, generator=g))
            want_h = h + d
            want = norm(want_h)
        out = torch.empty_like(h)
        for delta in (d, None):
            hh = h.clone() if delta is not None else want_h.clone()
            rc = lib.ssl_add_rmsnorm(hh.data_ptr(), hh.stride(0), L.ptr(delta),
                                     delta.stride(0) if delta is not None else 0,
                                     norm.weight.data_ptr(), out.data_ptr(), out.stride(0), rows,
                                     hidden, 1e-5, L.dtype_code(dtype), L.stream_ptr(gpu_device))
            L.check(rc, "ssl_add_rmsnorm")
            torch.cuda.synchronize()
            assert torch.equal(hh, want_h)  # the residual add rounds exactly as torch does
            tol = {torch.float32: 1e-6, torch.bfloat16: 8e-3, torch.float16: 1e-3}[dtype]
            assert _err(out.float().cpu(), want.float().cpu()) <= tol


def test_embed_rmsnorm_gathers_then_normalises(gpu_device):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    L, lib = _lib()
    for dtype, hidden in ((torch.bfloat16, 2048), (torch.float32, 300), (torch.float16, 8192)):
        g = torch.Generator().manual_seed(4)
        vocab, rows = 1000, 6
        emb = torch.randn(vocab, hidden + 8, generator=g).to(dtype).to(gpu_device)[:, :hidden]
        toks = torch.tensor([5, 999, 0, 5, -1, 1000], dtype=torch.int64, device=gpu_device)
        norm = LlamaRMSNorm(hidden, eps=1e-6).to(gpu_device, dtype)
        with torch.no_grad():
            norm.weight.copy_(1 + 0.2 * torch.randn(hidden, generator=g))
        h = torch.full((rows, hidden), 7.0, dtype=dtype, device=gpu_device)
        out = torch.empty_like(h)
        rc = lib.ssl_embed_rmsnorm(emb.data_ptr(), emb.stride(0), vocab, toks.data_ptr(),
                                   h.data_ptr(), h.stride(0), norm.weight.data_ptr(),
                                   out.data_ptr(), out.stride(0), rows, hidden, 1e-6,
                                   L.dtype_code(dtype), L.stream_ptr(gpu_device))
        L.check(rc, "ssl_embed_rmsnorm")
        torch.cuda.synchronize()
        assert torch.equal(h[:4], emb[toks[:4]])
        assert (h[4:] == 0).all()  # tokens outside the vocabulary give zero rows
        with torch.no_grad():
            want = norm(emb[toks[:4]])
        tol = {torch.float32: 1e-6, torch.bfloat16: 8e-3, torch.float16: 1e-3}[dtype]
        assert _err(out[:4].float().cpu(), want.float().cpu()) <= tol
        assert (out[4:] == 0).all()


@pytest.mark.parametrize("model_type", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_kv_append_matches_transformers(model_type, dtype, gpu_device):
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb
    from transformers import LlamaConfig

    L, lib = _lib()
    B, H, KH, hd, ctx = 3, 8, 2, 128, 40
    cfg = LlamaConfig(hidden_size=H * hd, num_attention_heads=H, num_key_value_heads=KH,
                      head_dim=hd, max_position_embeddings=ctx, rope_theta=500000.0)
    rot = LlamaRotaryEmbedding(cfg).to(gpu_device)
    cos, sin = rot(torch.zeros(1, dtype=dtype, device=gpu_device),
                   position_ids=torch.arange(ctx, device=gpu_device)[None])
    cos, sin = cos[0].contiguous(), sin[0].contiguous()
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, H * hd + 32, generator=g).to(dtype).to(gpu_device)[:, : H * hd]
    k = torch.randn(B, KH * hd, generator=g).to(dtype).to(gpu_device)
    v = torch.randn(B, KH * hd, generator=g).to(dtype).to(gpu_device)
    pos = torch.tensor([0, 17, 39], dtype=torch.int32, device=gpu_device)
    qn = kn = None
    qs, ks = q.reshape(B, H, hd), k.reshape(B, KH, hd)
    if model_type == "qwen3":
        from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

        qn_m, kn_m = Qwen3RMSNorm(hd, 1e-6).to(gpu_device, dtype), Qwen3RMSNorm(hd, 1e-6).to(gpu_device, dtype)
        with torch.no_grad():
            qn_m.weight.copy_(1 + 0.3 * torch.randn(hd, generator=g))
            kn_m.weight.copy_(1 + 0.3 * torch.randn(hd, generator=g))
            qs, ks = qn_m(qs), kn_m(ks)
        qn, kn = qn_m.weight, kn_m.weight
    c, s = cos[pos.long()], sin[pos.long()]  # [B, hd] -> [B, 1, hd] inside
    want_q, want_k = apply_rotary_pos_emb(qs, ks, c, s, unsqueeze_dim=1)
    q_out = torch.empty(B, H, hd, dtype=dtype, device=gpu_device)
    kc = torch.zeros(B, KH, ctx, hd, dtype=dtype, device=gpu_device)
    vc = torch.zeros_like(kc)
    rc = lib.ssl_rope_kv_append(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(),
                                v.stride(0), cos.data_ptr(), sin.data_ptr(), L.ptr(qn), L.ptr(kn),
                                1e-6, pos.data_ptr(), q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                B, H, KH, hd, ctx, L.dtype_code(dtype), L.stream_ptr(gpu_device))
    L.check(rc, "ssl_rope_kv_append")
    torch.cuda.synchronize()
    got_k = torch.stack([kc[b, :, int(pos[b])] for b in range(B)])
    got_v = torch.stack([vc[b, :, int(pos[b])] for b in range(B)])
    assert torch.equal(got_v, v.reshape(B, KH, hd))
    written = (kc != 0).any(-1).sum().item()
    assert written == B * KH  # one position per sequence and head, nothing else
    if model_type == "llama":
        assert torch.equal(q_out, want_q) and torch.equal(got_k, want_k)
    else:
        tol = 1e-6 if dtype == torch.float32 else 1e-2
        assert _err(q_out.float().cpu(), want_q.float().cpu()) <= tol
        assert _err(got_k.float().cpu(), want_k.float().cpu()) <= tol


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("heads,kvh", [(4, 4), (8, 2), (6, 2), (16, 1)])
@pytest.mark.parametrize("model_type,n_split",
                         [("llama", None), ("llama", 7), ("llama", 200), ("qwen3", None)])
def test_rope_attention_equals_rope_then_attention(dt, hd, heads, kvh, model_type, n_split,
                                                   gpu_device):
    """The fused launch against ssl_rope_kv_append + ssl_decode_attention on the
    same inputs: bit-identical output and caches (Qwen3's per-head norm sums
    its squares in another order: within one rounding)."""
    L, lib = _lib()
    dtype = DTYPES[dt]
    g = torch.Generator().manual_seed(hd * 7 + heads + kvh + (n_split or 0))
    B, ctx = 4, 300
    positions = [0, 63, 299, 128] if n_split is None else [64, 1, 150, 299]
    dev = gpu_device
    q = torch.randn(B, heads * hd + 64, generator=g).to(dtype).to(dev)[:, : heads * hd]
    k = torch.randn(B, kvh * hd, generator=g).to(dtype).to(dev)
    v = torch.randn(B, kvh * hd, generator=g).to(dtype).to(dev)
    cos = (torch.rand(ctx, hd, generator=g) * 2 - 1).to(dtype).to(dev)
    sin = (torch.rand(ctx, hd, generator=g) * 2 - 1).to(dtype).to(dev)
    qn = kn = None
    if model_type == "qwen3":
        qn = (1 + 0.3 * torch.randn(hd, generator=g)).to(dtype).to(dev)
        kn = (1 + 0.3 * torch.randn(hd, generator=g)).to(dtype).to(dev)
    kc0 = torch.randn(B, kvh, ctx, hd, generator=g).to(dtype).to(dev)
    vc0 = torch.randn(B, kvh, ctx, hd, generator=g).to(dtype).to(dev)
    pos = torch.tensor(positions, dtype=torch.int32, device=dev)
    code, st = L.dtype_code(dtype), L.stream_ptr(dev)

    kcA, vcA = kc0.clone(), vc0.clone()
    q_out = torch.empty(B, heads, hd, dtype=dtype, device=dev)
    rc = lib.ssl_rope_kv_append(q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(),
                                v.stride(0), cos.data_ptr(), sin.data_ptr(), L.ptr(qn), L.ptr(kn),
                                1e-6, pos.data_ptr(), q_out.data_ptr(), kcA.data_ptr(),
                                vcA.data_ptr(), B, heads, kvh, hd, ctx, code, st)
    L.check(rc, "ssl_rope_kv_append")
    outA = _attention(q_out, kcA, vcA, pos, heads, kvh, hd, ctx, n_split)

    kcB, vcB = kc0.clone(), vc0.clone()
    ns = n_split or lib.ssl_decode_attention_splits(B, heads, kvh, ctx)
    ws = torch.empty(lib.ssl_decode_attention_workspace_size(B, heads, hd, ns), dtype=torch.uint8,
                     device=dev)
    cnt = torch.zeros(lib.ssl_decode_attention_counter_count(B, heads, kvh), dtype=torch.int32,
                      device=dev)
    outB = torch.full((B, heads * hd), float("nan"), dtype=dtype, device=dev)
    rc = lib.ssl_decode_rope_attention(
        q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
        cos.data_ptr(), sin.data_ptr(), L.ptr(qn), L.ptr(kn), 1e-6, pos.data_ptr(),
        kcB.data_ptr(), vcB.data_ptr(), outB.data_ptr(), outB.stride(0), B, heads, kvh, hd, ctx,
        hd ** -0.5, ns, ws.data_ptr(), ws.numel(), cnt.data_ptr(), cnt.numel(), code, st)
    L.check(rc, "ssl_decode_rope_attention")
    torch.cuda.synchronize()
    assert (cnt == 0).all()
    assert torch.equal(vcB, vcA)
    if model_type == "llama":
        assert torch.equal(kcB, kcA)
        assert torch.equal(outB, outA)
    else:
        tol = {"f32": 1e-6, "bf16": 1e-2, "f16": 2e-3}[dt]
        changed = (kcB != kc0).any(-1)
        assert torch.equal(changed, (kcA != kc0).any(-1))  # only the new positions
        assert _err(kcB.float().cpu(), kcA.float().cpu()) <= tol
        assert _err(outB.float().cpu(), outA.float().cpu()) <= 2 * tol


def test_silu_mul_matches_torch(gpu_device):
    L, lib = _lib()
    for dtype in (torch.float32, torch.bfloat16):
        g = torch.Generator().manual_seed(3)
        gate = torch.randn(4, 5472, generator=g).to(dtype).to(gpu_device)
        up = torch.randn(4, 5472, generator=g).to(dtype).to(gpu_device)
        n = 5461
        out = torch.zeros(4, 5464, dtype=dtype, device=gpu_device)
        rc = lib.ssl_silu_mul(gate.data_ptr(), gate.stride(0), up.data_ptr(), up.stride(0),
                              out.data_ptr(), out.stride(0), 4, n, L.dtype_code(dtype),
                              L.stream_ptr(gpu_device))
        L.check(rc, "ssl_silu_mul")
        want = torch.nn.functional.silu(gate[:, :n]) * up[:, :n]
        torch.cuda.synchronize()
        tol = 1e-6 if dtype == torch.float32 else 8e-3
        assert _err(out[:, :n].float().cpu(), want.float().cpu()) <= tol
        assert (out[:, n:] == 0).all()


# ---------------------------------------------------------------- engine --


class _ReferenceSLR(torch.nn.Module):
    """The reference GPU modules' arithmetic on the CPU, in the model's dtype.
    Block S (ssalaad/efficient/ls_linear.py:124-137): F.linear(F.linear(x, B),
    A) rounded as torch rounds it, then x·Sᵀ accumulated in fp32 onto that
    output and rounded once, as the in-place op does (addmm_inplace.py:41-82).
    2:4 S (ls_linear.py:211-219): y = F.linear(x, S), then y += latent·Aᵀ
    with one rounding (addmm_), latent = F.linear(x, B)."""

    def __init__(self, A, B, S_dense, nm=False):
        super().__init__()
        self.A, self.B, self.S, self.nm = A, B, S_dense, nm

    def forward(self, x):
        F = torch.nn.functional
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if self.nm:
            latent = F.linear(x2, self.B)
            y = F.linear(x2, self.S)
            y = (y.float() + latent.float() @ self.A.float().t()).to(x.dtype)
        else:
            y = F.linear(F.linear(x2, self.B), self.A)
            y = (y.float() + x2.float() @ self.S.float().t()).to(x.dtype)
        return y.reshape(*shape[:-1], y.shape[-1])


def _slr_pair(*args, **kwargs):
    model, dense, _ = _slr_triple(*args, **kwargs)
    return model, dense


def _slr_triple(model_type, dtype, kv_heads, dev, seed=0, head_dim=64, heads=4, layers=2,
                nm=False):
    """An SLR-compressed model on the GPU, its dense float64 twin on the CPU
    (every projection W = A·B + S from the same dtype-valued factors) and, for
    16-bit dtypes, the same model on the CPU with the reference module's
    arithmetic in that dtype (None for fp32). With `nm`, S is 2:4-sparse along
    the input features (two of every four kept). dev=None builds no GPU model."""
    import copy

    from ssalaad_amd import LRSLinear
    from ssalaad_amd.bundle import build_model_from_config

    cfg = {"model_type": model_type, "hidden_size": 256, "intermediate_size": 352,
           "num_hidden_layers": layers, "num_attention_heads": heads,
           "num_key_value_heads": kv_heads, "head_dim": head_dim, "vocab_size": 384,
           "max_position_embeddings": 128, "rms_norm_eps": 1e-6, "rope_theta": 10000.0,
           "hidden_act": "silu", "tie_word_embeddings": False}
    torch.manual_seed(seed)
    g = torch.Generator().manual_seed(seed)
    model = build_model_from_config(cfg, attn_implementation="sdpa")
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" in name:
                prm.copy_(1 + 0.1 * torch.randn(prm.shape, generator=g))
            elif "embed" in name:
                prm.copy_(torch.randn(prm.shape, generator=g))
            else:
                prm.copy_(0.1 * torch.randn(prm.shape, generator=g))
    model = model.to(dtype)
    mirror = copy.deepcopy(model).eval() if dtype != torch.float32 else None
    dense = build_model_from_config(cfg, attn_implementation="eager").double()
    dense.load_state_dict({k: t.double() for k, t in model.state_dict().items()})
    p, r = 32, 32
    for li in range(layers):
        for part, proj in (("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
                           ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
                           ("mlp", "down_proj")):
            parent = model.get_submodule(f"model.layers.{li}.{part}")
            old = getattr(parent, proj)
            n, m = old.out_features, old.in_features
            NB, NBK = n // p, m // p
            k = NB * NBK // 2
            slots = torch.randperm(NB * NBK, generator=g)[:k].sort().values
            crow = torch.zeros(NB + 1, dtype=torch.int64)
            crow[1:] = torch.bincount(slots // NBK, minlength=NB).cumsum(0)
            vals = (0.05 * torch.randn(k, p, p, generator=g)).to(dtype)
            A = (0.1 * torch.randn(n, r, generator=g)).to(dtype)
            B = (0.1 * torch.randn(r, m, generator=g)).to(dtype)
            S = torch.sparse_bsr_tensor(crow, slots % NBK, vals, size=(n, m))
            if nm:
                keep = torch.rand(n, m // 4, 4, generator=g).argsort(-1).argsort(-1) < 2
                Sd = ((0.05 * torch.randn(n, m, generator=g)) * keep.reshape(n, m)).to(dtype)
                with torch.no_grad():
                    dense.get_submodule(f"model.layers.{li}.{part}.{proj}").weight.copy_(
                        A.double() @ B.double() + Sd.double())
                if mirror is not None:
                    setattr(mirror.get_submodule(f"model.layers.{li}.{part}"), proj,
                            _ReferenceSLR(A, B, Sd, nm=True))
                if dev is not None:
                    setattr(parent, proj, LRSLinear(A.to(dev), B.to(dev), Sd.to(dev),
                                                    in_features=m, out_features=n, nm_n=2, nm_m=4))
                continue
            with torch.no_grad():
                dense.get_submodule(f"model.layers.{li}.{part}.{proj}").weight.copy_(
                    A.double() @ B.double() + S.to_dense().double())
            if mirror is not None:
                setattr(mirror.get_submodule(f"model.layers.{li}.{part}"), proj,
                        _ReferenceSLR(A, B, S.to_dense()))
            if dev is None:
                continue
            setattr(parent, proj, LRSLinear(
                A.to(dev), B.to(dev), torch.sparse_bsr_tensor(crow.to(dev), (slots % NBK).to(dev),
                                                              vals.to(dev), size=(n, m)),
                in_features=m, out_features=n, block_p=p, block_q=p))
    return (model.to(dev).eval() if dev is not None else None), dense.eval(), mirror


TOL_MODEL = {torch.float32: 1e-5, torch.bfloat16: 3e-2}  # bf16: the ceiling of the relative bar
BF16_VS_REFERENCE = 2.0


def _mirror_logits(mirror, ids):
    """Full-sequence logits of the reference-arithmetic CPU model (float32 copy)."""
    with torch.no_grad():
        return mirror(input_ids=ids, use_cache=False).logits.float().numpy()


def _bar(dtype, ref_err):
    """The logits bar: 1e-5 for fp32; for 16-bit, twice the reference's own
    error (ref_err) up to the ceiling."""
    if dtype == torch.float32:
        return TOL_MODEL[dtype]
    return min(TOL_MODEL[dtype], BF16_VS_REFERENCE * ref_err)


@pytest.mark.parametrize("model_type,kv_heads,head_dim,heads", [
    ("llama", 4, 64, 4), ("llama", 2, 128, 4), ("qwen3", 2, 64, 8),
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_engine_steps_match_the_oracle(model_type, kv_heads, head_dim, heads, dtype, gpu_device):
    from ssalaad_amd import DecodeEngine

    model, dense, mirror = _slr_triple(model_type, dtype, kv_heads, gpu_device, head_dim=head_dim,
                                       heads=heads)
    P = dor.params_from_hf(dense)
    B, T = 3, 12
    ids = torch.randint(0, 384, (B, T), generator=torch.Generator().manual_seed(7))
    ref = _mirror_logits(mirror, ids) if mirror is not None else None
    eng = DecodeEngine(model, max_batch=4, max_context=T)
    cache = dor.KVCache.empty(len(P.layers), B, P.kv_heads, T, P.head_dim)
    worst = ref_worst = 0.0
    for t in range(T):
        got = eng.step(ids[:, t], [t] * B).float().cpu().numpy()
        want = dor.decode_step(P, cache, ids[:, t].numpy(), [t] * B)
        worst = max(worst, _err(got, want))
        if ref is not None:
            ref_worst = max(ref_worst, _err(ref[:, t], want))
    print(f"[decode] {model_type} kv{kv_heads} hd{head_dim} {dtype}: worst logits error "
          f"{worst:.2e} (reference arithmetic: {ref_worst:.2e})")
    assert worst <= _bar(dtype, ref_worst)


@pytest.mark.parametrize("seed", range(12))
def test_random_engine_configs_match_the_oracle(seed, gpu_device):
    """Random decoder shapes through DecodeEngine, every step against the oracle:
    LLaMA or Qwen3, 2–16 query heads (the configs need hidden 256 to be a
    multiple) over any divisor as key/value heads, head_dim 64/128/256, fp32 or
    bf16, 1–4 sequences, 4–20 steps."""
    from ssalaad_amd import DecodeEngine

    rng = np.random.default_rng(900 + seed)
    model_type = ("llama", "qwen3")[int(rng.integers(2))]
    heads = int(rng.choice([2, 4, 8, 16]))
    kvh = int(rng.choice([d for d in range(1, heads + 1) if heads % d == 0]))
    hd = int(rng.choice([64, 128, 256]))
    dtype = (torch.float32, torch.bfloat16)[int(rng.integers(2))]
    B, T = int(rng.integers(1, 5)), int(rng.integers(4, 21))
    model, dense, mirror = _slr_triple(model_type, dtype, kvh, gpu_device, seed=seed, head_dim=hd,
                                       heads=heads)
    P = dor.params_from_hf(dense)
    ids = torch.randint(0, 384, (B, T), generator=torch.Generator().manual_seed(seed))
    ref = _mirror_logits(mirror, ids) if mirror is not None else None
    eng = DecodeEngine(model, max_batch=B, max_context=T)
    cache = dor.KVCache.empty(len(P.layers), B, P.kv_heads, T, P.head_dim)
    case = (seed, model_type, heads, kvh, hd, dtype, B, T)
    errs, ref_errs = [], []
    for t in range(T):
        got = eng.step(ids[:, t], [t] * B).float().cpu().numpy()
        want = dor.decode_step(P, cache, ids[:, t].numpy(), [t] * B)
        errs.append(_err(got, want))
        if ref is not None:
            ref_errs.append(_err(ref[:, t], want))
    worst, ref_worst = max(errs), max(ref_errs, default=0.0)
    assert worst <= _bar(dtype, ref_worst), (case, worst, ref_worst)


@pytest.mark.parametrize("model_type,kv_heads", [("llama", 2), ("qwen3", 4)])
def test_engine_with_2to4_projections_matches_the_oracle(model_type, kv_heads, gpu_device):
    """Every projection with 2:4 S (bf16): the grouped q/k/v and gate/up launches
    and the decode step on packed 2:4 blocks, against the oracle at every step."""
    from ssalaad_amd import DecodeEngine

    model, dense, mirror = _slr_triple(model_type, torch.bfloat16, kv_heads, gpu_device, seed=11,
                                       nm=True)
    assert all(getattr(m, "kind", "") == "nm" for n_, m in model.named_modules()
               if n_.endswith(("q_proj", "down_proj")))
    P = dor.params_from_hf(dense)
    B, T = 2, 10
    ids = torch.randint(0, 384, (B, T), generator=torch.Generator().manual_seed(12))
    ref = _mirror_logits(mirror, ids)
    eng = DecodeEngine(model, max_batch=B, max_context=T)
    cache = dor.KVCache.empty(len(P.layers), B, P.kv_heads, T, P.head_dim)
    errs, ref_errs = [], []
    for t in range(T):
        got = eng.step(ids[:, t], [t] * B).float().cpu().numpy()
        want = dor.decode_step(P, cache, ids[:, t].numpy(), [t] * B)
        errs.append(_err(got, want))
        ref_errs.append(_err(ref[:, t], want))
    assert max(errs) <= _bar(torch.bfloat16, max(ref_errs)), (max(errs), max(ref_errs))


def test_engine_ragged_positions_and_batch_sizes(gpu_device):
    """Sequences at different positions in one step, and steps of 1 to 3 rows
    sharing the same cache slots (one graph per batch size)."""
    from ssalaad_amd import DecodeEngine

    model, dense = _slr_pair("llama", torch.float32, 2, gpu_device, seed=3)
    P = dor.params_from_hf(dense)
    ids = torch.randint(0, 384, (3, 10), generator=torch.Generator().manual_seed(8))
    eng = DecodeEngine(model, max_batch=3, max_context=16)
    cache = dor.KVCache.empty(len(P.layers), 3, P.kv_heads, 16, P.head_dim)
    # schedule: (rows in the step, position per row)
    sched = [(3, [0, 0, 0]), (1, [1]), (2, [2, 1]), (3, [3, 2, 1]), (1, [4]), (3, [5, 3, 2]),
             (2, [6, 4]), (3, [7, 5, 3])]
    for rows, positions in sched:
        toks = [int(ids[b, positions[b]]) for b in range(rows)]
        got = eng.step(toks, positions).cpu().numpy()
        sub = dor.KVCache([k[:rows] for k in cache.k], [v[:rows] for v in cache.v])
        want = dor.decode_step(P, sub, toks, positions)
        assert _err(got, want) <= TOL_MODEL[torch.float32], (rows, positions)


def test_engine_graph_replays_equal_eager_steps(gpu_device):
    """The captured step replayed with other GPU work in between gives exactly
    the eager step's logits, every replay."""
    from ssalaad_amd import DecodeEngine

    model, _ = _slr_pair("llama", torch.bfloat16, 2, gpu_device, seed=4)
    ids = torch.randint(0, 384, (2, 8), generator=torch.Generator().manual_seed(9))
    ge = DecodeEngine(model, max_batch=2, max_context=8, use_graphs=True)
    ee = DecodeEngine(model, max_batch=2, max_context=8, use_graphs=False)
    for t in range(8):
        a = ge.step(ids[:, t], [t, t]).clone()
        junk = torch.randn(1024, 1024, device=gpu_device).sum()  # eager work between replays
        b = ee.step(ids[:, t], [t, t]).clone()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(a, b), t


def test_generate_matches_the_oracle_greedy_loop(gpu_device):
    from ssalaad_amd import generate

    model, dense = _slr_pair("llama", torch.float32, 4, gpu_device, seed=5)
    P = dor.params_from_hf(dense)
    prompt = torch.randint(0, 384, (2, 5), generator=torch.Generator().manual_seed(10))
    out = generate(model, prompt, 8)
    assert out.shape == (2, 13) and torch.equal(out[:, :5], prompt)
    assert np.array_equal(out.numpy(), dor.greedy(P, prompt.numpy(), 8))
    assert torch.equal(generate(model, prompt, 0), prompt)


def test_engine_rejects_positions_outside_the_cache(gpu_device):
    from ssalaad_amd import DecodeEngine

    model, _ = _slr_pair("llama", torch.float32, 4, gpu_device, seed=6, layers=1)
    eng = DecodeEngine(model, max_batch=2, max_context=4)
    with pytest.raises(ValueError, match="positions"):
        eng.step([1, 2], [0, 4])
    with pytest.raises(ValueError, match="positions"):
        eng.step([1], [-1])
    with pytest.raises(ValueError, match="tokens"):
        eng.step([1, 2, 3], [0, 0, 0])
