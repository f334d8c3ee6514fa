"""KV-cached decode of a compressed LLaMA / Qwen3 model on the HIP kernels.

The reference generates greedily by recomputing the whole prefix with the
Hugging Face forward each step (ssalaad/inference/generate.py:1-26) and has no
cached decode. `DecodeEngine` runs one token per sequence per step from a
per-layer key/value cache instead, with the same per-token arithmetic as the
Hugging Face forward of the model `build_efficient_model` returns:

  per layer   add_rmsnorm (residual add fused; the embedding gather at layer 0)
              -> q,k,v in one fused SLR launch
              -> one launch: rope, cache append and split-context attention (its
              slices merged by the last one to finish) -> o_proj
              -> add_rmsnorm -> gate,up in one fused SLR launch -> silu·up
              -> down_proj
  then        the final add_rmsnorm and the LM head (a plain library GEMM).

Every step of a batch size is captured once in a HIP graph and replayed; the
positions live in device memory, so one graph serves every position. The
projections are this package's `LRSLinear` modules (plain `nn.Linear` layers
of an uncompressed projection run as library GEMMs). There is no CPU path:
the engine needs the HIP library and a ROCm device.

`generate(model, input_ids, max_new_tokens)` keeps the reference's signature,
checks and greedy rule on top of the engine; the prompt is fed through the
same decode step one position at a time.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _lib, _runtime
from .ls_linear import LRSLinearGroup, _LRSLinearBase


def _round_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


class _Layer:
    __slots__ = ("in_norm", "post_norm", "q_norm", "k_norm", "qkv", "o", "gu", "down")


def _group(*mods: nn.Module):
    """One callable returning every module's output for the same x: a fused
    launch when every member is an SLR module that can share one."""
    if all(isinstance(m, _LRSLinearBase) for m in mods):
        try:
            return LRSLinearGroup(*mods)
        except ValueError:
            pass
    return lambda x: tuple(m(x) for m in mods)


class DecodeEngine:
    """Greedy-decoding state for one model: caches, buffers and step graphs.

    `step(tokens, positions)` takes one token per sequence (batch row b is
    cache slot b) at its position and returns the logits [B, vocab] (a view of
    an engine buffer, valid until the next step). Positions may differ per
    sequence; every cached position below a sequence's position must have
    been written by an earlier step.
    """

    def __init__(self, model: nn.Module, *, max_batch: int, max_context: int,
                 use_graphs: bool = True) -> None:
        cfg = model.config
        if cfg.model_type not in ("llama", "qwen3"):
            raise ValueError(f"Unsupported model type: {cfg.model_type}")
        if getattr(cfg, "hidden_act", "silu") != "silu":
            raise ValueError(f"unsupported activation {cfg.hidden_act}; the decode step uses silu")
        if any(t != "full_attention" for t in (getattr(cfg, "layer_types", None) or [])):
            raise NotImplementedError("sliding-window layers are not supported by the decode step")
        hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        if hd not in (64, 128, 256):
            raise NotImplementedError(f"head_dim {hd}: the decode attention runs 64, 128 or 256")
        rot = model.model.rotary_emb
        if getattr(rot, "rope_type", "default") == "dynamic":
            raise NotImplementedError("dynamic rotary scaling is not supported by the decode step")
        if max_batch < 1 or max_context < 1:
            raise ValueError("max_batch and max_context must be positive")
        embed = model.model.embed_tokens.weight
        if not embed.is_cuda:
            raise ValueError("the decode engine runs on a ROCm GPU; move the model to 'cuda' first")
        self.lib = _lib.load()
        self.device = embed.device
        self.dtype = embed.dtype
        self.dt = _lib.dtype_code(self.dtype)
        self.hidden = cfg.hidden_size
        self.heads = cfg.num_attention_heads
        self.kv_heads = cfg.num_key_value_heads
        self.head_dim = getattr(cfg, "head_dim", None) or self.hidden // self.heads
        self.eps = float(cfg.rms_norm_eps)
        self.scale = self.head_dim ** -0.5
        self.max_batch, self.max_context = max_batch, max_context
        self.embed = embed
        self.norm = model.model.norm.weight
        self.lm_head = model.lm_head
        self.layers: list[_Layer] = []
        for layer in model.model.layers:
            at, mlp = layer.self_attn, layer.mlp
            L = _Layer()
            L.in_norm = layer.input_layernorm.weight
            L.post_norm = layer.post_attention_layernorm.weight
            L.q_norm = at.q_norm.weight if hasattr(at, "q_norm") else None
            L.k_norm = at.k_norm.weight if hasattr(at, "k_norm") else None
            L.qkv = _group(at.q_proj, at.k_proj, at.v_proj)
            L.o = at.o_proj
            L.gu = _group(mlp.gate_proj, mlp.up_proj)
            L.down = mlp.down_proj
            self.layers.append(L)
        self.ffn = model.model.layers[0].mlp.down_proj.in_features
        dev, dt = self.device, self.dtype
        nl, kvh, hd = len(self.layers), self.kv_heads, self.head_dim
        self.k_cache = torch.zeros(nl, max_batch, kvh, max_context, hd, dtype=dt, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        with torch.no_grad():
            pos = torch.arange(max_context, device=dev)[None]
            cos, sin = rot(torch.zeros(1, dtype=dt, device=dev), position_ids=pos)
        self.cos = cos[0].to(dt).contiguous()
        self.sin = sin[0].to(dt).contiguous()
        self.h = torch.zeros(max_batch, self.hidden, dtype=dt, device=dev)
        self.xn = torch.zeros_like(self.h)
        self.att = torch.zeros(max_batch, self.heads * hd, dtype=dt, device=dev)
        self.act = torch.zeros(max_batch, _round_up(self.ffn, 8), dtype=dt, device=dev)
        self.tokens = torch.zeros(max_batch, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(max_batch, dtype=torch.int32, device=dev)
        ws = self.lib.ssl_decode_attention_workspace_size(max_batch, self.heads, hd, 64)
        self.attn_ws = torch.empty(max(ws, 16), dtype=torch.uint8, device=dev)
        # arrival counters of the attention slices: zero at rest, reset by the kernel
        nc = self.lib.ssl_decode_attention_counter_count(max_batch, self.heads, self.kv_heads)
        self.attn_cnt = torch.zeros(max(nc, 1), dtype=torch.int32, device=dev)
        self.use_graphs = use_graphs
        # The device's wait-status word sits in host memory the kernels write
        # directly: checked before every step with a plain read, so a fused
        # launch whose wait gave up is reported by the first step that starts
        # after its store landed, at no per-step cost.
        self._status = _runtime.status_word(dev)
        self._stream = torch.cuda.Stream(dev)
        self._graphs: dict[int, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}

    # ------------------------------------------------------------------ calls
    def _check(self, rc: int, what: str) -> None:
        _lib.check(rc, what)

    def _add_rmsnorm(self, B: int, delta: torch.Tensor | None, w: torch.Tensor) -> None:
        st = _lib.stream_ptr(self.device)
        rc = self.lib.ssl_add_rmsnorm(
            self.h.data_ptr(), self.h.stride(0), _lib.ptr(delta),
            delta.stride(0) if delta is not None else 0, w.data_ptr(), self.xn.data_ptr(),
            self.xn.stride(0), B, self.hidden, self.eps, self.dt, st)
        self._check(rc, "ssl_add_rmsnorm")

    def _body(self, B: int) -> torch.Tensor:
        lib, st = self.lib, _lib.stream_ptr(self.device)
        H, KH, hd, ctx = self.heads, self.kv_heads, self.head_dim, self.max_context
        n_split = lib.ssl_decode_attention_splits(B, H, KH, ctx)
        delta = None
        for li, L in enumerate(self.layers):
            if li == 0:  # h = embed[tokens], fused with the first norm
                rc = lib.ssl_embed_rmsnorm(
                    self.embed.data_ptr(), self.embed.stride(0), self.embed.shape[0],
                    self.tokens.data_ptr(), self.h.data_ptr(), self.h.stride(0),
                    L.in_norm.data_ptr(), self.xn.data_ptr(), self.xn.stride(0), B, self.hidden,
                    self.eps, self.dt, st)
                self._check(rc, "ssl_embed_rmsnorm")
            else:
                self._add_rmsnorm(B, delta, L.in_norm)
            x = self.xn[:B]
            q, k, v = L.qkv(x)
            # rotary embedding, cache append and attention in one launch
            rc = lib.ssl_decode_rope_attention(
                q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0),
                self.cos.data_ptr(), self.sin.data_ptr(), _lib.ptr(L.q_norm), _lib.ptr(L.k_norm),
                self.eps, self.pos.data_ptr(), self.k_cache[li].data_ptr(),
                self.v_cache[li].data_ptr(), self.att.data_ptr(), self.att.stride(0), B, H, KH, hd,
                ctx, self.scale, n_split, self.attn_ws.data_ptr(), self.attn_ws.numel(),
                self.attn_cnt.data_ptr(), self.attn_cnt.numel(), self.dt, st)
            self._check(rc, "ssl_decode_rope_attention")
            o = L.o(self.att[:B])
            self._add_rmsnorm(B, o, L.post_norm)
            g, u = L.gu(x)
            rc = lib.ssl_silu_mul(g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0),
                                  self.act.data_ptr(), self.act.stride(0), B, self.ffn, self.dt,
                                  st)
            self._check(rc, "ssl_silu_mul")
            delta = L.down(self.act[:B, : self.ffn])
        self._add_rmsnorm(B, delta, self.norm)
        return self.lm_head(self.xn[:B])

    # ---------------------------------------------------------------- public
    def clear_status(self) -> None:
        """Reset the device's wait-status word once this engine's work is done."""
        self._stream.synchronize()
        _runtime.reset_status(self.device)

    @torch.no_grad()
    def step(self, tokens, positions) -> torch.Tensor:
        tokens = torch.as_tensor(tokens, dtype=torch.int64).reshape(-1)
        positions = torch.as_tensor(positions, dtype=torch.int32).reshape(-1)
        B = tokens.numel()
        if B < 1 or B > self.max_batch or positions.numel() != B:
            raise ValueError(f"a step takes 1 to {self.max_batch} tokens, one position each")
        if not tokens.is_cuda and tokens.numel() and (
                int(tokens.min()) < 0 or int(tokens.max()) >= self.embed.shape[0]):
            raise ValueError(f"token ids must lie in [0, {self.embed.shape[0]})")
        pos_h = positions.to("cpu")
        if int(pos_h.min()) < 0 or int(pos_h.max()) >= self.max_context:
            raise ValueError(f"positions must lie in [0, {self.max_context})")
        if self._status.read() != 0:
            raise RuntimeError(
                "a fused SLR launch of an earlier step gave up waiting for another "
                "workgroup (bounded wait); its logits are unreliable. Call clear_status() "
                "before stepping again.")
        cur = torch.cuda.current_stream(self.device)
        s = self._stream
        s.wait_stream(cur)
        with torch.cuda.stream(s):
            self.tokens[:B].copy_(tokens, non_blocking=False)
            self.pos[:B].copy_(pos_h, non_blocking=False)
            if not self.use_graphs:
                out = self._body(B)
            elif B in self._graphs:
                g, out = self._graphs[B]
                g.replay()
            else:
                out = self._body(B)  # eager first run: also warms plans and workspaces
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=s):
                    gout = self._body(B)
                self._graphs[B] = (g, gout)
        cur.wait_stream(s)
        return out


@torch.no_grad()
def generate(model, input_ids: torch.Tensor, max_new_tokens: int, *,
             engine: DecodeEngine | None = None) -> torch.Tensor:
    """Greedy generation with the cached decode step; the reference's checks and
    output (ssalaad/inference/generate.py:12-26): the prompt followed by
    `max_new_tokens` argmax tokens."""
    if input_ids.ndim != 2 or input_ids.shape[1] == 0:
        raise ValueError("Expected a nonempty batch of input token IDs.")
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be nonnegative.")
    if input_ids.shape[1] + max_new_tokens > model.config.max_position_embeddings:
        raise ValueError("Prompt and output exceed the configured context length.")
    B, T = input_ids.shape
    if max_new_tokens == 0:
        return input_ids
    eng = engine or DecodeEngine(model, max_batch=B, max_context=T + max_new_tokens)
    dev = eng.device
    ids = input_ids.to(dev)
    finite = torch.ones((), dtype=torch.bool, device=dev)
    logits = None
    for t in range(T):
        logits = eng.step(ids[:, t], [t] * B)
    out = [ids]
    for t in range(T, T + max_new_tokens):
        finite &= torch.isfinite(logits).all()
        nxt = logits.argmax(-1)
        out.append(nxt[:, None])
        if t + 1 < T + max_new_tokens:
            logits = eng.step(nxt, [t] * B)
    if not bool(finite):
        raise FloatingPointError("Non-finite inference logits.")
    return torch.cat(out, dim=1).to(input_ids.device)
