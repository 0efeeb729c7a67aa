"""Decoder building blocks (``src/llmopt/model/layers.py``): RMSNorm, the SwiGLU MLP, the
paged-cache attention layer and the pre-norm decoder layer.

The projections are ``nn.Linear`` modules named as the reference names them (``q_proj`` ...
``down_proj``), so ``quantize_model_`` swaps them for :class:`QuantLinear` exactly as it
does in the reference. :meth:`PagedAttentionLayer.fuse_qkv` and :meth:`SwiGLUMLP.fuse_gate_up`
then merge the quantized projections into one packed weight each (one kernel launch for q, k
and v; one for gate and up with the SiLU-times-up product in the kernel's epilogue). On HIP
devices the attention step writes K/V with the cache-write kernels and, for one query token
per sequence, runs the paged decode-attention kernel; RMSNorm (with the residual add in front
of it) and the rotary embedding run as one kernel each (``llmopt_rmsnorm``, ``llmopt_rope``)
with the reference's roundings. Elsewhere every step is the reference's torch sequence.
"""

from __future__ import annotations

import torch
from torch import nn

from llmopt.attention.paged_attention import PagedAttention, PagedAttentionConfig
from llmopt.model.rotary import RotaryEmbedding, apply_rotary_pos_emb
from llmopt.quantization.fused import FusedQuantLinear, QuantSwiGLU
from llmopt.quantization.quant_linear import QuantLinear

__all__ = ["DecoderLayer", "PagedAttentionLayer", "RMSNorm", "SwiGLUMLP"]


def _hip(x: torch.Tensor) -> bool:
    return x.device.type == "cuda" and x.dtype in (torch.bfloat16, torch.float16)


class RMSNorm(nn.Module):
    """``x / sqrt(mean(x^2) + eps) * weight`` in fp32, returned in the input dtype
    (``layers.py:14-31``)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.fused_ops = True  # False: always the torch sequence (a reference-style comparator)

    def _reference(self, x: torch.Tensor) -> torch.Tensor:
        x32 = x.to(torch.float32)
        inv = torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)
        return (x32 * inv * self.weight.to(torch.float32)).to(x.dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused_ops and _hip(x):
            from llmopt.kernels import ops

            if ops.rmsnorm_supported(x, self.weight):
                return ops.rmsnorm(x, self.weight, self.eps)[0]
        return self._reference(x)

    def add_forward(self, x, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:  # noqa: ANN001
        """``(norm(h), h)`` with ``h = residual + x``: the residual add and the norm after it
        (``layers.py:185-195``), one kernel on HIP devices. ``x`` may be a linear's
        ``PartialSums`` (:meth:`SwiGLUMLP.forward` with ``defer``), which the kernel adds up."""
        if self.fused_ops and _hip(x):
            from llmopt.kernels import ops

            if ops.rmsnorm_supported(x, self.weight, residual):
                y, h = ops.rmsnorm(x, self.weight, self.eps, residual)
                return y, h
        if not isinstance(x, torch.Tensor):
            x = x.materialize()
        h = residual + x
        return self._reference(h), h


class SwiGLUMLP(nn.Module):
    """``down(silu(gate(x)) * up(x))`` (``layers.py:34-44``)."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        self.gate_up: QuantSwiGLU | None = None

    def fuse_gate_up(self) -> bool:
        """Merge quantized gate and up projections into one :class:`QuantSwiGLU`; returns
        whether it did (both must be :class:`QuantLinear` with the same settings)."""
        if self.gate_up is not None:
            return True
        if not (isinstance(self.gate_proj, QuantLinear) and isinstance(self.up_proj, QuantLinear)):
            return False
        self.gate_up = QuantSwiGLU(self.gate_proj, self.up_proj)
        del self.gate_proj, self.up_proj
        return True

    def forward(self, x: torch.Tensor, defer: bool = False):  # noqa: ANN201 - Tensor or ops.PartialSums
        """With ``defer``, a quantized ``down_proj`` may return its K-split partial sums, for the
        residual add + RMSNorm that follows to add up (:meth:`RMSNorm.add_forward`)."""
        if self.gate_up is not None:
            h = self.gate_up(x)
        else:
            h = torch.nn.functional.silu(self.gate_proj(x)) * self.up_proj(x)
        if defer and isinstance(self.down_proj, QuantLinear):
            return self.down_proj.forward_deferred(h)
        return self.down_proj(h)


class PagedAttentionLayer(nn.Module):
    """Self-attention over a :class:`PagedKVCache` (``layers.py:47-163``).

    ``forward(hidden [seq * q_len, hidden], positions [seq * q_len], cache, block_ids,
    context_lens, token_offsets, q_len)``: projects q/k/v, rotates q and k, writes this step's
    K/V at ``token_offsets`` (default ``context_lens - q_len``), attends over the cached context
    and projects the result. Without a cache, each sequence attends causally over its own
    ``q_len`` tokens.
    """

    def __init__(self, config: object, layer_idx: int, backend: str = "auto") -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        hidden = config.hidden_size
        self.q_proj = nn.Linear(hidden, self.num_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(hidden, self.num_kv_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(hidden, self.num_kv_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, hidden, bias=False)
        self.qkv_proj: FusedQuantLinear | None = None
        self.rotary = RotaryEmbedding(self.head_dim, config.max_position_embeddings, config.rope_theta)
        self.fused_ops = True  # False: the torch rotary sequence even on HIP devices
        self.attn = PagedAttention(self.num_heads, self.num_kv_heads, self.head_dim,
                                   config=PagedAttentionConfig(block_size=16), backend=backend)

    def fuse_qkv(self) -> bool:
        """Merge quantized q, k and v projections into one :class:`FusedQuantLinear`."""
        if self.qkv_proj is not None:
            return True
        parts = (self.q_proj, self.k_proj, self.v_proj)
        if not all(isinstance(p, QuantLinear) for p in parts):
            return False
        self.qkv_proj = FusedQuantLinear(parts)
        del self.q_proj, self.k_proj, self.v_proj
        return True

    @staticmethod
    def _fused_cache_write(cache: object, q: torch.Tensor) -> bool:
        """Whether the rotary kernel can store k and v into ``cache`` itself: a paged cache on
        the device holding the activations' dtype."""
        kc = getattr(cache, "key_cache", None)
        vc = getattr(cache, "value_cache", None)
        return (isinstance(kc, torch.Tensor) and isinstance(vc, torch.Tensor) and kc.dim() == 5
                and kc.dtype == q.dtype and vc.dtype == q.dtype and kc.device == q.device)

    def _project(self, hidden: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        if self.qkv_proj is not None:
            return self.qkv_proj(hidden)
        return self.q_proj(hidden), self.k_proj(hidden), self.v_proj(hidden)

    def forward(self, hidden: torch.Tensor, positions: torch.Tensor, cache: object | None = None,
                block_ids: torch.Tensor | None = None, context_lens: torch.Tensor | None = None,
                token_offsets: torch.Tensor | None = None, q_len: int = 1) -> torch.Tensor:
        total = int(hidden.shape[0])
        seqs = total // max(1, q_len)
        q, k, v = self._project(hidden)
        # Token-major [seq, q_len, heads, head_dim]: the cache layout, and cos/sin broadcast
        # over the heads of each token.
        paged = cache is not None and block_ids is not None and context_lens is not None
        offsets = None
        if paged:
            offsets = token_offsets if token_offsets is not None else context_lens - q_len
        written = False  # k and v already in the cache
        if self.fused_ops and _hip(q) and paged and q_len == 1 and self._fused_cache_write(cache, q):
            from llmopt.kernels import ops

            self.rotary.check(positions)
            if self.attn.backend == "hip":
                # Decode: rotary step, cache write and attention in one launch.
                try:
                    out = ops.paged_decode_attention_rope(
                        q.view(total, self.num_heads, self.head_dim),
                        k.view(total, self.num_kv_heads, self.head_dim),
                        v.view(total, self.num_kv_heads, self.head_dim), positions, self.rotary.cos_cached,
                        self.rotary.sin_cached, cache.key_cache[self.layer_idx], cache.value_cache[self.layer_idx],
                        block_ids, context_lens, offsets, self.attn.scale, self.attn.config.softcap)
                    return self.o_proj(out.view(total, self.num_heads * self.head_dim))
                except NotImplementedError:
                    pass  # a shape outside the attention kernel: the rotary kernel, then the module
            # Decode: the rotary kernel stores k and v straight into the cache slots.
            q = ops.rope_kv_write_decode(
                q.view(total, self.num_heads, self.head_dim), k.view(total, self.num_kv_heads, self.head_dim),
                v.view(total, self.num_kv_heads, self.head_dim), positions, self.rotary.cos_cached,
                self.rotary.sin_cached, cache.key_cache[self.layer_idx], cache.value_cache[self.layer_idx],
                block_ids, offsets)
            q = q.view(seqs, q_len, self.num_heads, self.head_dim)
            written = True
        elif self.fused_ops and _hip(q):
            from llmopt.kernels import ops

            self.rotary.check(positions)
            q, k, v = ops.rope(q.view(total, self.num_heads, self.head_dim),
                               k.view(total, self.num_kv_heads, self.head_dim), positions,
                               self.rotary.cos_cached, self.rotary.sin_cached,
                               v=v.view(total, self.num_kv_heads, self.head_dim))
            q = q.view(seqs, q_len, self.num_heads, self.head_dim)
            k = k.view(seqs, q_len, self.num_kv_heads, self.head_dim)
            v = v.view(seqs, q_len, self.num_kv_heads, self.head_dim)
        else:
            v = v.reshape(seqs, q_len, self.num_kv_heads, self.head_dim)
            q = q.reshape(seqs, q_len, self.num_heads, self.head_dim)
            k = k.reshape(seqs, q_len, self.num_kv_heads, self.head_dim)
            cos, sin = self.rotary(positions, dtype=q.dtype)
            cos = cos.view(seqs, q_len, 1, self.head_dim)
            sin = sin.view(seqs, q_len, 1, self.head_dim)
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
            k = k.contiguous()
            v = v.contiguous()
        query = q.permute(0, 2, 1, 3)  # [seq, heads, q_len, head_dim]
        if paged:
            if written:
                pass
            elif q_len == 1:
                cache.write_decode(self.layer_idx, block_ids, offsets, k[:, 0], v[:, 0])
            else:
                cache.write(self.layer_idx, block_ids, offsets, k, v)
            out = self.attn.forward(query, cache, self.layer_idx, block_ids, context_lens, q_len)
        else:
            out = self._causal_attention(query, k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3))
        out = out.permute(0, 2, 1, 3).reshape(total, self.num_heads * self.head_dim)
        return self.o_proj(out)

    def _causal_attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """Cache-free path: ``[seq, heads, q_len, d]`` attending causally over its own tokens
        (the reference's ``_dense_attention``, ``layers.py:145-163``), computed in fp32."""
        group = self.num_heads // self.num_kv_heads
        k = k.repeat_interleave(group, dim=1).float()
        v = v.repeat_interleave(group, dim=1).float()
        scores = torch.matmul(q.float(), k.transpose(-1, -2).contiguous()) * self.attn.scale
        q_len = int(q.shape[2])
        mask = torch.ones(q_len, q_len, dtype=torch.bool, device=q.device).triu(1)
        scores = scores.masked_fill(mask, float("-inf"))
        return torch.matmul(torch.softmax(scores, dim=-1), v).to(q.dtype)


class DecoderLayer(nn.Module):
    """Pre-norm block: ``h + attn(norm(h))``, then ``h + mlp(norm(h))`` (``layers.py:166-195``)."""

    def __init__(self, config: object, layer_idx: int, backend: str = "auto") -> None:
        super().__init__()
        self.self_attn = PagedAttentionLayer(config, layer_idx, backend)
        self.mlp = SwiGLUMLP(config.hidden_size, config.intermediate_size)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, hidden: torch.Tensor, positions: torch.Tensor, cache: object | None = None,
                block_ids: torch.Tensor | None = None, context_lens: torch.Tensor | None = None,
                token_offsets: torch.Tensor | None = None, q_len: int = 1) -> torch.Tensor:
        hidden, mlp_out = self.forward_chained(hidden, None, positions, cache, block_ids, context_lens,
                                               token_offsets, q_len)
        return hidden + mlp_out

    def forward_chained(self, hidden: torch.Tensor, pending, positions: torch.Tensor,  # noqa: ANN001
                        cache: object | None = None, block_ids: torch.Tensor | None = None,
                        context_lens: torch.Tensor | None = None, token_offsets: torch.Tensor | None = None,
                        q_len: int = 1, defer_mlp: bool = False) -> tuple[torch.Tensor, object]:
        """The layer with its final residual add left to the caller: takes ``hidden`` plus the
        previous layer's not-yet-added MLP output ``pending`` (or None) and returns ``(hidden,
        mlp_out)``. The input stream is ``hidden + pending``, formed inside the first norm's
        kernel, so a stack of layers runs one fused add + norm per residual add. With
        ``defer_mlp`` the MLP output may be its down projection's partial sums, which the next
        layer's first norm adds up (one launch fewer, the same bits)."""
        if pending is None:
            normed = self.input_layernorm(hidden)
        else:
            normed, hidden = self.input_layernorm.add_forward(pending, hidden)
        attn = self.self_attn(normed, positions, cache, block_ids, context_lens, token_offsets, q_len)
        normed, hidden = self.post_attention_layernorm.add_forward(attn, hidden)
        return hidden, self.mlp(normed, defer=defer_mlp)
