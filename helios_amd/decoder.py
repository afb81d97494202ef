"""The reference's Qwen3 decoder forward for packed ticks, on the paged-KV path.

Mirrors Qwen3Model._forward_packed (src/helios/runtime/qwen3/model.py:92-110) and the
TransformerBlock / GroupedQueryAttention / FeedForward forwards it runs
(layers.py:13-27, :131-164, :202-232), with random-init weights (no checkpoint is
fetched). This is the caller of the hot path, kept to measure it in place: torch runs
the projections, MLP and norms on hipBLASLt / elementwise kernels, and the attention
step goes through ``PackedBatchCache.attend_projected`` (fused q/k norm + RoPE + KV
append, then paged attention) or, with ``fused_rope=False``, through the reference's
own sequence (torch q/k norm and RoPE, then ``attend``).

The q, k and v projections are one GEMM over concatenated weights, and gate/up another;
the arithmetic is otherwise the reference's.
"""

from __future__ import annotations

import torch

from helios_amd import ops
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import PackedBatchCache


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward (layers.py:36-40)."""
    dtype = x.dtype
    x = x.float()
    return (x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * weight).to(dtype)


def _rope_tables(config: Qwen3Config, device) -> tuple[torch.Tensor, torch.Tensor]:
    """rope_parameters (layers.py:43-51)."""
    inv = 1.0 / (config.rope_base ** (torch.arange(0, config.head_dim, 2, dtype=torch.float32) / config.head_dim))
    angles = torch.arange(config.context_length, dtype=torch.float32).unsqueeze(1) * inv.unsqueeze(0)
    angles = torch.cat((angles, angles), dim=1)
    return torch.cos(angles).to(device), torch.sin(angles).to(device)


def _apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """apply_rope with position_ids (layers.py:54-72)."""
    half = x.shape[-1] // 2
    c = cos[positions].unsqueeze(1)
    s = sin[positions].unsqueeze(1)
    return (x * c + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * s).to(x.dtype)


class PagedQwen3Decoder:
    """Random-init Qwen3 weights in the reference's layout, on one device."""

    def __init__(self, config: Qwen3Config, device, *, seed: int = 0, std: float = 0.02) -> None:
        self.config = config
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(seed)
        dt = config.dtype
        hq, hkv, d = config.n_heads * config.head_dim, config.n_kv_heads * config.head_dim, config.head_dim

        def w(*shape):
            return (torch.randn(shape, generator=g, device=self.device, dtype=torch.float32) * std).to(dt)

        self.embedding = w(config.vocab_size, config.hidden_size)  # tied with the output
        self.layers = []
        for _ in range(config.n_layers):
            self.layers.append({
                "qkv": w(hq + 2 * hkv, config.hidden_size),
                "o": w(config.hidden_size, hq),
                "gate_up": w(2 * config.hidden_dim, config.hidden_size),
                "down": w(config.hidden_size, config.hidden_dim),
                "input_norm": torch.ones(config.hidden_size, device=self.device),
                "post_norm": torch.ones(config.hidden_size, device=self.device),
                "q_norm": torch.ones(d, device=self.device),
                "k_norm": torch.ones(d, device=self.device),
            })
        self.final_norm = torch.ones(config.hidden_size, device=self.device)
        self.cos, self.sin = _rope_tables(config, self.device)

    @torch.inference_mode()
    def forward_packed(self, input_ids: torch.Tensor, cache: PackedBatchCache, *,
                       fused_rope: bool = True, attention_events: list | None = None,
                       greedy: bool = False) -> torch.Tensor:
        """Logits of the tick's logit rows (model.py:92-110), or with ``greedy`` their
        argmax token ids (engine.py:470-473). ``attention_events`` collects (start, end)
        CUDA events around each layer's attention step.

        With ``fused_rope`` (this build's sequence) the greedy ids come from the fused
        final-norm / logits / argmax kernels and no logits are written; otherwise the
        reference's logits are computed and ``argmax`` taken."""
        config = self.config
        if input_ids.shape != (1, sum(cache.counts)):
            raise ValueError(f"input_ids must be [1, {sum(cache.counts)}]: one token per packed row of the tick.")
        hq, hkv, d = config.n_heads * config.head_dim, config.n_kv_heads * config.head_dim, config.head_dim
        eps = config.rms_norm_eps
        x = self.embedding[input_ids]
        tokens = x.shape[1]
        for index, layer in enumerate(self.layers):
            h = _rms_norm(x, layer["input_norm"], eps)
            qkv = h @ layer["qkv"].t()
            q, k, v = qkv[..., :hq], qkv[..., hq:hq + hkv], qkv[..., hq + hkv:]
            if attention_events is not None:
                start = torch.cuda.Event(enable_timing=True)
                start.record()
            if fused_rope:
                context = cache.attend_projected(index, q, k, v, layer["q_norm"], layer["k_norm"],
                                                 self.cos, self.sin, eps)
            else:
                qh = q.reshape(1, tokens, config.n_heads, d).transpose(1, 2)
                kh = k.reshape(1, tokens, config.n_kv_heads, d).transpose(1, 2)
                vh = v.reshape(1, tokens, config.n_kv_heads, d).transpose(1, 2)
                qh = _apply_rope(_rms_norm(qh, layer["q_norm"], eps), self.cos, self.sin, cache.positions)
                kh = _apply_rope(_rms_norm(kh, layer["k_norm"], eps), self.cos, self.sin, cache.positions)
                context = cache.attend(index, qh, kh, vh)
            if attention_events is not None:
                end = torch.cuda.Event(enable_timing=True)
                end.record()
                attention_events.append((start, end))
            context = context.transpose(1, 2).reshape(1, tokens, -1)
            x = x + context @ layer["o"].t()
            h = _rms_norm(x, layer["post_norm"], eps)
            gate, up = (h @ layer["gate_up"].t()).chunk(2, dim=-1)
            x = x + (torch.nn.functional.silu(gate) * up) @ layer["down"].t()
        cache.advance_packed()
        if greedy and fused_rope:
            return ops.final_norm_logits_argmax(x, cache.logit_indices, self.final_norm, self.embedding,
                                                eps).token_ids
        x = x.index_select(1, cache.logit_indices)
        logits = (_rms_norm(x, self.final_norm, eps).to(config.dtype) @ self.embedding.t())[0]
        return logits.argmax(dim=-1) if greedy else logits
