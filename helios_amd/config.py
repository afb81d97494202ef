"""Model shape the paged KV pool is sized from.

The pool and the attention path read only the shape fields here. Their names, order and
defaults are the Qwen3-4B values of the reference's config (src/helios/runtime/qwen3/config.py:9-20),
so a config object built for the reference's decoder can be handed to these classes
unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Qwen3Config:
    vocab_size: int = 151_936          # tied embedding rows
    context_length: int = 40_960       # longest sequence a page table must cover
    hidden_size: int = 2_560           # residual width
    n_heads: int = 32                  # query heads per layer
    n_layers: int = 36                 # one K and one V pool tensor each
    hidden_dim: int = 9_728            # SwiGLU intermediate width
    head_dim: int = 128                # elements per head row
    n_kv_heads: int = 8                # heads per pool token row
    rope_base: float = 1_000_000.0     # RoPE theta
    rms_norm_eps: float = 1e-6
    dtype: torch.dtype = torch.bfloat16

    def __post_init__(self) -> None:
        if self.n_kv_heads <= 0 or self.n_heads % self.n_kv_heads:
            raise ValueError(f"{self.n_heads} query heads cannot be grouped over {self.n_kv_heads} KV heads")
        if self.head_dim <= 0 or self.n_layers <= 0 or self.context_length <= 0:
            raise ValueError("head_dim, n_layers and context_length must be positive")

    @property
    def group_size(self) -> int:
        """Query heads that share one KV head."""
        return self.n_heads // self.n_kv_heads


def qwen3_4b_config(dtype: torch.dtype = torch.bfloat16) -> Qwen3Config:
    """The Qwen3-4B shape in the given compute dtype."""
    return Qwen3Config(dtype=dtype)
