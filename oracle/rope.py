"""Per-head RMSNorm + RoPE of new queries/keys, restated in numpy (test infrastructure).

Follows RMSNorm.forward (layers.py:30-40), rope_parameters (layers.py:43-51) and
apply_rope with position_ids (layers.py:54-72), as GroupedQueryAttention.forward applies
them (layers.py:146-160). Values are rounded to the element type at the same two points
as the reference: after the norm's scale, and after the rotation.
"""

from __future__ import annotations

import numpy as np


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16 or fp16 (nearest even) and return them as float32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rope_tables(head_dim: int, rows: int, base: float) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [rows, head_dim] in float32: angles p * base^(-2i/d), halves repeated."""
    inv = (1.0 / (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)))).astype(np.float32)
    ang = np.arange(rows, dtype=np.float32)[:, None] * inv[None, :]
    ang = np.concatenate([ang, ang], axis=1).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def norm_rope(x: np.ndarray, weight: np.ndarray, cos: np.ndarray, sin: np.ndarray,
              positions: np.ndarray, eps: float, dtype: str = "bf16") -> np.ndarray:
    """x: [rows, heads, d] (values already representable in `dtype`), positions [rows].
    Returns [rows, heads, d] float32 holding `dtype` values."""
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    n = round_to((x * r).astype(np.float32) * np.asarray(weight, np.float32), dtype)
    c = cos[np.asarray(positions, np.int64)][:, None, :]
    s = sin[np.asarray(positions, np.int64)][:, None, :]
    half = d // 2
    rot = np.concatenate([-n[..., half:], n[..., :half]], axis=-1)
    return round_to((n * c).astype(np.float32) + (rot * s).astype(np.float32), dtype)
