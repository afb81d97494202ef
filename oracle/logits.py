"""Final RMSNorm + lm_head + greedy argmax of the logit rows, restated in numpy (test
infrastructure only: imported by tests/, __graft_entry__.smoke() and bench.py's CPU leg).

Follows Qwen3Model.forward_packed's last two lines (model.py:108-110): the logit rows are
selected, RMSNorm'd in fp32 (RMSNorm.forward, layers.py:29-39) and cast to the model
dtype, then multiplied by the tied embedding (a bias-free Linear whose bf16 output is
rounded once). The engine's greedy pick is heads.argmax(dim=-1) (engine.py:470-473):
the first index of the largest rounded logit.
"""

from __future__ import annotations

import numpy as np

from oracle.rope import round_to


def final_norm(hidden: np.ndarray, indices: np.ndarray, weight: np.ndarray, eps: float,
               dtype: str = "bf16") -> np.ndarray:
    """Rows ``hidden[indices]`` normalised as RMSNorm.forward does: fp32 x * rsqrt(mean(x^2)
    + eps), times the fp32 weight, rounded to ``dtype``. Returns float32 [n, hidden]."""
    x = np.asarray(hidden, np.float32)[np.asarray(indices, np.int64)]
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    return round_to((x * r).astype(np.float32) * np.asarray(weight, np.float32), dtype)


def logits(normed: np.ndarray, embedding: np.ndarray, dtype: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """(exact float64 logits, logits rounded to ``dtype`` as float32), both [n, vocab]."""
    exact = np.asarray(normed, np.float64) @ np.asarray(embedding, np.float64).T
    return exact, round_to(exact.astype(np.float32), dtype)


def greedy(rounded: np.ndarray) -> np.ndarray:
    """First index of the row maximum (torch.argmax's tie rule), int64 [n]."""
    return np.argmax(np.asarray(rounded), axis=-1).astype(np.int64)


def final_norm_logits_argmax(hidden: np.ndarray, indices: np.ndarray, weight: np.ndarray,
                             embedding: np.ndarray, eps: float, dtype: str = "bf16"):
    """(token ids, rounded logits, exact logits) of the logit rows."""
    normed = final_norm(hidden, indices, weight, eps, dtype)
    exact, rounded = logits(normed, embedding, dtype)
    return greedy(rounded), rounded, exact
