"""The final-norm / logits / greedy-argmax oracle: against the reference's op sequence in
torch (CPU), a pure-Python brute force, and cases whose answer is fixed in advance (a
planted winner, exact ties, scale invariance of the norm)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dense_torch, logits as lg
from oracle.rope import round_to


def _case(seed, rows=40, hidden=256, vocab=300, picks=7):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, rows, hidden, generator=g).to(torch.bfloat16)
    w = (1 + 0.2 * torch.randn(hidden, generator=g)).float()
    emb = (0.05 * torch.randn(vocab, hidden, generator=g)).to(torch.bfloat16)
    idx = torch.randperm(rows, generator=g)[:picks]
    return x, w, emb, idx


@pytest.mark.parametrize("seed", range(3))
def test_matches_reference_op_sequence(seed):
    x, w, emb, idx = _case(seed)
    # model.py:108-110 in torch: index_select, RMSNorm (fp32, cast back), Linear.
    sel = x.index_select(1, idx)
    normed = dense_torch.rms_norm(sel, w, 1e-6)[0]
    ref_logits = torch.nn.functional.linear(normed.float(), emb.float()).to(torch.bfloat16)
    ref_ids = ref_logits.argmax(dim=-1)
    ids, rounded, exact = lg.final_norm_logits_argmax(x[0].float().numpy(), idx.numpy(), w.numpy(),
                                                      emb.float().numpy(), 1e-6)
    # The norm: equal up to one bf16 ulp (sum order of the mean of squares).
    got_n = lg.final_norm(x[0].float().numpy(), idx.numpy(), w.numpy(), 1e-6)
    ref_n = normed.float().numpy()
    assert np.all(np.abs(got_n - ref_n) <= 2.0 ** -7 * np.abs(ref_n) + 1e-12)
    assert np.mean(got_n != ref_n) < 1e-2
    # The logits: fp32 (torch) vs float64 sums, each rounded once.
    ref_l = ref_logits.float().numpy()
    assert np.all(np.abs(rounded - ref_l) <= 2.0 ** -7 * np.abs(ref_l) + 1e-6)
    # The pick: identical wherever the top two exact logits are apart by more than the
    # rounding can move them.
    top2 = np.sort(exact, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2.0 ** -6 * np.abs(top2[:, 1])
    assert clear.sum() >= 3
    np.testing.assert_array_equal(ids[clear], ref_ids.numpy()[clear])


def test_brute_force_loops():
    rng = np.random.default_rng(1)
    hidden, vocab = 8, 11
    x = round_to(rng.standard_normal((5, hidden)).astype(np.float32), "bf16")
    w = (1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    emb = round_to(rng.standard_normal((vocab, hidden)).astype(np.float32), "bf16")
    idx = np.array([4, 0, 2])
    ids, rounded, _ = lg.final_norm_logits_argmax(x, idx, w, emb, 1e-6)
    for j, r in enumerate(idx):
        row = [float(v) for v in x[r]]
        ms = sum(v * v for v in row) / hidden
        inv = 1.0 / (ms + 1e-6) ** 0.5
        normed = [float(round_to(np.float32(v * inv * float(w[k])), "bf16")) for k, v in enumerate(row)]
        best, best_v = None, None
        for v in range(vocab):
            s = sum(normed[k] * float(emb[v, k]) for k in range(hidden))
            s = float(round_to(np.float32(s), "bf16"))
            assert s == rounded[j, v]
            if best is None or s > best_v:  # strict: the first maximal index stays
                best, best_v = v, s
        assert ids[j] == best


def test_planted_winner_and_ties():
    rng = np.random.default_rng(2)
    hidden, vocab = 128, 500
    x = round_to(rng.standard_normal((3, hidden)).astype(np.float32), "bf16")
    w = np.ones(hidden, np.float32)
    emb = round_to(0.01 * rng.standard_normal((vocab, hidden)).astype(np.float32), "bf16")
    normed = lg.final_norm(x, np.arange(3), w, 1e-6)
    # Row 0: the normalised row itself as vocab entry 321 dominates every other logit.
    emb[321] = normed[0]
    # Row 1: entries 77 and 402 are equal and dominant: the first index wins.
    emb[77] = normed[1]
    emb[402] = normed[1]
    ids, rounded, _ = lg.final_norm_logits_argmax(x, np.arange(3), w, emb, 1e-6)
    assert ids[0] == 321
    assert ids[1] == 77 and rounded[1, 77] == rounded[1, 402]
    # torch.argmax breaks the same tie the same way.
    assert int(torch.from_numpy(rounded[1]).to(torch.bfloat16).argmax()) == 77


def test_norm_is_scale_invariant():
    rng = np.random.default_rng(3)
    x = round_to(rng.standard_normal((4, 256)).astype(np.float32), "bf16")
    w = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    a = lg.final_norm(x, np.arange(4), w, 0.0)
    b = lg.final_norm(x * 4.0, np.arange(4), w, 0.0)  # a power of two scales exactly
    np.testing.assert_array_equal(a, b)
    # A constant row normalises to sign * weight.
    c = lg.final_norm(np.full((1, 256), -2.5, np.float32), np.arange(1), w, 0.0)
    np.testing.assert_array_equal(c[0], round_to(-w, "bf16"))
