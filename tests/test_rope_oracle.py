"""The q/k norm + RoPE oracle: against the reference's op sequence in torch (CPU) and
against closed forms that a dropped term, a wrong sign or a swapped half would break."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dense_torch, rope


@pytest.mark.parametrize("seed", range(3))
def test_matches_reference_op_sequence(seed):
    g = torch.Generator().manual_seed(seed)
    rows, heads, d = 37, 5, 128
    x = torch.randn(rows, heads, d, generator=g).to(torch.bfloat16)
    w = (1 + 0.3 * torch.randn(d, generator=g)).float()
    cos, sin = dense_torch.rope_parameters(d, 4096, 1_000_000.0)
    pos = torch.randint(0, 4096, (rows,), generator=g)
    ref = dense_torch.apply_rope(dense_torch.rms_norm(x.transpose(0, 1).unsqueeze(0), w, 1e-6),
                                 cos, sin, pos.unsqueeze(0))[0].transpose(0, 1)
    got = rope.norm_rope(x.float().numpy(), w.numpy(), cos.numpy(), sin.numpy(), pos.numpy(), 1e-6)
    ref = ref.float().numpy()
    # 1/sqrt vs torch.rsqrt and the order of the sum of squares may differ by one fp32
    # ulp, which can move a bf16 rounding of a normalised element by one ulp; the
    # rotation carries that to both members of its pair. Bound: 2 bf16 ulps of the
    # pair norm.
    norm = np.sqrt(ref[..., :64] ** 2 + ref[..., 64:] ** 2)
    tol = 2 * 2.0 ** -7 * np.concatenate([norm, norm], axis=-1) + 1e-6
    assert np.all(np.abs(got - ref) <= tol)
    assert np.mean(got != ref) < 5e-3


def test_tables_match_reference():
    # Small angles only: for angles of thousands of radians, numpy's and torch's float32
    # cos/sin round differently (up to ~2e-4). The kernel takes the model's own tables,
    # so the tests pass the same table to both sides.
    cos, sin = rope.rope_tables(128, 64, 1_000_000.0)
    tc, ts = dense_torch.rope_parameters(128, 64, 1_000_000.0)
    np.testing.assert_allclose(cos, tc.numpy(), atol=1e-5)
    np.testing.assert_allclose(sin, ts.numpy(), atol=1e-5)


def test_closed_forms():
    rng = np.random.default_rng(0)
    d = 128
    cos, sin = rope.rope_tables(d, 64, 10_000.0)
    w = np.ones(d, np.float32)
    # Position 0 rotates by zero: the output is the normalised input.
    x = rope.round_to(rng.standard_normal((3, 2, d)).astype(np.float32), "bf16")
    out = rope.norm_rope(x, w, cos, sin, np.zeros(3, np.int64), 0.0)
    rms = np.sqrt(np.mean(x * x, axis=-1, keepdims=True))
    np.testing.assert_allclose(out, x / rms, rtol=1e-2, atol=1e-2)
    # A constant vector normalises to sign * weight.
    c = np.full((1, 1, d), -3.0, np.float32)
    np.testing.assert_array_equal(rope.norm_rope(c, w, cos, sin, np.zeros(1, np.int64), 0.0), -np.ones((1, 1, d)))
    # The rotation of pair (i, i + 64) at position p is by angle p * base^(-2i/d):
    # a unit vector on dim i comes out as (cos, sin) on (i, i + 64).
    e = np.zeros((1, 1, d), np.float32)
    e[0, 0, 5] = 1.0
    p = 17
    out = rope.norm_rope(e, w, cos, sin, np.array([p]), 0.0)[0, 0]
    ang = p * 10_000.0 ** (-2 * 5 / d)
    scale = np.sqrt(d)  # a one-hot vector has rms 1 / sqrt(d)
    assert abs(out[5] - scale * np.cos(ang)) < 0.05 * scale
    assert abs(out[5 + 64] - scale * np.sin(ang)) < 0.05 * scale
    assert np.count_nonzero(out) == 2
    # Rotation keeps each pair's norm.
    x = rope.round_to(rng.standard_normal((4, 3, d)).astype(np.float32), "bf16")
    n0 = rope.norm_rope(x, w, cos, sin, np.zeros(4, np.int64), 0.0)
    n1 = rope.norm_rope(x, w, cos, sin, np.array([1, 9, 33, 63]), 0.0)
    pair = lambda v: v[..., :64] ** 2 + v[..., 64:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(n1), pair(n0), rtol=3e-2, atol=3e-2)
