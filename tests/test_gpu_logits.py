"""Final RMSNorm + lm_head + greedy argmax on the GPU, through the C ABI: against the
numpy oracle on small vocabularies, and against the reference's op sequence in torch
(fp32 logits on the same GPU) at the Qwen3-4B shape (hidden 2560, vocab 151936)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops
from oracle import dense_torch, logits as lg
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu

BF16_ULP = 2.0 ** -7
FP16_ULP = 2.0 ** -10


def _inputs(device, rows, hidden, vocab, picks, dtype=torch.bfloat16, seed=0, std=0.05):
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(rows, hidden, generator=g, device=device).to(dtype)
    w = (1 + 0.2 * torch.randn(hidden, generator=g, device=device)).float()
    emb = (std * torch.randn(vocab, hidden, generator=g, device=device)).to(dtype)
    idx = torch.randperm(rows, generator=g, device=device)[:picks]
    return x, w, emb, idx


def _check_picks(ids, maxl, exact, ulp, what):
    """ids must pick a logit within rounding of the exact maximum; where the top two are
    further apart than that, the pick is the oracle's exactly."""
    ids = np.asarray(ids)
    rows = np.arange(exact.shape[0])
    top = exact.max(axis=-1)
    tol = 4 * ulp * np.abs(top) + 1e-5
    assert np.all(ids >= 0), what
    assert np.all(exact[rows, ids] >= top - tol), (what, (top - exact[rows, ids]).max())
    assert np.all(np.abs(np.asarray(maxl) - top) <= tol), what
    top2 = np.sort(exact, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > tol
    np.testing.assert_array_equal(ids[clear], exact.argmax(axis=-1)[clear], err_msg=what)
    return int(clear.sum())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("picks", [1, 5, 16, 37, 160, 200])
def test_matches_oracle(device, dtype, picks):
    say("logits oracle", dtype, picks)
    rows, hidden, vocab = 240, 256, 1000
    x, w, emb, idx = _inputs(device, rows, hidden, vocab, picks, dtype, seed=picks)
    res = ops.final_norm_logits_argmax(x, idx, w, emb, 1e-6, return_logits=True)
    torch.cuda.synchronize()
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    ulp = BF16_ULP if dtype == torch.bfloat16 else FP16_ULP
    want_ids, want_rounded, exact = lg.final_norm_logits_argmax(
        x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), emb.float().cpu().numpy(), 1e-6, name)
    got = res.logits.float().cpu().numpy()
    # Each logit is rounded once (2 ulps for the fp32 vs float64 sums and the oracle's
    # double rounding); besides, an element of the normalised row may round one ulp the
    # other way (rsqrt and the sum of squares differ in the last fp32 bit), which moves
    # every logit of that row by at most ulp(max |row|) * max |embedding| per element.
    normed = lg.final_norm(x.float().cpu().numpy(), idx.cpu().numpy(), w.cpu().numpy(), 1e-6, name)
    flip = 2 * ulp * np.abs(normed).max(axis=1, keepdims=True) * float(emb.float().abs().max())
    bad = np.abs(got - want_rounded) > 2 * ulp * np.abs(want_rounded) + flip + 1e-6
    where = np.argwhere(bad)[:5]
    assert not bad.any(), (int(bad.sum()), [(int(r), int(c), float(got[r, c]), float(want_rounded[r, c]),
                                             float(exact[r, c])) for r, c in where])
    assert np.mean(got != want_rounded) < 2e-2
    clear = _check_picks(res.token_ids.cpu(), res.max_logits.cpu(), exact, ulp, name)
    assert clear >= picks // 2
    # The kernel's own logits and pick agree exactly (same rounded values, first index).
    np.testing.assert_array_equal(res.token_ids.cpu().numpy(), got.argmax(axis=-1))
    np.testing.assert_array_equal(res.max_logits.cpu().numpy(), got.max(axis=-1))


def test_ties_and_planted_winners(device):
    say("logits ties")
    rows, hidden, vocab = 8, 384, 777  # vocab tail: 777 = 6 x 128 + 9
    x, w, emb, idx = _inputs(device, rows, hidden, vocab, 4, seed=3, std=0.01)
    idx = torch.tensor([5, 2, 7, 0], device=device)
    normed = dense_torch.rms_norm(x[idx].unsqueeze(0), w, 1e-6)[0]
    emb[130] = normed[0]          # a winner in the second vocab tile
    emb[776] = normed[1]          # the last vocab row
    emb[3] = normed[2]            # an exact tie: the first index wins ...
    emb[600] = normed[2]          # ... over a later tile
    emb[400] = normed[3]
    emb[401] = normed[3]          # a tie inside one tile
    res = ops.final_norm_logits_argmax(x, idx, w, emb, 1e-6)
    torch.cuda.synchronize()
    assert res.token_ids.cpu().tolist() == [130, 776, 3, 400]
    ref = torch.nn.functional.linear(normed.float(), emb.float()).to(torch.bfloat16).argmax(dim=-1)
    assert ref.cpu().tolist() == [130, 776, 3, 400]


def test_bad_index_and_empty(device):
    say("logits bad index")
    x, w, emb, _ = _inputs(device, 10, 128, 300, 1, seed=4)
    idx = torch.tensor([3, 10, -1, 9], device=device)
    res = ops.final_norm_logits_argmax(x, idx, w, emb, 1e-6)
    torch.cuda.synchronize()
    ids = res.token_ids.cpu().tolist()
    assert ids[1] == -1 and ids[2] == -1 and ids[0] >= 0 and ids[3] >= 0
    assert torch.isnan(res.max_logits[1:3]).all()
    empty = ops.final_norm_logits_argmax(x, idx[:0], w, emb, 1e-6)
    assert empty.token_ids.numel() == 0
    with pytest.raises(ValueError):
        ops.final_norm_logits_argmax(x[:, :100].contiguous(), idx, w[:100].contiguous(), emb[:, :100].contiguous(), 1e-6)


@pytest.mark.parametrize("picks", [1, 129])
def test_qwen3_4b_shape_against_reference_sequence(device, picks):
    """The C5 tick's greedy heads: 2560 hidden, 151936 vocab, 129 logit rows."""
    say("logits qwen3-4b", picks)
    rows, hidden, vocab = 1152, 2560, 151936
    x, w, emb, _ = _inputs(device, rows, hidden, vocab, picks, seed=9, std=0.02)
    idx = torch.arange(rows - picks, rows, device=device)
    res = ops.final_norm_logits_argmax(x, idx, w, emb, 1e-6, return_logits=picks == 1)
    # model.py:108-110 on the same GPU, the logits in fp32 (exact enough to rank).
    normed = dense_torch.rms_norm(x.index_select(0, idx).unsqueeze(0), w, 1e-6)[0]
    exact = torch.nn.functional.linear(normed.float(), emb.float())
    ref_pick = exact.to(torch.bfloat16).argmax(dim=-1)
    torch.cuda.synchronize()
    exact_np = exact.double().cpu().numpy()
    clear = _check_picks(res.token_ids.cpu(), res.max_logits.cpu(), exact_np, BF16_ULP, "c5")
    assert clear >= picks // 2
    if picks > 1:  # torch's own bf16 rounding of the logits picks the same token nearly always
        same = (res.token_ids == ref_pick).float().mean().item()
        assert same >= 0.9, same
    if res.logits is not None:
        ref_l = exact.to(torch.bfloat16).float()
        diff = (res.logits.float() - ref_l).abs()
        assert (diff <= 2 * BF16_ULP * ref_l.abs() + 1e-5).all()
