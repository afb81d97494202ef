"""Randomized mixed ticks against the float64 oracle.

Each case draws, from its seed, the shapes the kernels branch on:
- the group size: 1, 2, 4 or 8 (tuned at head_dim 128), or 3 (the generic kernel);
- head_dim: 128, or 64 / 96 (the generic kernel);
- dtype (bf16 or fp16), page size (256 or 512) and the attention window;
- the tick's mix: decode rows, short and long chunks, rows crossing page boundaries.

Every output row is compared with the oracle at the dtype's bound. The fused append +
attention call must also leave the pools and the output with the bits of a separate
append followed by attention.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import synth
from tests.gpu_cases import DeviceTick, compare, say

pytestmark = pytest.mark.gpu

CASES = 64
WINDOWS = [(-1, 0), (-1, 0), (-1, 0), (200, 0), (700, 0), (-1, 64), (300, 100)]


def _draw(seed: int):
    rng = np.random.default_rng(1000 + seed)
    g = int(rng.choice([1, 2, 4, 8, 4, 3]))
    hkv = int(rng.choice([1, 2, 4, 8])) if g != 8 else int(rng.choice([1, 2, 4]))
    head_dim = int(rng.choice([128, 128, 128, 64, 96]))
    dtype = torch.float16 if rng.random() < 0.35 else torch.bfloat16
    page_size = int(rng.choice([256, 256, 512]))
    window = WINDOWS[int(rng.integers(len(WINDOWS)))]
    batch = int(rng.integers(1, 10))
    max_cached = int(rng.choice([100, 700, 2000]))
    max_chunk = int(rng.choice([2, 40, 300]))
    need = batch * (-(-(max_cached + max_chunk) // page_size) + 1)
    w = synth.small_mixed(2000 + seed, n_q_heads=g * hkv, n_kv_heads=hkv, batch=batch, max_cached=max_cached,
                          max_chunk=max_chunk, num_pages=need + 4, page_size=page_size, head_dim=head_dim)
    return w, dtype, window


@pytest.mark.parametrize("seed", range(CASES))
def test_random_tick_matches_oracle(device, seed):
    w, dtype, window = _draw(seed)
    say(f"random tick {seed}: G={w.n_q_heads // w.n_kv_heads} hkv={w.n_kv_heads} d={w.head_dim} {dtype} "
        f"page={w.page_size} window={window} q_lens={w.q_lens} k_lens={w.k_lens}")
    tick = DeviceTick(w, dtype, device, pool_on_device=True)
    out = tick.attend(window=window, exact_grid=seed % 2 == 0)
    ref, _ = tick.oracle(window=window)
    compare(out, ref, what=f"random tick {seed}")
    # fused append + attention from the pools before the append
    k_pool, v_pool = tick.fresh_pools()
    plan = tick.plan(window=window)
    fused = plan.run(tick.q, k_pool, v_pool, tick.block_table, append=(tick.k_new, tick.v_new, tick.write_slots))
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    assert torch.equal(k_pool.view(torch.int16), tick.k_pool.view(torch.int16))
    assert torch.equal(v_pool.view(torch.int16), tick.v_pool.view(torch.int16))
    expect = plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table)
    assert torch.equal(fused.view(torch.int16), expect.view(torch.int16))
