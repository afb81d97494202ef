"""Split decode rows over repeated runs of one plan.

A decode row longer than 256 keys is split over several workgroups. Each writes a
partial (o / l, max, sum) to the plan's workspace, and the combine kernel merges the
row's partials in split order. Every run of the plan reuses the same partial slots.

One plan is run many times, alternating V and -V in the pool. Negating V keeps every
softmax weight and negates every product, so the output of a -V run is the exact
negation of a V run's output. The checks:
- every V run gives the bits of the first, and every -V run their negation;
- a partial left over from the previous run (a slot not rewritten, or read before it
  was) would mix signs or values in some row;
- the first run is checked against the float64 oracle on sampled rows.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import synth
from tests.gpu_cases import DeviceTick, compare, say

pytestmark = pytest.mark.gpu

RUNS = 16


def _decoders(seed: int, hq: int, hkv: int, batch: int, lo: int, hi: int) -> synth.Workload:
    """A decode-only tick with contexts uniform in [lo, hi] (several splits per row)."""
    rng = np.random.default_rng(seed)
    cached = [int(x) for x in rng.integers(lo, hi + 1, batch)]
    pages = [-(-(c + 1) // 256) for c in cached]
    perm = [int(p) for p in rng.permutation(sum(pages) + 8)]
    tables, i = [], 0
    for n in pages:
        tables.append(perm[i:i + n])
        i += n
    return synth.Workload(f"decoders G={hq // hkv}", [1] * batch, cached, tables, sum(pages) + 8,
                          n_q_heads=hq, n_kv_heads=hkv, seed=seed)


CASES = {
    "c2 bf16": (synth.c2, torch.bfloat16, (-1, 0)),
    "c2 fp16, window 1000": (synth.c2, torch.float16, (1000, 0)),
    "G=8 bf16": (lambda: _decoders(31, 64, 8, 24, 300, 9000), torch.bfloat16, (-1, 0)),
    "G=1 bf16": (lambda: _decoders(32, 8, 8, 40, 300, 5000), torch.bfloat16, (-1, 0)),
    "G=2 fp16": (lambda: _decoders(33, 16, 8, 40, 300, 5000), torch.float16, (-1, 0)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_repeated_runs_merge_split_rows_exactly(device, name):
    make, dtype, window = CASES[name]
    w = make()
    say(f"split merge {name}: batch={w.batch} max_k={w.max_k} runs={RUNS}")
    tick = DeviceTick(w, dtype, device, pool_on_device=True)
    plan = tick.plan(window=window)
    v_neg = -tick.v_pool
    first = plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table)
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    sample = list(range(0, w.batch, max(1, w.batch // 12)))
    ref, _ = tick.oracle(window=window, rows={b: [0] for b in sample})
    compare(first, ref, what=f"split merge {name}", rows=np.array(sample))
    # Compared as values (an output that cancels to +0 stays +0 under -V); every other
    # value must match bit for bit.
    want_neg = -first
    out = torch.empty_like(first)
    for i in range(RUNS):
        neg = i % 2 == 0
        plan.run(tick.q, tick.k_pool, v_neg if neg else tick.v_pool, tick.block_table, out=out)
        bad = (out != (want_neg if neg else first)).any(dim=2).any(dim=1)
        assert not bool(bad.any()), (name, i, "rows differ", torch.nonzero(bad).flatten()[:8].tolist())
    assert plan.error_word() == 0
