"""Split decode rows and split chunk blocks over repeated runs of one plan.

A decode row longer than 256 keys is split over several workgroups, and so is a chunk
row block whose key tiles are split. Each split writes a partial (o / l, max, sum) to the
plan's workspace, and the combine kernel merges each row's partials in split order.
Every run of the plan reuses the same partial slots.

One plan is run many times, alternating V and c * V in the pool. Scaling V keeps every
softmax weight and scales every product, so a c * V run's output is c times a V run's
output up to rounding: the decode kernel's packed dot2 products (P V) and the chunk
kernel's MFMA accumulations are not exactly odd in V (a dot2 result negates exactly in
about 99 % of random cases), so c = -1 holds to within an ulp of the output, and c = 2
exactly only where no output is subnormal (chunk cases run in bf16). The checks:
- every V run gives the bits of the first V run, and every c * V run the bits of the
  first c * V run (the launches are deterministic);
- the first c * V run is c times the first V run to within two ulps of the output type
  at the row's largest magnitude (a split partial is stored in the output type, so one
  partial's rounding reaches the merged row at the partial's scale); a partial left over
  from the previous run (a slot not rewritten, or read before it was) would mix values of
  the other sign into some row, an error of the size of the values themselves;
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


def _mixed(seed: int, decoders: int, chunk: int, cached: int) -> synth.Workload:
    """Decode rows of 1000-3000 keys plus one chunk of ``chunk`` rows after ``cached``
    cached keys, whose row blocks the plan splits over key tiles."""
    rng = np.random.default_rng(seed)
    done = [int(x) for x in rng.integers(1000, 3001, decoders)] + [cached]
    q_lens = [1] * decoders + [chunk]
    pages = [-(-(c + n) // 256) for c, n in zip(done, q_lens)]
    perm = [int(p) for p in rng.permutation(sum(pages) + 8)]
    tables, i = [], 0
    for n in pages:
        tables.append(perm[i:i + n])
        i += n
    return synth.Workload("mixed split chunk", q_lens, done, tables, sum(pages) + 8, seed=seed)


# name: (workload, dtype, window, scale c of the alternate runs)
CASES = {
    "c2 bf16": (synth.c2, torch.bfloat16, (-1, 0), -1.0),
    "c2 fp16, window 1000": (synth.c2, torch.float16, (1000, 0), -1.0),
    "G=8 bf16": (lambda: _decoders(31, 64, 8, 24, 300, 9000), torch.bfloat16, (-1, 0), -1.0),
    "G=1 bf16": (lambda: _decoders(32, 8, 8, 40, 300, 5000), torch.bfloat16, (-1, 0), -1.0),
    "G=2 fp16": (lambda: _decoders(33, 16, 8, 40, 300, 5000), torch.float16, (-1, 0), -1.0),
    "c3 bf16 (split chunk blocks)": (synth.c3, torch.bfloat16, (-1, 0), 2.0),
    "1024-row chunk after 4096 keys": (lambda: _mixed(34, 8, 1024, 4096), torch.bfloat16, (-1, 0), 2.0),
}


@pytest.mark.parametrize("name", list(CASES))
def test_repeated_runs_merge_split_rows_exactly(device, name):
    make, dtype, window, scale = CASES[name]
    w = make()
    say(f"split merge {name}: batch={w.batch} max_k={w.max_k} runs={RUNS}")
    tick = DeviceTick(w, dtype, device, pool_on_device=True)
    plan = tick.plan(window=window)
    v_alt = tick.v_pool * scale
    first = plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table)
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    sample = list(range(0, w.batch, max(1, w.batch // 12)))
    rows = {b: [0] for b in sample}
    for b, n in enumerate(w.q_lens):  # chunk rows: the first, middle and last of each
        if n > 1:
            rows[b] = sorted({0, 63, 64, n // 2, n - 1})
    ref, _ = tick.oracle(window=window, rows=rows)
    flat = [w.cu_seq_q[b] + r for b, rs in sorted(rows.items()) for r in rs]
    compare(first, ref, what=f"split merge {name}", rows=np.array(flat))
    # The first c * V run: c times the first V run to within two ulps of the output type
    # at each (row, head)'s largest magnitude.
    first_alt = plan.run(tick.q, tick.k_pool, v_alt, tick.block_table)
    ulp = 2.0 ** (-7 if dtype == torch.bfloat16 else -10)
    want = first.float() * scale
    err = (first_alt.float() - want).abs()
    bound = 2 * ulp * want.abs().amax(dim=2, keepdim=True) + 1e-6
    bad = (err > bound).any(dim=2).any(dim=1)
    assert not bool(bad.any()), (name, "scaled run", torch.nonzero(bad).flatten()[:8].tolist(),
                                 float(err.max()))
    # Later runs, alternating: each repeats its first run's bits. Compared as values (an
    # output that cancels to +0 may come out as -0 in another run).
    out = torch.empty_like(first)
    for i in range(RUNS):
        alt = i % 2 == 0
        plan.run(tick.q, tick.k_pool, v_alt if alt else tick.v_pool, tick.block_table, out=out)
        bad = (out != (first_alt if alt else first)).any(dim=2).any(dim=1)
        assert not bool(bad.any()), (name, i, "rows differ", torch.nonzero(bad).flatten()[:8].tolist())
    assert plan.error_word() == 0
