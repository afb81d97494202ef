"""Runs whose packed query rows are read through a row map (``VarlenAttnPlan.run(...,
query_rows=...)``, ``hx_varlen_attn_run_rows``).

The shared-prefix cascade runs its prefix levels over member rows that repeat the tick's
decode rows, and reads them in place through such a map. The result must be the run on
the gathered queries, bit for bit, for decode rows, chunk rows and the generic kernel's
shapes; a map entry outside the query tensor raises its error-word bit and reads row 0.
"""

from __future__ import annotations

import pytest
import torch

from helios_amd import _capi, ops, synth
from tests.gpu_cases import DeviceTick, say

pytestmark = pytest.mark.gpu

CASES = {
    "mixed tick, tuned (32/8 heads, d=128)": lambda: synth.small_mixed(71, batch=6),
    "mixed tick, generic (8/2 heads, d=64)": lambda: synth.small_mixed(72, n_q_heads=8, n_kv_heads=2,
                                                                        head_dim=64, batch=5),
    "decode only": lambda: synth.c2(seed=73, batch=8, num_pages=128),
}


@pytest.mark.parametrize("name", list(CASES))
def test_row_map_equals_gathered_queries(device, name):
    w = CASES[name]()
    tick = DeviceTick(w, torch.bfloat16, device)
    say(f"query row map: {name}, rows {w.total_q}")
    g = torch.Generator(device="cpu").manual_seed(5)
    n_big = 3 * w.total_q + 7
    big = torch.randn((n_big, w.n_q_heads, w.head_dim), generator=g).to(torch.bfloat16).to(device)
    rows = torch.randint(0, n_big, (w.total_q,), generator=g)
    rows[: min(4, w.total_q)] = rows[0]  # repeated rows, as cascade members repeat
    rows = rows.to(device)
    plan = tick.plan()
    want, want_lse = plan.run(big.index_select(0, rows), tick.k_pool, tick.v_pool, tick.block_table,
                              return_lse=True)
    got, got_lse = plan.run(big, tick.k_pool, tick.v_pool, tick.block_table, return_lse=True,
                            query_rows=rows)
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    assert got.shape == want.shape == (w.total_q, w.n_q_heads, w.head_dim)
    assert torch.equal(got, want), name
    assert torch.equal(got_lse, want_lse), name


def test_row_map_entry_outside_the_queries_is_reported(device):
    w = synth.small_mixed(74, batch=4)
    tick = DeviceTick(w, torch.bfloat16, device)
    say("query row map: out-of-range entry")
    rows = torch.arange(w.total_q, dtype=torch.int64, device=device)
    rows[w.total_q - 1] = w.total_q + 100  # past the end of tick.q
    plan = tick.plan()
    plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table, query_rows=rows)
    torch.cuda.synchronize()
    assert plan.error_word() & _capi.HX_WERR_BAD_QUERY_ROW
    with pytest.raises(RuntimeError, match="query row map"):
        plan.check_errors()


def test_row_map_argument_checks(device):
    w = synth.small_mixed(75, batch=3)
    tick = DeviceTick(w, torch.bfloat16, device)
    plan = tick.plan()
    rows = torch.arange(w.total_q, dtype=torch.int64, device=device)
    with pytest.raises(ValueError, match="query_rows must be"):
        plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table, query_rows=rows.to(torch.int32))
    with pytest.raises(ValueError, match="query_rows must be"):
        plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table, query_rows=rows[:-1])
    with pytest.raises(ValueError, match="cannot be combined"):
        plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table, query_rows=rows,
                 append=(tick.k_new, tick.v_new, tick.write_slots))
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    assert ops.describe_error_word(_capi.HX_WERR_BAD_QUERY_ROW) == "a query row map entry outside the query tensor"
