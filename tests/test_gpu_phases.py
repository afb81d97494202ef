"""Phased attention calls (``VarlenAttnPlan.run(phases=...)``).

* A call given the tick's new rows (``append=``) writes them into the pool whichever
  phases it launches: the decode kernel's own workgroups, workgroups added to the decode
  launch, or the append kernel when the call launches no work that writes them (a
  decode-phase call on a chunk-only tick, a combine-only call). Checked bit for bit
  against the rows given.
* On shapes the generic kernel serves, ``run_overlapped`` gives the bits of ``run``.
"""

from __future__ import annotations

import pytest
import torch

from helios_amd import ops, synth
from tests.gpu_cases import DeviceTick, say

pytestmark = pytest.mark.gpu


def _chunk_only() -> synth.Workload:
    """One sequence prefilling 300 rows after 100 cached keys (two pages)."""
    return synth.Workload("chunk only", [300], [100], [[5, 2]], 8, seed=61)


def _decode_only() -> synth.Workload:
    return synth.c2(seed=62, batch=8, num_pages=128)


CASES = {
    "chunk-only tick": _chunk_only,
    "decode-only tick": _decode_only,
    "mixed tick": lambda: synth.small_mixed(63, batch=6),
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("phases", [("decode",), ("chunk",), ("combine",), ("decode", "chunk", "combine")])
def test_append_is_written_by_every_phase_set(device, name, phases):
    w = CASES[name]()
    tick = DeviceTick(w, torch.bfloat16, device)
    say(f"append with phases {phases}: {name}, rows {w.total_q}")
    plan = tick.plan()
    k_pool, v_pool = tick.fresh_pools()
    plan.run(tick.q, k_pool, v_pool, tick.block_table, phases=phases,
             append=(tick.k_new, tick.v_new, tick.write_slots))
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    flat = lambda p: p.view(-1, w.n_kv_heads, w.head_dim)  # noqa: E731
    slots = tick.write_slots
    assert torch.equal(flat(k_pool).index_select(0, slots), tick.k_new), (name, phases)
    assert torch.equal(flat(v_pool).index_select(0, slots), tick.v_new), (name, phases)


def test_generic_shape_overlapped_matches_run(device):
    """head_dim 64 (generic kernel), decode rows and chunks on two streams."""
    w = synth.small_mixed(64, n_q_heads=8, n_kv_heads=2, head_dim=64, batch=6)
    assert 1 in w.q_lens and max(w.q_lens) > 1
    tick = DeviceTick(w, torch.bfloat16, device)
    plan = tick.plan()
    assert not plan.tuned
    ref = plan.run(tick.q, tick.k_pool, tick.v_pool, tick.block_table)
    side = torch.cuda.Stream(device=device)
    got = ops.run_overlapped(plan, tick.q, tick.k_pool, tick.v_pool, tick.block_table, side)
    torch.cuda.synchronize()
    assert plan.error_word() == 0
    assert torch.equal(got, ref)


def test_stream_handle_is_the_current_stream(device):
    """Launches go to torch's current stream: the raw handle lookup agrees with
    ``torch.cuda.current_stream`` on the default stream, under ``torch.cuda.stream`` and
    for a device given without an index."""
    side = torch.cuda.Stream(device=device)
    assert ops._stream_ptr(device) == torch.cuda.current_stream(device).cuda_stream
    with torch.cuda.stream(side):
        assert ops._stream_ptr(device) == side.cuda_stream
        assert ops._stream_ptr(torch.device("cuda")) == side.cuda_stream
    assert ops._stream_ptr(device) == torch.cuda.current_stream(device).cuda_stream
