"""The device work plan, entry by entry, against the Python model of the planner.

plan_kernel lists a tick's chunk row blocks in LDS and runs the split-size search and the
item, partial-slot and combine-record offsets as passes over that list (the search
evaluates every candidate in one pass when they are few, else bisects). Past 1024 chunk
sequences or 4096 row blocks it walks each sequence's blocks serially instead. Both paths
must write exactly the lists of tests/plan_model.py: sequence info, decode items, chunk
items, their first partial rows, and combine records, with the header counts.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops, synth
from tests import plan_model
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


def _device_lists(q_lens, k_lens, hq, hkv, window=(-1, 0), page_size=256, device=None):
    batch = len(q_lens)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    max_q, max_k = max(q_lens), max(k_lens)
    stride = max(1, -(-max_k // 256))
    plan = ops.VarlenAttnPlan(
        torch.from_numpy(cu_q).to(device), torch.from_numpy(cu_k).to(device),
        torch.tensor(k_lens, dtype=torch.int32, device=device),
        total_q=int(cu_q[-1]), max_q=max_q, max_k=max_k, n_q_heads=hq, n_kv_heads=hkv, head_dim=128,
        page_size=page_size, block_table_stride=stride, total_k_rows=int(cu_k[-1]), window=window,
        q_lens=q_lens, k_lens=k_lens)
    torch.cuda.synchronize()
    ws = plan.workspace[plan._ws_offset:plan._ws_offset + plan.ws_bytes].cpu().numpy()
    lay = plan_model.layout(batch, max_q, max_k, hq, hkv)
    hdr = ws[:256].view(np.int32)
    n_dec, n_pf, n_comb, err = (int(x) for x in hdr[:4])
    words = lambda off, n: ws[off:off + 4 * n].view(np.int32)  # noqa: E731
    got = (
        words(lay["seq_info"], 4 * batch).reshape(-1, 4),
        words(lay["dec_items"], 4 * n_dec).reshape(-1, 4),
        words(lay["pf_items"], 4 * n_pf).reshape(-1, 4),
        words(lay["pf_base"], n_pf),
        words(lay["comb_seqs"], 4 * n_comb).reshape(-1, 4),
    )
    # Each chunk item carries a copy of its sequence's seq_info entry.
    pf_seq = words(lay["pf_seq"], 4 * n_pf).reshape(-1, 4)
    assert np.array_equal(pf_seq, got[0][got[2][:, 0]]) if n_pf else True
    want = plan_model.plan_lists(q_lens, k_lens, hq, hkv, window, lay["max_dec"], lay["cslot_cap"], page_size,
                                 cu_k=cu_k)
    return got, want, err, plan.hints


def _check(name, q_lens, k_lens, hq=32, hkv=8, window=(-1, 0), device=None):
    got, want, err, hints = _device_lists(q_lens, k_lens, hq, hkv, window, device=device)
    say(name, "items", [len(x) for x in got])
    assert err == 0
    assert (len(got[1]), len(got[2]), len(got[4])) == tuple(hints)
    for what, g, w in zip(("seq_info", "decode items", "chunk items", "partial bases", "combine records"),
                          got, want):
        assert g.shape == w.shape, (name, what, g.shape, w.shape)
        mism = np.flatnonzero((g != w).reshape(len(g), -1).any(axis=1)) if len(g) else []
        assert len(mism) == 0, (name, what, mism[:5], g[mism[:3]], w[mism[:3]])


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4"])
def test_plan_lists_of_bench_workloads(device, name):
    w = getattr(synth, name)()
    _check(name, w.q_lens, w.k_lens, device=device)


def test_plan_lists_of_the_full_tick(device):
    cached, counts = synth.c5_lengths(5)
    _check("c5", counts, [c + n for c, n in zip(cached, counts)], device=device)


@pytest.mark.parametrize("hq,hkv,window", [(8, 8, (-1, 0)), (16, 2, (300, 0)), (32, 8, (700, 64)),
                                           (32, 16, (-1, -1))])
def test_plan_lists_groups_and_windows(device, hq, hkv, window):
    for seed in range(3):
        w = synth.small_mixed(40 + seed, n_q_heads=hq, n_kv_heads=hkv, batch=9, max_cached=3000,
                              max_chunk=900, num_pages=200)
        _check(f"mixed {seed} G={hq // hkv} {window}", w.q_lens, w.k_lens, hq, hkv, window, device=device)


def test_plan_lists_long_chunk_binary_search(device):
    """A chunk at 140000 keys: over 1024 candidate split sizes, so the split size comes
    from the binary search rather than the one-pass evaluation of every candidate."""
    _check("long chunk", [128, 1, 1, 300], [140000, 5000, 300, 9000], device=device)


def test_plan_lists_at_the_block_list_capacity(device):
    """4096 row blocks: the largest tick the block list holds."""
    q_lens = [4096] * 64 + [1] * 3
    k_lens = [4096] * 64 + [300, 5000, 9000]
    _check("4096 blocks", q_lens, k_lens, device=device)


def test_plan_lists_past_the_list_capacities(device):
    """Past 1024 chunk sequences, and past 4096 row blocks, the serial walk runs."""
    rng = np.random.default_rng(7)
    q_lens = [2] * 1030 + [1] * 20
    k_lens = [int(x) for x in rng.integers(2, 3000, 1030)] + [int(x) for x in rng.integers(1, 9000, 20)]
    _check("1030 chunk sequences", q_lens, k_lens, device=device)
    q_lens = [4160] * 64 + [1] * 3
    k_lens = [4160] * 64 + [300, 5000, 9000]
    _check("4160 blocks", q_lens, k_lens, device=device)
