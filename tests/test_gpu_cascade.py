"""Shared-prefix cascade on the GPU: decode rows that share restored prefix pages attend to
them once per group; outputs match the float64 oracle and the non-cascade path."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedBatchCache, PagedKVCache, _PrefixCascade
from oracle import attention
from tests.gpu_cases import say, tolerance

pytestmark = pytest.mark.gpu


def _pool(device, pages=96, seed=3, dtype=torch.bfloat16, n_heads=32, n_kv_heads=8):
    config = Qwen3Config(context_length=8192, n_layers=2, dtype=dtype, n_heads=n_heads, n_kv_heads=n_kv_heads)
    pool = KVPagePool(config, pages, device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    for t in pool.keys + pool.values:
        t.normal_(generator=g)
    return pool


def _shared_caches(pool, cached, prefix_pages=8):
    """A prefix of `prefix_pages` full pages, then requests that restore min(prefix,
    their full pages) of it (shared page objects) and own the rest."""
    prefix = PagedKVCache(pool, 8192)
    prefix.pages.extend(pool.acquire(prefix_pages))
    prefix.length = prefix_pages * 256
    caches = []
    for n in cached:
        cache = PagedKVCache(pool, 8192)
        shared = min(prefix_pages, n // 256)
        cache.pages.extend(prefix.pages[:shared])
        cache.pages.extend(pool.acquire(-(-n // 256) - shared))
        cache.length = n
        caches.append(cache)
    return prefix, caches


def _oracle(pool, caches, counts, q, layer=0):
    k = pool.keys[layer].float().cpu().numpy()
    v = pool.values[layer].float().cpu().numpy()
    tables = [[p.index for p in c.pages] for c in caches]
    ends = [c.length + n for c, n in zip(caches, counts)]
    cu = np.concatenate([[0], np.cumsum(counts)])
    out, _ = attention.paged_varlen_attention(q.float().cpu().numpy(), k, v, cu, ends, tables,
                                              scale=1 / np.sqrt(128))
    return out


def _compare(got, want, what, dtype=torch.bfloat16):
    max_abs, mean_abs = tolerance(dtype)
    err = np.abs(got - want)
    say(what, f"max_abs={err.max():.3e} mean_abs={err.mean():.3e}")
    assert err.max() <= max_abs and err.mean() <= mean_abs, (what, err.max(), err.mean())


@pytest.fixture
def always_cascade(monkeypatch):
    """Levels cost nothing, so every shared page range with two rows becomes a level."""
    monkeypatch.setattr(_PrefixCascade, "US_PER_LEVEL", 0.0)
    monkeypatch.setattr(_PrefixCascade, "US_PER_BLOCK_PAGE", 0.0)


def test_levels_follow_shared_pages(device, always_cascade):
    say("cascade levels")
    pool = _pool(device)
    _, caches = _shared_caches(pool, [300, 2100, 700, 2100, 1600, 40, 999])
    batch = PagedBatchCache(caches)
    levels = _PrefixCascade.levels(batch, [1] * len(caches))
    # shared full pages: 300 -> 1, 2100 -> 8, 700 -> 2, 2100 -> 8, 1600 -> 6, 40 -> 0, 999 -> 3;
    # free levels: one per distinct count, up to three, the deepest covering rows 1 and 3
    assert len(levels) <= _PrefixCascade.MAX_LEVELS
    prev = 0
    for ref, first, end, rows in levels:
        assert first == prev and end > first and len(rows) >= 2 and 5 not in rows
        prev = end
    assert levels[-1][2] == 8 and levels[-1][3] == [1, 3]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("counts_kind", ["decode", "mixed"])
def test_cascade_matches_oracle_and_plain_path(device, counts_kind, dtype, always_cascade):
    say("cascade", counts_kind, dtype)
    cached = [2100, 2300, 300, 2100, 1700, 520, 2048, 900, 2800]
    counts = [1] * len(cached)
    if counts_kind == "mixed":
        counts[2] = 130  # a chunk row block next to the decode rows
    outs = []
    for cascade in (True, False):
        pool = _pool(device, dtype=dtype)
        _, caches = _shared_caches(pool, cached)
        batch = PackedBatchCache(caches, prefix_cascade=cascade)
        batch.prepare_packed(counts)
        assert (batch._cascade is not None) == cascade
        total = sum(counts)
        g = torch.Generator(device=device).manual_seed(11)
        q = torch.randn((1, 32, total, 128), generator=g, device=device).to(dtype)
        k = torch.randn((1, 8, total, 128), generator=g, device=device).to(dtype)
        v = torch.randn((1, 8, total, 128), generator=g, device=device).to(dtype)
        out = batch.attend(0, q, k, v)
        torch.cuda.synchronize()
        want = _oracle(pool, caches, counts, q[0].transpose(0, 1))
        got = out[0].transpose(0, 1).float().cpu().numpy()
        _compare(got, want, f"cascade={cascade} {dtype}", dtype)
        outs.append(got)
        batch.advance_packed()
    _compare(outs[0], outs[1], "cascade vs plain", dtype)


@pytest.mark.parametrize("n_heads,n_kv_heads", [(64, 8), (16, 8)])
def test_cascade_other_group_sizes(device, n_heads, n_kv_heads, always_cascade):
    """G = 8 (the level batch runs two head quads per KV head) and G = 2."""
    say("cascade group", n_heads, n_kv_heads)
    cached = [2100, 2300, 300, 2100, 1700, 520]
    counts = [1, 1, 90, 1, 1, 1]
    pool = _pool(device, n_heads=n_heads, n_kv_heads=n_kv_heads)
    _, caches = _shared_caches(pool, cached)
    batch = PackedBatchCache(caches, prefix_cascade=True)
    batch.prepare_packed(counts)
    assert batch._cascade is not None
    total = sum(counts)
    g = torch.Generator(device=device).manual_seed(12)
    q = torch.randn((1, n_heads, total, 128), generator=g, device=device).to(torch.bfloat16)
    k = torch.randn((1, n_kv_heads, total, 128), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((1, n_kv_heads, total, 128), generator=g, device=device).to(torch.bfloat16)
    out = batch.attend(0, q, k, v)
    torch.cuda.synchronize()
    want = _oracle(pool, caches, counts, q[0].transpose(0, 1))
    _compare(out[0].transpose(0, 1).float().cpu().numpy(), want, f"cascade G={n_heads // n_kv_heads}")


def test_uniform_decode_cascade_over_ticks(device, always_cascade):
    say("cascade uniform ticks")
    pool = _pool(device)
    _, caches = _shared_caches(pool, [2047, 2100, 600, 2300])
    batch = PagedBatchCache(caches)
    for tick in range(3):
        batch.prepare(1)
        assert batch._cascade is not None
        g = torch.Generator(device=device).manual_seed(tick)
        q = torch.randn((4, 32, 1, 128), generator=g, device=device).to(torch.bfloat16)
        k = torch.randn((4, 8, 1, 128), generator=g, device=device).to(torch.bfloat16)
        v = torch.randn((4, 8, 1, 128), generator=g, device=device).to(torch.bfloat16)
        out = batch.attend(1, q, k, v)
        torch.cuda.synchronize()
        want = _oracle(pool, caches, [1] * 4, q[:, :, 0], layer=1)
        _compare(out[:, :, 0].float().cpu().numpy(), want, f"tick {tick}")
        batch.advance(1)


def test_attn_merge_matches_joint_softmax(device):
    say("attn merge")
    g = torch.Generator(device="cpu").manual_seed(0)
    rows, heads, d, ka, kb = 5, 4, 128, 37, 53
    q = torch.randn(rows, heads, d, generator=g)
    keys = torch.randn(ka + kb, heads, d, generator=g)
    vals = torch.randn(ka + kb, heads, d, generator=g)

    def part(lo, hi):
        s = torch.einsum("rhd,khd->rhk", q, keys[lo:hi]) / np.sqrt(d)
        lse = torch.logsumexp(s, dim=-1)
        o = torch.einsum("rhk,khd->rhd", torch.softmax(s, dim=-1), vals[lo:hi])
        return o, lse

    o_a, lse_a = part(0, ka)
    o_b, lse_b = part(ka, ka + kb)
    o_all, lse_all = part(0, ka + kb)
    total = rows + 3  # o_b rows sit among others at rows 3..7
    out = torch.zeros(total, heads, d)
    out[3:] = o_b
    lse_out = torch.full((heads, total), -float("inf"))
    lse_out[:, 3:] = lse_b.t()
    out_d = out.to(torch.bfloat16).to(device)
    lse_d = lse_out.to(device).contiguous()
    ops.attn_merge(out_d, lse_d, o_a.to(torch.bfloat16).to(device), lse_a.t().contiguous().to(device),
                   torch.arange(3, total, device=device))
    torch.cuda.synchronize()
    torch.testing.assert_close(out_d[3:].float().cpu(), o_all, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(lse_d[:, 3:].cpu(), lse_all.t(), atol=1e-4, rtol=1e-4)
    assert not out_d[:3].float().any()


def test_attn_merge_folds_several_parts(device):
    say("attn merge parts")
    g = torch.Generator(device="cpu").manual_seed(1)
    heads, d = 4, 128
    sizes = [29, 41, 17, 23]  # key sets of the batch-B result and three levels
    rows = 6
    q = torch.randn(rows, heads, d, generator=g)
    keys = torch.randn(sum(sizes), heads, d, generator=g)
    vals = torch.randn(sum(sizes), heads, d, generator=g)
    edges = [0, *torch.cumsum(torch.tensor(sizes), 0).tolist()]

    def part(lo, hi, r):
        s = torch.einsum("hd,khd->hk", q[r], keys[lo:hi]) / np.sqrt(d)
        return torch.einsum("hk,khd->hd", torch.softmax(s, dim=-1), vals[lo:hi]), torch.logsumexp(s, dim=-1)

    # rows 1, 3, 4 are merged; row 1 has parts of levels 1 and 2, row 3 of levels 1-3,
    # row 4 of level 3 only; the o_a rows are grouped by level as the cascade lays them out
    members = {1: [1, 2], 3: [1, 2, 3], 4: [3]}
    level_rows = {lv: [r for r in sorted(members) if lv in members[r]] for lv in (1, 2, 3)}
    o_a, lse_a, where = [], [], {}
    for lv in (1, 2, 3):
        for r in level_rows[lv]:
            o, lse = part(edges[lv], edges[lv + 1], r)
            where[(r, lv)] = len(o_a)
            o_a.append(o)
            lse_a.append(lse)
    out = torch.zeros(rows, heads, d)
    lse_out = torch.full((heads, rows), -float("inf"))
    want = torch.zeros(rows, heads, d)
    for r in range(rows):
        o, lse = part(edges[0], edges[1], r)
        out[r], lse_out[:, r] = o, lse
        keep = [0] + members.get(r, [])
        idx = torch.cat([torch.arange(edges[k], edges[k + 1]) for k in keep])
        s = torch.einsum("hd,khd->hk", q[r], keys[idx]) / np.sqrt(d)
        want[r] = torch.einsum("hk,khd->hd", torch.softmax(s, dim=-1), vals[idx])
    out_rows = sorted(members)
    part_start = [0]
    part_idx = []
    for r in out_rows:
        part_idx += [where[(r, lv)] for lv in members[r]]
        part_start.append(len(part_idx))
    out_d = out.to(torch.bfloat16).to(device)
    lse_d = lse_out.contiguous().to(device)
    ops.attn_merge(out_d, lse_d, torch.stack(o_a).to(torch.bfloat16).to(device),
                   torch.stack(lse_a).t().contiguous().to(device),
                   torch.tensor(out_rows, device=device),
                   parts=(torch.tensor(part_start, dtype=torch.int32, device=device),
                          torch.tensor(part_idx, dtype=torch.int32, device=device)))
    torch.cuda.synchronize()
    torch.testing.assert_close(out_d.float().cpu(), want, atol=2e-2, rtol=2e-2)
    # untouched rows keep their batch-B result bit for bit
    for r in (0, 2, 5):
        assert torch.equal(out_d[r].cpu(), out[r].to(torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attn_merge_vector_and_scalar_paths_agree(device, dtype):
    """The 16-byte merge (16-byte aligned rows) and the 2-byte one (other strides) give the
    same bits, with up to 7 parts per row (more than one batch of four) and parts whose
    log-sum-exp is -inf."""
    say(f"attn merge paths {dtype}")
    g = torch.Generator(device="cpu").manual_seed(2)
    heads, d, rows, n_a = 4, 128, 5, 16
    out = torch.randn(rows, heads, d, generator=g)
    lse_out = torch.randn(heads, rows, generator=g)
    lse_out[:, 4] = -float("inf")
    o_a = torch.randn(n_a, heads, d, generator=g)
    lse_a = torch.randn(heads, n_a, generator=g) * 3
    lse_a[:, 5] = -float("inf")
    members = {0: [0, 1, 2, 3, 4, 5, 6], 2: [7, 8], 3: [9], 4: [10, 5, 11, 12, 13]}
    out_rows = sorted(members)
    part_start, part_idx = [0], []
    for r in out_rows:
        part_idx += members[r]
        part_start.append(len(part_idx))
    parts = (torch.tensor(part_start, dtype=torch.int32, device=device),
             torch.tensor(part_idx, dtype=torch.int32, device=device))
    rows_d = torch.tensor(out_rows, device=device)
    a_d = o_a.to(dtype).to(device)
    la_d = lse_a.contiguous().to(device)

    def run(out_t):
        lse_t = lse_out.clone().contiguous().to(device)
        ops.attn_merge(out_t, lse_t, a_d, la_d, rows_d, parts=parts)
        return out_t, lse_t

    vec_out, vec_lse = run(out.to(dtype).to(device))
    wide = torch.zeros(rows, heads, d + 4, dtype=dtype, device=device)
    wide[:, :, :d] = out.to(dtype).to(device)
    sc_out, sc_lse = run(wide[:, :, :d])  # head stride 132: not 16-byte aligned
    assert sc_out.stride(1) % 8 != 0
    torch.cuda.synchronize()
    assert torch.equal(vec_out.cpu(), sc_out.cpu())
    assert torch.equal(vec_lse.cpu(), sc_lse.cpu())
    assert torch.equal(vec_out[1].cpu(), out[1].to(dtype))  # not a member: untouched


@pytest.mark.parametrize("cascade", [True, False])
def test_overlapped_streams_give_the_same_bits(device, cascade, always_cascade):
    """Chunk rows and the cascade's batch A on a second stream, decode rows on the
    current one: the same kernels on the same inputs, so the same bits."""
    say("overlap streams", cascade)
    cached = [2100, 2300, 300, 2100, 1700, 520, 2048, 900, 2800]
    counts = [1] * len(cached)
    counts[2], counts[7] = 130, 64
    outs = []
    for overlap in (True, False):
        pool = _pool(device)
        _, caches = _shared_caches(pool, cached)
        batch = PackedBatchCache(caches, prefix_cascade=cascade, overlap=overlap)
        batch.prepare_packed(counts)
        total = sum(counts)
        g = torch.Generator(device=device).manual_seed(21)
        for layer in range(2):
            q = torch.randn((1, 32, total, 128), generator=g, device=device).to(torch.bfloat16)
            k = torch.randn((1, 8, total, 128), generator=g, device=device).to(torch.bfloat16)
            v = torch.randn((1, 8, total, 128), generator=g, device=device).to(torch.bfloat16)
            outs.append(batch.attend(layer, q, k, v).clone())
        torch.cuda.synchronize()
        if overlap:
            want = _oracle(pool, caches, counts, q[0].transpose(0, 1), layer=1)
            _compare(outs[-1][0].transpose(0, 1).float().cpu().numpy(), want, "overlap")
        batch.advance_packed()
    assert torch.equal(outs[0], outs[2]) and torch.equal(outs[1], outs[3])


def test_merge_in_the_combine_launch_equals_the_merge_pass(device, always_cascade):
    """``run(..., merge=...)`` folds the levels into the members' rows in batch B's combine
    launch. Its out and lse equal batch B's run followed by ``attn_merge`` over the same
    parts, bit for bit, for members whose rows have one split after their levels (merged
    by the launch's extra workgroups) and members with several (merged by their combine
    records), and it leaves other rows as the run writes them."""
    say("cascade merge folded into the combine launch")
    pool = _pool(device, pages=200)
    cached = [8 * 256 + 5, 8 * 256 + 40, 8 * 256 + 300, 5000, 6100, 3 * 256 + 10, 7000, 2100, 600, 300]
    _prefix, caches = _shared_caches(pool, cached, prefix_pages=8)
    batch = PagedBatchCache(caches)
    batch.prepare(1)
    cas = batch._cascade
    assert cas is not None
    levels = _PrefixCascade.levels(batch, [1] * len(caches))
    shift = [0] * len(caches)
    for _ref, _first, end, members in levels:
        for b in members:
            shift[b] = max(shift[b], end)
    splits = {b: (cached[b] + 1 - 256 * shift[b] - 1) // 256 + 1 for b in range(len(caches)) if shift[b]}
    assert 1 in splits.values() and max(splits.values()) > 1, splits
    g = torch.Generator(device="cpu").manual_seed(9)
    q = torch.randn((len(caches), 32, 128), generator=g).to(torch.bfloat16).to(device)
    kp, vp = pool.keys[0], pool.values[0]
    rows_a, (out_rows, part_start, part_idx) = cas.rows_a, cas.merge
    o_a, lse_a = cas.plan_a.run(q, kp, vp, cas.bt_a, return_lse=True, query_rows=rows_a)
    want, want_lse = cas.plan_b.run(q, kp, vp, cas.bt_b, return_lse=True)
    plain = want.clone()
    ops.attn_merge(want, want_lse, o_a, lse_a, out_rows, parts=(part_start, part_idx))
    member_seq, member_of_seq = cas.members
    merge = ops.MergeParts(o_a, lse_a, member_seq, member_of_seq, part_start, part_idx)
    got, got_lse = cas.plan_b.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge)
    torch.cuda.synchronize()
    assert cas.plan_b.error_word() == 0
    assert torch.equal(got, want)
    assert torch.equal(got_lse, want_lse)
    members = set(out_rows.tolist())
    assert not torch.equal(got, plain)  # the levels changed the members' rows
    for r in range(len(caches)):
        if r not in members:
            assert torch.equal(got[r], plain[r])
    with pytest.raises(ValueError, match="combine phase"):
        cas.plan_b.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge, phases=("decode",))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_level_combine_in_the_decode_launch(device, dtype, always_cascade, monkeypatch):
    """``MergeParts(level_plan=plan_a)`` after batch A ran only its decode and chunk
    phases: batch A's combine records run as extra workgroups of batch B's decode launch,
    or in a combine launch of their own when the merging call has no decode launch.
    Either way batch A's rows and log-sum-exps, and batch B's merged out and lse, equal
    batch A's full run followed by the merging run, bit for bit."""
    say("level batch's combine in batch B's decode launch", dtype)
    pool = _pool(device, pages=200, dtype=dtype)
    cached = [8 * 256 + 5, 8 * 256 + 40, 8 * 256 + 300, 5000, 6100, 3 * 256 + 10, 7000, 2100, 600, 300]
    _prefix, caches = _shared_caches(pool, cached, prefix_pages=8)
    batch = PagedBatchCache(caches)
    batch.prepare(1)
    cas = batch._cascade
    assert cas is not None
    pa, pb = cas.plan_a, cas.plan_b
    assert pa.hints[2] > 0, pa.hints  # some level rows are split: batch A has combine records
    g = torch.Generator(device="cpu").manual_seed(11)
    q = torch.randn((len(caches), 32, 128), generator=g).to(dtype).to(device)
    kp, vp = pool.keys[0], pool.values[0]
    rows_a, (_out_rows, part_start, part_idx) = cas.rows_a, cas.merge
    member_seq, member_of_seq = cas.members
    o_ref, lse_ref = pa.run(q, kp, vp, cas.bt_a, return_lse=True, query_rows=rows_a)
    want, want_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True,
                            merge=ops.MergeParts(o_ref, lse_ref, member_seq, member_of_seq, part_start, part_idx))

    def level_run():  # batch A without its combine; rows it leaves hold a marker
        o_a = torch.full_like(o_ref, 7.0)
        lse_a = torch.full_like(lse_ref, 3.0)
        pa.run(q, kp, vp, cas.bt_a, out=o_a, lse_out=lse_a, query_rows=rows_a, phases=("decode", "chunk"))
        return o_a, lse_a, ops.MergeParts(o_a, lse_a, member_seq, member_of_seq, part_start, part_idx, level_plan=pa)

    o_a, lse_a, merge = level_run()
    got, got_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge)
    # The merging call without a decode launch: batch A's records get a launch of their own.
    o_c, lse_c, merge_c = level_run()
    out_c = torch.empty_like(want)
    lse_out_c = torch.empty_like(want_lse)
    pb.run(q, kp, vp, cas.bt_b, out=out_c, lse_out=lse_out_c, phases=("decode", "chunk"))
    pb.run(q, kp, vp, cas.bt_b, out=out_c, lse_out=lse_out_c, phases=("combine",), merge=merge_c)
    torch.cuda.synchronize()
    assert pa.error_word() == 0 and pb.error_word() == 0
    for o, lse, out, out_lse in ((o_a, lse_a, got, got_lse), (o_c, lse_c, out_c, lse_out_c)):
        assert torch.equal(o, o_ref)
        assert torch.equal(lse, lse_ref)
        assert torch.equal(out, want)
        assert torch.equal(out_lse, want_lse)
    with pytest.raises(ValueError, match="level_plan"):
        pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge._replace(level_plan=object()))
    # Checked mode reads both plans' error words after the call (and raises on neither).
    monkeypatch.setattr(ops, "CHECK_ERRORS", True)
    _o, _l, merge_d = level_run()
    pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge_d)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_level_chunk_in_the_merging_call(device, dtype, always_cascade, monkeypatch):
    """``MergeParts(level_plan=plan_a, level_block_table=..., level_query_rows=...)`` with
    batch A not run at all: batch A's chunk items share batch B's chunk launch (ahead of
    batch B's decode launch, which runs batch A's combine records). Batch A's rows and
    log-sum-exps, and batch B's merged out and lse, equal batch A's full run followed by
    the merging run, bit for bit; so does the cascade's attend, which takes this path."""
    say("level batch's chunk items in batch B's chunk launch", dtype)
    pool = _pool(device, pages=200, dtype=dtype)
    cached = [8 * 256 + 5, 8 * 256 + 40, 8 * 256 + 300, 5000, 6100, 3 * 256 + 10, 7000, 2100, 600, 300]
    _prefix, caches = _shared_caches(pool, cached, prefix_pages=8)
    batch = PagedBatchCache(caches)
    batch.prepare(1)
    cas = batch._cascade
    assert cas is not None
    pa, pb = cas.plan_a, cas.plan_b
    assert pa.hints[0] == 0 and pa.hints[1] > 0 and pa.hints[2] > 0, pa.hints
    g = torch.Generator(device="cpu").manual_seed(11)
    q = torch.randn((len(caches), 32, 128), generator=g).to(dtype).to(device)
    kp, vp = pool.keys[0], pool.values[0]
    rows_a, (_out_rows, part_start, part_idx) = cas.rows_a, cas.merge
    member_seq, member_of_seq = cas.members
    o_ref, lse_ref = pa.run(q, kp, vp, cas.bt_a, return_lse=True, query_rows=rows_a)
    want, want_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True,
                            merge=ops.MergeParts(o_ref, lse_ref, member_seq, member_of_seq, part_start, part_idx))
    o_a = torch.full_like(o_ref, 7.0)
    lse_a = torch.full_like(lse_ref, 3.0)
    merge = ops.MergeParts(o_a, lse_a, member_seq, member_of_seq, part_start, part_idx, level_plan=pa,
                           level_block_table=cas.bt_a, level_query_rows=rows_a)
    got, got_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge)
    out = cas.attend(q, kp, vp)
    torch.cuda.synchronize()
    assert pa.error_word() == 0 and pb.error_word() == 0
    assert torch.equal(o_a, o_ref) and torch.equal(lse_a, lse_ref)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)
    assert torch.equal(out, want)
    with pytest.raises(ValueError, match="level_block_table"):
        pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge._replace(level_block_table=None))
    with pytest.raises(ValueError, match="three phases"):
        pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge, phases=("decode", "combine"))
    with pytest.raises(ValueError, match="level_query_rows"):
        pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge._replace(level_query_rows=rows_a[:-1]))
    # Checked mode reads both plans' error words after the call (and raises on neither).
    monkeypatch.setattr(ops, "CHECK_ERRORS", True)
    pb.run(q, kp, vp, cas.bt_b, return_lse=True, merge=merge)


def test_level_combine_of_long_levels_gets_its_own_launch(device, always_cascade):
    """Levels longer than 8192 keys (40 shared pages here) want 512-thread combine
    workgroups, which a decode launch does not hold: batch A's records then get a combine
    launch of their own inside the merging call. Bits as batch A's full run followed by
    the merging run."""
    say("level batch over 40 shared pages: its combine in a launch of its own")
    config = Qwen3Config(context_length=16384, n_layers=1, dtype=torch.bfloat16)
    pool = KVPagePool(config, 400, device=device)
    g = torch.Generator(device=device).manual_seed(13)
    for t in pool.keys + pool.values:
        t.normal_(generator=g)
    prefix = PagedKVCache(pool, 16384)
    prefix.pages.extend(pool.acquire(40))
    prefix.length = 40 * 256
    caches = []
    for n in [40 * 256 + 7, 40 * 256 + 300, 41 * 256 + 5, 44 * 256, 38 * 256 + 9, 12000]:
        cache = PagedKVCache(pool, 16384)
        shared = min(40, n // 256)
        cache.pages.extend(prefix.pages[:shared])
        cache.pages.extend(pool.acquire(-(-n // 256) - shared))
        cache.length = n
        caches.append(cache)
    batch = PagedBatchCache(caches)
    batch.prepare(1)
    cas = batch._cascade
    assert cas is not None
    pa, pb = cas.plan_a, cas.plan_b
    assert pa.max_k > 8192 and pa.hints[2] > 0, (pa.max_k, pa.hints)
    q = torch.randn((len(caches), 32, 128), generator=torch.Generator(device="cpu").manual_seed(5)).to(
        torch.bfloat16).to(device)
    kp, vp = pool.keys[0], pool.values[0]
    rows_a, (_out_rows, part_start, part_idx) = cas.rows_a, cas.merge
    member_seq, member_of_seq = cas.members
    o_ref, lse_ref = pa.run(q, kp, vp, cas.bt_a, return_lse=True, query_rows=rows_a)
    want, want_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True,
                            merge=ops.MergeParts(o_ref, lse_ref, member_seq, member_of_seq, part_start, part_idx))
    o_a = torch.full_like(o_ref, 7.0)
    lse_a = torch.full_like(lse_ref, 3.0)
    pa.run(q, kp, vp, cas.bt_a, out=o_a, lse_out=lse_a, query_rows=rows_a, phases=("decode", "chunk"))
    got, got_lse = pb.run(q, kp, vp, cas.bt_b, return_lse=True,
                          merge=ops.MergeParts(o_a, lse_a, member_seq, member_of_seq, part_start, part_idx,
                                               level_plan=pa))
    # Batch A's chunk items in the merging call too (its records then get their launch
    # between the shared chunk launch and batch B's decode launch).
    o_f = torch.full_like(o_ref, 7.0)
    lse_f = torch.full_like(lse_ref, 3.0)
    got_f, got_lse_f = pb.run(q, kp, vp, cas.bt_b, return_lse=True,
                              merge=ops.MergeParts(o_f, lse_f, member_seq, member_of_seq, part_start, part_idx,
                                                   level_plan=pa, level_block_table=cas.bt_a,
                                                   level_query_rows=rows_a))
    torch.cuda.synchronize()
    assert pa.error_word() == 0 and pb.error_word() == 0
    assert torch.equal(o_a, o_ref) and torch.equal(lse_a, lse_ref)
    assert torch.equal(got, want) and torch.equal(got_lse, want_lse)
    assert torch.equal(o_f, o_ref) and torch.equal(lse_f, lse_ref)
    assert torch.equal(got_f, want) and torch.equal(got_lse_f, want_lse)
    # And the attend path itself against the oracle.
    out = cas.attend(q, kp, vp)
    _compare(out.float().cpu().numpy(), _oracle(pool, caches, [1] * len(caches), q), "cascade attend, 40-page levels")
