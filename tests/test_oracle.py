"""Pins the CPU oracle (test infrastructure) before it is trusted as the checker.

Each oracle function is checked against something it does not share code with:
closed forms, brute-force loops, torch library routines (index_copy_, index_select,
scaled_dot_product_attention), invariances, and committed golden fixtures.
"""

from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from helios_amd import synth
from oracle import attention as oa
from oracle import dense_torch, kv_bytes

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------------ input generator
def test_splitmix64_matches_published_sequence():
    # SplitMix64 (Steele, Lea, Flood 2014) seeded with 0: the first outputs of the
    # published reference implementation.
    got = [int(x) for x in synth.splitmix64(0, 3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_normal_moments_and_determinism():
    a = synth.normal(11, (1 << 18,), np.float64)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert np.array_equal(a, synth.normal(11, (1 << 18,), np.float64))
    assert not np.array_equal(a[:16], synth.normal(12, (16,), np.float64))


def test_workload_shapes_follow_the_configs():
    w1 = synth.c1()
    assert w1.cached == [37, 256, 300, 611] and w1.k_lens == [38, 257, 301, 612]
    assert [len(t) for t in w1.tables] == [1, 2, 2, 3]
    assert sorted(p for t in w1.tables for p in t) == sorted(set(p for t in w1.tables for p in t))
    w2 = synth.c2()
    assert w2.batch == 64 and all(512 <= c <= 4096 for c in w2.cached)
    assert w2.unique_pages() == sum(len(t) for t in w2.tables)
    w3 = synth.c3()
    assert w3.q_lens[-2:] == [1024, 992] and w3.cached[-2:] == [0, 512] and w3.total_q == 2048
    w4 = synth.c4()
    assert w4.k_lens[:8] == [32768] * 8 and all(len(t) == 128 for t in w4.tables[:8])
    assert all(t[:16] == w4.tables[0][:16] for t in w4.tables[:8])
    assert w4.k_lens[8] == 8192 and w4.q_lens[8] == 4096
    # unique pages: 16 shared + 8 * 112 private for the decoders
    assert w4.decode_bytes() == 2 * (16 + 8 * 112) * 256 * 8 * 128 * 2 + 2 * 8 * 32 * 128 * 2


# ------------------------------------------------------------------ byte movers
def test_kv_append_matches_index_copy_and_leaves_other_slots():
    rng = np.random.default_rng(0)
    pool_k = rng.integers(0, 2**16, size=(4, 256, 2, 8), dtype=np.uint16)
    pool_v = rng.integers(0, 2**16, size=(4, 256, 2, 8), dtype=np.uint16)
    slots = np.array([5, 256 * 3 + 255, 300, 0], dtype=np.int64)
    k_new = rng.integers(0, 2**16, size=(4, 2, 8), dtype=np.uint16)
    v_new = rng.integers(0, 2**16, size=(4, 2, 8), dtype=np.uint16)
    ek = torch.from_numpy(pool_k.astype(np.int32)).view(-1, 2, 8).clone()
    ek.index_copy_(0, torch.from_numpy(slots), torch.from_numpy(k_new.astype(np.int32)))
    before = pool_k.copy()
    kv_bytes.kv_append(pool_k, pool_v, slots, k_new, v_new)
    assert np.array_equal(pool_k.reshape(-1, 2, 8).astype(np.int32), ek.numpy())
    untouched = np.setdiff1d(np.arange(4 * 256), slots)
    assert np.array_equal(pool_k.reshape(-1, 2, 8)[untouched], before.reshape(-1, 2, 8)[untouched])
    assert np.array_equal(pool_v.reshape(-1, 2, 8)[slots], v_new)


def test_kv_gather_matches_index_select_and_loops():
    rng = np.random.default_rng(1)
    pool = rng.integers(0, 2**16, size=(5, 256, 3, 4), dtype=np.uint16)
    pages, length = [3, 0, 4], 600
    got = kv_bytes.kv_gather(pool, pages, length)
    t = torch.from_numpy(pool.astype(np.int32))
    ref = t.index_select(0, torch.tensor(pages)).reshape(-1, 3, 4)[:length].permute(1, 0, 2).unsqueeze(0)
    assert np.array_equal(got.astype(np.int32), ref.numpy())
    for j in (0, 255, 256, 511, 599):
        for h in range(3):
            assert np.array_equal(got[0, h, j], pool[pages[j // 256], j % 256, h])


def test_kv_copy_pages_is_a_per_layer_page_copy():
    rng = np.random.default_rng(2)
    layers = [rng.integers(0, 2**16, size=(8, 256, 2, 4), dtype=np.uint16) for _ in range(3)]
    before = [x.copy() for x in layers]
    kv_bytes.kv_copy_pages(layers, [1, 6], [4, 2])
    for x, b in zip(layers, before):
        assert np.array_equal(x[4], b[1]) and np.array_equal(x[2], b[6])
        for p in (0, 1, 3, 5, 6, 7):
            assert np.array_equal(x[p], b[p])


# ------------------------------------------------------------------ attention
def _tiny(seed, n, L, hq, hkv, d):
    q = synth.normal(seed, (n, hq, d), np.float64)
    k = synth.normal(seed + 1, (L, hkv, d), np.float64)
    v = synth.normal(seed + 2, (L, hkv, d), np.float64)
    return q, k, v


def test_single_key_returns_its_value():
    q, k, v = _tiny(3, 1, 1, 4, 2, 8)
    out, lse = oa.attend_dense(q, k, v, scale=0.5)
    for h in range(4):
        assert np.allclose(out[0, h], v[0, h // 2])
        assert np.isclose(lse[h, 0], 0.5 * q[0, h] @ k[0, h // 2])


def test_equal_keys_average_the_visible_values():
    q, k, v = _tiny(4, 3, 7, 2, 1, 8)
    k[:] = k[0]
    out, _ = oa.attend_dense(q, k, v, scale=1.0)
    for i in range(3):  # row i sees keys 0 .. 4 + i
        assert np.allclose(out[i, 0], v[: 5 + i, 0].mean(axis=0))


def test_dominant_key_selects_its_value():
    q, k, v = _tiny(5, 1, 9, 1, 1, 8)
    k[6] = 40.0 * q[0, 0] / np.linalg.norm(q[0, 0])
    out, _ = oa.attend_dense(q, k, v, scale=1.0)
    assert np.allclose(out[0, 0], v[6, 0], atol=1e-9)


@pytest.mark.parametrize("window", [(-1, 0), (-1, -1), (2, 0), (1, 1), (0, 0)])
def test_attention_matches_brute_force_loops(window):
    q, k, v = _tiny(6, 3, 6, 4, 2, 4)
    out, _ = oa.attend_dense(q, k, v, scale=0.7, window=window)
    ref = oa.brute_force_attention(q.tolist(), k.tolist(), v.tolist(), scale=0.7, window=window)
    assert np.allclose(out, np.asarray(ref), atol=1e-12)


def test_fresh_prefill_is_textbook_causal_softmax():
    q, k, v = _tiny(7, 5, 5, 2, 2, 8)
    out, _ = oa.attend_dense(q, k, v, scale=0.3)
    s = np.einsum("ihd,jhd->hij", q, k) * 0.3
    s = np.where(np.tril(np.ones((5, 5), bool))[None], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.allclose(out, np.einsum("hij,jhd->ihd", p, v), atol=1e-12)


def test_attention_matches_torch_sdpa_with_gqa():
    q, k, v = _tiny(8, 37, 300, 8, 2, 16)
    out, _ = oa.attend_dense(q, k, v, scale=0.25)
    tq = torch.from_numpy(q).permute(1, 0, 2)[None]
    tk = torch.from_numpy(k).permute(1, 0, 2)[None].repeat_interleave(4, dim=1)
    tv = torch.from_numpy(v).permute(1, 0, 2)[None].repeat_interleave(4, dim=1)
    mask = torch.arange(300)[None, :] <= (263 + torch.arange(37))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=0.25)
    assert np.allclose(out, ref[0].permute(1, 0, 2).numpy(), atol=1e-12)


def test_paged_equals_dense_and_ignores_page_placement():
    w = synth.small_mixed(21, num_pages=24)
    x = synth.host_inputs(w, np.float64)
    out, lse = oa.paged_varlen_attention(x["q"], x["k_pool"], x["v_pool"], w.cu_seq_q, w.k_lens, w.tables)
    perm = synth.permutation(99, w.num_pages)
    inv = np.argsort(perm)
    k2, v2 = x["k_pool"][perm], x["v_pool"][perm]
    tables2 = [[int(inv[p]) for p in t] for t in w.tables]
    out2, lse2 = oa.paged_varlen_attention(x["q"], k2, v2, w.cu_seq_q, w.k_lens, tables2)
    assert np.array_equal(out, out2) and np.array_equal(lse, lse2)
    for b in range(w.batch):
        q0, q1 = w.cu_seq_q[b], w.cu_seq_q[b + 1]
        L = w.k_lens[b]
        kd = oa.gather_sequence(x["k_pool"], w.tables[b], L)
        vd = oa.gather_sequence(x["v_pool"], w.tables[b], L)
        o, _ = oa.attend_dense(x["q"][q0:q1], kd, vd, scale=1 / math.sqrt(128))
        assert np.array_equal(o, out[q0:q1])


def test_reference_dense_torch_path_agrees_with_float64_oracle():
    w = synth.c1()
    x = synth.host_inputs(w, np.float32)
    out, _ = oa.paged_varlen_attention(x["q"], x["k_pool"], x["v_pool"], w.cu_seq_q, w.k_lens, w.tables)
    q = torch.from_numpy(x["q"]).permute(1, 0, 2)[None]
    ref = dense_torch.packed_attention(q, torch.from_numpy(x["k_pool"]), torch.from_numpy(x["v_pool"]),
                                       w.tables, w.cached, w.q_lens)
    assert np.allclose(ref[0].permute(1, 0, 2).numpy(), out, atol=2e-6)


# ------------------------------------------------------------------ golden fixtures
def test_golden_c1_fixture():
    meta = json.loads((GOLDEN / "c1_meta.json").read_text())
    fixture = np.load(GOLDEN / "c1_bf16.npz")
    w = synth.c1(meta["seed"])
    assert w.tables == meta["tables"] and w.k_lens == meta["k_lens"]
    x = synth.host_inputs(w, np.float32)
    bits = {}
    for name, arr in x.items():
        b16 = torch.from_numpy(arr).to(torch.bfloat16).view(torch.int16).numpy()
        bits[name] = hashlib.sha256(b16.tobytes()).hexdigest()
    assert bits == meta["input_sha256_bf16"]
    xb = {n: torch.from_numpy(a).to(torch.bfloat16).to(torch.float64).numpy() for n, a in x.items()}
    kv_bytes.kv_append(xb["k_pool"], xb["v_pool"], w.write_slots(), xb["k_new"], xb["v_new"])
    out, lse = oa.paged_varlen_attention(xb["q"], xb["k_pool"], xb["v_pool"], w.cu_seq_q, w.k_lens, w.tables)
    assert np.allclose(out, fixture["out"], atol=1e-6, rtol=0)
    assert np.allclose(lse, fixture["lse"], atol=1e-6, rtol=0)


def test_golden_brute_force_vectors():
    cases = json.loads((GOLDEN / "tiny_attention.json").read_text())
    assert len(cases) >= 4
    for case in cases:
        q, k, v = (np.asarray(case[n], dtype=np.float64) for n in ("q", "k", "v"))
        out, _ = oa.attend_dense(q, k, v, scale=case["scale"], window=tuple(case["window"]))
        assert np.allclose(out, np.asarray(case["out"]), atol=1e-12)
