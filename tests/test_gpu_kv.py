"""KV append, page copy and page gather on the GPU: bit-exact against torch's
index_copy_ / index_select / copy_ and the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops
from oracle import dense_torch, kv_bytes
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


def random_bits(shape, dtype, device, seed):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    width = torch.finfo(dtype).bits
    int_t = {16: torch.int16, 32: torch.int32}[width]
    lo, hi = -(2 ** (width - 1)), 2 ** (width - 1) - 1
    return torch.randint(lo, hi, shape, generator=g, dtype=torch.int64).to(int_t).view(dtype).to(device)


def bits(t):
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_append_matches_index_copy(device, dtype):
    say("append", dtype)
    P, S, H, D, T = 12, 256, 8, 128, 77
    k_pool = random_bits((P, S, H, D), dtype, device, 1)
    v_pool = random_bits((P, S, H, D), dtype, device, 2)
    k_new = random_bits((T, H, D), dtype, device, 3)
    v_new = random_bits((T, H, D), dtype, device, 4)
    slots = torch.randperm(P * S, generator=torch.Generator().manual_seed(5))[:T].to(device)
    ek, ev = bits(k_pool).clone().view(-1, H, D), bits(v_pool).clone().view(-1, H, D)
    ek.index_copy_(0, slots, bits(k_new))
    ev.index_copy_(0, slots, bits(v_new))
    ops.kv_append(k_pool, v_pool, slots, k_new, v_new)
    torch.cuda.synchronize()
    assert torch.equal(bits(k_pool).view(-1, H, D), ek)
    assert torch.equal(bits(v_pool).view(-1, H, D), ev)
    # the numpy restatement agrees on the same bits
    hk = bits(random_bits((P, S, H, D), dtype, "cpu", 1)).numpy()
    hv = bits(random_bits((P, S, H, D), dtype, "cpu", 2)).numpy()
    kv_bytes.kv_append(hk, hv, slots.cpu().numpy(), bits(k_new).cpu().numpy(), bits(v_new).cpu().numpy())
    assert np.array_equal(hk, bits(k_pool).cpu().numpy())


def test_append_from_strided_views_and_page_boundaries(device):
    say("append strided")
    P, S, H, D, B, T = 4, 256, 8, 128, 3, 5
    k_pool = torch.zeros((P, S, H, D), dtype=torch.bfloat16, device=device)
    v_pool = torch.zeros_like(k_pool)
    # keys as the model produces them: [B, T, H, D] memory viewed as [B, H, T, D]
    k = torch.randn(B, T, H, D, device=device).to(torch.bfloat16).transpose(1, 2)
    v = torch.randn(B, T, H, 2 * D, device=device).to(torch.bfloat16)[..., :D].transpose(1, 2)
    packed_k = k.transpose(1, 2).reshape(-1, H, D)
    packed_v = v.transpose(1, 2).reshape(-1, H, D)
    assert packed_v.stride(1) == 2 * D  # really strided
    slots = torch.tensor([253, 254, 255, 256, 257, 511, 512, 0, 1, 2, 767, 766, 765, 764, 1023],
                         device=device)
    ops.kv_append(k_pool, v_pool, slots, packed_k, packed_v)
    torch.cuda.synchronize()
    assert torch.equal(k_pool.view(-1, H, D)[slots], packed_k)
    assert torch.equal(v_pool.view(-1, H, D)[slots], packed_v)
    mask = torch.ones(P * S, dtype=torch.bool, device=device)
    mask[slots] = False
    assert not k_pool.view(-1, H, D)[mask].any()


@pytest.mark.parametrize("dtype,heads,dim", [
    (torch.bfloat16, 3, 128),   # 16-byte words, 3 heads: the division form
    (torch.bfloat16, 8, 96),    # 12 words per head row: the division form
    (torch.float32, 2, 6),      # 8-byte words
    (torch.float16, 4, 64),     # 8 words, 4 heads: the shift form
])
def test_append_other_head_shapes(device, dtype, heads, dim):
    say("append shape", dtype, heads, dim)
    P, S, T = 3, 256, 301
    k_pool = random_bits((P, S, heads, dim), dtype, device, 11)
    v_pool = random_bits((P, S, heads, dim), dtype, device, 12)
    k_new = random_bits((T, heads, dim), dtype, device, 13)
    v_new = random_bits((T, heads, dim), dtype, device, 14)
    slots = torch.randperm(P * S, generator=torch.Generator().manual_seed(15))[:T]
    slots[7], slots[100] = -1, P * S  # skipped rows
    slots = slots.to(device)
    keep = (slots >= 0) & (slots < P * S)
    ek, ev = bits(k_pool).clone().view(-1, heads, dim), bits(v_pool).clone().view(-1, heads, dim)
    ek.index_copy_(0, slots[keep], bits(k_new)[keep])
    ev.index_copy_(0, slots[keep], bits(v_new)[keep])
    ops.kv_append(k_pool, v_pool, slots, k_new, v_new)
    torch.cuda.synchronize()
    assert torch.equal(bits(k_pool).view(-1, heads, dim), ek)
    assert torch.equal(bits(v_pool).view(-1, heads, dim), ev)


def test_append_skips_out_of_range_slots_and_empty(device):
    say("append out-of-range slots")
    P, S, H, D = 2, 256, 8, 128
    k_pool = torch.zeros((P, S, H, D), dtype=torch.bfloat16, device=device)
    v_pool = torch.zeros_like(k_pool)
    k_new = torch.ones((4, H, D), dtype=torch.bfloat16, device=device)
    slots = torch.tensor([-1, 3, P * S, 500], device=device)
    ops.kv_append(k_pool, v_pool, slots, k_new, k_new)
    torch.cuda.synchronize()
    flat = k_pool.view(-1, H, D)
    assert flat[3].eq(1).all() and flat[500].eq(1).all()
    assert int(flat.ne(0).any(dim=(1, 2)).sum()) == 2
    ops.kv_append(k_pool, v_pool, slots[:0], k_new[:0], k_new[:0])
    torch.cuda.synchronize()


@pytest.mark.parametrize("with_values", [True, False])
def test_copy_pages_all_layers_bit_exact(device, with_values):
    say("copy pages", with_values)
    layers, P = 36, 10
    shape = (P, 256, 8, 128)
    ks = [random_bits(shape, torch.bfloat16, device, 10 + i) for i in range(layers)]
    vs = [random_bits(shape, torch.bfloat16, device, 100 + i) for i in range(layers)]
    before_k = [bits(t).clone() for t in ks]
    before_v = [bits(t).clone() for t in vs]
    src, dst = [1, 5, 2, 9], [6, 0, 7, 3]
    ops.kv_copy_pages(ks, vs if with_values else None, src, dst)
    torch.cuda.synchronize()
    for t, b in zip(ks, before_k):
        ref = b.clone()
        ref[dst] = b[src]
        assert torch.equal(bits(t), ref)
    for t, b in zip(vs, before_v):
        if with_values:
            ref = b.clone()
            ref[dst] = b[src]
            assert torch.equal(bits(t), ref)
        else:
            assert torch.equal(bits(t), b)


def test_copy_pages_chunks_over_many_tensors_and_pages(device):
    say("copy pages chunked")
    P = 150
    shape = (P, 256, 1, 64)  # 32 KiB pages
    ks = [random_bits(shape, torch.float16, device, 7 + i) for i in range(40)]
    vs = [random_bits(shape, torch.float16, device, 70 + i) for i in range(40)]
    src, dst = list(range(0, 70)), list(range(75, 145))
    before = [bits(t).clone() for t in ks + vs]
    ops.kv_copy_pages(ks, vs, src, dst)
    torch.cuda.synchronize()
    for t, b in zip(ks + vs, before):
        ref = b.clone()
        ref[dst] = b[src]
        assert torch.equal(bits(t), ref)
    with pytest.raises(ValueError):
        ops.kv_copy_pages(ks, vs, [1, 2], [2, 3])  # overlap


@pytest.mark.parametrize("length", [1, 255, 256, 257, 600, 1024])
def test_gather_matches_index_select(device, length):
    say("gather", length)
    P = 6
    pool = random_bits((P, 256, 8, 128), torch.bfloat16, device, 42)
    pages = [4, 1, 5, 0][: (length + 255) // 256]
    got = ops.kv_gather(pool, pages, length)
    ref = dense_torch.gather(bits(pool), pages, length)
    torch.cuda.synchronize()
    assert got.shape == (1, 8, length, 128)
    assert torch.equal(bits(got), ref)
    host = kv_bytes.kv_gather(bits(pool).cpu().numpy(), pages, length)
    assert np.array_equal(host, bits(got).cpu().numpy())


def test_gather_invalid_page_yields_zeros(device):
    say("gather invalid page")
    pool = torch.ones((3, 256, 8, 128), dtype=torch.bfloat16, device=device)
    got = ops.kv_gather(pool, [1, 7], 300)
    torch.cuda.synchronize()
    assert got[:, :, :256].eq(1).all() and not got[:, :, 256:].any()


@pytest.mark.parametrize("dtype,heads,dim", [(torch.float32, 2, 6), (torch.uint8, 3, 5)])
def test_gather_narrow_rows_take_the_generic_path(device, dtype, heads, dim):
    """Rows that are not 16-byte multiples (24 B, 5 B) go through the element-wise kernel."""
    say("gather generic", dtype)
    g = torch.Generator(device="cpu").manual_seed(8)
    pool = torch.randint(0, 255, (4, 256, heads, dim), generator=g).to(dtype).to(device)
    got = ops.kv_gather(pool, [2, 0, 3], 700)
    torch.cuda.synchronize()
    ref = pool.index_select(0, torch.tensor([2, 0, 3], device=device)).reshape(-1, heads, dim)[:700]
    assert torch.equal(got[0].permute(1, 0, 2), ref)


def test_c4_restore_of_16_prefix_pages_over_36_layers(device):
    """The C4 restore at its full size, through the pool: a request restores a 16-page
    prefix snapshot with ``restore_blocks(copy=True)``, which copies those pages for all
    36 layers, K and V (72 tensors of [pages, 256, 8, 128] bf16, more than a launch's
    tensor table holds; the pool's constant layer stride lets one launch cover them).
    Every destination page equals its source bit for bit, as torch's copy_ of the same
    pages gives, and no other page changes."""
    from helios_amd.config import Qwen3Config
    from helios_amd.paged_cache import KVPagePool, PagedKVCache

    say("c4 restore 36 layers x 16 pages")
    config = Qwen3Config()
    pool = KVPagePool(config, 40, device=device)
    g = torch.Generator(device=device).manual_seed(17)
    flat = pool.storage.view(torch.int16)
    flat.copy_(torch.randint(-32768, 32767, flat.shape, generator=g, device=device, dtype=torch.int16))
    source = PagedKVCache(pool, config.context_length)
    source.pages.extend(pool.acquire(18))
    source.length = 16 * 256 + 300
    snapshot = source.snapshot_block(0, 16 * 256)
    before = flat.clone()
    request = PagedKVCache(pool, config.context_length)
    request.restore_blocks([snapshot], copy=True)
    torch.cuda.synchronize()
    src = [p.index for p in snapshot.pages]
    dst = [p.index for p in request.pages]
    assert len(dst) == 16 and not set(src) & set(dst) and request.length == 16 * 256
    expect = before.clone()
    expect[:, :, dst] = before[:, :, src]      # torch's copy of the same pages, every layer
    assert torch.equal(flat, expect)
    assert all(p not in src for p in dst) and request.pages[0] is not snapshot.pages[0]
