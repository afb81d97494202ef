"""Fused q/k RMSNorm + RoPE + KV append on the GPU: against the numpy oracle and the
reference's own op sequence in torch, and attend_projected against norm/RoPE in torch
followed by attend."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import ops
from helios_amd.config import Qwen3Config
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedKVCache
from oracle import dense_torch, rope
from tests.gpu_cases import MAX_ABS, MEAN_ABS, say

pytestmark = pytest.mark.gpu


def pair_close(got: torch.Tensor, ref: torch.Tensor) -> bool:
    """|got - ref| <= 2 ulps of the rotated pair's norm, element by element. RoPE turns
    each pair (i, i + 64) of normalised values by an angle; a one-ulp change of those
    inputs moves both outputs by about one ulp of the pair norm, even where an output
    itself is near zero, so the bound is taken at the pair norm."""
    g, r = got.float().cpu(), ref.float().cpu()
    eps = 2.0 ** -7 if got.dtype == torch.bfloat16 else 2.0 ** -10
    half = r.shape[-1] // 2
    norm = torch.sqrt(r[..., :half] ** 2 + r[..., half:] ** 2)
    tol = 2 * eps * torch.cat([norm, norm], dim=-1) + 1e-6
    return bool(((g - r).abs() <= tol).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 7, 300])
@pytest.mark.parametrize("offset", [0, 1], ids=["aligned16", "unaligned"])
def test_kernel_matches_oracle_and_reference_ops(device, dtype, rows, offset):
    """offset 0: 16-byte aligned rows (the 16-byte-access kernel); offset 1 shifts the
    projection by one element, which sends the launch to the 2-byte-access kernel."""
    say("qk rope", dtype, rows, offset)
    g = torch.Generator(device="cpu").manual_seed(rows)
    hq, hkv, d = 32, 8, 128
    proj = torch.randn(rows, (hq + 2 * hkv) * d + offset, generator=g).to(dtype).to(device)[:, offset:]
    q = proj[:, : hq * d].view(rows, hq, d)              # strided views of one projection
    k = proj[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
    v = proj[:, (hq + hkv) * d:].view(rows, hkv, d)
    wq = (1 + 0.2 * torch.randn(d, generator=g)).float().to(device)
    wk = (1 + 0.2 * torch.randn(d, generator=g)).float().to(device)
    cos, sin = dense_torch.rope_parameters(d, 40960, 1_000_000.0)
    cos, sin = cos.to(device), sin.to(device)
    positions = torch.randint(0, 40960, (rows,), generator=g).to(device)
    pages = 4
    k_pool = torch.randn(pages, 256, hkv, d, generator=g).to(dtype).to(device)
    v_pool = torch.randn(pages, 256, hkv, d, generator=g).to(dtype).to(device)
    k_before, v_before = k_pool.clone(), v_pool.clone()
    slots = torch.randperm(pages * 256, generator=g)[:rows]
    if rows > 3:
        slots[1] = -1            # skipped
        slots[2] = pages * 256   # skipped
    slots = slots.to(device)
    q_out = ops.qk_norm_rope_append(q, k, v, wq, wk, cos, sin, positions, k_pool, v_pool, slots, 1e-6)
    torch.cuda.synchronize()

    # Reference op sequence (layers.py) on the same device.
    def ref(x, w):
        y = dense_torch.rms_norm(x.transpose(0, 1).unsqueeze(0), w, 1e-6)
        return dense_torch.apply_rope(y, cos, sin, positions.unsqueeze(0))[0].transpose(0, 1)

    # rsqrt is the hardware approximation (as in torch on this device) and the sum of
    # squares runs in another order, so a normalised element can differ by one ulp.
    q_ref, k_ref = ref(q, wq), ref(k, wk)
    assert pair_close(q_out, q_ref)
    assert (q_out != q_ref).float().mean().item() < 5e-3
    # numpy oracle
    name = "bf16" if dtype == torch.bfloat16 else "fp16"
    q_np = rope.norm_rope(q.float().cpu().numpy(), wq.cpu().numpy(), cos.cpu().numpy(),
                          sin.cpu().numpy(), positions.cpu().numpy(), 1e-6, name)
    assert pair_close(q_out, torch.from_numpy(q_np).to(dtype))
    # pools: rotated keys and raw values at the valid slots, nothing else touched
    kf, vf = k_pool.view(-1, hkv, d), v_pool.view(-1, hkv, d)
    kb, vb = k_before.view(-1, hkv, d), v_before.view(-1, hkv, d)
    valid = (slots >= 0) & (slots < pages * 256)
    vs = slots[valid]
    assert pair_close(kf[vs], k_ref[valid])
    assert torch.equal(vf[vs].view(torch.int16), v[valid].contiguous().view(torch.int16))
    untouched = torch.ones(pages * 256, dtype=torch.bool, device=device)
    untouched[vs] = False
    assert torch.equal(kf[untouched].view(torch.int16), kb[untouched].view(torch.int16))
    assert torch.equal(vf[untouched].view(torch.int16), vb[untouched].view(torch.int16))


@pytest.mark.parametrize("hq,hkv", [(64, 8), (16, 2), (8, 8)])
def test_kernel_other_head_counts(device, hq, hkv):
    """Head counts whose last 4-head group is partial (16 + 2 * 2 = 20 heads) or that
    take more passes per row (64 + 16 = 80 heads), both layouts."""
    say("qk rope heads", hq, hkv)
    g = torch.Generator(device="cpu").manual_seed(hq + hkv)
    d, rows = 128, 37
    for offset in (0, 1):
        proj = torch.randn(rows, (hq + 2 * hkv) * d + offset, generator=g).to(torch.bfloat16).to(device)[:, offset:]
        q = proj[:, : hq * d].view(rows, hq, d)
        k = proj[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
        v = proj[:, (hq + hkv) * d:].view(rows, hkv, d)
        wq = (1 + 0.2 * torch.randn(d, generator=g)).float().to(device)
        wk = (1 + 0.2 * torch.randn(d, generator=g)).float().to(device)
        cos, sin = dense_torch.rope_parameters(d, 4096, 1_000_000.0)
        cos, sin = cos.to(device), sin.to(device)
        positions = torch.randint(0, 4096, (rows,), generator=g).to(device)
        k_pool = torch.zeros(2, 256, hkv, d, dtype=torch.bfloat16, device=device)
        v_pool = torch.zeros_like(k_pool)
        slots = torch.randperm(512, generator=g)[:rows].to(device)
        q_out = ops.qk_norm_rope_append(q, k, v, wq, wk, cos, sin, positions, k_pool, v_pool, slots, 1e-6)
        torch.cuda.synchronize()

        def ref(x, w):
            y = dense_torch.rms_norm(x.transpose(0, 1).unsqueeze(0), w, 1e-6)
            return dense_torch.apply_rope(y, cos, sin, positions.unsqueeze(0))[0].transpose(0, 1)

        assert pair_close(q_out, ref(q, wq))
        assert pair_close(k_pool.view(-1, hkv, d)[slots], ref(k, wk))
        assert torch.equal(v_pool.view(-1, hkv, d)[slots].view(torch.int16), v.contiguous().view(torch.int16))


def test_attend_projected_matches_torch_norm_rope_then_attend(device):
    say("attend_projected")
    config = Qwen3Config(context_length=8192, n_layers=2, dtype=torch.bfloat16)
    d, hq, hkv = config.head_dim, config.n_heads, config.n_kv_heads
    g = torch.Generator(device=device).manual_seed(2)
    lengths, counts = [700, 0, 255, 1500], [1, 300, 1, 40]
    total = sum(counts)
    cos, sin = dense_torch.rope_parameters(d, config.context_length, config.rope_base)
    cos, sin = cos.to(device), sin.to(device)
    wq = (1 + 0.1 * torch.randn(d, generator=g, device=device)).float()
    wk = (1 + 0.1 * torch.randn(d, generator=g, device=device)).float()
    x_q = torch.randn((1, total, hq * d), generator=g, device=device).to(config.dtype)
    x_k = torch.randn((1, total, hkv * d), generator=g, device=device).to(config.dtype)
    x_v = torch.randn((1, total, hkv * d), generator=g, device=device).to(config.dtype)
    outs, pools = [], []
    for fused in (True, False):
        pool = KVPagePool(config, 32, device=device)
        gp = torch.Generator(device=device).manual_seed(7)
        for t in pool.keys + pool.values:
            t.copy_(torch.randn(t.shape, generator=gp, device=device).to(t.dtype))
        caches = []
        for n in lengths:
            cache = PagedKVCache(pool, config.context_length)
            if n:
                cache.pages.extend(pool.acquire(-(-n // 256)))
                cache.length = n
            caches.append(cache)
        batch = PackedBatchCache(caches)
        batch.prepare_packed(counts)
        if fused:
            out = batch.attend_projected(1, x_q, x_k, x_v, wq, wk, cos, sin, config.rms_norm_eps)
        else:
            q = x_q.view(1, total, hq, d).transpose(1, 2)
            k = x_k.view(1, total, hkv, d).transpose(1, 2)
            v = x_v.view(1, total, hkv, d).transpose(1, 2)
            q = dense_torch.apply_rope(dense_torch.rms_norm(q, wq, config.rms_norm_eps), cos, sin, batch.positions)
            k = dense_torch.apply_rope(dense_torch.rms_norm(k, wk, config.rms_norm_eps), cos, sin, batch.positions)
            out = batch.attend(1, q, k, v)
        torch.cuda.synchronize()
        outs.append(out.float().cpu())
        pools.append((pool.keys[1].clone(), pool.values[1].clone()))
        batch.advance_packed()
    diff = (outs[0] - outs[1]).abs()
    assert outs[0].shape == (1, hq, total, d)
    assert diff.max().item() <= MAX_ABS and diff.mean().item() <= MEAN_ABS
    assert pair_close(pools[0][0], pools[1][0])
    assert torch.equal(pools[0][1].view(torch.int16), pools[1][1].view(torch.int16))
