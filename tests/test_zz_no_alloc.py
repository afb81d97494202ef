"""hx_varlen_attn_noalloc (the attention entry point that allocates nothing: its plan and
split partials live in the library's per-GPU scratch array) against hx_varlen_attn with a
caller workspace, through the C ABI: two calls in a row, the second on a smaller tick,
each bit-identical to the workspace entry point and within the bf16 bound of the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helios_amd import _capi, synth
from tests.gpu_cases import DeviceTick, compare, say

pytestmark = pytest.mark.gpu


def _args(tick: DeviceTick, out: torch.Tensor, lse: torch.Tensor) -> list:
    w = tick.w
    return [
        tick.q.data_ptr(), tick.q.stride(0), tick.q.stride(1),
        tick.k_pool.data_ptr(), tick.v_pool.data_ptr(), tick.k_pool.stride(1), tick.k_pool.stride(2),
        w.num_pages, w.page_size, tick.block_table.data_ptr(), tick.block_table.shape[1],
        tick.cu_seq_q.data_ptr(), tick.cu_seq_k.data_ptr(), tick.seqused_k.data_ptr(),
        w.batch, w.total_q, w.max_q, w.max_k, 0,
        w.n_q_heads, w.n_kv_heads, w.head_dim, 1 / math.sqrt(w.head_dim), -1, 0, _capi.HX_DTYPE_BF16,
        out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(),
    ]


def test_noalloc_matches_workspace_entry_on_two_calls(device):
    lib = _capi.lib()
    stream = torch.cuda.current_stream(device).cuda_stream
    ticks = [
        synth.small_mixed(91, batch=9, max_cached=3000, max_chunk=400, num_pages=128),  # split partials
        synth.small_mixed(92, batch=3, max_cached=600, max_chunk=90, num_pages=32),     # smaller
    ]
    for w in ticks:
        say("noalloc", w.name, "batch", w.batch, "rows", w.total_q, "max_k", w.max_k)
        tick = DeviceTick(w, torch.bfloat16, device)
        shape = (w.total_q, w.n_q_heads, w.head_dim)
        out_a = torch.full(shape, float("nan"), dtype=torch.bfloat16, device=device)
        lse_a = torch.full((w.n_q_heads, w.total_q), float("nan"), dtype=torch.float32, device=device)
        out_b, lse_b = torch.empty_like(out_a), torch.empty_like(lse_a)
        need = lib.hx_varlen_attn_workspace_bytes(w.batch, w.max_q, w.max_k, w.n_q_heads, w.n_kv_heads,
                                                  w.head_dim)
        assert 0 < need <= 128 << 20
        workspace = torch.empty(need + 256, dtype=torch.uint8, device=device)
        ws = workspace.data_ptr() + (-workspace.data_ptr()) % 256
        torch.cuda.synchronize()
        code = lib.hx_varlen_attn_noalloc(*_args(tick, out_a, lse_a), stream)
        assert code == _capi.HX_OK, _capi.strerror(code)
        code = lib.hx_varlen_attn(*_args(tick, out_b, lse_b), ws, need, stream)
        assert code == _capi.HX_OK, _capi.strerror(code)
        torch.cuda.synchronize()
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
        assert torch.equal(lse_a, lse_b)
        ref, ref_lse = tick.oracle()
        compare(out_a, ref, what=f"noalloc {w.name}")
        assert np.abs(lse_a.cpu().numpy() - ref_lse).max() < 5e-3


def test_noalloc_rejects_a_tick_beyond_the_scratch(device):
    """A tick whose plan and partials exceed the 128 MiB scratch array (64 decode rows of
    up to 2^20 keys: about 2.2 GB of split partials) is refused with HX_E_TOO_LARGE
    before anything is launched: the output keeps its bits."""
    lib = _capi.lib()
    stream = torch.cuda.current_stream(device).cuda_stream
    w = synth.small_mixed(93, batch=3, max_cached=600, max_chunk=90, num_pages=32)
    tick = DeviceTick(w, torch.bfloat16, device)
    batch, max_q, max_k = 64, 1, 1 << 20
    need = lib.hx_varlen_attn_workspace_bytes(batch, max_q, max_k, w.n_q_heads, w.n_kv_heads, w.head_dim)
    assert need > 128 << 20
    out = torch.full((w.total_q, w.n_q_heads, w.head_dim), float("nan"), dtype=torch.bfloat16, device=device)
    lse = torch.full((w.n_q_heads, w.total_q), float("nan"), dtype=torch.float32, device=device)
    before = out.clone()
    args = _args(tick, out, lse)
    args[14:18] = [batch, w.total_q, max_q, max_k]   # batch, total_q, max_q, max_k
    torch.cuda.synchronize()
    code = lib.hx_varlen_attn_noalloc(*args, stream)
    assert code == _capi.HX_E_TOO_LARGE, _capi.strerror(code)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), before.view(torch.int16))
