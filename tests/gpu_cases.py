"""Helpers shared by the GPU parity tests: seeded device inputs for a workload and
the float64 oracle's answer for the same (bf16/fp16-rounded) inputs."""

from __future__ import annotations

import sys

import numpy as np
import torch

from helios_amd import ops, synth
from oracle import attention as oa
from oracle import kv_bytes

MAX_ABS = 2e-2   # tolerance of bf16 attention output vs the fp64 oracle (max |err|)
MEAN_ABS = 2e-3  # and mean |err|
# fp16 carries 3 more mantissa bits than bf16, so its bound is 8x tighter at the same
# headroom over one rounding of the output (|o| up to about 4 in these cases). Split
# partials stored in bf16 for an fp16 run (an 8-bit mantissa) exceed it on
# sharp-softmax rows, where the output is a single V row.
FP16_MAX_ABS = 4e-3
FP16_MEAN_ABS = 3e-4


def tolerance(dtype: torch.dtype) -> tuple[float, float]:
    """(max-abs, mean-abs) bound of attention output in ``dtype`` against the oracle."""
    return (FP16_MAX_ABS, FP16_MEAN_ABS) if dtype == torch.float16 else (MAX_ABS, MEAN_ABS)


def say(*parts) -> None:
    print("[case]", *parts, file=sys.stderr, flush=True)


class DeviceTick:
    """Inputs of one workload on the device, new tokens already appended."""

    def __init__(self, w: synth.Workload, dtype: torch.dtype, device: torch.device, *,
                 pool_on_device: bool = False):
        self.w = w
        self.dtype = dtype
        self.device = device
        s = w.seed * 7919
        T = w.total_q
        self.q = torch.from_numpy(synth.normal(s + 1, (T, w.n_q_heads, w.head_dim))).to(dtype).to(device)
        self.k_new = torch.from_numpy(synth.normal(s + 2, (T, w.n_kv_heads, w.head_dim))).to(dtype).to(device)
        self.v_new = torch.from_numpy(synth.normal(s + 3, (T, w.n_kv_heads, w.head_dim))).to(dtype).to(device)
        self.pool_on_device = pool_on_device
        self.k_pool, self.v_pool = self.fresh_pools()
        self.block_table = torch.from_numpy(w.block_table()).to(device)
        self.cu_seq_q = torch.tensor(w.cu_seq_q, dtype=torch.int32, device=device)
        self.cu_seq_k = torch.tensor(w.cu_seq_k, dtype=torch.int32, device=device)
        self.seqused_k = torch.tensor(w.k_lens, dtype=torch.int32, device=device)
        self.write_slots = torch.from_numpy(w.write_slots()).to(device)
        ops.kv_append(self.k_pool, self.v_pool, self.write_slots, self.k_new, self.v_new)

    def fresh_pools(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The tick's K and V pools before the append (the same bits every call)."""
        w, s, dtype, device = self.w, self.w.seed * 7919, self.dtype, self.device
        shape = (w.num_pages, w.page_size, w.n_kv_heads, w.head_dim)
        if self.pool_on_device:
            g = torch.Generator(device=device)
            g.manual_seed(s + 4)
            k = torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)
            v = torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)
            return k, v
        return (torch.from_numpy(synth.normal(s + 4, shape)).to(dtype).to(device),
                torch.from_numpy(synth.normal(s + 5, shape)).to(dtype).to(device))

    def plan(self, *, window=(-1, 0)) -> ops.VarlenAttnPlan:
        w = self.w
        return ops.VarlenAttnPlan(
            self.cu_seq_q, self.cu_seq_k, self.seqused_k, total_q=w.total_q, max_q=w.max_q,
            max_k=w.max_k, n_q_heads=w.n_q_heads, n_kv_heads=w.n_kv_heads,
            head_dim=w.head_dim, page_size=w.page_size,
            block_table_stride=self.block_table.shape[1], window=window,
            q_lens=w.q_lens, k_lens=w.k_lens)

    def attend(self, *, window=(-1, 0), exact_grid=False, return_lse=False):
        w = self.w
        if exact_grid:
            plan = self.plan(window=window)
            res = plan.run(self.q, self.k_pool, self.v_pool, self.block_table, return_lse=return_lse)
            assert plan.error_word() == 0
            return res
        aux = ops.AuxRequest(lse=True) if return_lse else None
        return ops.varlen_attn(self.q, self.k_pool, self.v_pool, self.cu_seq_q, self.cu_seq_k,
                               w.max_q, w.max_k, window_size=window,
                               enable_gqa=w.n_q_heads > w.n_kv_heads, seqused_k=self.seqused_k,
                               block_table=self.block_table, num_splits=1, return_aux=aux)

    def oracle(self, *, window=(-1, 0), rows=None):
        """float64 oracle on the device's rounded inputs, reading only the used pages."""
        w = self.w
        used = sorted({p for t, L in zip(w.tables, w.k_lens)
                       for p in t[: (L + w.page_size - 1) // w.page_size]})
        remap = {p: i for i, p in enumerate(used)}
        idx = torch.tensor(used, dtype=torch.long, device=self.device)
        kp = self.k_pool.index_select(0, idx).float().cpu().numpy()
        vp = self.v_pool.index_select(0, idx).float().cpu().numpy()
        tables = [[remap.get(p, 0) for p in t] for t in w.tables]
        q = self.q.float().cpu().numpy()
        return oa.paged_varlen_attention(q, kp, vp, w.cu_seq_q, w.k_lens, tables, window=window, rows=rows)


def host_append_reference(w: synth.Workload, dtype) -> dict[str, np.ndarray]:
    """Host copies (float64) of the rounded inputs with the new tokens appended."""
    x = synth.host_inputs(w, np.float32)
    xr = {n: torch.from_numpy(a).to(dtype).to(torch.float64).numpy() for n, a in x.items()}
    kv_bytes.kv_append(xr["k_pool"], xr["v_pool"], w.write_slots(), xr["k_new"], xr["v_new"])
    return xr


def compare(got: torch.Tensor, ref: np.ndarray, *, what: str, max_abs=None, mean_abs=None,
            rows: np.ndarray | None = None) -> tuple[float, float]:
    """Assert ``got`` is within the bound of its dtype (``tolerance``) of ``ref``."""
    d_max, d_mean = tolerance(got.dtype)
    max_abs = d_max if max_abs is None else max_abs
    mean_abs = d_mean if mean_abs is None else mean_abs
    g = got.float().cpu().numpy().astype(np.float64)
    if rows is not None:
        g, ref = g[rows], ref[rows]
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - ref)
    mx, mean = float(err.max()), float(err.mean())
    say(what, f"max_abs={mx:.3e} mean_abs={mean:.3e}")
    assert mx <= max_abs, f"{what}: max abs error {mx} > {max_abs}"
    assert mean <= mean_abs, f"{what}: mean abs error {mean} > {mean_abs}"
    return mx, mean
