"""Benchmark of the paged-KV hot path on one MI355X.

One step = one attention layer of a decode-only tick at Qwen3-4B shape: append the
new token's K/V of 64 sequences into a 2048-page x 256-token pool (bf16, 8 KV heads,
head_dim 128), then paged GQA decode attention of 32 query heads over context lengths
uniform in [512, 4096] (seeded), page tables drawn from a shuffled free list.
Synthetic N(0, 1) data. Steps rotate over four layer pools (2 GiB each) so no step
finds the previous step's pages in cache. The defaults (20 timed steps after 5 warm-up
steps) time the first ~3 ms of sustained decode work in a fresh process, when the shader
clock is still settling (it dips about 9 % between ~1.5 and ~6 ms into the load).

Printed JSON (one line):
  value     algorithmic HBM bytes per step / step time, in GB/s: every visible key's K
            and V row (8 heads x 128 x bf16, new token included), q read, o written,
            and the append's read + write of the new rows.
  roofline  the decode-attention kernel alone (its launches captured in a HIP graph,
            one per pool copy, replayed `steps` times between two HIP events after the
            timed loop; the kernel also performs the tick's KV append): its algorithmic
            bytes (K/V + q + o + the append's read and write) / its mean duration,
            against the 8 TB/s HBM3E peak. `traffic` = HBM bytes per launch measured
            by rocprofv3 FETCH_SIZE + WRITE_SIZE (scaled by a copy-kernel calibration)
            when profiles/decode_c2_pmc.json holds that measurement, else null.
  packed_tick  the mixed tick (32 decoders + 1024- and 992-token chunks): one layer's
            append + attention time, and tokens/s of 36 such layers (attention and KV
            work only; the model's GEMMs are not part of this path).
  long_context  the long-context tick (8 x 32768 keys with a shared 16-page prefix +
            a 4096-token chunk) and the 36-layer restore copy of 16 prefix pages.
  tick_metadata  host time of PackedBatchCache.prepare_packed with the reference's
            per-token lists and copies vs the metadata kernel, and the kernel's time.
  norm_rope_append  q/k RMSNorm + RoPE + KV append of one layer's new rows: the
            reference's torch op sequence vs the fused kernel (64 and 2048 rows).
  full_tick  a full random-init Qwen3-4B continuous-batching tick (128 decoders + a
            1024-token chunk, shared prefix pages): tokens/s and the attention step's
            share, for this build's path and for the reference's op sequence.
  cpu_baseline  the reference's dense-KV path (gather, repeat_interleave, SDPA) in
            torch fp32 on the host cores, on one full decode layer of the same tick.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
N_LAYERS_MODEL = 36
POOL_COPIES = 4


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-packed-tick", action="store_true")
    p.add_argument("--full-tick", action=argparse.BooleanOptionalAction, default=True,
                   help="full random-init Qwen3-4B tick (128 decoders + a 1024-token chunk)")
    p.add_argument("--only", default=None,
                   help="comma-separated side legs to run after the decode leg (packed_tick, "
                        "long_context, tick_metadata, norm_rope_append, greedy_heads, full_tick); "
                        "no CPU baseline. For profiling one leg.")
    p.add_argument("--pmc-pass", action="store_true",
                   help="short run for rocprofv3 counter collection: a calibration page "
                        "copy of known size, then a few decode steps")
    args = p.parse_args()
    if args.only is not None:
        args.only = [name.strip() for name in args.only.split(",") if name.strip()]
        unknown = [name for name in args.only if name not in SIDE_LEGS]
        if unknown:
            p.error(f"unknown legs {unknown}; choose from {list(SIDE_LEGS)}")
    return args


SIDE_LEGS = ("packed_tick", "long_context", "tick_metadata", "norm_rope_append", "greedy_heads", "full_tick")


class DecodeBench:
    """Device state of the decode tick: pools, new rows, metadata, plan."""

    def __init__(self, w, device, copies: int):
        import torch

        from helios_amd import ops

        self.w = w
        self.device = device
        shape = (w.num_pages, w.page_size, w.n_kv_heads, w.head_dim)
        g = torch.Generator(device=device)
        g.manual_seed(1234)
        self.k_pools, self.v_pools = [], []
        for _ in range(copies):
            self.k_pools.append(torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16))
            self.v_pools.append(torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16))
        T = w.total_q
        self.q = torch.randn((T, w.n_q_heads, w.head_dim), generator=g, device=device, dtype=torch.bfloat16)
        self.k_new = torch.randn((T, w.n_kv_heads, w.head_dim), generator=g, device=device, dtype=torch.bfloat16)
        self.v_new = torch.randn((T, w.n_kv_heads, w.head_dim), generator=g, device=device, dtype=torch.bfloat16)
        self.slots = torch.from_numpy(w.write_slots()).to(device)
        self.block_table = torch.from_numpy(w.block_table()).to(device)
        cu_q = torch.tensor(w.cu_seq_q, dtype=torch.int32, device=device)
        cu_k = torch.tensor(w.cu_seq_k, dtype=torch.int32, device=device)
        used = torch.tensor(w.k_lens, dtype=torch.int32, device=device)
        self.plan = ops.VarlenAttnPlan(
            cu_q, cu_k, used, total_q=T, max_q=w.max_q, max_k=w.max_k,
            n_q_heads=w.n_q_heads, n_kv_heads=w.n_kv_heads, head_dim=w.head_dim,
            page_size=w.page_size, block_table_stride=self.block_table.shape[1],
            window=(-1, 0), q_lens=w.q_lens, k_lens=w.k_lens)
        self.out = torch.empty_like(self.q)
        self.ops = ops

    def step(self, layer: int, events=None):
        """Append the new rows and attend, as PagedBatchCache.attend does. The decode
        launch appends: decode rows inside their split workgroups, and on a tick with
        chunk rows every row in workgroups added to that launch. A tick without decode
        rows appends first. events[0..3] bracket (append, decode, combine + chunk)."""
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        in_decode = self.plan.hints[0] != 0
        if events is not None:
            events[0].record()
        if not in_decode:
            self.ops.kv_append(kp, vp, self.slots, self.k_new, self.v_new)
        if events is not None:
            events[1].record()
        self.plan.run(self.q, kp, vp, self.block_table, out=self.out, phases=("decode",),
                      append=(self.k_new, self.v_new, self.slots) if in_decode else None)
        if events is not None:
            events[2].record()
        self.plan.run(self.q, kp, vp, self.block_table, out=self.out, phases=("combine", "chunk"))
        if events is not None:
            events[3].record()

    def phase(self, layer: int, name: str):
        """One kernel of the step alone: the decode kernel (with the appends of the step;
        "decode_only" without them), the chunk kernel or the combine kernel."""
        kp, vp = self.k_pools[layer], self.v_pools[layer]
        fused = name == "decode" and self.plan.hints[0] != 0
        self.plan.run(self.q, kp, vp, self.block_table, out=self.out,
                      phases=("decode",) if name == "decode_only" else (name,),
                      append=(self.k_new, self.v_new, self.slots) if fused else None)

    def append(self, layer: int):
        """The separate append kernel alone (what a tick with chunk rows runs first)."""
        self.ops.kv_append(self.k_pools[layer], self.v_pools[layer], self.slots, self.k_new, self.v_new)


GRAPH_WARM_S = 0.02     # replays before timing: the clocks ramp over the first milliseconds
GRAPH_TIMED_S = 0.02    # the timed replays span at least this long
GRAPH_REPLAY_S = 4e-4   # one replay holds enough launches to hide the host's replay cost


def graph_time_us(calls, replays: int) -> float:
    """Mean device time of one call of ``calls`` (each launching one kernel), measured by
    capturing them in one HIP graph and replaying it between two events on the current
    stream.

    - The graph holds ``calls`` repeated so that one replay lasts about GRAPH_REPLAY_S: a
      replay costs the host about 17 us, which a single short launch (a 64-row append,
      a combine) would otherwise measure instead of itself.
    - It is replayed ``replays`` times, or more so that the timed replays span
      GRAPH_TIMED_S, after GRAPH_WARM_S of untimed replays (a short MFMA-bound launch
      measured cold runs up to 15 % slower than in steady state)."""
    import math

    import torch

    def capture(repeat: int):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(repeat):
                for call in calls:
                    call()
        return graph

    def replay_s(graph, n: int) -> float:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(n):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e-3 / n

    for call in calls:   # warm (first launches, allocator) outside the graph
        call()
    torch.cuda.synchronize()
    probe = capture(1)
    probe.replay()
    torch.cuda.synchronize()
    device_s = replay_s(probe, 20)  # an upper bound on the calls' device time
    del probe
    repeat = max(1, min(64, math.ceil(GRAPH_REPLAY_S / device_s)))
    graph = capture(repeat)
    once = max(replay_s(graph, 1), 1e-6)
    for _ in range(math.ceil(GRAPH_WARM_S / once)):
        graph.replay()
    replays = max(replays, math.ceil(GRAPH_TIMED_S / once))
    us = replay_s(graph, replays) * 1e6 / (repeat * len(calls))
    del graph
    return us


def cpu_baseline(w, seconds_budget: float = 20.0):
    """The reference's dense-KV attention (oracle.dense_torch) on the host cores."""
    import numpy as np
    import torch

    from oracle import dense_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    used = sorted({p for t in w.tables for p in t})
    remap = {p: i for i, p in enumerate(used)}
    tables = [[remap[p] for p in t] for t in w.tables]
    g = torch.Generator().manual_seed(5)
    shape = (len(used), w.page_size, w.n_kv_heads, w.head_dim)
    kp = torch.randn(shape, generator=g)
    vp = torch.randn(shape, generator=g)
    q = torch.randn((1, w.n_q_heads, w.total_q, w.head_dim), generator=g)
    times = []
    with torch.inference_mode():
        for rep in range(2 + 5):
            t0 = time.perf_counter()
            dense_torch.packed_attention(q, kp, vp, tables, w.cached, w.q_lens)
            dt = time.perf_counter() - t0
            if rep >= 2:
                times.append(dt)
            if sum(times) > seconds_budget:
                break
    sec = statistics.median(times)
    nbytes = w.decode_bytes()
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    del np
    return {
        "value": round(nbytes / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"one full decode layer of the same tick ({w.batch} sequences, "
                   f"{sum(w.k_lens)} keys), torch fp32 dense-KV path "
                   f"(index_select gather, repeat_interleave, SDPA), median of {len(times)} "
                   f"reps: {sec * 1e3:.1f} ms/layer; CPU: {cpu_model}"),
    }


def cpu_tick_baseline(w, *, rows_kept: dict[int, int] | None = None, seconds_budget: float = 12.0):
    """The reference's packed CPU branch (paged_cache.py:521-546, restated op for op in
    oracle.dense_torch) on one layer of tick ``w``, timed on the host cores. With
    ``rows_kept`` = {sequence: n}, only the last n query rows of those sequences are
    computed (a bounded sample of a long chunk: the rows that see the most keys)."""
    import torch

    from oracle import dense_torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cached, counts = list(w.cached), list(w.q_lens)
    for b, n in (rows_kept or {}).items():
        cached[b] += counts[b] - n
        counts[b] = n
    ends = [c + n for c, n in zip(cached, counts)]
    used = sorted({p for t, e in zip(w.tables, ends) for p in t[: -(-e // w.page_size)]})
    remap = {p: i for i, p in enumerate(used)}
    tables = [[remap.get(p, 0) for p in t] for t in w.tables]
    g = torch.Generator().manual_seed(6)
    shape = (len(used), w.page_size, w.n_kv_heads, w.head_dim)
    kp, vp = torch.randn(shape, generator=g), torch.randn(shape, generator=g)
    q = torch.randn((1, w.n_q_heads, sum(counts), w.head_dim), generator=g)
    times = []
    with torch.inference_mode():
        for rep in range(2 + 5):
            t0 = time.perf_counter()
            dense_torch.packed_attention(q, kp, vp, tables, cached, counts)
            dt = time.perf_counter() - t0
            if rep >= 1:
                times.append(dt)
            if sum(times) > seconds_budget and len(times) >= 2:
                break
    sec = statistics.median(times)
    flops = 4 * w.n_q_heads * w.head_dim * sum(
        sum(min(e, c + i + 1) for i in range(n)) for c, n, e in zip(cached, counts, ends))
    return {"rows": sum(counts), "keys_visible": flops // (4 * w.n_q_heads * w.head_dim),
            "ms_per_layer": round(sec * 1e3, 1), "rows_per_s": round(sum(counts) / sec, 1),
            "gflops": round(flops / sec / 1e9, 2), "cores": cores, "reps": len(times)}


def packed_tick(device, steps: int = 200, warmup: int = 200):
    """One layer of the mixed tick: append + decode/chunk attention, wall time. About
    25 ms of warm-up steps go first: after the pools are filled the clocks take a few
    milliseconds to settle (5 warm-up steps and 30 timed ones read about 10 % high)."""
    import torch

    from helios_amd import synth

    w = synth.c3()
    b = DecodeBench(w, device, copies=2)
    for i in range(warmup):
        b.step(i % 2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        b.step(i % 2)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    assert b.plan.error_word() == 0, "attention plan reported an error"
    # per-kernel device time, each kernel's launches replayed from a HIP graph
    us = {name: graph_time_us([lambda i=i, name=name: b.phase(i, name) for i in range(2)], steps)
          for name in ("decode", "decode_only", "chunk", "combine")}
    us["append_separate"] = graph_time_us([lambda i=i: b.append(i) for i in range(2)], steps)
    res = {
        "workload": "c3: 32 decoders ctx U[1024,4096] + chunks 1024@0 and 992@512, bf16",
        "tokens": w.total_q,
        "us_per_layer": round(sec * 1e6, 2),
        "tick_ms_36_layers": round(sec * N_LAYERS_MODEL * 1e3, 3),
        "tokens_per_s_attention_only": round(w.total_q / (sec * N_LAYERS_MODEL), 1),
        "kernel_us": {k: round(v, 2) for k, v in us.items()},
        "decode_rows_us": round(us["decode_only"], 2),
        "decode_rows_gbs": round(w.decode_bytes() / (us["decode_only"] * 1e-6) / 1e9, 1),
        "chunk_rows_us": round(us["chunk"] + us["combine"], 2),
        "chunk_kernel_tflops": round(w.chunk_flops() / (us["chunk"] * 1e-6) / 1e12, 1),
        "chunk_kernel_mfma_frac": round(w.chunk_flops() / (us["chunk"] * 1e-6) / 2.5e15, 4),
        "chunk_rows_mfma_frac": round(w.chunk_flops() / ((us["chunk"] + us["combine"]) * 1e-6) / 2.5e15, 4),
    }
    del b
    torch.cuda.empty_cache()
    return res


def long_context(device, steps: int = 10, warmup: int = 3):
    """The long-context tick: 8 decoders at 32768 keys whose first 16 pages are shared,
    plus one 4096-token chunk at positions 4096-8191; and the restore of 16 prefix pages
    (K and V of all 36 layers) by page copy."""
    import torch

    from helios_amd import ops, synth

    w = synth.c4()
    b = DecodeBench(w, device, copies=1)
    for _ in range(warmup):
        b.step(0)
    torch.cuda.synchronize()
    assert b.plan.error_word() == 0, "attention plan reported an error"
    append_us = graph_time_us([lambda: b.append(0)], steps)
    decode_us = graph_time_us([lambda: b.phase(0, "decode_only")], steps)
    decode_append_us = graph_time_us([lambda: b.phase(0, "decode")], steps)
    chunk_kernel_us = graph_time_us([lambda: b.phase(0, "chunk")], steps)
    combine_us = graph_time_us([lambda: b.phase(0, "combine")], steps)
    chunk_us = chunk_kernel_us + combine_us
    del b
    torch.cuda.empty_cache()
    # restore copy: 16 prefix pages of every layer, keys and values, in the pool layout
    # KVPagePool allocates (one [2, layers, pages, ...] tensor, per-layer views)
    layers, n = N_LAYERS_MODEL, 16
    store = torch.randn((2, layers, 2 * n, w.page_size, w.n_kv_heads, w.head_dim), device=device,
                        dtype=torch.bfloat16)
    kl = [store[0, layer] for layer in range(layers)]
    vl = [store[1, layer] for layer in range(layers)]
    src, dst = list(range(n)), list(range(n, 2 * n))
    for _ in range(3):
        ops.kv_copy_pages(kl, vl, src, dst)
    cev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(10)]
    for a_, b_ in cev:
        a_.record()
        ops.kv_copy_pages(kl, vl, src, dst)
        b_.record()
    torch.cuda.synchronize()
    copy_us = statistics.median(a_.elapsed_time(b_) for a_, b_ in cev) * 1e3
    copy_bytes = 2 * layers * 2 * n * kl[0][0].numel() * 2
    # every copied page of every layer, K and V, bit for bit (72 tensors, one launch)
    for t in kl + vl:
        assert torch.equal(t[dst].view(torch.int16), t[src].view(torch.int16)), "restore copy differs"
    del kl, vl, store
    torch.cuda.empty_cache()
    # page gather (_gather_cpu's paged -> dense [1, 8, L, 128]) of one 32768-key sequence
    pool = torch.randn((160, w.page_size, w.n_kv_heads, w.head_dim), device=device, dtype=torch.bfloat16)
    pages = torch.randperm(160, device=device)[:128].to(torch.int32)
    length = 128 * w.page_size
    for _ in range(3):
        ops.kv_gather(pool, pages, length)
    gev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(10)]
    for a_, b_ in gev:
        a_.record()
        dense = ops.kv_gather(pool, pages, length)
        b_.record()
    torch.cuda.synchronize()
    gather_us = statistics.median(a_.elapsed_time(b_) for a_, b_ in gev) * 1e3
    gather_bytes = 2 * length * w.n_kv_heads * w.head_dim * 2
    assert torch.equal(dense[0, 3, 300], pool[int(pages[1]), 300 - 256, 3])
    del pool, dense
    torch.cuda.empty_cache()
    return {
        "workload": "c4: 8 decoders x 32768 keys (first 16 pages shared) + chunk 4096 rows at "
                    "positions 4096-8191; restore of 16 prefix pages x 36 layers x K/V",
        "append_us": round(append_us, 2),
        "decode_rows_us": round(decode_us, 2),
        "decode_launch_with_all_appends_us": round(decode_append_us, 2),
        "decode_rows_gbs_unique": round(w.decode_bytes() / (decode_us * 1e-6) / 1e9, 1),
        "chunk_rows_us": round(chunk_us, 2),
        "chunk_kernel_us": round(chunk_kernel_us, 2),
        "chunk_kernel_tflops": round(w.chunk_flops() / (chunk_kernel_us * 1e-6) / 1e12, 1),
        "chunk_kernel_mfma_frac": round(w.chunk_flops() / (chunk_kernel_us * 1e-6) / 2.5e15, 4),
        "chunk_rows_mfma_frac": round(w.chunk_flops() / (chunk_us * 1e-6) / 2.5e15, 4),
        "restore_copy_us": round(copy_us, 2),
        "restore_copy_gbs_rw": round(copy_bytes / (copy_us * 1e-6) / 1e9, 1),
        "gather_32k_keys_us": round(gather_us, 2),
        "gather_gbs_rw": round(gather_bytes / (gather_us * 1e-6) / 1e9, 1),
    }


def tick_metadata_leg(device, ticks: int = 20):
    """Per-tick metadata of PackedBatchCache.prepare_packed: built on the host (numpy,
    pageable copies) vs the metadata kernel, on the mixed tick (32 decoders + chunks
    of 1024 and 992) and on a 128-decoder + 1024-chunk tick (the full-model shape).
    Host time per prepare_packed call (what the scheduler thread waits for) and the
    kernel's own time."""
    import numpy as np
    import torch

    from helios_amd.config import Qwen3Config
    from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedKVCache

    config = Qwen3Config(n_layers=1)
    rng = np.random.default_rng(7)
    shapes = {
        "c3_mixed_tick": ([int(x) for x in rng.integers(1023, 4096, 32)] + [0, 512], [1] * 32 + [1024, 992]),
        "decoders128_chunk1024": ([int(x) for x in rng.integers(1023, 8192, 128)] + [0], [1] * 128 + [1024]),
    }
    out = {}
    for name, (lengths, counts) in shapes.items():
        res = {"sequences": len(counts), "tokens": sum(counts)}
        for mode in ("host_numpy", "device_kernel"):
            pages = sum(-(-(n + c * (ticks + 2)) // 256) for n, c in zip(lengths, counts)) + 8
            pool = KVPagePool(config, pages, device=device)
            caches = []
            for n in lengths:
                cache = PagedKVCache(pool, config.context_length)
                cache.pages.extend(pool.acquire(-(-n // 256)))
                cache.length = n
                caches.append(cache)
            batch = PackedBatchCache(caches, device_metadata=mode == "device_kernel")
            times = []
            for i in range(ticks + 2):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                batch.prepare_packed(counts)
                t1 = time.perf_counter()
                batch.advance_packed()
                if i >= 2:
                    times.append(t1 - t0)
            torch.cuda.synchronize()
            res[f"{mode}_us"] = round(statistics.median(times) * 1e6, 1)
            if mode == "device_kernel":
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                batch.prepare_packed(counts)
                seq = batch._device_meta.last["seq"]
                ev[0].record()
                from helios_amd import ops
                ops.tick_metadata(seq, batch.block_table, 256, total_q=sum(counts),
                                  cu_seq_q=batch.cu_seq_q, cu_seq_k=batch.cu_seq_k,
                                  seqused_k=batch.seqused_k, write_slots=batch.write_slots,
                                  positions=batch.positions[0], logit_indices=batch.logit_indices,
                                  n_logits=len(counts))
                ev[1].record()
                torch.cuda.synchronize()
                res["kernel_us"] = round(ev[0].elapsed_time(ev[1]) * 1e3, 2)
            del batch, caches, pool
            torch.cuda.empty_cache()
        out[name] = res
    return out


def _graph_time_us(fn, reps: int, per_graph: int = 10) -> tuple[float, float]:
    """(device µs per call, host µs per eager call) of ``fn``. Device time: ``per_graph``
    calls captured in a HIP graph (on a default-priority side stream) and replayed, so
    host launch overhead does not leave the GPU idle between them."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            fn()
    graph.replay()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record()
        graph.replay()
        b.record()
    torch.cuda.synchronize()
    device_us = statistics.median(a.elapsed_time(b) for a, b in ev) * 1e3 / per_graph
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    del graph
    return round(device_us, 2), round((t1 - t0) / reps * 1e6, 1)


def norm_rope_leg(device, reps: int = 50):
    """q_norm/k_norm + RoPE + KV append of one layer's new rows: the reference's torch op
    sequence (layers.py:146-160, then _write's two index_copy_) vs the fused kernel, for
    the 64-row decode tick and the 2048-row mixed tick."""
    import torch

    from helios_amd import ops
    from oracle import dense_torch

    d, hq, hkv = 128, 32, 8
    cos, sin = dense_torch.rope_parameters(d, 40960, 1_000_000.0)
    cos, sin = cos.to(device), sin.to(device)
    g = torch.Generator(device=device).manual_seed(3)
    out = {}
    for rows in (64, 2048):
        proj = torch.randn((1, rows, (hq + 2 * hkv) * d), generator=g, device=device).to(torch.bfloat16)
        q = proj[..., : hq * d].view(1, rows, hq, d)
        k = proj[..., hq * d:(hq + hkv) * d].view(1, rows, hkv, d)
        v = proj[..., (hq + hkv) * d:].view(1, rows, hkv, d)
        wq = torch.ones(d, device=device)
        wk = torch.ones(d, device=device)
        positions = torch.randint(0, 8192, (1, rows), generator=g, device=device)
        k_pool = torch.zeros((2048, 256, hkv, d), device=device, dtype=torch.bfloat16)
        v_pool = torch.zeros_like(k_pool)
        slots = torch.randperm(2048 * 256, generator=g, device=device)[:rows]

        def reference():
            qq = dense_torch.apply_rope(dense_torch.rms_norm(q.transpose(1, 2), wq, 1e-6), cos, sin, positions)
            kk = dense_torch.apply_rope(dense_torch.rms_norm(k.transpose(1, 2), wk, 1e-6), cos, sin, positions)
            pk = kk.transpose(1, 2).reshape(-1, hkv, d)
            pv = v.reshape(-1, hkv, d)
            k_pool.view(-1, hkv, d).index_copy_(0, slots, pk)
            v_pool.view(-1, hkv, d).index_copy_(0, slots, pv)
            return qq

        def fused():
            return ops.qk_norm_rope_append(q[0], k[0], v[0], wq, wk, cos, sin, positions, k_pool,
                                           v_pool, slots, 1e-6)

        res = {}
        for name, fn in (("reference_ops", reference), ("fused_kernel", fused)):
            res[f"{name}_gpu_us"], res[f"{name}_host_us"] = _graph_time_us(fn, reps)
        nbytes = rows * (hq + 2 * hkv) * d * 2 * 2 + rows * 2 * d * 4 * 2
        res["fused_gbs"] = round(nbytes / (res["fused_kernel_gpu_us"] * 1e-6) / 1e9, 1)
        out[f"rows_{rows}"] = res
        del k_pool, v_pool, proj
        torch.cuda.empty_cache()
    return out


def greedy_heads_leg(device, reps: int = 30):
    """The tick's greedy heads at the Qwen3-4B shape (hidden 2560, tied vocab 151936):
    the reference's sequence (index_select, RMSNorm, Linear to bf16 logits, argmax;
    model.py:108-110, engine.py:470-473) vs the fused final-norm / logits / argmax
    kernels, for 1, 64 and 129 logit rows of a 1152-row tick."""
    import torch

    from helios_amd import ops
    from oracle import dense_torch

    hidden, vocab, rows = 2560, 151936, 1152
    g = torch.Generator(device=device).manual_seed(7)
    x = torch.randn((rows, hidden), generator=g, device=device).to(torch.bfloat16)
    emb = (0.02 * torch.randn((vocab, hidden), generator=g, device=device)).to(torch.bfloat16)
    w = torch.ones(hidden, device=device)
    weight_bytes = vocab * hidden * 2
    out = {"weight_bytes": weight_bytes}
    for n in (1, 64, 129):
        idx = torch.arange(rows - n, rows, device=device)

        def reference():
            h = dense_torch.rms_norm(x.index_select(0, idx), w, 1e-6)
            return torch.nn.functional.linear(h, emb).argmax(dim=-1)

        def fused():
            return ops.final_norm_logits_argmax(x, idx, w, emb, 1e-6).token_ids

        same = bool(torch.equal(reference(), fused()))
        res = {"same_ids": same}
        for name, fn in (("reference_ops", reference), ("fused_kernels", fused)):
            res[f"{name}_gpu_us"], res[f"{name}_host_us"] = _graph_time_us(fn, reps)
        t = res["fused_kernels_gpu_us"] * 1e-6
        res["fused_weight_gbs"] = round(weight_bytes / t / 1e9, 1)
        res["fused_hbm_frac"] = round(weight_bytes / t / 1e9 / HBM_PEAK_GBS, 4)
        res["fused_tflops"] = round(2.0 * n * hidden * vocab / t / 1e12, 1)
        out[f"rows_{n}"] = res
    del emb
    torch.cuda.empty_cache()
    return out


def full_tick_leg(device, ticks: int = 4, seed: int = 5):
    """Full random-init Qwen3-4B forward of one continuous-batching tick: 128 decoders
    (contexts uniform in 1024-8192, each sharing up to 16 pages of a 4096-token system
    prefix) plus one 1024-token prefill chunk that also starts from the shared prefix;
    1152 packed tokens, one logit row per sequence, greedy token ids out. Every tick is
    rolled back with truncate() so each timed tick is the same. Reports tokens/s of the
    whole tick and the attention step's share (q/k norm + RoPE + KV append + paged
    attention), for this build's path (metadata kernel, fused norm/RoPE/append,
    shared-prefix cascade, fused final-norm/logits/argmax) and for the reference's
    sequence on the same attention kernels (host-built metadata, torch norm/RoPE,
    attend, every row reading its own prefix pages, bf16 logits then argmax)."""
    import torch

    from helios_amd import synth
    from helios_amd.config import Qwen3Config
    from helios_amd.decoder import PagedQwen3Decoder
    from helios_amd.paged_cache import KVPagePool, PackedBatchCache

    config = Qwen3Config()
    lengths, counts = synth.c5_lengths(seed)
    ctx = lengths[:-1]
    model = PagedQwen3Decoder(config, device, seed=seed)
    pool = KVPagePool(config, synth.c5_pool_pages(lengths, counts), device=device)
    g = torch.Generator(device=device).manual_seed(seed)
    pool.storage.normal_(generator=g)
    prefix, caches = synth.shared_prefix_caches(pool, lengths)
    tokens = sum(counts)
    input_ids = torch.randint(0, config.vocab_size, (1, tokens), generator=g, device=device)

    def tick(batch, fused, events=None):
        batch.prepare_packed(counts)
        ids = model.forward_packed(input_ids, batch, fused_rope=fused, attention_events=events, greedy=True)
        for cache, n in zip(caches, lengths):
            cache.truncate(n)
        return ids

    res = {"workload": "Qwen3-4B random-init bf16, 36 layers: 128 decoders ctx U[1024,8192] "
                       "sharing <=16 pages of a 4096-token prefix + one 1024-token chunk after "
                       "that prefix; 1152 packed tokens", "tokens": tokens}
    picks = {}
    for name, device_meta, fused in (("this_build", True, True), ("reference_sequence", False, False)):
        batch = PackedBatchCache(caches, device_metadata=device_meta, prefix_cascade=device_meta)
        for _ in range(2):
            tick(batch, fused)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(ticks):
            ids = tick(batch, fused)
        torch.cuda.synchronize()
        sec = (time.perf_counter() - t0) / ticks
        events = []
        tick(batch, fused, events)
        torch.cuda.synchronize()
        attn_ms = sum(a.elapsed_time(b) for a, b in events)
        res[name] = {
            "ms_per_tick": round(sec * 1e3, 3),
            "tokens_per_s": round(tokens / sec, 1),
            "decode_tokens_per_s": round(len(ctx) / sec, 1),
            "attention_ms_per_tick": round(attn_ms, 3),
            "attention_share": round(attn_ms / (sec * 1e3), 4),
        }
        assert bool(((ids >= 0) & (ids < config.vocab_size)).all())
        picks[name] = ids
        del batch
    # How far this build's greedy picks are from the reference sequence's own maximum:
    # the two forwards round differently (attention order, fused RoPE, cascade merge), so
    # near-ties of a random-init model's flat logits may resolve differently.
    batch = PackedBatchCache(caches, device_metadata=False, prefix_cascade=False)
    batch.prepare_packed(counts)
    ref_logits = model.forward_packed(input_ids, batch, fused_rope=False).float()
    for cache, n in zip(caches, lengths):
        cache.truncate(n)
    top = ref_logits.max(dim=-1).values
    gap = top - ref_logits.gather(1, picks["this_build"].unsqueeze(1))[:, 0]
    res["greedy_vs_reference_sequence"] = {
        "same_ids": round(float((picks["this_build"] == picks["reference_sequence"]).float().mean()), 4),
        "max_logit_gap_of_picks": round(float(gap.max()), 5),
        "max_logit_mean": round(float(top.mean()), 4),
        "top2_gap_median": round(float((top - ref_logits.topk(2, dim=-1).values[:, 1]).median()), 5),
    }
    del batch
    del model, pool, caches, prefix
    torch.cuda.empty_cache()
    return res


def pmc_pass(device):
    """Counter-collection run: a page copy of known size, then decode-tick steps, then
    mixed-tick and long-context steps (their chunk launches carry the MFMA counters)."""
    import torch

    from helios_amd import ops, synth

    layers = 4
    pools = [torch.zeros((256, 256, 8, 128), dtype=torch.bfloat16, device=device) for _ in range(layers)]
    src, dst = list(range(0, 64)), list(range(128, 192))
    for _ in range(3):
        ops.kv_copy_pages(pools, None, src, dst)
    torch.cuda.synchronize()
    copy_bytes = layers * 64 * pools[0][0].numel() * 2
    del pools
    b = DecodeBench(synth.c2(), device, copies=POOL_COPIES)
    for i in range(8):
        b.step(i % POOL_COPIES)
    torch.cuda.synchronize()
    decode_bytes = b.w.decode_bytes()
    del b
    chunk_flops = {}
    for name in ("c3", "c4"):
        w = getattr(synth, name)()
        b = DecodeBench(w, device, copies=1)
        for _ in range(3):
            b.step(0)
        torch.cuda.synchronize()
        chunk_flops[name] = w.chunk_flops()
        del b
        torch.cuda.empty_cache()
    print(json.dumps({"pmc_pass": True, "copy_read_bytes_per_dispatch": copy_bytes,
                      "copy_write_bytes_per_dispatch": copy_bytes,
                      "decode_algorithmic_bytes": decode_bytes,
                      "chunk_flops": chunk_flops}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the paged-KV "
              "path has no multi-GPU form in this build.", file=sys.stderr)
        sys.exit(2)
    import torch

    from helios_amd import _capi, synth

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm device", file=sys.stderr)
        sys.exit(1)
    _capi.lib()
    device = torch.device("cuda", 0)
    if args.pmc_pass:
        pmc_pass(device)
        return

    w = synth.c2()
    b = DecodeBench(w, device, copies=POOL_COPIES)
    step_bytes = w.decode_bytes() + w.append_bytes()
    for i in range(args.warmup):
        b.step(i % POOL_COPIES)
    # Timed region: K steps, wall clock, synchronised on both sides (no events inside).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        b.step(i % POOL_COPIES)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert b.plan.error_word() == 0, "attention plan reported an error"
    ms_per_step = elapsed * 1e3 / args.steps
    # Kernel timing: each kernel launched back to back from a replayed HIP graph (one
    # launch per pool copy, the graph replayed many times) between two HIP events on the
    # stream the launches run on, so the mean carries no host launch gaps.
    decode_us = graph_time_us([lambda i=i: b.phase(i, "decode") for i in range(POOL_COPIES)], args.steps)
    combine_us = graph_time_us([lambda i=i: b.phase(i, "combine") for i in range(POOL_COPIES)], args.steps)
    append_us = graph_time_us([lambda i=i: b.append(i) for i in range(POOL_COPIES)], args.steps)
    kernel_bytes = w.decode_bytes() + w.append_bytes()  # the decode kernel appends too
    achieved = kernel_bytes / (decode_us * 1e-6) / 1e9
    traffic = None
    pmc = ROOT / "profiles" / "decode_c2_pmc.json"
    if pmc.exists():
        try:
            traffic = json.loads(pmc.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    result = {
        "metric": "paged decode attn HBM GB/s (% peak) + packed-tick tokens/s, Qwen3-4B shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/q, seeded context lengths and page tables",
        "config": {
            "workload": "decode-only tick, one attention layer incl. KV append: 64 seqs, ctx "
                        "U[512,4096] seeded, 32q/8kv heads, d=128, 2048-page x 256-token pool",
            "batch": w.batch,
            "keys": sum(w.k_lens),
            "step_bytes": step_bytes,
            "pct_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "ms_per_tick_36_layers": round(ms_per_step * N_LAYERS_MODEL, 4),
            "kernel_us": {"kv_append_separate": round(append_us, 2),
                          "decode_attention_with_append": round(decode_us, 2),
                          "split_combine": round(combine_us, 2)},
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_kernel (paged split-K decode attention with the fused KV append)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": kernel_bytes,
        },
    }
    del b
    torch.cuda.empty_cache()
    legs = {
        "packed_tick": packed_tick,
        "long_context": long_context,
        "tick_metadata": tick_metadata_leg,
        "norm_rope_append": norm_rope_leg,
        "greedy_heads": greedy_heads_leg,
        "full_tick": full_tick_leg,
    }
    if args.only is not None:
        chosen = args.only
    else:
        chosen = [] if args.no_packed_tick else list(legs)[:5]
        if args.full_tick:
            chosen.append("full_tick")
    for name in chosen:
        result[name] = legs[name](device)
    if args.only is None and not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w)
        # The same dense-KV path on the mixed tick (whole layer) and on the long-context
        # tick (its 8 decode rows and the last 512 of its 4096 chunk rows).
        c4 = synth.c4()
        result["cpu_baseline_ticks"] = {
            "c3_mixed_tick": cpu_tick_baseline(synth.c3()),
            "c4_sample_decoders_and_last_512_chunk_rows": cpu_tick_baseline(c4, rows_kept={8: 512}),
        }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
