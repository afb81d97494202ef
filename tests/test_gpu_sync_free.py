"""A steady-state tick never waits for the device.

The reference issues its attention calls stream-ordered from one scheduler thread and
tests that its decode path does not synchronise (tests/test_continuous_batching.py:499-518).
Here two back-to-back ticks of the full-model workload's shape run on the default GPU
path: Qwen3-4B width (32 / 8 heads, hidden 2560, FFN 9728) with 2 layers, 128 decoders
holding up to 16 pages of one shared 4096-token prefix (the shared-prefix cascade is
active) and one request prefilling a 1024-token chunk. Each tick is
``prepare_packed`` + ``forward_packed`` (device tick metadata, fused q/k norm + RoPE +
append, cascade attention, greedy heads) + ``advance_packed``.

The two ticks run with torch's sync debug mode set to "error" (a blocking copy, a
stream or device synchronisation, an ``.item()`` raise) and with
``torch.cuda.synchronize`` and the ``synchronize`` methods of events and streams
replaced by functions that raise. One tick runs before them, so that first-use set-up
(library load, pinned staging, GEMM selection) is outside the check.
"""

from __future__ import annotations

import pytest
import torch

from helios_amd import synth
from helios_amd.config import Qwen3Config
from helios_amd.decoder import PagedQwen3Decoder
from helios_amd.paged_cache import KVPagePool, PackedBatchCache
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu


class _Waited(RuntimeError):
    pass


def _refuse(*_args, **_kwargs):
    raise _Waited("a tick waited for the device")


def test_two_cascade_ticks_never_wait(device, monkeypatch):
    config = Qwen3Config(n_layers=2)
    lengths, counts = synth.c5_lengths(5)
    pool = KVPagePool(config, synth.c5_pool_pages(lengths, counts) + 64, device=device)
    pool.storage.normal_(generator=torch.Generator(device=device).manual_seed(5))
    _prefix, caches = synth.shared_prefix_caches(pool, lengths)
    model = PagedQwen3Decoder(config, device, seed=5)
    tokens = sum(counts)
    g = torch.Generator(device=device).manual_seed(53)
    inputs = [torch.randint(0, config.vocab_size, (1, tokens), generator=g, device=device) for _ in range(3)]
    batch = PackedBatchCache(caches)

    def tick(i):
        batch.prepare_packed(counts)
        assert batch._cascade is not None, "the tick should take the shared-prefix cascade"
        cascade = batch._cascade
        ids = model.forward_packed(inputs[i], batch, greedy=True)
        return ids, cascade

    say("sync-free: warm-up tick")
    tick(0)
    torch.cuda.synchronize()

    say("sync-free: two ticks under sync debug mode 'error'")
    monkeypatch.setattr(torch.cuda, "synchronize", _refuse)
    monkeypatch.setattr(torch.cuda.Event, "synchronize", _refuse)
    monkeypatch.setattr(torch.cuda.Stream, "synchronize", _refuse)
    torch.cuda.set_sync_debug_mode("error")
    try:
        results = [tick(1), tick(2)]
    finally:
        torch.cuda.set_sync_debug_mode("default")
        monkeypatch.undo()
    torch.cuda.synchronize()

    for ids, cascade in results:
        assert cascade.plan_a.error_word() == 0 and cascade.plan_b.error_word() == 0
        assert ids.shape == (len(counts),)
        assert bool(((ids >= 0) & (ids < config.vocab_size)).all())
    # Each tick committed its tokens: decoders grew by 3, the chunk request by 3 chunks.
    assert [c.length for c in caches] == [n + 3 * c for n, c in zip(lengths, counts)]
