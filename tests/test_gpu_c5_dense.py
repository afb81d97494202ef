"""The full-model tick's sharing pattern at Qwen3-4B width, end to end, against a dense fp32
model on the GPU.

The reference states that its paged path equals the dense-KV model for a restored prefix
continuation (tests/test_paged_attention.py:153-178). Here the paged side is this build's
whole tick at Qwen3-4B width (hidden 2560, 32 / 8 heads, head_dim 128, FFN 9728, vocab
151936) with 4 layers, random-init bf16 weights:

1. one request prefills a 4096-token prefix (one 4096-row chunk);
2. 80 requests restore its 16 pages zero-copy (shared page handles, as a prefix-cache hit
   leaves them) and prefill suffixes of 1 to 150 tokens in one packed tick;
3. a tick of the 80 as decode rows, sharing the prefix pages (the shared-prefix cascade
   runs with levels of more than 64 rows), plus one more restored request prefilling a
   1024-token chunk after the prefix;
4. a decode tick of all 81.

Every logit row of every tick is compared with an independent dense forward in torch
fp32 on the GPU (the reference's layer math, layers.py:13-27, :131-191, :202-232, with
dense K/V kept per request): no HIP kernel of this build takes part in it.

The bound is stated against bf16 rounding itself: the same dense forward with the
reference's bf16 roundings (bf16 weights, activations, K/V, norm and RoPE outputs,
attention in fp32 on bf16 inputs) deviates from the fp32 one by some amount E_ref per
tick; this build must stay within 2 E_ref (plus 1e-3 of the logit scale). Its own extra
roundings (bf16 softmax weights in P V, split partials stored in bf16) are of the same
order. A request reading the wrong prefix page, a RoPE position off by one, a merge
that drops a level or a key appended to the wrong slot moves logits by O(1) of their scale.
"""

from __future__ import annotations

import math

import pytest
import torch

from helios_amd.config import Qwen3Config
from helios_amd.decoder import PagedQwen3Decoder
from helios_amd.paged_cache import KVPagePool, PackedBatchCache, PagedKVCache, _PrefixCascade
from tests.gpu_cases import say

pytestmark = pytest.mark.gpu

PREFIX = 4096
DECODERS = 80
CHUNK = 1024
FACTOR = 2.0       # this build's error against fp32, at most FACTOR x bf16 dense's (+ SLACK)
SLACK = 1e-3       # of the logit scale
ABS_REL = 3e-2     # and never above 3 % of the row's largest logit


class DenseModel:
    """Dense-KV forward of ``model``'s weights in torch on the GPU: fp32 throughout, or
    with the reference's bf16 roundings (``bf16=True``). Per-request K/V lists grow as
    tokens run through it."""

    def __init__(self, model: PagedQwen3Decoder, *, bf16: bool) -> None:
        self.m = model
        self.cfg = model.config
        self.bf16 = bf16
        self.w = [{k: v.float() for k, v in layer.items()} for layer in model.layers]
        self.emb = model.embedding.float()
        self.final = model.final_norm.float()

    def r(self, t: torch.Tensor) -> torch.Tensor:
        return t.to(torch.bfloat16).float() if self.bf16 else t

    def rms(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        return self.r(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.cfg.rms_norm_eps) * w)

    def run(self, state: list, ids: list[int], start: int) -> torch.Tensor:
        """Tokens ``ids`` at positions start.. after the request's K/V in ``state`` (a list
        of per-layer (k, v) [hkv, S, d], extended in place); returns the logits of the
        last new row, fp32."""
        cfg, r = self.cfg, self.r
        hq, hkv, d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        T = len(ids)
        x = self.emb[torch.tensor(ids, device=self.emb.device)]
        cos = self.m.cos[start:start + T].float()
        sin = self.m.sin[start:start + T].float()
        half = d // 2

        def rope(v):
            return r(v * cos + torch.cat((-v[..., half:], v[..., :half]), -1) * sin)

        for li, w in enumerate(self.w):
            h = self.rms(x, w["input_norm"])
            qkv = r(h @ w["qkv"].t())
            q = qkv[:, :hq * d].reshape(T, hq, d).transpose(0, 1)
            k = qkv[:, hq * d:(hq + hkv) * d].reshape(T, hkv, d).transpose(0, 1)
            v = qkv[:, (hq + hkv) * d:].reshape(T, hkv, d).transpose(0, 1)
            q = rope(self.rms(q, w["q_norm"]))
            k = rope(self.rms(k, w["k_norm"]))
            if len(state) <= li:
                state.append((k, v))
            else:
                pk, pv = state[li]
                state[li] = (torch.cat((pk, k), 1), torch.cat((pv, v), 1))
            K, V = state[li]
            S = K.shape[1]
            G = hq // hkv
            qg = q.reshape(hkv, G * T, d)
            scores = (qg @ K.transpose(1, 2).contiguous()).reshape(hkv, G, T, S) / math.sqrt(d)
            visible = torch.arange(S, device=x.device)[None, :] <= (S - T + torch.arange(T, device=x.device))[:, None]
            p = torch.softmax(scores.masked_fill(~visible, float("-inf")), -1)
            ctx = (p.reshape(hkv, G * T, S) @ V).reshape(hq, T, d)
            ctx = r(ctx).transpose(0, 1).reshape(T, hq * d)
            x = r(x + r(ctx @ w["o"].t()))
            h = self.rms(x, w["post_norm"])
            gate, up = r(h @ w["gate_up"].t()).chunk(2, -1)
            act = r(r(torch.nn.functional.silu(gate)) * up)
            x = r(x + r(act @ w["down"].t()))
        return r(self.rms(x[-1:], self.final) @ self.emb.t())[0]


def _rel_errors(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    """(max over rows of max |err| / max |ref|, mean over rows of mean |err| / mean |ref|)."""
    err = (got.float() - ref).abs()
    row_max = err.amax(1) / ref.abs().amax(1)
    row_mean = err.mean(1) / ref.abs().mean(1)
    return float(row_max.max()), float(row_mean.mean())


def test_c5_sharing_pattern_matches_dense_fp32_model(device):
    config = Qwen3Config(n_layers=4)
    model = PagedQwen3Decoder(config, device, seed=7)
    gen = torch.Generator().manual_seed(17)

    def draw(n: int) -> list[int]:
        return torch.randint(0, config.vocab_size, (n,), generator=gen).tolist()

    suffix = torch.randint(1, 151, (DECODERS,), generator=gen).tolist()
    prefix_ids = draw(PREFIX)
    own = [draw(n) for n in suffix]
    step3, step4 = draw(DECODERS), draw(DECODERS + 1)
    chunk_ids = draw(CHUNK)
    pages = PREFIX // 256 + DECODERS * 2 + CHUNK // 256 + 16
    pool = KVPagePool(config, pages, device=device)

    def tick(caches, counts, tokens):
        batch = PackedBatchCache(caches)
        batch.prepare_packed(counts)
        out = model.forward_packed(torch.tensor([tokens], device=device), batch)
        return out, batch

    got = {}   # tick -> logits [rows, vocab]
    prefix = PagedKVCache(pool, config.context_length)
    got[1], _ = tick([prefix], [PREFIX], prefix_ids)
    snap = prefix.snapshot_block(0, PREFIX)
    decoders = []
    for _ in range(DECODERS):
        c = PagedKVCache(pool, config.context_length)
        c.restore_blocks([snap])
        decoders.append(c)
    assert decoders[0].pages[0] is prefix.pages[0]
    got[2], _ = tick(decoders, suffix, [t for seq in own for t in seq])
    late = PagedKVCache(pool, config.context_length)
    late.restore_blocks([snap])
    got[3], b3 = tick(decoders + [late], [1] * DECODERS + [CHUNK], step3 + chunk_ids)
    levels = _PrefixCascade.levels(b3, [1] * DECODERS + [CHUNK])
    assert b3._cascade is not None and max(len(m) for *_, m in levels) > 64
    got[4], _ = tick(decoders + [late], [1] * (DECODERS + 1), step4)
    torch.cuda.synchronize()

    results = {}
    for name, bf16 in (("fp32", False), ("bf16", True)):
        dense = DenseModel(model, bf16=bf16)
        pre_state: list = []
        rows = {1: [dense.run(pre_state, prefix_ids, 0)]}
        rows[2], rows[3], rows[4] = [], [], []
        for i in range(DECODERS):
            st = [(k.clone(), v.clone()) for k, v in pre_state]
            rows[2].append(dense.run(st, own[i], PREFIX))
            rows[3].append(dense.run(st, [step3[i]], PREFIX + suffix[i]))
            rows[4].append(dense.run(st, [step4[i]], PREFIX + suffix[i] + 1))
        st = [(k.clone(), v.clone()) for k, v in pre_state]
        rows[3].append(dense.run(st, chunk_ids, PREFIX))
        rows[4].append(dense.run(st, [step4[-1]], PREFIX + CHUNK))
        results[name] = {t: torch.stack(v) for t, v in rows.items()}
        del dense
    for t in (1, 2, 3, 4):
        truth = results["fp32"][t]
        e_ref, m_ref = _rel_errors(results["bf16"][t], truth)
        e_got, m_got = _rel_errors(got[t], truth)
        say(f"tick {t} ({truth.shape[0]} rows): this build max {e_got:.3e} mean {m_got:.3e}; "
            f"bf16 dense max {e_ref:.3e} mean {m_ref:.3e}")
        assert torch.isfinite(got[t]).all()
        assert e_got <= FACTOR * e_ref + SLACK, (t, e_got, e_ref)
        assert m_got <= FACTOR * m_ref + SLACK, (t, m_got, m_ref)
        assert e_got <= ABS_REL, (t, e_got)
