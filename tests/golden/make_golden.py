"""Write the golden fixtures in this directory (run from the repo root).

  c1_meta.json / c1_bf16.npz  configuration 1 (4 sequences, cached 37/256/300/611,
      one new token each, 16-page pool, seeded page permutation): the page tables,
      sha256 of the bf16 bits of every input, and the float64 attention output and
      lse for the bf16-rounded inputs after the new tokens are appended. The output
      is produced by the float64 oracle and accepted only if torch's
      scaled_dot_product_attention in float64 (the reference's dense CPU path, op for
      op) agrees to 1e-12.
  tiny_attention.json  tiny single-sequence cases evaluated by pure-Python loops
      (oracle.attention.brute_force_attention) for several masks.

The reference code itself is not imported or run: the fixtures come from the
restatement and are cross-checked against torch library routines.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from helios_amd import synth  # noqa: E402
from oracle import attention as oa  # noqa: E402
from oracle import dense_torch, kv_bytes  # noqa: E402

OUT = Path(__file__).resolve().parent


def c1_fixture(seed: int = 1) -> None:
    w = synth.c1(seed)
    x = synth.host_inputs(w, np.float32)
    sha = {}
    xb = {}
    for name, arr in x.items():
        t = torch.from_numpy(arr).to(torch.bfloat16)
        sha[name] = hashlib.sha256(t.view(torch.int16).numpy().tobytes()).hexdigest()
        xb[name] = t.to(torch.float64).numpy()
    kv_bytes.kv_append(xb["k_pool"], xb["v_pool"], w.write_slots(), xb["k_new"], xb["v_new"])
    out, lse = oa.paged_varlen_attention(xb["q"], xb["k_pool"], xb["v_pool"], w.cu_seq_q, w.k_lens, w.tables)
    q = torch.from_numpy(xb["q"]).permute(1, 0, 2)[None]
    ref = dense_torch.packed_attention(q, torch.from_numpy(xb["k_pool"]), torch.from_numpy(xb["v_pool"]),
                                       w.tables, w.cached, w.q_lens)[0].permute(1, 0, 2).numpy()
    err = float(np.abs(ref - out).max())
    if err > 1e-12:
        raise SystemExit(f"oracle and torch SDPA disagree by {err}")
    np.savez_compressed(OUT / "c1_bf16.npz", out=out.astype(np.float64), lse=lse.astype(np.float64))
    meta = {
        "seed": seed,
        "tables": w.tables,
        "k_lens": w.k_lens,
        "cached": w.cached,
        "write_slots": [int(s) for s in w.write_slots()],
        "input_sha256_bf16": sha,
        "max_abs_vs_torch_sdpa_f64": err,
    }
    (OUT / "c1_meta.json").write_text(json.dumps(meta, indent=1) + "\n")


def tiny_cases() -> None:
    cases = []
    specs = [((-1, 0), 3, 6, 4, 2, 4, 0.7), ((-1, -1), 2, 5, 2, 1, 4, 1.0),
             ((2, 0), 4, 7, 4, 1, 3, 0.5), ((1, 1), 3, 6, 2, 2, 4, 0.9),
             ((-1, 0), 1, 1, 2, 1, 4, 0.3), ((-1, 0), 5, 5, 4, 4, 2, 1.3)]
    for i, (window, n, L, hq, hkv, d, scale) in enumerate(specs):
        q = synth.normal(500 + i, (n, hq, d), np.float64)
        k = synth.normal(600 + i, (L, hkv, d), np.float64)
        v = synth.normal(700 + i, (L, hkv, d), np.float64)
        out = oa.brute_force_attention(q.tolist(), k.tolist(), v.tolist(), scale=scale, window=window)
        cases.append({"window": list(window), "scale": scale, "q": q.tolist(), "k": k.tolist(),
                      "v": v.tolist(), "out": out})
    (OUT / "tiny_attention.json").write_text(json.dumps(cases) + "\n")


if __name__ == "__main__":
    c1_fixture()
    tiny_cases()
    print("wrote", sorted(p.name for p in OUT.iterdir() if p.suffix in (".json", ".npz")))
