"""Python call surface of the MI355X paged-KV hot path.

``varlen_attn`` keeps the keyword surface the reference uses at
src/helios/runtime/qwen3/paged_cache.py:316-329 and :506-519
(torch 2.13 ``torch.nn.attention.varlen.varlen_attn`` with ``block_table=``), so
that module can import it in place of torch's. ``kv_append``, ``kv_copy_pages`` and
``kv_gather`` replace ``PagedBatchCache._write`` (paged_cache.py:335-345),
``KVCache.restore_blocks``' copy (cache.py:131-147) and ``_gather_cpu``
(paged_cache.py:405-414).

Every function validates its arguments on the host (ValueError, like
``_validate_attention_inputs`` at paged_cache.py:352-375), allocates outputs and
workspaces with ``torch.empty`` on the query's device (the caching allocator owns
them), and launches on ``torch.cuda.current_stream()`` without synchronising.
"""

from __future__ import annotations

import ctypes
import math
import os
from collections.abc import Sequence
from typing import NamedTuple

import torch

from helios_amd import _capi

_SUPPORTED = {torch.bfloat16: _capi.HX_DTYPE_BF16, torch.float16: _capi.HX_DTYPE_FP16}

# With HELIOS_AMD_CHECK_ERRORS=1 every attention run synchronises and raises RuntimeError
# when the kernels flagged bad metadata (a page id outside the pool, a length clamped to
# max_k / max_q / the table width, a malformed cu_seq_q, or a plan / run mismatch). Off by
# default: reading the flag is a device-to-host round trip per call, and the reference's
# hot path never synchronises (tests/test_continuous_batching.py:499-518). The kernels
# never read or write out of bounds either way.
CHECK_ERRORS = os.environ.get("HELIOS_AMD_CHECK_ERRORS", "") not in ("", "0")

_WERR_TEXT = {
    _capi.HX_WERR_BAD_PAGE: "a block-table page id outside the pool",
    _capi.HX_WERR_CLAMPED_LEN: "a sequence length beyond max_k, max_q or the block table",
    _capi.HX_WERR_BAD_CU_SEQ: "cu_seq_q not monotone or beyond the query rows",
    _capi.HX_WERR_GRID: "more work items than the launch grid covered",
    _capi.HX_WERR_PLAN_MISMATCH: "a run whose shape differs from its plan",
    _capi.HX_WERR_BAD_QUERY_ROW: "a query row map entry outside the query tensor",
}


def describe_error_word(word: int) -> str:
    """Text for the HX_WERR_* bits of an attention workspace error word."""
    parts = [text for bit, text in _WERR_TEXT.items() if word & bit]
    return "; ".join(parts) if parts else "no error"


class MergeParts(NamedTuple):
    """A shared-prefix cascade merge for ``VarlenAttnPlan.run(..., merge=...)``: member k
    is the decode row of sequence ``member_seq[k]`` (``member_of_seq[b]``: sequence b's
    member index or -1); its parts are rows ``part_idx[part_start[k]:part_start[k + 1]]``
    of ``level_out`` ``[A, H, 128]`` with log-sum-exps ``level_lse`` ``[H, A]``. All on the
    device; the int arrays are contiguous int32.

    ``level_plan``: the plan that produces ``level_out`` / ``level_lse``, when its run so
    far covered only its decode and chunk phases (``phases=("decode", "chunk")``, same
    stream): the merging run then does that plan's combine phase too, in workgroups added
    to its own decode launch, instead of a launch of its own.

    ``level_block_table`` (and ``level_query_rows``, int64 rows of the merging run's
    query): the level plan has not run at all and holds no decode rows; the merging run
    (all three phases, no append) runs its chunk items too, in one chunk launch with its
    own, ahead of its decode launch. ``level_out`` / ``level_lse`` are then outputs of
    that run (any contents on entry)."""

    level_out: torch.Tensor
    level_lse: torch.Tensor
    member_seq: torch.Tensor
    member_of_seq: torch.Tensor
    part_start: torch.Tensor
    part_idx: torch.Tensor
    level_plan: "VarlenAttnPlan | None" = None
    level_block_table: torch.Tensor | None = None
    level_query_rows: torch.Tensor | None = None


class AuxRequest(NamedTuple):
    """Auxiliary outputs of varlen_attn (same field as torch's AuxRequest)."""

    lse: bool = False


def _stream_ptr(device: torch.device) -> int:
    """The current stream's handle on ``device`` (the raw lookup: no Stream object)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    device = tensors[0].device
    if device.type != "cuda":
        raise RuntimeError(
            "helios_amd kernels run on a ROCm device only; got tensors on "
            f"{device}. There is no CPU fallback."
        )
    for t in tensors[1:]:
        if t.device != device:
            raise ValueError("All tensors must be on the same device.")
    return device


def _elem_bytes(t: torch.Tensor) -> int:
    return t.element_size()


# --------------------------------------------------------------------- KV append
def kv_append(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    write_slots: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
) -> None:
    """``k_cache.view(-1, Hkv, d).index_copy_(0, write_slots, keys)``, same for V.

    ``k_cache``/``v_cache``: pool tensors whose trailing dims are ``[Hkv, d]`` and
    that are contiguous (``[num_pages, page_size, Hkv, d]`` in the reference).
    ``keys``/``values``: ``[T, Hkv, d]`` with a contiguous last dim (any row/head
    strides). ``write_slots``: int64 ``[T]`` flat slot ids (page * page_size + offset).
    """
    device = _require_gpu(k_cache, v_cache, write_slots, keys, values)
    _check_append(k_cache, v_cache, write_slots, keys, values)
    n_kv, head_dim = keys.shape[1], keys.shape[2]
    write_slots = write_slots.contiguous()
    pool_rows = k_cache.numel() // (n_kv * head_dim)
    code = _capi.lib().hx_kv_append(
        k_cache.data_ptr(), v_cache.data_ptr(), pool_rows,
        keys.data_ptr(), keys.stride(0), keys.stride(1),
        values.data_ptr(), values.stride(0), values.stride(1),
        write_slots.data_ptr(), keys.shape[0],
        n_kv, head_dim, _elem_bytes(keys),
        _stream_ptr(device),
    )
    _capi.check(code, "hx_kv_append")


def _check_append(k_cache, v_cache, write_slots, keys, values) -> None:
    """Argument checks shared by kv_append and the fused append path."""
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise ValueError("Key and value pools must have identical shapes and dtypes.")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV pools must be contiguous.")
    if keys.ndim != 3 or values.shape != keys.shape:
        raise ValueError("Appended keys and values must be [tokens, kv_heads, head_dim].")
    n_kv, head_dim = keys.shape[1], keys.shape[2]
    if tuple(k_cache.shape[-2:]) != (n_kv, head_dim):
        raise ValueError("Appended K/V heads do not match the pool layout.")
    if keys.dtype != k_cache.dtype or values.dtype != k_cache.dtype:
        raise ValueError("Appended K/V dtype must match the pool dtype.")
    if write_slots.dtype != torch.int64 or write_slots.ndim != 1 or write_slots.shape[0] != keys.shape[0]:
        raise ValueError("write_slots must be int64 [tokens].")
    if keys.stride(2) != 1 or values.stride(2) != 1:
        raise ValueError("Appended K/V must have a contiguous head_dim.")


# ----------------------------------------------------- q/k norm + RoPE + append
def qk_norm_rope_append(
    queries: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    write_slots: torch.Tensor,
    eps: float,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """q_norm/k_norm + apply_rope of the new rows (layers.py:146-160) fused with the KV
    append (paged_cache.py:335-345).

    ``queries`` ``[T, Hq, 128]``, ``keys``/``values`` ``[T, Hkv, 128]`` (projection
    outputs; contiguous last dim, any row/head strides); ``q_norm_weight``/``k_norm_weight``
    fp32 ``[128]``; ``cos``/``sin`` fp32 ``[rope_rows, 128]``; ``positions`` int64 ``[T]``
    (flattened, e.g. ``PackedBatchCache.positions[0]``). Returns the normalised, rotated
    queries ``[T, Hq, 128]`` (``out`` if given); rotated keys and raw values land in the
    pools at ``write_slots``.
    """
    device = _require_gpu(queries, keys, values, q_norm_weight, k_norm_weight, cos, sin,
                          positions, k_cache, v_cache, write_slots)
    _check_append(k_cache, v_cache, write_slots, keys, values)
    if queries.ndim != 3 or queries.shape[0] != keys.shape[0] or queries.shape[2] != keys.shape[2]:
        raise ValueError("queries must be [tokens, q_heads, head_dim] matching the keys.")
    if queries.dtype != keys.dtype or queries.stride(2) != 1:
        raise ValueError("queries must share the K/V dtype and have a contiguous head_dim.")
    head_dim = queries.shape[2]
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w.dtype != torch.float32 or w.numel() != head_dim or not w.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 [head_dim] tensor.")
    if (cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape
            or cos.ndim != 2 or cos.shape[1] != head_dim or not cos.is_contiguous()
            or not sin.is_contiguous()):
        raise ValueError("cos/sin must be contiguous float32 [rows, head_dim] tables.")
    positions = positions.reshape(-1)
    if positions.dtype != torch.int64 or positions.numel() != queries.shape[0]:
        raise ValueError("positions must be int64 with one entry per row.")
    positions = positions.contiguous()
    if out is None:
        out = torch.empty(queries.shape, dtype=queries.dtype, device=device)
    elif out.shape != queries.shape or out.dtype != queries.dtype or out.stride(2) != 1:
        raise ValueError("out must match the queries' shape and dtype.")
    dtype = {torch.bfloat16: _capi.HX_DTYPE_BF16, torch.float16: _capi.HX_DTYPE_FP16}.get(queries.dtype)
    if dtype is None:
        raise ValueError("q/k/v must be bfloat16 or float16.")
    pool_rows = k_cache.numel() // (keys.shape[1] * head_dim)
    code = _capi.lib().hx_qk_norm_rope_append(
        queries.data_ptr(), queries.stride(0), queries.stride(1),
        keys.data_ptr(), keys.stride(0), keys.stride(1),
        values.data_ptr(), values.stride(0), values.stride(1),
        q_norm_weight.data_ptr(), k_norm_weight.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        positions.data_ptr(), queries.shape[0],
        queries.shape[1], keys.shape[1], head_dim, float(eps), dtype,
        out.data_ptr(), out.stride(0), out.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), pool_rows, write_slots.contiguous().data_ptr(),
        _stream_ptr(device),
    )
    _capi.check(code, "hx_qk_norm_rope_append")
    return out


# ------------------------------------------------------------ attention merge
def attn_merge(out: torch.Tensor, lse_out: torch.Tensor, o_a: torch.Tensor, lse_a: torch.Tensor,
               rows: torch.Tensor, parts: tuple[torch.Tensor, torch.Tensor] | None = None) -> None:
    """In place: merge attention results over disjoint key sets by log-sum-exp weights.

    Without ``parts``, ``(o_a[j], lse_a[:, j])`` merges into ``(out[rows[j]],
    lse_out[:, rows[j]])``. With ``parts = (part_start, part_idx)`` (int32 ``[n + 1]`` and
    ``[P]``), entry j merges the o_a rows ``part_idx[part_start[j]:part_start[j + 1]]``
    into ``out[rows[j]]`` in one pass. ``out`` ``[T, H, 128]`` and ``o_a`` ``[A, H, 128]``
    (contiguous last dim), ``lse_out`` fp32 ``[H, T]``, ``lse_a`` fp32 ``[H, A]``
    contiguous, ``rows`` int64 ``[n]`` without repeats. A part index outside ``[0, A)``
    is skipped."""
    device = _require_gpu(out, lse_out, o_a, lse_a, rows)
    if out.ndim != 3 or o_a.ndim != 3 or out.shape[1:] != o_a.shape[1:] or out.dtype != o_a.dtype:
        raise ValueError("out and o_a must be [rows, heads, head_dim] of one dtype.")
    if out.stride(2) != 1 or o_a.stride(2) != 1:
        raise ValueError("out and o_a need a contiguous head_dim.")
    n_a, heads = o_a.shape[0], o_a.shape[1]
    n = rows.numel()
    if lse_out.dtype != torch.float32 or tuple(lse_out.shape) != (heads, out.shape[0]) or not lse_out.is_contiguous():
        raise ValueError("lse_out must be contiguous float32 [heads, rows].")
    # The kernel bounds part indices by lse_a's row stride, so that stride must be o_a's
    # row count: lse_a contiguous [heads, n_a].
    if lse_a.dtype != torch.float32 or tuple(lse_a.shape) != (heads, n_a) or not lse_a.is_contiguous():
        raise ValueError("lse_a must be contiguous float32 [heads, rows].")
    if rows.dtype != torch.int64 or rows.ndim != 1 or not rows.is_contiguous():
        raise ValueError("rows must be contiguous int64 [n].")
    start_ptr = idx_ptr = None
    n_parts = 0
    if parts is None:
        if n != n_a:
            raise ValueError("without parts, rows must have one entry per o_a row.")
    else:
        part_start, part_idx = parts
        for name, t in (("part_start", part_start), ("part_idx", part_idx)):
            if t.dtype != torch.int32 or t.ndim != 1 or not t.is_contiguous() or t.device != device:
                raise ValueError(f"{name} must be a contiguous int32 vector on the device.")
        if part_start.numel() != n + 1:
            raise ValueError("part_start must have one entry per row plus one.")
        start_ptr, idx_ptr = part_start.data_ptr(), part_idx.data_ptr()
        n_parts = part_idx.numel()
    dtype = _SUPPORTED.get(out.dtype)
    if dtype is None:
        raise ValueError("attention outputs must be bfloat16 or float16.")
    code = _capi.lib().hx_attn_merge(
        out.data_ptr(), out.stride(0), out.stride(1), lse_out.data_ptr(), out.shape[0],
        o_a.data_ptr(), o_a.stride(0), o_a.stride(1), lse_a.data_ptr(), n_a,
        rows.data_ptr(), start_ptr, idx_ptr, n_parts, n, heads, o_a.shape[2], dtype, _stream_ptr(device),
    )
    _capi.check(code, "hx_attn_merge")


# --------------------------------------------------------------- logits and argmax
class GreedyHeads(NamedTuple):
    """Result of ``final_norm_logits_argmax``: ``token_ids`` int64 ``[n]`` (-1 for an index
    outside the hidden rows), ``max_logits`` fp32 ``[n]``, and ``logits`` ``[n, vocab]``
    in the model dtype when they were asked for (else None)."""

    token_ids: torch.Tensor
    max_logits: torch.Tensor
    logits: torch.Tensor | None


def final_norm_logits_argmax(
    hidden_states: torch.Tensor,
    logit_indices: torch.Tensor,
    norm_weight: torch.Tensor,
    embedding: torch.Tensor,
    eps: float,
    *,
    return_logits: bool = False,
) -> GreedyHeads:
    """Greedy heads of a packed tick: the final RMSNorm of the logit rows, the tied
    lm_head and argmax, replacing ``x.index_select(1, logit_indices)``,
    ``self.output(self.final_norm(x).to(dtype))`` (model.py:108-110) and
    ``heads.argmax(dim=-1)`` (engine.py:470-473) for greedy sampling.

    ``hidden_states`` ``[T, hidden]`` or ``[1, T, hidden]`` (the last layer's output,
    contiguous last dim); ``logit_indices`` int64 ``[n]``; ``norm_weight`` fp32
    ``[hidden]``; ``embedding`` ``[vocab, hidden]`` in the model dtype. Ties go to the
    smallest vocab index, as in ``torch.argmax``. The logits are computed in fp32,
    rounded to the model dtype like the Linear's output, and written out only with
    ``return_logits``.
    """
    if hidden_states.ndim == 3:
        if hidden_states.shape[0] != 1:
            raise ValueError("hidden_states must be [tokens, hidden] or [1, tokens, hidden].")
        hidden_states = hidden_states[0]
    device = _require_gpu(hidden_states, logit_indices, norm_weight, embedding)
    if hidden_states.ndim != 2 or embedding.ndim != 2 or embedding.shape[1] != hidden_states.shape[1]:
        raise ValueError("embedding must be [vocab, hidden] matching hidden_states.")
    if hidden_states.dtype != embedding.dtype:
        raise ValueError("hidden_states and embedding must share a dtype.")
    dtype = _SUPPORTED.get(embedding.dtype)
    if dtype is None:
        raise ValueError("hidden_states and embedding must be bfloat16 or float16.")
    if hidden_states.stride(1) != 1 or embedding.stride(1) != 1:
        raise ValueError("hidden_states and embedding need a contiguous last dimension.")
    hidden = hidden_states.shape[1]
    if norm_weight.dtype != torch.float32 or tuple(norm_weight.shape) != (hidden,) or not norm_weight.is_contiguous():
        raise ValueError("norm_weight must be contiguous float32 [hidden].")
    if logit_indices.dtype != torch.int64 or logit_indices.ndim != 1 or not logit_indices.is_contiguous():
        raise ValueError("logit_indices must be contiguous int64 [n].")
    n, vocab = logit_indices.numel(), embedding.shape[0]
    token_ids = torch.empty(n, dtype=torch.int64, device=device)
    max_logits = torch.empty(n, dtype=torch.float32, device=device)
    logits = torch.empty((n, vocab), dtype=embedding.dtype, device=device) if return_logits else None
    if n == 0:
        return GreedyHeads(token_ids, max_logits, logits)
    lib = _capi.lib()
    ws_bytes = lib.hx_logits_workspace_bytes(n, vocab, hidden)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    code = lib.hx_final_norm_logits_argmax(
        hidden_states.data_ptr(), hidden_states.stride(0), hidden_states.shape[0],
        logit_indices.data_ptr(), n, norm_weight.data_ptr(), float(eps),
        embedding.data_ptr(), embedding.stride(0), vocab, hidden, dtype,
        token_ids.data_ptr(), max_logits.data_ptr(),
        logits.data_ptr() if logits is not None else None, vocab,
        workspace.data_ptr(), ws_bytes, _stream_ptr(device),
    )
    _capi.check(code, "hx_final_norm_logits_argmax")
    return GreedyHeads(token_ids, max_logits, logits)


# --------------------------------------------------------------- tick metadata
def tick_metadata(
    seq: torch.Tensor,
    block_table: torch.Tensor,
    page_size: int,
    *,
    total_q: int,
    cu_seq_q: torch.Tensor,
    cu_seq_k: torch.Tensor,
    seqused_k: torch.Tensor,
    write_slots: torch.Tensor,
    positions: torch.Tensor | None = None,
    logit_indices: torch.Tensor | None = None,
    n_logits: int = 0,
) -> None:
    """Per-tick metadata of ``PagedBatchCache.prepare`` / ``PackedBatchCache.prepare_packed``
    (paged_cache.py:221-270, :418-494) computed on the device.

    ``seq``: int32 ``[3 * B]`` = lengths before the tick, tokens this tick, logit rows.
    Writes ``cu_seq_q`` / ``cu_seq_k`` (int32 ``[B+1]``), ``seqused_k`` (int32 ``[B]``),
    ``write_slots`` and optionally ``positions`` (int64, ``total_q`` rows) and
    ``logit_indices`` (int64, ``n_logits`` rows), all preallocated on the device.
    """
    device = _require_gpu(seq, block_table, cu_seq_q, cu_seq_k, seqused_k, write_slots)
    batch = seq.numel() // 3
    if seq.dtype != torch.int32 or seq.numel() != 3 * batch or batch < 1 or not seq.is_contiguous():
        raise ValueError("seq must be a contiguous int32 tensor of 3 * batch values.")
    if block_table.dtype != torch.int32 or block_table.ndim != 2 or block_table.shape[0] != batch:
        raise ValueError("block_table must be int32 [batch, width].")
    if block_table.stride(1) != 1:
        raise ValueError("block_table rows must be contiguous.")
    for name, t, n, dt in (("cu_seq_q", cu_seq_q, batch + 1, torch.int32),
                           ("cu_seq_k", cu_seq_k, batch + 1, torch.int32),
                           ("seqused_k", seqused_k, batch, torch.int32),
                           ("write_slots", write_slots, total_q, torch.int64)):
        if t.dtype != dt or t.numel() < n or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {dt} tensor of at least {n} values.")
    for name, t, n in (("positions", positions, total_q), ("logit_indices", logit_indices, n_logits)):
        if t is not None and (t.dtype != torch.int64 or t.numel() < n or not t.is_contiguous()
                              or t.device != device):
            raise ValueError(f"{name} must be a contiguous int64 tensor of at least {n} values.")
    if n_logits > 0 and logit_indices is None:
        raise ValueError("logit_indices is required when n_logits > 0.")
    code = _capi.lib().hx_tick_metadata(
        seq.data_ptr(), batch, total_q, n_logits,
        block_table.data_ptr(), block_table.stride(0), page_size,
        cu_seq_q.data_ptr(), cu_seq_k.data_ptr(), seqused_k.data_ptr(),
        positions.data_ptr() if positions is not None else None,
        write_slots.data_ptr(),
        logit_indices.data_ptr() if logit_indices is not None else None,
        _stream_ptr(device),
    )
    _capi.check(code, "hx_tick_metadata")


# --------------------------------------------------------------------- page copy
def kv_copy_pages(
    k_caches: Sequence[torch.Tensor],
    v_caches: Sequence[torch.Tensor] | None,
    src_pages: Sequence[int],
    dst_pages: Sequence[int],
) -> None:
    """Copy whole pages for every layer: ``cache[l][dst[i]] = cache[l][src[i]]``.

    Bit-exact; the page-granular form of KVCache.snapshot_block/restore_blocks
    (cache.py:109-147). ``src_pages``/``dst_pages`` are host lists; destinations
    must be distinct and disjoint from the sources.
    """
    if len(src_pages) != len(dst_pages):
        raise ValueError("Source and destination page lists differ in length.")
    if not k_caches:
        return
    tensors = list(k_caches) + (list(v_caches) if v_caches is not None else [])
    device = _require_gpu(*tensors)
    shape, dtype = k_caches[0].shape, k_caches[0].dtype
    if v_caches is not None and len(v_caches) != len(k_caches):
        raise ValueError("Key and value layer lists differ in length.")
    for t in tensors:
        if t.shape != shape or t.dtype != dtype or not t.is_contiguous():
            raise ValueError("Every pool tensor must share one contiguous [pages, ...] layout.")
    n_layers, n_pages = len(k_caches), len(src_pages)
    if n_pages == 0:
        return
    page_bytes = k_caches[0][0].numel() * k_caches[0].element_size()
    k_ptrs = (ctypes.c_void_p * n_layers)(*[t.data_ptr() for t in k_caches])
    v_ptrs = (
        (ctypes.c_void_p * n_layers)(*[t.data_ptr() for t in v_caches])
        if v_caches is not None
        else None
    )
    src = (ctypes.c_int32 * n_pages)(*[int(p) for p in src_pages])
    dst = (ctypes.c_int32 * n_pages)(*[int(p) for p in dst_pages])
    code = _capi.lib().hx_kv_copy_pages(
        k_ptrs, v_ptrs, n_layers, src, dst, n_pages, shape[0], page_bytes, _stream_ptr(device)
    )
    _capi.check(code, "hx_kv_copy_pages")


# --------------------------------------------------------------------- page gather
def kv_gather(cache: torch.Tensor, pages: torch.Tensor | Sequence[int], length: int) -> torch.Tensor:
    """Paged -> dense ``[1, Hkv, length, d]`` (``_gather_cpu``, paged_cache.py:405-414)."""
    device = _require_gpu(cache)
    if cache.ndim != 4 or not cache.is_contiguous():
        raise ValueError("cache must be a contiguous [pages, page_size, kv_heads, head_dim] pool.")
    num_pages, page_size, n_kv, head_dim = cache.shape
    if not isinstance(pages, torch.Tensor):
        pages = torch.tensor(list(pages), dtype=torch.int32, device=device)
    if pages.ndim != 1 or pages.dtype != torch.int32 or pages.device != device:
        raise ValueError("pages must be an int32 vector on the cache's device.")
    pages = pages.contiguous()
    if length < 0 or length > pages.shape[0] * page_size:
        raise ValueError("length exceeds the listed pages.")
    out = torch.empty((1, n_kv, length, head_dim), dtype=cache.dtype, device=device)
    code = _capi.lib().hx_kv_gather(
        cache.data_ptr(), num_pages, page_size, n_kv, head_dim, cache.element_size(),
        pages.data_ptr(), pages.shape[0], length, out.data_ptr(), _stream_ptr(device),
    )
    _capi.check(code, "hx_kv_gather")
    return out


# --------------------------------------------------------------------- attention
def _window(window_size, is_causal: bool) -> tuple[int, int]:
    if window_size is None:
        return (-1, 0) if is_causal else (-1, -1)
    left, right = (int(x) for x in window_size)
    if is_causal:
        right = 0 if right < 0 else min(right, 0)
    return left, right


def workspace_bytes(batch: int, max_q: int, max_k: int, n_q_heads: int, n_kv_heads: int, head_dim: int) -> int:
    nbytes = _capi.lib().hx_varlen_attn_workspace_bytes(batch, max_q, max_k, n_q_heads, n_kv_heads, head_dim)
    if nbytes == 0:
        raise ValueError(
            "Unsupported attention shape: head_dim must be a multiple of 8 from 8 to 256 and "
            "n_q_heads a multiple of n_kv_heads."
        )
    return nbytes


def count_items(q_lens: Sequence[int], k_lens: Sequence[int], n_q_heads: int, n_kv_heads: int,
                window: tuple[int, int]) -> tuple[int, int, int]:
    """Exact work-item counts the device planner will produce for these lengths."""
    batch = len(q_lens)
    ql = (ctypes.c_int32 * max(batch, 1))(*q_lens)
    kl = (ctypes.c_int32 * max(batch, 1))(*k_lens)
    nd, np_, nc = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    code = _capi.lib().hx_varlen_attn_count_items(
        ql, kl, batch, n_q_heads, n_kv_heads, window[0], window[1],
        ctypes.byref(nd), ctypes.byref(np_), ctypes.byref(nc),
    )
    _capi.check(code, "hx_varlen_attn_count_items")
    return nd.value, np_.value, nc.value


class VarlenAttnPlan:
    """Work plan for one set of varlen metadata, reusable across layers.

    Built once per tick (the reference's metadata is identical for all 36 layers),
    then ``run`` is called per layer. ``q_lens``/``k_lens`` (host lists), when given,
    size the launch grids exactly; otherwise the bounds from (batch, max_q, max_k)
    are used and surplus workgroups exit at once.
    """

    def __init__(
        self,
        cu_seq_q: torch.Tensor,
        cu_seq_k: torch.Tensor | None,
        seqused_k: torch.Tensor | None,
        *,
        total_q: int,
        max_q: int,
        max_k: int,
        n_q_heads: int,
        n_kv_heads: int,
        head_dim: int,
        page_size: int,
        block_table_stride: int,
        total_k_rows: int = 0,
        window: tuple[int, int] = (-1, 0),
        q_lens: Sequence[int] | None = None,
        k_lens: Sequence[int] | None = None,
    ) -> None:
        device = _require_gpu(cu_seq_q)
        for name, t in (("cu_seq_q", cu_seq_q), ("cu_seq_k", cu_seq_k), ("seqused_k", seqused_k)):
            if t is None:
                continue
            if t.dtype != torch.int32 or t.ndim != 1 or t.device != device:
                raise ValueError(f"{name} must be an int32 vector on the query's device.")
        batch = cu_seq_q.shape[0] - 1
        if batch < 0:
            raise ValueError("cu_seq_q must have batch + 1 entries.")
        if cu_seq_k is not None and cu_seq_k.shape[0] != batch + 1:
            raise ValueError("cu_seq_k must have batch + 1 entries.")
        if seqused_k is not None and seqused_k.shape[0] != batch:
            raise ValueError("seqused_k must have batch entries.")
        if seqused_k is None and cu_seq_k is None:
            raise ValueError("Either seqused_k or cu_seq_k is required.")
        if max_q < 0 or max_k < 0:
            raise ValueError("max_q and max_k must be non-negative.")
        self.device = device
        self.batch = batch
        self.total_q = total_q
        self.max_q = max_q
        self.max_k = max_k
        self.n_q_heads = n_q_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.block_table_stride = block_table_stride
        self.window = window
        # The tuned kernels (split-K decode, MFMA chunk, combine) serve head_dim 128 with
        # 1, 2, 4 or 8 query heads per KV head; other shapes run one generic kernel that
        # covers every row in a single launch.
        self.tuned = head_dim == 128 and n_kv_heads > 0 and n_q_heads % n_kv_heads == 0 \
            and n_q_heads // n_kv_heads in (1, 2, 4, 8)
        self._metadata = (cu_seq_q.contiguous(), None if cu_seq_k is None else cu_seq_k.contiguous(),
                          None if seqused_k is None else seqused_k.contiguous())
        self.ws_bytes = workspace_bytes(max(batch, 0), max_q, max_k, n_q_heads, n_kv_heads, head_dim)
        self.workspace = torch.empty(self.ws_bytes + 256, dtype=torch.uint8, device=device)
        base = self.workspace.data_ptr()
        self._ws_offset = (-base) % 256
        self.ws_ptr = base + self._ws_offset
        if q_lens is not None and k_lens is not None:
            self.hints = count_items(q_lens, k_lens, n_q_heads, n_kv_heads, window)
        else:
            self.hints = (-1, -1, -1)
        cu_q, cu_k, used = self._metadata
        code = _capi.lib().hx_varlen_attn_plan(
            cu_q.data_ptr(),
            None if cu_k is None else cu_k.data_ptr(),
            None if used is None else used.data_ptr(),
            batch, total_q, max_q, max_k, total_k_rows, page_size, block_table_stride,
            n_q_heads, n_kv_heads, head_dim, window[0], window[1],
            self.ws_ptr, self.ws_bytes, _stream_ptr(device),
        )
        _capi.check(code, "hx_varlen_attn_plan")

    def error_word(self) -> int:
        """HX_WERR_* bits raised so far (synchronises the device to read them)."""
        off = self._ws_offset + _capi.lib().hx_varlen_attn_error_word_offset()
        return int(self.workspace[off:off + 4].view(torch.int32).item())

    def check_errors(self) -> None:
        """Raise RuntimeError if the plan or a run flagged bad metadata (synchronises)."""
        word = self.error_word()
        if word:
            raise RuntimeError(f"paged attention metadata error {word:#x}: {describe_error_word(word)}")

    def run(
        self,
        query: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        block_table: torch.Tensor | None,
        *,
        scale: float | None = None,
        out: torch.Tensor | None = None,
        return_lse: bool = False,
        lse_out: torch.Tensor | None = None,
        phases: tuple[str, ...] = ("decode", "chunk", "combine"),
        append: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
        query_rows: torch.Tensor | None = None,
        merge: MergeParts | None = None,
    ) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
        """Attention for one layer. ``phases`` launches a subset of the three kernels
        (decode splits, chunk rows, split combine); a full result needs all three, with
        the combine after the other two (the launch order within one call), into the
        same ``out`` (and ``lse_out``, when the log-sum-exp is wanted). Profilers use it
        to time each kernel, and ``run_overlapped`` to run decode and chunk rows on two
        streams.

        ``append=(k_new, v_new, write_slots)`` first writes the tick's new K/V rows
        into the pool (index_copy_ semantics, as ``kv_append``) in the same call: decode
        rows inside the decode kernel, chunk rows by the append kernel beforehand.

        ``query_rows`` (int64 ``[total_q]`` on the device) reads packed row t's query
        from ``query[query_rows[t]]``, so ``query`` may be any ``[N, n_q_heads,
        head_dim]``; ``out`` and the log-sum-exp stay ``[total_q, ...]``. It is the
        result of ``run(query.index_select(0, query_rows), ...)`` without the gather. An
        entry outside ``[0, N)`` reads row 0 and sets an error-word bit. Not combined
        with ``append``.

        ``merge`` (``MergeParts``) folds a shared-prefix cascade's level results into its
        members' rows inside the combine launch: the bits of this run followed by
        ``attn_merge`` over the same parts, one launch fewer. It needs the combine phase
        and the log-sum-exp output (``return_lse`` or ``lse_out``), on the tuned shapes.
        """
        _require_gpu(query, k_cache, v_cache)
        unknown = set(phases) - {"decode", "combine", "chunk"}
        if unknown:
            raise ValueError(f"unknown attention phases {sorted(unknown)}")
        if query.device != self.device:
            raise ValueError("Query is not on the plan's device.")
        if query.dtype not in _SUPPORTED:
            raise ValueError("varlen_attn supports bfloat16 and float16 queries.")
        rows_in = self.total_q if query_rows is None else query.shape[0]
        if query.ndim != 3 or query.shape[0] != rows_in or query.shape[1] != self.n_q_heads \
                or query.shape[2] != self.head_dim:
            raise ValueError("Query must be [total_q, n_q_heads, head_dim] as planned.")
        if query_rows is not None:
            if append is not None:
                raise ValueError("query_rows and append cannot be combined.")
            if query_rows.dtype != torch.int64 or query_rows.ndim != 1 or not query_rows.is_contiguous() \
                    or query_rows.numel() != self.total_q or query_rows.device != self.device:
                raise ValueError("query_rows must be contiguous int64 [total_q] on the plan's device.")
            if query.shape[0] < 1:
                raise ValueError("query_rows needs a query tensor of at least one row.")
        if k_cache.shape != v_cache.shape or k_cache.dtype != query.dtype or v_cache.dtype != query.dtype:
            raise ValueError("Key/value caches must match each other and the query dtype.")
        if k_cache.stride() != v_cache.stride():
            raise ValueError("Key and value caches must share strides.")
        if self.page_size > 0:
            if k_cache.ndim != 4 or k_cache.shape[1] != self.page_size:
                raise ValueError("Paged caches must be [num_pages, page_size, kv_heads, head_dim].")
            if block_table is None or block_table.dtype != torch.int32 or block_table.ndim != 2 \
                    or block_table.shape[0] != self.batch or block_table.device != self.device:
                raise ValueError("block_table must be int32 [batch, width] on the query's device.")
            if block_table.stride(1) != 1 or block_table.shape[1] != self.block_table_stride \
                    or block_table.stride(0) != self.block_table_stride:
                raise ValueError("block_table must be row-contiguous with the planned width.")
            num_pages = k_cache.shape[0]
            row_stride, head_stride = k_cache.stride(1), k_cache.stride(2)
            if k_cache.stride(0) != self.page_size * row_stride:
                raise ValueError("Pages must be laid out back to back.")
        else:
            if k_cache.ndim != 3:
                raise ValueError("Packed caches must be [total_k, kv_heads, head_dim].")
            num_pages = 0
            row_stride, head_stride = k_cache.stride(0), k_cache.stride(1)
        if k_cache.shape[-2] != self.n_kv_heads or k_cache.shape[-1] != self.head_dim or k_cache.stride(-1) != 1:
            raise ValueError("Key/value caches must be [..., n_kv_heads, head_dim] with contiguous head_dim.")
        if query.stride(2) != 1:
            query = query.contiguous()
        out_shape = (self.total_q, self.n_q_heads, self.head_dim)
        if out is None:
            out = torch.empty(out_shape, dtype=query.dtype, device=query.device)
        elif tuple(out.shape) != out_shape or out.dtype != query.dtype or out.stride(2) != 1:
            raise ValueError("out must be [total_q, n_q_heads, head_dim] of the query's dtype.")
        lse = lse_out
        if lse is not None:
            if lse.dtype != torch.float32 or tuple(lse.shape) != (self.n_q_heads, self.total_q) \
                    or not lse.is_contiguous():
                raise ValueError("lse_out must be contiguous float32 [n_q_heads, total_q].")
        elif return_lse:
            lse = torch.empty((self.n_q_heads, self.total_q), dtype=torch.float32, device=query.device)
        scale = 1.0 / math.sqrt(self.head_dim) if scale is None else float(scale)
        hints = (
            self.hints[0] if "decode" in phases else 0,
            self.hints[1] if "chunk" in phases else 0,
            self.hints[2] if "combine" in phases else 0,
        )
        if not self.tuned:
            # The generic kernel covers every row in one launch: it runs in the call that
            # holds the decode phase, or in the chunk phase of a tick without decode rows,
            # never twice for one layer.
            once = "decode" in phases or ("chunk" in phases and self.hints[0] == 0)
            hints = (self.hints[0], self.hints[1], hints[2]) if once else (0, 0, hints[2])
        common = (
            query.data_ptr(), query.stride(0), query.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), row_stride, head_stride,
            num_pages, self.page_size,
            None if block_table is None else block_table.data_ptr(), self.block_table_stride,
            self.batch, self.total_q, self.max_q, self.max_k,
            self.n_q_heads, self.n_kv_heads, self.head_dim,
            scale, self.window[0], self.window[1], _SUPPORTED[query.dtype],
            out.data_ptr(), out.stride(0), out.stride(1),
            None if lse is None else lse.data_ptr(),
        )
        if merge is not None:
            if append is not None or query_rows is not None:
                raise ValueError("merge cannot be combined with append or query_rows.")
            if "combine" not in phases or lse is None or not self.tuned:
                raise ValueError("merge needs the combine phase, the lse output and a tuned shape.")
            lo, ll = merge.level_out, merge.level_lse
            n_a = lo.shape[0] if lo.ndim == 3 else -1
            if lo.ndim != 3 or lo.shape[1:] != (self.n_q_heads, self.head_dim) or lo.dtype != query.dtype \
                    or lo.stride(2) != 1 or lo.device != self.device:
                raise ValueError("merge.level_out must be [rows, n_q_heads, head_dim] of the query's dtype.")
            if ll.dtype != torch.float32 or tuple(ll.shape) != (self.n_q_heads, n_a) or not ll.is_contiguous():
                raise ValueError("merge.level_lse must be contiguous float32 [n_q_heads, rows].")
            for name in ("member_seq", "member_of_seq", "part_start", "part_idx"):
                t = getattr(merge, name)
                if t.dtype != torch.int32 or t.ndim != 1 or not t.is_contiguous() or t.device != self.device:
                    raise ValueError(f"merge.{name} must be a contiguous int32 vector on the device.")
            n_members = merge.member_seq.numel()
            if merge.part_start.numel() != n_members + 1 or merge.member_of_seq.numel() != self.batch:
                raise ValueError("merge.part_start needs members + 1 entries and member_of_seq one per sequence.")
            lp = merge.level_plan
            if lp is None:
                code = _capi.lib().hx_varlen_attn_run_merged(
                    *common, lo.data_ptr(), lo.stride(0), lo.stride(1), ll.data_ptr(), n_a,
                    merge.member_seq.data_ptr(), merge.member_of_seq.data_ptr(), n_members,
                    merge.part_start.data_ptr(), merge.part_idx.data_ptr(), merge.part_idx.numel(),
                    *hints, self.ws_ptr, self.ws_bytes, _stream_ptr(query.device))
                _capi.check(code, "hx_varlen_attn_run_merged")
            else:
                if not isinstance(lp, VarlenAttnPlan) or lp.device != self.device or lp.n_q_heads != self.n_q_heads \
                        or lp.n_kv_heads != self.n_kv_heads or lp.head_dim != self.head_dim or lp.total_q != n_a:
                    raise ValueError("merge.level_plan must be the plan of level_out: same device and heads, "
                                     "total_q = level_out rows.")
                lbt, lrows = merge.level_block_table, merge.level_query_rows
                if lbt is None and lrows is not None:
                    raise ValueError("merge.level_query_rows needs merge.level_block_table.")
                if lbt is not None:
                    # The level plan's chunk items run in this call (see MergeParts).
                    if set(phases) != {"decode", "chunk", "combine"}:
                        raise ValueError("a merge that runs the level plan's chunk items needs all three phases.")
                    if lp.hints[0] != 0 or lp.page_size != self.page_size:
                        raise ValueError("merge.level_plan must hold no decode rows and share the page size to "
                                         "run in this call.")
                    if lp.page_size > 0 and (lbt.dtype != torch.int32 or lbt.ndim != 2 or lbt.shape[0] != lp.batch
                                             or lbt.shape[1] != lp.block_table_stride or lbt.stride(1) != 1
                                             or lbt.stride(0) != lp.block_table_stride or lbt.device != self.device):
                        raise ValueError("merge.level_block_table must be the level plan's row-contiguous int32 "
                                         "[batch, width] table on the device.")
                    if lrows is None or lrows.dtype != torch.int64 or lrows.ndim != 1 or not lrows.is_contiguous() \
                            or lrows.numel() != lp.total_q or lrows.device != self.device:
                        raise ValueError("merge.level_query_rows must be contiguous int64 [level rows] on the device.")
                level_chunk = (None, 0, None, 0, 0, -1, -1) if lbt is None else (
                    lbt.data_ptr(), lp.block_table_stride, lrows.data_ptr(), query.shape[0], lp.hints[1],
                    lp.window[0], lp.window[1])
                code = _capi.lib().hx_varlen_attn_run_cascade(
                    *common, lo.data_ptr(), lo.stride(0), lo.stride(1), ll.data_ptr(), n_a,
                    lp.batch, lp.max_q, lp.max_k, lp.hints[2], lp.ws_ptr, lp.ws_bytes, *level_chunk,
                    merge.member_seq.data_ptr(), merge.member_of_seq.data_ptr(), n_members,
                    merge.part_start.data_ptr(), merge.part_idx.data_ptr(), merge.part_idx.numel(),
                    *hints, self.ws_ptr, self.ws_bytes, _stream_ptr(query.device))
                _capi.check(code, "hx_varlen_attn_run_cascade")
        elif query_rows is not None:
            code = _capi.lib().hx_varlen_attn_run_rows(
                *common[:3], query_rows.data_ptr(), query.shape[0], *common[3:], *hints,
                self.ws_ptr, self.ws_bytes, _stream_ptr(query.device))
            _capi.check(code, "hx_varlen_attn_run_rows")
        elif append is None:
            code = _capi.lib().hx_varlen_attn_run(
                *common, *hints, self.ws_ptr, self.ws_bytes, _stream_ptr(query.device))
            _capi.check(code, "hx_varlen_attn_run")
        else:
            k_new, v_new, slots = append
            _check_append(k_cache, v_cache, slots, k_new, v_new)
            if k_new.shape[0] != self.total_q:
                raise ValueError("append rows must match the packed query rows.")
            if not k_cache.is_contiguous() or not v_cache.is_contiguous():
                raise ValueError("KV pools must be contiguous.")
            pool_rows = k_cache.numel() // (self.n_kv_heads * self.head_dim)
            slots = slots.contiguous()
            code = _capi.lib().hx_varlen_attn_append_run(
                *common,
                k_new.data_ptr(), k_new.stride(0), k_new.stride(1),
                v_new.data_ptr(), v_new.stride(0), v_new.stride(1),
                slots.data_ptr(), pool_rows,
                *hints, self.ws_ptr, self.ws_bytes, _stream_ptr(query.device))
            _capi.check(code, "hx_varlen_attn_append_run")
        if CHECK_ERRORS:
            self.check_errors()
            if merge is not None and merge.level_plan is not None:
                merge.level_plan.check_errors()  # its combine records (and chunk items) ran in this call
        return (out, lse) if return_lse else out


def run_overlapped(plan: "VarlenAttnPlan", query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   block_table: torch.Tensor | None, side: torch.cuda.Stream, *, return_lse: bool = False,
                   side_first=None):
    """``plan.run`` with the chunk rows (MFMA-bound) on ``side`` while the decode rows
    (HBM-bound) run on the current stream; the combine runs after both. The new K/V rows
    must already be in the pool. ``side_first`` is an optional callable queued on the
    side stream before the chunk launch (work that must also overlap the decode rows);
    its return value is returned last, and any tensors in it are marked as used by the
    current stream. Falls back to ``plan.run`` when one kind of row is absent, and for
    shapes the generic kernel serves (it covers every row in one launch)."""
    dec, pf, _ = plan.hints
    has_chunk = pf != 0 and plan.max_q >= 2
    if dec == 0 or (not has_chunk and side_first is None) or not plan.tuned:
        extra = side_first() if side_first is not None else None
        res = plan.run(query, k_cache, v_cache, block_table, return_lse=return_lse)
        return (res, extra) if side_first is not None else res
    main = torch.cuda.current_stream(query.device)
    out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    lse = torch.empty((plan.n_q_heads, plan.total_q), dtype=torch.float32, device=query.device) if return_lse else None
    forked = torch.cuda.Event()
    forked.record(main)
    side.wait_event(forked)
    extra = None
    with torch.cuda.stream(side):
        if side_first is not None:
            extra = side_first()
        if has_chunk:
            plan.run(query, k_cache, v_cache, block_table, out=out, lse_out=lse, phases=("chunk",))
    joined = torch.cuda.Event()
    joined.record(side)
    plan.run(query, k_cache, v_cache, block_table, out=out, lse_out=lse, phases=("decode",))
    main.wait_event(joined)
    if extra is not None:
        for t in (extra if isinstance(extra, tuple) else (extra,)):
            if isinstance(t, torch.Tensor):
                t.record_stream(main)
    plan.run(query, k_cache, v_cache, block_table, out=out, lse_out=lse, phases=("combine",))
    res = (out, lse) if return_lse else out
    return (res, extra) if side_first is not None else res


def varlen_attn(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cu_seq_q: torch.Tensor,
    cu_seq_k: torch.Tensor | None,
    max_q: int,
    max_k: int,
    is_causal: bool = False,
    return_aux: AuxRequest | None = None,
    *,
    window_size: tuple[int, int] | None = None,
    enable_gqa: bool = False,
    seqused_k: torch.Tensor | None = None,
    block_table: torch.Tensor | None = None,
    num_splits: int | None = None,
    scale: float | None = None,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Drop-in for the paged ``varlen_attn`` call at paged_cache.py:316-329 / :506-519.

    ``query``: ``[total_q, Hq, d]``. With ``block_table`` (int32 ``[B, W]``),
    ``key``/``value`` are pools ``[num_pages, page_size, Hkv, d]`` and sequence b
    has ``seqused_k[b]`` keys (else ``cu_seq_k[b+1]-cu_seq_k[b]``); without it they
    are packed ``[total_k, Hkv, d]`` located by ``cu_seq_k``. ``window_size=(-1, 0)``
    is the bottom-right causal mask. ``num_splits`` is accepted for signature parity:
    the split schedule is fixed by each sequence's length, and the combine order is
    fixed, so results are deterministic for any value.
    """
    del num_splits
    device = _require_gpu(query, key, value, cu_seq_q)
    if query.ndim != 3:
        raise ValueError("query must be [total_q, n_q_heads, head_dim].")
    n_q_heads, head_dim = query.shape[1], query.shape[2]
    n_kv_heads = key.shape[-2]
    if n_q_heads != n_kv_heads and not enable_gqa:
        raise ValueError("Query and KV head counts differ; pass enable_gqa=True.")
    if n_kv_heads < 1 or n_q_heads % n_kv_heads:
        raise ValueError(f"GQA needs n_q_heads ({n_q_heads}) to be a multiple of n_kv_heads ({n_kv_heads}).")
    window = _window(window_size, is_causal)
    paged = block_table is not None
    if paged:
        page_size = key.shape[1]
        bt_stride = block_table.shape[1] if block_table.ndim == 2 else 0
        if block_table.stride(-1) != 1:
            block_table = block_table.contiguous()
        total_k_rows = 0
    else:
        if cu_seq_k is None:
            raise ValueError("Packed keys need cu_seq_k.")
        page_size, bt_stride = 0, 0
        total_k_rows = key.shape[0]
    plan = VarlenAttnPlan(
        cu_seq_q, cu_seq_k, seqused_k,
        total_q=query.shape[0], max_q=max_q, max_k=max_k,
        n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
        page_size=page_size, block_table_stride=bt_stride, total_k_rows=total_k_rows,
        window=window,
    )
    want_lse = bool(return_aux is not None and return_aux.lse)
    del device
    return plan.run(query, key, value, block_table, scale=scale, return_lse=want_lse)
