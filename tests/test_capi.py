"""The C ABI library loads and exports every declared symbol; host-only entry
points behave (no GPU work is launched here)."""

from __future__ import annotations

import ctypes
import math
import subprocess

import pytest

from helios_amd import _capi, ops, synth


def test_library_exports_every_header_function():
    names = _capi.header_functions()
    assert len(names) == len(set(names)) >= 10
    assert set(names) == set(_capi.SIGNATURES), "binding table out of sync with the header"
    lib = _capi.lib()
    for name in names:
        assert getattr(lib, name) is not None
    out = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert set(names) <= exported


def test_loader_rejects_a_library_of_another_abi_version(monkeypatch):
    monkeypatch.setattr(_capi, "_lib", None)
    monkeypatch.setattr(_capi, "ABI_VERSION", _capi.ABI_VERSION + 1)
    with pytest.raises(_capi.HeliosLibraryError, match="ABI version"):
        _capi.lib()


def test_abi_version_and_strerror():
    assert _capi.lib().hx_abi_version() == _capi.ABI_VERSION == 6
    assert _capi.strerror(0) == "success"
    assert "invalid" in _capi.strerror(_capi.HX_E_INVALID_ARG)
    with pytest.raises(ValueError):
        _capi.check(_capi.HX_E_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _capi.check(1, "x")


def test_workspace_bytes_supported_shapes():
    lib = _capi.lib()
    assert lib.hx_varlen_attn_workspace_bytes(64, 1, 4097, 32, 8, 128) > 0
    # any head_dim that is a multiple of 8 up to 256, any group size (the generic kernel)
    for hq, hkv, d in ((32, 8, 64), (48, 8, 128), (2, 1, 8), (64, 1, 256), (12, 4, 96)):
        assert lib.hx_varlen_attn_workspace_bytes(64, 1, 4097, hq, hkv, d) > 0, (hq, hkv, d)
    for d in (0, 4, 12, 130, 264):
        assert lib.hx_varlen_attn_workspace_bytes(64, 1, 4097, 32, 8, d) == 0, d
    assert lib.hx_varlen_attn_workspace_bytes(64, 1, 4097, 30, 8, 128) == 0  # not a multiple
    with pytest.raises(ValueError):
        ops.workspace_bytes(1, 1, 1, 32, 8, 100)


def _expected_counts(w: synth.Workload, window=(-1, 0)):
    """Work items from the closed forms: decode rows split keys in 256s; chunk rows go in
    blocks of rows_per_item, and when the unsplit blocks launch fewer than 512 workgroups
    each block's 64-key tiles are cut into splits of at least max(4, ceil(tiles * Hkv /
    512)) tiles, every split row adding one combine record. When the split workgroups
    spill past R >= 1 whole rounds of 256 (one chunk workgroup per CU), the split size is
    the smallest one, up to the largest block's tiles, whose count fits R rounds, or one
    round when that size is at most ceil(1.25 x chunk tiles x Hkv / 256). Then only
    blocks longer than max(split size, ceil(1.25 x chunk tiles x Hkv / 256)) split."""
    nd = nc = npf = 0
    G = w.n_q_heads // w.n_kv_heads
    gw = min(G, 4)
    quads = G // gw
    rows_per_item = 64 * (4 // gw)

    def tiles(n, L, row0):
        off = L - n
        row_end = min(n, row0 + rows_per_item)
        klo = 0 if window[0] < 0 else max(0, off + row0 - window[0])
        khi = L - 1 if window[1] < 0 else min(L - 1, off + row_end - 1 + window[1])
        return (khi // 64 + 1 - klo // 64) if khi >= klo else 0

    blocks = [(n, L, r0) for n, L in zip(w.q_lens, w.k_lens) if n > 1 for r0 in range(0, n, rows_per_item)]
    items0 = len(blocks) * quads
    tiles0 = sum(tiles(*blk) for blk in blocks) * quads
    split = 0
    if items0 and items0 * w.n_kv_heads < 512:
        split = max(4, -(-tiles0 * w.n_kv_heads // 512))

    def split_count(t, st, keep=None):
        keep = st if keep is None else keep
        return 1 if not st or t <= keep else min(64, -(-t // st))

    def wgs(st):
        return w.n_kv_heads * quads * sum(split_count(tiles(*blk), st) for blk in blocks)

    if split:
        st0, w0 = split, wgs(split)
        rounds, max_t = w0 // 256, max(tiles(*blk) for blk in blocks)
        if rounds >= 1 and w0 % 256 and max_t > st0 and wgs(max_t) <= rounds * 256:
            split = min(st for st in range(st0, max_t + 1) if wgs(st) <= rounds * 256)
        # one round instead when its split size is at most 1.25 x the tiles per CU
        if w0 > 256 and max_t > st0 and wgs(max_t) <= 256:
            s1 = min(st for st in range(st0, max_t + 1) if wgs(st) <= 256)
            if s1 <= -(-5 * tiles0 * w.n_kv_heads // (4 * 256)):
                split = s1
    keep = max(split, -(-5 * tiles0 * w.n_kv_heads // (4 * 256)))
    for n, L in zip(w.q_lens, w.k_lens):
        if n == 1:
            lo = 0 if window[0] < 0 else max(0, L - 1 - window[0])
            splits = (L - 1) // 256 - lo // 256 + 1 if L > 0 else 1
            nd += splits
            nc += splits > 1
    for n, L, r0 in blocks:
        t = tiles(n, L, r0)
        s = split_count(t, split, keep)
        npf += s * quads
        if s > 1:
            nc += -(-min(rows_per_item, n - r0) // 8)  # combine records of up to 8 rows
    return nd, npf, nc


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4"])
def test_count_items_matches_closed_form(name):
    w = getattr(synth, name)()
    assert ops.count_items(w.q_lens, w.k_lens, 32, 8, (-1, 0)) == _expected_counts(w)


@pytest.mark.parametrize("chunks", [[(1024, 5120)], [(2048, 2048)], [(2048, 6144)], [(1536, 4096)],
                                    [(3000, 3000)], [(512, 8192)], [(768, 3000)],
                                    [(1024, 1024), (992, 1504)]])
def test_chunk_splits_fill_whole_rounds(chunks):
    """Chunk splits whose per-block rounding would spill into a partial extra round of
    256 workgroups get the smallest larger split size that fits the whole rounds."""
    q_lens = [n for n, _ in chunks] + [1] * 4
    k_lens = [L for _, L in chunks] + [700, 1300, 257, 4096]
    w = synth.Workload("rounds", q_lens, [L - n for n, L in zip(q_lens, k_lens)],
                       [[0] * (-(-L // 256)) for L in k_lens], 64)
    counts = ops.count_items(q_lens, k_lens, 32, 8, (-1, 0))
    assert counts == _expected_counts(w)
    # Without the refinement most of these spill to 536-696 workgroups (a partial third
    # round); with it every one fits two rounds (or one).
    assert counts[1] * 8 <= 512


def test_count_items_windows_and_groups():
    w = synth.small_mixed(5, n_q_heads=8, n_kv_heads=8)
    assert ops.count_items(w.q_lens, w.k_lens, 8, 8, (-1, 0)) == _expected_counts(w)
    w = synth.small_mixed(6, n_q_heads=16, n_kv_heads=2)
    assert ops.count_items(w.q_lens, w.k_lens, 16, 2, (300, 0)) == _expected_counts(w, (300, 0))
    assert ops.count_items([1, 1], [0, 1], 32, 8, (-1, 0)) == (2, 0, 0)


def test_copy_pages_rejects_bad_ids_on_the_host():
    lib = _capi.lib()
    ptrs = (ctypes.c_void_p * 1)(16)
    src = (ctypes.c_int32 * 2)(0, 1)
    dst = (ctypes.c_int32 * 2)(1, 2)
    assert lib.hx_kv_copy_pages(ptrs, None, 1, src, dst, 2, 4, 1 << 19, None) == _capi.HX_E_OVERLAP
    dst2 = (ctypes.c_int32 * 2)(3, 3)
    assert lib.hx_kv_copy_pages(ptrs, None, 1, src, dst2, 2, 4, 1 << 19, None) == _capi.HX_E_OVERLAP
    dst3 = (ctypes.c_int32 * 2)(2, 4)
    assert lib.hx_kv_copy_pages(ptrs, None, 1, src, dst3, 2, 4, 1 << 19, None) == _capi.HX_E_INVALID_ARG
    assert lib.hx_kv_copy_pages(ptrs, None, 1, src, dst, 0, 4, 1 << 19, None) == _capi.HX_OK


def test_attention_entry_points_reject_bad_arguments_on_the_host():
    lib = _capi.lib()
    # workspace missing -> HX_E_WORKSPACE before any launch
    assert lib.hx_varlen_attn_plan(16, 16, 16, 1, 1, 1, 1, 0, 256, 1, 32, 8, 128, -1, 0,
                                   None, 0, None) == _capi.HX_E_WORKSPACE
    # unsupported head_dim (not a multiple of 8)
    assert lib.hx_varlen_attn_plan(16, 16, 16, 1, 1, 1, 1, 0, 256, 1, 32, 8, 68, -1, 0,
                                   None, 0, None) == _capi.HX_E_UNSUPPORTED
    # page size not a multiple of 256
    assert lib.hx_varlen_attn_plan(16, 16, 16, 1, 1, 1, 1, 0, 128, 1, 32, 8, 128, -1, 0,
                                   None, 0, None) == _capi.HX_E_INVALID_ARG
    # append: bad element size
    assert lib.hx_kv_append(16, 16, 10, 16, 8, 8, 16, 8, 8, 16, 1, 1, 8, 3, None) == _capi.HX_E_INVALID_ARG
    # gather: length beyond the listed pages
    assert lib.hx_kv_gather(16, 4, 256, 8, 128, 2, 16, 1, 257, 16, None) == _capi.HX_E_INVALID_ARG


def test_cascade_run_rejects_a_bad_level_plan_on_the_host():
    """hx_varlen_attn_run_cascade checks the level plan's workspace and rows before any
    launch or device access (the pointers below are never dereferenced): a missing level
    workspace, one that is misaligned or too small for the level shape, and level rows
    that are not 8-byte aligned are refused; so is a level chunk run (a level block
    table given) without its query row map or with a block-table width below 1."""
    lib = _capi.lib()
    mib = 1 << 20

    def call(level_out=64 * mib, level_ws=128 * mib, level_ws_bytes=1 << 30, level_bt=None, level_bt_stride=0,
             level_rows=None):
        return lib.hx_varlen_attn_run_cascade(
            16 * mib, 4096, 128, 32 * mib, 48 * mib, 1024, 128, 16, 256, 8 * mib, 4,
            2, 2, 1, 512, 32, 8, 128, 1 / math.sqrt(128), -1, 0, _capi.HX_DTYPE_BF16,
            96 * mib, 4096, 128, 112 * mib,
            level_out, 4096, 128, 120 * mib, 2,
            1, 2, 512, -1, level_ws, level_ws_bytes,
            level_bt, level_bt_stride, level_rows, 2, -1, -1, -1,
            121 * mib, 122 * mib, 1, 123 * mib, 124 * mib, 1,
            -1, -1, -1, 256 * mib, 1 << 30, None)

    assert call(level_ws=None) == _capi.HX_E_INVALID_ARG
    assert call(level_ws=128 * mib + 8) == _capi.HX_E_WORKSPACE
    assert call(level_ws_bytes=16) == _capi.HX_E_WORKSPACE
    assert call(level_out=64 * mib + 4) == _capi.HX_E_INVALID_ARG
    assert call(level_bt=125 * mib, level_bt_stride=2) == _capi.HX_E_INVALID_ARG       # no row map
    assert call(level_bt=125 * mib, level_bt_stride=0, level_rows=126 * mib) == _capi.HX_E_INVALID_ARG


def test_noalloc_rejects_a_tick_beyond_its_scratch():
    """hx_varlen_attn_noalloc checks the shape against its scratch array before it touches
    the device: a tick whose workspace exceeds HX_NOALLOC_SCRATCH_BYTES (128 MiB) returns
    HX_E_TOO_LARGE, and an unsupported head_dim HX_E_UNSUPPORTED, with no launch."""
    lib = _capi.lib()
    batch, max_k = 4096, 32768
    assert lib.hx_varlen_attn_workspace_bytes(batch, 1, max_k, 32, 8, 128) > 128 << 20
    args = [None, 0, 0, None, None, 0, 0, 1, 256, None, 128, None, None, None,
            batch, batch, 1, max_k, 0, 32, 8, 128, 1 / math.sqrt(128), -1, 0, _capi.HX_DTYPE_BF16,
            None, 0, 0, None, None]
    assert lib.hx_varlen_attn_noalloc(*args) == _capi.HX_E_TOO_LARGE
    args[21] = 100   # head_dim
    assert lib.hx_varlen_attn_noalloc(*args) == _capi.HX_E_UNSUPPORTED
    assert "no-allocation scratch" in _capi.strerror(_capi.HX_E_TOO_LARGE)


def test_chunk_split_policy_known_answers():
    """The planner's split choices on three tick shapes, as workgroup counts (items x 8 KV
    heads): C3's blocks of up to 16 tiles stay whole and the 8 longer ones per KV head
    split in three (384); a 1024-row chunk at position 4096 (blocks of 65-80 tiles)
    splits once per block into one round (256); C4 does not split (512)."""
    c3 = synth.c3()
    assert ops.count_items(c3.q_lens, c3.k_lens, 32, 8, (-1, 0))[1] * 8 == 384
    q_lens, k_lens = [1024] + [1] * 4, [5120, 700, 1300, 257, 4096]
    assert ops.count_items(q_lens, k_lens, 32, 8, (-1, 0))[1] * 8 == 256
    c4 = synth.c4()
    assert ops.count_items(c4.q_lens, c4.k_lens, 32, 8, (-1, 0))[1] * 8 == 512
