"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, validates arguments on the host, and its tile pruning rule visits
exactly the KV tiles that hold a visible (query, key) pair."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from inkling_fa4 import _abi, autotune_configs

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "ifa4.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ifa4_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for must in ("ifa4_validate", "ifa4_prefill_fwd", "ifa4_decode_fwd",
                 "ifa4_decode_workspace_bytes", "ifa4_status_str"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    names = _declared_functions()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_abi.SIGNATURES), "ctypes view out of sync with include/ifa4.h"
    nm = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(ifa4_\w+)", nm))
    assert set(names) <= exported


def test_abi_version_and_struct_size():
    assert _abi.lib().ifa4_abi_version() == 1
    a = _abi.make_args()
    a.struct_size = 12
    assert _abi.lib().ifa4_validate(ctypes.byref(a)) == _abi.IFA4_EINVAL


def test_status_strings():
    for code in range(5):
        assert _abi.status_str(code).startswith("IFA4")
    assert "unknown" in _abi.status_str(99)


# fake, well-aligned device addresses: ifa4_validate never dereferences them
_P = 1 << 20


def _good(**kw):
    base = dict(batch=2, n_heads=8, kv_heads=2, head_dim=128, rel_extent=128, rel_width=128,
                max_seqlen_q=64, max_seqlen_k=64, total_q=128, total_k=128,
                q=_P, k=2 * _P, v=3 * _P, rel=4 * _P, out=5 * _P,
                cu_seqlens_q=6 * _P, cu_seqlens_k=7 * _P,
                q_stride_t=8 * 128, q_stride_h=128, k_stride_t=2 * 128, k_stride_h=128,
                v_stride_t=2 * 128, v_stride_h=128, rel_stride_t=0, rel_stride_h=128,
                out_stride_t=8 * 128, out_stride_h=128, softmax_scale=1 / 128,
                qkv_dtype=_abi.IFA4_BF16, rel_dtype=_abi.IFA4_FP32)
    base.update(kw)
    return _abi.make_args(**base)


def _validate(**kw):
    return _abi.lib().ifa4_validate(ctypes.byref(_good(**kw)))


@pytest.mark.parametrize("kw,expect", [
    ({}, _abi.IFA4_OK),
    ({"head_dim": 64, "q_stride_h": 64, "k_stride_h": 64, "v_stride_h": 64, "out_stride_h": 64},
     _abi.IFA4_OK),
    ({"qkv_dtype": _abi.IFA4_FP16, "rel_dtype": _abi.IFA4_BF16}, _abi.IFA4_OK),
    ({"batch": 0, "q": 0, "k": 0}, _abi.IFA4_OK),  # empty batch: nothing is touched
    ({"q": 0}, _abi.IFA4_EINVAL),
    ({"k": 0}, _abi.IFA4_EINVAL),
    # no keys at all: K/V may be null (an empty tensor's storage), nothing is read
    ({"k": 0, "v": 0, "total_k": 0, "max_seqlen_k": 0}, _abi.IFA4_OK),
    ({"q": 0, "out": 0, "total_q": 0, "max_seqlen_q": 0}, _abi.IFA4_OK),
    ({"cu_seqlens_k": 0}, _abi.IFA4_EINVAL),
    ({"rel": 0}, _abi.IFA4_EINVAL),
    ({"rel": 0, "rel_extent": 0}, _abi.IFA4_OK),  # no bias at all
    ({"n_heads": 6, "kv_heads": 4}, _abi.IFA4_EINVAL),
    ({"kv_heads": 0}, _abi.IFA4_EINVAL),
    ({"rel_width": 64}, _abi.IFA4_EINVAL),
    ({"window_left": -2}, _abi.IFA4_EINVAL),
    ({"causal": 2}, _abi.IFA4_EINVAL),
    ({"qkv_dtype": 7}, _abi.IFA4_EINVAL),
    ({"max_seqlen_q": -1}, _abi.IFA4_EINVAL),
    ({"q_stride_t": -8}, _abi.IFA4_EINVAL),
    ({"softmax_scale": float("nan")}, _abi.IFA4_EINVAL),
    ({"head_dim": 96}, _abi.IFA4_EUNSUPPORTED),
    ({"qkv_dtype": _abi.IFA4_FP32}, _abi.IFA4_EUNSUPPORTED),
    ({"softmax_scale": -0.5}, _abi.IFA4_EUNSUPPORTED),
    ({"q": _P + 8}, _abi.IFA4_EUNSUPPORTED),          # 16-byte loads need alignment
    ({"k_stride_t": 2 * 128 + 4}, _abi.IFA4_EUNSUPPORTED),
    ({"lse": 9 * _P, "lse_stride_h": 64}, _abi.IFA4_EINVAL),  # lse rows overlap
    ({"lse": 9 * _P, "lse_stride_h": 128}, _abi.IFA4_OK),
])
def test_validate(kw, expect):
    assert _validate(**kw) == expect


def _first_len_at_limit(stride_bytes, extra_bytes=0):
    """Smallest length L with (L + 128) * stride_bytes + extra_bytes >= 2 GiB."""
    return -(-((1 << 31) - extra_bytes) // stride_bytes) - 128


def test_validate_span_limits():
    """A sequence (plus the 128 rows a tile may read past its end) must span
    less than 2 GiB of K, V, Q and per-token bias: the kernels address it
    through a buffer resource with 32-bit offsets.  Checked one step on each
    side of the limit."""
    lk = _first_len_at_limit(2 * 128 * 2)  # k_stride_t = 256 bf16
    ok = dict(max_seqlen_k=lk - 1, total_k=2 * lk)
    assert _validate(**ok) == _abi.IFA4_OK
    assert _validate(**dict(ok, max_seqlen_k=lk)) == _abi.IFA4_EUNSUPPORTED
    lq = _first_len_at_limit(8 * 128 * 2)  # q_stride_t = 1024 bf16
    ok = dict(max_seqlen_q=lq - 1, total_q=2 * lq)
    assert _validate(**ok) == _abi.IFA4_OK
    assert _validate(**dict(ok, max_seqlen_q=lq)) == _abi.IFA4_EUNSUPPORTED
    # per-token fp32 bias rows of 8 * 128 floats (rel_stride_t = 1024)
    lr = _first_len_at_limit(1024 * 4, extra_bytes=128 * 4)
    ok = dict(max_seqlen_q=lr - 1, total_q=2 * lr, rel_stride_t=1024)
    assert _validate(**ok) == _abi.IFA4_OK
    assert _validate(**dict(ok, max_seqlen_q=lr)) == _abi.IFA4_EUNSUPPORTED


def _decode_ws(**kw):
    a = _good(batch=2, total_q=2, max_seqlen_q=1, **kw)
    return _abi.lib().ifa4_decode_workspace_bytes(ctypes.byref(a))


def test_decode_head_span_limits():
    """Decode addresses the bias of all heads of a token, and the query heads
    of a GQA group, through one buffer resource each: the span over the heads
    must stay below 2 GiB as well.  8 heads, fp32 bias of width 128, bf16 q of
    head_dim 128; one step on each side of the limit.  Prefill addresses every
    head from its own base: head-major layouts past 2 GiB still validate."""
    sh = -(-((1 << 31) // 4 - 128) // 7)  # smallest rel_stride_h with (7 sh + 128) * 4 >= 2 GiB
    assert _decode_ws(rel_stride_h=sh - 1) > 0
    assert _decode_ws(rel_stride_h=sh) == 0
    assert _decode_ws(rel_stride_h=sh, rel_extent=0, rel=0) > 0  # no bias read
    ql = -(-((1 << 31) // 2 - 128) // 7)  # smallest q_stride_h with 7 ql * 2 + 256 >= 2 GiB
    qh = -(-ql // 8) * 8  # the first multiple of 8 (16-byte rows) at or past it
    assert _decode_ws(q_stride_h=qh - 8) > 0
    assert _decode_ws(q_stride_h=qh) == 0
    lib = _abi.lib()
    a = _good(batch=2, total_q=2, max_seqlen_q=1, q_stride_h=qh)
    assert lib.ifa4_decode_fwd(ctypes.byref(a), 256, 1 << 30, None) == _abi.IFA4_EUNSUPPORTED
    # prefill: q as the transpose of a head-major [H, T, D] tensor of >= 2 GiB
    assert _validate(q_stride_h=qh) == _abi.IFA4_OK
    assert _validate(rel_stride_h=sh) == _abi.IFA4_OK
    t = 1 << 21  # tokens: 8 heads x 2M tokens x 128 x 2 bytes = 4 GiB
    assert _validate(q_stride_t=128, q_stride_h=t * 128, total_q=t) == _abi.IFA4_OK


def test_launch_entry_points_reject_bad_args_before_any_launch():
    lib = _abi.lib()
    bad = _good(head_dim=96)
    assert lib.ifa4_prefill_fwd(ctypes.byref(bad), None) == _abi.IFA4_EUNSUPPORTED
    assert lib.ifa4_decode_fwd(ctypes.byref(bad), None, 0, None) == _abi.IFA4_EUNSUPPORTED
    assert lib.ifa4_prefill_fwd(None, None) == _abi.IFA4_EINVAL


def test_decode_workspace_and_contract():
    lib = _abi.lib()
    a = _good(batch=64, total_q=64, max_seqlen_q=1, max_seqlen_k=16384, total_k=600000,
              causal=0)
    ws = lib.ifa4_decode_workspace_bytes(ctypes.byref(a))
    # causal decode sees key 0 only (top-left alignment): one split suffices
    a_causal = _good(batch=64, total_q=64, max_seqlen_q=1, max_seqlen_k=16384, causal=1)
    assert lib.ifa4_decode_workspace_bytes(ctypes.byref(a_causal)) < ws
    tile = _abi.Ifa4Tile()
    assert lib.ifa4_decode_tile(ctypes.byref(a), ctypes.byref(tile)) == _abi.IFA4_OK
    # stream-K: min(896, steps) persistent waves; one (o, lse) partial slot per
    # (segment, wave) pair that can occur = segments + waves; then 2 ints per segment
    segs, group = 64 * 2, 8 // 2
    steps = segs * (16384 // 32)
    waves = min(896, steps)
    assert tile.kv_chunk == 32 * -(-steps // waves)
    assert ws >= (segs + waves) * group * (128 + 1) * 4 + segs * 2 * 4
    # missing / small workspace is reported, nothing launched
    assert lib.ifa4_decode_fwd(ctypes.byref(a), None, 0, None) == _abi.IFA4_EWORKSPACE
    assert lib.ifa4_decode_fwd(ctypes.byref(a), 256, ws - 1, None) == _abi.IFA4_EWORKSPACE
    # decode needs one query per sequence
    b = _good(batch=4, total_q=5, max_seqlen_q=2)
    assert lib.ifa4_decode_workspace_bytes(ctypes.byref(b)) == 0
    assert lib.ifa4_decode_fwd(ctypes.byref(b), 256, 1 << 30, None) == _abi.IFA4_EINVAL
    # GQA groups above 16 are not served by the decode kernels
    c = _good(batch=2, total_q=2, n_heads=32, kv_heads=1, max_seqlen_q=1)
    assert lib.ifa4_decode_fwd(ctypes.byref(c), 256, 1 << 30, None) == _abi.IFA4_EUNSUPPORTED


def test_tile_table_view():
    t = _abi.prefill_tile(128)
    assert (t.block_q, t.block_k) == (128, 64)
    assert t.kv_chunk == 0
    # the reference benchmark's shape (batch 1, 4 heads) splits at S >= 1024 ...
    cfg = autotune_configs.get_preset(4096)
    assert {k: cfg[k] for k in ("BLOCK_Q", "BLOCK_K", "num_warps", "num_stages")} == {
        "BLOCK_Q": t.block_q, "BLOCK_K": t.block_k, "num_warps": t.waves,
        "num_stages": t.stages}
    assert cfg["KV_CHUNK"] > 0 and cfg["KV_CHUNK"] % t.block_k == 0
    assert autotune_configs.get_preset(1024)["KV_CHUNK"] > 0
    # ... short ones and full grids do not
    assert autotune_configs.get_preset(64)["KV_CHUNK"] == 0
    assert autotune_configs.get_preset(4096, batch=8, n_heads=8)["KV_CHUNK"] == 0
    assert autotune_configs.get_preset(1024, batch=8, n_heads=8)["KV_CHUNK"] == 0
    presets = autotune_configs.PRESETS["gfx950"]
    # the reference's layout: (threshold, BLOCK_Q, BLOCK_K, num_warps, num_stages)
    # buckets at the swept lengths, each holding the shape get_preset reports
    assert [b[0] for b in presets["buckets"]] == [1024, 2048, 4096, 8192]
    for b in presets["buckets"]:
        assert b[1:] == presets["default"] == (t.block_q, t.block_k, t.waves, t.stages)
    assert autotune_configs._detect_arch().startswith("gfx")


def _needed_tiles(lens_q, lens_k, causal, window, bq, bk, bottom_right=False):
    """KV tiles holding at least one visible pair, per query tile (brute force
    over the visibility mask; bottom_right: query i at key position i + lk - lq)."""
    n = 0
    for lq, lk in zip(lens_q, lens_k):
        i = torch.arange(lq).unsqueeze(1) + ((lk - lq) if bottom_right else 0)
        j = torch.arange(lk).unsqueeze(0)
        vis = torch.ones(lq, lk, dtype=torch.bool)
        if causal:
            vis &= i >= j
        if window >= 0:
            vis &= (i - j) <= window
        for q0 in range(0, lq, bq):
            cols = vis[q0:q0 + bq].any(0)
            for k0 in range(0, lk, bk):
                n += bool(cols[k0:k0 + bk].any())
    return n


@pytest.mark.parametrize("seed", range(6))
def test_pruning_visits_exactly_the_tiles_with_visible_pairs(seed):
    g = torch.Generator().manual_seed(seed)
    batch = 3
    lens_q = torch.randint(1, 400, (batch,), generator=g).tolist()
    extra = torch.randint(0, 300, (batch,), generator=g).tolist()
    lens_k = [a + b for a, b in zip(lens_q, extra)]
    window = [-1, 63, 5, 200, -1, 0][seed]
    causal = seed != 4
    cu_q = [0] + list(torch.tensor(lens_q).cumsum(0).tolist())
    cu_k = [0] + list(torch.tensor(lens_k).cumsum(0).tolist())
    t = _abi.prefill_tile(128)
    visited, total = _abi.count_tiles(cu_q, cu_k, 1, causal=causal, window_left=window)
    need = _needed_tiles(lens_q, lens_k, causal, window, t.block_q, t.block_k)
    assert visited == need
    all_tiles, _ = _abi.count_tiles(cu_q, cu_k, 1, causal=causal, window_left=window,
                                    no_prune=True)
    assert all_tiles == total


def test_chunked_window_workload_tile_counts():
    """128 new tokens over a 384-key cache, window 63: 2 of 6 KV tiles per
    query tile are visited."""
    cu_q = [128 * b for b in range(17)]
    cu_k = [384 * b for b in range(17)]
    visited, total = _abi.count_tiles(cu_q, cu_k, 8, causal=True, window_left=63)
    assert (visited, total) == (16 * 8 * 2, 16 * 8 * 6)


def _paged_ok(**kw):
    base = dict(block_size=16, block_table=8 * _P, seqused_k=9 * _P, block_table_stride=1024,
                k_stride_block=16 * 2 * 128, v_stride_block=16 * 2 * 128, num_blocks=40000,
                max_blocks_per_seq=1024)
    base.update(kw)
    return _abi.make_paged(**base)


def _decode_args(**kw):
    base = dict(batch=64, total_q=64, max_seqlen_q=1, max_seqlen_k=16384, causal=0,
                cu_seqlens_k=0, total_k=0)
    base.update(kw)
    return _good(**base)


@pytest.mark.parametrize("kw,expect", [
    ({}, _abi.IFA4_OK),
    ({"block_size": 8}, _abi.IFA4_EINVAL),           # 1024 blocks of 8 < 16384 keys
    ({"block_size": 8, "max_blocks_per_seq": 2048}, _abi.IFA4_OK),
    ({"block_size": 12}, _abi.IFA4_EINVAL),          # not a power of two
    ({"block_size": 4, "max_blocks_per_seq": 4096}, _abi.IFA4_EINVAL),
    ({"block_size": 1 << 17}, _abi.IFA4_EINVAL),
    ({"block_table": 0}, _abi.IFA4_EINVAL),
    ({"seqused_k": 0}, _abi.IFA4_EINVAL),
    ({"seqused_k": 9 * _P + 2}, _abi.IFA4_EINVAL),
    ({"num_blocks": 0}, _abi.IFA4_EINVAL),
    ({"max_blocks_per_seq": 1023}, _abi.IFA4_EINVAL),  # cannot address max_seqlen_k
    ({"k_stride_block": 16 * 2 * 128 + 4}, _abi.IFA4_EUNSUPPORTED),
    ({"block_table_stride": -1}, _abi.IFA4_EINVAL),
    ({"block_table_stride": 0}, _abi.IFA4_OK),        # every sequence shares one row
    ({"struct_size": 8}, _abi.IFA4_EINVAL),
])
def test_paged_validation(kw, expect):
    lib = _abi.lib()
    a = _decode_args()
    kv = _paged_ok(**kw)
    ws = lib.ifa4_decode_paged_workspace_bytes(ctypes.byref(a), ctypes.byref(kv))
    # the workspace query accepts exactly the valid descriptions; a valid call
    # without workspace stops at the workspace check, an invalid one before it
    assert (ws > 0) == (expect == _abi.IFA4_OK)
    st = lib.ifa4_decode_paged_fwd(ctypes.byref(a), ctypes.byref(kv), None, 0, None)
    assert st == (_abi.IFA4_EWORKSPACE if expect == _abi.IFA4_OK else expect)


def test_paged_workspace_layout():
    lib = _abi.lib()
    a = _decode_args()
    contiguous = _decode_args(cu_seqlens_k=7 * _P, total_k=600000)
    ws = lib.ifa4_decode_paged_workspace_bytes(ctypes.byref(a), ctypes.byref(_paged_ok()))
    # same layout; a paged cache streams up to 2048 waves (896 contiguous)
    segs, group = 64 * 2, 8 // 2
    assert ws >= (segs + 2048) * group * (128 + 1) * 4 + segs * 2 * 4
    assert ws > lib.ifa4_decode_workspace_bytes(ctypes.byref(contiguous))
    # the contiguous entry points still need cu_seqlens_k
    assert lib.ifa4_decode_workspace_bytes(ctypes.byref(a)) == 0
    assert lib.ifa4_decode_paged_fwd(ctypes.byref(a), None, 256, 1 << 30, None) == \
        _abi.IFA4_EINVAL


@pytest.mark.parametrize("seed", range(6))
def test_pruning_bottom_right_visits_exactly_the_tiles_with_visible_pairs(seed):
    """Bottom-right alignment, with Lq below and above Lk."""
    g = torch.Generator().manual_seed(100 + seed)
    batch = 3
    lens_q = torch.randint(1, 400, (batch,), generator=g).tolist()
    lens_k = [max(1, a + b) for a, b in
              zip(lens_q, torch.randint(-150, 300, (batch,), generator=g).tolist())]
    window = [-1, 63, 5, 200, -1, 0][seed]
    causal = seed != 4
    cu_q = [0] + list(torch.tensor(lens_q).cumsum(0).tolist())
    cu_k = [0] + list(torch.tensor(lens_k).cumsum(0).tolist())
    t = _abi.prefill_tile(128)
    visited, total = _abi.count_tiles(cu_q, cu_k, 1, causal=causal, window_left=window,
                                      bottom_right=True)
    need = _needed_tiles(lens_q, lens_k, causal, window, t.block_q, t.block_k,
                         bottom_right=True)
    assert visited == need


@pytest.mark.parametrize("kw,qkw,paged,expect", [
    ({}, {}, False, _abi.IFA4_OK),
    ({}, {}, True, _abi.IFA4_OK),
    ({}, {"kv_dtype": _abi.IFA4_BF16}, False, _abi.IFA4_EUNSUPPORTED),
    ({}, {"k_scale": 0.0}, False, _abi.IFA4_EINVAL),
    ({}, {"v_scale": float("nan")}, False, _abi.IFA4_EINVAL),
    ({}, {"struct_size": 4}, False, _abi.IFA4_EINVAL),
    ({"n_heads": 16, "kv_heads": 1}, {}, False, _abi.IFA4_OK),            # fp8: groups <= 16
    ({"n_heads": 32, "kv_heads": 1}, {}, False, _abi.IFA4_EUNSUPPORTED),
    ({"k_stride_t": 2 * 128 + 8}, {}, False, _abi.IFA4_EUNSUPPORTED),      # 16-byte fp8 rows
    ({"k_stride_t": 2 * 128 + 16}, {}, False, _abi.IFA4_OK),
    ({"head_dim": 64, "q_stride_h": 64, "k_stride_h": 64, "v_stride_h": 64,
      "out_stride_h": 64, "k_stride_t": 128, "v_stride_t": 128}, {}, True,
     _abi.IFA4_EUNSUPPORTED),                                               # D 64 fp8: blocks >= 16
])
def test_quant_validation(kw, qkw, paged, expect):
    lib = _abi.lib()
    a = _decode_args(cu_seqlens_k=7 * _P, total_k=600000, **kw)
    kv = _paged_ok(block_size=8, max_blocks_per_seq=2048) if paged else None
    qt = _abi.make_quant(k_scale=0.01, v_scale=0.02)
    for k, v in qkw.items():
        setattr(qt, k, v)
    kv_ref = ctypes.byref(kv) if kv is not None else None
    ws = lib.ifa4_decode_quant_workspace_bytes(ctypes.byref(a), kv_ref, ctypes.byref(qt))
    assert (ws > 0) == (expect == _abi.IFA4_OK)
    st = lib.ifa4_decode_quant_fwd(ctypes.byref(a), kv_ref, ctypes.byref(qt), None, 0, None)
    assert st == (_abi.IFA4_EWORKSPACE if expect == _abi.IFA4_OK else expect)
    if expect == _abi.IFA4_OK and not paged:
        if a.kv_heads % 2 == 0 and a.k_stride_h == a.head_dim == 128:
            # adjacent kv heads of an fp8 cache stream in pairs over min(1024,
            # steps) waves: a segment is (sequence, kv head pair) of 2 * group heads
            segs, group, waves = 64 * a.kv_heads // 2, 2 * a.n_heads // a.kv_heads, 1024
        else:
            # one kv head per segment over min(2048, steps) waves
            segs, group, waves = 64 * a.kv_heads, a.n_heads // a.kv_heads, 2048
        assert ws >= (segs + waves) * group * (128 + 1) * 4 + segs * 2 * 4
        assert ws > lib.ifa4_decode_workspace_bytes(ctypes.byref(a))
    assert lib.ifa4_decode_quant_fwd(ctypes.byref(a), kv_ref, None, 256, 1 << 30, None) == \
        _abi.IFA4_EINVAL


def _fp8_ws(paged=False, **kw):
    lib = _abi.lib()
    a = _decode_args(cu_seqlens_k=7 * _P, total_k=600000, **kw)
    kv = _paged_ok(block_size=16, max_blocks_per_seq=1024) if paged else None
    qt = _abi.make_quant(k_scale=0.01, v_scale=0.02)
    return lib.ifa4_decode_quant_workspace_bytes(ctypes.byref(a),
                                                 ctypes.byref(kv) if kv is not None else None,
                                                 ctypes.byref(qt))


def _layout_bytes(segs, group, waves):
    """Decode workspace layout: (segments + waves) partial slots of group heads,
    o rows of 128 fp32 and one lse each (both 256-byte aligned), 2 ints per segment."""
    slots = segs + waves
    o = (slots * group * 128 * 4 + 255) // 256 * 256
    lse = (slots * group * 4 + 255) // 256 * 256
    return o + lse + segs * 2 * 4


@pytest.mark.parametrize("paged", [False, True])
def test_fp8_decode_kv_head_pair_layouts(paged):
    """An fp8 cache of d 128 whose adjacent kv heads sit side by side in each row
    streams them in pairs: the workspace is laid out for batch x Hkv/2 segments
    of 2 x group heads over 1024 waves (1536 for a paged cache).  A padded head
    stride, an odd number of kv heads or more than 8 query heads per pair keep one
    kv head per segment over 2048 waves."""
    pair_waves = 1536 if paged else 1024
    assert _fp8_ws(paged) == _layout_bytes(64 * 1, 8, pair_waves)
    assert _fp8_ws(paged, n_heads=16, kv_heads=4) == _layout_bytes(64 * 2, 8, pair_waves)
    assert _fp8_ws(paged, n_heads=6, kv_heads=2) == _layout_bytes(64 * 1, 6, pair_waves)
    # unpaired: strided heads, 3 kv heads, a group of 8 (16 query heads per pair)
    assert _fp8_ws(paged, k_stride_h=144, v_stride_h=144, k_stride_t=2 * 144,
                   v_stride_t=2 * 144) == _layout_bytes(64 * 2, 4, 2048)
    assert _fp8_ws(paged, n_heads=6, kv_heads=3, k_stride_t=3 * 128,
                   v_stride_t=3 * 128) == _layout_bytes(64 * 3, 2, 2048)
    assert _fp8_ws(paged, n_heads=16, kv_heads=2) == _layout_bytes(64 * 2, 8, 2048)
