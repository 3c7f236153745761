"""Split-KV prefill: query tiles whose KV range is cut into chunks, one
workgroup per chunk, partials merged by log-sum-exp in a second pass.

IFA4_FLAG_SPLIT_KV_2 forces chunks of two KV tiles on every call, so small
inputs exercise many chunks, chunk boundaries inside the causal diagonal, the
window edge and the bias band, and query tiles with a single chunk (written
directly) next to split ones.  Each result is compared with the oracle (out
atol/rtol 2e-2, lse 1e-3) and with the unsplit kernel (the same tiles merged
in another order: lse within 1e-4).  The automatic plan is checked on the
reference's own benchmark shape (batch 1, Hq = Hkv = 4, per-token bias of
extent 1024), where the tile table splits (src/inkling_fa4/reference.py:19-40
is the semantics throughout).
"""
import ctypes

import pytest
import torch

from inkling_fa4 import _abi, inkling_fa4_rel_attention, testing
from oracle import ref_rel_attn_with_lse

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3
SPLIT2 = _abi.IFA4_FLAG_SPLIT_KV_2


def _run(case, dev, flags=0, bottom_right=False):
    c = case.to(dev)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, window_size=c.window_size,
                                         softmax_scale=c.scale, return_lse=True,
                                         bottom_right=bottom_right, _flags=flags)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _check_split(case, dev, bottom_right=False):
    print(f"split-KV {case.name}: causal {case.causal}, window {case.window_left}", flush=True)
    got_out, got_lse = _run(case, dev, SPLIT2, bottom_right)
    ref_out, ref_lse = _run(case, dev, 0, bottom_right)
    want_out, want_lse = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                               case.cu_k, case.scale, case.rel_extent,
                                               causal=case.causal,
                                               window_left=case.window_or_none,
                                               bottom_right=bottom_right)
    rows = ~torch.isnan(want_out).any(-1)  # rows with a visible key
    torch.testing.assert_close(got_out.float()[rows], want_out.float()[rows], atol=ATOL,
                               rtol=RTOL)
    torch.testing.assert_close(got_lse.T[rows], want_lse.T[rows], atol=LSE_ATOL, rtol=0)
    assert bool((got_out[~rows] == 0).all()) and bool((got_lse.T[~rows] == float("-inf")).all())
    torch.testing.assert_close(got_out.float(), ref_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got_lse, ref_lse, atol=1e-4, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("causal,window", [(True, -1), (False, -1), (True, 100), (False, 300)])
def test_split_ragged_gqa(cuda, causal, window):
    case = testing.make_case("split", [700, 64, 1, 333, 0, 1030], [700, 64, 1, 333, 0, 1030],
                             8, 2, 128, torch.bfloat16, seed=71, causal=causal,
                             window_left=window, scale=0.2)
    _check_split(case, cuda)


@pytest.mark.gpu
@pytest.mark.parametrize("bottom_right", [False, True])
def test_split_chunked_lq_ne_lk_per_token_bias(cuda, bottom_right):
    case = testing.make_case("split_chunk", [128, 300, 513], [384, 250, 1500], 6, 3, 128,
                             torch.bfloat16, seed=72, causal=True, rel_table=False,
                             rel_std=2.0, rel_extent=200, rel_dtype=torch.bfloat16)
    _check_split(case, cuda, bottom_right)


@pytest.mark.gpu
def test_split_fp16_d64_table(cuda):
    case = testing.make_case("split_d64", [900, 257], [900, 257], 4, 4, 64, torch.float16,
                             seed=73, causal=True, scale=0.125)
    _check_split(case, cuda)


def _workspace_bytes(batch, n_heads, kv_heads, seq, causal=True, flags=0):
    a = _abi.make_args(q=1 << 20, k=1 << 20, v=1 << 20, rel=1 << 20, out=1 << 20,
                       cu_seqlens_q=1 << 20, cu_seqlens_k=1 << 20, q_stride_t=n_heads * 128,
                       q_stride_h=128, k_stride_t=kv_heads * 128, k_stride_h=128,
                       v_stride_t=kv_heads * 128, v_stride_h=128, rel_stride_t=0,
                       rel_stride_h=128, out_stride_t=n_heads * 128, out_stride_h=128,
                       total_q=batch * seq, total_k=batch * seq, batch=batch, n_heads=n_heads,
                       kv_heads=kv_heads, head_dim=128, rel_extent=128, rel_width=128,
                       max_seqlen_q=seq, max_seqlen_k=seq, causal=int(causal), flags=flags,
                       qkv_dtype=_abi.IFA4_BF16, rel_dtype=_abi.IFA4_FP32)
    return _abi.lib().ifa4_prefill_workspace_bytes(ctypes.byref(a)), a


def test_split_plan_on_the_host():
    # enough balanced work for the chip: no split, no workspace
    assert _workspace_bytes(8, 8, 2, 4096)[0] == 0
    assert _workspace_bytes(8, 8, 2, 2048)[0] == 0
    # a full grid of short sequences: no split either (partials cost more)
    assert _workspace_bytes(8, 8, 2, 1024)[0] == 0
    # one sequence of 4096 over 4 heads (128 workgroups): split
    n, a = _workspace_bytes(1, 4, 4, 4096)
    assert n > 0
    lib = _abi.lib()
    assert lib.ifa4_prefill_fwd_ws(ctypes.byref(a), None, 0, None) == _abi.IFA4_EWORKSPACE
    assert lib.ifa4_prefill_fwd_ws(ctypes.byref(a), 1 << 20, n - 1, None) == _abi.IFA4_EWORKSPACE
    # short sequences never split (a single KV tile per query tile)
    assert _workspace_bytes(1, 4, 4, 64)[0] == 0
    # grids of up to half the resident slots split only with long KV ranges:
    # 256 workgroups with 16-tile ranges split, with 8-tile ranges not
    assert _workspace_bytes(8, 4, 4, 1024)[0] > 0
    assert _workspace_bytes(16, 4, 4, 512)[0] == 0
    assert _workspace_bytes(8, 8, 2, 512)[0] == 0
    # 512 workgroups never split
    assert _workspace_bytes(1, 4, 4, 16384)[0] == 0
    # below the slots the chunk is lengthened until the chunks with work fit
    # them at once; the split is taken at half the longest range or less, or
    # when it saves 16 tiles or more
    chunk = lambda batch, heads, seq: _abi.prefill_tile(  # noqa: E731
        128, batch=batch, n_heads=heads, seq_len=seq).kv_chunk // 64
    assert chunk(1, 4, 4096) == 10    # balanced share 9: 528 chunks, 10: 476
    assert chunk(1, 4, 8192) == 43    # 33: 632 chunks, 43: 512
    assert chunk(5, 4, 2048) == 16    # 320 workgroups, ranges of 32 tiles
    assert chunk(3, 4, 4096) == 44    # 384 workgroups, saves 20 of 64 tiles
    assert _workspace_bytes(5, 4, 4, 2048)[0] > 0
    assert _workspace_bytes(3, 4, 4, 4096)[0] > 0
    assert _workspace_bytes(12, 4, 4, 1024)[0] == 0  # 12 of 16 tiles
    assert _workspace_bytes(6, 4, 4, 2048)[0] == 0   # 22 of 32 tiles
    assert _workspace_bytes(7, 8, 8, 1024)[0] == 0   # 14 of 16 tiles
    # the test flag splits everything with more than two tiles per query tile
    assert _workspace_bytes(8, 8, 2, 4096, flags=SPLIT2)[0] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("seq", [1024, 4096])
def test_split_plan_reference_benchmark_shape(cuda, seq):
    """batch 1, Hq = Hkv = 4, head_dim 128, causal, per-token bf16 bias of
    extent 1024 (benchmarks/benchmark_prefill.py:20-49): the table splits it."""
    assert _workspace_bytes(1, 4, 4, seq)[0] > 0
    case = testing.make_case("reference_config", [seq], [seq], 4, 4, 128, torch.bfloat16, seed=74,
                             rel_extent=1024, rel_table=False, rel_dtype=torch.bfloat16,
                             rel_std=1.0)
    print(f"reference benchmark shape, seq {seq}", flush=True)
    got_out, got_lse = _run(case, cuda)
    want_out, want_lse = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                               case.cu_k, case.scale, case.rel_extent,
                                               causal=True)
    torch.testing.assert_close(got_out.float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got_lse, want_lse, atol=LSE_ATOL, rtol=0)
