"""Allocation-free decode (ifa4_decode_fwd_noalloc) through the C ABI.

Two calls in a row, the second on a smaller input, each compared with
ifa4_decode_fwd on a caller-allocated workspace (the same kernels, so the
results must be bit-identical) and with the oracle (out atol/rtol 2e-2, lse
1e-3).  The host-side checks (a call needing more than the scratch array,
malformed arguments) are exercised without a GPU: they return before any
device call.
"""
import ctypes

import pytest
import torch

from inkling_fa4 import _abi, testing
from oracle import ref_rel_attn_with_lse

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3
SCRATCH_BYTES = 32 << 20  # IFA4_DECODE_SCRATCH_BYTES
_P = 1 << 20              # fake, aligned device address (never dereferenced)


def _args(c, out, lse):
    q, k, v, rel = c.q, c.k, c.v, c.rel
    return _abi.make_args(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), rel=rel.data_ptr(), out=out.data_ptr(),
        lse=lse.data_ptr(), cu_seqlens_q=c.cu_q.data_ptr(), cu_seqlens_k=c.cu_k.data_ptr(),
        q_stride_t=q.stride(0), q_stride_h=q.stride(1), k_stride_t=k.stride(0),
        k_stride_h=k.stride(1), v_stride_t=v.stride(0), v_stride_h=v.stride(1),
        rel_stride_t=rel.stride(0), rel_stride_h=rel.stride(1), out_stride_t=out.stride(0),
        out_stride_h=out.stride(1), lse_stride_h=lse.stride(0), total_q=q.shape[0],
        total_k=k.shape[0], batch=c.cu_q.numel() - 1, n_heads=q.shape[1], kv_heads=k.shape[1],
        head_dim=q.shape[2], rel_extent=c.rel_extent, rel_width=rel.shape[2],
        max_seqlen_q=c.max_q, max_seqlen_k=c.max_k, window_left=c.window_left,
        causal=int(c.causal), softmax_scale=c.scale, qkv_dtype=_abi.IFA4_BF16,
        rel_dtype=_abi.IFA4_FP32)


def _run_both(c):
    """(out, lse) from the allocation-free entry point and from ifa4_decode_fwd."""
    lib = _abi.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = []
    for noalloc in (True, False):
        out = torch.empty_like(c.q)
        lse = torch.empty(c.q.shape[1], c.q.shape[0], dtype=torch.float32, device=c.q.device)
        a = _args(c, out, lse)
        if noalloc:
            st = lib.ifa4_decode_fwd_noalloc(ctypes.byref(a), stream)
        else:
            n = lib.ifa4_decode_workspace_bytes(ctypes.byref(a))
            assert 0 < n <= SCRATCH_BYTES
            ws = torch.empty(n, dtype=torch.uint8, device=c.q.device)
            st = lib.ifa4_decode_fwd(ctypes.byref(a), ctypes.c_void_p(ws.data_ptr()), n, stream)
        assert st == _abi.IFA4_OK, _abi.status_str(st)
        res.append((out, lse))
    torch.cuda.synchronize()
    return res


@pytest.mark.gpu
def test_noalloc_decode_matches_workspace_entry_point(cuda):
    first = testing.decode(seed=61, batch=24, lo=1000, hi=9000, causal=False)
    second = testing.decode(seed=62, batch=5, lo=40, hi=3000, causal=False)
    for case in (first, second):
        c = case.to(cuda)
        print(f"noalloc decode: batch {c.cu_q.numel() - 1}, max_k {c.max_k}", flush=True)
        (out_na, lse_na), (out_ws, lse_ws) = _run_both(c)
        assert torch.equal(out_na, out_ws) and torch.equal(lse_na, lse_ws)
        want_out, want_lse = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                                   case.cu_k, case.scale, case.rel_extent,
                                                   causal=False)
        torch.testing.assert_close(out_na.cpu().float(), want_out.float(), atol=ATOL, rtol=RTOL)
        torch.testing.assert_close(lse_na.cpu(), want_lse, atol=LSE_ATOL, rtol=0)


def _fake(batch, max_k):
    return _abi.make_args(
        q=_P, k=_P, v=_P, rel=_P, out=_P, cu_seqlens_q=_P, cu_seqlens_k=_P, q_stride_t=1024,
        q_stride_h=128, k_stride_t=256, k_stride_h=128, v_stride_t=256, v_stride_h=128,
        rel_stride_t=0, rel_stride_h=128, out_stride_t=1024, out_stride_h=128,
        total_q=batch, total_k=batch * max_k, batch=batch, n_heads=8, kv_heads=2,
        head_dim=128, rel_extent=128, rel_width=128, max_seqlen_q=1, max_seqlen_k=max_k,
        causal=0, softmax_scale=0.1, qkv_dtype=_abi.IFA4_BF16, rel_dtype=_abi.IFA4_FP32)


def test_noalloc_rejects_oversize_and_bad_arguments_on_the_host():
    lib = _abi.lib()
    small = _fake(64, 16384)
    assert 0 < lib.ifa4_decode_workspace_bytes(ctypes.byref(small)) <= SCRATCH_BYTES
    big = _fake(20000, 4096)
    assert lib.ifa4_decode_workspace_bytes(ctypes.byref(big)) > SCRATCH_BYTES
    assert lib.ifa4_decode_fwd_noalloc(ctypes.byref(big), None) == _abi.IFA4_EWORKSPACE
    bad = _fake(64, 16384)
    bad.kv_heads = 3  # 8 heads are not a multiple of 3
    assert lib.ifa4_decode_fwd_noalloc(ctypes.byref(bad), None) == _abi.IFA4_EINVAL
    two_queries = _fake(64, 16384)
    two_queries.total_q = 65
    assert lib.ifa4_decode_fwd_noalloc(ctypes.byref(two_queries), None) == _abi.IFA4_EINVAL
    empty = _fake(0, 16384)
    assert lib.ifa4_decode_fwd_noalloc(ctypes.byref(empty), None) == _abi.IFA4_OK
