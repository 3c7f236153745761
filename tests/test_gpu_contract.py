"""The boundary's contract, end to end.

* The ctypes bindings that INTEGRATION.md shows a maintainer adding on the
  reference side (`prefill_via_c_abi`, `decode_via_c_abi` with its workspace)
  are taken verbatim from that file, executed, and their output compared with
  the oracle (out atol/rtol 2e-2, lse 1e-3): the documented bindings are the
  tested ones.
* cu_seqlens are read only on the device, where each sequence's range is
  clamped to the tensors' rows (include/ifa4.h).  A cu_seqlens_k whose last
  offset runs past total_k gives exactly the result of the clamped array, and
  decode with a cu_seqlens_q that is not arange writes out = 0, lse = -inf
  for the rows of the sequence that holds two queries, while the sequence
  with one query is decoded as usual.
"""
import os
import re

import pytest
import torch

from inkling_fa4 import inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode, testing
from oracle import ref_rel_attn, ref_rel_attn_with_lse

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _integration_binding(name="prefill_via_c_abi"):
    """The python block of INTEGRATION.md that defines `name`, executed."""
    with open(os.path.join(REPO, "INTEGRATION.md")) as f:
        text = f.read()
    blocks = [b for b in re.findall(r"```python\n(.*?)```", text, re.S)
              if f"def {name}" in b]
    assert len(blocks) == 1, f"INTEGRATION.md holds one {name} binding"
    ns = {}
    exec(compile(blocks[0], f"INTEGRATION.md:{name}", "exec"), ns)
    return ns[name]


def test_integration_binding_compiles():
    assert callable(_integration_binding())
    assert callable(_integration_binding("decode_via_c_abi"))


@pytest.mark.gpu
@pytest.mark.parametrize("causal,window", [(True, -1), (False, 40)])
def test_integration_binding_matches_oracle(cuda, causal, window):
    prefill_via_c_abi = _integration_binding()
    case = testing.make_case("ctypes", [64, 33, 17, 200], [64, 33, 17, 260], 8, 2, 128,
                             torch.bfloat16, seed=51, causal=causal, window_left=window)
    c = case.to(cuda)
    print(f"ctypes binding: causal {causal}, window {window}", flush=True)
    out = prefill_via_c_abi(c.q, c.k, c.v, c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k,
                            c.rel_extent, causal=causal, window_left=window, scale=c.scale)
    torch.cuda.synchronize()
    want = ref_rel_attn(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k, case.scale,
                        case.rel_extent, causal=causal, window_left=case.window_or_none)
    torch.testing.assert_close(out.cpu().float(), want.float(), atol=ATOL, rtol=RTOL)
    # the torch binding on the same inputs (it may split the KV range of this
    # small grid and merge the chunks: equal up to that rounding)
    ref = inkling_fa4_rel_attention(*c.args(), causal=causal, window_size=c.window_size,
                                    softmax_scale=c.scale)
    torch.testing.assert_close(out.float(), ref.float(), atol=1e-2, rtol=1e-2)


@pytest.mark.gpu
def test_integration_decode_binding_matches_oracle(cuda):
    decode_via_c_abi = _integration_binding("decode_via_c_abi")
    lens_k = [300, 5000, 1234, 1, 70]
    case = testing.make_case("ctypes_decode", [1] * 5, lens_k, 8, 2, 128, torch.bfloat16,
                             seed=54, causal=False)
    c = case.to(cuda)
    print("ctypes decode binding: 5 caches", flush=True)
    out, lse = decode_via_c_abi(c.q, c.k, c.v, c.rel, c.cu_q, c.cu_k, c.max_k, c.rel_extent,
                                scale=c.scale)
    torch.cuda.synchronize()
    want_out, want_lse = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                               case.cu_k, case.scale, case.rel_extent,
                                               causal=False)
    torch.testing.assert_close(out.cpu().float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.cpu(), want_lse, atol=LSE_ATOL, rtol=0)


@pytest.mark.gpu
def test_prefill_cu_seqlens_k_past_total_is_clamped(cuda):
    case = testing.make_case("clamp", [64, 33, 17], [64, 33, 17], 8, 2, 128, torch.bfloat16,
                             seed=52, causal=False)
    c = case.to(cuda)
    bad_k = torch.tensor([0, 64, 97, 114 + 1000], dtype=torch.int32, device=cuda)
    print("prefill with cu_seqlens_k[-1] past total_k", flush=True)
    got, lse = inkling_fa4_rel_attention(c.q, c.k, c.v, c.rel, c.cu_q, bad_k, c.max_q,
                                         c.max_k + 1000, c.rel_extent, causal=False,
                                         softmax_scale=c.scale, return_lse=True)
    # same max_seqlen_k, so that both calls get the same tile plan
    want, want_lse = inkling_fa4_rel_attention(c.q, c.k, c.v, c.rel, c.cu_q, c.cu_k, c.max_q,
                                               c.max_k + 1000, c.rel_extent, causal=False,
                                               softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(lse, want_lse)


@pytest.mark.gpu
def test_decode_cu_seqlens_q_not_arange(cuda):
    lens_k = [300, 5000, 1234]
    case = testing.make_case("dec_cuq", [1, 1, 1], lens_k, 8, 2, 128, torch.bfloat16, seed=53,
                             causal=False)
    c = case.to(cuda)
    cu_q = torch.tensor([0, 0, 2, 3], dtype=torch.int32, device=cuda)  # 0, 2 and 1 queries
    print("decode with cu_seqlens_q = [0, 0, 2, 3]", flush=True)
    out, lse = inkling_fa4_rel_attention_decode(c.q, c.k, c.v, c.rel, cu_q, c.cu_k, 2, c.max_k,
                                                c.rel_extent, causal=False,
                                                softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    out, lse = out.cpu(), lse.cpu()
    assert torch.equal(out[:2], torch.zeros_like(out[:2]))
    assert bool((lse[:, :2] == float("-inf")).all())
    # row 2 is sequence 2's single query against its own keys
    ks = int(case.cu_k[2])
    one = torch.tensor([0, 1], dtype=torch.int32)
    want_out, want_lse = ref_rel_attn_with_lse(
        case.q[2:3], case.k[ks:], case.v[ks:], case.rel[2:3], one,
        torch.tensor([0, lens_k[2]], dtype=torch.int32), case.scale, case.rel_extent,
        causal=False)
    torch.testing.assert_close(out[2:].float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[:, 2:], want_lse, atol=LSE_ATOL, rtol=0)
