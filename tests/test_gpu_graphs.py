"""HIP graph capture of the torch ops, the form a serving loop replays.

Each op is captured once in a torch.cuda.CUDAGraph (hipGraph on ROCm) with
static input tensors, then replayed three times.  Before each replay the
static inputs get new values and an eager call of the same op runs on other
tensors (the program's own work between replays), with a synchronisation
after it; every replay's output must equal, bit for bit, an eager call on the
same inputs (the kernels are deterministic: no atomics, fixed merge order).
The captured path allocates its outputs and workspaces from the graph's pool
and records no memset.  Covers prefill (unsplit, and split KV with its merge
pass), decode on a contiguous, a paged and an fp8 cache.
"""
import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_paged, testing)

pytestmark = pytest.mark.gpu


def _prefill_case(split, seed):
    if split:  # batch 1 over 4 heads: the tile table splits this grid
        return testing.make_case("graph_split", [1500], [1500], 4, 4, 128, torch.bfloat16,
                                 seed=seed, rel_extent=1024, rel_table=False,
                                 rel_dtype=torch.bfloat16)
    return testing.make_case("graph_prefill", [700, 64, 33], [700, 64, 33], 8, 2, 128,
                             torch.bfloat16, seed=seed)


def _decode_case(seed):
    return testing.make_case("graph_decode", [1] * 6, [300, 5000, 1234, 1, 70, 2048], 8, 2,
                             128, torch.bfloat16, seed=seed, causal=False)


def _runner(kind, case, dev):
    """fn(static) -> outputs, and the static tensors it reads."""
    c = case.to(dev)
    if kind.startswith("prefill"):
        static = {"q": c.q, "k": c.k, "v": c.v, "rel": c.rel}
        return (lambda s: inkling_fa4_rel_attention(
            s["q"], s["k"], s["v"], s["rel"], c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
            causal=True, return_lse=True)), static
    if kind == "decode_paged":
        pk = testing.paginate(case, block_size=16, seed=3, spare_blocks=2, fill=0.0).to(dev)
        static = {"q": c.q, "k": pk.k_cache, "v": pk.v_cache, "rel": c.rel}
        return (lambda s: inkling_fa4_rel_attention_decode_paged(
            s["q"], s["k"], s["v"], s["rel"], c.cu_q, pk.seqused_k, pk.block_table, c.max_q,
            c.max_k, c.rel_extent, causal=False, return_lse=True)), static
    if kind == "decode_fp8":
        k8, v8, ks, vs, _ = testing.fp8_kv(case)
        static = {"q": c.q, "k": k8.to(dev), "v": v8.to(dev), "rel": c.rel}
        return (lambda s: inkling_fa4_rel_attention_decode(
            s["q"], s["k"], s["v"], s["rel"], c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
            causal=False, return_lse=True, k_scale=ks, v_scale=vs)), static
    static = {"q": c.q, "k": c.k, "v": c.v, "rel": c.rel}
    return (lambda s: inkling_fa4_rel_attention_decode(
        s["q"], s["k"], s["v"], s["rel"], c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=False, return_lse=True)), static


@pytest.mark.parametrize("kind", ["prefill", "prefill_split", "decode", "decode_paged",
                                  "decode_fp8"])
def test_graph_replays_equal_eager_calls(cuda, kind):
    make = (lambda seed: _prefill_case(kind == "prefill_split", seed)) \
        if kind.startswith("prefill") else _decode_case
    fn, static = _runner(kind, make(81), cuda)
    print(f"graph capture: {kind}", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up before capture, as torch asks
        for _ in range(2):
            fn(static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, g_lse = fn(static)
    other_fn, other = _runner(kind, make(99), cuda)
    for replay in range(3):
        _, fresh = _runner(kind, make(82 + replay), cuda)  # new values, same shapes
        for name, t in static.items():
            if t.stride(0) == 0:  # a per-head table shared by every token
                t[0].copy_(fresh[name][0])
            else:
                t.copy_(fresh[name])
        other_fn(other)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_out, want_lse = fn(static)
        torch.cuda.synchronize()
        print(f"  replay {replay}", flush=True)
        assert torch.equal(g_out, want_out), f"{kind}: replay {replay} out differs"
        assert torch.equal(g_lse, want_lse), f"{kind}: replay {replay} lse differs"
