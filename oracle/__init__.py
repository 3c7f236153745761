"""CPU oracle for relative-bias flash attention -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or, for the
baseline, the thing timed on the host).  The product path
(`inkling_fa4`, the HIP library) never imports it and has no CPU fallback.

Contents
  reference.py   fp32 PyTorch restatement of `ref_rel_attn`
                 (reference: src/inkling_fa4/reference.py:4-40), plus the
                 log-sum-exp the reference does not return.
  merge.py       closed-form log-sum-exp merge of split partials (the
                 split-KV decode combine; no reference counterpart).
  rproj.py       relative logits from the RelLogitsProj factors (fp32 einsum),
                 then the oracle (no kernel counterpart in the reference).
  paged.py       paged KV cache (block tables) -> contiguous varlen K/V, and
                 the oracle over a paged cache (the serving format of
                 outputs/architecture.md:117-120; no kernel counterpart in
                 the reference).

How each function is pinned (see tests/test_oracle_*.py):
  ref_rel_attn   golden vectors written by tests/golden/make_golden.py from
                 the reference's own reference.py (12 cases covering every
                 convention: bias sign/extent, top-left causal, left window,
                 NaN rows, dtype rounding, GQA map, stride-0 tables); torch
                 SDPA with an additive mask (independent attention core);
                 Toeplitz structure of stride-0 tables; a float64 loop
                 restatement on tiny shapes; softmax/LSE identities.
  lse output     scipy.special.logsumexp of the masked scores (independent
                 library routine) and sum_j exp(s_ij - lse_i) == 1.
  merge_partials split-count invariance (1, 2, 7 and one split per key) and
                 equality with the unsplit oracle.
  rel_logits_from_proj  an explicit loop on a tiny shape; a rank-one W that
                 reproduces a per-head table.
  gather_paged   identity tables reproduce the contiguous cache; invariance
                 under physical block permutation and block size; rows no
                 sequence owns (NaN-filled) never reach the result.
"""
from .reference import ref_rel_attn, ref_rel_attn_with_lse  # noqa: F401
from .merge import merge_partials  # noqa: F401
from .paged import gather_paged, ref_rel_attn_paged_with_lse  # noqa: F401
from .rproj import ref_rel_attn_rproj_with_lse, rel_logits_from_proj  # noqa: F401
