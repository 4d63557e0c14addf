"""Test oracle for the tattn attention path.

THIS PACKAGE IS TEST INFRASTRUCTURE. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it, and only to check results (or, for the
baseline, as the thing timed on the host CPU). The product package `tattn` never imports it:
on a GPU it runs the HIP kernels or raises.

Contents
--------
- `oracle.reference`: a CPU restatement of the reference's PyTorch algorithms
  (`src/tattn/reference.py`): the materialised definition, the tiled online-softmax forward
  and the FlashAttention-2 backward, in fp32, plus the benchmark's FLOP formula
  (`bench/bench.py:31-35`).
- `oracle.exact`: float64 numpy brute force (definition, log-sum-exp, gradients in closed
  form) that pins `oracle.reference` independently of torch's kernels.

How each function is pinned (none is "parity unpinned"):
- `naive_attention`: against `exact.attention_fwd` (float64 brute force), and against the
  closed-form special cases (N=1 gives O=V; zero queries give the mean / cumulative mean of V;
  key/value permutation invariance when non-causal; causal row 0 gives V_0).
- `tiled_forward`: O against `exact`, block-size independence at 1e-5 (the reference's own
  test, `tests/test_attention.py:80-90`), M against the float64 log-sum-exp in base 2.
- `tiled_backward`: against float64 closed-form gradients (`exact.attention_bwd`) and against
  torch autograd of the definition; special cases N=1 (dQ=dK=0, dV=dO).
- `flops`: against hand-computed values of 4*B*H*N^2*D.
"""
