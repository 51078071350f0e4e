"""CPU oracle for the PKM lookup path — TEST INFRASTRUCTURE ONLY.

A plain restatement, in PyTorch CPU ops, of what the reference computes on this
path. Each function cites the reference file:line it follows. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or, for bench.py, as the timed CPU
baseline) — never as a compute path of the product.

How each function is pinned (checks in tests/test_oracle_*.py):
  eb.eb_forward           F.embedding_bag (library routine), brute-force loops,
                          closed forms (single-entry bag = row copy, linearity)
  eb.eb_backward          autograd of F.embedding_bag, fp64 gradcheck of the
                          forward, brute-force loops
  eb.eb_double_backward   autograd double backward of a differentiable
                          restatement, fp64 gradgradcheck, brute-force loops
  pkm.get_indices         brute force over all n^2 key pairs on tiny tables,
                          numpy argsort on margin-certified tie-free inputs
"""
