"""CPU oracle for goda's attention hot path — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
may import this package, and only as the checker (or the timed CPU baseline).
The product path (`goda_amd`) never imports it and has no CPU fallback.

Modules
  attention  restatement of goda's eager attention (PyTorch SDPA on the CPU
             with goda's mask rules), RoPE, ALiBi, KV-cache semantics and the
             split-K log-sum-exp merge; every function cites the reference
             file:line it follows.
  brute      float64 numpy brute force (explicit softmax loops) used to pin
             `attention` on small shapes.

Pinning (see tests/test_oracle.py): every function here is checked against the
float64 brute force, closed forms or invariants chosen so that a dropped term,
a wrong sign or index, or a transposed operand fails a check. The reference
ships no golden vectors for this path, so parity is pinned by those checks
rather than by reference-held fixtures.
"""
