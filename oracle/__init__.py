"""CPU oracle for the batch-1 Q4_0 decode path -- TEST INFRASTRUCTURE ONLY.

A restatement, in C (q4_0_ref.c) and numpy, of what the reference
(hxmmxh/Spark-vllm-ascend) computes on this path.  It exists to check the
HIP kernels: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and never as the thing measured or shipped.
The product package does not import it.

Modules:
  bf16       bf16 round-to-nearest-even and helpers
  q4_0       GGUF Q4_0 block format: generator, decode, dequant, GEMV
  ops        add+RMSNorm, per-head RMSNorm, neox RoPE + cos/sin table, SwiGLU
  attention  paged gather, unsplit attention (fp64) and the reference's
             split-KV online softmax with LSE merge
  model      one decoder layer and an N-layer greedy decode, teacher-forced
  cpu_path   the reference's PyTorch CPU path (bf16 weights + F.linear),
             timed as the CPU baseline

How each function is pinned (known-answer tests, closed forms, invariants)
is listed in the function docstrings and exercised in tests/test_oracle_*.py.
Functions with no such pin say "parity unpinned" in their docstring.
"""
