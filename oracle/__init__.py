"""CPU oracle of the Talm QLoRA kernel set — TEST INFRASTRUCTURE, not product code.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this package, and only as the checker (or the timed CPU baseline), never as the thing that is
measured or shipped. The product (`talm_amd`) never imports it and has no CPU fallback.

Each function restates one algorithm of the reference (otarernazar-eng/Talm, paths relative to
its root) on the CPU, citing the file:line it follows:

- `nf4`      grouped and per-projection NF4 dequantization (C, bit-exact; numpy twin)
- `norm`     fused (add +) RMSNorm forward / backward
- `rope`     rotary embedding of q and k, forward / backward
- `swiglu`   SwiGLU forward / backward
- `head`     vocabulary-chunked LM head + cross-entropy with the online log-sum-exp and the
             rescaled gradient accumulator, and its closed-form (two-pass) twin
- `codebook` the NF4 level table from its published construction

How each function is pinned (the checks live in tests/test_oracle.py):
- NF4: the level table against the QLoRA normal-quantile construction; the fp32 -> fp16 rounding
  against numpy's IEEE cast on normals, subnormals, ties and overflow; the double rounding of the
  scale against a case where a fused multiply-add differs; the nibble order against the
  reference's own closed form (solution/test_fuzz.py:860-868); C twin == numpy twin.
- norm: float64 closed form, the invariant mean(xhat^2) = 1 - eps * rstd^2, and the backward
  against central finite differences of the forward.
- rope: complex-multiplication form of the rotation, identity at position 0, and the backward as
  the exact adjoint (transpose) of the forward.
- swiglu: silu closed form, and the backward against finite differences.
- head: the online chunked statistics against the direct two-pass float64 formulas (chunk-width
  invariance), the gradient against finite differences of the loss, the argmax against numpy's
  first-maximum on planted ties (solution/test_kernels.py:250-282), the label shift and the
  ignore index (solution/test_kernels.py:497-519).
- every function also against the committed golden fixtures of tests/golden/ (expected values
  from PyTorch: float64 autograd, float32 elementwise ops, a float64 full softmax), in
  tests/test_golden.py. The double-quant code table is such a fixture (an input, not an
  oracle function).
"""
