"""CPU oracle for the mlx-train-perf hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in PyTorch-CPU fp32/fp64, the reference's own naive/stock algorithms for the
two hot-path parts (fused linear cross-entropy; flash attention with GQA / causal / packed masks).
It is the checker the GPU kernels are compared against and the CPU baseline `bench.py` reports.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it, and only
as the checker or the timed CPU baseline -- never as a product path. The product package
(`mlx-train-perf_amd/mlx_train_perf`) never imports it and fails loudly when its HIP extension is
missing.

Pinning (each function's docstring cites the reference file:line it follows):
- lce.naive_forward / lce.forward: the reference's hand-computed KAT (tests/test_naive.py:9-19),
  the closed-form invariants lse >= max logit, nll >= 0, chunk-boundary independence
  (tests/test_chunked.py:95-99), and the committed golden fixtures under tests/golden/.
- lce.backward: torch autograd of lce.forward (an independent differentiation of the closed form),
  the per-row invariant sum_v (p - onehot) = 0, and finite differences on tiny shapes.
- quant.quantize_affine / dequantize_affine: the documented MLX affine formula and nibble order
  (typings/mlx/core/__init__.pyi:3229-3246,3298-3302) and the positional KAT of
  tests/test_quant_layout.py:5-16 (k in {0, 1, 7, 8, 63}).
- attention.attention_forward: the row-0 closed form (tests/test_attention_kernel_fwd.py:522-544),
  the constant-V GQA discriminator (tests/test_attention_reference.py:111-136), an independently
  built logsumexp (tests/test_attention_reference.py:56-80).
- attention.attention_backward: torch autograd of attention_forward and finite differences
  (recipe of tests/test_attention_reference.py:139-202).
- attention.segment_allowed: the 4x4 KAT of tests/test_attention_segments.py:68-87 and the
  per-segment composition identity (tests/test_attention_segments.py:32-57, 90-131).
"""
