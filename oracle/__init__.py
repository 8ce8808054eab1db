"""CPU oracle of the attention and residual+LayerNorm hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as
the checker (or the timed CPU baseline) - never as a product code path.  The
product (``triton-transformer-kernels_amd/transformer_opt``) never imports it.

Contents (each function cites the reference file:line it restates):

* ``attention``: the reference's explicit PyTorch attention
  (transformer_opt/dispatch.py:69-96 and
  benchmarks/torch_transformer_benchmark.py:97-111), its kernel-contract
  variant (all-masked rows give zeros, transformer_opt/kernels/
  attention.py:253-254), a chunked form for large shapes, and an independent
  float64 brute force used to pin the restatement.
* ``layernorm``: the fused residual + LayerNorm semantics
  (transformer_opt/kernels/residual_layer_norm.py:95-126) in explicit torch
  ops, plus a float64 brute force.
* ``model``: the organizer's explicit pre-LN Transformer, weight copy, random
  cases and comparator (benchmarks/torch_transformer_benchmark.py:29-356).

The reference is Python (PyTorch + Triton), so there is no C reference to
build into ``oracle/_ref``; the restatement is pinned by the float64 brute
force, by library routines (``F.scaled_dot_product_attention``,
``F.layer_norm``, ``nn.TransformerEncoderLayer``), by closed forms and by the
invariants listed in tests/test_oracle.py.
"""
