"""CPU oracle for the FlatQuant W4A4 hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference library computes on its
PyTorch fallback path (libarry/quant_ops, ``use_cuda=False``):

* ``fq_reference``     — per-token Kronecker transform + dynamic int4 quantize
                          (``src/quant_ops/ops/quantization/flatquant/ops.py:78-130``)
                          and dequantize (``flatquant/ops.py:156-178``);
* ``int4_reference``   — 8-nibble pack / unpack and the int4 GEMM
                          (``src/quant_ops/ops/quantization/int4_matmul/ops.py:23-103``);
* ``decompose``        — ``get_decompose_dim`` (``src/quant_ops/utils/decompose.py:11-39``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or as the timed
CPU baseline). The product package ``quant_ops_amd`` never imports it; its GPU
path fails loudly when the HIP library is missing instead of falling back here.

Pinning (each function is checked against something other than itself, see
``tests/test_oracle.py``):

* transform: brute force ``y = x @ kron(L, R)`` in float64 on small shapes, norm
  preservation for orthogonal transforms, identity transforms;
* scale / quantize: closed forms with explicit rounding to the input dtype,
  ties-to-even known answers, clamp limits, the all-zero fp16 token;
* pack / unpack: the closed form ``word = sum_i (q_i + 8) << 4 i`` and the
  known answers 0x76543210 / -1 / 0;
* GEMM: int64 brute force on small shapes, exact-integer argument for fp32;
* decompose: the docstring known answers ``4096 -> (64, 64)``, ``2048 -> (32, 64)``
  and an exhaustive closed-form check.

No golden vectors ship with the reference (its tests generate CUDA-seeded data at
run time and store nothing), and no part of the reference can be built here
(CUDA sources, no nvcc), so ``oracle/_ref`` stays empty.
"""
