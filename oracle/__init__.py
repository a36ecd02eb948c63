"""ORACLE -- test infrastructure only, never the product.

CPU restatements of WeightFerry's quantized-weight hot path, against which the tests hold the GPU kernels:

* ``lib``         -- ctypes binding of ``wf_oracle.c`` (scalar C restatement; the reference's flat-index formulas,
                     enhancers/gguf_dequant.py:72-256, enhancers/fused_kernels.py:84-174).
* ``np_oracle``   -- numpy restatement written in the block-loop form of the GGML format (a second, independent
                     formulation of the same bits), plus the fp64 GEMM reference.
* ``torch_chain`` -- torch-CPU restatement of ComfyUI-GGUF's dequant op chain (the reference's CPU path: its
                     ``dequantize`` returns None for CPU data, enhancers/gguf_dequant.py:300,308); the CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import this package.
Parity status of each function is listed in the test that pins it.
"""
