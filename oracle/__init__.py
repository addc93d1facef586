"""CPU oracle for diffucore's quantized denoiser hot path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the reference
algorithms that the HIP kernels in ``diffucore_amd`` must reproduce:

* ``oracle.quant``  - per-row int8 quantizer and the ConvRot Hadamard rotation
  (reference ``src/diffucore/models/_int8.py``).
* ``oracle.gemm``   - exact int32 GEMM and the rescale / bias / cast epilogue
  (``_int8.py:200-207, 313-323``; ``kernels/int8_gemm_sm75.cu:31-38``).
* ``oracle.attn``   - K-mean smoothing, per-64-key-block K quantization,
  per-token Q quantization and the INT8-QK / 16-bit-PV attention algorithm
  (``kernels/int8_attn_sm80.cu``).
* ``oracle.cpu_path`` - the reference's own CPU execution path as torch CPU ops,
  timed as the CPU baseline.
* ``oracle.fp`` - exact float32 helpers (fused multiply-add, bf16 rounding).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this package, and only as the checker. The ``diffucore_amd``
package never imports it: its hot path runs on the HIP kernels or raises.
"""
