"""CPU oracle for the fp8 (OCP e4m3) W8A16 linear -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of nemotron_infer's quantized-weight
linear so that the HIP kernels can be checked against it.  It is the checker, never the
thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``nemotron_infer_amd``) never imports it and fails loudly when its HIP library is missing.

Modules
-------
``e4m3``    closed-form OCP E4M3 decode table and the reference's per-row / per-tensor
            quantizers (RNE, clamp to +-448).
``linear``  the torch fp32 dequant-then-``F.linear`` oracle (tools/ref_full_model.py:44-49,
            137), an fp64 brute-force oracle for small shapes, the bf16 RNE closed form and
            the parity metrics (rel_l2, max-abs in bf16 ulp with a magnitude floor).
``cref``    ctypes loader for ``gemv_ref.c``: the reference's sequential fp32 CPU GEMV
            (tests/ops/test_gemm.cu:505-513) restated in plain C.

Pinning (what checks each function against something other than itself)
-----------------------------------------------------------------------
* ``e4m3.decode_lut``  -- torch.float8_e4m3fn's own decode (independent implementation)
  and the OCP spec's fixed points (max 448, min subnormal 2^-9, NaN at 0x7F/0xFF, -0 at 0x80).
* ``e4m3.quantize_rne`` -- torch's float->float8_e4m3fn cast on a dense sweep incl. ties.
* ``linear.linear_fp8_w8a16`` -- fp64 brute force on the committed golden fixtures
  (tests/golden), which are generated from closed-form inputs (test_gemm.cu:311-316,
  540-544) and seeded draws.
* ``cref`` sequential GEMV -- fp64 brute force on the same fixtures (fp32 error bound).
No function of this oracle is "parity unpinned".

The reference itself cannot be compiled here (CUDA/nvcc/cuBLASLt only), so there is no
``oracle/_ref`` build.
"""
