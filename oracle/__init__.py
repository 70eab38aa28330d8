"""CPU oracle for the quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithm of every function on the path
(pico-kernels: quantize.py, gemm_int4.py, gemm_fp8.py, gemm_splitk.py; each function cites
the file:line it follows). It exists to check the HIP library, never to run in its place:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it, and the product modules in ``pico-kernels_amd/`` never do.

How each function is pinned (see the tests named in brackets):

* ``e4m3_from_f32`` / ``e4m3_to_f32``: exhaustive over all 65536 fp16 inputs and 2^20 fp32
  samples against torch's ``float8_e4m3fn`` cast (the library routine the reference calls at
  gemm_fp8.py:95), plus the OCP table of all 256 codes [tests/test_oracle.py].
* ``quantize_int4``, ``quantize_col``, ``rtn_layer``, ``fp8_quantize``: golden vectors written by
  importing the reference's own CPU functions in the build container
  (tests/golden/make_golden.py), checked bit for bit [tests/test_oracle.py].
* ``pack_int4_n`` / ``unpack_int4_n``: closed form + lossless round trip over every code,
  and the golden vectors.
* ``gptq_layer``: golden vectors (tolerance, fp32 linear algebra), the reference's own
  invariants (act-order permutation consistency, beats RTN) and the closed form that a
  diagonal Hessian reduces it to RTN. Its column loop is ``gptq_sweep``, which the golden
  vectors therefore pin as well.
* GEMM references (``w4a16_ref``, ``int4_gemm_ref``, ``fp8_gemm_ref``): the reference tests'
  closed forms (tests/test_gemm_int4.py:26, tests/test_gemm_fp8.py:24), checked against
  float64 integer-exact products and brute force on small shapes.
* ``decode_attention_ref`` (flash_decoding.eager_decode, flash_decoding.py:126-133): closed
  forms of the softmax-weighted sum (constant V, identical keys, N = 1, a dominant score).
"""

from .quant import (  # noqa: F401
    E4M3_MAX,
    e4m3_from_f32,
    e4m3_to_f32,
    fp8_quantize,
    gptq_layer,
    gptq_sweep,
    pack_int4_n,
    quantize_col,
    quantize_int4,
    rtn_group_codes,
    rtn_layer,
    unpack_int4_n,
)
from .gemm import (  # noqa: F401
    fp8_gemm_ref,
    int4_gemm_ref,
    rel_fro,
    splitk_ref,
    w4a16_ref,
)
from .attention import decode_attention_ref  # noqa: F401
