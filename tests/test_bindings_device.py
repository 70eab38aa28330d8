"""Every binding that hands tensor addresses to a kernel refuses tensors that are not on the
GPU (a host address given to a kernel would fault the device instead of failing the call).
Checked without a GPU: the refusal comes before any library call."""

from __future__ import annotations

import pytest
import torch

import _pk

f16, i32, u8 = torch.float16, torch.int32, torch.uint8


def _z(*shape, dtype=torch.float32):
    return torch.zeros(*shape, dtype=dtype)


CASES = [
    ("w4a16_gemm", lambda: _pk.w4a16_gemm(_z(1, 256, dtype=f16), _z(256, 32, dtype=i32), None, 0,
                                          1.0, f16)),
    ("w4a16_gemm_strips", lambda: _pk.w4a16_gemm_strips(_z(1, 256, dtype=f16), _z(256, 32, dtype=i32),
                                                        None, 0, 1.0, f16)),
    ("w4a16_gemm_partials", lambda: _pk.w4a16_gemm_partials(_z(1, 256, dtype=f16),
                                                            _z(256, 32, dtype=i32), None, 0, 2)),
    ("w4a16_prep_activations", lambda: _pk.w4a16_prep_activations(_z(1, 256), None, 1.0)),
    ("splitk_reduce", lambda: _pk.splitk_reduce(_z(2, 1, 8), 1.0, _z(1, 8))),
    ("fp8_gemm", lambda: _pk.fp8_gemm(_z(16, 16, dtype=u8), _z(16, 16, dtype=u8), 1.0, torch.float32)),
    ("gemm_dense", lambda: _pk.gemm_dense(_z(16, 16, dtype=f16), _z(16, 16, dtype=f16),
                                          torch.float32, 1)),
    ("absmax", lambda: _pk.absmax(_z(8))),
    ("cast_e4m3", lambda: _pk.cast_e4m3(_z(8), 1.0)),
    ("quantize_int4", lambda: _pk.quantize_int4(_z(8), 1.0)),
    ("pack_int4", lambda: _pk.pack_int4(_z(2, 8, dtype=torch.int8))),
    ("unpack_int4", lambda: _pk.unpack_int4(_z(2, 4, dtype=u8))),
    ("quantize_group", lambda: _pk.quantize_group(_z(128, 8), 4, 128, half_math=False,
                                                  want_qweight=True, want_scales=True,
                                                  want_fake=False)),
    ("gptq_block", lambda: _pk.gptq_block(_z(8, 8), _z(8, 8), _z(8, 8), 0, 8, 4, 0)),
    ("flash_decode", lambda: _pk.flash_decode(_z(1, 1, 64, dtype=f16), _z(1, 1, 256, 64, dtype=f16),
                                              _z(1, 1, 256, 64, dtype=f16), 128, 0.125)),
]


@pytest.mark.parametrize("name,call", CASES, ids=[c[0] for c in CASES])
def test_host_tensors_are_refused(name, call):
    with pytest.raises(ValueError, match=f"{name}: every tensor must be on one GPU"):
        call()
