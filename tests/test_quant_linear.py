"""QuantLinear (the packed-int4 nn.Linear that calls the W4A16 kernel) on the GPU: its codes
and scales are rtn_layer's (quantize.py:63-68) on W^T, its forward equals x @ (q*s)^T + b,
quantize_model_int4 swaps a model's linear layers, and save/load reproduces outputs bit for
bit. Row counts 1, 8 and 128 run the GEMV, the register-dequant kernel and the GEMM."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

import oracle
import quant_linear as ql

pytestmark = pytest.mark.gpu


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _linear(i, o, bias, seed):
    lin = nn.Linear(i, o, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(o, i, generator=_gen(seed)) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(o, generator=_gen(seed + 1)) * 0.1)
    return lin


@pytest.mark.parametrize("M", [1, 8, 128])
@pytest.mark.parametrize("bias", [True, False])
def test_from_linear_matches_rtn_and_closed_form(M, bias, cuda):
    i, o = 1024, 768
    lin = _linear(i, o, bias, 10 + M)
    q = ql.QuantLinear.from_linear(lin.to(cuda).half(), 128)
    w_kn = lin.weight.detach().cpu().half().t().contiguous().numpy()
    codes, _, s16 = oracle.rtn_group_codes(w_kn, 4, 128)
    deq = codes.astype(np.float32) * s16.astype(np.float32).repeat(128, axis=0)
    assert np.array_equal(q.dequantized_weight().t().cpu().numpy(), deq)
    x = torch.randn(M, i, generator=_gen(20 + M)).half()
    y = q(x.to(cuda))
    ref = x.float().numpy() @ deq
    if bias:
        ref = ref + lin.bias.detach().cpu().half().float().numpy()
    assert y.dtype == torch.float16 and y.shape == (M, o)
    assert oracle.rel_fro(y.float().cpu().numpy(), ref) <= 2e-3


def test_leading_dims_and_model_swap(cuda):
    torch.manual_seed(0)
    model = nn.Sequential(_linear(512, 1024, True, 30), nn.GELU(), _linear(1024, 512, True, 31)).to(cuda).half()
    x = torch.randn(2, 5, 512, generator=_gen(32)).half().to(cuda)
    ql.quantize_model_int4(model, 128)
    assert all(isinstance(model[k], ql.QuantLinear) for k in (0, 2))
    y = model(x)
    assert y.shape == (2, 5, 512)
    # reference: the same dequantized weights in fp32
    h = x.float() @ model[0].dequantized_weight().t() + model[0].bias.float()
    h = torch.nn.functional.gelu(h.half().float())
    ref = h @ model[2].dequantized_weight().t() + model[2].bias.float()
    assert oracle.rel_fro(y.float().cpu().numpy(), ref.cpu().numpy()) <= 5e-3


def test_save_load_reproduces_outputs(tmp_path, cuda):
    model = nn.Sequential(_linear(256, 512, True, 40), nn.ReLU(), _linear(512, 256, False, 41)).to(cuda).half()
    ql.quantize_model_int4(model, 128)
    x = torch.randn(8, 256, generator=_gen(42)).half().to(cuda)
    y0 = model(x)
    path = str(tmp_path / "q.safetensors")
    ql.save_quantized(model, path)
    fresh = nn.Sequential(nn.Linear(256, 512), nn.ReLU(), nn.Linear(512, 256, bias=False)).to(cuda).half()
    ql.load_quantized(fresh, path)
    assert torch.equal(fresh(x), y0)
