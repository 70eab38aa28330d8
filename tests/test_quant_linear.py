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


# ---- the reference's quantize_model layout: one scale per input feature --------------------

def _wq(method, w, X):
    import quantize

    return quantize.rtn_layer(w, 4) if method == "rtn" else quantize.gptq_layer(w, X, 4)


@pytest.mark.parametrize("method", ["rtn", "gptq"])
@pytest.mark.parametrize("M", [1, 8, 128])
def test_reference_layout_forward(method, M, cuda):
    """What quantize_model writes back (quantize.py:175-179: rtn_layer / gptq_layer with
    group_size=None on W [out, in], fp32 like the reference's model) packed and run: codes
    and per-input scales reproduce wq, and the forward equals x @ wq^T + b within 1e-3, with
    the output in the input's dtype."""
    i, o = 1024, 768
    lin = _linear(i, o, True, 60 + M).to(cuda)
    X = torch.randn(512, i, generator=_gen(61)).to(cuda)
    q = ql.QuantLinear.from_linear(lin, method=method, x=X if method == "gptq" else None)
    assert q.scheme == "per_input"
    wq = _wq(method, lin.weight.detach(), X).float()
    deq = q.dequantized_weight()
    assert float(((deq - wq).abs() / wq.abs().amax(dim=0).clamp_min(1e-30)).max()) < 1e-6
    x = torch.randn(M, i, generator=_gen(62 + M)).to(cuda)
    ref = x @ wq.t() + lin.bias.detach().half().float()
    for dt, tol in ((torch.float32, 1e-3), (torch.float16, 2e-3), (torch.bfloat16, 1e-2)):
        y = q(x.to(dt))
        assert y.dtype == dt and y.shape == (M, o)
        assert oracle.rel_fro(y.float().cpu().numpy(), ref.cpu().numpy()) <= tol, dt


def test_reference_layout_fp16_model(cuda):
    """A half-precision model's written-back weight (wq rounded to fp16) still packs: the
    codes are recovered exactly and the forward matches x @ wq^T."""
    lin = _linear(512, 256, False, 70).to(cuda).half()
    wq = _wq("rtn", lin.weight.detach(), None)
    assert wq.dtype == torch.float16
    q = ql.QuantLinear.from_quantized_weight(wq)
    x = torch.randn(16, 512, generator=_gen(71)).half().to(cuda)
    ref = x.float() @ wq.float().t()
    assert oracle.rel_fro(q(x).float().cpu().numpy(), ref.cpu().numpy()) <= 2e-3


def test_from_quantized_weight_rejects_unquantized(cuda):
    w = torch.randn(64, 128, generator=_gen(72)).to(cuda)
    with pytest.raises(ValueError):
        ql.QuantLinear.from_quantized_weight(w)


def test_quantize_model_gptq_sequential(cuda):
    """quantize_model_int4(method="gptq") against the reference's loop (quantize.py:132-157,
    173-179): each layer's calibration inputs recorded with the layers before it already
    quantized, gptq_layer, the weight written back. Given the same calibration inputs the
    packed model matches that fake-quantized model (GPTQ's rounding decisions depend on
    them, so they are recorded once and passed to both)."""
    torch.manual_seed(0)
    make = lambda: nn.Sequential(_linear(256, 512, True, 80), nn.GELU(), _linear(512, 256, True, 81)).to(cuda)
    data = torch.randn(128, 256, generator=_gen(82)).to(cuda)

    def capture(model, mod):
        seen = []
        h = mod.register_forward_hook(lambda m, inp, out: seen.append(inp[0].detach()))
        with torch.no_grad():
            model(data)
        h.remove()
        return torch.cat(seen).reshape(-1, seen[0].shape[-1])

    fake = make()
    xs = {}
    for k in (0, 2):  # the reference's loop: capture, gptq_layer, write back
        xs[str(k)] = capture(fake, fake[k])
        with torch.no_grad():
            fake[k].weight.data = _wq("gptq", fake[k].weight.data, xs[str(k)])
    packed = make()
    ql.quantize_model_int4(packed, method="gptq", x=xs)
    assert all(isinstance(packed[k], ql.QuantLinear) and packed[k].scheme == "per_input" for k in (0, 2))
    # the callable form sees each layer with the ones before it already packed
    seen = []
    ql.quantize_model_int4(make(), method="gptq", x=lambda name, mod: seen.append(name) or xs[name])
    assert seen == ["0", "2"]
    x = torch.randn(4, 7, 256, generator=_gen(83)).to(cuda)
    with torch.no_grad():
        y = packed(x)
        ref = fake(x)
    assert y.dtype == torch.float32 and y.shape == (4, 7, 256)
    assert oracle.rel_fro(y.cpu().numpy(), ref.cpu().numpy()) <= 2e-3


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_prep_activations_exact(dt, cuda):
    """pk_w4a16_prep_activations: fp16(fp32(x) * s[k] * mul), bit for bit; no scale: the cast."""
    import _pk

    x = (torch.randn(5, 264, generator=_gen(90)) * 3).to(dt)
    s = torch.rand(264, generator=_gen(91)) * 0.01 + 1e-4
    mul = 1.0 / float(s.max())
    y = _pk.w4a16_prep_activations(x.to(cuda), s.to(cuda), mul)
    xf = x.float().numpy()
    ref = ((xf * s.numpy()).astype(np.float32) * np.float32(mul)).astype(np.float16)
    assert np.array_equal(y.cpu().numpy(), ref)
    cast = _pk.w4a16_prep_activations(x.to(cuda), None, 1.0)
    assert np.array_equal(cast.cpu().numpy(), xf.astype(np.float16))


def test_save_load_reference_layout_and_rejections(tmp_path, cuda):
    from safetensors.torch import load_file, save_file

    model = nn.Sequential(_linear(256, 512, True, 95), nn.ReLU(), _linear(512, 256, False, 96)).to(cuda)
    ql.quantize_model_int4(model, method="rtn")
    x = torch.randn(8, 256, generator=_gen(97)).to(cuda)
    y0 = model(x)
    path = str(tmp_path / "q.safetensors")
    ql.save_quantized(model, path)
    fresh = nn.Sequential(nn.Linear(256, 512), nn.ReLU(), nn.Linear(512, 256, bias=False)).to(cuda)
    ql.load_quantized(fresh, path)
    assert fresh[0].scheme == "per_input" and torch.equal(fresh(x), y0)
    # a layer of another shape
    other = nn.Sequential(nn.Linear(256, 520), nn.ReLU(), nn.Linear(520, 256, bias=False)).to(cuda)
    with pytest.raises(ValueError):
        ql.load_quantized(other, path)
    # tensors of the wrong shape, a wrong format name, an old version
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        md = dict(f.metadata())
    tensors = load_file(path)
    bad = dict(tensors)
    bad["0.scales"] = tensors["0.scales"][None, :].contiguous()  # (1, in): would broadcast
    for t, meta in ((bad, md), (tensors, {**md, "format": "something-else"}), (tensors, {**md, "version": "1"})):
        p2 = str(tmp_path / "bad.safetensors")
        save_file(t, p2, metadata=meta)
        fresh = nn.Sequential(nn.Linear(256, 512), nn.ReLU(), nn.Linear(512, 256, bias=False)).to(cuda)
        with pytest.raises(ValueError):
            ql.load_quantized(fresh, p2)


def test_host_activations_raise(cuda):
    """Activations left on the host (of any dtype and row count: the decode fast path, the
    strip call, the input cast and the block GEMM) raise instead of reaching a kernel."""
    torch.manual_seed(7)
    q = ql.QuantLinear.from_linear(nn.Linear(256, 512).to(cuda), 128)
    q(torch.randn(1, 256, device=cuda).half())  # the fast path prepared
    for x in (torch.randn(1, 256).half(), torch.randn(16, 256), torch.randn(16, 256).half(),
              torch.randn(2, 256).bfloat16()):
        with pytest.raises(ValueError, match="GPU|cuda"):
            q(x)
