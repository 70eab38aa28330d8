"""The packed on-disk format of quant_linear (safetensors + metadata), on the CPU: a model's
QuantLinear layers round-trip bit for bit, an nn.Linear of the same shape is replaced on
load, and files of another format are refused."""

from __future__ import annotations

import pytest
import torch
from torch import nn

import quant_linear as ql


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _random_qlinear(i: int, o: int, bias: bool, seed: int, group: int = 128) -> ql.QuantLinear:
    q = ql.QuantLinear(i, o, bias, group)
    g = _gen(seed)
    q.qweight.copy_(torch.randint(-2**31, 2**31 - 1, q.qweight.shape, generator=g, dtype=torch.int64).to(torch.int32))
    q.scales.copy_((torch.rand(q.scales.shape, generator=g) * 0.01).half())
    if bias:
        q.bias.copy_(torch.randn(o, generator=g).half())
    return q


def test_round_trip_and_replace(tmp_path):
    src = nn.Sequential(_random_qlinear(256, 64, True, 1), nn.ReLU(), _random_qlinear(128, 32, False, 2, 64))
    path = str(tmp_path / "m.safetensors")
    ql.save_quantized(src, path)
    dst = nn.Sequential(nn.Linear(256, 64), nn.ReLU(), nn.Linear(128, 32, bias=False))
    ql.load_quantized(dst, path)
    for a, b in ((src[0], dst[0]), (src[2], dst[2])):
        assert isinstance(b, ql.QuantLinear) and b.group_size == a.group_size
        assert torch.equal(a.qweight, b.qweight) and torch.equal(a.scales, b.scales)
        assert (a.bias is None) == (b.bias is None)
        if a.bias is not None:
            assert torch.equal(a.bias, b.bias)


def test_metadata_and_foreign_files(tmp_path):
    from safetensors import safe_open
    from safetensors.torch import save_file

    path = str(tmp_path / "m.safetensors")
    ql.save_quantized(nn.Sequential(_random_qlinear(128, 16, True, 3)), path)
    with safe_open(path, framework="pt") as f:
        md = f.metadata()
    assert md["format"] == ql.FORMAT and md["version"] == "1"
    other = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(2)}, other, metadata={"format": "something-else"})
    with pytest.raises(AssertionError):
        ql.load_quantized(nn.Sequential(nn.Linear(128, 16)), other)
    with pytest.raises(AssertionError):  # shape mismatch
        ql.load_quantized(nn.Sequential(nn.Linear(256, 16)), path)


def test_shape_contract():
    with pytest.raises(AssertionError):
        ql.QuantLinear(100, 64)  # in_features not a multiple of the group
    with pytest.raises(AssertionError):
        ql.QuantLinear(128, 60)  # out_features not whole int32 words
