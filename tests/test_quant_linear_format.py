"""The packed on-disk format of quant_linear (safetensors + metadata), on the CPU: a model's
QuantLinear layers (group and per-input layouts) round-trip bit for bit, an nn.Linear of the
same shape is replaced on load, and files of another format or version, layers of another
shape and tensors of another shape or dtype are refused with ValueError before anything is
copied."""

from __future__ import annotations

import pytest
import torch
from torch import nn

import quant_linear as ql


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _random_qlinear(i: int, o: int, bias: bool, seed: int, group: int = 128,
                    scheme: str = "group") -> ql.QuantLinear:
    q = ql.QuantLinear(i, o, bias, group, scheme=scheme)
    g = _gen(seed)
    q.qweight.copy_(torch.randint(-2**31, 2**31 - 1, q.qweight.shape, generator=g, dtype=torch.int64).to(torch.int32))
    q.scales.copy_((torch.rand(q.scales.shape, generator=g) * 0.01).to(q.scales.dtype))
    if bias:
        q.bias.copy_(torch.randn(o, generator=g).half())
    return q


def test_round_trip_and_replace(tmp_path):
    src = nn.Sequential(_random_qlinear(256, 64, True, 1), nn.ReLU(), _random_qlinear(128, 32, False, 2, 64),
                        nn.ReLU(), _random_qlinear(32, 96, True, 4, scheme="per_input"))
    path = str(tmp_path / "m.safetensors")
    ql.save_quantized(src, path)
    dst = nn.Sequential(nn.Linear(256, 64), nn.ReLU(), nn.Linear(128, 32, bias=False), nn.ReLU(),
                        nn.Linear(32, 96))
    ql.load_quantized(dst, path)
    assert dst[4].scheme == "per_input" and dst[4].scales.dtype == torch.float32
    assert dst[4]._smax == float(src[4].scales.max())
    for a, b in ((src[0], dst[0]), (src[2], dst[2]), (src[4], dst[4])):
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
    assert md["format"] == ql.FORMAT and md["version"] == str(ql.FORMAT_VERSION)
    other = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(2)}, other, metadata={"format": "something-else"})
    with pytest.raises(ValueError):
        ql.load_quantized(nn.Sequential(nn.Linear(128, 16)), other)
    with pytest.raises(ValueError):  # layer shape mismatch
        ql.load_quantized(nn.Sequential(nn.Linear(256, 16)), path)
    old = str(tmp_path / "old.safetensors")
    save_file({"0.qweight": torch.zeros(128, 2, dtype=torch.int32)}, old,
              metadata={**md, "version": "1"})
    with pytest.raises(ValueError):
        ql.load_quantized(nn.Sequential(nn.Linear(128, 16)), old)


@pytest.mark.parametrize("key,bad", [
    ("0.scales", lambda t: t[None, 0, :].contiguous()),      # (1, out): would broadcast
    ("0.scales", lambda t: t.float()),                      # wrong dtype
    ("0.qweight", lambda t: t[:, :1].contiguous()),         # wrong shape
    ("0.bias", lambda t: t[:8].contiguous()),
    ("0.bias", None),                                       # missing
])
def test_tensor_checks_before_copy(tmp_path, key, bad):
    from safetensors import safe_open
    from safetensors.torch import load_file, save_file

    path = str(tmp_path / "m.safetensors")
    ql.save_quantized(nn.Sequential(_random_qlinear(256, 16, True, 5)), path)
    with safe_open(path, framework="pt") as f:
        md = dict(f.metadata())
    t = load_file(path)
    if bad is None:
        del t[key]
    else:
        t[key] = bad(t[key])
    p2 = str(tmp_path / "bad.safetensors")
    save_file(t, p2, metadata=md)
    dst = nn.Sequential(nn.Linear(256, 16))
    with pytest.raises(ValueError):
        ql.load_quantized(dst, p2)
    assert isinstance(dst[0], nn.Linear)  # nothing replaced


def test_shape_contract():
    with pytest.raises(ValueError):
        ql.QuantLinear(256 + 32, 64)  # in_features not a multiple of the group
    with pytest.raises(ValueError):
        ql.QuantLinear(128, 60)  # out_features not whole int32 words
    with pytest.raises(ValueError):
        ql.QuantLinear(100, 64, scheme="per_input")  # in_features not a multiple of 32
    with pytest.raises(ValueError):
        ql.QuantLinear(128, 64, scheme="per_row")


def test_column_tiles_in_memory_pack_order_outside(tmp_path):
    """Layers whose shape allows it keep qweight in 128 x 256 blocks (word j of input row k at
    ((k // 128) * T + j // 32) * 4096 + (k % 128) * 32 + j % 32, T = out / 256); codes(), the
    state dict and the file hold pack_int4_n order, and a round trip through either restores
    the same memory."""
    import _pk

    q = ql.QuantLinear(512, 768, True, 128)
    assert q.tiled and not ql.QuantLinear(512, 776, True, 128).tiled
    assert not ql.QuantLinear(512, 768, True, 32).tiled
    assert ql.QuantLinear(512, 768, True, scheme="per_input").tiled
    g = _gen(21)
    words = torch.randint(-2**31, 2**31 - 1, (512, 96), generator=g, dtype=torch.int64).to(torch.int32)
    q.set_codes(words)
    flat = q.qweight.reshape(-1)
    for k, j in ((0, 0), (5, 33), (511, 95), (100, 64), (257, 31), (128, 0), (127, 32)):
        assert int(flat[((k // 128) * 3 + j // 32) * 4096 + (k % 128) * 32 + j % 32]) == int(words[k, j])
    assert torch.equal(q.codes(), words)
    assert torch.equal(_pk.untile_weights(_pk.tile_weights(words)), words)
    sd = q.state_dict()
    assert torch.equal(sd["qweight"], words)
    q2 = ql.QuantLinear(512, 768, True, 128)
    q2.load_state_dict(sd)
    assert torch.equal(q2.qweight, q.qweight)
    q.scales.copy_((torch.rand(q.scales.shape, generator=g) * 0.01).half())
    path = str(tmp_path / "t.safetensors")
    ql.save_quantized(nn.Sequential(q), path)
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        assert torch.equal(f.get_tensor("0.qweight"), words)
    dst = nn.Sequential(nn.Linear(512, 768))
    ql.load_quantized(dst, path)
    assert dst[0].tiled and torch.equal(dst[0].qweight, q.qweight)
    assert torch.equal(dst[0].scales, q.scales)
