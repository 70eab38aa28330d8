"""Packed int4 linear layers on MI355X: the consumer of the W4A16 kernel.

The reference quantizes a model by writing fake-quantized floats back into every
``nn.Linear`` (quantize.quantize_model, quantize.py:160-181, ``mod.weight.data = wq`` at
:179): the weights stay 16-bit in memory and every matmul reads them at full width. This
module keeps them packed instead:

* ``QuantLinear.from_linear(linear, group_size=128)`` quantizes ``W^T`` ``(in, out)`` with the
  arithmetic of ``quantize.rtn_layer(W^T, 4, group_size)`` (groups of ``group_size`` input
  features per output column, ``s = max|w|.clamp_min(1e-12) / 7``, codes in [-7, 7]) and
  stores the ``(in, out/8)`` int32 words (``pack_int4_n`` byte order) and ``(in/group, out)``
  fp16 scales; ``forward`` is one ``w4a16_gemm`` call over the flattened leading dimensions.
* ``quantize_model_int4(model)`` replaces the model's ``nn.Linear`` layers in place.
* ``save_quantized(model, path)`` / ``load_quantized(model, path)`` write and read every
  ``QuantLinear``'s tensors as one safetensors file (no pickle) whose metadata records the
  format, its version and each layer's group size and shape. Loaded layers take the device
  of the module they replace; ``forward`` needs them on the GPU.

Weights need ``in % group_size == 0`` and ``out % 8 == 0`` (whole int32 words).
"""

from __future__ import annotations

import json

import torch
from torch import nn

import _pk
import gemm_int4

__all__ = ["QuantLinear", "quantize_model_int4", "save_quantized", "load_quantized", "FORMAT"]

FORMAT = "pico-kernels-amd/w4a16-group"
FORMAT_VERSION = 1


class QuantLinear(nn.Module):
    """``y = x @ W^T + b`` with ``W`` stored as group-quantized int4 (see the module doc)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 group_size: int = 128, device: torch.device | str | None = None):
        super().__init__()
        assert in_features % group_size == 0, "in_features must be a multiple of group_size"
        assert out_features % 8 == 0, "out_features must be a multiple of 8"
        self.in_features, self.out_features, self.group_size = in_features, out_features, group_size
        self.register_buffer("qweight", torch.zeros(in_features, out_features // 8,
                                                    dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.zeros(in_features // group_size, out_features,
                                                   dtype=torch.float16, device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                     device=device))
        else:
            self.bias = None

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 128) -> "QuantLinear":
        w = linear.weight.detach()
        # quantized on the GPU; the layer lives where the source layer lives
        q = cls(linear.in_features, linear.out_features, linear.bias is not None, group_size,
                w.device)
        w_kn = w.to(_pk.gpu_device()).t().contiguous()  # (in, out): groups along the inputs
        qweight, scales = gemm_int4.quantize_int4_group(w_kn, group_size)
        q.qweight.copy_(qweight)
        q.scales.copy_(scales)
        if linear.bias is not None:
            q.bias.copy_(linear.bias.detach().to(torch.float16))
        return q

    def dequantized_weight(self) -> torch.Tensor:
        """``(out, in)`` fp32 ``q * scale`` (for inspection and tests)."""
        return gemm_int4.dequantize_int4_group(self.qweight, self.scales, self.group_size).t()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        assert x.shape[-1] == self.in_features
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype != torch.float16:
            x2 = x2.half()
        y = _pk.w4a16_gemm(x2, self.qweight, self.scales, self.group_size, 1.0, torch.float16)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*lead, self.out_features)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, group_size={self.group_size}, int4")


def quantize_model_int4(model: nn.Module, group_size: int = 128,
                        predicate=None) -> nn.Module:
    """Replace every ``nn.Linear`` of ``model`` (those ``predicate(name, module)`` accepts, if
    given) by a ``QuantLinear``; layers whose shapes the packed format cannot hold are left
    as they are. Returns ``model``."""
    targets = []
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and (predicate is None or predicate(name, mod)):
            if mod.in_features % group_size == 0 and mod.out_features % 8 == 0:
                targets.append(name)
    for name in targets:
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        setattr(parent, child, QuantLinear.from_linear(getattr(parent, child), group_size))
    return model


def _quant_layers(model: nn.Module) -> dict[str, QuantLinear]:
    return {n: m for n, m in model.named_modules() if isinstance(m, QuantLinear)}


def save_quantized(model: nn.Module, path: str) -> None:
    """Write every ``QuantLinear`` of ``model`` to one safetensors file."""
    from safetensors.torch import save_file

    layers = _quant_layers(model)
    tensors, meta = {}, {}
    for name, q in layers.items():
        tensors[f"{name}.qweight"] = q.qweight.detach().cpu().contiguous()
        tensors[f"{name}.scales"] = q.scales.detach().cpu().contiguous()
        if q.bias is not None:
            tensors[f"{name}.bias"] = q.bias.detach().cpu().contiguous()
        meta[name] = {"in_features": q.in_features, "out_features": q.out_features,
                      "group_size": q.group_size, "bias": q.bias is not None}
    save_file(tensors, path, metadata={"format": FORMAT, "version": str(FORMAT_VERSION),
                                       "layers": json.dumps(meta, sort_keys=True)})


def load_quantized(model: nn.Module, path: str) -> nn.Module:
    """Load a file written by ``save_quantized`` into ``model``: every layer named in the file
    becomes a ``QuantLinear`` (replacing an ``nn.Linear`` of the same shape, or filling an
    existing ``QuantLinear``). Returns ``model``."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        md = f.metadata() or {}
        assert md.get("format") == FORMAT, f"{path}: not a {FORMAT} file"
        assert int(md.get("version", "0")) == FORMAT_VERSION, f"{path}: unsupported version"
        layers = json.loads(md["layers"])
        for name, info in layers.items():
            parent_name, _, child = name.rpartition(".")
            parent = model.get_submodule(parent_name) if parent_name else model
            cur = getattr(parent, child)
            assert isinstance(cur, (nn.Linear, QuantLinear)), f"{name} is not a linear layer"
            assert (cur.in_features, cur.out_features) == (info["in_features"], info["out_features"]), \
                f"{name}: shape differs from the file"
            dev = cur.qweight.device if isinstance(cur, QuantLinear) else cur.weight.device
            q = QuantLinear(info["in_features"], info["out_features"], info["bias"],
                            info["group_size"], dev)
            q.qweight.copy_(f.get_tensor(f"{name}.qweight"))
            q.scales.copy_(f.get_tensor(f"{name}.scales"))
            if info["bias"]:
                q.bias.copy_(f.get_tensor(f"{name}.bias"))
            setattr(parent, child, q)
    return model
