"""Packed int4 linear layers on MI355X: the consumer of the W4A16 kernel.

The reference quantizes a model by writing fake-quantized floats back into every
``nn.Linear`` (quantize.quantize_model, quantize.py:160-181, ``mod.weight.data = wq`` at
:179): the weights stay 16/32-bit in memory and every matmul reads them at full width. This
module keeps them packed instead, in one of two layouts (``QuantLinear.scheme``):

* ``"per_input"`` -- exactly what the reference's ``quantize_model`` produces: ``rtn_layer``
  or ``gptq_layer`` with ``group_size=None`` (quantize.py:63-115) quantize every input column
  of ``W [out, in]`` with one scale over all output rows (quantize.py:52-54), so
  ``wq[:, j] = q[:, j] * s_j``. ``QuantLinear.from_quantized_weight(wq)`` recovers ``s_j``
  and the codes ``q`` from such a weight and stores the codes as ``(in, out/8)`` int32 words
  (``pack_int4_n`` byte order) plus ``s`` as an ``(in,)`` fp32 vector. ``forward`` folds
  ``s`` into the activations (``pk_w4a16_prep_activations``: ``fp16(x * s / max s)``, the
  input cast in the same pass) and runs the W4A16 kernel in its per-tensor mode with
  ``max s`` as the epilogue scale: ``x @ wq^T`` as ``(x * s) @ q^T``.
* ``"group"`` -- groups of ``group_size`` input features per output column (the layout of
  ``quantize.rtn_layer(W^T, 4, group_size)``: ``s = max|w|.clamp_min(1e-12) / 7`` per group,
  codes in [-7, 7]) with ``(in/group, out)`` fp16 scales, the kernel's group mode.

``QuantLinear.from_linear(linear, method=...)``: ``method=None`` quantizes to the group
layout; ``"rtn"`` / ``"gptq"`` (with calibration inputs ``x``) run this build's ``rtn_layer`` /
``gptq_layer`` (group_size None) -- the reference's own per-layer call -- and pack the result.
``quantize_model_int4(model, method=...)`` replaces a model's ``nn.Linear`` layers in place.
``save_quantized`` / ``load_quantized`` write and read every ``QuantLinear`` as one safetensors
file (no pickle) whose metadata records the format, its version and each layer's layout and
shape; ``load_quantized`` checks each tensor's shape and dtype before copying and raises
``ValueError`` on any mismatch.

In memory, layers whose shape allows it (``in`` and ``out`` multiples of 256, groups of a
multiple of 64 inputs or per-input scales: ``QuantLinear.tiled``) keep ``qweight`` in blocks
of 128 inputs x 256 outputs, each 16 KB block contiguous (``_pk.tile_weights``), which the
kernels stream in long runs (``pk_w4a16_gemm_tiled``). For decode, layers whose shape allows
it (``out % 16 == 0``, ``in % 128 == 0``, groups of a multiple of 32 that divide 128 or are
multiples of it, or per-input scales: ``QuantLinear.decode``) keep a second copy of the codes
and group scales in the strip layout (``_pk.strip_weights`` / ``strip_scales``: each
16-output strip's inputs contiguous), and calls of at most ``decode_rows`` rows run the
one-launch strip GEMV on it (``pk_w4a16_gemm_strips``; ``decode_rows``: 8 rows, or 4 on layers
of more than 16384 outputs). The int4 codes are a quarter of the
fp16 weights' bytes, so both copies together are half of them; ``decode_layout=False`` keeps
one copy. The copies are derived buffers, outside the state dict. ``codes()`` /
``set_codes()``, the state dict and the file format use ``pack_int4_n`` order either way.

The output has the input's dtype (fp16, bf16 or fp32, as ``nn.Linear``); other inputs are
computed in fp16. A finite bf16 / fp32 activation whose fp16 form would be infinite (beyond
65504, after the per-input scales for that scheme) raises ``ValueError``: one device reduction
and synchronisation per call on such inputs, skipped under graph capture and when
``QuantLinear.range_check`` is False (then such values become infinities, as torch's own fp16
cast makes them). Weights need ``out % 8 == 0`` (whole int32 words) and ``in % 32 == 0``
(the kernel's K), group layers ``in % group_size == 0``.
"""

from __future__ import annotations

import json

import torch
from torch import nn

import _pk
import gemm_int4

__all__ = ["QuantLinear", "quantize_model_int4", "save_quantized", "load_quantized", "FORMAT"]

FORMAT = "pico-kernels-amd/w4a16"
FORMAT_VERSION = 2
SCHEMES = ("group", "per_input")
_OUT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
# Rows up to which forward runs the strip-layout GEMV (when the layer keeps that copy): 8, or 4
# on layers of more than 1024 strips of 16 output columns. Measured on MI355X (graphs over
# rotating weight copies, against the block layout's kernels): M = 1..4 faster on every
# Llama-3-8B layer (4096 x 11008 M = 4: 8.5 against 10.4 us); M = 5..8 faster on qkv (M = 8:
# 7.4 against 9.0), o_proj (5.6 against 7.7), down (11.7 against 13.7), gate_up (4096 x 14336:
# 11.9 against 12.8), 4096 x 11008 (11.0 against 12.2) and 5120 x 13824 (14.2 against 16.2);
# slower on 4096 x 28672 (1792 strips: 22.1 against 21.7).
DECODE_MAX_ROWS = 8
DECODE_MAX_ROWS_WIDE = 4
DECODE_WIDE_STRIPS = 1024


def decode_rows(in_features: int, out_features: int) -> int:
    """Rows up to which a layer of this shape runs its strip copy."""
    wide = out_features // 16 > DECODE_WIDE_STRIPS
    return DECODE_MAX_ROWS_WIDE if wide else DECODE_MAX_ROWS


class QuantLinear(nn.Module):
    """``y = x @ W^T + b`` with ``W`` stored as int4 codes and scales (see the module doc)."""

    # bf16 / fp32 inputs: raise ValueError when the fp16 cast would overflow (see the module doc)
    range_check: bool = True

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 group_size: int = 128, device: torch.device | str | None = None,
                 scheme: str = "group", decode_layout: bool = True):
        super().__init__()
        if scheme not in SCHEMES:
            raise ValueError(f"scheme must be one of {SCHEMES}, not {scheme!r}")
        if out_features % 8:
            raise ValueError("out_features must be a multiple of 8")
        if in_features % 32:
            raise ValueError("in_features must be a multiple of 32")
        if scheme == "group" and in_features % group_size:
            raise ValueError("in_features must be a multiple of group_size")
        self.in_features, self.out_features, self.scheme = in_features, out_features, scheme
        self.group_size = group_size if scheme == "group" else 0
        # qweight in 128 x 256 blocks (see the module doc) where the shape allows
        self.tiled = _pk.tiles_ok(in_features, out_features, self.group_size)
        self.register_buffer("qweight", torch.zeros(in_features, out_features // 8,
                                                    dtype=torch.int32, device=device))
        if scheme == "group":
            self.register_buffer("scales", torch.zeros(in_features // group_size, out_features,
                                                       dtype=torch.float16, device=device))
        else:
            self.register_buffer("scales", torch.zeros(in_features, dtype=torch.float32,
                                                       device=device))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.float16,
                                                     device=device))
        else:
            self.bias = None
        self._smax = 1.0  # per_input: max of the scales (the epilogue scale)
        # the decode copy: codes (and group scales) in the strip layout, derived from the above
        self.decode = bool(decode_layout) and _pk.strips_ok(in_features, out_features,
                                                            self.group_size)
        self.register_buffer("qstrips", torch.zeros_like(self.qweight) if self.decode else None,
                             persistent=False)
        self.register_buffer("sstrips", torch.zeros_like(self.scales)
                             if self.decode and scheme == "group" else None, persistent=False)
        self._calls: dict = {}  # prepared strip-GEMV calls by output dtype (see _strips_call)
        self._fast = None       # the fp16 one, for forward's decode fast path
        self.decode_rows = decode_rows(in_features, out_features)

    # ---- construction -------------------------------------------------------------------
    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = 128, method: str | None = None,
                    x: torch.Tensor | None = None) -> "QuantLinear":
        """Quantize ``linear``: ``method=None`` to the group layout; ``"rtn"`` or ``"gptq"``
        (calibration inputs ``x``, ``[n, in]``) as the reference's ``quantize_model`` does
        (quantize.py:175-178), packed in the per-input layout."""
        if method is None:
            return cls._from_linear_group(linear, group_size)
        import quantize

        w = linear.weight.detach()
        if method == "rtn":
            wq = quantize.rtn_layer(w, 4)
        elif method == "gptq":
            if x is None:
                raise ValueError("method='gptq' needs calibration inputs x")
            wq = quantize.gptq_layer(w, x, 4)
        else:
            raise ValueError(f"method must be None, 'rtn' or 'gptq', not {method!r}")
        return cls.from_quantized_weight(wq, None if linear.bias is None else linear.bias.detach())

    @classmethod
    def _from_linear_group(cls, linear: nn.Linear, group_size: int) -> "QuantLinear":
        w = linear.weight.detach()
        # quantized on the GPU; the layer lives where the source layer lives
        q = cls(linear.in_features, linear.out_features, linear.bias is not None, group_size,
                w.device)
        w_kn = w.to(_pk.gpu_device()).t().contiguous()  # (in, out): groups along the inputs
        qweight, scales = gemm_int4.quantize_int4_group(w_kn, group_size)
        q.set_codes(qweight)
        q.scales.copy_(scales)
        if linear.bias is not None:
            q.bias.copy_(linear.bias.detach().to(torch.float16))
        q._refresh()
        return q

    @classmethod
    def from_quantized_weight(cls, wq: torch.Tensor, bias: torch.Tensor | None = None,
                              bits: int = 4) -> "QuantLinear":
        """Pack a weight ``[out, in]`` that ``rtn_layer`` / ``gptq_layer`` with
        ``group_size=None`` wrote (every input column an integer multiple of its own scale,
        codes within ``±(2^(bits-1) - 1)``): ``s_j = max|wq[:, j]| / qmax``,
        ``q = round(wq / s)``. Raises ``ValueError`` if ``wq`` is not of that form."""
        if bits != 4:
            raise ValueError("only 4-bit codes pack into the W4A16 layout")
        out_f, in_f = wq.shape
        dev = wq.device
        w = wq.detach().to(_pk.gpu_device()).float()
        qmax = 2 ** (bits - 1) - 1
        s = w.abs().amax(dim=0) / qmax                  # (in,)
        safe = torch.where(s > 0, s, torch.ones_like(s))
        q = torch.round(w / safe)
        # each element a whole multiple of its column's scale: up to the rounding of the
        # written-back weight (fp32, or fp16 / bf16 for a half-precision model)
        if bool((q.abs() > qmax).any()) or not bool(
                ((w - q * safe).abs() <= 5e-2 * safe + 1e-30).all()):
            raise ValueError("weight is not a per-input-column int4 quantization "
                             "(rtn_layer / gptq_layer with group_size=None)")
        s = torch.where(s > 0, s, torch.full_like(s, 1e-12 / qmax))
        layer = cls(in_f, out_f, bias is not None, 0, dev, scheme="per_input")
        codes = q.t().contiguous().to(torch.int8)       # (in, out)
        layer.set_codes(gemm_int4.pack_int4_n(codes).view(torch.int32))
        layer.scales.copy_(s)
        if bias is not None:
            layer.bias.copy_(bias.to(torch.float16))
        layer._refresh()
        return layer

    # ---- codes ------------------------------------------------------------------------
    def codes(self) -> torch.Tensor:
        """The packed codes as ``(in, out/8)`` int32 words in ``pack_int4_n`` order."""
        return _pk.untile_weights(self.qweight) if self.tiled else self.qweight

    def set_codes(self, words: torch.Tensor) -> None:
        """Store ``(in, out/8)`` int32 words given in ``pack_int4_n`` order."""
        words = words.to(self.qweight.device)
        self.qweight.copy_(_pk.tile_weights(words) if self.tiled else words)
        if self.decode:
            self.qstrips.copy_(_pk.strip_weights(words))  # in place: prepared calls stay valid

    # ---- use ----------------------------------------------------------------------------
    def dequantized_weight(self) -> torch.Tensor:
        """``(out, in)`` fp32 ``q * scale`` (for inspection and tests)."""
        if self.scheme == "group":
            return gemm_int4.dequantize_int4_group(self.codes(), self.scales, self.group_size).t()
        q = gemm_int4.unpack_int4_n(self.codes().contiguous().view(torch.uint8)).float()
        return (q * self.scales.to(q.device)[:, None]).t()

    def _strips_call(self, out_dtype: torch.dtype) -> "_pk.PreparedStrips":
        """The prepared strip-GEMV call for this output dtype (made on first use; dropped by
        _refresh, by moves such as .to() and in copies, which rebuild it from their own
        buffers)."""
        call = self._calls.get(out_dtype)
        if call is None or call._keep[0] is not self.qstrips or call._keep[2] is not self.bias:
            scale = self._smax if self.scheme == "per_input" else 1.0
            call = _pk.PreparedStrips(self.qstrips, self.sstrips, self.group_size, scale, out_dtype,
                                      self.bias)
            self._calls[out_dtype] = call
            if out_dtype == torch.float16 and self.scheme == "group":
                self._fast = call
        return call

    def _drop_calls(self) -> None:
        self._calls = {}
        self._fast = None

    _PREPARED_FROM = frozenset(("qstrips", "sstrips", "bias", "scales", "qweight"))

    def __setattr__(self, name, value):
        # a prepared call holds the addresses of these buffers: reassigning one drops it
        if name in QuantLinear._PREPARED_FROM and "_calls" in self.__dict__:
            self._drop_calls()
        super().__setattr__(name, value)

    def _apply(self, fn, *args, **kwargs):
        self._drop_calls()  # buffers may move: prepared calls hold their addresses
        return super()._apply(fn, *args, **kwargs)

    def __getstate__(self):
        # prepared calls are derived (and hold a C handle): copies and pickles rebuild them
        state = super().__getstate__() if hasattr(super(), "__getstate__") else self.__dict__.copy()
        state = dict(state)
        state["_calls"], state["_fast"] = {}, None
        return state

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # decode fast path: fp16 rows of a group layer with a strip copy, one prepared call
        fast = self._fast
        if (fast is not None and x.dim() == 2 and x.dtype == torch.float16
                and x.shape[0] <= self.decode_rows and x.shape[1] == self.in_features):
            return fast(x)
        assert x.shape[-1] == self.in_features
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if (x2.dtype == torch.float16 and self.scheme == "group" and self.decode
                and x2.shape[0] <= self.decode_rows):
            return self._strips_call(torch.float16)(x2).view(*lead, self.out_features)
        out_dtype = x.dtype if x.dtype in _OUT_DTYPES else torch.float16
        strips = self.decode and x2.shape[0] <= self.decode_rows
        # the bias is added in the matmul's epilogue (before the one rounding to out_dtype)
        if self.scheme == "per_input":
            # x * s / max s in fp16 (the input cast in the same pass), then max s in the epilogue
            s = self.scales if self.scales.dtype == torch.float32 else self.scales.float()
            xp = _pk.w4a16_prep_activations(x2, s, 1.0 / self._smax)
            if self.range_check:
                _pk.check_fp16_range(x2, "QuantLinear", xp)
            if strips:
                y = self._strips_call(out_dtype)(xp)
            else:
                y = _pk.w4a16_gemm(xp, self.qweight, None, 0, self._smax, out_dtype,
                                   bias=self.bias, tiled=self.tiled)
        else:
            xp = x2 if x2.dtype == torch.float16 else _pk.w4a16_prep_activations(x2, None, 1.0)
            if self.range_check and xp is not x2:
                _pk.check_fp16_range(x2, "QuantLinear", xp)
            if strips:
                y = self._strips_call(out_dtype)(xp)
            else:
                s = self.scales if self.scales.dtype == torch.float16 else self.scales.half()
                y = _pk.w4a16_gemm(xp, self.qweight, s, self.group_size, 1.0, out_dtype,
                                   bias=self.bias, tiled=self.tiled)
        return y.reshape(*lead, self.out_features)

    def _refresh(self) -> None:
        """Rebuild what derives from the buffers: the per-input epilogue scale and the decode
        copy in the strip layout (call after changing ``qweight`` or ``scales`` directly)."""
        self._drop_calls()
        if self.scheme == "per_input":
            self._smax = float(self.scales.float().max().item())
        if self.decode:
            self.qstrips = _pk.strip_weights(self.codes()).to(self.qweight.device)
            if self.scheme == "group":
                self.sstrips = _pk.strip_scales(self.scales.half()).to(self.scales.device)

    # the state dict holds the codes in pack_int4_n order, whatever the layout in memory
    def _save_to_state_dict(self, destination, prefix, keep_vars):
        super()._save_to_state_dict(destination, prefix, keep_vars)
        if self.tiled:
            destination[prefix + "qweight"] = self.codes()

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)
        if self.tiled and prefix + "qweight" in state_dict:
            # A new tensor, never an in-place rewrite: under load_state_dict(assign=True) the
            # buffer is the caller's own state-dict tensor, which must keep pack_int4_n order.
            self.qweight = _pk.tile_weights(self.qweight)
        self._refresh()

    def extra_repr(self) -> str:
        lay = f"group_size={self.group_size}" if self.scheme == "group" else "per-input scales"
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, {lay}, int4"
                + (", 128x256 blocks" if self.tiled else "")
                + (", strip copy for decode" if self.decode else ""))


def quantize_model_int4(model: nn.Module, group_size: int = 128, predicate=None,
                        method: str | None = None, x=None) -> nn.Module:
    """Replace every ``nn.Linear`` of ``model`` (those ``predicate(name, module)`` accepts, if
    given) by a ``QuantLinear``; layers whose shapes the packed format cannot hold are left
    as they are. ``method=None``: the group layout; ``"rtn"`` / ``"gptq"``: the reference's
    ``quantize_model`` per layer (quantize.py:175-179), with ``x`` the calibration inputs of
    each layer for GPTQ -- a mapping from layer name to ``[n, in]`` activations, or a callable
    ``x(name, module)`` returning them (the reference captures them by running the model,
    quantize.py:132-157). Returns ``model``."""
    targets = []
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and (predicate is None or predicate(name, mod)):
            ok = mod.out_features % 8 == 0 and mod.in_features % 32 == 0
            if method is None:
                ok = ok and mod.in_features % group_size == 0
            if ok:
                targets.append(name)
    for name in targets:
        parent_name, _, child = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        lin = getattr(parent, child)
        xs = None
        if method == "gptq":
            xs = x(name, lin) if callable(x) else (x or {}).get(name)
            if xs is None:
                raise ValueError(f"no calibration inputs for {name}")
        setattr(parent, child, QuantLinear.from_linear(lin, group_size, method, xs))
    return model


def _quant_layers(model: nn.Module) -> dict[str, QuantLinear]:
    return {n: m for n, m in model.named_modules() if isinstance(m, QuantLinear)}


def save_quantized(model: nn.Module, path: str) -> None:
    """Write every ``QuantLinear`` of ``model`` to one safetensors file."""
    from safetensors.torch import save_file

    layers = _quant_layers(model)
    tensors, meta = {}, {}
    for name, q in layers.items():
        tensors[f"{name}.qweight"] = q.codes().detach().cpu().contiguous()
        tensors[f"{name}.scales"] = q.scales.detach().cpu().contiguous()
        if q.bias is not None:
            tensors[f"{name}.bias"] = q.bias.detach().cpu().contiguous()
        meta[name] = {"in_features": q.in_features, "out_features": q.out_features,
                      "group_size": q.group_size, "bias": q.bias is not None,
                      "scheme": q.scheme}
    save_file(tensors, path, metadata={"format": FORMAT, "version": str(FORMAT_VERSION),
                                       "layers": json.dumps(meta, sort_keys=True)})


_ST_DTYPES = {torch.int32: "I32", torch.float16: "F16", torch.float32: "F32"}


def _read(f, key: str, like: torch.Tensor, path: str) -> torch.Tensor:
    """The file's tensor `key`, after checking its shape and dtype against `like`."""
    try:
        sl = f.get_slice(key)
    except Exception as e:  # missing tensor
        raise ValueError(f"{path}: missing tensor {key}") from e
    shape, dtype = tuple(sl.get_shape()), sl.get_dtype()
    if shape != tuple(like.shape) or dtype != _ST_DTYPES[like.dtype]:
        raise ValueError(f"{path}: {key} is {dtype}{list(shape)}, expected "
                         f"{_ST_DTYPES[like.dtype]}{list(like.shape)}")
    return f.get_tensor(key)


def load_quantized(model: nn.Module, path: str) -> nn.Module:
    """Load a file written by ``save_quantized`` into ``model``: every layer named in the file
    becomes a ``QuantLinear`` (replacing an ``nn.Linear`` of the same shape, or filling an
    existing ``QuantLinear``). Raises ``ValueError`` when the file's format, version, a layer's
    shape or any tensor's shape or dtype does not match. Returns ``model``."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        md = f.metadata() or {}
        if md.get("format") != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} file (format {md.get('format')!r})")
        if md.get("version") != str(FORMAT_VERSION):
            raise ValueError(f"{path}: format version {md.get('version')!r}, expected {FORMAT_VERSION}")
        try:
            layers = json.loads(md["layers"])
        except (KeyError, ValueError) as e:
            raise ValueError(f"{path}: no layer table") from e
        for name, info in layers.items():
            parent_name, _, child = name.rpartition(".")
            parent = model.get_submodule(parent_name) if parent_name else model
            cur = getattr(parent, child)
            if not isinstance(cur, (nn.Linear, QuantLinear)):
                raise ValueError(f"{name} is not a linear layer")
            if (cur.in_features, cur.out_features) != (info["in_features"], info["out_features"]):
                raise ValueError(f"{name}: the model's layer is {cur.in_features}x{cur.out_features}, "
                                 f"the file's {info['in_features']}x{info['out_features']}")
            dev = cur.qweight.device if isinstance(cur, QuantLinear) else cur.weight.device
            q = QuantLinear(info["in_features"], info["out_features"], info["bias"],
                            info["group_size"] or 128, dev, scheme=info.get("scheme", "group"))
            q.set_codes(_read(f, f"{name}.qweight", q.qweight, path))
            q.scales.copy_(_read(f, f"{name}.scales", q.scales, path))
            if info["bias"]:
                q.bias.copy_(_read(f, f"{name}.bias", q.bias, path))
            q._refresh()
            setattr(parent, child, q)
    return model
