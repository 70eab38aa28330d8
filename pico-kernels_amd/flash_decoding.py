"""KV cache and split-KV decode attention on MI355X -- drop-in for the reference's
``flash_decoding`` module.

Reference entry points kept with their signatures (flash_decoding.py):
  * ``KVCache(batch, heads, head_dim, max_len, device, dtype=torch.float16)`` with
    ``append(k, v) -> (k_prefix, v_prefix)`` and ``reset()``           (:30-45)
  * ``flash_decoding(q, k, v, split_size=256) -> (B, H, 1, D)`` fp32   (:88-123)
  * ``eager_decode(q, k, v) -> (B, H, 1, D)`` in ``q``'s dtype        (:126-133)

``flash_decoding`` asserts ``N % split_size == 0`` as the reference does and runs the HIP
split-KV kernel behind ``pk_flash_decode`` (per-split max / sum / weighted sum in fp32, then
one ordered combine), reading a ``KVCache`` prefix view in place. ``eager_decode`` is the
reference's naive helper (the full softmax through torch matmuls), kept for callers that
compare against it.
"""

from __future__ import annotations

import math

import torch

import _pk

__all__ = ["KVCache", "flash_decoding", "eager_decode"]


class KVCache:
    """Append-only K/V cache ``(B, H, max_len, D)``; ``append`` returns the filled prefix."""

    def __init__(self, batch: int, heads: int, head_dim: int, max_len: int,
                 device, dtype=torch.float16):
        self.k = torch.empty(batch, heads, max_len, head_dim, device=device, dtype=dtype)
        self.v = torch.empty(batch, heads, max_len, head_dim, device=device, dtype=dtype)
        self.pos = 0

    def append(self, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Write one step's ``k, v`` (each ``(B, H, 1, D)``) at the next position."""
        assert self.pos < self.k.shape[2], "KVCache is full"
        self.k[:, :, self.pos:self.pos + 1] = k
        self.v[:, :, self.pos:self.pos + 1] = v
        self.pos += 1
        return self.k[:, :, :self.pos], self.v[:, :, :self.pos]

    def reset(self) -> None:
        self.pos = 0


def flash_decoding(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   split_size: int = 256) -> torch.Tensor:
    B, H, _, D = q.shape
    N = k.shape[2]
    assert N % split_size == 0, "N must divide split_size"
    assert q.is_cuda and k.is_cuda and v.is_cuda, "flash_decoding: inputs must be on the GPU"
    assert q.dtype == k.dtype == v.dtype == torch.float16, "flash_decoding: fp16 q, k, v expected"
    o = _pk.flash_decode(q[:, :, 0, :], k, v, split_size, 1.0 / math.sqrt(D))
    return o[:, :, None, :]


def eager_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Single-query attention materialising the full N-vector (fp32 math, ``q.dtype`` out)."""
    D = q.shape[-1]
    qf, kf, vf = q.float(), k.float(), v.float()
    s = (qf @ kf.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(D))
    return (torch.softmax(s, dim=-1) @ vf).to(q.dtype)
