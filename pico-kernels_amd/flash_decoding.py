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

__all__ = ["KVCache", "flash_decoding", "eager_decode", "check_correctness", "bench"]


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


def _harness_checks() -> list:
    """Self-check at the reference's check shape (flash_decoding.py:128-138: B2 H4 N2048 D64,
    split 256): split-KV decode against ``eager_decode``, max absolute error and
    torch.allclose at atol = rtol = 1e-2."""
    from _timing import Check

    def measure():
        g = torch.Generator(device="cuda").manual_seed(0)
        q, k, v = (torch.randn(2, 4, n, 64, device="cuda", dtype=torch.float16, generator=g)
                   for n in (1, 2048, 2048))
        o = flash_decoding(q, k, v, split_size=256).float()
        ref = eager_decode(q, k, v).float()
        return {"max_abs_err": (o - ref).abs().max().item(),
                "allclose_1e-2": bool(torch.allclose(o, ref, atol=1e-2, rtol=1e-2))}

    return [Check("split256_B2H4N2048D64", measure, {"allclose_1e-2": (True, True)})]


def _harness_rows() -> list:
    """The reference's benchmark cases (flash_decoding.py:141-152: B2 H4 D64, split 256,
    N = 1K..8K): ``eager_decode`` against ``flash_decoding``, in milliseconds."""
    from _timing import Row

    def build(n):
        def make():
            q, k, v = (torch.randn(2, 4, m, 64, device="cuda", dtype=torch.float16)
                       for m in (1, n, n))
            return {"eager": lambda: eager_decode(q, k, v),
                    "flash_decoding": lambda: flash_decoding(q, k, v, split_size=256)}
        return make

    return [Row(f"B=2,H=4,N={n},D=64", build(n)) for n in (1024, 2048, 4096, 8192)]


def check_correctness() -> bool:
    """Run and print the module's self-check (see ``_harness_checks``)."""
    from _timing import run_checks

    return run_checks("flash_decoding", _harness_checks())


def bench() -> None:
    """Time and print the module's benchmark rows (see ``_harness_rows``)."""
    from _timing import run_rows

    run_rows("flash_decoding", _harness_rows())


if __name__ == "__main__":
    import sys

    from _timing import main

    sys.exit(main("flash_decoding", _harness_checks(), _harness_rows()))
