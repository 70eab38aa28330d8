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


def check_correctness(N: int = 2048, D: int = 64, split_size: int = 256) -> None:
    """The reference's self-check (flash_decoding.py:128-138): split-KV decode against
    eager_decode, max abs error and allclose at 1e-2."""
    torch.manual_seed(0)
    B, H = 2, 4
    q = torch.randn(B, H, 1, D, device="cuda", dtype=torch.float16)
    k = torch.randn(B, H, N, D, device="cuda", dtype=torch.float16)
    v = torch.randn(B, H, N, D, device="cuda", dtype=torch.float16)
    o = flash_decoding(q, k, v, split_size=split_size)
    ref = eager_decode(q, k, v)
    err = (o.float() - ref.float()).abs().max().item()
    print(f"flash-decoding vs eager (N={N}): max abs err {err:.3e} | "
          f"allclose {torch.allclose(o.float(), ref.float(), atol=1e-2, rtol=1e-2)}")


def bench() -> None:
    """The reference's benchmark table (flash_decoding.py:141-152): eager decode against
    split-KV decode at B=2, H=4, D=64, split 256, N = 1K..8K (milliseconds)."""
    from _timing import do_bench

    B, H, D = 2, 4, 64
    print(f"{'N':>7} {'eager decode':>13} {'flash-decoding':>15} {'speedup':>8}")
    print("-" * 46)
    for N in (1024, 2048, 4096, 8192):
        q = torch.randn(B, H, 1, D, device="cuda", dtype=torch.float16)
        k = torch.randn(B, H, N, D, device="cuda", dtype=torch.float16)
        v = torch.randn(B, H, N, D, device="cuda", dtype=torch.float16)
        ms_eager = do_bench(lambda: eager_decode(q, k, v))
        ms_fd = do_bench(lambda: flash_decoding(q, k, v, split_size=256))
        print(f"{N:>7} {ms_eager:>12.3f}m {ms_fd:>12.3f}m {ms_eager / ms_fd:>7.2f}x")


if __name__ == "__main__":
    from _timing import banner

    print(banner())
    print("=== correctness ===")
    check_correctness()
    print("=== benchmark (decode, M=1) ===")
    bench()
