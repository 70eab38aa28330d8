"""Split-KV decode attention (drop-in flash_decoding, flash_decoding.py:30-133) on the GPU:
the reference's own tests with CPU-seeded inputs, parity with the float64 oracle over every
head dim and both kernel paths, split invariance, determinism, KV-cache views read in place."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import flash_decoding
import oracle

pytestmark = pytest.mark.gpu

TOL = 2e-5  # relative Frobenius error vs float64 (fp32 accumulation and exponentials)


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _qkv(B, H, N, D, seed, scale=1.0):
    q = (torch.randn(B, H, 1, D, generator=_gen(seed)) * scale).half()
    k = torch.randn(B, H, N, D, generator=_gen(seed + 1)).half()
    v = torch.randn(B, H, N, D, generator=_gen(seed + 2)).half()
    return q, k, v


def test_flash_decoding_matches_eager(cuda):
    """The reference's test (tests/test_flash_decoding.py:19-29)."""
    q, k, v = _qkv(2, 4, 1024, 64, 0)
    o = flash_decoding.flash_decoding(q.to(cuda), k.to(cuda), v.to(cuda), split_size=256)
    ref = flash_decoding.eager_decode(q.to(cuda), k.to(cuda), v.to(cuda))
    assert o.shape == (2, 4, 1, 64) and o.dtype == torch.float32
    assert torch.allclose(o.float(), ref.float(), atol=1e-2, rtol=1e-2)


def test_flash_decoding_is_causal_correct(cuda):
    """The reference's test (tests/test_flash_decoding.py:32-40): D = 32, split 128."""
    q, k, v = _qkv(1, 1, 512, 32, 1)
    o = flash_decoding.flash_decoding(q.to(cuda), k.to(cuda), v.to(cuda), split_size=128)
    ref = flash_decoding.eager_decode(q.to(cuda), k.to(cuda), v.to(cuda))
    assert torch.allclose(o.float(), ref.float(), atol=1e-2, rtol=1e-2)


def test_kv_cache_append_and_reset(cuda):
    """The reference's test (tests/test_flash_decoding.py:43-53)."""
    cache = flash_decoding.KVCache(batch=1, heads=2, head_dim=16, max_len=8, device=cuda,
                                   dtype=torch.float16)
    k = torch.randn(1, 2, 1, 16, generator=_gen(2)).half().to(cuda)
    v = torch.randn(1, 2, 1, 16, generator=_gen(3)).half().to(cuda)
    kc, vc = cache.append(k, v)
    assert cache.pos == 1 and kc.shape == (1, 2, 1, 16)
    assert torch.equal(kc[0, 0, 0], k[0, 0, 0])
    cache.reset()
    assert cache.pos == 0


# (B, H, N, D, split): 1, 2, 4, 8 or 16 register-resident row passes of a 256-thread
# workgroup; the 64- and 128-thread one-pass path; chunked online softmax for splits past 16
# passes (with a partial last chunk); splits that are not a whole number of passes (masked
# rows); D = 256; one split covering all of N; one-row splits
CASES = [(2, 4, 1024, 64, 256), (1, 2, 512, 32, 128), (2, 3, 2048, 128, 256), (1, 8, 1024, 16, 256),
         (3, 2, 4096, 64, 512), (2, 2, 1024, 128, 128), (1, 4, 256, 64, 16), (2, 2, 512, 64, 8),
         (1, 3, 640, 16, 64), (1, 2, 4096, 32, 1024), (4, 8, 4096, 128, 2048),
         (1, 2, 8192, 64, 1024), (1, 2, 4096, 128, 512), (1, 1, 8192, 16, 8192),
         (2, 2, 1152, 64, 384), (1, 2, 2880, 64, 960), (1, 1, 96, 64, 3), (1, 1, 777, 64, 777),
         (2, 3, 1024, 256, 256), (1, 2, 512, 256, 2), (1, 2, 4096, 256, 1024),
         (1, 2, 64, 64, 1), (1, 1, 200, 128, 40)]


@pytest.mark.parametrize("B,H,N,D,split", CASES)
def test_matches_float64_oracle(B, H, N, D, split, cuda):
    q, k, v = _qkv(B, H, N, D, 10 * D + split)
    o = flash_decoding.flash_decoding(q.to(cuda), k.to(cuda), v.to(cuda), split_size=split)
    ref = oracle.decode_attention_ref(q.numpy(), k.numpy(), v.numpy())
    assert oracle.rel_fro(o[:, :, 0].cpu().numpy(), ref) < TOL


def test_split_invariance_and_determinism(cuda):
    q, k, v = _qkv(2, 4, 4096, 64, 50)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    outs = {}
    for s in (32, 256, 512, 1024, 4096):
        o1 = flash_decoding.flash_decoding(qg, kg, vg, split_size=s)
        o2 = flash_decoding.flash_decoding(qg, kg, vg, split_size=s)
        assert torch.equal(o1, o2), f"split {s} not reproducible"
        outs[s] = o1.cpu().numpy()
    for s in outs:
        assert oracle.rel_fro(outs[s], outs[256]) < 1e-5


def test_kv_cache_prefix_read_in_place(cuda):
    """A prefix view of a longer cache (strided along N's parent dims) gives the same bits as
    a contiguous copy."""
    B, H, D, L, pos = 2, 4, 64, 4096, 1024
    cache = flash_decoding.KVCache(B, H, D, L, device=cuda)
    k = torch.randn(B, H, pos, D, generator=_gen(60)).half().to(cuda)
    v = torch.randn(B, H, pos, D, generator=_gen(61)).half().to(cuda)
    cache.k[:, :, :pos] = k
    cache.v[:, :, :pos] = v
    cache.pos = pos
    kc, vc = cache.k[:, :, :pos], cache.v[:, :, :pos]
    assert not kc.is_contiguous()
    q = torch.randn(B, H, 1, D, generator=_gen(62)).half().to(cuda)
    a = flash_decoding.flash_decoding(q, kc, vc, split_size=256)
    b = flash_decoding.flash_decoding(q, kc.contiguous(), vc.contiguous(), split_size=256)
    assert torch.equal(a, b)


def test_large_logits_and_divisibility(cuda):
    """Logits of a few hundred (q scaled by 16) stay finite through the max shift; N not a
    multiple of the split is refused as in the reference."""
    q, k, v = _qkv(1, 2, 1024, 64, 70, scale=16.0)
    o = flash_decoding.flash_decoding(q.to(cuda), k.to(cuda), v.to(cuda), split_size=256)
    assert torch.isfinite(o).all()
    ref = oracle.decode_attention_ref(q.numpy(), k.numpy(), v.numpy())
    assert oracle.rel_fro(o[:, :, 0].cpu().numpy(), ref) < 1e-4
    with pytest.raises(AssertionError):
        flash_decoding.flash_decoding(q.to(cuda), k[:, :, :1000].to(cuda), v[:, :, :1000].to(cuda),
                                      split_size=256)


def test_one_launch_combine_matches_two_launch(cuda):
    """B*H <= 512 combines in the split kernel's last workgroup; more heads take a combine
    launch. The same (b, h) gives the same bits either way, and the arrival counters are zero
    after every call."""
    import _pk

    H_big, N, D, split = 520, 512, 64, 128
    q, k, v = _qkv(1, H_big, N, D, 80)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    assert _pk.flash_decode_launches(1, H_big, N, D, split) == 2
    assert _pk.flash_decode_launches(1, 24, N, D, split) == 1
    two = flash_decoding.flash_decoding(qg, kg, vg, split_size=split)
    one = flash_decoding.flash_decoding(qg[:, :24], kg[:, :24], vg[:, :24], split_size=split)
    assert torch.equal(one, two[:, :24])
    key = (cuda.index, torch.cuda.current_stream(cuda).cuda_stream)
    assert int(torch.count_nonzero(_pk._workspaces[key][:64 << 10]).item()) == 0


def test_shares_the_gemm_workspace(cuda):
    """Decode attention and the W4A16 GEMV alternate on one stream's workspace."""
    import gemm_int4

    q, k, v = _qkv(2, 4, 2048, 128, 90)
    qg, kg, vg = q.to(cuda), k.to(cuda), v.to(cuda)
    ref = oracle.decode_attention_ref(q.numpy(), k.numpy(), v.numpy())
    a = torch.randn(1, 4096, generator=_gen(91)).half().to(cuda)
    w = (torch.randn(4096, 4096, generator=_gen(92)) * 0.02).half().to(cuda)
    qw, sc = gemm_int4.quantize_int4_group(w, 128)
    y0 = gemm_int4.w4a16_gemm(a, qw, sc, 128, out_dtype=torch.float32)
    for _ in range(3):
        o = flash_decoding.flash_decoding(qg, kg, vg, split_size=256)
        assert oracle.rel_fro(o[:, :, 0].cpu().numpy(), ref) < TOL
        assert torch.equal(gemm_int4.w4a16_gemm(a, qw, sc, 128, out_dtype=torch.float32), y0)


def test_graph_replays(cuda):
    """Captured once, replayed with eager work and synchronisation between replays: each replay
    equals the eager result."""
    import _pk

    B, H, N, D, split = 2, 8, 4096, 128, 256
    q, k, v = _qkv(B, H, N, D, 95)
    qg, kg, vg = q[:, :, 0].to(cuda), k.to(cuda), v.to(cuda)
    scale = 1.0 / math.sqrt(D)
    eager = _pk.flash_decode(qg, kg, vg, split, scale)
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        _pk.flash_decode(qg, kg, vg, split, scale)  # the stream's workspace exists before capture
        torch.cuda.synchronize(cuda)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = _pk.flash_decode(qg, kg, vg, split, scale)
    torch.cuda.synchronize(cuda)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, eager), rep
        assert torch.equal(_pk.flash_decode(qg, kg, vg, split, scale), eager)
