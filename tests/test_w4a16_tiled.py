"""W4A16 on weights in blocks (pk_w4a16_gemm_tiled, the layout QuantLinear keeps in memory):
the same codes as pack_int4_n's (K, N/8) words in 16 KB blocks of 128 rows x 256 columns,
ordered by row block and then column tile. Through the C ABI, every kernel that reads the
layout -- the GEMV
(M <= 4, 256- and 512-row slices), the register-dequant kernel (5 <= M <= 128) and the
packed-B GEMM (M > 64, unsplit and split-K) -- must give bitwise the result of pk_w4a16_gemm
on the rows layout (itself checked against the oracle), for group sizes 64 / 128 / 256, the
per-tensor mode, bias, every output dtype and explicit splits; the headline shape is also
checked against the float64 oracle directly. Shapes or splits no tile-reading kernel takes
are refused with an error, never run on a rows-only kernel."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, G, seed, cuda):
    a = torch.randn(M, K, generator=_gen(seed)).half().to(cuda)
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half().to(cuda)
    if G:
        qw, sc = gemm_int4.quantize_int4_group(w, G)
    else:
        q = torch.randint(-8, 8, (K, N), generator=_gen(seed + 2), dtype=torch.int8)
        qw = gemm_int4.pack_int4_n(q.to(cuda)).view(torch.int32)
        sc = None
    return a, qw, sc


def _both(a, qw, sc, G, out_dtype=torch.float32, split_k=0, bias=None, scale=1.0):
    rows = _pk.w4a16_gemm(a, qw, sc, G, scale, out_dtype, split_k=split_k, bias=bias)
    tiles = _pk.w4a16_gemm(a, _pk.tile_weights(qw), sc, G, scale, out_dtype, split_k=split_k,
                           bias=bias, tiled=True)
    return rows, tiles


@pytest.mark.parametrize("M,K,N", [
    (1, 4096, 11008),   # the decode headline: 43 tiles x 16 slices
    (2, 1024, 768), (3, 512, 512), (4, 2048, 1280),
    (1, 14336, 4096),   # 512-row slices (two 64-row blocks per wave)
    (5, 1024, 512), (8, 4096, 6144), (16, 2048, 768), (17, 1024, 1024), (32, 4096, 4096),
    (33, 2048, 512), (48, 1024, 2304), (64, 4096, 1024),
    (65, 1024, 512), (96, 2048, 1024), (128, 4096, 6144), (128, 1024, 1024),
    (256, 1024, 768), (300, 768, 512), (2048, 4096, 4096),
])
def test_tiled_bitwise_equal_rows(M, K, N, cuda):
    a, qw, sc = _case(M, K, N, 128, M + K + N, cuda)
    kid, _ = _pk.w4a16_plan(M, N, K, 128, 0)
    assert kid in (_pk.KERNEL_GEMV, _pk.KERNEL_SKINNY, _pk.KERNEL_GEMM_TR4)
    rows, tiles = _both(a, qw, sc, 128)
    assert torch.equal(rows, tiles), (M, K, N, kid)


def test_tiled_headline_against_oracle(cuda):
    M, K, N = 1, 4096, 11008
    a = torch.randn(M, K, generator=_gen(7)).half()
    w = (torch.randn(K, N, generator=_gen(8)) * 0.02).half()
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    qw = torch.from_numpy(oracle.pack_int4_n(codes).view(np.int32).copy()).to(cuda)
    sc = torch.from_numpy(s16).to(cuda)
    out = _pk.w4a16_gemm(a.to(cuda), _pk.tile_weights(qw), sc, 128, 1.0, torch.float32, tiled=True)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(out.cpu().numpy(), ref) < 1e-3


@pytest.mark.parametrize("G", [0, 64, 256])
@pytest.mark.parametrize("M", [1, 8, 40, 200])
def test_tiled_groups_and_per_tensor(G, M, cuda):
    K, N = 2048, 768
    a, qw, sc = _case(M, K, N, G, 100 + G + M, cuda)
    rows, tiles = _both(a, qw, sc, G, scale=0.37 if G == 0 else 1.0)
    assert torch.equal(rows, tiles)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M", [2, 24, 100, 512])
def test_tiled_bias_and_dtypes(out_dtype, M, cuda):
    K, N = 1024, 1024
    a, qw, sc = _case(M, K, N, 128, 200 + M, cuda)
    bias = torch.randn(N, generator=_gen(3)).to(cuda)
    for b in (bias, bias.half()):
        rows, tiles = _both(a, qw, sc, 128, out_dtype=out_dtype, bias=b)
        assert torch.equal(rows, tiles)


@pytest.mark.parametrize("M,split", [(1, 8), (1, 4), (3, 16), (8, 2), (32, 4), (128, 2), (256, 4)])
def test_tiled_explicit_splits(M, split, cuda):
    K, N = 4096, 1024
    a, qw, sc = _case(M, K, N, 128, 300 + M + split, cuda)
    kid, used = _pk.w4a16_plan(M, N, K, 128, split)
    if kid not in (_pk.KERNEL_GEMV, _pk.KERNEL_SKINNY, _pk.KERNEL_GEMM_TR4):
        with pytest.raises(_pk.PicoKernelsError):
            _pk.w4a16_gemm(a, _pk.tile_weights(qw), sc, 128, 1.0, torch.float32, split_k=split,
                           tiled=True)
        return
    if kid == _pk.KERNEL_GEMV:
        # the GEMV's VALU kernel (slices other than 256 / 512 rows) reads rows only
        ks = K // used
        if ks not in (256, 512):
            with pytest.raises(_pk.PicoKernelsError):
                _pk.w4a16_gemm(a, _pk.tile_weights(qw), sc, 128, 1.0, torch.float32,
                               split_k=split, tiled=True)
            return
    rows, tiles = _both(a, qw, sc, 128, split_k=split)
    assert torch.equal(rows, tiles)


def test_tiled_rejects_shapes_it_cannot_read(cuda):
    a, qw, sc = _case(4, 1024, 520, 128, 9, cuda)          # N % 256 != 0
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_gemm(a, qw, sc, 128, 1.0, torch.float32, tiled=True)
    a, qw, sc = _case(4, 1024, 512, 32, 10, cuda)          # group 32
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_gemm(a, _pk.tile_weights(qw), sc, 32, 1.0, torch.float32, tiled=True)
    a, qw, sc = _case(256, 1024, 512, 128, 11, cuda)       # unsplit packed-B GEMM, unaligned output
    wide = torch.empty((256, 520), dtype=torch.float16, device=cuda)
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_gemm(a, _pk.tile_weights(qw), sc, 128, 1.0, torch.float16, split_k=1,
                       out=wide[:, 4:516], tiled=True)


def test_tiled_repeatable(cuda):
    a, qw, sc = _case(1, 4096, 11008, 128, 12, cuda)
    qt = _pk.tile_weights(qw)
    first = _pk.w4a16_gemm(a, qt, sc, 128, 1.0, torch.float16, tiled=True)
    for _ in range(3):
        assert torch.equal(first, _pk.w4a16_gemm(a, qt, sc, 128, 1.0, torch.float16, tiled=True))


def test_tiled_rows_beyond_32bit_offsets(cuda):
    """A block-layout call whose activations span more than 2 GiB (a ~75k-token prefill on the
    14336-deep down projection) runs in equal row chunks: each chunk bitwise the call on those
    rows alone, sample rows against the oracle."""
    M, K, N = 75000, 14336, 256
    assert M * K * 2 >= 2 ** 31
    g = torch.Generator(device=cuda).manual_seed(7)
    a = torch.randn(M, K, device=cuda, dtype=torch.float16, generator=g)
    w = (torch.randn(K, N, generator=_gen(8)) * 0.02).half()
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    qw = torch.from_numpy(oracle.pack_int4_n(codes).view(np.int32).copy()).to(cuda)
    sc = torch.from_numpy(s16).to(cuda)
    qt = _pk.tile_weights(qw)
    y = _pk.w4a16_gemm(a, qt, sc, 128, 1.0, torch.float16, tiled=True)
    rows = _pk.lib().pk_w4a16_tiled_rows_per_call(M, K)
    assert 0 < rows < M
    for r0 in range(0, M, rows):
        part = _pk.w4a16_gemm(a[r0:r0 + rows], qt, sc, 128, 1.0, torch.float16, tiled=True)
        assert torch.equal(y[r0:r0 + rows], part), r0
    pick = [0, 1, rows - 1, rows, M - 1]
    ref = oracle.w4a16_ref(a[pick].cpu().numpy(), codes, s16, 128)
    assert oracle.rel_fro(y[pick].float().cpu().numpy(), ref) <= 1e-3
