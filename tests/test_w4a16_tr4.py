"""The W4A16 GEMM that keeps the int4 weights packed in LDS (w4a16_tr4.hip, plan kernel id 4):
against the float64 dequantise-and-matmul oracle, through the C ABI, on every k-tile remainder
its unrolled loop has (1 to 7 tiles of 128 k), ragged M, group sizes 64 / 128 / 256 and the
per-tensor mode, strided activations, an output view wider than N, every output dtype; split-K
(fp32 partial planes and the ordered reduce) from 65 rows, automatic and explicit splits;
results bitwise reproducible run to run."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu


def _case(M, K, N, G, seed, cuda):
    g = torch.Generator()
    g.manual_seed(seed)
    a = torch.randn(M, K, generator=g).half()
    w = (torch.randn(K, N, generator=g) * 0.02).half()
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    qw = torch.from_numpy(oracle.pack_int4_n(codes).view(np.int32).copy()).to(cuda)
    sc = torch.from_numpy(s16).to(cuda)
    return a, codes, s16, qw, sc


@pytest.mark.parametrize("M,K,N,G", [
    (256, 128, 256, 128),    # one k-tile
    (256, 256, 512, 64),     # two, group 64 (each k half its own scale row)
    (300, 384, 256, 128),    # three, ragged M
    (256, 512, 768, 256),    # four, group 256
    (384, 640, 256, 128),    # five
    (512, 768, 512, 128),    # six (one pass of the unrolled loop)
    (257, 896, 256, 64),     # seven (loop + one), one row past a tile
    (2048, 4096, 4096, 128), # the prefill shape
    (65, 896, 256, 64),      # 64-row tiles (up to 128 rows): seven k-tiles, one row past a tile
    (128, 640, 512, 128),    # 64-row tiles: five k-tiles, two full tiles
    (100, 768, 768, 256),    # 64-row tiles: six k-tiles, group 256, ragged rows
])
def test_tr4_matches_oracle(M, K, N, G, cuda):
    a, codes, s16, qw, sc = _case(M, K, N, G, M + K + N, cuda)
    assert _pk.w4a16_plan(M, N, K, G, 1) == (_pk.KERNEL_GEMM_TR4, 1)
    out = _pk.w4a16_gemm(a.to(cuda), qw, sc, G, 1.0, torch.float32, split_k=1)
    again = _pk.w4a16_gemm(a.to(cuda), qw, sc, G, 1.0, torch.float32, split_k=1)
    assert torch.equal(out, again), "not bitwise reproducible"
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err < 1e-3, err  # dequantised weights rounded to fp16 (as the other GEMMs): ~2.7e-4


def test_tr4_per_tensor_mode(cuda):
    """int4_gemm's per-tensor path (codes in [-8, 7], the scale in the epilogue)."""
    g = torch.Generator()
    g.manual_seed(11)
    M, K, N = 2048, 512, 2048  # unsplit (smaller outputs take split-K kernels)
    a = torch.randn(M, K, generator=g).half()
    q = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int8)
    packed = torch.from_numpy(oracle.pack_int4_n(q.numpy()))
    assert _pk.w4a16_plan(M, N, K, 0, 0) == (_pk.KERNEL_GEMM_TR4, 1)
    out = gemm_int4.int4_gemm(a.to(cuda), packed.to(cuda), 0.037)
    ref = (a.double().numpy() @ q.double().numpy()) * 0.037
    assert oracle.rel_fro(out.cpu().numpy(), ref) < 1e-5  # codes are exact in fp16


@pytest.mark.parametrize("M", [384, 96])  # 128-row tiles, 64-row tiles
@pytest.mark.parametrize("out_dtype,tol", [(torch.float16, 2e-3), (torch.bfloat16, 1e-2),
                                           (torch.float32, 1e-3)])
def test_tr4_output_dtypes(M, out_dtype, tol, cuda):
    K, N, G = 512, 512, 128
    a, codes, s16, qw, sc = _case(M, K, N, G, 5, cuda)
    assert _pk.w4a16_plan(M, N, K, G, 1) == (_pk.KERNEL_GEMM_TR4, 1)
    out = _pk.w4a16_gemm(a.to(cuda), qw, sc, G, 1.0, out_dtype, split_k=1)
    assert out.dtype == out_dtype
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(out.float().cpu().numpy(), ref) < tol


@pytest.mark.parametrize("M,split", [(320, 0), (72, 1)])  # automatic (split-K), 64-row tiles
def test_tr4_strided_operands(M, split, cuda):
    """A with lda > K and an output view into a wider buffer (ldc > N): the same bits as
    contiguous operands."""
    K, N, G = 512, 512, 128
    a, codes, s16, qw, sc = _case(M, K, N, G, 9, cuda)
    a_wide = torch.zeros(M, K + 64, dtype=torch.float16)
    a_wide[:, :K] = a
    a_view = a_wide.to(cuda)[:, :K]
    big = torch.full((M, N + 256), 7.0, dtype=torch.float16, device=cuda)
    out_view = big[:, 128:128 + N]
    _pk.w4a16_gemm(a_view, qw, sc, G, 1.0, torch.float16, split_k=split, out=out_view)
    ref = _pk.w4a16_gemm(a.to(cuda), qw, sc, G, 1.0, torch.float16, split_k=split)
    assert torch.equal(out_view, ref)
    assert torch.all(big[:, :128] == 7.0) and torch.all(big[:, 128 + N:] == 7.0)


# (M, K, N, G, automatic split): the sweep's qkv layer at 128 rows (64-row tiles, 4 slices),
# ragged rows with a one-tile slice, group 64 and 256, the largest slice count (16), 64-row
# tiles at 129 rows (8 of 16 and of 112 k-tiles), the sweep's down layer (8 of 112), 128-row
# tiles with a power of two chosen over the most slices (4 of 112, not 7), and a slice count
# that is not a power of two (15 of 15 k-tiles, reduced by the generic-count kernel)
SPLIT_CASES = [
    (128, 4096, 6144, 128, 4),
    (65, 1024, 512, 64, 8),
    (100, 2048, 256, 256, 16),
    (129, 2048, 1024, 128, 8),
    (129, 14336, 2048, 128, 8),
    (128, 14336, 4096, 128, 8),
    (256, 14336, 4096, 128, 4),
    (128, 1920, 256, 128, 15),
]


@pytest.mark.parametrize("M,K,N,G,auto", SPLIT_CASES)
def test_tr4_split_k_matches_oracle(M, K, N, G, auto, cuda):
    a, codes, s16, qw, sc = _case(M, K, N, G, 40 + M + N, cuda)
    assert _pk.w4a16_plan(M, N, K, G, 0) == (_pk.KERNEL_GEMM_TR4, auto)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    base = None
    for s in (0, 1, 2):
        out = _pk.w4a16_gemm(ag, qw, sc, G, 1.0, torch.float32, split_k=s)
        again = _pk.w4a16_gemm(ag, qw, sc, G, 1.0, torch.float32, split_k=s)
        assert torch.equal(out, again), f"split {s} not bitwise reproducible"
        err = oracle.rel_fro(out.cpu().numpy(), ref)
        assert err < 1e-3, (s, err)
        # splits differ only by fp32 reassociation
        base = out if base is None else base
        assert oracle.rel_fro(out.cpu().numpy(), base.cpu().numpy()) < 1e-6


def test_tr4_split_k_per_tensor_strided_out(cuda):
    """Per-tensor mode through split-K (the tensor scale applied by the reduce), fp16 out into
    a view wider than N: the same bits as a contiguous output, the margins untouched."""
    g = torch.Generator()
    g.manual_seed(12)
    M, K, N = 96, 1024, 512
    a = torch.randn(M, K, generator=g).half()
    q = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int8)
    packed = torch.from_numpy(oracle.pack_int4_n(q.numpy()).view(np.int32).copy()).to(cuda)
    kid, split = _pk.w4a16_plan(M, N, K, 0, 0)
    assert kid == _pk.KERNEL_GEMM_TR4 and split > 1
    ag = a.to(cuda)
    out = _pk.w4a16_gemm(ag, packed, None, 0, 0.037, torch.float32)
    ref = (a.double().numpy() @ q.double().numpy()) * 0.037
    assert oracle.rel_fro(out.cpu().numpy(), ref) < 1e-5  # codes are exact in fp16
    dense = _pk.w4a16_gemm(ag, packed, None, 0, 0.037, torch.float16)
    big = torch.full((M, N + 256), 3.0, dtype=torch.float16, device=cuda)
    _pk.w4a16_gemm(ag, packed, None, 0, 0.037, torch.float16, out=big[:, 128:128 + N])
    assert torch.equal(big[:, 128:128 + N], dense)
    assert torch.all(big[:, :128] == 3.0) and torch.all(big[:, 128 + N:] == 3.0)


@pytest.mark.parametrize("M", [33, 48, 64])
@pytest.mark.parametrize("K,N", [(4096, 11008), (14336, 4096)])
def test_tr4_mid_rows_on_large_layers(M, K, N, cuda):
    """33..64 rows of layers of more than 4096 x 8192 weights run the packed-B GEMM with an
    automatic split: one 128-row tile, most of it past M, split-K partials and the ordered
    reduce; against the oracle, bitwise repeatable, and on the block layout bitwise equal."""
    a, codes, s16, qw, sc = _case(M, K, N, 128, 900 + M + K % 97, cuda)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
    assert kid == _pk.KERNEL_GEMM_TR4 and split > 1
    ag = a.to(cuda)
    out = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32)
    assert torch.equal(out, _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32))
    assert oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= 1e-3
    tiles = _pk.w4a16_gemm(ag, _pk.tile_weights(qw), sc, 128, 1.0, torch.float32, tiled=True)
    assert torch.equal(out, tiles)


@pytest.mark.parametrize("pad,offset", [(4, 0), (1, 0), (4, 1)])
def test_tr4_strided_and_offset_weight_views(pad, offset, cuda):
    """Row-layout weights as a view into a wider buffer (ldq = N/8 + pad words) starting
    `offset` words in: a 16-byte aligned base and row pitch run the packed-B GEMM, anything
    else the GEMM that gathers B through registers; both against the oracle, bitwise repeatable."""
    M, K, N, G = 128, 1024, 512, 128
    a, codes, s16, qw, sc = _case(M, K, N, G, 77 + pad + offset, cuda)
    wide = torch.zeros((K, N // 8 + pad + offset), dtype=torch.int32, device=cuda)
    view = wide[:, offset:offset + N // 8]
    view.copy_(qw)
    assert view.stride(0) == N // 8 + pad + offset and view.data_ptr() % 16 == 4 * offset % 16
    ag = a.to(cuda)
    out = _pk.w4a16_gemm(ag, view, sc, G, 1.0, torch.float32)
    assert torch.equal(out, _pk.w4a16_gemm(ag, view, sc, G, 1.0, torch.float32))
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(out.cpu().numpy(), ref) < 1e-3
    if pad % 4 == 0 and offset == 0:  # aligned: the same kernel and bits as contiguous weights
        assert torch.equal(out, _pk.w4a16_gemm(ag, qw, sc, G, 1.0, torch.float32))
