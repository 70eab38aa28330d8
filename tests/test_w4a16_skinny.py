"""W4A16 for 5 <= M <= 128 rows (the register-dequant MFMA kernel between the GEMV and the
LDS-tiled GEMM): parity with dequantize + fp32 matmul on CPU-seeded inputs, every path the
kernel has (one, two or four 16-row activation blocks, one or two row parts, 16 or 8 columns
per lane, 4 or 8 waves per workgroup, group scales or one tensor scale, ragged column tiles,
k-step counts per wave that are not a multiple of the prefetch depth, split-K partials and
their ordered reduction)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu

W4A16_TOL = 1e-3  # max relative Frobenius error vs dequant + fp32 matmul


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, seed, cuda, G=128):
    a = torch.randn(M, K, generator=_gen(seed)).half()
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), G)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    return a, qw, sc, codes, s16


@pytest.mark.parametrize("M", [5, 8, 16, 17, 24, 32])
@pytest.mark.parametrize("K,N", [(4096, 4096), (384, 528), (1152, 784), (640, 16)])
def test_skinny_group128(M, K, N, cuda):
    """N = 528 / 784 / 16 leave a ragged last column tile; K = 384 / 640 / 1152 need 3, 5 and
    9 slices of 4 waves (one 32-row k-step per wave), K = 4096 four k-steps per wave."""
    assert _pk.w4a16_plan(M, N, K, 128, 0)[0] == _pk.KERNEL_SKINNY
    a, qw, sc, codes, s16 = _case(M, K, N, 10 * M + K % 97 + N % 89, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err <= W4A16_TOL, f"rel err {err:.3e}"


@pytest.mark.parametrize("G", [32, 64, 256])
def test_skinny_group_sizes(G, cuda):
    M, K, N = 12, 1024, 512
    a, qw, sc, codes, s16 = _case(M, K, N, 40 + G, cuda, G=G)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, G, out_dtype=torch.float32)
    assert oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, G)) <= W4A16_TOL


@pytest.mark.parametrize("M", [8, 32])
def test_skinny_split_k_deterministic(M, cuda):
    """Every explicit split whose wave rows (K / split / waves) fit in one group is bitwise
    reproducible, and splits agree up to fp32 reassociation; other splits go to the GEMM, except
    that two 16-row blocks (M = 32) take wave rows of whole 128-row groups (split 1: 256 rows).
    Splits 4 and 8 run 8 waves per workgroup, 16 (128-row slices) 4 waves."""
    K, N = 2048, 1024
    a, qw, sc, codes, s16 = _case(M, K, N, 60 + M, cuda)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    spanning = M > 16
    assert _pk.w4a16_plan(M, N, K, 128, 1) == ((_pk.KERNEL_SKINNY, 1) if spanning
                                               else (_pk.KERNEL_GEMM, 1))
    base = None
    for s in ((1, 4, 8, 16) if spanning else (4, 8, 16)):
        assert _pk.w4a16_plan(M, N, K, 128, s) == (_pk.KERNEL_SKINNY, s)
        o1 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        o2 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        assert torch.equal(o1, o2), f"split {s} not reproducible"
        assert oracle.rel_fro(o1.cpu().numpy(), ref) <= W4A16_TOL
        base = o1 if base is None else base
        # fp32 reassociation, amplified ~10x by removing the +8 offset (as in the GEMV test)
        assert oracle.rel_fro(o1.cpu().numpy(), base.cpu().numpy()) < 1e-5


@pytest.mark.parametrize("M,K,N,split", [(32, 4096, 14336, 0), (24, 14336, 4096, 0),
                                         (17, 2048, 1024, 1), (20, 4096, 512, 1),
                                         (32, 4096, 768, 2), (30, 8192, 1280, 4)])
def test_skinny_group_spanning_waves(M, K, N, split, cuda):
    """Two 16-row blocks whose waves take several 128-row groups (gate_up and down at M = 32
    halve their slices this way; 2, 4 and 8 groups per wave here): each group's sums are
    scaled and added at its boundary. Within the oracle's tolerance, bitwise repeatable, the
    one-launch handoff bitwise equal to the partials plus the ordered reduce, and the block
    layout bitwise equal to the rows."""
    kid, used = _pk.w4a16_plan(M, N, K, 128, split)
    assert kid == _pk.KERNEL_SKINNY and K // used // 8 > 128, (kid, used)
    a, qw, sc, codes, s16 = _case(M, K, N, 500 + M + N % 97, cuda)
    ag = a.to(cuda)
    out = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, split_k=split)
    assert torch.equal(out, _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, split_k=split))
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(out.cpu().numpy(), ref) <= W4A16_TOL
    if used > 1:
        parts = _pk.w4a16_gemm_partials(ag, qw, sc, 128, used)
        two = torch.empty((M, N), dtype=torch.float32, device=cuda)
        _pk.splitk_reduce(parts, 1.0, two)
        assert torch.equal(out, two)
    if N % 256 == 0:
        tiles = _pk.w4a16_gemm(ag, _pk.tile_weights(qw), sc, 128, 1.0, torch.float32,
                               split_k=split, tiled=True)
        assert torch.equal(out, tiles)


@pytest.mark.parametrize("M,split", [(8, 4), (20, 8)])
def test_skinny_partials_then_reduce(M, split, cuda):
    """The two split-K phases reproduce the one-call result bit for bit, and a slice's partial
    is that K range's product."""
    K, N = 2048, 768
    a, qw, sc, codes, s16 = _case(M, K, N, 80 + M, cuda)
    ag = a.to(cuda)
    parts = _pk.w4a16_gemm_partials(ag, qw, sc, 128, split)
    assert tuple(parts.shape) == (split, M, N)
    out = torch.empty((M, N), dtype=torch.float32, device=cuda)
    _pk.splitk_reduce(parts, 1.0, out)
    fused = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=split, out_dtype=torch.float32)
    assert torch.equal(out, fused)
    ks = K // split
    s = split - 1
    ref = oracle.w4a16_ref(a.numpy()[:, s * ks:], codes[s * ks:], s16[s * ks // 128:], 128)
    assert oracle.rel_fro(parts[s].cpu().numpy(), ref) <= W4A16_TOL


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16])
def test_skinny_output_dtypes(out_dtype, cuda):
    M, K, N = 16, 1024, 1040
    a, qw, sc, codes, s16 = _case(M, K, N, 90, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    tol = {torch.float16: 2e-3, torch.bfloat16: 1e-2}[out_dtype]
    assert oracle.rel_fro(out.float().cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= tol


@pytest.mark.parametrize("M", [8, 30])
def test_skinny_per_tensor_int4_gemm(M, cuda):
    """The reference's int4_gemm (one tensor scale, gemm_int4.py:75-92) at skinny M: the codes
    are exact in fp16, so only the fp32 summation order differs from the closed form."""
    K, N = 1024, 512
    a = torch.randn(M, K, generator=_gen(95)).half()
    w = torch.randn(K, N, generator=_gen(96)).half()
    w_q, scale = gemm_int4.quantize_int4(w.to(cuda))
    c = gemm_int4.int4_gemm(a.to(cuda), gemm_int4.pack_int4_n(w_q), scale)
    ref = oracle.int4_gemm_ref(a.numpy(), w_q.cpu().numpy(), scale)
    assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("M", [9, 48, 100])
def test_skinny_strided_activations(M, cuda):
    """A row stride larger than K (a view into a wider buffer) is read in place, for one
    16-row block, several, and two row parts (the second part's A and C rows offset). N % 256
    != 0 keeps the packed-B GEMM out above 64 rows."""
    K, N = 1024, 528
    a, qw, sc, codes, s16 = _case(M, K, N, 97 + M, cuda)
    assert _pk.w4a16_plan(M, N, K, 128, 0)[0] == _pk.KERNEL_SKINNY
    wide = torch.zeros(M, K + 64, dtype=torch.float16)
    wide[:, :K] = a
    view = wide.to(cuda)[:, :K]
    out = gemm_int4.w4a16_gemm(view, qw, sc, 128, out_dtype=torch.float32)
    assert oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= W4A16_TOL


@pytest.mark.parametrize("M", [48, 100])
@pytest.mark.parametrize("out_dtype,tol", [(torch.float16, 2e-3), (torch.bfloat16, 1e-2)])
def test_skinny_out_view_and_dtypes(M, out_dtype, tol, cuda):
    """fp16 / bf16 output into a view of a wider buffer (ldc > N) with lda = K + 64, at two
    and four 16-row blocks (two row parts at 100): bitwise the contiguous call, the guard
    columns untouched."""
    K, N = 2048, 1040
    a, qw, sc, codes, s16 = _case(M, K, N, 150 + M, cuda)
    assert _pk.w4a16_plan(M, N, K, 128, 0)[0] == _pk.KERNEL_SKINNY
    ag = a.to(cuda)
    dense = _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, out_dtype)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(dense.float().cpu().numpy(), ref) <= tol
    wide_a = torch.zeros(M, K + 64, dtype=torch.float16, device=cuda)
    wide_a[:, :K] = ag
    wide_c = torch.full((M, N + 256), 5.0, dtype=out_dtype, device=cuda)
    _pk.w4a16_gemm(wide_a[:, :K], qw, sc, 128, 1.0, out_dtype, out=wide_c[:, :N])
    assert torch.equal(wide_c[:, :N], dense)
    assert bool((wide_c[:, N:] == 5.0).all())


def test_skinny_ineligible_shapes_use_gemm(cuda):
    """N % 16 != 0 or K % 128 != 0 stay on the LDS-tiled GEMM, still correct."""
    for M, K, N in ((8, 1024, 520), (8, 1056, 512)):
        assert _pk.w4a16_plan(M, N, K, 32, 0)[0] == _pk.KERNEL_GEMM
        a, qw, sc, codes, s16 = _case(M, K, N, 98 + N, cuda, G=32)
        out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 32, out_dtype=torch.float32)
        assert oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 32)) <= W4A16_TOL


@pytest.mark.parametrize("M,K,split", [(8, 3200, 5), (8, 4096, 2), (24, 3200, 5), (24, 4096, 1)])
def test_skinny_per_tensor_long_wave_rows(M, K, split, cuda):
    """One tensor scale puts no group limit on a wave's rows: 5 (4 waves), 8 and 16 k-steps
    (8 waves) per wave run the prefetch ring through refills and a partial last round."""
    N = 528
    assert _pk.w4a16_plan(M, N, K, 0, split) == (_pk.KERNEL_SKINNY, split)
    a = torch.randn(M, K, generator=_gen(110 + K)).half()
    q = torch.randint(-8, 8, (K, N), generator=_gen(111), dtype=torch.int8)
    qw = gemm_int4.pack_int4_n(q.to(cuda)).view(torch.int32)
    scale = 0.0123
    out = _pk.w4a16_gemm(a.to(cuda), qw, None, 0, scale, torch.float32, split_k=split)
    ref = oracle.int4_gemm_ref(a.numpy(), q.numpy(), scale)
    assert oracle.rel_fro(out.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("M", [33, 48, 64, 65, 100, 128])
@pytest.mark.parametrize("K,N", [(4096, 4000), (1152, 784), (640, 16)])
def test_skinny_four_blocks(M, K, N, cuda):
    """33 <= M <= 128: four 16-row blocks and 128-column tiles; above 64 rows two row parts
    per tile (their workgroups paired on one XCD), the second part ragged unless M = 128
    (N % 256 != 0 there: the packed-B GEMM takes the others)."""
    assert _pk.w4a16_plan(M, N, K, 128, 0)[0] == _pk.KERNEL_SKINNY
    a, qw, sc, codes, s16 = _case(M, K, N, 7 * M + K % 89 + N % 83, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err <= W4A16_TOL, f"rel err {err:.3e}"


@pytest.fixture
def layout():
    """Sets the register-dequant layout (pk_w4a16_skinny_layout) and restores the automatic
    one afterwards."""
    def set_layout(cfg: str) -> None:
        c, w = (int(x) for x in cfg.split(","))
        _pk.w4a16_skinny_layout(c, w)
    yield set_layout
    _pk.w4a16_skinny_layout(0, 0)


def test_skinny_layout_setter_rejects_bad_values():
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_skinny_layout(12, 8)
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_skinny_layout(8, 6)
    _pk.w4a16_skinny_layout(0, 0)


@pytest.mark.parametrize("M", [8, 24, 64, 128])
def test_skinny_layouts_agree(M, cuda, layout):
    """The tile layouts (columns per lane, waves): at one wave count the column width changes
    only which lane holds a column, so 16 and 8 columns per lane give the same bits; 8 waves
    split a slice's rows differently (fp32 reassociation only)."""
    K, N, split = 4096, 1040, 8
    a, qw, sc, codes, s16 = _case(M, K, N, 120 + M, cuda)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    outs = {}
    for cfg in ("16,4", "8,4", "16,8", "8,8"):
        layout(cfg)
        if M > 32 and cfg.startswith("16"):
            continue  # four blocks always use 8 columns per lane
        sp = split if cfg.endswith(",4") else 4
        assert _pk.w4a16_plan(M, N, K, 128, sp) == (_pk.KERNEL_SKINNY, sp)
        o = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=sp, out_dtype=torch.float32)
        assert oracle.rel_fro(o.cpu().numpy(), ref) <= W4A16_TOL, cfg
        outs[cfg] = o
    if "16,4" in outs:
        assert torch.equal(outs["16,4"], outs["8,4"])
        assert torch.equal(outs["16,8"], outs["8,8"])
    assert oracle.rel_fro(outs["8,8"].cpu().numpy(), outs["8,4"].cpu().numpy()) < 1e-5


@pytest.mark.parametrize("cfg", ["8,4", "8,8", "16,8"])
@pytest.mark.parametrize("M", [5, 20, 40, 97])
def test_skinny_layouts_edges(cfg, M, cuda, layout):
    """Every layout on ragged tiles, ragged row blocks and parts, per-tensor and group scales,
    and the automatic split (8 waves need slices of 8 * 32 rows)."""
    layout(cfg)
    for K, N, G in ((2048, 528, 128), (1024, 784, 64), (2560, 272, 32)):
        assert _pk.w4a16_plan(M, N, K, G, 0)[0] == _pk.KERNEL_SKINNY
        a, qw, sc, codes, s16 = _case(M, K, N, 130 + M + N, cuda, G=G)
        out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, G, out_dtype=torch.float32)
        err = oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, G))
        assert err <= W4A16_TOL, (K, N, G, err)
    K, N = 3072, 400
    a = torch.randn(M, K, generator=_gen(140 + M)).half()
    q = torch.randint(-8, 8, (K, N), generator=_gen(141), dtype=torch.int8)
    qw = gemm_int4.pack_int4_n(q.to(cuda)).view(torch.int32)
    out = _pk.w4a16_gemm(a.to(cuda), qw, None, 0, 0.02, torch.float32)
    assert oracle.rel_fro(out.cpu().numpy(), oracle.int4_gemm_ref(a.numpy(), q.numpy(), 0.02)) < 1e-5
