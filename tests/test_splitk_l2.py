"""Split-K slices that hand off through one XCD's L2 (the GEMV for M <= 4, the register-dequant
kernel for 5 <= M <= 16): the one-launch result must equal, bit for bit, the two-phase form
(per-slice partials, then the ordered pk_splitk_reduce), whatever the tile count (a multiple
of 8, not, fewer than 8), and the arrival counters at the head of the workspace must be zero
again after every call, so one workspace serves any sequence of shapes, including the
kernels that reduce in a second launch (more rows) and the dense split-K GEMM."""

from __future__ import annotations

import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu

COUNTER_BYTES = 64 << 10


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, seed, cuda):
    a = torch.randn(M, K, generator=_gen(seed)).half()
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), 128)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    return a, qw, sc, codes, s16


def _two_phase(ag, qw, sc, split, cuda):
    M = ag.shape[0]
    N = qw.shape[1] * 8
    parts = _pk.w4a16_gemm_partials(ag, qw, sc, 128, split)
    out = torch.empty((M, N), dtype=torch.float32, device=cuda)
    return _pk.splitk_reduce(parts, 1.0, out)


def _counters_zero(cuda) -> bool:
    key = (cuda.index, torch.cuda.current_stream(cuda).cuda_stream)
    ws = _pk._workspaces[key]
    return int(torch.count_nonzero(ws[:COUNTER_BYTES]).item()) == 0


# N: 11008 = 43 tiles of 256 columns (not a multiple of 8), 4096 = 16, 512 = 2 (< 8),
# 2016 = 8 tiles with a ragged last one; K = 14336 gives 28 slices of 512 rows (two row
# blocks per wave), K = 8192 32 slices of 256 rows.
@pytest.mark.parametrize("M,K,N", [(1, 4096, 11008), (1, 4096, 4096), (3, 2048, 512),
                                   (4, 4096, 2016), (1, 14336, 4096), (2, 1024, 11008),
                                   (2, 14336, 2048), (1, 8192, 4096)])
def test_gemv_l2_handoff_matches_two_phase(M, K, N, cuda):
    a, qw, sc, codes, s16 = _case(M, K, N, 1000 + M + N % 97, cuda)
    ag = a.to(cuda)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
    assert kid == _pk.KERNEL_GEMV and split > 1
    assert _pk.w4a16_launches(M, N, K, 128, 0) == (2 if N % 32 else 1)  # N % 32: VALU kernel
    one = gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32)
    assert torch.equal(one, _two_phase(ag, qw, sc, split, cuda))
    assert torch.equal(one, gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32))
    assert _counters_zero(cuda)
    assert oracle.rel_fro(one.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= 1e-4


# Tiles of 128 or 256 columns: 48, 86 (not a multiple of 8), 32, 5 (fewer than 8, ragged);
# one 16-row block (one launch), two (one launch on the smaller layers: 32 and 17 rows) and
# four (two launches: 48, 128, 100). Above 64 rows
# N % 256 != 0 keeps the packed-B GEMM out.
@pytest.mark.parametrize("M,K,N", [(8, 4096, 6144), (12, 4096, 11008), (32, 4096, 4096),
                                   (17, 2048, 528), (8, 14336, 4096), (128, 4096, 4000),
                                   (100, 2048, 1040), (48, 4096, 2048), (5, 1024, 4112),
                                   (16, 4096, 1024), (32, 14336, 4096), (24, 4096, 14336)])
def test_skinny_one_call_matches_two_phase(M, K, N, cuda):
    a, qw, sc, codes, s16 = _case(M, K, N, 1100 + M + N % 89, cuda)
    ag = a.to(cuda)
    kid, split = _pk.w4a16_plan(M, N, K, 128, 0)
    assert kid == _pk.KERNEL_SKINNY and split > 1
    # one launch for one 16-row block, and for two on layers of at most 4096 x 6144 weights
    # or with wave rows spanning several groups (half the slices)
    single = M <= 16 or (M <= 32 and (K * N <= 4096 * 6144 or K // split // 8 > 128))
    assert _pk.w4a16_launches(M, N, K, 128, 0) == (1 if single else 2)
    one = gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32)
    assert torch.equal(one, _two_phase(ag, qw, sc, split, cuda))
    assert torch.equal(one, gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32))
    assert _counters_zero(cuda)
    assert oracle.rel_fro(one.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= 1e-3


@pytest.mark.parametrize("M,split", [(12, 4), (8, 16), (16, 8), (5, 2)])
def test_skinny_explicit_splits_one_call(M, split, cuda):
    """Explicit splits run the one-launch handoff too (16 slices take two batches of loads in
    the last workgroup's sum), with fp16 output and a tensor scale."""
    K, N = 4096 if split > 2 else 1024, 1024
    a, qw, sc, codes, s16 = _case(M, K, N, 1150 + M + split, cuda)
    ag = a.to(cuda)
    assert _pk.w4a16_plan(M, N, K, 128, split) == (_pk.KERNEL_SKINNY, split)
    assert _pk.w4a16_launches(M, N, K, 128, split) == 1
    one = _pk.w4a16_gemm(ag, qw, sc, 128, 0.5, torch.float16, split_k=split)
    parts = _pk.w4a16_gemm_partials(ag, qw, sc, 128, split)
    two = torch.empty((M, N), dtype=torch.float16, device=cuda)
    _pk.splitk_reduce(parts, 0.5, two)
    assert torch.equal(one, two)
    assert _counters_zero(cuda)
    ref = 0.5 * oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(one.float().cpu().numpy(), ref) <= 2e-3


def test_one_workspace_many_shapes(cuda):
    """Alternate GEMV, skinny, LDS-tiled GEMM and dense split-K calls on the stream's one
    workspace, several rounds: every call stays right and the counters stay zero."""
    cases = [(1, 4096, 4096), (8, 2048, 1024), (128, 1024, 512), (2, 14336, 1024), (20, 4096, 2048)]
    data = [_case(M, K, N, 1200 + i, cuda) for i, (M, K, N) in enumerate(cases)]
    refs = [oracle.w4a16_ref(d[0].numpy(), d[3], d[4], 128) for d in data]
    b = torch.randn(1024, 512, generator=_gen(1299)).half()
    a16 = torch.randn(256, 1024, generator=_gen(1298)).half()
    ref16 = a16.float() @ b.float()
    for rep in range(3):
        for (M, K, N), d, ref in zip(cases, data, refs):
            out = gemm_int4.w4a16_gemm(d[0].to(cuda), d[1], d[2], 128, out_dtype=torch.float32)
            assert oracle.rel_fro(out.cpu().numpy(), ref) <= 1e-3, (rep, M, K, N)
            assert _counters_zero(cuda), (rep, M, K, N)
        c16 = _pk.gemm_f16(a16.to(cuda), b.to(cuda), torch.float32, 4)
        assert oracle.rel_fro(c16.cpu().numpy(), ref16.numpy()) < 1e-5
        assert _counters_zero(cuda)


def test_l2_handoff_in_graph_replays(cuda):
    """Captured once, replayed with eager work and synchronisation between replays: every
    replay equals the eager result (the counters reset themselves inside the graph)."""
    M, K, N = 1, 4096, 11008
    a, qw, sc, codes, s16 = _case(M, K, N, 1300, cuda)
    ag = a.to(cuda)
    eager = gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream(cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, out=out)  # workspace for this stream
        torch.cuda.synchronize(cuda)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            _pk.w4a16_gemm(ag, qw, sc, 128, 1.0, torch.float32, out=out)
    torch.cuda.synchronize(cuda)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, eager), rep
        other = gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float32)  # eager work between
        assert torch.equal(other, eager)
