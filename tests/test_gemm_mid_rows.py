"""The LDS-tiled W4A16 GEMM at 33..127 rows (its 64-row and ragged 128-row tiles), on the
shapes that still reach it now that the register-dequant kernel takes most of that range:
N % 16 != 0, K % 128 != 0, an explicit split whose wave rows exceed a group, and (above 64
rows) layers of more than 4096 x 4096 weights. Each against the numpy oracle
(oracle.w4a16_ref: the reference's dequant + fp32 matmul, gemm_int4.py:21-55), split and
unsplit, and bitwise reproducible."""

from __future__ import annotations

import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _case(M, K, N, G, seed, cuda):
    a = torch.randn(M, K, generator=_gen(seed)).half()
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), G)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    return a, qw, sc, codes, s16


# (K, N, group, splits): N % 16 != 0 (automatic split 2, and unsplit); K % 128 != 0 (group
# 32); an explicit split of 1 the register-dequant kernel rejects (wave rows > group);
# K * N > 4096^2 (rows above 64 only). Every N is off the packed-B kernel's N % 256 == 0.
SHAPES = [(1024, 520, 128, (0, 1)), (1056, 512, 32, (0,)), (2048, 1040, 128, (1,)),
          (1024, 16400, 128, (0, 2))]


@pytest.mark.parametrize("M", [33, 48, 63, 65, 100, 127])
@pytest.mark.parametrize("K,N,G,splits", SHAPES)
def test_lds_gemm_mid_rows(M, K, N, G, splits, cuda):
    if K * N > 4096 * 4096 and M <= 64:
        pytest.skip("the register-dequant kernel takes this layer at <= 64 rows")
    a, qw, sc, codes, s16 = _case(M, K, N, G, 3000 + M + N % 97 + K % 89, cuda)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    for split in splits:
        kid, used = _pk.w4a16_plan(M, N, K, G, split)
        assert kid == _pk.KERNEL_GEMM, (M, K, N, split, kid)
        out = gemm_int4.w4a16_gemm(ag, qw, sc, G, split_k=split or None, out_dtype=torch.float32)
        err = oracle.rel_fro(out.cpu().numpy(), ref)
        assert err <= TOL, (split, used, err)
        again = gemm_int4.w4a16_gemm(ag, qw, sc, G, split_k=split or None, out_dtype=torch.float32)
        assert torch.equal(out, again)
