"""The dispatch order the one-launch split-K forms rely on: the workgroups of a 1-D grid go to
the XCDs round-robin, workgroup b to XCD (b + c) % (XCC count), where the starting XCD c
depends on what was dispatched before; so workgroups whose ids differ by a multiple of 8 share
an XCD, and all slices of a column tile -- the blocks the GEMV (xcd_tile_slice in
pk_common.h), the register-dequant kernel and split-KV decode attention give one tile -- share
one XCD and its L2. Recorded per workgroup (hwreg XCC_ID) on launches with the product
kernels' grid sizes, block sizes and LDS, including grids larger than the machine holds at
once. A partition mode or dispatcher that broke the rule fails here instead of silently
corrupting the in-L2 handoff."""

from __future__ import annotations

import pytest
import torch

import _probes

pytestmark = pytest.mark.gpu


def _tile_of_gemv(b: int, split: int) -> int:
    """xcd_tile_slice: the column tile of workgroup b (GEMV and decode attention)."""
    return (b & 7) + 8 * ((b >> 3) // split)


def _tile_of_skinny(b: int, split: int, pair: bool) -> int:
    """The register-dequant kernel's one-launch grid: 128-column tiles in pairs on one XCD."""
    x, j = b & 7, b >> 3
    g = (j >> 1 if pair else j) // split
    return 16 * g + 2 * x + (j & 1) if pair else 8 * g + x


# (what, grid, threads, lds bytes, split, tile formula):
#  GEMV M=1 4096x11008: 43 tiles -> 48 slots x 16 slices, 4 waves, ~10 KB LDS
#  GEMV K=14336: 28 slices of 512 rows
#  decode attention B8 H32 N8192 split 256: 256 heads x 32 splits (larger than one residency)
#  register-dequant qkv M=8: 48 tiles of 128 columns x 4 slices, 8 waves, 34 KB LDS
CASES = [
    ("gemv_4096x11008", 8 * 6 * 16, 256, 9728, 16, lambda b: _tile_of_gemv(b, 16)),
    ("gemv_14336x4096", 8 * 2 * 28, 256, 9728, 28, lambda b: _tile_of_gemv(b, 28)),
    ("decode_B8H32_S32", 8 * 32 * 32, 256, 8192, 32, lambda b: _tile_of_gemv(b, 32)),
    ("skinny_qkv_M8", 48 * 4, 512, 34304, 4, lambda b: _tile_of_skinny(b, 4, True)),
]


@pytest.mark.parametrize("what,grid,threads,lds,split,tile_of", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("spin", [0, 200])
def test_workgroups_round_robin_over_xcds(what, grid, threads, lds, split, tile_of, spin, cuda):
    nxcc = _probes.xcc_count()
    assert nxcc in (1, 2, 4, 8), nxcc  # the product enables the handoff only for these
    out = torch.full((grid,), -1, dtype=torch.int32, device=cuda)
    _probes.xcc_probe(grid, threads, lds, spin, out)
    xcc = out.cpu().tolist()
    assert all(0 <= v < nxcc for v in xcc), sorted(set(xcc))
    # the dispatch rule itself: round-robin from the XCD of workgroup 0
    c = xcc[0]
    bad = [b for b in range(grid) if xcc[b] != (b + c) % nxcc]
    assert not bad, (f"{what}: {len(bad)} workgroups off the (b + {c}) % {nxcc} rule, first "
                     f"{bad[:8]}; XCC ids of workgroups 0..15: {xcc[:16]}")
    # what the kernels need from it: every slice of a tile on one XCD
    seen: dict[int, int] = {}
    for b in range(grid):
        t = tile_of(b)
        assert seen.setdefault(t, xcc[b]) == xcc[b], (what, b, t)
