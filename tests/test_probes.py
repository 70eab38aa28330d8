"""The measurement probes behind `bench.py --hbm-ceiling` and `--mfma-ceiling`: the read probes
visit every word of the buffer exactly once (the XOR of their per-workgroup or per-wave results
equals the XOR of all words: the grid-stride probe for several grids and a ragged length, the
strip-pattern probe for several strip counts, strip sizes and blocks per wave), and the MFMA
probe's constant-operand run gives the closed-form sum."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _probes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("grid", [1, 7, 256, 2048])
@pytest.mark.parametrize("words", [4, 4 * 1000 + 4, 4 * 65536])
def test_read_probe_reads_every_word_once(grid, words, cuda):
    g = torch.Generator()
    g.manual_seed(grid + words)
    host = torch.randint(-2**31, 2**31 - 1, (words,), generator=g, dtype=torch.int64).to(torch.int32)
    src = host.to(cuda)
    out = torch.zeros(grid, dtype=torch.int32, device=cuda)
    _probes.read_probe(src, out, grid)
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    assert got == want


@pytest.mark.parametrize("strips,kb,u", [(688, 32, 4), (9, 11, 2), (16, 5, 8), (1, 1, 1)])
def test_strip_read_probe_reads_every_word_once(strips, kb, u, cuda):
    g = torch.Generator()
    g.manual_seed(strips * 100 + kb * 10 + u)
    words = strips * kb * 256  # kb blocks of 1 KB per strip
    host = torch.randint(-2**31, 2**31 - 1, (words,), generator=g, dtype=torch.int64).to(torch.int32)
    out = torch.zeros(64 * -(-strips // 8), dtype=torch.int32, device=cuda)
    _probes.strip_read_probe(host.to(cuda), strips, u, out)
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    assert got == want


def test_read_probe_rejects_bad_sizes(cuda):
    src = torch.zeros(3, dtype=torch.int32, device=cuda)  # 12 bytes: not a multiple of 16
    out = torch.zeros(4, dtype=torch.int32, device=cuda)
    with pytest.raises(_probes.ProbeError):
        _probes.read_probe(src, out, 4)


def test_mfma_probe_constant_operands(cuda):
    """fp16: every product is 0.5 * 0.5 and each accumulator element sums 16 of them per MFMA,
    so every lane's output is iters * 8 accumulators * 16 elements * 16 * 0.25."""
    grid, iters = 4, 10
    out = torch.zeros(grid * 512, dtype=torch.float32, device=cuda)
    _probes.mfma_probe(False, False, grid, iters, out)
    assert torch.all(out == iters * 8 * 16 * 16 * 0.25)
    _probes.mfma_probe(True, True, grid, iters, out)  # random fp8 operands: finite sums
    assert torch.isfinite(out).all()
