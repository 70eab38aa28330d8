"""GPTQ column sweep on the GPU (pk_gptq_block): bit for bit the reference's column loop
(quantize.py:104-110, restated as oracle.gptq_sweep) on any block of columns, for every scale
domain shape (groups of rows, ragged last group, one scale per column up to thousands of rows),
bit widths and block offsets; and the whole gptq_layer with its two-level lazy batching
against the sequential oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import oracle
from quantize import gptq_layer

pytestmark = pytest.mark.gpu


def _ratio(n: int, rng) -> np.ndarray:
    """Upper-triangular ratios of a damped random Hessian's inverse (the reference's ratio)."""
    x = rng.standard_normal((2 * n, n)).astype(np.float32)
    h = (x.T @ x) / np.float32(2 * n) + np.float32(0.01) * np.eye(n, dtype=np.float32)
    hinv = np.linalg.inv(h).astype(np.float32)
    r = np.zeros_like(hinv)
    for j in range(n):
        r[j, j + 1:] = hinv[j, j + 1:] / hinv[j, j]
    return r


# (out, in, b0, nb, bits, group): groups of 128 / 16 / 64 rows with a ragged last group, one
# scale per column over 300 and 5000 rows (1024 threads, several rows each), 2- to 8-bit, a
# block in the middle of a wider matrix, a block shorter than the limit
CASES = [(256, 128, 0, 128, 4, 128), (200, 96, 0, 96, 4, 64), (48, 64, 0, 64, 3, 16),
         (300, 64, 0, 64, 4, 0), (5000, 16, 0, 4, 4, 0), (130, 200, 64, 37, 8, 128),
         (64, 40, 8, 32, 2, 0), (1100, 32, 0, 32, 4, 1024)]


@pytest.mark.parametrize("out,n_in,b0,nb,bits,group", CASES)
def test_block_sweep_is_the_reference_loop(out, n_in, b0, nb, bits, group, cuda):
    assert nb <= _pk.gptq_block_cols(out, group)
    rng = np.random.default_rng(out + n_in + nb + bits)
    w = (rng.standard_normal((out, n_in)) * 0.1).astype(np.float32)
    r = _ratio(n_in, rng)
    gs = None if group == 0 else group
    ref_block, ref_err = oracle.gptq_sweep(w[:, b0:b0 + nb], r[b0:b0 + nb, b0:b0 + nb], bits, gs)
    q = torch.from_numpy(w).to(cuda)
    err = torch.full((out, nb + 3), float("nan"), device=cuda)
    _pk.gptq_block(q, torch.from_numpy(r).to(cuda), err, b0, nb, bits, group)
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, b0:b0 + nb], ref_block)
    assert np.array_equal(err[:, :nb].cpu().numpy(), ref_err)
    assert np.array_equal(qh[:, :b0], w[:, :b0]) and np.array_equal(qh[:, b0 + nb:], w[:, b0 + nb:])
    assert torch.isnan(err[:, nb:]).all()  # nothing written past the block


def test_block_limits_and_errors(cuda):
    assert _pk.gptq_block_cols(4096, 128) == 128
    assert _pk.gptq_block_cols(4096, 0) == 8
    assert _pk.gptq_block_cols(14336, 0) == 2
    q = torch.zeros(64, 32, device=cuda)
    r = torch.zeros(32, 32, device=cuda)
    e = torch.zeros(64, 32, device=cuda)
    with pytest.raises(_pk.PicoKernelsError):
        _pk.gptq_block(q, r, e, 16, 32, 4, 0)  # columns past the matrix
    with pytest.raises(_pk.PicoKernelsError):
        _pk.gptq_block(q, r, e, 0, 8, 1, 0)  # 1-bit has no levels


@pytest.mark.parametrize("out,n_in,group", [(96, 300, 16), (600, 272, 0), (2000, 160, 0),
                                            (256, 384, 128)])
def test_gptq_layer_matches_sequential_oracle(out, n_in, group, cuda):
    """Whole layers: the kernel's sweeps plus the GEMM updates between them (inner blocks of
    8..128 columns, 128-column outer blocks) against the one-column-at-a-time oracle."""
    rng = np.random.default_rng(out * 7 + n_in)
    W = (rng.standard_normal((out, n_in)) * 0.1).astype(np.float32)
    X = rng.standard_normal((2 * n_in, n_in)).astype(np.float32)
    X[:, : n_in // 8] *= 4.0
    gs = None if group == 0 else group
    ours = gptq_layer(torch.from_numpy(W).to(cuda), torch.from_numpy(X).to(cuda), 4,
                      group_size=gs).cpu().numpy()
    ref = oracle.gptq_layer(W, X, 4, group_size=gs)
    # the GEMM updates between sweeps round differently from the sequential loop, so a value
    # near a rounding tie can take the neighbouring code and the error feedback carries that
    # on: element-wise agreement (the golden vectors' bar) plus a loose overall bound
    close = np.isclose(ours, ref, atol=1e-4, rtol=1e-3)
    assert close.mean() > 0.99, f"{(~close).sum()} of {close.size} differ"
    assert oracle.rel_fro(ours, ref) < 1e-2


def test_gptq_layer_leaves_its_input_alone(cuda):
    g = torch.Generator()
    g.manual_seed(5)
    W = torch.randn(64, 48, generator=g).to(cuda)
    X = torch.randn(32, 48, generator=g).to(cuda)
    W0 = W.clone()
    gptq_layer(W, X, 4, act_order=False)
    assert torch.equal(W, W0)


@pytest.mark.parametrize("group", [0, 128])
def test_gptq_layer_loss_matches_sequential_oracle(group, cuda):
    """At 1024 x 1024 the error feedback carries rounding differences (GEMM order, the inverse)
    into a few percent of the codes, as between any two fp32 implementations; the GPTQ
    objective ||X (Q - W)^T||^2 stays within 0.5% of the sequential oracle's, and well below
    round-to-nearest's."""
    g = torch.Generator()
    g.manual_seed(1)
    W = torch.randn(1024, 1024, generator=g) * 0.02
    X = torch.randn(1024, 1024, generator=g)
    X[:, :128] *= 4
    gs = None if group == 0 else group
    ref = torch.from_numpy(oracle.gptq_layer(W.numpy(), X.numpy(), 4, group_size=gs))
    ours = gptq_layer(W.to(cuda), X.to(cuda), 4, group_size=gs).cpu()
    rtn = torch.from_numpy(oracle.rtn_layer(W.t().contiguous().numpy(), 4, gs)).t()

    def loss(q):
        return float(((X @ (q - W).t()) ** 2).sum() / ((X @ W.t()) ** 2).sum())

    assert abs(loss(ours) / loss(ref) - 1) < 5e-3, (loss(ours), loss(ref))
    assert loss(ours) < 0.9 * loss(rtn)
    assert torch.isclose(ours, ref, atol=1e-4, rtol=1e-3).float().mean() > 0.9


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 100, 128, 129, 300, 1000])
def test_blocked_cholesky_matches_one_call(n, cuda):
    """gptq_layer's blocked factorisation equals torch.linalg.cholesky to fp32 rounding and
    reports a matrix that is not positive definite."""
    import quantize

    g = torch.Generator()
    g.manual_seed(n)
    x = torch.randn(max(n // 2, 4), n, generator=g)
    h = (x.t() @ x) / x.shape[0]
    h.diagonal().add_(0.01 * torch.diagonal(h).mean())
    h = h.to(cuda)
    L, ok = quantize._blocked_cholesky(h)
    assert ok
    ref = torch.linalg.cholesky(h.double())
    assert ((L.double() - ref).norm() / ref.norm()).item() < 1e-5
    assert torch.equal(L, torch.tril(L))
    bad = h.clone()
    bad[n - 1, n - 1] = -1.0
    assert not quantize._blocked_cholesky(bad)[1]
