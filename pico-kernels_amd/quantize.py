"""Round-to-nearest and GPTQ weight quantization on MI355X -- drop-in for the quantization
primitives of the reference's ``quantize`` module.

Reference entry points kept with their signatures (file:line in the reference repository):
  * ``quantize_col(w, bits, group_size=None)``  quantize.py:42-60
  * ``rtn_layer(w, bits, group_size=None)``     quantize.py:63-68
  * ``gptq_layer(w, x, bits, damp=0.01, act_order=True, group_size=None)``
                                                 quantize.py:71-115

``quantize_col`` / ``rtn_layer`` run one HIP kernel (``pk_quantize_group``) that reproduces the
reference's torch arithmetic bit for bit: fp32 for ``rtn_layer`` (which widens first) and the
tensor's own dtype for ``quantize_col`` on an fp16/bf16 vector. ``gptq_layer`` keeps the
reference's update rule (each column's rounding error is pushed onto the later columns with
the fixed ratios ``H^-1[j, j+1:] / H^-1[j, j]``) but runs it on the GPU as a blocked
("lazy batch") sweep: columns are quantized one by one inside a block of 128, the block's
accumulated errors reach the remaining columns through one matmul. That is the same sum of
rank-1 updates, reassociated, so results agree with the sequential form to fp32 rounding.

The PicoLM perplexity driver of the reference (quantize.py:121-265) is not part of this path.
"""

from __future__ import annotations

import torch

import _pk

__all__ = ["quantize_col", "rtn_layer", "gptq_layer"]

_GPTQ_BLOCK = 128


def quantize_col(w: torch.Tensor, bits: int, group_size: int | None = None) -> torch.Tensor:
    """Symmetric round-to-nearest quantization of a column ``[out]`` (quantize.py:42-60).

    ``group_size=None`` uses one scale for the whole vector; otherwise consecutive groups of
    ``group_size`` elements share a scale (the last group may be shorter).
    """
    if bits >= 16:
        return w
    wg = _pk.to_gpu(w).reshape(-1, 1)
    half_math = wg.dtype in (torch.float16, torch.bfloat16)
    _, _, fake = _pk.quantize_group(wg, bits, group_size, half_math=half_math, want_qweight=False,
                                    want_scales=False, want_fake=True, fake_dtype=w.dtype)
    fake = fake.reshape(w.shape)
    return fake if w.is_cuda else fake.to(w.device)


def rtn_layer(w: torch.Tensor, bits: int, group_size: int | None = None) -> torch.Tensor:
    """Naive round-to-nearest over every column -- the GPTQ baseline (quantize.py:63-68)."""
    if bits >= 16:
        return w.clone()
    assert w.dim() == 2
    wg = _pk.to_gpu(w)
    _, _, fake = _pk.quantize_group(wg, bits, group_size, half_math=False, want_qweight=False,
                                    want_scales=False, want_fake=True, fake_dtype=w.dtype)
    return fake if w.is_cuda else fake.to(w.device)


def _blocked_cholesky(h: torch.Tensor, nb: int = 128) -> tuple[torch.Tensor, bool]:
    """Lower Cholesky factor of a symmetric positive definite fp32 matrix, right-looking in
    blocks of ``nb`` columns: each diagonal block factored by the solver, the panel below it
    by a triangular solve, the trailing matrix updated by one GEMM. The same factorisation as
    one ``torch.linalg.cholesky`` call (to fp32 rounding) in 8.7 ms instead of 12.8 at 4096
    rows on MI355X, where the solver's one-call path spends its time in small diagonal-block
    kernels. Returns (L, ok); ok is False if a pivot was not positive."""
    a = h.clone()
    n = a.shape[0]
    infos = []
    for j in range(0, n, nb):
        e = min(j + nb, n)
        ljj, info = torch.linalg.cholesky_ex(a[j:e, j:e])
        infos.append(info)
        a[j:e, j:e] = ljj
        if e < n:
            # panel = A_ij L_jj^-T (a right-sided solve), trailing -= panel panel^T in the GEMM
            panel = torch.linalg.solve_triangular(ljj.t(), a[e:, j:e], upper=True, left=False)
            a[e:, j:e] = panel
            a[e:, e:].addmm_(panel, panel.t(), alpha=-1.0)
    ok = int(torch.stack(infos).abs().sum().item()) == 0
    return torch.tril(a), ok


def gptq_layer(w: torch.Tensor, x: torch.Tensor, bits: int, damp: float = 0.01,
               act_order: bool = True, group_size: int | None = None) -> torch.Tensor:
    """GPTQ-quantize one linear layer ``w`` (``[out, in]``) given activations ``x`` (``[n, in]``).

    Same algorithm as quantize.py:71-115 (Hessian ``X^T X / n`` with damping
    ``damp * mean(diag)``, its inverse, optional activation ordering by ``diag(H)``, column
    sweep with error feedback, un-permute). Output has ``w``'s dtype and device. The column
    sweep runs in blocks on the GPU (``pk_gptq_block``); inside a block it is the reference's
    loop bit for bit, between blocks the updates are GEMMs.
    """
    if bits >= 16:
        return w.clone()
    dev = _pk.gpu_device() if not w.is_cuda else w.device
    W = w.to(dev).float()
    X = x.to(dev).float()
    out_dim, in_dim = W.shape
    n = X.shape[0]

    H = (X.t() @ X) / n
    energy = torch.diagonal(H).clone()
    H.diagonal().add_(damp * energy.mean())
    # H is symmetric positive definite once damped: invert through its Cholesky factor (half
    # the time of a general inverse at 4096); fall back to the general inverse, as the
    # reference computes it (quantize.py:94), when the factorisation fails.
    L, ok = _blocked_cholesky(H)
    Hinv = torch.cholesky_inverse(L) if ok else torch.linalg.inv(H)

    order = None
    if act_order:
        order = torch.argsort(energy, descending=True)
        W = W[:, order]
        Hinv = Hinv[order][:, order]
    # ratios[j, c] = Hinv[j, c] / Hinv[j, j] for c > j (strictly upper triangle).
    ratios = torch.triu(Hinv / torch.diagonal(Hinv).unsqueeze(1), diagonal=1)

    # Lazy batching on two levels: the HIP kernel sweeps `nb` columns at a time (the error
    # feedback inside the sweep follows the reference's column order exactly); a small GEMM
    # carries a sweep's errors to the rest of its 128-column block, and one GEMM per block
    # carries the block's errors to every later column.
    Q = W.clone(memory_format=torch.contiguous_format)  # never the caller's tensor
    ratios = ratios.contiguous()
    g = 0 if group_size is None else int(group_size)
    nb = min(_GPTQ_BLOCK, _pk.gptq_block_cols(out_dim, g))
    assert nb >= 1, f"gptq_layer: a scale group of {out_dim if g == 0 else g} rows is too large"
    err = torch.empty((out_dim, _GPTQ_BLOCK), dtype=torch.float32, device=dev)
    for o0 in range(0, in_dim, _GPTQ_BLOCK):
        o1 = min(o0 + _GPTQ_BLOCK, in_dim)
        for b0 in range(o0, o1, nb):
            b1 = min(b0 + nb, o1)
            e = err[:, b0 - o0:b1 - o0]
            _pk.gptq_block(Q, ratios, e, b0, b1 - b0, bits, g)
            if b1 < o1:
                Q[:, b1:o1].sub_(e @ ratios[b0:b1, b1:o1])
        if o1 < in_dim:
            Q[:, o1:].sub_(err[:, :o1 - o0] @ ratios[o0:o1, o1:])

    if order is not None:
        Q = Q[:, torch.argsort(order)]
    return Q.to(w.dtype).to(w.device)
