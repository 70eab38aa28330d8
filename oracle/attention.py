"""Decode attention oracle (test infrastructure only): float64 numpy restatement of the
reference's single-query attention.

``decode_attention_ref`` follows flash_decoding.eager_decode (flash_decoding.py:126-133):
``softmax(q @ K^T * scale) @ V`` per (batch, head) with ``scale = 1/sqrt(D)``, computed here
in float64 from the fp16 inputs. flash_decoding.flash_decoding (flash_decoding.py:47-115)
reorganises the same sum into per-split (max, sum, acc) partials; it agrees with this to
floating-point reassociation.

Pinned by closed forms in tests/test_oracle.py: constant V rows return that row whatever
the scores; identical keys give the mean of the V rows; N = 1 returns v_0; one dominant
score returns its V row.
"""

from __future__ import annotations

import numpy as np


def decode_attention_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                         sm_scale: float | None = None) -> np.ndarray:
    """q (B, H, 1 or absent, D), k/v (B, H, N, D) -> (B, H, D) float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    if q.ndim == 4:
        q = q[:, :, 0, :]
    D = q.shape[-1]
    scale = 1.0 / np.sqrt(D) if sm_scale is None else float(sm_scale)
    s = np.einsum("bhd,bhnd->bhn", q, k) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("bhn,bhnd->bhd", p, v)
