"""The reduce-launch form of the one-launch split-K kernels: what a device takes when the
library's placement probe finds workgroups off the XCD rule the in-L2 handoff needs (or the
XCC count does not divide 8, or PK_SPLITK_IN_L2=0). It must give the bits of the one-launch
form. The switch is read once per process, so the reduce-launch side runs in one child
process with PK_SPLITK_IN_L2=0 and hands its outputs back through a .npz file."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import _pk

ROOT = Path(__file__).resolve().parents[1]

# The shapes: the split-K GEMV (M = 1, row layout, 16 slices), the register-dequant kernel with
# one 16-row block (M = 8, 4096 x 4096 blocks) and with group-spanning waves (M = 32,
# 4096 x 14336 blocks), and split-KV decode attention.
CASES = r"""
import sys
import numpy as np
import torch

def gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g

def run(dev):
    import _pk, gemm_int4, flash_decoding
    out = {}
    for name, (M, K, N, tiled) in {"gemv": (1, 4096, 11008, False), "skinny8": (8, 4096, 4096, True),
                                   "skinny32": (32, 14336, 4096, True)}.items():
        a = torch.randn(M, K, generator=gen(M + N)).half().to(dev)
        w = (torch.randn(K, N, generator=gen(K + N)) * 0.02).half().to(dev)
        qw, sc = gemm_int4.quantize_int4_group(w, 128)
        q = _pk.tile_weights(qw) if tiled else qw
        y = _pk.w4a16_gemm(a, q, sc, 128, 1.0, torch.float32, tiled=tiled)
        out[name] = y.cpu().numpy()
        out[name + "_launches"] = np.array(_pk.w4a16_launches(M, N, K, 128, 0))
    B, H, N, D = 2, 4, 2048, 64
    q = torch.randn(B, H, 1, D, generator=gen(1)).half().to(dev)
    k = torch.randn(B, H, N, D, generator=gen(2)).half().to(dev)
    v = torch.randn(B, H, N, D, generator=gen(3)).half().to(dev)
    out["decode"] = flash_decoding.flash_decoding(q, k, v, split_size=256).cpu().numpy()
    out["decode_launches"] = np.array(_pk.flash_decode_launches(B, H, N, D, 256))
    return out
"""

CHILD = CASES + r"""
if __name__ == "__main__":
    sys.path[:0] = [sys.argv[1], sys.argv[2]]
    np.savez(sys.argv[3], **run(torch.device("cuda", 0)))
"""


@pytest.mark.gpu
def test_reduce_launch_form_gives_the_one_launch_bits(cuda, tmp_path):
    scope: dict = {}
    exec(compile(CASES, "cases", "exec"), scope)
    mine = scope["run"](cuda)
    script = tmp_path / "child.py"
    script.write_text(CHILD)
    npz = tmp_path / "reduce.npz"
    env = dict(os.environ, PK_SPLITK_IN_L2="0")
    print("child: PK_SPLITK_IN_L2=0, GEMV M=1 / skinny M=8, 32 / decode attention", flush=True)
    subprocess.run([sys.executable, str(script), str(ROOT), str(ROOT / "pico-kernels_amd"), str(npz)],
                   env=env, check=True, timeout=100)
    theirs = np.load(npz, allow_pickle=False)
    for name in ("gemv", "skinny8", "skinny32", "decode"):
        assert int(mine[name + "_launches"]) == 1, name      # this device passed the probe
        assert int(theirs[name + "_launches"]) == 2, name    # the reduce-launch form ran
        assert np.array_equal(mine[name], theirs[name]), name
