"""Write the golden vectors under tests/golden/ by running the reference's own CPU functions.

Run in the build container only (it needs the read-only reference checkout):

    python tests/golden/make_golden.py --reference /root/reference

The reference's quantization helpers are pure torch and run on CPU tensors. Their results
depend on torch's rounding chain (fp16 intermediates, true fp32 division, half-to-even
rounding, non-saturating e4m3 cast), which no closed form pins bit for bit, so these
fixtures are the bit-exact anchor for the oracle and the HIP kernels. Inputs are drawn from
seeded CPU generators and stored next to the outputs; nothing of the reference is copied,
only its input/output values.

Functions covered (reference file:line):
  gemm_int4.quantize_int4  gemm_int4.py:58-62     gemm_int4.pack_int4_n   gemm_int4.py:65-72
  gemm_fp8.quantize        gemm_fp8.py:89-95      quantize.quantize_col   quantize.py:42-60
  quantize.rtn_layer       quantize.py:63-68      quantize.gptq_layer     quantize.py:71-115
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy().copy()
    return t.numpy().copy()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import gemm_fp8  # noqa: E402  (reference module, CPU helpers only)
    import gemm_int4  # noqa: E402
    import quantize  # noqa: E402

    arrays: dict[str, np.ndarray] = {}
    meta: dict[str, object] = {"torch": torch.__version__, "cases": {}}

    # --- gemm_int4.quantize_int4 ---------------------------------------------------------
    cases = {
        "qi4_f16_n01": (torch.randn(256, 256, generator=_gen(0)).half()),
        "qi4_f16_n002": (torch.randn(512, 256, generator=_gen(1)) * 0.02).half(),
        "qi4_f32": torch.randn(128, 64, generator=_gen(2)),
    }
    # fp32 values one to three ulps around (k + 1/2) * scale: w / scale and w * (1 / scale)
    # round to different codes for some of them, so this case tells true division from a
    # reciprocal multiply (fp16 inputs cannot: their quotient is rounded to fp16 first)
    mx = np.float32(1.4501545429229736)
    step = np.float32(float(mx) / 7.0)

    def nudge(v, d):
        for _ in range(abs(d)):
            v = np.nextafter(v, np.float32(np.inf) if d > 0 else np.float32(-np.inf))
        return v

    ties = [nudge(np.float32((k + 0.5) * float(step)), d) for k in range(-7, 7) for d in range(-3, 4)]
    cases["qi4_f32_ties"] = torch.from_numpy(np.array(ties + [mx], dtype=np.float32).reshape(9, 11))
    for name, w in cases.items():
        q, scale = gemm_int4.quantize_int4(w)
        arrays[name + "_in"] = _np(w)
        arrays[name + "_codes"] = _np(q)
        meta["cases"][name] = {"fn": "gemm_int4.quantize_int4", "scale": scale}

    # --- gemm_int4.pack_int4_n (all 16 codes incl. +7) -------------------------------------
    q = torch.randint(-8, 8, (64, 128), generator=_gen(3), dtype=torch.int8)
    arrays["pack_in"] = _np(q)
    arrays["pack_out"] = _np(gemm_int4.pack_int4_n(q))
    meta["cases"]["pack"] = {"fn": "gemm_int4.pack_int4_n"}

    # --- gemm_fp8.quantize -------------------------------------------------------------------
    cases = {
        "fp8_f16_n01": torch.randn(256, 256, generator=_gen(4)).half(),
        "fp8_f16_wide": (torch.randn(128, 128, generator=_gen(5)) * 3.0).half(),
        "fp8_f32": torch.randn(64, 128, generator=_gen(6)),
    }
    for name, x in cases.items():
        x8, scale = gemm_fp8.quantize(x)
        arrays[name + "_in"] = _np(x)
        arrays[name + "_out"] = _np(x8)
        meta["cases"][name] = {"fn": "gemm_fp8.quantize", "scale": scale}

    # --- quantize.quantize_col ---------------------------------------------------------------
    qc_cases = [
        ("qc_f32_b4_g128", torch.randn(300, generator=_gen(7)), 4, 128),
        ("qc_f32_b3_g16", torch.randn(64, generator=_gen(8)), 3, 16),
        ("qc_f32_b8_none", torch.randn(200, generator=_gen(9)), 8, None),
        ("qc_f16_b4_g64", torch.randn(200, generator=_gen(10)).half(), 4, 64),
        ("qc_f16_b2_none", (torch.randn(96, generator=_gen(11)) * 0.02).half(), 2, None),
    ]
    for name, w, bits, gs in qc_cases:
        arrays[name + "_in"] = _np(w)
        arrays[name + "_out"] = _np(quantize.quantize_col(w, bits, gs))
        meta["cases"][name] = {"fn": "quantize.quantize_col", "bits": bits, "group_size": gs}

    # --- quantize.rtn_layer ------------------------------------------------------------------
    rtn_cases = [
        ("rtn_f16_b4_g128", (torch.randn(512, 96, generator=_gen(12)) * 0.02).half(), 4, 128),
        ("rtn_f32_b3_none", torch.randn(256, 64, generator=_gen(13)), 3, None),
        ("rtn_f16_b4_g128_tail", (torch.randn(300, 40, generator=_gen(14)) * 0.02).half(), 4, 128),
        ("rtn_f32_b8_g32", torch.randn(128, 48, generator=_gen(15)), 8, 32),
    ]
    for name, w, bits, gs in rtn_cases:
        arrays[name + "_in"] = _np(w)
        arrays[name + "_out"] = _np(quantize.rtn_layer(w, bits, gs))
        meta["cases"][name] = {"fn": "quantize.rtn_layer", "bits": bits, "group_size": gs}

    # --- quantize.gptq_layer -----------------------------------------------------------------
    W = torch.randn(64, 32, generator=_gen(16))
    X = torch.randn(16, 32, generator=_gen(17))
    X[:, :8] *= 4.0
    arrays["gptq_w"] = _np(W)
    arrays["gptq_x"] = _np(X)
    for ao in (True, False):
        for gs in (None, 16):
            name = f"gptq_ao{int(ao)}_g{gs or 0}"
            arrays[name + "_out"] = _np(quantize.gptq_layer(W, X, 4, act_order=ao, group_size=gs))
            meta["cases"][name] = {"fn": "quantize.gptq_layer", "bits": 4, "act_order": ao,
                                   "group_size": gs}

    np.savez_compressed(OUT / "reference_vectors.npz", **arrays)
    (OUT / "reference_vectors.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")
    total = sum(a.nbytes for a in arrays.values())
    print(f"wrote {len(arrays)} arrays ({total / 1024:.0f} KiB raw) to {OUT}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
