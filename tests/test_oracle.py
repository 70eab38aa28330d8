"""Pin the CPU oracle (CPU only, no GPU).

The oracle is what the HIP kernels are checked against, so it is itself checked against:
  * the golden vectors written by running the reference's own functions (bit for bit);
  * torch's float8_e4m3fn cast, exhaustively over fp16 and on fp32 samples (the library
    routine the reference's gemm_fp8.quantize calls);
  * closed forms, invariants of the reference's tests, and brute force on tiny shapes;
  * planted mistakes: plausible wrong variants of the oracle must fail the same checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import quant as oq


# ---------------------------------------------------------------------------------------
# e4m3 codec
# ---------------------------------------------------------------------------------------
def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_exhaustive_fp16_matches_torch():
    x16 = np.arange(65536, dtype=np.uint16).view(np.float16)
    ours = oracle.e4m3_from_f32(x16.astype(np.float32))
    ref = _torch_e4m3(x16.astype(np.float32))
    assert np.array_equal(ours, ref), f"{np.count_nonzero(ours != ref)} mismatches"
    # torch's fp16 -> e4m3 path agrees with widening first
    assert np.array_equal(_torch_e4m3(x16), ref)


def test_e4m3_fp32_samples_and_boundaries_match_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    edges = np.array([448.0, 464.0, np.nextafter(464.0, 0), np.nextafter(464.0, 1000), 480.0,
                      2.0**-6, 2.0**-9, 2.0**-10, 3 * 2.0**-11, np.inf, -np.inf, np.nan, 0.0,
                      -0.0, 1e-30, 240.0, 232.0, 0.0009765625], dtype=np.float32)
    x = np.concatenate([x, edges, -edges])
    assert np.array_equal(oracle.e4m3_from_f32(x), _torch_e4m3(x))


def test_e4m3_decode_table():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = oracle.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert ours[0x7E] == 448.0 and ours[0x08] == 2.0**-6 and ours[0x01] == 2.0**-9
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])


def test_e4m3_roundtrip_is_identity_on_the_grid():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    back = oracle.e4m3_from_f32(oracle.e4m3_to_f32(codes))
    # +0 and -0 are distinct codes and must survive
    assert np.array_equal(back, codes)


# ---------------------------------------------------------------------------------------
# golden vectors (reference functions run in the build container)
# ---------------------------------------------------------------------------------------
def test_quantize_int4_matches_reference(golden):
    arrays, meta = golden
    for name in ("qi4_f16_n01", "qi4_f16_n002", "qi4_f32", "qi4_f32_ties"):
        codes, scale = oracle.quantize_int4(arrays[name + "_in"])
        assert scale == meta["cases"][name]["scale"], name
        assert np.array_equal(codes, arrays[name + "_codes"]), name


def test_pack_matches_reference(golden):
    arrays, _ = golden
    assert np.array_equal(oracle.pack_int4_n(arrays["pack_in"]), arrays["pack_out"])
    assert np.array_equal(oracle.unpack_int4_n(arrays["pack_out"]), arrays["pack_in"])


def test_fp8_quantize_matches_reference(golden):
    arrays, meta = golden
    for name in ("fp8_f16_n01", "fp8_f16_wide", "fp8_f32"):
        b, scale = oracle.fp8_quantize(arrays[name + "_in"])
        assert scale == meta["cases"][name]["scale"], name
        assert np.array_equal(b, arrays[name + "_out"]), name


def test_quantize_col_matches_reference(golden):
    arrays, meta = golden
    for name, case in meta["cases"].items():
        if case["fn"] != "quantize.quantize_col":
            continue
        out = oracle.quantize_col(arrays[name + "_in"], case["bits"], case["group_size"])
        ref = arrays[name + "_out"]
        assert out.dtype == ref.dtype, name
        assert np.array_equal(out.view(np.uint8), ref.view(np.uint8)), name


def test_rtn_layer_matches_reference(golden):
    arrays, meta = golden
    for name, case in meta["cases"].items():
        if case["fn"] != "quantize.rtn_layer":
            continue
        out = oracle.rtn_layer(arrays[name + "_in"], case["bits"], case["group_size"])
        ref = arrays[name + "_out"]
        assert out.dtype == ref.dtype, name
        assert np.array_equal(out.view(np.uint8), ref.view(np.uint8)), name


def test_group_codes_reproduce_rtn_layer(golden):
    """The packed format's (codes, fp32 scales) rebuild rtn_layer's output exactly."""
    arrays, _ = golden
    for name in ("rtn_f16_b4_g128", "rtn_f16_b4_g128_tail"):
        w = arrays[name + "_in"]
        codes, s32, s16 = oracle.rtn_group_codes(w, 4, 128)
        assert codes.min() >= -7 and codes.max() <= 7
        rebuilt = (codes.astype(np.float32) * np.repeat(s32, 128, axis=0)[: w.shape[0]]).astype(np.float16)
        # integer codes carry no sign of zero; rtn_layer returns -0.0 for small negatives
        assert np.array_equal(rebuilt, arrays[name + "_out"]), name
        assert np.array_equal(s16, s32.astype(np.float16))


def test_gptq_layer_matches_reference(golden):
    arrays, meta = golden
    W, X = arrays["gptq_w"], arrays["gptq_x"]
    for name, case in meta["cases"].items():
        if case["fn"] != "quantize.gptq_layer":
            continue
        out = oracle.gptq_layer(W, X, case["bits"], act_order=case["act_order"],
                                group_size=case["group_size"])
        ref = arrays[name + "_out"]
        # fp32 linear algebra (inverse, rank-1 updates) in a different library: tolerance,
        # and at most a handful of codes may land on the other side of a rounding tie.
        close = np.isclose(out, ref, atol=1e-4, rtol=1e-4)
        assert close.mean() > 0.995, f"{name}: {(~close).sum()} of {close.size} differ"


# ---------------------------------------------------------------------------------------
# closed forms and invariants
# ---------------------------------------------------------------------------------------
def test_pack_roundtrip_every_code():
    q = np.tile(np.arange(-8, 8, dtype=np.int8), (3, 4))  # all 16 codes incl. +7
    p = oracle.pack_int4_n(q)
    assert p.shape == (3, 32) and p.dtype == np.uint8
    assert np.array_equal(oracle.unpack_int4_n(p), q)
    # closed form of one byte: low nibble = even column
    assert p[0, 0] == ((-8 & 0xF) | ((-7 & 0xF) << 4))


def test_gptq_act_order_is_permutation_consistent():
    """The reference's own invariant (tests/test_quantize.py:15-32)."""
    rng = np.random.default_rng(0)
    W = rng.standard_normal((64, 32)).astype(np.float32)
    X = rng.standard_normal((16, 32)).astype(np.float32)
    X[:, :8] *= 4.0
    w_ao = oracle.gptq_layer(W, X, 4, act_order=True)
    H = X.T @ X / X.shape[0]
    order = np.argsort(-np.diag(H), kind="stable")
    w_manual = oracle.gptq_layer(W[:, order], X[:, order], 4, act_order=False)
    w_manual = w_manual[:, np.argsort(order, kind="stable")]
    assert np.allclose(w_ao, w_manual, atol=1e-5)


def test_gptq_beats_rtn():
    """The reference's own invariant (tests/test_quantize.py:45-53)."""
    rng = np.random.default_rng(2)
    W = (rng.standard_normal((128, 256)) * 0.1).astype(np.float32)
    X = rng.standard_normal((64, 256)).astype(np.float32)

    def mse(wq):
        return float(((X @ wq.T - X @ W.T) ** 2).mean())

    assert mse(oracle.gptq_layer(W, X, 4)) < mse(oracle.rtn_layer(W, 4))


def test_gptq_with_diagonal_hessian_is_rtn():
    """Orthogonal activation columns make H diagonal: every error-feedback ratio is zero and
    GPTQ reduces to round-to-nearest of each column."""
    rng = np.random.default_rng(3)
    W = rng.standard_normal((48, 16)).astype(np.float32)
    X = np.zeros((32, 16), dtype=np.float32)
    X[np.arange(16), np.arange(16)] = rng.uniform(0.5, 2.0, 16).astype(np.float32)
    for gs in (None, 16):
        assert np.array_equal(oracle.gptq_layer(W, X, 4, group_size=gs), oracle.rtn_layer(W, 4, gs))


def test_quantize_col_group_matches_manual():
    """The reference's manual check (tests/test_quantize.py:35-42), exact here."""
    rng = np.random.default_rng(1)
    w = rng.standard_normal(64).astype(np.float32)
    q = oracle.quantize_col(w, 4, group_size=16)
    for g in range(0, 64, 16):
        scale = np.float32(np.abs(w[g:g + 16]).max()) / np.float32(7.0)
        expected = np.clip(np.rint(w[g:g + 16] / scale), -7, 7) * scale
        assert np.array_equal(q[g:g + 16], expected.astype(np.float32))


def test_w4a16_ref_brute_force():
    rng = np.random.default_rng(4)
    M, K, N, G = 3, 64, 16, 32
    a = rng.standard_normal((M, K)).astype(np.float16)
    codes = rng.integers(-8, 8, (K, N)).astype(np.int8)
    scales = (rng.uniform(0.001, 0.01, (K // G, N))).astype(np.float16)
    ref = oracle.w4a16_ref(a, codes, scales, G)
    brute = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            brute[m, n] = sum(float(a[m, k]) * int(codes[k, n]) * float(scales[k // G, n]) for k in range(K))
    assert np.allclose(ref, brute, rtol=1e-5, atol=1e-6)


def test_fp8_and_splitk_refs_brute_force():
    rng = np.random.default_rng(5)
    a8 = rng.integers(0, 256, (4, 32)).astype(np.uint8)
    b8 = rng.integers(0, 256, (32, 5)).astype(np.uint8)
    a8[(a8 & 0x7F) == 0x7F] = 0
    b8[(b8 & 0x7F) == 0x7F] = 0
    out = oracle.fp8_gemm_ref(a8, 2.0, b8, 0.25)
    da, db = oracle.e4m3_to_f32(a8).astype(np.float64), oracle.e4m3_to_f32(b8).astype(np.float64)
    assert np.allclose(out, (da @ db) * 2.0, rtol=1e-6)
    a = rng.standard_normal((8, 64)).astype(np.float32)
    b = rng.standard_normal((64, 8)).astype(np.float32)
    assert np.allclose(oracle.splitk_ref(a, b, 4), a.astype(np.float64) @ b, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------------------
# planted mistakes: plausible wrong restatements must fail the golden checks
# ---------------------------------------------------------------------------------------
def test_planted_reciprocal_division_is_caught(golden):
    """Multiplying by 1/scale instead of dividing (what torch does on GPU tensors): on fp32
    inputs one to three ulps around (k + 1/2) * scale (the reference's own codes for them are
    the qi4_f32_ties fixture) the two round to different codes, so the golden check catches
    this restatement."""
    arrays, meta = golden
    name = "qi4_f32_ties"
    w = arrays[name + "_in"]
    scale = meta["cases"][name]["scale"]
    inv = np.float32(1.0) / np.float32(scale)
    wrong = np.clip(np.rint(w.astype(np.float32) * inv), -8, 7).astype(np.int8)
    assert np.count_nonzero(wrong != arrays[name + "_codes"]) > 0
    codes, _ = oracle.quantize_int4(w)
    assert np.array_equal(codes, arrays[name + "_codes"])


def test_reciprocal_division_same_codes_for_fp16_inputs():
    """Why the fp16 fixtures cannot tell the two apart: an fp16 input's quotient is rounded to
    fp16 before the round-to-integer, which absorbs the one-ulp fp32 difference. Checked on
    every finite fp16 value up to the maximum, for several maxima."""
    u = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    for mx in np.float16([0.7, 1.0, 1.4501545, 3.1251962, 9.487]):
        h = u[np.isfinite(u) & (np.abs(u) <= mx)]
        w = np.concatenate([h, np.array([mx], dtype=np.float16)]).reshape(1, -1)
        codes, scale = oracle.quantize_int4(w)
        inv = np.float32(1.0) / np.float32(scale)
        t = (w.astype(np.float32) * inv).astype(np.float16).astype(np.float32)
        assert np.array_equal(np.clip(np.rint(t), -8, 7).astype(np.int8), codes)


def test_planted_missing_fp16_rounding_is_caught(golden):
    """Skipping the fp16 rounding of x*scale before the e4m3 cast changes some bytes."""
    arrays, meta = golden
    name = "fp8_f16_n01"
    x = arrays[name + "_in"]
    scale = meta["cases"][name]["scale"]
    wrong = oracle.e4m3_from_f32(x.astype(np.float32) * np.float32(scale))
    assert np.count_nonzero(wrong != arrays[name + "_out"]) > 0


def test_planted_saturating_cast_is_caught():
    """A saturating encoder (448 for overflow) disagrees with torch at 470."""
    x = np.array([470.0, -470.0], dtype=np.float32)
    assert list(_torch_e4m3(x)) == [0x7F, 0xFF]
    assert list(oracle.e4m3_from_f32(x)) == [0x7F, 0xFF]


def test_decode_attention_ref_closed_forms():
    """Pins decode_attention_ref (flash_decoding.eager_decode, flash_decoding.py:126-133) by
    what softmax-weighted averaging fixes, so a wrong scale placement, a missing max shift,
    an unnormalised sum or a transposed operand fails."""
    rng = np.random.default_rng(0)
    B, H, N, D = 2, 3, 37, 16
    q = rng.standard_normal((B, H, 1, D)).astype(np.float16)
    k = rng.standard_normal((B, H, N, D)).astype(np.float16)
    # constant V rows: the output is that row whatever the scores
    row = rng.standard_normal((B, H, 1, D))
    np.testing.assert_allclose(oracle.decode_attention_ref(q, k, np.repeat(row, N, axis=2)),
                               row[:, :, 0, :], rtol=1e-12, atol=1e-12)
    # identical keys: equal weights, the mean of the V rows
    v = rng.standard_normal((B, H, N, D))
    kk = np.repeat(k[:, :, :1, :], N, axis=2)
    np.testing.assert_allclose(oracle.decode_attention_ref(q, kk, v), v.mean(axis=2), rtol=1e-12)
    # one cached row: that value row
    np.testing.assert_allclose(oracle.decode_attention_ref(q, k[:, :, :1], v[:, :, :1]),
                               v[:, :, 0], rtol=1e-12)
    # one dominant score (huge logits, no overflow thanks to the max shift): its value row
    k2 = np.zeros((1, 1, 5, 4))
    k2[0, 0, 3] = 1.0
    q2 = np.full((1, 1, 1, 4), 400.0)
    v2 = rng.standard_normal((1, 1, 5, 4))
    np.testing.assert_allclose(oracle.decode_attention_ref(q2, k2, v2), v2[:, :, 3], rtol=1e-12)
    # the scale multiplies the logits: scale 0 gives the plain mean of V
    np.testing.assert_allclose(oracle.decode_attention_ref(q, k, v, sm_scale=0.0),
                               v.mean(axis=2), rtol=1e-12)
