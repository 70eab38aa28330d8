"""W4A16 parity on the GPU: the drop-in gemm_int4 API and the group-128 / split-K path.

Inputs come from seeded CPU generators (vendor-independent), results are compared with the
CPU oracle:
  * quantize / pack: bit for bit (golden vectors from the reference's own functions);
  * matmuls: relative Frobenius error vs the dequantize + fp32 matmul closed form
    (tests/test_gemm_int4.py:26 of the reference), bar 1e-3 as the path requires;
  * split-K: the same result for every split (within fp32 reassociation) and bitwise
    identical output on repeated runs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import gemm_int4
import oracle

pytestmark = pytest.mark.gpu

W4A16_TOL = 1e-3  # max relative Frobenius error vs dequant + fp32 matmul


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _weights(K: int, N: int, seed: int, std: float = 0.02) -> torch.Tensor:
    return (torch.randn(K, N, generator=_gen(seed)) * std).half()


def _acts(M: int, K: int, seed: int) -> torch.Tensor:
    return torch.randn(M, K, generator=_gen(seed)).half()


def _group_case(M, K, N, seed, cuda, std=0.02, G=128):
    a = _acts(M, K, seed)
    w = _weights(K, N, seed + 1, std)
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), G)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    return a, w, qw, sc, codes, s16


# ---------------------------------------------------------------------------------------
# the reference's own tests, with CPU-seeded inputs
# ---------------------------------------------------------------------------------------
def test_int4_gemm_correctness(cuda):
    a = _acts(128, 256, 0)
    w = torch.randn(256, 512, generator=_gen(1)).half()
    w_q, scale = gemm_int4.quantize_int4(w.to(cuda))
    w_packed = gemm_int4.pack_int4_n(w_q)
    c = gemm_int4.int4_gemm(a.to(cuda), w_packed, scale)
    assert c.dtype == torch.float32 and c.shape == (128, 512)
    ref = a.float() @ (w_q.cpu().float() * scale)
    assert torch.allclose(c.cpu(), ref, atol=1e-1, rtol=1e-2)
    # decompression is exact, only the fp32 summation order differs
    assert oracle.rel_fro(c.cpu().numpy(), ref.numpy()) < 1e-5


def test_pack_roundtrip(cuda):
    q = torch.randint(-8, 8, (256, 256), generator=_gen(1), dtype=torch.int8)  # includes +7
    packed = gemm_int4.pack_int4_n(q.to(cuda))
    assert packed.shape == (256, 128) and packed.dtype == torch.uint8
    assert torch.equal(gemm_int4.unpack_int4_n(packed).cpu(), q)
    assert np.array_equal(packed.cpu().numpy(), oracle.pack_int4_n(q.numpy()))


def test_pack_shape_and_host_tensors(cuda):
    q = torch.randint(-8, 8, (256, 512), generator=_gen(2), dtype=torch.int8)
    packed = gemm_int4.pack_int4_n(q)  # host tensor in, host tensor out (staged via GPU)
    assert packed.shape == (256, 256) and packed.dtype == torch.uint8 and not packed.is_cuda
    assert np.array_equal(packed.numpy(), oracle.pack_int4_n(q.numpy()))


# ---------------------------------------------------------------------------------------
# bit-exact quantization against the reference's golden vectors
# ---------------------------------------------------------------------------------------
def test_quantize_int4_golden(golden, cuda):
    arrays, meta = golden
    for name in ("qi4_f16_n01", "qi4_f16_n002", "qi4_f32", "qi4_f32_ties"):
        w = torch.from_numpy(arrays[name + "_in"]).to(cuda)
        q, scale = gemm_int4.quantize_int4(w)
        assert scale == meta["cases"][name]["scale"], name
        assert np.array_equal(q.cpu().numpy(), arrays[name + "_codes"]), name


def test_pack_golden(golden, cuda):
    arrays, _ = golden
    out = gemm_int4.pack_int4_n(torch.from_numpy(arrays["pack_in"]).to(cuda))
    assert np.array_equal(out.cpu().numpy(), arrays["pack_out"])


def test_group_quant_matches_oracle(golden, cuda):
    arrays, _ = golden
    for name in ("rtn_f16_b4_g128",):
        w = arrays[name + "_in"]
        qw, sc = gemm_int4.quantize_int4_group(torch.from_numpy(w).to(cuda), 128)
        codes, _, s16 = oracle.rtn_group_codes(w, 4, 128)
        assert np.array_equal(qw.cpu().numpy().view(np.uint8), oracle.pack_int4_n(codes))
        assert np.array_equal(sc.cpu().numpy().view(np.uint16), s16.view(np.uint16))
    # a larger N(0, 0.02) weight, also fp32 input
    w = torch.randn(1024, 512, generator=_gen(3)) * 0.02
    for wt in (w, w.half()):
        qw, sc = gemm_int4.quantize_int4_group(wt.to(cuda), 128)
        codes, _, s16 = oracle.rtn_group_codes(wt.numpy(), 4, 128)
        assert np.array_equal(qw.cpu().numpy().view(np.uint8), oracle.pack_int4_n(codes))
        assert np.array_equal(sc.cpu().numpy(), s16)


@pytest.mark.parametrize("K,N", [(4096, 11008), (14336, 4096)])
def test_group_quant_bitwise_at_full_size(K, N, cuda):
    """The GPU's packed codes and fp16 scales at the headline GEMV's and the down
    projection's sizes are the oracle's bit for bit, so the full-size matmul parity tests
    (which hand the oracle its own codes) compare the same weights."""
    w = (torch.randn(K, N, generator=_gen(40 + K % 13)) * 0.02).half()
    qw, sc = gemm_int4.quantize_int4_group(w.to(cuda), 128)
    codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, 128)
    assert np.array_equal(qw.cpu().numpy().view(np.uint8), oracle.pack_int4_n(codes))
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), s16.view(np.uint16))


# ---------------------------------------------------------------------------------------
# W4A16 matmul parity
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16, 17, 32, 33, 64, 100, 128, 256, 300])
def test_w4a16_shapes(M, cuda):
    K, N = 1024, 264 * 2  # N not a multiple of the 128/256-column tiles
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 10 + M, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err <= W4A16_TOL, f"M={M}: rel err {err:.3e}"
    if M <= 4:  # skinny path: exact products, fp32 scale -> much tighter
        assert err <= 1e-4, f"M={M}: rel err {err:.3e}"


@pytest.mark.parametrize("M,K,N", [(128, 192, 528), (300, 320, 256), (600, 448, 784), (256, 64, 256)])
def test_w4a16_odd_k_tile_counts(M, K, N, cuda):
    """Odd numbers of 64-row K tiles end the MFMA kernels' two-stage loop on a lone tile; its
    accumulators must be complete before the epilogue reads them (group 64 so K can be 192)."""
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 5 * M + K, cuda, G=64)
    for out_dtype in (torch.float32, torch.float16):
        out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 64, out_dtype=out_dtype)
        ref = oracle.w4a16_ref(a.numpy(), codes, s16, 64)
        err = oracle.rel_fro(out.float().cpu().numpy(), ref)
        assert err <= (W4A16_TOL if out_dtype == torch.float32 else 2e-3), (M, K, N, out_dtype, err)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_w4a16_output_dtypes(out_dtype, cuda):
    a, w, qw, sc, codes, s16 = _group_case(64, 512, 256, 7, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    tol = {torch.float32: W4A16_TOL, torch.float16: 2e-3, torch.bfloat16: 1e-2}[out_dtype]
    assert oracle.rel_fro(out.float().cpu().numpy(), ref) <= tol


def test_decode_gemv_splitk_sweep_full_size(cuda):
    """The decode GEMV configuration: M=1, K=4096, N=11008, group 128, split-K in {1,2,4,8,16}."""
    M, K, N = 1, 4096, 11008
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 100, cuda)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    outs = {}
    for s in (1, 2, 4, 8, 16):
        assert _pk.w4a16_plan(M, N, K, 128, s) == (_pk.KERNEL_GEMV, s)
        o1 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        o2 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        assert torch.equal(o1, o2), f"split {s}: not bitwise reproducible"
        err = oracle.rel_fro(o1.cpu().numpy(), ref)
        assert err <= 1e-4, f"split {s}: rel err {err:.3e}"
        outs[s] = o1.cpu().numpy()
    for s in (2, 4, 8, 16):  # splits differ only by fp32 reassociation
        assert oracle.rel_fro(outs[s], outs[1]) < 1e-5
    auto = gemm_int4.w4a16_gemm(ag, qw, sc, 128, out_dtype=torch.float16)
    assert oracle.rel_fro(auto.float().cpu().numpy(), ref) <= 2e-3


def test_prefill_gemm_full_size(cuda):
    """The prefill configuration: M=2048, K=4096, N=4096 (MFMA path), fp16 output."""
    M, K, N = 2048, 4096, 4096
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 200, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    err = oracle.rel_fro(out.cpu().numpy(), ref)
    assert err <= W4A16_TOL, f"rel err {err:.3e}"


@pytest.mark.parametrize("M", [1, 8, 32, 128])
@pytest.mark.parametrize("K,N", [(4096, 6144), (4096, 4096), (4096, 14336), (14336, 4096)])
def test_llama3_sweep_shapes(M, K, N, cuda):
    """The Llama-3-8B linear layers (qkv, o, gate/up, down) at M in {1,8,32,128}."""
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 300 + M + K % 7 + N % 11, cuda)
    out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, out_dtype=torch.float32)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(out.cpu().numpy(), ref) <= W4A16_TOL


def test_gemm_split_k_deterministic_and_consistent(cuda):
    """The GEMM that dequantises B into LDS (N % 256 != 0 keeps the packed-B kernel out; M = 256
    is above the register-dequant kernel's range) at every split: bitwise reproducible, and
    splits agree up to fp32 reassociation."""
    M, K, N = 256, 4096, 1152
    assert all(_pk.w4a16_plan(M, N, K, 128, s) == (_pk.KERNEL_GEMM, s) for s in (1, 2, 4, 8))
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 400, cuda)
    ag = a.to(cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    base = None
    for s in (1, 2, 4, 8):
        o1 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        o2 = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=s, out_dtype=torch.float32)
        assert torch.equal(o1, o2)
        assert oracle.rel_fro(o1.cpu().numpy(), ref) <= W4A16_TOL
        base = o1 if base is None else base
        assert oracle.rel_fro(o1.cpu().numpy(), base.cpu().numpy()) < 1e-6


def test_workspace_counters_reset_between_calls(cuda):
    """Alternate shapes and splits on one workspace: every call must still be right."""
    cases = [_group_case(1, 2048, 2048, 500, cuda), _group_case(2, 4096, 1024, 501, cuda),
             _group_case(64, 1024, 2048, 502, cuda)]
    for rep in range(3):
        for (a, w, qw, sc, codes, s16), s in zip(cases, (8, 16, 4)):
            out = gemm_int4.w4a16_gemm(a.to(cuda), qw, sc, 128, split_k=s, out_dtype=torch.float32)
            assert oracle.rel_fro(out.cpu().numpy(), oracle.w4a16_ref(a.numpy(), codes, s16, 128)) <= W4A16_TOL


def test_linearity_in_activations(cuda):
    """Size-independent property: W(a1 + a2) == W a1 + W a2 (up to fp32 rounding)."""
    M, K, N = 4, 4096, 11008
    _, _, qw, sc, _, _ = _group_case(1, K, N, 600, cuda)
    a1 = (torch.randn(M, K, generator=_gen(601)) * 0.5).half()
    a2 = (torch.randn(M, K, generator=_gen(602)) * 0.5).half()
    s = (a1.float() + a2.float()).half()
    y1 = gemm_int4.w4a16_gemm(a1.to(cuda), qw, sc, out_dtype=torch.float32)
    y2 = gemm_int4.w4a16_gemm(a2.to(cuda), qw, sc, out_dtype=torch.float32)
    ys = gemm_int4.w4a16_gemm(s.to(cuda), qw, sc, out_dtype=torch.float32)
    # the sum was rounded to fp16, so compare against W applied to that rounding error too
    err = oracle.rel_fro(ys.cpu().numpy(), (y1 + y2).cpu().numpy())
    assert err < 2e-3


def test_int4_gemm_any_m_no_oob(cuda):
    """The reference kernel is mask-free and needs M % 64 == 0; any M must work here."""
    w = torch.randn(256, 256, generator=_gen(7)).half()
    w_q, scale = gemm_int4.quantize_int4(w.to(cuda))
    wp = gemm_int4.pack_int4_n(w_q)
    for M in (1, 3, 16, 65):
        a = _acts(M, 256, 8 + M)
        c = gemm_int4.int4_gemm(a.to(cuda), wp, scale)
        ref = oracle.int4_gemm_ref(a.numpy(), w_q.cpu().numpy(), scale)
        assert oracle.rel_fro(c.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("M", [1, 8, 100, 256])
def test_int4_gemm_bf16_activations(M, cuda):
    """bf16 activations (the reference wrapper admits them, gemm_int4.py:78): values within
    fp16's range convert exactly, so the result is bitwise the fp16 call on the same values
    (edge values 0, 2^-17 and -60000 included), and within 1e-5 of the float64 product of the
    bf16 values and the codes."""
    w = torch.randn(512, 512, generator=_gen(9)).half()
    w_q, scale = gemm_int4.quantize_int4(w.to(cuda))
    wp = gemm_int4.pack_int4_n(w_q)
    a = (torch.randn(M, 512, generator=_gen(20 + M)) * 3.0).to(torch.bfloat16)
    got = gemm_int4.int4_gemm(a.to(cuda), wp, scale)
    assert got.dtype == torch.float32
    assert torch.equal(got, gemm_int4.int4_gemm(a.to(cuda).half(), wp, scale))
    ref = (a.double().numpy() @ w_q.cpu().double().numpy()) * scale
    assert oracle.rel_fro(got.cpu().numpy(), ref) < 1e-5
    edge = a.clone()
    edge[0, :4] = torch.tensor([0.0, 2.0 ** -17, -60000.0, 1.5e-3], dtype=torch.bfloat16)
    assert torch.equal(gemm_int4.int4_gemm(edge.to(cuda), wp, scale),
                       gemm_int4.int4_gemm(edge.to(cuda).half(), wp, scale))


@pytest.mark.parametrize("M,split", [(1, 8), (3, 16), (64, 4), (128, 4)])
def test_partials_then_reduce_equals_fused(M, split, cuda):
    """The two phases of split-K (per-slice partials, ordered reduce) reproduce the fused
    call bit for bit, and each slice's partial is that K range's product."""
    K, N = 2048, 1024
    a, w, qw, sc, codes, s16 = _group_case(M, K, N, 700 + M, cuda)
    ag = a.to(cuda)
    parts = _pk.w4a16_gemm_partials(ag, qw, sc, 128, split)
    assert tuple(parts.shape) == (split, M, N)
    out = torch.empty((M, N), dtype=torch.float32, device=cuda)
    _pk.splitk_reduce(parts, 1.0, out)
    fused = gemm_int4.w4a16_gemm(ag, qw, sc, 128, split_k=split, out_dtype=torch.float32)
    assert torch.equal(out, fused)
    ks = K // split
    for s in (0, split - 1):
        sl = slice(s * ks, (s + 1) * ks)
        ref = oracle.w4a16_ref(a.numpy()[:, sl], codes[sl], s16[s * ks // 128:(s + 1) * ks // 128], 128)
        assert oracle.rel_fro(parts[s].cpu().numpy(), ref) <= W4A16_TOL


@pytest.mark.parametrize("S", [3, 33, 56, 70])
def test_splitk_reduce_any_slice_count(S, cuda):
    """Slice counts without a dedicated kernel (K = 14336 gives 56 slices of 256 rows) keep the
    fixed order: bit-equal to a sequential fp32 sum over slices 0..S-1."""
    M, N = 2, 1032
    g = _gen(800 + S)
    parts = torch.randn(S, M, N, generator=g)
    parts[:, 0, :8] = -0.0  # all slices -0.0: the sum must stay -0.0 (it starts from slice 0)
    acc = parts[0].numpy().copy()
    for s in range(1, S):
        acc = (acc + parts[s].numpy()).astype(np.float32)
    acc = (acc * np.float32(0.5)).astype(np.float32)
    out = torch.empty((M, N), dtype=torch.float32, device=cuda)
    _pk.splitk_reduce(parts.to(cuda), 0.5, out)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), acc.view(np.uint32))
