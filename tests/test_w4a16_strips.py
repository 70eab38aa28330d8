"""W4A16 decode GEMV on the strip layout (pk_w4a16_gemm_strips): each 16-column strip's K
rows contiguous, one workgroup per strip adding the whole of K in LDS -- one launch, no split-K
partials (the work of gemm_int4.py:21-55 at M = 1, which the reference splits over K with
gemm_splitk.py:26-80). The layout is a byte permutation of pack_int4_n's bytes with each nibble
biased by 8 (checked on the CPU against its definition); through the C ABI the GEMV must match the float64 oracle within
the W4A16 bar (relative Frobenius error <= 1e-3) at the headline and every Llama-3-8B layer at
M = 1, M = 1..8, every group size the layout takes, the per-tensor mode, bias, output dtypes
and strided activations, and repeat bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _pk
import oracle


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


# ---- CPU: the layout ----------------------------------------------------------------------
@pytest.mark.parametrize("K,N", [(128, 16), (256, 48), (1024, 512)])
def test_strip_layout_is_the_stated_permutation(K, N):
    words = torch.randint(-2**31, 2**31 - 1, (K, N // 8), generator=_gen(K + N),
                          dtype=torch.int64).to(torch.int32)
    st = _pk.strip_weights(words)
    assert st.shape == words.shape and st.dtype == torch.int32
    src = words.view(torch.uint8).numpy()          # (K, N/2) pack_int4_n bytes
    dst = st.contiguous().view(torch.uint8).numpy().reshape(-1)
    rng = np.random.default_rng(0)
    for _ in range(400):
        k, c = int(rng.integers(K)), int(rng.integers(N // 2))
        b, rs, g, e = k // 128, (k % 128) // 32, (k % 32) // 8, k % 8
        s, cps, h = c // 8, (c % 8) // 2, c % 2
        pos = ((((s * (K // 128) + b) * 4 + g) * 4 + rs) * 4 + cps) * 16 + 8 * h + e
        assert dst[pos] == src[k, c] ^ 0x88, (k, c)       # both nibbles biased by 8
    assert torch.equal(_pk.unstrip_weights(st), words)
    sc = torch.randn(K // 32, N, generator=_gen(1)).half()
    ss = _pk.strip_scales(sc)
    assert torch.equal(ss.view(N // 16, K // 32, 16)[3 % (N // 16), 2], sc[2, 16 * (3 % (N // 16)):][:16])
    assert torch.equal(_pk.unstrip_scales(ss), sc)


def test_strips_ok_rules():
    assert _pk.strips_ok(4096, 11008, 128) and _pk.strips_ok(14336, 4096, 128)
    assert _pk.strips_ok(4096, 4096, 0) and _pk.strips_ok(4096, 4096, 32)
    assert _pk.strips_ok(4096, 4096, 64) and _pk.strips_ok(4096, 4096, 256)
    assert not _pk.strips_ok(4096, 4104, 128)      # N % 16
    assert not _pk.strips_ok(4160, 4096, 64)       # K % 128
    assert not _pk.strips_ok(4096, 4096, 96)       # neither divides 128 nor a multiple of it
    assert not _pk.strips_ok(4096, 4096, 16)       # not a multiple of 32


def test_strips_plan_rule():
    """Two strips per workgroup with at least 32 blocks of K: for 5..8 rows on layers of
    320..512 strips (U = 2) or more than 768 (U = 1); for 2..4 rows on layers of more than 768
    strips and at most 64 blocks (U as for one strip). Eight waves at most with two strips."""
    for M in range(1, 9):
        for N, K in [(6144, 4096), (4096, 4096), (14336, 4096), (11008, 4096), (4096, 14336),
                     (8192, 2048), (5120, 4096), (8192, 8192), (12304, 4096), (13824, 5120),
                     (14336, 8192), (14336, 14336), (28672, 4096)]:
            ns, u, nw = _pk.w4a16_strips_plan(M, N, K)
            strips, kb = N // 16, K // 128
            want = 1
            if M > 4 and kb >= 32 and (320 <= strips <= 512 or strips > 768):
                want = 2
            if 2 <= M <= 4 and 32 <= kb <= 64 and strips > 768:
                want = 2
            assert ns == want, (M, N, K, ns)
            if ns == 2:
                assert nw <= 8, (M, N, K, nw)
                if M > 4:
                    assert u == (2 if strips <= 512 else 1), (M, N, K, u)
                else:
                    assert (u, nw) == (4, 8), (M, N, K, u, nw)
            elif M > 4:
                assert u == 2 and nw <= 8
    assert _pk.w4a16_strips_plan(8, 6144, 4096) == (2, 2, 8)
    assert _pk.w4a16_strips_plan(2, 14336, 4096) == (2, 4, 8)
    try:  # a fixed U of 8 (the measurement hook) keeps one strip per workgroup
        _pk.w4a16_strips_config(8)
        assert _pk.w4a16_strips_plan(2, 14336, 4096)[:2] == (1, 8)
        assert _pk.w4a16_strips_plan(8, 14336, 4096)[:2] == (2, 1)
    finally:
        _pk.w4a16_strips_config(0)
    with pytest.raises(_pk.PicoKernelsError):
        _pk.w4a16_strips_plan(9, 6144, 4096)


def test_strips_rejects_bad_arguments_without_a_gpu():
    f = _pk.lib().pk_w4a16_gemm_strips
    p = 1 << 20  # never dereferenced: every call fails its checks first
    args = dict(a=p, lda=4096, q=p, s=p, g=128, scale=1.0, bias=None, bd=1, c=p, cd=1, ldc=4096,
                M=1, N=4096, K=4096)

    def call(**kw):
        d = {**args, **kw}
        return f(d["a"], d["lda"], d["q"], d["s"], d["g"], d["scale"], d["bias"], d["bd"],
                 d["c"], d["cd"], d["ldc"], d["M"], d["N"], d["K"], None)

    assert call(M=9) == _pk.PK_EINVAL and b"1..8 rows" in _pk.lib().pk_last_error()
    assert call(M=0) == _pk.PK_EINVAL
    assert call(N=4104) == _pk.PK_EINVAL
    assert call(K=4160, lda=4160) == _pk.PK_EINVAL
    assert call(g=96) == _pk.PK_EINVAL
    assert call(a=p + 8) == _pk.PK_EINVAL
    assert call(q=p + 4) == _pk.PK_EINVAL
    assert call(lda=4100) == _pk.PK_EINVAL
    assert call(cd=7) == _pk.PK_EINVAL
    assert _pk.lib().pk_w4a16_strips_config(3) == _pk.PK_EINVAL


# ---- GPU: parity ----------------------------------------------------------------------------
def _case(M, K, N, G, seed):
    a = torch.randn(M, K, generator=_gen(seed)).half()
    w = (torch.randn(K, N, generator=_gen(seed + 1)) * 0.02).half()
    if G:
        codes, _, s16 = oracle.rtn_group_codes(w.numpy(), 4, G)
    else:
        codes = torch.randint(-8, 8, (K, N), generator=_gen(seed + 2), dtype=torch.int8).numpy()
        s16 = None
    words = torch.from_numpy(oracle.pack_int4_n(codes).view(np.int32).copy())
    return a, codes, s16, words


def _run(a, words, s16, G, cuda, out_dtype=torch.float32, scale=1.0, bias=None):
    qs = _pk.strip_weights(words).to(cuda)
    ss = None if s16 is None else _pk.strip_scales(torch.from_numpy(s16)).to(cuda)
    return _pk.w4a16_gemm_strips(a.to(cuda), qs, ss, G, scale, out_dtype,
                                 bias=None if bias is None else bias.to(cuda))


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", [(4096, 11008), (4096, 6144), (4096, 4096), (4096, 14336),
                                 (14336, 4096)])
def test_strips_m1_headline_and_llama_layers(K, N, cuda):
    a, codes, s16, words = _case(1, K, N, 128, K + N)
    y = _run(a, words, s16, 128, cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4   # exact products; MFMA and fp32 summation
    y2 = _run(a, words, s16, 128, cuda)
    assert torch.equal(y, y2)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("K,N", [(4096, 6144), (11008, 4096), (1024, 512), (128, 16), (14336, 1024)])
def test_strips_rows(M, K, N, cuda):
    a, codes, s16, words = _case(M, K, N, 128, 3 * M + K + N)
    y = _run(a, words, s16, 128, cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4, (M, K, N)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [2, 3, 4])
@pytest.mark.parametrize("K,N,G", [(4096, 12304, 128), (8192, 12304, 64)])
def test_strips_two_strips_staged_rows(M, K, N, G, cuda):
    """Two to four rows with two strips per workgroup (activations staged per wave in LDS and
    used for both strips; 769 strips, so the last pair holds one) against the oracle."""
    assert _pk.w4a16_strips_plan(M, N, K)[0] == 2
    a, codes, s16, words = _case(M, K, N, G, 13 * M + K)
    y = _run(a, words, s16, G, cuda)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4, (M, K, N)
    assert torch.equal(y, _run(a, words, s16, G, cuda))


@pytest.mark.gpu
@pytest.mark.parametrize("M", [5, 8])
@pytest.mark.parametrize("K,N,G,plan", [
    (4096, 5136, 128, (2, 2)),   # 321 strips: the last pair holds one strip
    (5120, 6144, 64, (2, 2)),    # 40 blocks: a partial last round; groups of 64
    (4096, 12304, 128, (2, 1)),  # 769 strips, odd
    (4096, 14336, 0, (2, 1)),    # per-tensor mode
])
def test_strips_two_strips_per_workgroup(M, K, N, G, plan, cuda):
    """The 5..8-row kernel with two strips per workgroup (one activation load for both)
    against the oracle, and repeatable bit for bit."""
    assert _pk.w4a16_strips_plan(M, N, K)[:2] == plan
    a, codes, s16, words = _case(M, K, N, G, 11 * M + N)
    y = _run(a, words, s16, G, cuda, scale=0.5 if G == 0 else 1.0)
    if G:
        ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    else:
        ref = oracle.int4_gemm_ref(a.numpy(), codes, 0.5)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4, (M, K, N)
    assert torch.equal(y, _run(a, words, s16, G, cuda, scale=0.5 if G == 0 else 1.0))


@pytest.mark.gpu
def test_strips_two_strips_bias_bf16_and_views(cuda):
    """Two strips per workgroup with a bias, bf16 output into a wider view and strided
    activations: nothing is written past the view."""
    M, K, N = 7, 4096, 6144
    assert _pk.w4a16_strips_plan(M, N, K)[0] == 2
    a, codes, s16, words = _case(M, K, N, 128, 123)
    bias = torch.randn(N, generator=_gen(124)).half()
    big = torch.zeros(M, K + 64, dtype=torch.float16)
    big[:, 32:32 + K] = a
    av = big.to(cuda)[:, 32:32 + K]
    qs = _pk.strip_weights(words).to(cuda)
    ss = _pk.strip_scales(torch.from_numpy(s16)).to(cuda)
    out = torch.full((M, N + 16), 7.0, dtype=torch.bfloat16, device=cuda)
    _pk.w4a16_gemm_strips(av, qs, ss, 128, 1.0, torch.bfloat16, out=out[:, :N], bias=bias.to(cuda))
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128) + bias.float().numpy()
    assert oracle.rel_fro(out[:, :N].float().cpu().numpy(), ref) <= 8e-3
    assert bool((out[:, N:] == 7.0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("G", [0, 32, 64, 256, 512, 384])
@pytest.mark.parametrize("M", [1, 6])
def test_strips_group_sizes(G, M, cuda):
    K, N = (3072, 1024) if G == 384 else (4096, 1024)
    a, codes, s16, words = _case(M, K, N, G, G + M)
    y = _run(a, words, s16, G, cuda, scale=0.5 if G == 0 else 1.0)
    if G:
        ref = oracle.w4a16_ref(a.numpy(), codes, s16, G)
    else:
        ref = oracle.int4_gemm_ref(a.numpy(), codes, 0.5)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias_dtype", [None, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [3, 7])  # the staged four-row kernel and the eight-row one
def test_strips_bias_and_dtypes(M, out_dtype, bias_dtype, cuda):
    K, N = 2048, 768
    a, codes, s16, words = _case(M, K, N, 128, 77 + M)
    bias = None if bias_dtype is None else torch.randn(N, generator=_gen(78)).to(bias_dtype)
    y = _run(a, words, s16, 128, cuda, out_dtype=out_dtype, bias=bias)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    if bias is not None:
        ref = ref + bias.float().numpy()
    assert y.dtype == out_dtype
    tol = {torch.float32: 1e-4, torch.float16: 1e-3, torch.bfloat16: 8e-3}[out_dtype]
    assert oracle.rel_fro(y.float().cpu().numpy(), ref) <= tol


@pytest.mark.gpu
@pytest.mark.parametrize("M", [4, 8])  # staged activations; per-lane loads (eight rows)
def test_strips_strided_activations_and_output_view(M, cuda):
    K, N = 4096, 2048
    a, codes, s16, words = _case(M, K, N, 128, 91)
    big = torch.zeros(M, K + 64, dtype=torch.float16)
    big[:, 32:32 + K] = a
    av = big.to(cuda)[:, 32:32 + K]                 # lda = K + 64, 64-byte offset
    qs = _pk.strip_weights(words).to(cuda)
    ss = _pk.strip_scales(torch.from_numpy(s16)).to(cuda)
    out = torch.full((M, N + 16), 7.0, dtype=torch.float32, device=cuda)
    _pk.w4a16_gemm_strips(av, qs, ss, 128, 1.0, torch.float32, out=out[:, :N])
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    assert oracle.rel_fro(out[:, :N].cpu().numpy(), ref) <= 1e-4
    assert bool((out[:, N:] == 7.0).all())          # nothing written past the view


@pytest.mark.gpu
@pytest.mark.parametrize("u", [2, 4, 8])
def test_strips_blocks_per_wave_agree(u, cuda):
    """Every blocks-per-wave choice (one round or several, 16 waves at most) gives the
    oracle's result."""
    M, K, N = 2, 14336, 1024
    a, codes, s16, words = _case(M, K, N, 128, 5)
    ref = oracle.w4a16_ref(a.numpy(), codes, s16, 128)
    try:
        _pk.w4a16_strips_config(u)
        y = _run(a, words, s16, 128, cuda)
    finally:
        _pk.w4a16_strips_config(0)
    assert oracle.rel_fro(y.cpu().numpy(), ref) <= 1e-4


# ---- QuantLinear's decode copy ----------------------------------------------------------------
def test_quant_linear_decode_copy_on_cpu():
    """The strip copy is derived from the codes and scales, outside the state dict, rebuilt on
    load; decode_layout=False keeps one copy (CPU: no kernel runs)."""
    import quant_linear as ql

    q = ql.QuantLinear(256, 512, bias=False, group_size=128)
    assert q.decode and q.qstrips is not None and q.sstrips is not None
    g = torch.Generator().manual_seed(9)
    words = torch.randint(-2**31, 2**31 - 1, (256, 64), generator=g, dtype=torch.int64).to(torch.int32)
    q.set_codes(words)
    q.scales.copy_(torch.rand(2, 512, generator=g).half())
    q._refresh()
    assert torch.equal(_pk.unstrip_weights(q.qstrips), words)
    assert torch.equal(_pk.unstrip_scales(q.sstrips), q.scales)
    sd = q.state_dict()
    assert set(sd) == {"qweight", "scales"}
    r = ql.QuantLinear(256, 512, bias=False, group_size=128)
    r.load_state_dict(sd)
    assert torch.equal(r.qstrips, q.qstrips) and torch.equal(r.sstrips, q.sstrips)
    one = ql.QuantLinear(256, 512, bias=False, group_size=128, decode_layout=False)
    assert not one.decode and one.qstrips is None
    assert not ql.QuantLinear(256, 520, group_size=128).decode        # out % 16
    assert ql.QuantLinear(256, 512, scheme="per_input").sstrips is None  # scales in activations


@pytest.mark.gpu
@pytest.mark.parametrize("scheme", ["group", "per_input"])
@pytest.mark.parametrize("M", [1, 2, 4, 5, 8])
def test_quant_linear_decode_rows_match_blocks(scheme, M, cuda):
    """Up to its decode_rows QuantLinear runs the strip copy: it agrees with the same layer
    without the copy (block layout) within the W4A16 bar; above that both run the same kernel
    bit for bit."""
    from torch import nn

    import quant_linear as ql

    lin = nn.Linear(1024, 768, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(768, 1024, generator=_gen(M)) * 0.02)
        lin.bias.copy_(torch.randn(768, generator=_gen(M + 1)) * 0.1)
    lin = lin.to(cuda)
    if scheme == "group":
        a = ql.QuantLinear.from_linear(lin, 128)
    else:
        a = ql.QuantLinear.from_linear(lin, method="rtn")
    b = ql.QuantLinear(1024, 768, True, a.group_size or 128, cuda, scheme=scheme, decode_layout=False)
    b.load_state_dict(a.state_dict())
    assert a.decode and not b.decode
    x = torch.randn(M, 1024, generator=_gen(M + 2)).half().to(cuda)
    ya, yb = a(x), b(x)
    if M <= a.decode_rows:
        rel = (torch.linalg.norm(ya.float() - yb.float()) / torch.linalg.norm(yb.float())).item()
        assert rel <= 1e-3, rel
    else:
        assert torch.equal(ya, yb)


@pytest.mark.gpu
def test_quant_linear_prepared_call_follows_its_buffers(cuda):
    """The decode fast path's prepared call is rebuilt whenever the strip copy is not the
    module's own buffer any more: after set_codes + _refresh, after .to(), and in a deep copy
    whose codes are then changed."""
    import copy

    from torch import nn

    import quant_linear as ql

    lin = nn.Linear(512, 256, bias=True).to(cuda)
    q = ql.QuantLinear.from_linear(lin, 128)
    x = torch.randn(1, 512, device=cuda, dtype=torch.float16)
    y0 = q(x)
    twin = copy.deepcopy(q)
    twin.set_codes(torch.zeros_like(twin.codes()))   # all-zero codes: output = bias (to the
    twin._refresh()                                  # rounding of the biased-code offset)
    yt = twin(x).float()
    assert torch.allclose(yt, twin.bias.float().expand(1, -1), atol=1e-3, rtol=0)
    assert not torch.allclose(yt, y0.float(), atol=1e-3, rtol=0)
    assert torch.equal(q(x), y0)                     # the original is untouched
    q2 = q.to(cuda)
    assert torch.equal(q2(x), y0)


@pytest.mark.gpu
def test_prepared_strips_handle(cuda):
    """pk_w4a16_strips_prepare / _run give the bits of pk_w4a16_gemm_strips for every row count;
    a bad fixed argument makes prepare return NULL with the reason; activations or outputs of
    the wrong dtype, device or shape raise; reassigning a QuantLinear's bias rebuilds its
    prepared call."""
    from torch import nn

    import quant_linear as ql

    K, N = 2048, 1024
    a, codes, s16, words = _case(8, K, N, 128, 41)
    qs = _pk.strip_weights(words).to(cuda)
    ss = _pk.strip_scales(torch.from_numpy(s16)).to(cuda)
    bias = torch.randn(N, generator=_gen(42)).half().to(cuda)
    ag = a.to(cuda)
    call = _pk.PreparedStrips(qs, ss, 128, 0.5, torch.float32, bias)
    via_ctypes = _pk.PreparedStrips(qs, ss, 128, 0.5, torch.float32, bias)
    via_ctypes.run = _pk.lib().pk_w4a16_strips_run  # the entry without the CPython module
    for M in range(1, 9):
        ref = _pk.w4a16_gemm_strips(ag[:M], qs, ss, 128, 0.5, torch.float32, bias=bias)
        assert torch.equal(call(ag[:M]), ref), M
        assert torch.equal(via_ctypes(ag[:M]), ref), M
    with pytest.raises(_pk.PicoKernelsError, match="group_size"):
        _pk.PreparedStrips(qs, ss, 96, 1.0, torch.float16)
    # activations or an output the prepared call cannot take raise before any launch
    for bad in (ag[:2].float(), ag[:2].cpu(), ag[:2, : K // 2]):
        with pytest.raises(ValueError, match="fp16"):
            call(bad)
    for bad_out in (torch.empty((2, N), dtype=torch.float16, device=cuda),
                    torch.empty((3, N), dtype=torch.float32, device=cuda),
                    torch.empty((N, 2), dtype=torch.float32, device=cuda).t()):
        with pytest.raises(ValueError, match="out must be"):
            call(ag[:2], bad_out)
    lin = nn.Linear(K, N).to(cuda)
    q = ql.QuantLinear.from_linear(lin, 128)
    x = ag[:1].contiguous()
    y0 = q(x)
    q.bias = q.bias + 1.0
    assert torch.allclose(q(x).float(), y0.float() + 1.0, atol=2e-3, rtol=0)
