"""numpy restatement of the reference's quantization arithmetic -- TEST INFRASTRUCTURE ONLY.

Never imported by the product modules. Every function names the reference file:line whose
arithmetic it restates; the torch rounding chain is spelled out explicitly:
  * fp16 tensor op with an fp32 "opmath": compute in float32, round to fp16 (RNE);
  * true IEEE float32 division (torch does not substitute a reciprocal on CPU tensors);
  * torch.round = round half to even (np.rint);
  * torch.clamp propagates NaN;
  * float8_e4m3fn cast = round to nearest even, NaN (0x7f) on overflow (no saturation).
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0  # torch.finfo(torch.float8_e4m3fn).max, gemm_fp8.py:24


# ---------------------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------------------
def _clamp_nan(x: np.ndarray, lo: float, hi: float) -> np.ndarray:
    """torch.clamp semantics: NaN stays NaN."""
    with np.errstate(invalid="ignore"):
        return np.where(x < lo, np.float32(lo), np.where(x > hi, np.float32(hi), x)).astype(np.float32)


def _round16(v: np.ndarray) -> np.ndarray:
    """Round float32 values to fp16 (RNE) and widen back: one fp16 tensor-op result."""
    with np.errstate(over="ignore"):
        return v.astype(np.float16).astype(np.float32)


def _f32(x: np.ndarray) -> np.ndarray:
    return np.asarray(x).astype(np.float32)


def _codes_to_int8(r: np.ndarray) -> np.ndarray:
    return np.where(np.isnan(r), 0, r).astype(np.int8)


# ---------------------------------------------------------------------------------------
# OCP fp8 e4m3 ("e4m3fn"): independent table-based implementation
# ---------------------------------------------------------------------------------------
def _e4m3_table() -> np.ndarray:
    """Values of the 256 e4m3fn codes from the OCP definition (NaN for S.1111.111)."""
    v = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 15 and m == 7:
            v[code] = np.nan
        elif e == 0:
            v[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            v[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return v


_E4M3_VALUES = _e4m3_table()
# Non-negative finite codes 0x00..0x7e are increasing in value: a sorted grid.
_POS_GRID = _E4M3_VALUES[:0x7F]


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    """Decode e4m3fn bytes (exact in float32)."""
    return _E4M3_VALUES[np.asarray(b, dtype=np.uint8)].astype(np.float32)


def e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    """Encode float32 values to e4m3fn bytes: nearest grid point, ties to the even code,
    magnitudes that round above 448 (anything above 464), Inf and NaN -> 0x7f | sign.

    Implemented as a search over the 127 non-negative grid values, independently of the
    bit-manipulation encoder used by the HIP kernels.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = np.signbit(x).astype(np.uint8) << 7
    with np.errstate(invalid="ignore"):
        a = np.abs(x.astype(np.float64))
    hi = np.searchsorted(_POS_GRID, a, side="left")  # first grid value >= a
    hi_c = np.clip(hi, 0, 0x7E)
    lo_c = np.clip(hi - 1, 0, 0x7E)
    d_hi = _POS_GRID[hi_c] - a
    d_lo = a - _POS_GRID[lo_c]
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((hi_c & 1) == 0))
    code = np.where(pick_hi, hi_c, lo_c).astype(np.uint8)
    code = np.where(a == _POS_GRID[hi_c], hi_c, code).astype(np.uint8)  # exact hits
    nan = np.isnan(a) | (a > 464.0)
    code = np.where(nan, np.uint8(0x7F), code).astype(np.uint8)
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------------------------------
# gemm_int4.py
# ---------------------------------------------------------------------------------------
def quantize_int4(w: np.ndarray) -> tuple[np.ndarray, float]:
    """gemm_int4.quantize_int4 (gemm_int4.py:58-62) on an fp16 or fp32 array.

    scale = max|w| / 7.0 in Python double; codes = int8(clamp(round(T(w / f32(scale))),
    -8, 7)) where T rounds the fp32 quotient to w's dtype. NaN codes become 0.
    """
    w = np.asarray(w)
    absmax = float(np.max(np.abs(w.astype(np.float32))))
    scale = absmax / 7.0
    with np.errstate(divide="ignore", invalid="ignore"):
        t = w.astype(np.float32) / np.float32(scale)
    if w.dtype == np.float16:
        t = _round16(t)
    r = _clamp_nan(np.rint(t), -8.0, 7.0)
    return _codes_to_int8(r), scale


def pack_int4_n(w_q: np.ndarray) -> np.ndarray:
    """gemm_int4.pack_int4_n (gemm_int4.py:65-72): byte j of a row = col 2j | col 2j+1 << 4."""
    q = np.asarray(w_q).astype(np.int32)
    K, N = q.shape
    assert N % 2 == 0
    lo = q[:, 0::2] & 0xF
    hi = q[:, 1::2] & 0xF
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_int4_n(packed: np.ndarray) -> np.ndarray:
    """Inverse of pack_int4_n: the in-kernel unpack of gemm_int4.py:44-49 (sign-extend,
    interleave low/high nibble)."""
    p = np.asarray(packed, dtype=np.uint8).astype(np.int32)
    lo = p & 0xF
    hi = p >> 4
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty((p.shape[0], 2 * p.shape[1]), dtype=np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


# ---------------------------------------------------------------------------------------
# quantize.py
# ---------------------------------------------------------------------------------------
def _group_scales(absmax: np.ndarray, qmax: int, half: bool) -> np.ndarray:
    """scale = absmax.clamp_min(1e-12) / qmax (quantize.py:53, 58) in fp32 or fp16 math."""
    floor = np.float32(np.float16(1e-12)) if half else np.float32(1e-12)
    a = np.where(absmax < floor, floor, absmax).astype(np.float32)
    s = a / np.float32(qmax)
    return _round16(s) if half else s.astype(np.float32)


def _rtn_groups(w32: np.ndarray, bits: int, group: int, half: bool):
    """Quantize a (L, C) float32 array column-wise in groups of `group` rows.

    Returns (codes float32 (NaN allowed), scales (ngroups, C) float32, fake float32)."""
    qmax = 2 ** (bits - 1) - 1
    L, C = w32.shape
    ng = -(-L // group)
    codes = np.empty_like(w32)
    fake = np.empty_like(w32)
    scales = np.empty((ng, C), dtype=np.float32)
    for g in range(ng):
        sl = slice(g * group, min((g + 1) * group, L))
        blk = w32[sl]
        am = np.max(np.abs(blk), axis=0)
        s = _group_scales(am, qmax, half)
        with np.errstate(divide="ignore", invalid="ignore"):
            t = blk / s
        if half:
            t = _round16(t)
        r = _clamp_nan(np.rint(t), -qmax, qmax)
        f = r * s
        if half:
            f = _round16(f)
        codes[sl], fake[sl], scales[g] = r, f, s
    return codes, scales, fake


def quantize_col(w: np.ndarray, bits: int, group_size: int | None = None) -> np.ndarray:
    """quantize.quantize_col (quantize.py:42-60) for a 1-D fp32 or fp16 array.

    fp32 input: all arithmetic in fp32. fp16 input: every tensor op rounds to fp16 and the
    1e-12 floor itself rounds to 0 in fp16."""
    w = np.asarray(w)
    if bits >= 16:
        return w
    half = w.dtype == np.float16
    L = w.shape[0]
    group = group_size if group_size else L
    _, _, fake = _rtn_groups(w.astype(np.float32).reshape(L, 1), bits, group, half)
    return fake.reshape(L).astype(w.dtype)


def rtn_layer(w: np.ndarray, bits: int, group_size: int | None = None) -> np.ndarray:
    """quantize.rtn_layer (quantize.py:63-68): widen to fp32, quantize every column (groups
    along dim 0), cast back to w's dtype."""
    w = np.asarray(w)
    if bits >= 16:
        return w.copy()
    L = w.shape[0]
    group = group_size if group_size else L
    _, _, fake = _rtn_groups(w.astype(np.float32), bits, group, False)
    return fake.astype(w.dtype)


def rtn_group_codes(w_kn: np.ndarray, bits: int = 4, group_size: int = 128):
    """The packed group format's integer content: rtn_layer's arithmetic (quantize.py:53-59)
    with the integer codes and scales kept. Returns (codes int8 (K, N), scales fp32
    (ceil(K/G), N), scales rounded to fp16)."""
    w = np.asarray(w_kn)
    codes, scales, _ = _rtn_groups(w.astype(np.float32), bits, group_size, False)
    return _codes_to_int8(codes), scales, scales.astype(np.float16)


def gptq_sweep(wq: np.ndarray, ratio: np.ndarray, bits: int,
               group_size: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """The column loop of quantize.gptq_layer (quantize.py:104-110) in fp32: for each column j
    in order, quantize it (quantize_col), then subtract outer(err, ratio[j, j+1:]) from every
    later column. ratio[j, c] = H_inv[j, c] / H_inv[j, j] above the diagonal. Returns the
    swept matrix and the per-column errors."""
    wq = np.array(wq, dtype=np.float32)
    errs = np.zeros_like(wq)
    for j in range(wq.shape[1]):                                     # :104-110
        col = wq[:, j].copy()
        q = quantize_col(col, bits, group_size)
        err = col - q
        wq[:, j + 1:] -= np.outer(err, ratio[j, j + 1:]).astype(np.float32)
        wq[:, j] = q
        errs[:, j] = err
    return wq, errs


def gptq_layer(w: np.ndarray, x: np.ndarray, bits: int, damp: float = 0.01,
               act_order: bool = True, group_size: int | None = None) -> np.ndarray:
    """quantize.gptq_layer (quantize.py:71-115), sequential column sweep, fp32.

    For small shapes only (O(in^2 * out) Python loop)."""
    w = np.asarray(w)
    if bits >= 16:
        return w.copy()
    W = w.astype(np.float32)
    X = np.asarray(x).astype(np.float32)
    out_dim, in_dim = W.shape
    n = X.shape[0]
    H = (X.T @ X) / np.float32(n)                                    # :88
    act_mag = np.diag(H).copy()                                       # :89
    H = H + np.float32(damp) * act_mag.mean(dtype=np.float32) * np.eye(in_dim, dtype=np.float32)
    H_inv = np.linalg.inv(H).astype(np.float32)                       # :92
    wq = W.copy()
    order = None
    if act_order:                                                     # :97-100
        order = np.argsort(-act_mag, kind="stable")
        wq = wq[:, order]
        H_inv = H_inv[order][:, order]
    ratio = np.zeros_like(H_inv)
    for j in range(in_dim):
        ratio[j, j + 1:] = H_inv[j, j + 1:] / H_inv[j, j]            # :106
    wq, _ = gptq_sweep(wq, ratio, bits, group_size)
    if order is not None:                                             # :110-111
        wq = wq[:, np.argsort(order, kind="stable")]
    return wq.astype(w.dtype)


# ---------------------------------------------------------------------------------------
# gemm_fp8.py
# ---------------------------------------------------------------------------------------
def fp8_quantize(x: np.ndarray) -> tuple[np.ndarray, float]:
    """gemm_fp8.quantize (gemm_fp8.py:89-95): scale = 448 / max|x| (Python double);
    bytes = e4m3(T(x * f32(scale))) with T = rounding to x's dtype (fp16 or fp32)."""
    x = np.asarray(x)
    scale = E4M3_MAX / float(np.max(np.abs(x.astype(np.float32))))
    y = x.astype(np.float32) * np.float32(scale)
    if x.dtype == np.float16:
        y = _round16(y)
    return e4m3_from_f32(y), scale
