"""Torch-facing wrappers of the C ABI: validate tensors on the host, pass raw device pointers and the
current HIP stream, return or fill caller-visible tensors. Allocation (when an output is not given)
happens here, on the host side of the ABI, never inside the library.

The reference's single custom op is exact::gemv (experiments/speed_fair_kaggle.py:698-702); it is
registered below under the same name with the same contract: (x16 int16 (K,), wT int8 (N, K) row-major,
Mg int64 (N, K/128)) -> int64 (N,), on the reference's own tensors with no repacking.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import ExactError

I8, I16, I32, I64 = torch.int8, torch.int16, torch.int32, torch.int64


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t, dtype, name, numel=None):
    if not isinstance(t, torch.Tensor):
        raise ExactError(f"{name}: expected a tensor")
    if t.device.type != "cuda":
        raise ExactError(f"{name}: expected a GPU tensor, got {t.device}")
    if t.dtype != dtype:
        raise ExactError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ExactError(f"{name}: expected a contiguous tensor")
    if numel is not None and t.numel() < numel:
        raise ExactError(f"{name}: expected at least {numel} elements, got {t.numel()}")
    return t


# ----------------------------------------------------------------------------- packed linears
class PackedLinear:
    """A linear in the packed device layout: wp int8 [Np/64][G][8][64][16], mp int16 [Np/64][G][64].
    Wide group scales (>= 2^15) add a high plane mh of the same layout: M = mh * 2^15 + mp.
    mode 'group': y = shr(t, 28 - s) + b; mode 'channel': M (N,) int64 with the per-row drop rule."""

    def __init__(self, wp, mp, N, K, bias=None, mode="group", M=None, Mbits=None, parts=None, mh=None):
        self.wp, self.mp, self.N, self.K = wp, mp, N, K
        self.mh = mh
        self.G = K // 128
        self.bias, self.mode, self.M, self.Mbits = bias, mode, M, Mbits
        # (name, first output column, width) of each linear fused into this one
        self.parts = [("", 0, N)] if parts is None else parts

    @staticmethod
    def alloc(N, K, device):
        if K % 128:
            raise ExactError(f"K = {K} is not a multiple of 128")
        nb = (N + 63) // 64
        G = K // 128
        wp = torch.empty(nb * G * 8192, dtype=I8, device=device)
        mp = torch.empty(nb * G * 64, dtype=I16, device=device)
        return wp, mp


def synth_linear(wp, mp, N, K, kw, km, m_lo, m_hi, thr_dev, n_off=0, Ntot=None):
    """Generate an (N, K) synthetic linear into rows [n_off, n_off + N) of a packed buffer of Ntot rows."""
    Ntot = N if Ntot is None else Ntot
    _lib.call("exact_synth_linear", ctypes.c_uint64(kw), ctypes.c_uint64(km), m_lo, m_hi, _ptr(thr_dev), _ptr(wp), _ptr(mp),
              N, K, n_off, Ntot, _stream())


def synth_vector(k, lo, hi, n, device):
    out = torch.empty(n, dtype=I64, device=device)
    _lib.call("exact_synth_vector", ctypes.c_uint64(k), lo, hi, _ptr(out), n, _stream())
    return out


def pack_linear(w_kn, m_gn, wp=None, mp=None, n_off=0, Ntot=None):
    """Pack a (K, N) int8 weight and (G, N) int16 scales (device tensors) into rows [n_off, n_off + N)."""
    K, N = w_kn.shape
    _need(w_kn, I8, "w_kn")
    _need(m_gn, I16, "m_gn")
    Ntot = N if Ntot is None else Ntot
    if wp is None:
        wp, mp = PackedLinear.alloc(Ntot, K, w_kn.device)
    _lib.call("exact_pack_linear", _ptr(w_kn), _ptr(m_gn), _ptr(wp), _ptr(mp), N, K, n_off, Ntot, _stream())
    return wp, mp


def pack_scales(m_gn, mp, N, K, n_off=0, Ntot=None):
    """Pack (G, N) int16 values into the scale layout (the high plane of wide scales)."""
    _need(m_gn, I16, "m_gn", (K // 128) * N)
    _lib.call("exact_pack_scales", _ptr(m_gn), _ptr(mp), N, K, n_off, N if Ntot is None else Ntot, _stream())
    return mp


def pack_group_linear(w_kn, M_gn, device, bias=None, parts=None):
    """PackedLinear of a (K, N) int8 weight (host array) with (G, N) non-negative integer group scales of any size
    below 2^30: int16 scales when every M < 2^15, else the two planes M = mh * 2^15 + (M mod 2^15)."""
    M = np.asarray(M_gn, np.int64)
    K, N = np.shape(w_kn)
    if M.shape != (K // 128, N) or K % 128:
        raise ExactError(f"group scales of shape ({K // 128}, {N}) expected, got {M.shape}")
    if M.min() < 0 or M.max() >= 1 << 30:
        raise ExactError("group scales must lie in [0, 2^30)")
    wide = M.max() >= 1 << 15
    wp, mp = pack_linear(np_to_dev(w_kn, I8, device), np_to_dev(M & 0x7FFF if wide else M, I16, device))
    mh = None
    if wide:
        mh = torch.empty_like(mp)
        pack_scales(np_to_dev(M >> 15, I16, device), mh, N, K)
    return PackedLinear(wp, mp, N, K, bias, parts=parts, mh=mh)


# ----------------------------------------------------------------------------- linears
def gemv_g128(x, abits, lin, out=None):
    """t (R, N) int64 = sum_g acc_g * M_g for R <= 15 (abits 15) / 16 (abits 7) rows."""
    return _linear("exact_gemv_g128", x, abits, lin, out)


def gemv_g128_acc(x, abits, lin, out):
    """out (R, N) += sum_g acc_g * M_g (out holds zeros or a running total)."""
    return _linear("exact_gemv_g128_acc", x, abits, lin, out)


def gemv_qrow_acc(xs, part, nparts, abits, lin, out, s_out, K=None, zero=None):
    """out (R, N) += qrow(xs[:, :K], abits) . W in one launch, the row shifts from the producer's slice bit lengths
    part (R, nparts); s_out (R,) int32 receives the shifts. xs: int64 (R, ldx). zero: an int64 tensor the launch
    also clears."""
    R, ldx = xs.shape
    K = lin.K if K is None else K
    if K != lin.K:
        raise ExactError(f"gemv_qrow_acc: K = {K}, linear has K = {lin.K}")
    _need_packed(lin, "gemv_qrow_acc")
    _need(xs, I64, "xs")
    _need(part, I32, "part", R * nparts)
    _need(out, I64, "out", R * lin.N)
    _need(s_out, I32, "s_out", R)
    _lib.call("exact_gemv_g128_qrow_acc", _ptr(xs), ldx, _ptr(part), nparts, abits, _ptr(lin.wp), _ptr(lin.mp), _ptr(lin.mh),
              _ptr(out), _ptr(s_out), R, lin.N, K, _ptr(zero), 0 if zero is None else _need(zero, I64, "zero").numel(),
              _stream())
    return out


SWIGLU_GEMV_ROWS = 4      # rows of one exact_gemv_g128_swiglu launch whose h the quantising down GEMV reads
SWIGLU_GEMV_MAX_ROWS = 8  # rows exact_gemv_g128_swiglu takes
SWIGLU_PART_COLS = 32     # columns per slice bit length of exact_gemv_g128_swiglu
XQ_PARTS_MAX = 1024       # slice bit lengths per row that exact_gemv_g128_qrow_acc takes


def gemv_swiglu(xq, lin, s, silu, h, part, t=None):
    """h (R, I) = SwiGLU of the gate|up totals xq . W (lin: the packed gate|up linear, N = 2I) and part (R, I / 64) = bit
    lengths of max |h| per SWIGLU_PART_COLS columns, in one launch that keeps the totals in registers; t (optional,
    (R, 2I)) receives the totals. The down GEMV quantises h: gemv_qrow_acc(h, part, I // SWIGLU_PART_COLS, ...)."""
    R, K = xq.shape
    I = lin.N // 2
    if K != lin.K or lin.N % 2:
        raise ExactError(f"gemv_swiglu: x has K = {K}, linear is {lin.N} x {lin.K}")
    _need_packed(lin, "gemv_swiglu")
    _lib.call("exact_gemv_g128_swiglu", _ptr(_need(xq, I16, "xq", R * K)), _ptr(lin.wp), _ptr(lin.mp), _ptr(lin.mh),
              _ptr(_need(s, I32, "s", R)), _ptr(silu), _ptr(_need(h, I64, "h", R * I)),
              _ptr(_need(part, I32, "part", R * (I // SWIGLU_PART_COLS))), _ptr(None if t is None else _need(t, I64, "t", R * 2 * I)), R, I,
              K, _stream())
    return h, part


NORM_FUSE_ROWS = 2        # rows of one exact_gemv_g128_norm_acc launch
NORM_FUSE_KMAX = 256 * 24


def norm_gemv_one_block_per_cu(N, K, R=1, cus=0):
    """True when exact_gemv_g128_norm_acc runs its 8-wave blocks, one per CU (rows wider than 1024 whose group-split
    tasks fit one round): then each CU normalises the row once. With more tasks every one of its 4-wave blocks
    normalises the row (at 14B's q|k|v, hundreds of blocks of 5120-wide rows: 5.33 against 4.20 ms a decode step).
    The launch takes at most NORM_FUSE_ROWS rows; the split is the library's own (exact_gemv_g128_norm_acc_blockwaves),
    on `cus` compute units (0: the current device's)."""
    if R > NORM_FUSE_ROWS:
        return False
    return _lib.load().exact_gemv_g128_norm_acc_blockwaves(int(R), int(N), int(K), int(cus)) == 8


def gemv_norm_acc(x_in, res_t, res_s, g, lin, out, s_out, x_out=None, xq_out=None):
    """out (R, N) += qrow(irms(x, g), 15) . W in one launch, with x = x_in + rs(res_t, 28 - res_s) (res_t may be None):
    every block normalises the rows itself; block 0 writes x to x_out (not x_in: the other blocks still read it), the
    row shifts to s_out and, when given, the int16 rows to xq_out."""
    R, K = x_in.shape
    if K != lin.K:
        raise ExactError(f"gemv_norm_acc: x has K = {K}, linear has K = {lin.K}")
    _need_packed(lin, "gemv_norm_acc")
    _need(x_in, I64, "x_in")
    _need(g, I64, "g", K)
    _need(out, I64, "out", R * lin.N)
    _need(s_out, I32, "s_out", R)
    if res_t is not None:
        _need(res_t, I64, "res_t", R * K)
        _need(res_s, I32, "res_s", R)
    if x_out is not None:
        _need(x_out, I64, "x_out", R * K)
    if xq_out is not None:
        _need(xq_out, I16, "xq_out", R * K)
    _lib.call("exact_gemv_g128_norm_acc", _ptr(x_in), _ptr(x_out), _ptr(res_t), _ptr(res_s), _ptr(g), _ptr(lin.wp),
              _ptr(lin.mp), _ptr(lin.mh), _ptr(out), _ptr(s_out), _ptr(xq_out), R, lin.N, K, _stream())
    return out


NORM_SWIGLU_KMAX = 128 * 16   # row width of one exact_gemv_g128_norm_swiglu launch with 4-wave blocks
NORM_SWIGLU_WIDE_KMAX = 128 * 64   # ... and with 8-wave blocks (I a multiple of 128)


def gemv_norm_swiglu(x_in, res_t, res_s, g, lin, s_out, silu, h, part, x_out=None, t=None):
    """The gate|up GEMV of gemv_swiglu on rows that it normalises itself (as gemv_norm_acc): x = x_in + rs(res_t,
    28 - res_s) (res_t may be None), xq = qrow(irms(x, g), 15), h and part = SwiGLU of xq . W and its slice bit lengths,
    in one launch. Block 0 writes x to x_out (not x_in or res_t) and the row shifts to s_out; t (optional, (R, 2I))
    receives the gate|up totals."""
    R, K = x_in.shape
    I = lin.N // 2
    if K != lin.K or lin.N % 2:
        raise ExactError(f"gemv_norm_swiglu: x has K = {K}, linear is {lin.N} x {lin.K}")
    _need_packed(lin, "gemv_norm_swiglu")
    _need(x_in, I64, "x_in")
    _need(g, I64, "g", K)
    _need(s_out, I32, "s_out", R)
    if res_t is not None:
        _need(res_t, I64, "res_t", R * K)
        _need(res_s, I32, "res_s", R)
    if x_out is not None:
        _need(x_out, I64, "x_out", R * K)
    _lib.call("exact_gemv_g128_norm_swiglu", _ptr(x_in), _ptr(x_out), _ptr(res_t), _ptr(res_s), _ptr(g), _ptr(lin.wp),
              _ptr(lin.mp), _ptr(lin.mh), _ptr(s_out), _ptr(silu), _ptr(_need(h, I64, "h", R * I)),
              _ptr(_need(part, I32, "part", R * (I // SWIGLU_PART_COLS))),
              _ptr(None if t is None else _need(t, I64, "t", R * 2 * I)), R, I, K, _stream())
    return h, part


GEMV_CHUNK_ROWS = {15: 15, 7: 16}   # int8 rows: one GEMV row chunk in exact_gemm_g128, the GEMM beyond; int16 rows
                                    # above 15 take exact_gemm_g128_a16 (one GEMV chunk of 16 with colterm, digit rows beyond)
A16_DIGIT_ROWS = 16                 # int16 rows above this many run on the GEMM as digit rows (exact_gemm_g128_a16)
_DIGIT_ROWS = {}                     # device -> int8 workspace of the A16 digit rows


def colterm(lin):
    """sum_g colsum_g * M_g per output column (int64, N): the A16 digit GEMM's 128 * colsum term. One A8 GEMV of
    an all-ones row, cached on the linear."""
    ct = getattr(lin, "_colterm", None)
    if ct is None:
        ones = torch.ones((1, lin.K), dtype=I8, device=lin.wp.device)
        ct = gemv_g128(ones, 7, lin).reshape(-1)
        lin._colterm = ct
    return ct


def gemm_g128(x, abits, lin, out=None, zeroed=False, x8=None):
    """t = x . W for any R; zeroed: out holds zeros, so split paths add into it without a clear launch.
    x8: the digit rows of the int16 x that its producer wrote (used above A16_DIGIT_ROWS rows)."""
    R, K = x.shape
    sfx = "_zeroed" if zeroed and out is not None else ""
    _need_packed(lin, "gemm_g128")
    if x8 is not None and abits == 15 and R > A16_DIGIT_ROWS:
        if K != lin.K:
            raise ExactError(f"exact_gemm_g128_digits: x has K = {K}, linear has K = {lin.K}")
        if out is None:
            out = torch.empty((R, lin.N), dtype=I64, device=x.device)
        _need(out, I64, "out", R * lin.N)
        _lib.call("exact_gemm_g128_digits", _digits(x8, R, K), _ptr(lin.wp), _ptr(lin.mp), _ptr(lin.mh), _ptr(colterm(lin)),
                  _ptr(out), R, lin.N, K, int(bool(sfx)), _stream())
        return out
    if abits != 15 or R <= GEMV_CHUNK_ROWS[15]:
        return _linear("exact_gemm_g128" + sfx, x, abits, lin, out)
    # A16 on the int8 GEMM as interleaved digit rows (exact_gemm_g128_a16)
    if K != lin.K:
        raise ExactError(f"exact_gemm_g128_a16: x has K = {K}, linear has K = {lin.K}")
    _need(x, I16, "x")
    if out is None:
        out = torch.empty((R, lin.N), dtype=I64, device=x.device)
    _need(out, I64, "out", R * lin.N)
    ct = colterm(lin)
    ws = _DIGIT_ROWS.get(x.device)
    if ws is None or ws.numel() < 2 * R * K:
        ws = torch.empty(2 * R * K, dtype=I8, device=x.device)
        _DIGIT_ROWS[x.device] = ws
    _lib.call("exact_gemm_g128_a16" + sfx, _ptr(x), _ptr(lin.wp), _ptr(lin.mp), _ptr(lin.mh), _ptr(ct), _ptr(ws), _ptr(out), R,
              lin.N, K, _stream())
    return out


def linear_t(x, abits, lin, out=None, zeroed=False, x8=None):
    """Dispatch: GEMV for decode-sized R, GEMM otherwise (TLinG, speed_fair_kaggle.py:735-742).
    zeroed: out already holds zeros (left by a clearing consumer), so the GEMV accumulates into it.
    x8: digit rows of x its producer wrote (int16 GEMM rows only)."""
    R = x.shape[0]
    if R <= (15 if abits == 15 else 16):
        if zeroed and out is not None:
            return gemv_g128_acc(x, abits, lin, out)
        return gemv_g128(x, abits, lin, out)
    return gemm_g128(x, abits, lin, out, zeroed=zeroed, x8=x8)


def _need_packed(lin, fn):
    """The packed buffers of lin hold ceil(N/64) * G tiles: wp int8 8192 B, mp (and mh) int16 64 per tile."""
    if lin.K <= 0 or lin.K % 128:
        raise ExactError(f"{fn}: K = {lin.K} is not a positive multiple of 128")
    tiles = ((lin.N + 63) // 64) * (lin.K // 128)
    _need(lin.wp, I8, f"{fn}: packed weights wp", tiles * 8192)
    _need(lin.mp, I16, f"{fn}: packed scales mp", tiles * 64)
    if lin.mh is not None:
        _need(lin.mh, I16, f"{fn}: wide-scale plane mh", tiles * 64)


def _linear(fn, x, abits, lin, out):
    R, K = x.shape
    if K != lin.K:
        raise ExactError(f"{fn}: x has K = {K}, linear has K = {lin.K}")
    _need_packed(lin, fn)
    _need(x, I16 if abits == 15 else I8, "x")
    if out is None:
        out = torch.empty((R, lin.N), dtype=I64, device=x.device)
    _need(out, I64, "out", R * lin.N)
    _lib.call(fn, _ptr(x), abits, _ptr(lin.wp), _ptr(lin.mp), _ptr(lin.mh), _ptr(out), R, lin.N, K, _stream())
    return out


def requant_group(t, s, b=None, out=None):
    R, N = t.shape
    out = torch.empty_like(t) if out is None else out
    _lib.call("exact_requant_group", _ptr(t), _ptr(_need(s, I32, "s", R)), _ptr(b), _ptr(out), R, N, _stream())
    return out


def requant_channel(acc, s, M, Mbits, b=None, out=None):
    R, N = acc.shape
    out = torch.empty_like(acc) if out is None else out
    _lib.call("exact_requant_channel", _ptr(acc), _ptr(_need(s, I32, "s", R)), _ptr(_need(M, I64, "M", N)), int(Mbits),
              _ptr(b), _ptr(out), R, N, _stream())
    return out


# ----------------------------------------------------------------------------- nonlinearities
def qrow(x, bits=15, xq=None, s=None):
    R, K = x.shape
    _need(x, I64, "x")
    xq = torch.empty((R, K), dtype=I16 if bits > 7 else I8, device=x.device) if xq is None else xq
    s = torch.empty(R, dtype=I32, device=x.device) if s is None else s
    _lib.call("exact_qrow", _ptr(x), bits, _ptr(xq), _ptr(s), R, K, _stream())
    return xq, s


def irms(x, g):
    R, D = x.shape
    y = torch.empty_like(_need(x, I64, "x"))
    _lib.call("exact_irms", _ptr(x), _ptr(_need(g, I64, "g", D)), _ptr(y), R, D, _stream())
    return y


def _digits(x8, R, K):
    return None if x8 is None else _ptr(_need(x8, I8, "x8", 2 * R * K))


def rmsnorm_qrow(x, g, bits=15, res_t=None, res_s=None, xq=None, s=None, clear=False, x8=None):
    """x += rs(res_t, 28 - res_s) (in place) when res_t is given; then qrow(irms(x, g), bits).
    clear: leave res_t zeroed for the next accumulating GEMV. x8: (2R, D) int8, also receives xq's digit rows."""
    R, D = x.shape
    _need(x, I64, "x")
    xq = torch.empty((R, D), dtype=I16 if bits > 7 else I8, device=x.device) if xq is None else xq
    s = torch.empty(R, dtype=I32, device=x.device) if s is None else s
    _lib.call("exact_rmsnorm_qrow", _ptr(x), _ptr(res_t), _ptr(res_s), _ptr(_need(g, I64, "g", D)), bits, _ptr(xq), _ptr(s),
              R, D, int(clear), _digits(x8, R, D), _stream())
    return xq, s


QSLICE, LSLICE = 1024, 4096   # row slice lengths of the multi-block row kernels


def swiglu_parts(R, I, device):
    return torch.empty(R * -(-I // QSLICE), dtype=I32, device=device)


def swiglu_part(t, s, silu, h, part, clear=False):
    """h (R, I) = SwiGLU of the gate|up totals and part = bit lengths of max |h| per 1024-column slice, without the
    qrow (the consumer GEMV quantises: gemv_qrow_acc)."""
    R, N2 = t.shape
    I = N2 // 2
    _lib.call("exact_swiglu_qrow", _ptr(_need(t, I64, "t")), _ptr(s), _ptr(silu), 15, None, None,
              _ptr(_need(part, I32, "part", R * -(-I // QSLICE))), R, I, int(clear), _ptr(_need(h, I64, "h", R * I)), None,
              _stream())
    return h, part


def swiglu_qrow(t, s, silu, bits=15, xq=None, sq=None, clear=False, part=None, h=None, x8=None):
    """h: optional (R, I) int64 scratch; with it and clear=False, t is left intact (trace capture).
    x8: (2R, I) int8, also receives xq's digit rows."""
    R, N2 = t.shape
    I = N2 // 2
    xq = torch.empty((R, I), dtype=I16 if bits > 7 else I8, device=t.device) if xq is None else xq
    sq = torch.empty(R, dtype=I32, device=t.device) if sq is None else sq
    part = swiglu_parts(R, I, t.device) if part is None else _need(part, I32, "part", R * -(-I // QSLICE))
    hp = None if h is None else _ptr(_need(h, I64, "h", R * I))
    _lib.call("exact_swiglu_qrow", _ptr(_need(t, I64, "t")), _ptr(s), _ptr(silu), bits, _ptr(xq), _ptr(sq), _ptr(part), R, I,
              int(clear), hp, _digits(x8, R, I), _stream())
    return xq, sq


def quant_rows(src, part, nparts, bits, xq, s, K=None, clear=False, x8=None, zero=None):
    """qrow of src rows (first K columns) given per-slice bit lengths of max |src| part (R, nparts) int32.
    x8: (2R, K) int8, also receives xq's digit rows. zero: an int64 tensor the launch also clears."""
    R, ld = src.shape
    K = ld if K is None else K
    _lib.call("exact_quant_rows", _ptr(_need(src, I64, "src")), ld, _ptr(_need(part, I32, "part", R * nparts)), nparts, bits,
              _ptr(xq), _ptr(_need(s, I32, "s", R)), R, K, int(clear), _digits(x8, R, K),
              _ptr(None if zero is None else _need(zero, I64, "zero")), 0 if zero is None else zero.numel(), _stream())
    return xq, s


def isilu(x, silu):
    y = torch.empty_like(_need(x, I64, "x"))
    _lib.call("exact_isilu", _ptr(x), _ptr(silu), _ptr(y), x.numel(), _stream())
    return y


def isig(x, sig):
    y = torch.empty_like(_need(x, I64, "x"))
    _lib.call("exact_isig", _ptr(x), _ptr(sig), _ptr(y), x.numel(), _stream())
    return y


def isoftmax(sc, expt, n_valid=None):
    R, N = sc.shape
    p = torch.empty_like(_need(sc, I64, "sc"))
    _lib.call("exact_isoftmax", _ptr(sc), _ptr(n_valid), _ptr(expt), _ptr(p), R, N, _stream())
    return p


# ----------------------------------------------------------------------------- attention / plumbing
def qkv_rope_cache(t, s, b, cos, sin, slot, pos, cache, qq, sq, H, KV, hd, clear=False):
    R = t.shape[0]
    kq, sk, v = cache
    Smax = kq.shape[2]
    _lib.call("exact_qkv_rope_cache", _ptr(t), _ptr(s), _ptr(b), _ptr(cos), _ptr(sin), _ptr(slot), _ptr(pos), _ptr(qq),
              _ptr(sq), _ptr(kq), _ptr(sk), _ptr(v), R, H, KV, hd, Smax, int(clear), _stream())


def attention(qq, sq, cache, slot, pos, expt, out, H, KV, hd, inv, obits=None):
    R = qq.shape[0]
    kq, sk, v = cache
    Smax = kq.shape[2]
    if obits is not None:
        _need(obits, I32, "obits", R * H)
    _lib.call("exact_attention", _ptr(qq), _ptr(sq), _ptr(kq), _ptr(sk), _ptr(v), _ptr(slot), _ptr(pos), _ptr(expt),
              _ptr(out), _ptr(obits), R, H, KV, hd, Smax, inv, _stream())
    return out


ATT_SPLIT_MAX = 4   # bit lengths a head that attention_qkv may write (blocks a head's p.V may take)


def attention_qkv(t, s, b, cos_t, sin_t, slot, pos, cache, expt, out, H, KV, hd, inv, obits=None, obn=1):
    """qkv_rope_cache + attention in one launch for rows that each own their (slot, position); t unchanged.
    obits (optional) gets obn entries per head (1, 2 or ATT_SPLIT_MAX; their max is the head's bit length): with obn > 1
    the library may split each head's p.V over obn blocks, one output slice each."""
    R = t.shape[0]
    kq, sk, v = cache
    _need(t, I64, "t", R * (H + 2 * KV) * hd)
    _need(out, I64, "out", R * H * hd)
    if obits is not None:
        _need(obits, I32, "obits", R * H * obn)
    args = (_ptr(t), _ptr(_need(s, I32, "s", R)), _ptr(b), _ptr(cos_t), _ptr(sin_t), _ptr(slot), _ptr(pos), _ptr(kq),
            _ptr(sk), _ptr(v), _ptr(expt), _ptr(out), _ptr(obits))
    if obn == 1:
        _lib.call("exact_attention_qkv", *args, R, H, KV, hd, kq.shape[2], inv, _stream())
    else:
        _lib.call("exact_attention_qkv_split", *args, obn, R, H, KV, hd, kq.shape[2], inv, _stream())
    return out


def prefill_workspace(R, H, KV, hd, nkeys, device):
    """Workspace of attention_prefill for up to R query rows over up to nkeys keys (digit copies of one slot's k
    and v, per-row softmax statistics)."""
    n = _lib.load().exact_attention_prefill_workspace(R, H, KV, hd, nkeys)
    if n < 0:
        raise ExactError(f"attention_prefill: unsupported R={R}, H={H}, KV={KV}, hd={hd}, nkeys={nkeys}")
    return torch.empty(int(n), dtype=I8, device=device)


def attention_prefill(qq, sq, cache, slot, pos, nkeys, expt, out, H, KV, hd, inv, ws, obits=None):
    """attention() for the rows of one sequence (positions increasing, all < nkeys) on the matrix cores."""
    R = qq.shape[0]
    kq, sk, v = cache
    Smax = kq.shape[2]
    if obits is not None:
        _need(obits, I32, "obits", R * H)
    _need(pos, I32, "pos", R)
    _need(ws, I8, "workspace")
    _lib.call("exact_attention_prefill", _ptr(qq), _ptr(sq), _ptr(kq), _ptr(sk), _ptr(v), int(slot), _ptr(pos), _ptr(expt),
              _ptr(out), _ptr(obits), _ptr(ws), ws.numel(), R, H, KV, hd, Smax, nkeys, inv, _stream())
    return out


def embed(ids, table, out):
    R = ids.shape[0]
    V, D = table.shape
    _lib.call("exact_embed", _ptr(_need(ids, I32, "ids")), _ptr(_need(table, I32, "emb")), _ptr(out), R, D, V, _stream())
    return out


def embed_table(lin, V, D):
    emb = torch.empty((V, D), dtype=I32, device=lin.wp.device)
    _lib.call("exact_embed_table", _ptr(lin.wp), _ptr(lin.mp), _ptr(emb), V, D, _stream())
    return emb


def logits_parts(R, N, device):
    return torch.empty(R * -(-N // LSLICE) * 2, dtype=I64, device=device)


def logits_argmax(t, s, lg=None, ids=None, clear=False, part=None):
    R, N = t.shape
    part = logits_parts(R, N, t.device) if part is None else _need(part, I64, "part", R * -(-N // LSLICE) * 2)
    _lib.call("exact_logits_argmax", _ptr(t), _ptr(s), _ptr(lg), _ptr(ids), _ptr(part), R, N, int(clear), _stream())
    return lg, ids


def temp_num(temp):
    """Temperature as the integer multiplier round(2^16 / temp) (exact_llm.py:249)."""
    return int(round((1 << 16) / temp))


def sample(lg, seed, step, tnum, expt, ids, p_out=None):
    """ids[r] = sample_int(lg[r], seed, step[r], tnum) (exact_llm.py:256-259), on the device."""
    R, V = lg.shape
    _lib.call("exact_sample", _ptr(_need(lg, I64, "lg")), R, V, ctypes.c_uint64(seed), _ptr(_need(step, I32, "step", R)), tnum,
              _ptr(expt), _ptr(_need(ids, I32, "ids", R)), _ptr(p_out), _stream())
    return ids


def advance(pos):
    _lib.call("exact_advance", _ptr(pos), pos.numel(), _stream())


def zero_(t):
    _lib.call("exact_zero", _ptr(t), t.numel() * t.element_size(), _stream())
    return t


# ----------------------------------------------------------------------------- mixture of experts
class ExpertLinears:
    """NE packed linears of one shape (N, K) in one allocation: expert e at wp[e * w_stride:], mp[e * m_stride:]."""

    def __init__(self, NE, N, K, device):
        nb, G = (N + 63) // 64, K // 128
        self.NE, self.N, self.K = NE, N, K
        self.w_stride, self.m_stride = nb * G * 8192, nb * G * 64
        self.wp = torch.empty(NE * self.w_stride, dtype=I8, device=device)
        self.mp = torch.empty(NE * self.m_stride, dtype=I16, device=device)

    def part(self, e):
        return (self.wp[e * self.w_stride:(e + 1) * self.w_stride], self.mp[e * self.m_stride:(e + 1) * self.m_stride])


def chunk_rows(abits):
    return 15 if abits == 15 else 16


def max_chunks(P, NE, chunk):
    """Capacity of moe_dispatch's chunk arrays for P pairs over NE experts in chunks of at most `chunk` pairs."""
    return min(P, -(-P // chunk) + NE)


def router_topk(t, s, expt, k, p_sel, e_sel, clear=False, NE=None, gate_col=-1, sig=None, gate=None):
    """Top-k of isoftmax(rs(t[:, :NE], 28 - s)); with gate_col >= 0 also gate = isig(rs(t[:, gate_col], 28 - s))."""
    R, ld = t.shape
    NE = ld if NE is None else NE
    _lib.call("exact_router_topk", _ptr(_need(t, I64, "t")), ld, _ptr(_need(s, I32, "s", R)), _ptr(expt),
              _ptr(_need(p_sel, I64, "p_sel", R * k)), _ptr(_need(e_sel, I32, "e_sel", R * k)), gate_col, _ptr(sig),
              _ptr(gate), R, NE, k, int(clear), _stream())
    return p_sel, e_sel


def moe_dispatch(e_sel, s, NE, k, chunk, out):
    """out: dict of int32 tensors pidx (P,), pair_row (P,), s_pair (P,), chunk_e/chunk_p0/chunk_n (max chunks,), nchunks (1,).
    The chunk arrays must hold max_chunks(P, NE, chunk) entries (the kernel writes every chunk it forms)."""
    R = s.shape[0]
    need = max_chunks(R * k, NE, chunk)
    for n in ("chunk_e", "chunk_p0", "chunk_n"):
        _need(out[n], I32, n, need)
    _lib.call("exact_moe_dispatch", _ptr(_need(e_sel, I32, "e_sel", R * k)), _ptr(_need(s, I32, "s", R)),
              *(_ptr(_need(out[n], I32, n)) for n in ("pidx", "pair_row", "s_pair", "chunk_e", "chunk_p0", "chunk_n",
                                                       "nchunks")), R, NE, k, chunk, _stream())
    return out


ROUTE_MAX = 64   # experts and (row, expert) pairs of one moe_route launch


def moe_route(t, s, expt, k, p_sel, e_sel, chunk, out, clear=False, NE=None, gate_col=-1, sig=None, gate=None):
    """router_topk then moe_dispatch in one launch (decode rows: at most ROUTE_MAX experts and pairs)."""
    R, ld = t.shape
    NE = ld if NE is None else NE
    need = max_chunks(R * k, NE, chunk)
    for n in ("chunk_e", "chunk_p0", "chunk_n"):
        _need(out[n], I32, n, need)
    _lib.call("exact_moe_route", _ptr(_need(t, I64, "t")), ld, _ptr(_need(s, I32, "s", R)), _ptr(expt),
              _ptr(_need(p_sel, I64, "p_sel", R * k)), _ptr(_need(e_sel, I32, "e_sel", R * k)), gate_col, _ptr(sig),
              _ptr(gate), R, NE, k, int(clear),
              *(_ptr(_need(out[n], I32, n)) for n in ("pidx", "pair_row", "s_pair", "chunk_e", "chunk_p0", "chunk_n",
                                                       "nchunks")), chunk, _stream())
    return p_sel, e_sel, out


def gemv_experts(x, abits, row_map, lin, disp, out):
    """out[p] += x[row_map[p]] . W_{expert of p} for the dispatched chunks (row_map None: x row p)."""
    _need(x, I16 if abits == 15 else I8, "x")
    _need(out, I64, "out")
    if x.shape[1] != lin.K or out.shape[1] != lin.N:
        raise ExactError(f"gemv_experts: x {tuple(x.shape)}, out {tuple(out.shape)} against ({lin.N}, {lin.K})")
    _lib.call("exact_gemv_g128_experts", _ptr(x), abits, _ptr(row_map), _ptr(lin.wp), _ptr(lin.mp), lin.w_stride,
              lin.m_stride, _ptr(disp["chunk_e"]), _ptr(disp["chunk_p0"]), _ptr(disp["chunk_n"]), _ptr(disp["nchunks"]),
              disp["chunk_e"].numel(), _ptr(out), lin.N, lin.K, _stream())
    return out


EXPERT_FUSE_CHUNK = 4   # pairs per dispatched chunk that the fused expert GEMVs below take


def _chunks(disp):
    return (_ptr(_need(disp["chunk_e"], I32, "chunk_e")), _ptr(_need(disp["chunk_p0"], I32, "chunk_p0")),
            _ptr(_need(disp["chunk_n"], I32, "chunk_n")), _ptr(_need(disp["nchunks"], I32, "nchunks", 1)),
            disp["chunk_e"].numel())


def gemv_experts_swiglu(x, row_map, lin, disp, s_pair, silu, h, part, chunk=EXPERT_FUSE_CHUNK):
    """The routed experts' gate|up GEMV with the SwiGLU in its epilogue (int16 rows; chunks of at most 4 pairs, from
    moe_dispatch with that chunk): h[p] = SwiGLU of x[row_map[p]] . W_e with shift s_pair[p], part[p * (I / 32) + b] =
    bit length of max |h[p]| over columns 32 b .. 32 b + 31; gemv_experts_qrow_acc takes them."""
    I = lin.N // 2
    P = h.shape[0]
    _need(x, I16, "x")
    if x.shape[1] != lin.K or lin.N % 2 or h.shape[1] != I:
        raise ExactError(f"gemv_experts_swiglu: x {tuple(x.shape)}, h {tuple(h.shape)} against ({lin.N}, {lin.K})")
    _lib.call("exact_gemv_g128_experts_swiglu", _ptr(x), _ptr(row_map), _ptr(lin.wp), _ptr(lin.mp), lin.w_stride,
              lin.m_stride, *_chunks(disp), chunk, _ptr(_need(s_pair, I32, "s_pair", P)), _ptr(silu),
              _ptr(_need(h, I64, "h", P * I)), _ptr(_need(part, I32, "part", P * (I // SWIGLU_PART_COLS))), I, lin.K,
              _stream())
    return h, part


def gemv_experts_qrow_acc(xs, part, nparts, lin, disp, out, s_out, chunk=EXPERT_FUSE_CHUNK):
    """out[p] += qrow(xs[p], 15) . W_e for the dispatched chunks (at most 4 pairs each), the shifts from the producer's
    slice bit lengths part (P, nparts); s_out[p] = the shift."""
    P, ldx = xs.shape
    _need(xs, I64, "xs")
    if ldx < lin.K or out.shape[1] != lin.N:
        raise ExactError(f"gemv_experts_qrow_acc: xs {tuple(xs.shape)}, out {tuple(out.shape)} against ({lin.N}, {lin.K})")
    _lib.call("exact_gemv_g128_experts_qrow_acc", _ptr(xs), ldx, _ptr(_need(part, I32, "part", P * nparts)), nparts,
              _ptr(lin.wp), _ptr(lin.mp), lin.w_stride, lin.m_stride, *_chunks(disp), chunk,
              _ptr(_need(out, I64, "out", P * lin.N)), _ptr(_need(s_out, I32, "s_out", P)), lin.N, lin.K, _stream())
    return out


def moe_swiglu_pair(x, row_map, elin, disp, s_pair, silu, eh, epart, slin, s, sh, spart, chunk=EXPERT_FUSE_CHUNK):
    """gemv_experts_swiglu(x, row_map, elin, disp, s_pair, silu, eh, epart) and gemv_swiglu(x, slin, s, silu, sh, spart)
    (the shared expert, R <= 2 rows of x) in one launch."""
    R, K = x.shape
    EI, SI = elin.N // 2, slin.N // 2
    P = eh.shape[0]
    _need(x, I16, "x")
    if elin.K != K or slin.K != K or elin.N % 2 or slin.N % 2 or eh.shape[1] != EI:
        raise ExactError(f"moe_swiglu_pair: x {tuple(x.shape)} against ({elin.N}, {elin.K}) and ({slin.N}, {slin.K})")
    _need_packed(slin, "moe_swiglu_pair")
    _lib.call("exact_moe_swiglu_pair", _ptr(x), _ptr(row_map), _ptr(elin.wp), _ptr(elin.mp), elin.w_stride, elin.m_stride,
              *_chunks(disp), chunk, _ptr(_need(s_pair, I32, "s_pair", P)), _ptr(silu), _ptr(_need(eh, I64, "eh", P * EI)),
              _ptr(_need(epart, I32, "epart", P * (EI // SWIGLU_PART_COLS))), EI, _ptr(slin.wp), _ptr(slin.mp),
              _ptr(slin.mh), _ptr(_need(s, I32, "s", R)), _ptr(_need(sh, I64, "sh", R * SI)),
              _ptr(_need(spart, I32, "spart", R * (SI // SWIGLU_PART_COLS))), R, SI, K, _stream())
    return eh, sh


def moe_qrow_pair(exs, epart, enparts, elin, disp, et, es_out, sxs, spart, snparts, slin, st, ss_out, zero=None,
                  chunk=EXPERT_FUSE_CHUNK):
    """gemv_experts_qrow_acc(exs, epart, enparts, elin, disp, et, es_out) and gemv_qrow_acc(sxs, spart, snparts, 15, slin,
    st, ss_out, zero=zero) (the shared expert's down GEMV, R <= 2 rows) in one launch."""
    P, eldx = exs.shape
    R, sldx = sxs.shape
    _need(exs, I64, "exs")
    _need(sxs, I64, "sxs")
    if eldx < elin.K or et.shape[1] != elin.N or sldx < slin.K:
        raise ExactError(f"moe_qrow_pair: xs {tuple(exs.shape)} / {tuple(sxs.shape)} against ({elin.N}, {elin.K}) and "
                         f"({slin.N}, {slin.K})")
    _need_packed(slin, "moe_qrow_pair")
    _lib.call("exact_moe_qrow_pair", _ptr(exs), eldx, _ptr(_need(epart, I32, "epart", P * enparts)), enparts, _ptr(elin.wp),
              _ptr(elin.mp), elin.w_stride, elin.m_stride, *_chunks(disp), chunk, _ptr(_need(et, I64, "et", P * elin.N)),
              _ptr(_need(es_out, I32, "es_out", P)), elin.N, elin.K, _ptr(sxs), sldx,
              _ptr(_need(spart, I32, "spart", R * snparts)), snparts, _ptr(slin.wp), _ptr(slin.mp), _ptr(slin.mh),
              _ptr(_need(st, I64, "st", R * slin.N)), _ptr(_need(ss_out, I32, "ss_out", R)), R, slin.N, slin.K,
              _ptr(zero), 0 if zero is None else _need(zero, I64, "zero").numel(), _stream())
    return et, st


EXPERT_CHUNK = {15: 128, 7: 256}   # pairs per dispatched chunk for gemm_experts: one 256-row matrix-core tile
_EXPERT_ROWS = {}                   # device -> int8 workspace of the gathered (digit) rows


def expert_colterm(lin):
    """(NE, N) int64: each expert's sum_g colsum_g M_g (A8 GEMVs of an all-ones row), cached on the ExpertLinears."""
    ct = getattr(lin, "_colterm", None)
    if ct is None:
        ones = torch.ones((1, lin.K), dtype=I8, device=lin.wp.device)
        ct = torch.empty((lin.NE, lin.N), dtype=I64, device=lin.wp.device)
        for e in range(lin.NE):
            wp, mp = lin.part(e)
            gemv_g128(ones, 7, PackedLinear(wp, mp, lin.N, lin.K), ct[e:e + 1])
        lin._colterm = ct
    return ct


def gemm_experts(x, abits, row_map, lin, disp, out, P):
    """out[p] = x[row_map[p]] . W_{expert of p} for the P dispatched pairs on the matrix cores; disp must come from
    moe_dispatch with chunk = EXPERT_CHUNK[abits] (row_map None: x row p)."""
    _need(x, I16 if abits == 15 else I8, "x")
    _need(out, I64, "out", P * lin.N)
    if x.shape[1] != lin.K or out.shape[1] != lin.N:
        raise ExactError(f"gemm_experts: x {tuple(x.shape)}, out {tuple(out.shape)} against ({lin.N}, {lin.K})")
    need = (2 if abits == 15 else 1) * P * lin.K
    ws = _EXPERT_ROWS.get(x.device)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=I8, device=x.device)
        _EXPERT_ROWS[x.device] = ws
    ct = expert_colterm(lin) if abits == 15 else None
    _lib.call("exact_gemm_g128_experts", _ptr(x), abits, _ptr(row_map), _ptr(lin.wp), _ptr(lin.mp), lin.w_stride, lin.m_stride,
              _ptr(ct), _ptr(ws), _ptr(disp["chunk_e"]), _ptr(disp["chunk_p0"]), _ptr(disp["chunk_n"]), _ptr(disp["nchunks"]),
              min(disp["chunk_e"].numel(), -(-P // EXPERT_CHUNK[abits]) + lin.NE), _ptr(out), P, lin.N, lin.K, _stream())
    return out


def moe_combine(x, t_ed, sh_pair, p_sel, pidx, k, t_sd=None, sh_s=None, gate=None, clear=False):
    R, D = x.shape
    _lib.call("exact_moe_combine", _ptr(_need(x, I64, "x")), _ptr(_need(t_ed, I64, "t_ed")), _ptr(sh_pair), _ptr(p_sel),
              _ptr(pidx), _ptr(t_sd), _ptr(sh_s), _ptr(gate), R, D, k, int(clear), _stream())
    return x


# ----------------------------------------------------------------------------- the reference's op
def gemv_rows(x16, wT, Mg, out=None):
    """out (N,) int64 = sum_g (sum_{k in g} x16[k] wT[n, k]) Mg[n, g] on the reference's own tensors: x16 int16 (K,),
    wT int8 (N, K) row-major (TLinG.wT, speed_fair_kaggle.py:730), Mg int64 (N, K/128) (:731). No repacking."""
    if x16.dim() != 1 or wT.dim() != 2 or Mg.dim() != 2:
        raise ExactError(f"exact::gemv: expected x16 (K,), wT (N, K), Mg (N, K/128); got {tuple(x16.shape)}, "
                         f"{tuple(wT.shape)}, {tuple(Mg.shape)}")
    N, K = wT.shape
    if x16.shape[0] != K or K % 128 or K == 0 or N == 0:
        raise ExactError(f"exact::gemv: x16 has {x16.shape[0]} values, wT is ({N}, {K}); K must be a positive multiple "
                         f"of 128 and equal to x16's length")
    if tuple(Mg.shape) != (N, K // 128):
        raise ExactError(f"exact::gemv: Mg must be ({N}, {K // 128}), got {tuple(Mg.shape)}")
    _need(x16, I16, "exact::gemv: x16")
    _need(wT, I8, "exact::gemv: wT")
    _need(Mg, I64, "exact::gemv: Mg")
    if x16.data_ptr() % 16 or wT.data_ptr() % 16:
        raise ExactError("exact::gemv: x16 and wT must start on a 16-byte boundary")
    out = torch.empty(N, dtype=I64, device=x16.device) if out is None else _need(out, I64, "exact::gemv: out", N)
    _lib.call("exact_gemv", _ptr(x16), _ptr(wT), _ptr(Mg), _ptr(out), N, K, _stream())
    return out


@torch.library.custom_op("exact::gemv", mutates_args=())
def gemv(x16: torch.Tensor, wT: torch.Tensor, Mg: torch.Tensor) -> torch.Tensor:
    """exact::gemv(x16, wT, Mg) -> int64 (N,) (speed_fair_kaggle.py:698-700): the reference's op, same tensors, same
    result; the output is allocated on x16's device and written by one launch on the current stream."""
    return gemv_rows(x16, wT, Mg)


@gemv.register_fake
def _gemv_fake(x16, wT, Mg):
    return torch.empty((wT.shape[0],), dtype=torch.int64, device=x16.device)


def np_to_dev(a, dtype, device):
    a = np.ascontiguousarray(a)
    if not a.flags.writeable:     # a read-only memory map (an artifact file): one transient host copy
        a = a.copy()
    return torch.from_numpy(a).to(device=device, dtype=dtype)


# ----------------------------------------------------------------------------- functional ops for torch callers
# The other entry points of the boundary as torch custom ops (the pattern of exact::gemv above): functional forms
# that allocate their outputs, leave their inputs unchanged and carry fake implementations, so torch.compile and
# graph capture see their shapes. Packed linears travel as (wp, mp, N); the wide-scale plane is not taken here.
@torch.library.custom_op("exact::gemm_g128", mutates_args=())
def gemm_op(x: torch.Tensor, abits: int, wp: torch.Tensor, mp: torch.Tensor, N: int) -> torch.Tensor:
    """t (R, N) int64 = sum_g (x_g . W_g) M_g for any R (GQLin / TLinG, speed_fair_kaggle.py:714-742)."""
    return linear_t(x, abits, PackedLinear(wp, mp, N, x.shape[1]))


@gemm_op.register_fake
def _gemm_op_fake(x, abits, wp, mp, N):
    return torch.empty((x.shape[0], N), dtype=I64, device=x.device)


@torch.library.custom_op("exact::rmsnorm_qrow", mutates_args=())
def rmsnorm_qrow_op(x: torch.Tensor, g: torch.Tensor, bits: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(xq, s) = qrow(irms(x, g), bits) (exact_llm.py:41-46, 100-106)."""
    return rmsnorm_qrow(x, g, bits)


@rmsnorm_qrow_op.register_fake
def _rmsnorm_qrow_op_fake(x, g, bits):
    R, D = x.shape
    return (torch.empty((R, D), dtype=I16 if bits > 7 else I8, device=x.device),
            torch.empty((R,), dtype=I32, device=x.device))


@torch.library.custom_op("exact::swiglu_qrow", mutates_args=())
def swiglu_qrow_op(t: torch.Tensor, s: torch.Tensor, silu: torch.Tensor, bits: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(hq, sh) = qrow(shr(isilu(g) u, 16), bits) of a fused gate|up total t (R, 2I) (exact_llm.py:179); t unchanged."""
    R, N2 = t.shape
    h = torch.empty((R, N2 // 2), dtype=I64, device=t.device)
    return swiglu_qrow(t, s, silu, bits, h=h)


@swiglu_qrow_op.register_fake
def _swiglu_qrow_op_fake(t, s, silu, bits):
    R, N2 = t.shape
    return (torch.empty((R, N2 // 2), dtype=I16 if bits > 7 else I8, device=t.device),
            torch.empty((R,), dtype=I32, device=t.device))


@torch.library.custom_op("exact::attention", mutates_args=())
def attention_op(qq: torch.Tensor, sq: torch.Tensor, kq: torch.Tensor, sk: torch.Tensor, v: torch.Tensor, slot: torch.Tensor,
                 pos: torch.Tensor, expt: torch.Tensor, inv: int) -> torch.Tensor:
    """out (R, H hd) = shr(isoftmax(shr((qq . kq) INV, 32 - sq - sk)) . v, 20) over keys 0..pos[r] of slot[r]
    (exact_llm.py:170-176); qq (R, H, hd), cache kq (B, KV, Smax, hd), sk (B, KV, Smax), v (B, KV, Smax, hd)."""
    R, H, hd = qq.shape
    out = torch.empty((R, H * hd), dtype=I64, device=qq.device)
    return attention(qq, sq, (kq, sk, v), slot, pos, expt, out, H, kq.shape[1], hd, inv)


@attention_op.register_fake
def _attention_op_fake(qq, sq, kq, sk, v, slot, pos, expt, inv):
    R, H, hd = qq.shape
    return torch.empty((R, H * hd), dtype=I64, device=qq.device)


@torch.library.custom_op("exact::router_topk", mutates_args=())
def router_topk_op(t: torch.Tensor, s: torch.Tensor, expt: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(p_sel Q20 int64, e_sel int32) = top-k of isoftmax(shr(t, 28 - s)), ties to the lower expert
    (moe_exact_kaggle.py:454-460); t unchanged."""
    R = t.shape[0]
    p_sel = torch.empty((R, k), dtype=I64, device=t.device)
    e_sel = torch.empty((R, k), dtype=I32, device=t.device)
    return router_topk(t, s, expt, k, p_sel, e_sel)


@router_topk_op.register_fake
def _router_topk_op_fake(t, s, expt, k):
    R = t.shape[0]
    return torch.empty((R, k), dtype=I64, device=t.device), torch.empty((R, k), dtype=I32, device=t.device)


@torch.library.custom_op("exact::logits_argmax", mutates_args=())
def logits_argmax_op(t: torch.Tensor, s: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(logits = shr(t, 28 - s) int64, ids = first argmax int32) of the head totals (exact_llm.py:180, 267)."""
    R, N = t.shape
    lg = torch.empty((R, N), dtype=I64, device=t.device)
    ids = torch.empty((R,), dtype=I32, device=t.device)
    return logits_argmax(t, s, lg, ids)


@logits_argmax_op.register_fake
def _logits_argmax_op_fake(t, s):
    R, N = t.shape
    return torch.empty((R, N), dtype=I64, device=t.device), torch.empty((R,), dtype=I32, device=t.device)
