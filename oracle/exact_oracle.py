"""CPU oracle for the exact integer forward path (numpy, int64).

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this module; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the reference the GPU results are compared with (or the timed CPU baseline), never as the thing
measured or shipped.

It restates the reference's numeric program (SPEC.md:14-32, v0.4) in numpy:
every function names the reference file:line it follows.  Arithmetic is int64 with numpy's
wrap-around semantics; float64 is used only where the reference uses it and only while every
partial sum stays below 2^53 (SPEC.md:30-32), so results are exact integers.

Pinning (what checks each function against something other than this file):
  * tables EXP_T / SILU_T            -> webverify/cells_tiny.json "tables" (bit-equal)
  * round_shift, bitlen, qrow, isqrt, irms, isoftmax, isilu, rope, requant_channel,
    attention row, SwiGLU, residual  -> replay of the 8 cells in cells_tiny.json (verdicts) and
                                        brute force with Python ints / math.isqrt
  * linear_group (GQLin)             -> closed form of the G1 test (speed_fair_kaggle.py:708)
  * Model.forward (IntModel)         -> golden logits written from the reference's own IntModel
                                        (tests/golden/make_golden.py) + the cells above
  * KV-cached decode                 -> equality with full recompute (attention_tc_longctx_kaggle.py:641-643)
  * Model.moe, moe_route, moe_weighted, isig / SIG_T
                                     -> vectors of the reference's own MoEInt.moe, SIG_T / isig and GQLin
                                        (tests/golden/make_golden_moe.py: per-channel and group-128 layers,
                                        ties across the top-k boundary) + planted mistakes that must fail
  * reduction order                  -> logits hashes identical with K permuted or reversed inside exact_mm
                                        and group_acc (exact_llm.py:76-79)
  * sampler (splitmix64, sample_int) -> known-answer values of splitmix64 from its published
                                        definition + brute-force inverse CDF
  * quantize_channel / quantize_group -> closed-form properties (the column / group maximum maps to
                                        +-127 exactly, |w - w8 sc| <= sc / 2, M = rint(sc 2^28), zero
                                        columns give w8 = 0, M = 0) checked on random and constructed inputs
"""
import hashlib
import math

import numpy as np

F = 16
ONE = 1 << F
I64 = np.int64


def h(a):
    """Conformance hash: sha256 of C-contiguous int64 bytes, first 16 hex (exact_llm.py:22)."""
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


# ----------------------------------------------------------------------------- primitives
def round_shift(a, n):
    """Round-half-up arithmetic shift right by n; n <= 0 shifts left (exact_llm.py:25-34; SPEC.md:19)."""
    a = np.asarray(a, dtype=I64)
    n = np.asarray(n, dtype=I64)
    if n.ndim == 0:
        n = int(n)
        if n <= 0:
            return a << I64(-n)
        return (a + I64(1 << (n - 1))) >> I64(n)
    right = np.maximum(n, 0)
    left = np.maximum(-n, 0)
    half = np.left_shift(I64(1), np.maximum(right - 1, 0))
    out = np.where(right > 0, (a + half) >> right, a)
    return out << left


shr = round_shift


def _bitlen32(v):
    # frexp is exact for integers below 2^53: v = m * 2^e with 0.5 <= m < 1, so e = bit length.
    return np.frexp(v.astype(np.float64))[1].astype(I64)


def bitlen(m):
    """Bit length of m >= 0 (0 -> 0); non-positive inputs give 0 (exact_llm.py:35-40)."""
    m = np.asarray(m, dtype=I64)
    hi = m >> I64(32)
    lo = m & I64(0xFFFFFFFF)
    out = np.where(hi > 0, 32 + _bitlen32(np.maximum(hi, 0)), _bitlen32(lo))
    return np.where(m > 0, out, 0).astype(I64)


def qrow(x, bits=15):
    """Per-row quantiser: s = max(bitlen(max|x|) - bits, 0); xq = clip(shr(x, s), +-(2^bits - 1))
    (exact_llm.py:41-46; SPEC.md:18)."""
    x = np.asarray(x, dtype=I64)
    m = np.abs(x).max(-1, keepdims=True)
    s = np.maximum(bitlen(m) - bits, 0)
    lim = (1 << bits) - 1
    return np.clip(round_shift(x, s), -lim, lim), s


def isqrt(n):
    """floor(sqrt(n)) for 0 <= n < 2^62 (exact_llm.py:97-99): float estimate, then integer correction."""
    n = np.asarray(n, dtype=I64)
    r = np.floor(np.sqrt(n.astype(np.float64))).astype(I64)
    for _ in range(2):
        r = np.where(r * r > n, r - 1, r)
        r = np.where((r + 1) * (r + 1) <= n, r + 1, r)
    return r


def irms(x, g):
    """Integer RMSNorm (exact_llm.py:100-106; SPEC.md:20): exact isqrt and floor division."""
    x = np.asarray(x, dtype=I64)
    k = np.maximum(bitlen(np.abs(x).max(-1, keepdims=True)) - 24, 0)
    xs = round_shift(x, k)
    ms = (xs * xs).sum(-1, keepdims=True) // x.shape[-1] + 1
    r = np.maximum(isqrt(ms), 1)
    y = (x << I64(F)) // (r << k)
    return round_shift(y * g, F)


# ----------------------------------------------------------------------------- tables
EXP_STEP = 8
SILU_STEP = 8


def exp_table():
    """Q24 exp(-i/256), i in [0, 40*256+2) (exact_llm.py:108). Python round() of the float64 value."""
    return np.array([round(math.exp(-i / 256) * (1 << 24)) for i in range(256 * 40 + 2)], I64)


def silu_table():
    """Q16 SiLU on [-16, 16) at 1/256 steps (exact_llm.py:117); same float64 expression order."""
    out = []
    for i in range(32 * 256 + 2):
        v = (i - 16 * 256) / 256
        out.append(round(v / (1 + math.exp(-v)) * ONE))
    return np.array(out, I64)


def sig_table():
    """Q16 sigmoid on [-16, 16) at 1/256 steps (moe_exact_kaggle.py:419)."""
    return np.array([round(1.0 / (1.0 + math.exp(-((i - 16 * 256) / 256))) * ONE) for i in range(32 * 256 + 2)], I64)


EXP_T = exp_table()
SILU_T = silu_table()
SIG_T = sig_table()


def isoftmax(sc, valid, table=None):
    """Integer softmax -> Q20 probabilities (exact_llm.py:109-115; SPEC.md:23)."""
    T = EXP_T if table is None else table
    sc = np.asarray(sc, dtype=I64)
    mx = np.where(valid, sc, np.iinfo(np.int64).min // 4).max(-1, keepdims=True)
    d = np.where(valid, mx - sc, 0)
    i = np.minimum(d >> I64(EXP_STEP), len(T) - 2)
    fr = d & I64((1 << EXP_STEP) - 1)
    e = T[i] - round_shift((T[i] - T[i + 1]) * fr, EXP_STEP)
    e = np.where(valid & (d < (40 << F)), e, 0)
    return (e << I64(20)) // e.sum(-1, keepdims=True)


def _lut16(x, T, top):
    t = np.clip(x, -16 * ONE, 16 * ONE - 1) + 16 * ONE
    i = t >> I64(8)
    fr = t & I64(255)
    y = T[i] + round_shift((T[i + 1] - T[i]) * fr, 8)
    return np.where(x >= 16 * ONE, top, np.where(x < -16 * ONE, 0, y))


def isilu(x, table=None):
    """Integer SiLU (exact_llm.py:118-122): identity at x >= 16, 0 below -16."""
    x = np.asarray(x, dtype=I64)
    return _lut16(x, SILU_T if table is None else table, x)


def isig(x, table=None):
    """Integer sigmoid (moe_exact_kaggle.py:420-424): 1.0 (Q16) at x >= 16, 0 below -16."""
    x = np.asarray(x, dtype=I64)
    return _lut16(x, SIG_T if table is None else table, ONE)


def rope_tables(T, hd, theta):
    """Q16 cos/sin tables (exact_llm.py:127-130, 157-158): float64 angles, rint to Q16."""
    inv = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd))
    ang = np.outer(np.arange(T, dtype=np.float64), inv)
    ang = np.concatenate([ang, ang], -1)
    return np.rint(np.cos(ang) * ONE).astype(I64), np.rint(np.sin(ang) * ONE).astype(I64)


def rot_half(x):
    """(a, b) -> (-b, a) on the last axis (exact_llm.py:131-132)."""
    a, b = np.split(x, 2, -1)
    return np.concatenate([-b, a], -1)


def rope(x, cos, sin):
    """shr(x*cos + rot_half(x)*sin, 16) (exact_llm.py:159-160; SPEC.md:21). x (..., T, hd), cos/sin (T, hd)."""
    return round_shift(x * cos + rot_half(x) * sin, F)


def inv_sqrt_hd(hd):
    """C = round(2^16 / sqrt(hd)) (exact_llm.py:164; SPEC.md:22)."""
    return int(round((1 << 16) / math.sqrt(hd)))


# ----------------------------------------------------------------------------- exact matmul
def exact_mm(a, b):
    """Exact integer product a (.., K) @ b (K, N) via float64 BLAS + rint (exact_llm.py:75-81).
    The caller guarantees every partial sum stays below 2^53."""
    r = np.matmul(np.asarray(a).astype(np.float64), np.asarray(b).astype(np.float64))
    return np.rint(r).astype(I64)


def group_acc(xq, w, G=128):
    """Per-group exact accumulators acc[g, r, n] = sum_{k in group g} xq[r, k] * w[k, n]
    (speed_fair_kaggle.py:723-724; the G1 closed form at :708). float64 per group is exact:
    |acc_g| < 2^31 (group128_quality_kaggle.py:419)."""
    R, K = xq.shape
    Gn = K // G
    xg = xq.reshape(R, Gn, G).transpose(1, 0, 2).astype(np.float64)      # (G, R, 128)
    wg = w.reshape(Gn, G, -1).astype(np.float64)                          # (G, 128, N)
    return np.rint(np.matmul(xg, wg)).astype(I64)


def linear_group(x, w, Mg, b=None, abits=15, n_chunk=16384):
    """Group-128 linear (GQLin, speed_fair_kaggle.py:714-725; SPEC.md:18):
    xq, s = qrow(x, abits); t = sum_g acc_g * M_g; y = shr(t, 28 - s) + b.
    w (K, N) int8, Mg (K/128, N) int (positive, < 2^27), b (N,) Q16 or None.
    abits = 15 is the spec (int16 activations); abits = 7 is exact_torch's A8 mode (exact_torch.py:99-100)."""
    y, _ = linear_group_t(x, w, Mg, b, abits, n_chunk)
    return y


_GROUP_T = None


def set_group_kernel(fn):
    """Route t = sum_g acc_g * M_g through fn(xq, w, Mg) (the C restatement in exact_c.c, used for
    large-model fixtures); None restores the numpy path."""
    global _GROUP_T
    _GROUP_T = fn


def linear_group_t(x, w, Mg, b=None, abits=15, n_chunk=16384):
    """linear_group returning (y, t) where t = sum_g acc_g * M_g is the raw int64 total."""
    x = np.asarray(x, dtype=I64)
    xq, s = qrow(x, abits)
    N = w.shape[1]
    if _GROUP_T is not None:
        t = _GROUP_T(xq, w, Mg)
    else:
        t = np.empty((x.shape[0], N), I64)
        for j in range(0, N, n_chunk):
            acc = group_acc(xq, w[:, j:j + n_chunk])                        # (G, R, n)
            t[:, j:j + n_chunk] = (acc * np.asarray(Mg[:, j:j + n_chunk], I64)[:, None, :]).sum(0)
    y = round_shift(t, 28 - s)
    return (y if b is None else y + b), t


def requant_channel(acc, s, M, Mbits, b=None):
    """Per-channel requant with the per-row overflow drop rule (exact_llm.py:93-96; SPEC.md:28;
    commit_audit_kaggle.py:442-445)."""
    acc = np.asarray(acc, dtype=I64)
    drop = np.maximum(bitlen(np.abs(acc).max(-1, keepdims=True)) + Mbits - 62, 0)
    y = round_shift(round_shift(acc, drop) * M, 28 - s - drop)
    return y if b is None else y + b


def linear_channel(x, w, M, b=None, abits=15):
    """Per-channel linear (QLin.__call__, exact_llm.py:89-96): one scale M per output column."""
    x = np.asarray(x, dtype=I64)
    xq, s = qrow(x, abits)
    acc = exact_mm(xq, w)
    Mbits = int(bitlen(np.array([np.asarray(M).max()]))[0])
    return requant_channel(acc, s, np.asarray(M, I64), Mbits, b)


class Lin:
    """A linear layer of the integer artifact: w (K, N) int8, scales and bias.
    mode 'group': Mg (K/128, N); mode 'channel': M (N,) with the drop rule."""

    def __init__(self, w, M, b=None, mode="group"):
        self.w = np.asarray(w, np.int8)
        self.M = np.asarray(M, I64)
        self.b = None if b is None else np.asarray(b, I64)
        self.mode = mode

    def __call__(self, x, abits=15):
        if self.mode == "group":
            return linear_group(x, self.w, self.M, self.b, abits)
        return linear_channel(x, self.w, self.M, self.b, abits)


# ----------------------------------------------------------------------------- float checkpoint -> integers
def quantize_channel(w_in_out):
    """Per-channel quantisation of a float (in, out) weight (QLin.__init__, exact_llm.py:83-86), float64:
    sc = max_k |w[k, n]| (1e-12 for an all-zero column) / 127; w8 = clip(rint(w / sc), -127, 127) int8;
    M = rint(sc * 2^28) int64."""
    w = np.asarray(w_in_out, np.float64)
    sc = np.abs(w).max(0)
    sc = np.where(sc == 0, 1e-12, sc) / 127.0
    return np.clip(np.rint(w / sc), -127, 127).astype(np.int8), np.rint(sc * (1 << 28)).astype(I64)


def quantize_group(w_in_out, G=128):
    """Group-128 quantisation (GQLin.__init__, speed_fair_kaggle.py:715-721; the reference takes the (out, in)
    checkpoint array and transposes it first): the per-channel rule of quantize_channel applied to every
    128-row group of the (in, out) weight; M (K/G, N)."""
    w = np.asarray(w_in_out, np.float64)
    K, N = w.shape
    w8 = np.empty((K, N), np.int8)
    M = np.empty((-(-K // G), N), I64)
    for gi, a in enumerate(range(0, K, G)):
        w8[a:a + G], M[gi] = quantize_channel(w[a:a + G])
    return w8, M


def q16(v):
    """Q16 integers of float64 values (norm gains, biases, embedding rows: exact_llm.py:85-87, 143, 163)."""
    return np.rint(np.asarray(v, np.float64) * ONE).astype(I64)


# ----------------------------------------------------------------------------- attention
def attention_head(q, k, v, valid, INV):
    """One head of integer attention (exact_llm.py:171-176; exact_torch.py:147-166):
    qq, sq = qrow(q); kk, sk = qrow(k); sc = shr((qq kk^T) * INV, 32 - sq - sk);
    p = isoftmax(sc, valid) (Q20); out = shr(p v, 20) in exact int64."""
    qq, sq = qrow(q)
    kk, sk = qrow(k)
    return attention_head_q(qq, sq, kk, sk, v, valid, INV)


def attention_head_q(qq, sq, kk, sk, v, valid, INV):
    """Attention for already-quantised q rows and cached k rows (the KV cache stores kq, sk, v:
    exact_torch.py:147-149)."""
    sc = round_shift(exact_mm(qq, kk.T) * INV, (F - sq - sk.T) + 16)
    p = isoftmax(sc, valid)
    return round_shift(np.matmul(p.astype(I64), np.asarray(v, I64)), 20)


# ----------------------------------------------------------------------------- MoE routing
def moe_route(p, k):
    """Top-k experts per row: stable sort of -p, so equal probabilities go to the lower expert index
    (moe_exact_kaggle.py:457)."""
    return np.argsort(-p, axis=-1, kind="stable")[:, :k]


def moe_weighted(p, sel, rows, e, ye):
    """Expert e's output rows weighted by the un-renormalised Q20 router probability:
    shr(p[rows, e] * ye, 20) (moe_exact_kaggle.py:465)."""
    return round_shift(p[rows, e][:, None] * ye, 20)


# ----------------------------------------------------------------------------- model
class Model:
    """Integer Qwen2-family model (IntModel, exact_llm.py:141-180) with group-128 or per-channel
    linears, optional MoE blocks (MoEInt, moe_exact_kaggle.py:433-482) and a KV cache
    (TModel.forward, exact_torch.py:171-193).

    weights: dict with
      emb  (V, D) int64 Q16 rows (the embedding lookup, exact_llm.py:163)
      layers: list of dicts with g1, g2 (D,) Q16; q, k, v, o, gate, up, down: Lin
              MoE layers instead of gate/up/down: router: Lin, experts: list of (gate, up, down) Lin,
              sg, su, sd: Lin (shared expert), sgate: Lin (N = 1)
      gf (D,) Q16, head: Lin
    cfg: dict with D, H, KV, hd, NL, theta, T (rope table length), topk (MoE)
    """

    def __init__(self, weights, cfg, abits=15):
        self.w = weights
        self.c = cfg
        self.abits = abits
        self.cos, self.sin = rope_tables(cfg["T"], cfg["hd"], cfg["theta"])
        self.INV = inv_sqrt_hd(cfg["hd"])

    def lin(self, L, x):
        return L(x, self.abits)

    def new_cache(self):
        return [dict(kq=None, sk=None, v=None) for _ in self.w["layers"]] + [dict(n=0)]

    def mlp(self, L, m):
        """SwiGLU MLP: down(shr(isilu(gate(m)) * up(m), 16)) (exact_llm.py:179)."""
        return self.lin(L["down"], round_shift(isilu(self.lin(L["gate"], m)) * self.lin(L["up"], m), F))

    def moe(self, L, m, stats=None):
        """MoE block (moe_exact_kaggle.py:454-467): router -> isoftmax Q20 -> top-k by stable sort of -p
        (ties -> lower index) -> per-expert SwiGLU weighted by the un-renormalised Q20 probability, plus
        the shared expert gated by the integer sigmoid."""
        T = m.shape[0]
        logits = self.lin(L["router"], m)
        NE = logits.shape[1]
        p = isoftmax(logits, np.ones((T, NE), bool))
        sel = moe_route(p, self.c["topk"])
        if stats is not None:
            stats.append(sel.copy())
        out = np.zeros_like(m)
        for e in range(NE):
            rows, _ = np.nonzero(sel == e)
            if len(rows) == 0:
                continue
            gp, up, dn = L["experts"][e]
            mm = m[rows]
            ye = self.lin(dn, round_shift(isilu(self.lin(gp, mm)) * self.lin(up, mm), F))
            out[rows] += moe_weighted(p, sel, rows, e, ye)
        ys = self.lin(L["sd"], round_shift(isilu(self.lin(L["sg"], m)) * self.lin(L["su"], m), F))
        return out + round_shift(isig(self.lin(L["sgate"], m)) * ys, F)

    def forward(self, ids, cache=None, stats=None, layers=None):
        """Logits (T, V) int64 Q16 for the new tokens ids; with a cache, positions continue from
        cache[-1]['n'] (exact_torch.py:171-193); without, this is IntModel.__call__ (exact_llm.py:161-180)."""
        c = self.c
        H, KV, hd = c["H"], c["KV"], c["hd"]
        rep = H // KV
        T = len(ids)
        p0 = cache[-1]["n"] if cache is not None else 0
        x = np.asarray(self.w["emb"][np.asarray(ids)], I64)
        cos, sin = self.cos[p0:p0 + T], self.sin[p0:p0 + T]
        Ls = self.w["layers"] if layers is None else self.w["layers"][:layers]
        for li, L in enumerate(Ls):
            a = irms(x, L["g1"])
            q = rope(self.lin(L["q"], a).reshape(T, H, hd).transpose(1, 0, 2), cos, sin)
            k = rope(self.lin(L["k"], a).reshape(T, KV, hd).transpose(1, 0, 2), cos, sin)
            v = self.lin(L["v"], a).reshape(T, KV, hd).transpose(1, 0, 2)
            kq, sk = qrow(k)
            if cache is not None and cache[li]["kq"] is not None:
                C = cache[li]
                kq = np.concatenate([C["kq"], kq], 1)
                sk = np.concatenate([C["sk"], sk], 1)
                v = np.concatenate([C["v"], v], 1)
            if cache is not None:
                cache[li].update(kq=kq, sk=sk, v=v)
            S = kq.shape[1]
            valid = np.arange(S)[None, :] <= (p0 + np.arange(T))[:, None]
            out = np.empty((H, T, hd), I64)
            for hh in range(H):
                kh = hh // rep
                qq, sq = qrow(q[hh])
                out[hh] = attention_head_q(qq, sq, kq[kh], sk[kh], v[kh], valid, self.INV)
            x = x + self.lin(L["o"], out.transpose(1, 0, 2).reshape(T, H * hd))
            m = irms(x, L["g2"])
            if "router" in L:
                x = x + self.moe(L, m, None if stats is None else stats.setdefault(li, []))
            else:
                x = x + self.mlp(L, m)
        if cache is not None:
            cache[-1]["n"] = p0 + T
        return self.lin(self.w["head"], irms(x, self.w["gf"]))

    __call__ = forward


# ----------------------------------------------------------------------------- sampler
MASK64 = (1 << 64) - 1


def splitmix64(seed, pos):
    """SplitMix64 output for counter (pos + 1) (exact_llm.py:243-247; Steele et al. 2014)."""
    z = (seed + (pos + 1) * 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def u20(seed, pos):
    """Uniform integer in [0, 2^20) (exact_llm.py:248)."""
    return splitmix64(seed, pos) >> 44


def temp_num(t):
    """Temperature as the integer multiplier round(2^16 / t) (exact_llm.py:249)."""
    return int(round((1 << 16) / t))


def isoftmax_row(lg):
    """Q20 probabilities of one logits row, all entries valid (exact_llm.py:250-255)."""
    lg = np.asarray(lg, I64)
    return isoftmax(lg[None, :], np.ones((1, lg.shape[0]), bool))[0]


def sample_int(lg_row, seed, pos, tnum):
    """Integer inverse-CDF sample (exact_llm.py:256-259)."""
    p = isoftmax_row(round_shift(np.asarray(lg_row, I64) * tnum, 16))
    cum = np.cumsum(p)
    target = (u20(seed, pos) * int(cum[-1])) >> 20
    return int(np.searchsorted(cum, target, side="right")), p


def step_hash(prev, lg_row):
    """Chained per-step logits hash (exact_llm.py:260-261)."""
    return hashlib.sha256(prev.encode() + np.ascontiguousarray(lg_row).tobytes()).hexdigest()[:16]


def greedy(lg_row):
    """Greedy token: first index of the maximum (exact_llm.py:267, numpy argmax)."""
    return int(np.asarray(lg_row).argmax())


def generate(model, prompt_ids, n, seed=0, temp=1.0, cached=True):
    """Generation with receipts (exact_llm.py:262-268). cached=False re-runs the full sequence every
    step like the reference; cached=True uses the KV cache (bit-identical by causality, SPEC v0.3).
    Returns (receipt, greedy_tokens, logits_rows)."""
    ids = list(prompt_ids)
    chain = "start"
    toks, gr, rows = [], [], []
    tnum = temp_num(temp)
    cache = model.new_cache() if cached else None
    pending = list(ids)
    for t in range(n):
        if cached:
            lg = model.forward(pending, cache)[-1]
        else:
            lg = model.forward(ids)[-1]
        tok, _ = sample_int(lg, seed, t, tnum)
        chain = step_hash(chain, lg)
        toks.append(tok)
        gr.append(greedy(lg))
        rows.append(lg.copy())
        ids.append(tok)
        pending = [tok]
    return dict(prompt=list(prompt_ids), seed=seed, temp=temp, tokens=toks, chain=chain), gr, rows


def greedy_decode(model, prompt_ids, n, cached=True):
    """Greedy decode (argmax feedback) returning (tokens, logits rows (n, V))."""
    cache = model.new_cache() if cached else None
    ids = list(prompt_ids)
    pending = list(ids)
    toks, rows = [], []
    for _ in range(n):
        lg = model.forward(pending, cache)[-1] if cached else model.forward(ids)[-1]
        tok = greedy(lg)
        toks.append(tok)
        rows.append(lg.copy())
        ids.append(tok)
        pending = [tok]
    return toks, np.stack(rows)
