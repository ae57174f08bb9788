"""GPU parity of integer attention (exact_llm.py:170-176; exact_torch.py:162-166) against the oracle:
the row kernel (decode and small prefill) and the matrix-core prefill kernel, bit-exact."""
import numpy as np
import pytest
import torch

import exact_oracle as O
from exact_amd import ops
from exact_amd.tables import exp_t

pytestmark = pytest.mark.gpu
DEV = "cuda"
I16, I32, I64 = torch.int16, torch.int32, torch.int64


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_case(seed, B, slot, H, KV, hd, Smax, nkeys, R, vmag, shifts=4):
    """A cache with nkeys written positions in `slot` (other slots hold unrelated data) and R query rows
    at positions nkeys - R .. nkeys - 1. vmag: ("small" | "large" | "wrap") magnitude of v; q and k row
    shifts drawn from [0, shifts) (or [0, shifts[0]) for q and [0, shifts[1]) for k). Shift sums above 32
    take the left-shift branch of shr; the kernel's float64 scores cover sums up to 33, int64 the rest."""
    rng = np.random.default_rng(seed)
    kq = rng.integers(-32767, 32768, (B, KV, Smax, hd))
    qs, ks = (shifts, shifts) if np.isscalar(shifts) else shifts
    sk = rng.integers(0, ks, (B, KV, Smax))
    if vmag == "small":
        v = rng.integers(-(1 << 29), 1 << 29, (B, KV, Smax, hd))
    elif vmag == "large":
        v = rng.integers(-(1 << 29), 1 << 29, (B, KV, Smax, hd)) << rng.integers(0, 20, (B, KV, Smax, 1))
    else:   # products beyond int64: the sum is taken modulo 2^64, as numpy's int64 matmul does
        v = rng.integers(-(1 << 62), 1 << 62, (B, KV, Smax, hd))
    qq = rng.integers(-32767, 32768, (R, H, hd))
    qq[0, 0, :4] = [32767, -32767, 0, -1]
    sq = rng.integers(0, qs, (R, H))
    pos = np.arange(nkeys - R, nkeys)
    return kq, sk, v, qq, sq, pos


def oracle_rows(kq, sk, v, qq, sq, pos, slot, H, KV, rows):
    hd = qq.shape[-1]
    out = np.zeros((len(rows), H * hd), np.int64)
    inv = O.inv_sqrt_hd(hd)
    S = int(pos[rows].max()) + 1
    valid = np.arange(S)[None, :] <= pos[rows][:, None]
    for h in range(H):
        kh = h // (H // KV)
        out[:, h * hd:(h + 1) * hd] = O.attention_head_q(qq[rows, h], sq[rows, h][:, None], kq[slot, kh, :S],
                                                         sk[slot, kh, :S][:, None], v[slot, kh, :S], valid, inv)
    return out


def to_dev(kq, sk, v, qq, sq, pos):
    d = lambda a, dt: torch.tensor(np.ascontiguousarray(a), dtype=dt, device=DEV)
    return (d(kq, I16), d(sk, I32), d(v, I64)), d(qq, I16), d(sq, I32), d(pos, I32)


def run_prefill(cache, qq, sq, pos, slot, nkeys, H, KV, hd):
    R = qq.shape[0]
    out = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    obits = torch.full((R, H), -1, dtype=I32, device=DEV)
    ws = ops.prefill_workspace(R, H, KV, hd, nkeys, DEV)
    ops.attention_prefill(qq, sq, cache, slot, pos, nkeys, torch.tensor(exp_t(), dtype=I32, device=DEV), out, H, KV, hd,
                          O.inv_sqrt_hd(hd), ws, obits)
    return host(out), host(obits)


def obits_of(out, H):
    a = np.abs(out.reshape(out.shape[0], H, -1)).max(-1)
    return np.vectorize(O.bitlen)(a)


@pytest.mark.parametrize("H,KV,nkeys,R,vmag,shifts", [(4, 2, 1, 1, "small", 4), (4, 2, 33, 33, "small", 4),
                                                      (4, 1, 100, 37, "large", 4), (2, 2, 64, 64, "wrap", 4),
                                                      (28, 4, 161, 129, "small", 4), (4, 2, 150, 150, "small", 22),
                                                      (7, 7, 190, 70, "large", 1), (4, 2, 120, 120, "small", (18, 17)),
                                                      (4, 2, 120, 120, "small", (18, 18))])
def test_prefill_matches_oracle(H, KV, nkeys, R, vmag, shifts):
    hd, Smax, slot = 128, 192, 1
    case = make_case(nkeys * 7 + R, 2, slot, H, KV, hd, Smax, nkeys, R, vmag, shifts)
    cache, qq, sq, pos = to_dev(*case)
    out, obits = run_prefill(cache, qq, sq, pos, slot, nkeys, H, KV, hd)
    want = oracle_rows(*case, slot, H, KV, np.arange(R))
    assert np.array_equal(out, want)
    assert np.array_equal(obits, obits_of(want, H))


@pytest.mark.parametrize("H,KV,nkeys,R,vmag,shifts", [(14, 2, 300, 300, "small", 4), (14, 2, 290, 257, "large", 4),
                                                      (4, 2, 1, 1, "small", 4), (4, 1, 100, 37, "large", 4),
                                                      (2, 2, 64, 64, "wrap", 4), (4, 2, 150, 150, "small", 22),
                                                      (4, 2, 120, 120, "small", (18, 18))])
def test_prefill_hd64_matches_oracle(H, KV, nkeys, R, vmag, shifts):
    """head dimension 64 (the 0.5B shape: 14 q heads over 2 KV heads) on the matrix-core prefill: two 32-dimension
    blocks per q.k product and two p.v consumer waves; bit-exact against the oracle, obits too"""
    hd, Smax, slot = 64, 320, 1
    case = make_case(nkeys * 5 + R, 2, slot, H, KV, hd, Smax, nkeys, R, vmag, shifts)
    cache, qq, sq, pos = to_dev(*case)
    out, obits = run_prefill(cache, qq, sq, pos, slot, nkeys, H, KV, hd)
    want = oracle_rows(*case, slot, H, KV, np.arange(R))
    assert np.array_equal(out, want)
    assert np.array_equal(obits, obits_of(want, H))


@pytest.mark.parametrize("R,nkeys", [(3, 50), (17, 17), (70, 100)])   # 70 x 4 heads: the blocks run in several rounds
def test_row_attention_matches_oracle(R, nkeys):
    H, KV, hd, Smax, slot = 4, 2, 128, max(64, nkeys), 1
    case = make_case(R + nkeys, 2, slot, H, KV, hd, Smax, nkeys, R, "large")
    cache, qq, sq, pos = to_dev(*case)
    out = torch.zeros((R, H * hd), dtype=I64, device=DEV)
    obits = torch.zeros((R, H), dtype=I32, device=DEV)
    slots = torch.full((R,), slot, dtype=I32, device=DEV)
    ops.attention(qq, sq, cache, slots, pos, torch.tensor(exp_t(), dtype=I32, device=DEV), out, H, KV, hd,
                  O.inv_sqrt_hd(hd), obits)
    want = oracle_rows(*case, slot, H, KV, np.arange(R))
    assert np.array_equal(host(out), want)
    assert np.array_equal(host(obits), obits_of(want, H))


@pytest.mark.parametrize("R,H,KV,hd,nkeys", [(80, 4, 2, 64, 300), (40, 8, 2, 128, 257), (65, 4, 1, 256, 70),
                                             (33, 8, 4, 128, 520)])
def test_row_attention_many_blocks_matches_oracle(R, H, KV, hd, nkeys):
    """More (row, head) blocks than one round (the batch-decode path, no prefetch), at hd 64, 128 and 256, over caches
    of 70 to 520 positions with rows at consecutive positions."""
    Smax, slot = nkeys + 8, 0
    case = make_case(R * 7 + nkeys, 1, slot, H, KV, hd, Smax, nkeys, R, "large")
    cache, qq, sq, pos = to_dev(*case)
    print(f"many-block attention R={R} H={H} hd={hd} nkeys={nkeys}", flush=True)
    out = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    obits = torch.zeros((R, H), dtype=I32, device=DEV)
    ops.attention(qq, sq, cache, torch.full((R,), slot, dtype=I32, device=DEV), pos,
                  torch.tensor(exp_t(), dtype=I32, device=DEV), out, H, KV, hd, O.inv_sqrt_hd(hd), obits)
    want = oracle_rows(*case, slot, H, KV, np.arange(R))
    assert np.array_equal(host(out), want)
    assert np.array_equal(host(obits), obits_of(want, H))


@pytest.mark.parametrize("H,KV,hd", [(28, 4, 128), (14, 2, 64)])
def test_prefill_full_size_2048(H, KV, hd):
    """Attention prefill at the 7B shape (28 q heads, 4 KV heads, hd 128) and the 0.5B shape (14, 2, hd 64), 2048
    tokens: every row equal to the row kernel's result, and 24 rows (first, last and random) equal to the oracle."""
    S, slot = 2048, 0
    case = make_case(2048, 1, slot, H, KV, hd, S, S, S, "small")
    cache, qq, sq, pos = to_dev(*case)
    out, obits = run_prefill(cache, qq, sq, pos, slot, S, H, KV, hd)
    ref = torch.zeros((S, H * hd), dtype=I64, device=DEV)
    refbits = torch.zeros((S, H), dtype=I32, device=DEV)
    ops.attention(qq, sq, cache, torch.zeros(S, dtype=I32, device=DEV), pos,
                  torch.tensor(exp_t(), dtype=I32, device=DEV), ref, H, KV, hd, O.inv_sqrt_hd(hd), refbits)
    assert np.array_equal(out, host(ref))
    assert np.array_equal(obits, host(refbits))
    rows = np.sort(np.concatenate([[0, 1, 31, 32, S - 1], np.random.default_rng(3).choice(S, 19, replace=False)]))
    assert np.array_equal(out[rows], oracle_rows(*case, slot, H, KV, rows))


@pytest.mark.parametrize("hd", [128, 64])
@pytest.mark.parametrize("change", ["swap", "steep", "tail"])
def test_prefill_with_unfit_exp_table_matches_row_kernel(change, hd):
    """An exp table outside the form the matrix-core path's float64 scores take (non-increasing, entries in
    [0, 2^24], steps below 2^24, T[0] > 0, zero from entry 4606 on) sends every block to the int64 scores: the
    result equals the row kernel's, which reads the table as the reference does, on the same table."""
    H, KV, nkeys, R, slot = 4, 2, 150, 150, 1
    case = make_case(11, 2, slot, H, KV, hd, 192, nkeys, R, "small")
    cache, qq, sq, pos = to_dev(*case)
    t = exp_t().astype(np.int64)
    if change == "swap":
        t[[40, 41]] = t[[41, 40]]
    elif change == "steep":
        t[0] = (1 << 24) + 3
    else:   # a nonzero entry past the 4606 entries the fast path keeps in LDS
        t[4700] = 1
    T = torch.tensor(t, dtype=I32, device=DEV)
    out = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    obits = torch.full((R, H), -1, dtype=I32, device=DEV)
    ws = ops.prefill_workspace(R, H, KV, hd, nkeys, DEV)
    ops.attention_prefill(qq, sq, cache, slot, pos, nkeys, T, out, H, KV, hd, O.inv_sqrt_hd(hd), ws, obits)
    ref = torch.zeros((R, H * hd), dtype=I64, device=DEV)
    refbits = torch.zeros((R, H), dtype=I32, device=DEV)
    ops.attention(qq, sq, cache, torch.full((R,), slot, dtype=I32, device=DEV), pos, T, ref, H, KV, hd,
                  O.inv_sqrt_hd(hd), refbits)
    assert np.array_equal(host(out), host(ref))
    assert np.array_equal(host(obits), host(refbits))


def test_attention_with_zero_exp_table_gives_zero_rows():
    """An exp table of zeros makes every softmax sum 0; numpy's int64 floor division by zero gives 0 (with a
    warning), so p = 0 and every output is 0. The kernels' divisions return 0 for a non-positive divisor rather
    than running a correction loop without end: the row kernel and the matrix-core prefill on the same case."""
    H, KV, hd, nkeys, R, slot = 4, 2, 128, 120, 120, 1
    case = make_case(5, 2, slot, H, KV, hd, 192, nkeys, R, "small")
    cache, qq, sq, pos = to_dev(*case)
    T = torch.zeros(len(exp_t()), dtype=I32, device=DEV)
    with np.errstate(divide="ignore"):
        assert (np.array([7], np.int64) << 20) // np.array([0], np.int64) == 0   # the reference's numpy behaviour
    out = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    obits = torch.full((R, H), -1, dtype=I32, device=DEV)
    ops.attention(qq, sq, cache, torch.full((R,), slot, dtype=I32, device=DEV), pos, T, out, H, KV, hd,
                  O.inv_sqrt_hd(hd), obits)
    assert not host(out).any() and not host(obits).any()
    out2 = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    ws = ops.prefill_workspace(R, H, KV, hd, nkeys, DEV)
    ops.attention_prefill(qq, sq, cache, slot, pos, nkeys, T, out2, H, KV, hd, O.inv_sqrt_hd(hd), ws, obits)
    assert not host(out2).any() and not host(obits).any()


@pytest.mark.parametrize("H,KV,hd,R,bias,Smax", [(28, 4, 128, 1, True, 96), (28, 4, 128, 4, False, 96),
                                                 (14, 2, 64, 3, True, 96), (4, 4, 256, 2, True, 96),
                                                 (8, 2, 128, 2, True, 8192), (16, 16, 128, 1, False, 300),
                                                 (40, 8, 128, 1, True, 200), (14, 2, 64, 2, True, 300),
                                                 (4, 4, 256, 1, True, 400), (28, 4, 128, 10, True, 96),
                                                 (28, 4, 128, 3, True, 500), (16, 16, 128, 2, True, 512),
                                                 (40, 8, 128, 8, True, 200), (14, 2, 64, 20, False, 256)])
@pytest.mark.parametrize("obn", [1, 2, 4])
def test_fused_qkv_attention_matches_two_launches(H, KV, hd, R, bias, Smax, obn):
    """exact_attention_qkv (obn = 1) and exact_attention_qkv_split (obn = 2, 4: each head's p.V over up to obn
    blocks) against exact_qkv_rope_cache + exact_attention (both oracle-pinned above and in the model tests):
    outputs and every cache entry equal; the max of a head's obn bit lengths is its obits, and entry i bounds the
    bit length of the head's i-th slice of hd / obn dimensions; rows in different slots at positions 0, Smax - 1
    and in between; the totals t are left unchanged."""
    from exact_amd.tables import host_tables
    rng = np.random.default_rng(H + R + hd)
    B = R + 2
    N = (H + 2 * KV) * hd
    kq = rng.integers(-32767, 32768, (B, KV, Smax, hd))
    sk = rng.integers(0, 4, (B, KV, Smax))
    v = rng.integers(-(1 << 29), 1 << 29, (B, KV, Smax, hd))
    slot = rng.permutation(B)[:R]
    pos = rng.integers(1, Smax - 1, R)
    pos[0] = 0
    if R > 1:
        pos[1] = Smax - 1
    t = rng.integers(-(1 << 44), 1 << 44, (R, N))
    s = rng.integers(0, 12, R)
    b = rng.integers(-(1 << 20), 1 << 20, N) if bias else None
    tabs = host_tables(Smax, hd, 1e6)
    d = lambda a, dt: torch.tensor(np.ascontiguousarray(a), dtype=dt, device=DEV)
    cos, sin, expt = d(tabs["cos"], I64), d(tabs["sin"], I64), d(exp_t(), I32)
    args = dict(H=H, KV=KV, hd=hd)
    inv = O.inv_sqrt_hd(hd)
    c_a = (d(kq, I16), d(sk, I32), d(v, I64))
    c_b = tuple(x.clone() for x in c_a)
    t_a, t_b = d(t, I64), d(t, I64)
    s_d, b_d, slot_d, pos_d = d(s, I32), None if b is None else d(b, I64), d(slot, I32), d(pos, I32)
    qq, sq = torch.empty((R, H * hd), dtype=I16, device=DEV), torch.empty((R, H), dtype=I32, device=DEV)
    out_a = torch.full((R, H * hd), -7, dtype=I64, device=DEV)
    out_b = torch.full((R, H * hd), -9, dtype=I64, device=DEV)
    ob_a = torch.full((R, H), -1, dtype=I32, device=DEV)
    ob_b = torch.full((R, H * obn), -2, dtype=I32, device=DEV)
    ops.qkv_rope_cache(t_a, s_d, b_d, cos, sin, slot_d, pos_d, c_a, qq, sq, clear=False, **args)
    ops.attention(qq, sq, c_a, slot_d, pos_d, expt, out_a, inv=inv, obits=ob_a, **args)
    ops.attention_qkv(t_b, s_d, b_d, cos, sin, slot_d, pos_d, c_b, expt, out_b, inv=inv, obits=ob_b, obn=obn, **args)
    assert np.array_equal(host(out_b), host(out_a))
    ob = host(ob_b).reshape(R, H, obn)
    assert np.array_equal(ob.max(-1), host(ob_a))
    slice_bits = np.vectorize(lambda m: int(m).bit_length())(np.abs(host(out_a)).reshape(R, H, obn, -1).max(-1))
    assert (ob >= slice_bits).all()
    for x, y in zip(c_b, c_a):
        assert np.array_equal(host(x), host(y))
    assert np.array_equal(host(t_b), t)


def test_row_attention_long_context_matches_oracle():
    """Decode attention over 8000 cached keys of an 8192-position cache (64 KiB of scores in LDS) against the oracle."""
    H, KV, hd, Smax, slot, nkeys = 4, 2, 128, 8192, 1, 8000
    kq, sk, v, qq, sq, pos = make_case(91, 2, slot, H, KV, hd, Smax, nkeys, 1, "small")
    cache, qd, sqd, posd = to_dev(kq, sk, v, qq, sq, pos)
    out = torch.full((1, H * hd), -7, dtype=I64, device=DEV)
    ops.attention(qd, sqd, cache, torch.tensor([slot], dtype=I32, device=DEV), posd,
                  torch.tensor(exp_t(), dtype=I32, device=DEV), out, H, KV, hd, O.inv_sqrt_hd(hd))
    assert np.array_equal(host(out), oracle_rows(kq, sk, v, qq, sq, pos, slot, H, KV, [0]))
