#!/usr/bin/env python3
"""Generates the main loop of the exact group-128 int8 prefill GEMM as one inline-asm block (gfx950).

    t[m][n] = sum_g M[g][n] * sum_{k in g} x[m][k] * W[n][k]        (SPEC.md:18; GQLin, speed_fair_kaggle.py:714-725)

Output: a C++ header with `gemm_asm_main_<variant>(...)`, a __device__ function whose body is a single `asm volatile`
statement. The kernel in gemm.hip computes every per-lane and per-wave value, passes them in pinned registers, and
calls it last; the block runs its whole K loop and stores its tile inside the asm.

Why assembly: the loop's matrix work (v_mfma_i32_16x16x64_i8) needs its operand fragments read from LDS well ahead
and an exact int64 multiply-add per output per group on the vector ALUs; the compiler's schedule waits for every
outstanding LDS read before each group and cannot keep a second fragment set live at this register pressure. Here
every register is fixed and every wait is exact.

Block: 512 threads = 8 waves (2 per SIMD), tile 256 rows x 128 columns; wave (wm = wave >> 1, wn = wave & 1) owns
rows 64 wm .. + 63 and packed weight tile nb0 + wn (64 columns). Per 128-wide group a wave runs 16 sub-tiles of
16 x 16 (4 row sub-tiles rs x 4 column sub-tiles cs), each a chain of two MFMAs over the group's two 64-k halves.
Lane l = 16 q + j holds, in sub-tile (rs, cs), rows 16 rs + 4 q + i (i = 0..3) of column 4 j + cs (columns are
permuted within the tile so that a lane's four columns are adjacent: its four scales are one 8-byte LDS read and its
outputs of one row are 32 contiguous bytes).

Stages: three LDS stages (group g in stage g mod 3 of the unrolled body). Group g + 3 is copied (buffer_load ... lds)
into stage g mod 3 once every wave has read its last fragment of group g: one barrier per group, after the 12th of its
32 MFMAs, which also waits for group g + 1's copies; the copies are issued one per MFMA after it. The 16 sub-tiles
run as 8 pairs of chains in 2 x 2 blocks, (rs, cs pair) = (0,0) (1,0) (0,1) (1,1) (2,0) (3,0) (2,1) (3,1), so that
every fragment is read 13 to 17 MFMAs before its first use: A sub-tiles 2, 3 of group g at its start (from stage g),
then, after the barrier, group g + 1's B columns 0, 1, its A sub-tiles 0, 1, its B columns 2, 3 (into the half its
predecessor's columns 0, 1 leave) and its scales. The rescale of a pair of chains runs two pairs after its MFMAs (no
MFMA -> VALU stall, far past the hazard distance). The body is unrolled over six groups (three stages x the B halves'
rotation); the last iteration is a separate copy without copies past the last group, so the loop has no branches.

Registers (VGPR):
  v0..v127     int64 totals T(rs, i, cs)  (PAIRS: v0..v63, T(rs, jp, cs) for the digit-row pair jp of a lane)
  v128..v175   B fragments: three halves, each 2 cs x 2 k halves (group g: columns 0, 1 in half 2g mod 3, 2, 3 in
               half 2g + 1 mod 3)
  v176..v207   A fragments: one buffer per row sub-tile x 2 k halves
  v208..v231   chain results, three pair slots x 2 chains x 4
  v232..v233   packed int16 scales of the incoming group; v234..v237 the scales in use (one per cs)
  v238..v243   copy offsets (A: 4 segments, B, scales)
  v244..v249   LDS read bases (A: stage group lo/hi x k half; B; scales)
  v250         output offset; v251, v252 the lane's first row and column; v253 temporary
Usage: python3 gen_gemm_asm.py > gemm_asm.inc
"""
import sys

# ---- fixed layout ---------------------------------------------------------------------------------------------------
A_STAGE = (0, 32768, 120832)                # A region of each stage (32 KiB: 256 rows x 128 bytes)
B_BASE, B_STAGE = 65536, 16384              # B regions: 2 packed tiles x 8 KiB per stage
M_BASE, M_STAGE = 114688, 2048              # scales: one 256-byte copy per wave per stage
LDS_BYTES = 153600
DPG = 7                                     # copies per wave per group: 4 A + 2 B + 1 scales

V_B, V_A, V_C, V_MP, V_MX = 128, 176, 208, 232, 234
V_ADMA, V_BDMA, V_MDMA = 238, 242, 243
V_ARD, V_BRD, V_MRD = 244, 248, 249
V_ST, V_ROW, V_COL, V_TMP = 250, 251, 252, 253

# scalar registers owned by the asm (s60..s95)
S = dict(iter=60, gd=61, g1=62, asoff=63, bg=64, bc0=65, bc1=66, mg=67, nbsb=68, nbsm=69, wavea=70, waveb=71,
         wavem=72, t0=73, t1=74, n8=75, dummy=76, mr=78, mc=80)   # dummy, mr: pairs; mc: 4 pairs (80..87)


def T(rs, i, cs, pairs):
    return 2 * ((rs * (2 if pairs else 4) + i) * 4 + cs)


def Bv(half, cs, kh):
    return V_B + 16 * half + 4 * ((cs % 2) * 2 + kh)


def Av(rs, kh):
    return V_A + 8 * rs + 4 * kh


PAIR_ORDER = [(0, 0), (1, 0), (0, 1), (1, 1), (2, 0), (3, 0), (2, 1), (3, 1)]   # (rs, cs pair)


def bhalf(k, cp):
    """B half of columns 2 cp, 2 cp + 1 for the group with local index k"""
    return (2 * k + cp) % 3


def Cv(slot, c):
    return V_C + 4 * (slot * 2 + c)


def vr(a, n=1):
    return f"v{a}" if n == 1 else f"v[{a}:{a + n - 1}]"


def s(name, n=1):
    a = S[name]
    return f"s{a}" if n == 1 else f"s[{a}:{a + n - 1}]"


class Emit:
    """Instruction stream with a model of the in-order LDS read queue (lgkmcnt)."""

    def __init__(self):
        self.lines = []
        self.fifo = []        # outstanding LDS reads, oldest first: set of VGPRs each one writes

    def __call__(self, line):
        self.lines.append(line)

    def label(self, name):
        self.lines.append(f"{name}:")

    def ds_read(self, op, dst, nregs, addr, off):
        self(f"{op} {vr(dst, nregs)}, {vr(addr)} offset:{off}")
        self.fifo.append(set(range(dst, dst + nregs)))

    def need(self, regs):
        """wait until no outstanding LDS read writes any of regs"""
        last = -1
        for k, w in enumerate(self.fifo):
            if w & regs:
                last = k
        if last < 0:
            return
        n = len(self.fifo) - 1 - last
        assert n <= 15
        self(f"s_waitcnt lgkmcnt({n})")
        self.fifo = self.fifo[last + 1:]

    def drain(self):
        self("s_waitcnt lgkmcnt(0)")
        self.fifo = []


def dma_ops(st):
    """copies of group s_gd into stage st, as 7 items of (SALU set-up, copy); every wave copies 4 A segments, 2 B
    segments and its scales. The M0 write and the copy are placed around other instructions (one wait state)."""
    items = []
    for i in range(4):
        items.append(([f"s_add_u32 m0, {s('wavea')}, {A_STAGE[st] + i * 1024}"],
                      f"buffer_load_dwordx4 {vr(V_ADMA + i)}, %[rA], {s('asoff')} offen lds"))
    for i in range(2):
        tmp = s('t0') if i == 0 else s('t1')
        items.append(([f"s_add_u32 {tmp}, {s('bg')}, {s('bc0') if i == 0 else s('bc1')}",
                       f"s_add_u32 m0, {s('waveb')}, {st * B_STAGE + i * 1024}"],
                      f"buffer_load_dwordx4 {vr(V_BDMA)}, %[rB], {tmp} offen lds"))
    items.append(([f"s_add_u32 m0, {s('wavem')}, {st * M_STAGE}"],
                  f"buffer_load_dword {vr(V_MDMA)}, %[rM], {s('mg')} offen lds"))
    return items


def dma(e, st, pairs):
    """all copies of group s_gd into stage st, back to back (prologue)"""
    for setup, load in dma_ops(st):
        for ln in setup:
            e(ln)
        e("s_nop 0")
        e(load)


def dma_advance(e):
    e(f"s_add_u32 {s('gd')}, {s('gd')}, 1")
    e(f"s_add_u32 {s('asoff')}, {s('asoff')}, 128")
    e(f"s_add_u32 {s('bg')}, {s('bg')}, {s('nbsb')}")
    e(f"s_add_u32 {s('mg')}, {s('mg')}, {s('nbsm')}")


def a_addr(st, kh):
    hi = 1 if st == 2 else 0
    return V_ARD + 2 * hi + kh, (0 if st == 2 else A_STAGE[st])


def read_a(e, rs, st, kh):
    base, off = a_addr(st, kh)
    e.ds_read("ds_read_b128", Av(rs, kh), 4, base, off + rs * 2048)


def read_b(e, half, cs, st, kh):
    e.ds_read("ds_read_b128", Bv(half, cs, kh), 4, V_BRD, st * B_STAGE + kh * 4096 + cs * 256)


def read_m(e, st):
    e.ds_read("ds_read_b64", V_MP, 2, V_MRD, st * M_STAGE)


def extract_scales(e):
    e.need({V_MP, V_MP + 1})
    e(f"v_and_b32 {vr(V_MX)}, 0xffff, {vr(V_MP)}")
    e(f"v_lshrrev_b32 {vr(V_MX + 1)}, 16, {vr(V_MP)}")
    e(f"v_and_b32 {vr(V_MX + 2)}, 0xffff, {vr(V_MP + 1)}")
    e(f"v_lshrrev_b32 {vr(V_MX + 3)}, 16, {vr(V_MP + 1)}")


def rescale_ops(pair, slot, pairs):
    """VALU instructions that add the pair's two chains into the totals (8 instructions, 2 chains x 4)"""
    rs, cp = PAIR_ORDER[pair]
    ops = []
    for c in range(2):
        cs = 2 * cp + c
        cr = Cv(slot, c)
        if pairs:
            # digit rows 4q + 2jp (hi) and 4q + 2jp + 1 (lo) of one activation row: 256 hi + lo per group
            for jp in range(2):
                tmp = 64 + jp   # the totals take v0..v63 here, so v64.. are free
                ops.append(f"v_lshl_add_u32 {vr(tmp)}, {vr(cr + 2 * jp)}, 8, {vr(cr + 2 * jp + 1)}")
                t = T(rs, jp, cs, True)
                ops.append(f"v_mad_i64_i32 {vr(t, 2)}, {s('dummy', 2)}, {vr(tmp)}, {vr(V_MX + cs)}, {vr(t, 2)}")
        else:
            for i in range(4):
                t = T(rs, i, cs, False)
                ops.append(f"v_mad_i64_i32 {vr(t, 2)}, {s('dummy', 2)}, {vr(cr + i)}, {vr(V_MX + cs)}, {vr(t, 2)}")
    return ops


def mfma(e, dst, a, b, acc):
    e.need({a, b})
    src_c = vr(dst, 4) if acc else "0"
    e(f"v_mfma_i32_16x16x64_i8 {vr(dst, 4)}, {vr(a, 4)}, {vr(b, 4)}, {src_c}")


X_AT = 12          # the group's barrier comes before its MFMA X_AT


def group(e, k, pairs, final, tag):
    """group with local index k of the unrolled body (stage k % 3, chain slots (8 k + p) % 3). final: the last
    iteration, whose groups 3, 4, 5 are the block's last three (no copies past them; the last two wait for all)"""
    st, st1 = k % 3, (k + 1) % 3
    # per MFMA m: LDS reads and copy items placed after it
    after = {m: [] for m in range(32)}
    # this group's A sub-tiles 2, 3 (stage g)
    for kh in range(2):
        after[kh].append(("ra", 2, st, kh))
        after[2 + kh].append(("ra", 3, st, kh))
    # after the barrier: group g + 1's B columns 0, 1 with the copies, its A sub-tiles 0, 1, its B columns 2, 3, scales
    copies = not (final and k >= 3)
    for n in range(4):
        after[X_AT + n].append(("rb", bhalf(k + 1, 0), n // 2, st1, n % 2))
    if copies:
        for n in range(7):
            after[X_AT + n].append(("dma", n))
    for kh in range(2):
        after[16 + kh].append(("ra", 0, st1, kh))
        after[18 + kh].append(("ra", 1, st1, kh))
    for n in range(4):
        after[24 + n].append(("rb", bhalf(k + 1, 1), 2 + n // 2, st1, n % 2))
    after[28].append(("rm", st1))
    items = dma_ops(st)
    pending_load = None
    for p in range(8):
        rs, cp = PAIR_ORDER[p]
        slot = (8 * k + p) % 3
        if p == 2:
            extract_scales(e)
        ops = rescale_ops((p - 2) % 8, (8 * k + p - 2) % 3, pairs)
        seq = [(0, 0), (1, 0), (0, 1), (1, 1)]   # (chain, k half)
        for n, (c, kh) in enumerate(seq):
            m = 4 * p + n
            if m == X_AT:
                e.drain()
                if final and k >= 4:
                    e("s_waitcnt vmcnt(0)")          # g + 2 was never copied
                else:
                    e(f"s_waitcnt vmcnt({DPG})")     # group g + 1 landed; g + 2 may stay in flight
                e("s_barrier")
            mfma(e, Cv(slot, c), Av(rs, kh), Bv(bhalf(k, cp), 2 * cp + c, kh), kh == 1)
            for ev in after[m]:
                if ev[0] == "dma":
                    setup, load = items[ev[1]]
                    for ln in setup:
                        e(ln)
                    pending_load = load
            e(ops[2 * n])
            if pending_load:                       # at least one wait state after the M0 write
                e(pending_load)
                pending_load = None
            e(ops[2 * n + 1])
            for ev in after[m]:
                if ev[0] == "ra":
                    read_a(e, ev[1], ev[2], ev[3])
                elif ev[0] == "rb":
                    read_b(e, ev[1], ev[2], ev[3], ev[4])
                elif ev[0] == "rm":
                    read_m(e, ev[1])
            if m == X_AT + 7:
                dma_advance(e)


def prologue_reads(e, k):
    """fragments of the first group (local index k) that its predecessor would have read"""
    st = k % 3
    for n in range(4):
        read_b(e, bhalf(k, 0), n // 2, st, n % 2)
    for kh in range(2):
        read_a(e, 0, st, kh)
        read_a(e, 1, st, kh)
    for n in range(4):
        read_b(e, bhalf(k, 1), 2 + n // 2, st, n % 2)
    read_m(e, st)


def store_full(e, pairs):
    rows = 2 if pairs else 4
    for rs in range(4):
        for i in range(rows):
            r = rs * (8 if pairs else 16) + i
            e(f"s_mul_i32 {s('t0')}, {s('n8')}, {r}")
            for cp in range(2):
                t = T(rs, i, 2 * cp, pairs)
                e(f"buffer_store_dwordx4 {vr(t, 4)}, {vr(V_ST)}, %[rT], {s('t0')} offen offset:{16 * cp}")


def store_masked(e, pairs):
    rows = 2 if pairs else 4
    for cs in range(4):
        e(f"v_add_u32 {vr(V_TMP)}, {cs}, {vr(V_COL)}")
        e(f"v_cmp_gt_i32 s[{S['mc'] + 2 * cs}:{S['mc'] + 2 * cs + 1}], %[N], {vr(V_TMP)}")
    for rs in range(4):
        for i in range(rows):
            r = rs * (8 if pairs else 16) + i
            e(f"v_add_u32 {vr(V_TMP)}, {r}, {vr(V_ROW)}")
            e(f"v_cmp_gt_i32 {s('mr', 2)}, %[M], {vr(V_TMP)}")
            e(f"s_mul_i32 {s('t0')}, {s('n8')}, {r}")
            e("s_nop 4")
            for cs in range(4):
                e(f"s_and_b64 exec, {s('mr', 2)}, s[{S['mc'] + 2 * cs}:{S['mc'] + 2 * cs + 1}]")
                e("s_nop 1")
                e(f"buffer_store_dwordx2 {vr(T(rs, i, cs, pairs), 2)}, {vr(V_ST)}, %[rT], {s('t0')} offen offset:{8 * cs}")
            e("s_mov_b64 exec, -1")


def add_colterm(e):
    """PAIRS: t += 128 * colterm[col] for the lane's four columns (loaded into the free A buffers)"""
    e(f"buffer_load_dwordx4 {vr(V_A, 4)}, {vr(V_TMP)}, %[rCt], 0 offen")
    e(f"buffer_load_dwordx4 {vr(V_A + 4, 4)}, {vr(V_TMP)}, %[rCt], 0 offen offset:16")
    e("s_waitcnt vmcnt(0)")
    for cs in range(4):
        ct = V_A + 2 * cs
        e(f"v_lshlrev_b64 {vr(ct, 2)}, 7, {vr(ct, 2)}")
    for rs in range(4):
        for jp in range(2):
            for cs in range(4):
                t, ct = T(rs, jp, cs, True), V_A + 2 * cs
                e(f"v_add_co_u32 {vr(t)}, vcc, {vr(t)}, {vr(ct)}")
                e(f"v_addc_co_u32 {vr(t + 1)}, vcc, {vr(t + 1)}, {vr(ct + 1)}, vcc")


def kernel_asm(pairs):
    e = Emit()
    tag = "P" if pairs else "A"
    L = lambda n: f".Lg{tag}_{n}"
    ntot = 64 if pairs else 128
    e("s_waitcnt vmcnt(0) lgkmcnt(0)")   # nothing of the compiler's own is outstanding in the counters used below
    # totals, chain results and scales in use start at zero (the first two rescales add zero)
    for a in range(0, ntot, 2):
        e(f"v_mov_b64 {vr(a, 2)}, 0")
    for a in range(V_C, V_C + 24, 2):
        e(f"v_mov_b64 {vr(a, 2)}, 0")
    e(f"v_mov_b64 {vr(V_MX, 2)}, 0")
    e(f"v_mov_b64 {vr(V_MX + 2, 2)}, 0")
    e(f"s_mov_b32 {s('g1')}, %[g1]")
    e(f"s_mov_b32 {s('gd')}, %[g0]")
    for nm in ("asoff", "bg", "bc0", "bc1", "mg", "nbsb", "nbsm", "wavea", "waveb", "wavem", "n8"):
        e(f"s_mov_b32 {s(nm)}, %[{nm}]")
    e(f"s_mov_b32 {s('iter')}, %[iters]")
    # entry phase k0 = 6 * iters - (g1 - g0): the first group runs as local index k0, so the last one is index 5
    for k0 in range(6):
        e(f"s_cmp_eq_u32 %[phase], {k0}")
        e(f"s_cbranch_scc1 {L(f'pro{k0}')}")
    e(f"s_branch {L('pro0')}")
    for k0 in range(6):
        e.label(L(f"pro{k0}"))
        e.fifo = []
        # copies of the first three groups into stages k0, k0 + 1, k0 + 2 (groups past g1 are not copied)
        for n in range(3):
            e(f"s_cmp_lt_u32 {s('gd')}, {s('g1')}")
            e(f"s_cbranch_scc0 {L(f'pro{k0}_n{n}')}")
            dma(e, (k0 + n) % 3, pairs)
            e.label(L(f"pro{k0}_n{n}"))
            dma_advance(e)
        # wait for the first group's copies: min(groups, 3) - 1 groups may stay in flight
        e(f"s_sub_u32 {s('t0')}, {s('g1')}, %[g0]")
        e(f"s_cmp_ge_u32 {s('t0')}, 3")
        e(f"s_cbranch_scc1 {L(f'pro{k0}_w3')}")
        e(f"s_cmp_eq_u32 {s('t0')}, 2")
        e(f"s_cbranch_scc1 {L(f'pro{k0}_w2')}")
        e("s_waitcnt vmcnt(0)")
        e(f"s_branch {L(f'pro{k0}_w')}")
        e.label(L(f"pro{k0}_w2"))
        e(f"s_waitcnt vmcnt({DPG})")
        e(f"s_branch {L(f'pro{k0}_w')}")
        e.label(L(f"pro{k0}_w3"))
        e(f"s_waitcnt vmcnt({2 * DPG})")
        e.label(L(f"pro{k0}_w"))
        e("s_barrier")
        prologue_reads(e, k0)
        e.drain()
        e(f"s_cmp_gt_u32 {s('iter')}, 1")
        e(f"s_cbranch_scc1 {L(f's{k0}')}")
        e(f"s_branch {L(f'f{k0}')}")
    # steady body (every group copies group g + 3 and keeps g + 2 in flight) and the last iteration's body. The LDS
    # queue model starts from the state a previous group leaves (every group issues the same reads in the same order).
    e_probe = Emit()
    for k in range(6):
        group(e_probe, k, pairs, False, f"{L('probe')}{k}")
    steady_fifo = list(e_probe.fifo)
    e.fifo = list(steady_fifo)
    e.label(L("loop"))
    for k in range(6):
        e.label(L(f"s{k}"))
        group(e, k, pairs, False, f"{L('s')}{k}")
    e(f"s_sub_u32 {s('iter')}, {s('iter')}, 1")
    e(f"s_cmp_gt_u32 {s('iter')}, 1")
    e(f"s_cbranch_scc1 {L('loop')}")
    e.fifo = list(steady_fifo)
    for k in range(6):
        e.label(L(f"f{k}"))
        group(e, k, pairs, True, f"{L('f')}{k}")
    # drain: the last group's pairs 6 and 7 (local index 5: chain slots (40 + 6) % 3, (40 + 7) % 3)
    e("s_nop 7")
    e("s_nop 7")
    for op in rescale_ops(6, (8 * 5 + 6) % 3, pairs) + rescale_ops(7, (8 * 5 + 7) % 3, pairs):
        e(op)
    e.drain()
    e("s_waitcnt vmcnt(0)")
    if pairs:
        e(f"v_mov_b32 {vr(V_TMP)}, %[ctoff]")
        add_colterm(e)
    e(f"s_cmp_eq_u32 %[full], 1")
    e(f"s_cbranch_scc0 {L('masked')}")
    store_full(e, pairs)
    e(f"s_branch {L('end')}")
    e.label(L("masked"))
    store_masked(e, pairs)
    e.label(L("end"))
    e("s_waitcnt vmcnt(0)")
    return e.lines


def emit_function(name, pairs):
    lines = kernel_asm(pairs)
    body = "\n".join(f'      "{ln}\\n"' for ln in lines)
    clob_v = [f'"v{i}"' for i in range(0, V_ADMA)] + [f'"v{V_TMP}"']
    clob_s = [f'"s{i}"' for i in range(60, 96)]
    ins = ["[g0] \"s\"(g0)", "[g1] \"s\"(g1)", "[iters] \"s\"(iters)", "[phase] \"s\"(phase)", "[full] \"s\"(full)",
           "[asoff] \"s\"(asoff)", "[bg] \"s\"(bg)", "[bc0] \"s\"(bc0)", "[bc1] \"s\"(bc1)", "[mg] \"s\"(mg)",
           "[nbsb] \"s\"(nbsb)", "[nbsm] \"s\"(nbsm)", "[wavea] \"s\"(wavea)", "[waveb] \"s\"(waveb)",
           "[wavem] \"s\"(wavem)", "[n8] \"s\"(n8)", "[M] \"s\"(M)", "[N] \"s\"(N)",
           "[rA] \"s\"(rA)", "[rB] \"s\"(rB)", "[rM] \"s\"(rM)", "[rT] \"s\"(rT)"]
    if pairs:
        ins += ["[rCt] \"s\"(rCt)", "[ctoff] \"v\"(ctoff)"]
    params = ("int g0, int g1, int iters, int phase, int full, int asoff, int bg, int bc0, int bc1, int mg, int nbsb, "
              "int nbsm, int wavea, int waveb, int wavem, int n8, int M, int N, __amdgpu_buffer_rsrc_t rA, "
              "__amdgpu_buffer_rsrc_t rB, __amdgpu_buffer_rsrc_t rM, __amdgpu_buffer_rsrc_t rT, int vadma0, "
              "int vadma1, int vadma2, int vadma3, int vbdma, int vmdma, int vard0, int vard1, int vard2, int vard3, "
              "int vbrd, int vmrd, int vst, int vrow, int vcol")
    if pairs:
        params += ", __amdgpu_buffer_rsrc_t rCt, int ctoff"
    pinned = [("vadma0", V_ADMA), ("vadma1", V_ADMA + 1), ("vadma2", V_ADMA + 2), ("vadma3", V_ADMA + 3),
              ("vbdma", V_BDMA), ("vmdma", V_MDMA), ("vard0", V_ARD), ("vard1", V_ARD + 1), ("vard2", V_ARD + 2),
              ("vard3", V_ARD + 3), ("vbrd", V_BRD), ("vmrd", V_MRD), ("vst", V_ST), ("vrow", V_ROW), ("vcol", V_COL)]
    outs = ", ".join(f'"+{{v{r}}}"({n})' for n, r in pinned)
    return f"""
// {name}: {'A16 as digit-row pairs (rows 2r = x >> 8, 2r + 1 = (x & 255) - 128; 256 hi + lo per group)' if pairs else 'A8'}
__device__ __forceinline__ void {name}({params}) {{
  asm volatile(
{body}
      : {outs}
      : {", ".join(ins)}
      : {", ".join(clob_v)}, {", ".join(clob_s)}, "vcc", "scc", "memory");
}}
"""


def main():
    out = ["// Generated by gen_gemm_asm.py; do not edit. The main loop and stores of k_gemm_asm (gemm.hip).",
           "#pragma once",
           f"#define GEMM_ASM_LDS_BYTES {LDS_BYTES}",
           f"#define GEMM_ASM_B_BASE {B_BASE}",
           f"#define GEMM_ASM_M_BASE {M_BASE}",
           f"#define GEMM_ASM_A_HI {A_STAGE[2]}"]
    out.append(emit_function("gemm_asm_main_a8", False))
    out.append(emit_function("gemm_asm_main_pairs", True))
    sys.stdout.write("\n".join(out) + "\n")


if __name__ == "__main__":
    main()
