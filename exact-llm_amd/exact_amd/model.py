"""Device model: the exact integer forward pass on one MI355X, driven from Python through the C ABI.

Mirrors the reference's torch twin and speed engine:
  TModel.forward(ids, cache, last_only) / new_cache()      exact_torch.py:126-193
  GraphDecoder(model).load_prefix / capture / step(token)   experiments/speed_fair_kaggle.py:590-645
with the layer order of IntModel.__call__ (exact_llm.py:161-180):
  x = emb[ids]; per layer: a = irms(x, g1); q, k, v = linears(a); RoPE; per-head integer attention;
  x += o(att); m = irms(x, g2); x += down(shr(isilu(gate(m)) * up(m), 16)); logits = head(irms(x, gf)).
Every step runs in hand-written HIP kernels (libexact_hip.so); Python only allocates buffers and
sequences launches on the current stream, so a whole decode step can be captured in a HIP graph.
"""
import collections
import hashlib
import operator

import numpy as np
import torch

from . import ops, synth
from .ops import I8, I16, I32, I64, PackedLinear, ExactError
from .tables import DeviceTables
from .trace import TraceLayout, TraceRecorder


def _lin_keys(seed, name):
    return synth.key(seed, name + ".w"), synth.key(seed, name + ".m"), synth.key(seed, name + ".b")


class DeviceWeights:
    """Packed device weights of one model. Layers hold fused q|k|v and gate|up linears (group mode) so
    a decode step issues one GEMV per fused linear; per-channel models keep separate linears."""

    def __init__(self, cfg, device):
        self.cfg, self.device = cfg, device
        self.layers = []
        self.mode = "group"
        self.tables = None   # host integer tables shipped with the weights (an artifact's), else built

    # -- seeded synthetic model generated on the device
    @classmethod
    def synthetic(cls, cfg, seed, device, layers=None):
        self = cls(cfg, device)
        thr = torch.tensor(synth.thresholds().astype(np.int64), dtype=I64).to(torch.int32).to(device)
        if any(n % 64 for n in ((cfg.MI, cfg.SI) if cfg.moe else (cfg.I,))):
            raise ExactError("fused gate|up linears need intermediate sizes that are multiples of 64")
        D, H, KV, hd = cfg.D, cfg.H, cfg.KV, cfg.hd
        nl = cfg.NL if layers is None else layers

        def fused(parts, K, bias):
            # each part starts on a 64-row boundary of the packed buffer (and of the output row)
            offs, N = [], 0
            for _, n in parts:
                offs.append(N)
                N = offs[-1] + n if len(offs) == len(parts) else -(-(offs[-1] + n) // 64) * 64
            wp, mp = PackedLinear.alloc(N, K, device)
            bs = []
            for (name, n), off in zip(parts, offs):
                kw, km, kb = _lin_keys(seed, name)
                ops.synth_linear(wp, mp, n, K, kw, km, synth.M_LO, synth.M_HI, thr, n_off=off, Ntot=N)
                if bias:
                    bs.append(ops.synth_vector(kb, synth.BIAS[0], synth.BIAS[1], n, device))
            b = torch.cat(bs) if bias else None
            if bias and N != sum(n for _, n in parts):
                raise ExactError("biased fused linears need 64-row aligned parts")
            return PackedLinear(wp, mp, N, K, b, parts=[(name.split(".")[-1], off, n) for (name, n), off in zip(parts, offs)])

        for li in range(nl):
            L = dict(
                g1=ops.synth_vector(synth.key(seed, f"L{li}.g1"), *synth.GAIN, D, device),
                g2=ops.synth_vector(synth.key(seed, f"L{li}.g2"), *synth.GAIN, D, device),
                qkv=fused([(f"L{li}.q", H * hd), (f"L{li}.k", KV * hd), (f"L{li}.v", KV * hd)], D, True),
                o=fused([(f"L{li}.o", D)], H * hd, False))
            if cfg.moe:
                # router logits and the shared expert's gate logit in one GEMV (gate at column gate_col)
                L["router"] = fused([(f"L{li}.router", cfg.NE), (f"L{li}.sgate", 1)], D, False)
                # experts: gate|up (2 MI x D) and down (D x MI) of all NE experts, each in one allocation
                egu = ops.ExpertLinears(cfg.NE, 2 * cfg.MI, D, device)
                edn = ops.ExpertLinears(cfg.NE, D, cfg.MI, device)
                for e in range(cfg.NE):
                    wp, mp = egu.part(e)
                    for name, off in ((f"L{li}.e{e}.gate", 0), (f"L{li}.e{e}.up", cfg.MI)):
                        kw, km, _ = _lin_keys(seed, name)
                        ops.synth_linear(wp, mp, cfg.MI, D, kw, km, synth.M_LO, synth.M_HI, thr, n_off=off,
                                         Ntot=2 * cfg.MI)
                    wp, mp = edn.part(e)
                    kw, km, _ = _lin_keys(seed, f"L{li}.e{e}.down")
                    ops.synth_linear(wp, mp, D, cfg.MI, kw, km, synth.M_LO, synth.M_HI, thr)
                L["egu"], L["edown"] = egu, edn
                L["sgu"] = fused([(f"L{li}.sg", cfg.SI), (f"L{li}.su", cfg.SI)], D, False)
                L["sd"] = fused([(f"L{li}.sd", D)], cfg.SI, False)
            else:
                L["gateup"] = fused([(f"L{li}.gate", cfg.I), (f"L{li}.up", cfg.I)], D, False)
                L["down"] = fused([(f"L{li}.down", D)], cfg.I, False)
            self.layers.append(L)
        self.gf = ops.synth_vector(synth.key(seed, "gf"), *synth.GAIN, D, device)
        emb = fused([("emb", cfg.V)], D, False)
        self.emb = ops.embed_table(emb, cfg.V, D)
        self.head = emb if cfg.tie else fused([("head", cfg.V)], D, False)
        return self

    # -- from integer arrays in the oracle's layout (w (K, N) int8; group M (G, N) or channel M (N,))
    @classmethod
    def from_arrays(cls, cfg, arrays, device, mode="group", tables=None):
        """arrays: emb (V, D) Q16, gf, head.w / head.M (/ head.b), and per layer i: f'{i}.g1', f'{i}.g2',
        f'{i}.{name}.w' / '.M' / '.b' for name in q, k, v, o, gate, up, down. Group mode fuses q|k|v and
        gate|up into one packed linear each (parts adjacent, in that order), as the decode step expects;
        channel mode keeps them separate. tables: optional host integer tables (exp, silu, sig, cos, sin) that
        the model then uses instead of building its own (an artifact's shipped tables)."""
        if cfg.moe:
            raise ExactError("integer arrays of MoE models are not supported; use DeviceWeights.synthetic")
        self = cls(cfg, device)
        self.mode = mode
        self.tables = tables

        def group_lin(pfxs):
            ws = [np.asarray(arrays[p + ".w"]) for p in pfxs]
            Ms = [np.asarray(arrays[p + ".M"], np.int64) for p in pfxs]
            K = ws[0].shape[0]
            if any(w.shape[0] != K for w in ws) or any(M.shape != (K // 128, w.shape[1]) for w, M in zip(ws, Ms)):
                raise ExactError(f"{pfxs}: weights (K, N) with group scales (K/128, N) expected")
            M = np.concatenate(Ms, 1)
            w = np.concatenate(ws, 1)
            bs = [arrays.get(p + ".b") for p in pfxs]
            if any(b is not None for b in bs):
                b = np.concatenate([np.zeros(w_.shape[1], np.int64) if b_ is None else np.asarray(b_, np.int64)
                                    for w_, b_ in zip(ws, bs)])
                bt = ops.np_to_dev(b, I64, device)
            else:
                bt = None
            parts, off = [], 0
            for p, w_ in zip(pfxs, ws):
                parts.append((p.rsplit(".", 1)[-1], off, w_.shape[1]))
                off += w_.shape[1]
            return ops.pack_group_linear(w, M, device, bt, parts)   # wide scales (>= 2^15) as two planes

        def channel_lin(pfx):
            w = np.asarray(arrays[pfx + ".w"])
            K, N = w.shape
            M = np.asarray(arrays[pfx + ".M"], np.int64)
            b = arrays.get(pfx + ".b")
            bt = None if b is None else ops.np_to_dev(b, I64, device)
            ones = torch.ones((K // 128, N), dtype=I16, device=device)
            wp, mp = ops.pack_linear(ops.np_to_dev(w, I8, device), ones)
            Mbits = int(M.max()).bit_length()
            return PackedLinear(wp, mp, N, K, bt, "channel", ops.np_to_dev(M, I64, device), Mbits)

        for i in range(cfg.NL):
            L = dict(g1=ops.np_to_dev(arrays[f"{i}.g1"], I64, device), g2=ops.np_to_dev(arrays[f"{i}.g2"], I64, device))
            if mode == "group":
                L.update(qkv=group_lin([f"{i}.q", f"{i}.k", f"{i}.v"]), o=group_lin([f"{i}.o"]),
                         gateup=group_lin([f"{i}.gate", f"{i}.up"]), down=group_lin([f"{i}.down"]))
            else:
                L.update({k: channel_lin(f"{i}.{k}") for k in ("q", "k", "v", "o", "gate", "up", "down")})
            self.layers.append(L)
        self.gf = ops.np_to_dev(arrays["gf"], I64, device)
        emb = np.asarray(arrays["emb"], np.int64)
        if np.abs(emb).max() >= 1 << 31:
            raise ExactError("embedding rows must fit int32")
        self.emb = ops.np_to_dev(emb, I32, device)
        # the head follows its scales: (G, N) group-128, (N,) per-channel (the reference's group engines keep a
        # per-channel head, speed_fair_kaggle.py:780)
        self.head = group_lin(["head"]) if np.ndim(arrays["head.M"]) == 2 else channel_lin("head")
        return self

    @classmethod
    def from_artifact(cls, path, device, verify=True):
        """A model from an on-disk exact artifact (exact_amd.artifact; SPEC.md:7-12): integer weights, scales and
        the shipped tables, each file checked against the manifest's SHA-256 first."""
        from . import artifact
        cfg, mode, arrays, tables = artifact.load(path, verify=verify)
        return cls.from_arrays(cfg, arrays, device, mode=mode, tables=tables)


class Cache:
    """Static KV cache: per layer kq int16 (B, KV, Smax, hd), sk int32 (B, KV, Smax), v int64 (B, KV, Smax, hd),
    plus the filled length of every slot (host side)."""

    def __init__(self, cfg, B, Smax, device, layers):
        self.B, self.Smax = B, Smax
        self.layers = [(torch.zeros((B, cfg.KV, Smax, cfg.hd), dtype=I16, device=device),
                        torch.zeros((B, cfg.KV, Smax), dtype=I32, device=device),
                        torch.zeros((B, cfg.KV, Smax, cfg.hd), dtype=I64, device=device)) for _ in range(layers)]
        self.n = [0] * B


def _check_slot(slot, cache):
    """The kernels bound positions, not slots: a slot outside the cache would write keys and values outside it."""
    try:
        ok = 0 <= operator.index(slot) < cache.B
    except TypeError:
        ok = False
    if not ok:
        raise ExactError(f"slot {slot!r} is outside the cache's {cache.B} sequences")


class Workspace:
    """Activation buffers for R rows (allocated once; reused by every step and by captured graphs).
    t buffers start zeroed and are left zeroed by the kernels that consume them."""

    def __init__(self, cfg, R, device, nq, I, abits=15):
        D, H, hd, V = cfg.D, cfg.H, cfg.hd, cfg.V
        z = lambda *sh, dt=I64: torch.zeros(sh, dtype=dt, device=device)
        adt = I16 if abits == 15 else I8
        self.R = R
        self.x, self.xq, self.s = z(R, D), z(R, D, dt=adt), z(R, dt=I32)
        # the q|k|v and down totals in one allocation: a decode pass clears both with one range (the o projection's
        # zero argument) after the norm-fused q|k|v GEMV has read the down totals as its residual
        self.t_qd = z(R * nq + R * D)
        self.t_qkv, self.qq, self.sq = self.t_qd[:R * nq].view(R, nq), z(R, H, hd, dt=I16), z(R, H, dt=I32)
        self.x2 = z(R, D)   # the other residual buffer of decode passes (the norm-fused GEMVs read one, write the other)
        self.att, self.aq, self.sa = z(R, H * hd), z(R, H * hd, dt=adt), z(R, dt=I32)
        self.t_o, self.t_gu, self.hq, self.sh = z(R, D), z(R, 2 * I), z(R, I, dt=adt), z(R, dt=I32)
        self.t_d, self.t_head = self.t_qd[R * nq:].view(R, D), z(R, V)
        self.logits = z(R, V)
        self.s28 = torch.full((R,), 28, dtype=I32, device=device)
        # slice bit lengths of the SwiGLU rows: per 1024 columns (exact_swiglu_qrow) or per 32 or 64
        # (exact_gemv_g128_swiglu)
        self.part_sw = z(R * -(-max(I, cfg.SI if cfg.moe else 0) // 32), dt=I32)
        self.part_lg = ops.logits_parts(R, V, device)
        self.obits = z(R, H * ops.ATT_SPLIT_MAX, dt=I32)   # per-head bit lengths, up to ATT_SPLIT_MAX a head
        self.ids, self.slot, self.pos = z(R, dt=I32), z(R, dt=I32), z(R, dt=I32)
        # the greedy ids are written over the input ids (read once, by the embedding at the start of the pass): the
        # next decode step consumes them with no copy launch in between
        self.next_ids = self.ids
        self.seq = None   # (slot, keys) when the rows are one sequence's consecutive positions (prefill)
        self.h = None     # (R, I) SwiGLU values when the gate|up totals must stay intact (trace capture)
        self.hsh = None   # (R, SI) SwiGLU values of the MoE shared expert (decode rows)
        self.eh = self.part_eh = None   # the routed experts' SwiGLU values per pair and their slice bit lengths
        self.I = I
        # int16 GEMM rows (prefill above 16 rows): the producers also write their rows' int8 digit rows, which the
        # GEMM reads directly (exact_gemm_g128_digits) instead of splitting them in a launch of its own
        self.dig = None
        if abits == 15 and R > ops.A16_DIGIT_ROWS:
            hmax = max(I, cfg.SI if cfg.moe else 0)
            self.dig = dict(x=z(2 * R, D, dt=I8), a=z(2 * R, H * hd, dt=I8), h=z(2 * R, hmax, dt=I8))
        if cfg.moe:
            k, P = cfg.topk, R * cfg.topk
            # chunk arrays for the smallest chunks this workspace may be dispatched with (the fused decode GEMVs' 4 pairs)
            nch = ops.max_chunks(P, cfg.NE, min(ops.EXPERT_FUSE_CHUNK, ops.chunk_rows(abits)))
            self.gate_col = -(-cfg.NE // 64) * 64
            self.t_rt, self.p_sel, self.e_sel = z(R, self.gate_col + 1), z(R, k), z(R, k, dt=I32)
            self.gate = z(R)
            self.disp = dict(pidx=z(P, dt=I32), pair_row=z(P, dt=I32), s_pair=z(P, dt=I32), chunk_e=z(nch, dt=I32),
                             chunk_p0=z(nch, dt=I32), chunk_n=z(nch, dt=I32), nchunks=z(1, dt=I32))
            self.t_egu, self.ehq, self.esh = z(P, 2 * cfg.MI), z(P, cfg.MI, dt=adt), z(P, dt=I32)
            self.t_ed = z(P, D)
            self.t_sgu, self.shq, self.ssh = z(R, 2 * cfg.SI), z(R, cfg.SI, dt=adt), z(R, dt=I32)
            self.t_sd = z(R, D)
            self.part_esw = ops.swiglu_parts(P, cfg.MI, device)


class TModel:
    """Exact integer model on the GPU (the reference's TModel + GraphDecoder engine, exact_torch.py:126-193)."""

    def __init__(self, weights, Smax=512, batch=1, abits=15):
        self.w = weights
        self.cfg = c = weights.cfg
        self.dev = weights.device
        self.abits = abits
        self.Smax, self.batch = Smax, batch
        self.tab = DeviceTables(self.dev, Smax, c.hd, c.theta) if weights.tables is None else \
            DeviceTables.from_host(self.dev, weights.tables, Smax, c.hd)
        self.nl = len(weights.layers)
        self.nq = (c.H + 2 * c.KV) * c.hd
        self.I = c.I if not c.moe else 1
        self._ws = {}
        self._pws = None
        self._graphs = collections.OrderedDict()   # captured prefill passes

    # ---------------------------------------------------------------- buffers
    def new_cache(self, B=None):
        return Cache(self.cfg, self.batch if B is None else B, self.Smax, self.dev, self.nl)

    # rows from which prefill attention runs on the matrix cores, per head dimension (the row kernel is faster below:
    # at hd 64, 14 q heads, 128 rows take 21.5 us there and 19.1 us in the row kernel, 256 rows 26.5 and 41.2 us)
    PREFILL_MIN_ROWS = {64: 160, 128: 96}
    QROW_FUSE_ROWS = 2
    # widest rows whose norm runs inside the consuming GEMVs (every block repeats the row's three reductions; at
    # 3584-wide rows that costs as much as the separate launch it saves, at 5120 more, at 896 less: 7.0 vs 8.2 us)
    NORM_FUSE_D = 2048
    NORM_SWIGLU = True   # norm-fused decode: the SwiGLU in the gate|up GEMV's epilogue too
    BATCH_SWIGLU = True   # decode rows above QROW_FUSE_ROWS: the SwiGLU in the gate|up GEMV's epilogue, then a qrow launch
    QKV_NORM = True   # dense decode rows wider than NORM_FUSE_D: the attention norm inside the q|k|v GEMV
    MOE_NORM = True   # MoE decode rows: the attention norm inside the q|k|v GEMV, the expert norm inside the router GEMV
    MOE_ROUTE = True   # MoE decode rows: top-k routing and dispatch in one launch
    MOE_PAIR = True   # MoE decode rows: the routed and shared experts' GEMVs paired in one launch each (up, down)
    FFN_NORM = True   # decode rows with the attention norm in the q|k|v GEMV: the FFN norm in the SwiGLU GEMV too
    BATCH_ATTN = True   # batched decode rows: the q|k|v epilogue inside the attention launch
    ATT_SPLIT = 4   # decode attention with the q|k|v epilogue: bit lengths a head, so its p.V may run in that many blocks
    SHARED_SWIGLU = True   # MoE decode rows: the shared expert's SwiGLU in its gate|up GEMV's epilogue
    EXPERT_SWIGLU = True   # MoE decode rows: the routed experts' SwiGLU and qrow inside their GEMVs
    EXPERT_GEMM_MIN_PAIRS = 64   # (row, expert) pairs from which the MoE experts run as one grouped GEMM

    def _prefill_ws(self, R):
        if self._pws is None or self._pws[0] < R:
            self._pws = (R, ops.prefill_workspace(R, self.cfg.H, self.cfg.KV, self.cfg.hd, self.Smax, self.dev))
        return self._pws[1]

    def workspace(self, R):
        if R not in self._ws:
            self._ws[R] = Workspace(self.cfg, R, self.dev, self.nq, self.I, self.abits)
        return self._ws[R]

    # ---------------------------------------------------------------- linears
    def _lin(self, x, lin, out, x8=None):
        """t for a group-mode linear (the consumer kernel applies shr(t, 28 - s) + b and leaves out zeroed,
        so decode-sized calls accumulate into it without a separate clear). x8: x's digit rows, when its producer
        wrote them."""
        return ops.linear_t(x, self.abits, lin, out, zeroed=True, x8=x8)

    def _lin_channel(self, x, s, lin, out):
        """channel mode: y = requant_channel(acc) written over out; the consumer then uses s = 28."""
        acc = ops.linear_t(x, self.abits, lin)
        ops.requant_channel(acc, s, lin.M, lin.Mbits, lin.bias, out=out)
        return out

    # ---------------------------------------------------------------- one pass over R rows
    def forward_rows(self, ws, want_logits=True, trace=None, independent=False, last_only=False):
        """Runs the model on ws.ids with (slot, pos) per row; KV of each row is written into the cache
        at (slot, pos). Leaves logits in ws.logits and greedy ids in ws.next_ids (last_only: of the last row only, the
        others are left as they were; the final norm, the head and the argmax run on that row alone).
        independent: every row is a different sequence (decode), so no row attends to another row's new key and
        the q/k/v epilogue runs inside the attention launch.
        trace: (TraceLayout, int64 device buffer): every linear's totals t are produced in the buffer's slots
        and left there (the buffer is zeroed first); the consumer kernels read them without clearing."""
        c, R, tab = self.cfg, ws.R, self.tab
        H, KV, hd, D = c.H, c.KV, c.hd, c.D
        group = self.w.mode == "group"
        keep = trace is not None
        if keep:
            layout, tbuf = trace
            if layout.R != R or tbuf.numel() < layout.total:
                raise ExactError("trace buffer does not match the rows of this pass")
            if ws.h is None:
                ws.h = torch.zeros((R, ws.I), dtype=I64, device=self.dev)
            tbuf.zero_()
            slot = lambda key: layout.slot(tbuf, key)
        clear = group and not keep
        # decode passes of up to QROW_FUSE_ROWS rows: the o and down GEMVs quantise their int64 inputs themselves (no
        # qrow launch); every 64-row block of the GEMV re-reads its slice of the row, which costs more than the saved
        # launch at 8 rows
        xfuse = group and R <= self.QROW_FUSE_ROWS
        afuse = xfuse and ws.seq is None and (R == 1 or independent)
        # batched decode rows (each its own sequence): the q|k|v epilogue inside the attention launch as well, whose
        # totals the attention output's qrow launch then clears (caches of up to 256 positions: 8 threads per key)
        bfuse = (self.BATCH_ATTN and group and not xfuse and ws.seq is None and independent and hd % 64 == 0 and hd <= 128
                 and self.Smax <= 256)
        # decode rows of dense int16 models: residual + RMSNorm + qrow run inside the GEMVs that consume them (q|k|v,
        # gate|up, head), which read one residual buffer and write the other
        nfuse = (afuse and self.abits == 15 and not c.moe and R <= ops.NORM_FUSE_ROWS and D <= self.NORM_FUSE_D
                 and self.w.head.mode == "group")
        # wider dense rows: the attention's residual + RMSNorm + qrow inside the q|k|v GEMV only (8-wave blocks, one per
        # CU, read the row once); the FFN norm stays a launch of its own before the SwiGLU GEMV
        qfuse = (self.QKV_NORM and group and afuse and not nfuse and self.abits == 15 and (self.MOE_NORM or not c.moe)
                 and R <= ops.NORM_FUSE_ROWS and D <= ops.NORM_FUSE_KMAX
                 and (ops.norm_gemv_one_block_per_cu(self.w.layers[0]["qkv"].N, D, R) or D <= self.NORM_FUSE_D))
        # MoE decode rows: the residual + RMSNorm + qrow before the experts inside the router GEMV, which also writes the
        # quantised row the experts read (one launch instead of the norm and the router GEMV)
        rfuse = (self.MOE_NORM and c.moe and qfuse and self.w.layers[0]["router"].bias is None)
        # decode rows of dense int16 models whose gate|up GEMV is not the norm-fused one: the SwiGLU runs in the gate|up
        # GEMV's epilogue (no totals, no atomics, one launch fewer)
        sfuse = (xfuse and not nfuse and not c.moe and self.abits == 15 and R <= ops.SWIGLU_GEMV_ROWS and c.I % 64 == 0
                 and c.I // ops.SWIGLU_PART_COLS <= ops.XQ_PARTS_MAX and self.w.layers[0]["gateup"].bias is None)
        # norm-fused decode rows whose gate|up GEMV also runs the SwiGLU in its epilogue
        nsfuse = (nfuse and self.NORM_SWIGLU and R <= ops.SWIGLU_GEMV_ROWS and c.I % 64 == 0 and D <= ops.NORM_SWIGLU_KMAX
                  and c.I // ops.SWIGLU_PART_COLS <= ops.XQ_PARTS_MAX and self.w.layers[0]["gateup"].bias is None)
        # decode rows above QROW_FUSE_ROWS (bs8): the SwiGLU in the gate|up GEMV's epilogue as well, then one qrow launch
        # over its slice bit lengths before the down GEMV (no gate|up totals, no SwiGLU launch)
        sqfuse = (self.BATCH_SWIGLU and group and not xfuse and not c.moe and self.abits == 15 and R <= ops.SWIGLU_GEMV_MAX_ROWS
                  and c.I % 64 == 0 and self.w.layers[0]["gateup"].bias is None)
        # ... and with the attention norm inside the q|k|v GEMV, the FFN norm inside the SwiGLU GEMV (8-wave blocks, about
        # one per CU)
        fsfuse = (self.FFN_NORM and sfuse and qfuse and D > ops.NORM_SWIGLU_KMAX and D <= ops.NORM_SWIGLU_WIDE_KMAX
                  and c.I % 128 == 0)
        if ws.h is None and not c.moe and ((xfuse and (c.I > 8192 or nfuse or sfuse)) or sqfuse):
            ws.h = torch.zeros((R, ws.I), dtype=I64, device=self.dev)
        x_cur, x_nxt = ws.x, ws.x2
        ops.embed(ws.ids, self.w.emb, ws.x)
        dx = da = dh = None
        if group and ws.dig is not None:
            dx, da = ws.dig["x"], ws.dig["a"]
            dh = ws.dig["h"]
        res_t, res_s = None, None
        for li, L in enumerate(self.w.layers):
            cache = self._cache.layers[li]
            if keep:
                t_qkv, t_o, t_gu, t_d = (slot(f"L{li}.{k}") for k in ("qkv", "o", "gateup", "down"))
            else:
                t_qkv, t_o, t_gu, t_d = ws.t_qkv, ws.t_o, ws.t_gu, ws.t_d
            if nfuse or qfuse:
                ops.gemv_norm_acc(x_cur, res_t, res_s, L["g1"], L["qkv"], t_qkv, ws.s,
                                  x_out=x_nxt if res_t is not None else None)
                if res_t is not None:
                    x_cur, x_nxt = x_nxt, x_cur
                s_qkv, b_qkv = ws.s, L["qkv"].bias
            else:
                ops.rmsnorm_qrow(x_cur, L["g1"], self.abits, res_t, res_s, ws.xq, ws.s, clear=clear, x8=dx)
            if nfuse or qfuse:
                pass
            elif group:
                self._lin(ws.xq, L["qkv"], t_qkv, x8=dx)
                s_qkv, b_qkv = ws.s, L["qkv"].bias
            else:
                off = 0
                for part in ("q", "k", "v"):
                    lin = L[part]
                    y = self._lin_channel(ws.xq, ws.s, lin, torch.empty((R, lin.N), dtype=I64, device=self.dev))
                    ws.t_qkv[:, off:off + lin.N].copy_(y)
                    off += lin.N
                s_qkv, b_qkv = ws.s28, None
            nob = H   # bit lengths per row that attention leaves in ws.obits
            if afuse or bfuse:
                ops.attention_qkv(t_qkv, s_qkv, b_qkv, tab.cos, tab.sin, ws.slot, ws.pos, cache, tab.exp, ws.att, H, KV, hd,
                                  tab.inv, ws.obits, obn=self.ATT_SPLIT)
                nob = H * self.ATT_SPLIT
            else:
                ops.qkv_rope_cache(t_qkv if group else ws.t_qkv, s_qkv, b_qkv, tab.cos, tab.sin, ws.slot, ws.pos, cache,
                                   ws.qq, ws.sq, H, KV, hd, clear=clear)
                if ws.seq is not None:
                    ops.attention_prefill(ws.qq, ws.sq, cache, ws.seq[0], ws.pos, ws.seq[1], tab.exp, ws.att, H, KV, hd,
                                          tab.inv, self._prefill_ws(R), ws.obits)
                else:
                    ops.attention(ws.qq, ws.sq, cache, ws.slot, ws.pos, tab.exp, ws.att, H, KV, hd, tab.inv, ws.obits)
            if nfuse:   # also clears the down totals the q|k|v GEMV read as its residual (t_qkv and t_d are one range)
                ops.gemv_qrow_acc(ws.att, ws.obits, nob, self.abits, L["o"], t_o, ws.sa, zero=ws.t_qd if clear else None)
            elif xfuse:   # clears the q|k|v totals attention left (and, q|k|v norm-fused, the down totals it read)
                ops.gemv_qrow_acc(ws.att, ws.obits, nob, self.abits, L["o"], t_o, ws.sa,
                                  zero=(ws.t_qd if qfuse else t_qkv) if afuse and clear else None)
            else:
                ops.quant_rows(ws.att, ws.obits, nob, self.abits, ws.aq, ws.sa, x8=da, zero=t_qkv if bfuse and clear else None)
            if nfuse and nsfuse:   # norm + gate|up + SwiGLU in one launch
                ops.gemv_norm_swiglu(x_cur, t_o, ws.sa, L["g2"], L["gateup"], ws.s, tab.silu, ws.h, ws.part_sw,
                                     x_out=x_nxt, t=t_gu if keep else None)
                x_cur, x_nxt = x_nxt, x_cur
                ops.gemv_qrow_acc(ws.h, ws.part_sw, c.I // ops.SWIGLU_PART_COLS, self.abits, L["down"], t_d, ws.sh,
                                  zero=t_o if clear else None)   # the o totals the gate|up GEMV read
                res_t, res_s = t_d, ws.sh
                continue
            if nfuse:
                ops.gemv_norm_acc(x_cur, t_o, ws.sa, L["g2"], L["gateup"], t_gu, ws.s, x_out=x_nxt)
                x_cur, x_nxt = x_nxt, x_cur
                ops.swiglu_part(t_gu, ws.s, tab.silu, ws.h, ws.part_sw, clear=clear)
                ops.gemv_qrow_acc(ws.h, ws.part_sw, -(-c.I // ops.QSLICE), self.abits, L["down"], t_d, ws.sh,
                                  zero=t_o if clear else None)   # the o totals the gate|up GEMV read
                res_t, res_s = t_d, ws.sh
                continue
            if group:
                if not xfuse:
                    self._lin(ws.aq, L["o"], t_o, x8=da)
                if rfuse:   # x_out: the other blocks still read x_cur; t_o is cleared by the shared expert's down GEMV
                    ops.gemv_norm_acc(x_cur, t_o, ws.sa, L["g2"], L["router"], ws.t_rt, ws.s, x_out=x_nxt, xq_out=ws.xq)
                    x_cur, x_nxt = x_nxt, x_cur
                elif fsfuse:
                    pass
                else:
                    ops.rmsnorm_qrow(x_cur, L["g2"], self.abits, t_o, ws.sa, ws.xq, ws.s, clear=clear, x8=dx)
            else:
                self._lin_channel(ws.aq, ws.sa, L["o"], ws.t_o)
                ops.rmsnorm_qrow(ws.x, L["g2"], self.abits, ws.t_o, ws.s28, ws.xq, ws.s)
            if c.moe:
                if not group:
                    raise ExactError("MoE layers need group-128 linears")
                self._moe(ws, L, dx, dh, x=x_cur, routed=rfuse, zero=t_o if rfuse and clear else None)
                res_t, res_s = None, None
                continue
            if fsfuse:   # the down GEMV clears the o totals the norm read
                ops.gemv_norm_swiglu(x_cur, t_o, ws.sa, L["g2"], L["gateup"], ws.s, tab.silu, ws.h, ws.part_sw,
                                     x_out=x_nxt, t=t_gu if keep else None)
                x_cur, x_nxt = x_nxt, x_cur
                ops.gemv_qrow_acc(ws.h, ws.part_sw, c.I // ops.SWIGLU_PART_COLS, self.abits, L["down"], t_d, ws.sh,
                                  zero=t_o if clear else None)
                res_t, res_s = t_d, ws.sh
            elif sfuse:
                ops.gemv_swiglu(ws.xq, L["gateup"], ws.s, tab.silu, ws.h, ws.part_sw, t=t_gu if keep else None)
                ops.gemv_qrow_acc(ws.h, ws.part_sw, c.I // ops.SWIGLU_PART_COLS, self.abits, L["down"], t_d, ws.sh)
                res_t, res_s = t_d, ws.sh
            elif sqfuse:
                ops.gemv_swiglu(ws.xq, L["gateup"], ws.s, tab.silu, ws.h, ws.part_sw, t=t_gu if keep else None)
                ops.quant_rows(ws.h, ws.part_sw, c.I // ops.SWIGLU_PART_COLS, self.abits, ws.hq, ws.sh, x8=dh)
                self._lin(ws.hq, L["down"], t_d, x8=dh)
                res_t, res_s = t_d, ws.sh
            elif group:
                self._lin(ws.xq, L["gateup"], t_gu, x8=dx)
                if xfuse and c.I > 8192:   # rows beyond one workgroup: SwiGLU slices, then the down GEMV quantises
                    ops.swiglu_part(t_gu, ws.s, tab.silu, ws.h, ws.part_sw, clear=clear)
                    ops.gemv_qrow_acc(ws.h, ws.part_sw, -(-c.I // ops.QSLICE), self.abits, L["down"], t_d, ws.sh)
                else:
                    ops.swiglu_qrow(t_gu, ws.s, tab.silu, self.abits, ws.hq, ws.sh, clear=clear, part=ws.part_sw,
                                    h=ws.h if keep else None, x8=dh)
                    self._lin(ws.hq, L["down"], t_d, x8=dh)
                res_t, res_s = t_d, ws.sh
            else:
                I = L["gate"].N
                yg = self._lin_channel(ws.xq, ws.s, L["gate"], torch.empty((R, I), dtype=I64, device=self.dev))
                yu = self._lin_channel(ws.xq, ws.s, L["up"], torch.empty((R, I), dtype=I64, device=self.dev))
                ws.t_gu[:, :I].copy_(yg)
                ws.t_gu[:, I:].copy_(yu)
                ops.swiglu_qrow(ws.t_gu, ws.s28, tab.silu, self.abits, ws.hq, ws.sh, part=ws.part_sw)
                self._lin_channel(ws.hq, ws.sh, L["down"], ws.t_d)
                res_t, res_s = ws.t_d, ws.s28
        head = self.w.head
        if nfuse:
            t_head = slot("head") if keep else ws.t_head
            ops.gemv_norm_acc(x_cur, res_t, res_s, self.w.gf, head, t_head, ws.s)
            ops.logits_argmax(t_head, ws.s, ws.logits if want_logits else None, ws.next_ids, clear=clear,
                              part=ws.part_lg)
            return ws
        if last_only and R > 1 and not keep:
            # a prompt's last row only: its final norm, head GEMV and argmax; the other rows' residual totals are
            # cleared for the next pass that accumulates into them
            r = slice(R - 1, R)
            if clear and res_t is not None:
                ops.zero_(res_t[:R - 1])
            ops.rmsnorm_qrow(x_cur[r], self.w.gf, self.abits, None if res_t is None else res_t[r],
                             None if res_s is None else res_s[r], ws.xq[r], ws.s[r], clear=clear)
            if head.mode == "group":
                self._lin(ws.xq[r], head, ws.t_head[r])
                ops.logits_argmax(ws.t_head[r], ws.s[r], ws.logits[r] if want_logits else None, ws.next_ids[r],
                                  clear=clear, part=ws.part_lg)
            else:
                acc = ops.linear_t(ws.xq[r], self.abits, head)
                ops.requant_channel(acc, ws.s[r], head.M, head.Mbits, head.bias, out=ws.t_head[r])
                ops.logits_argmax(ws.t_head[r], ws.s28[r], ws.logits[r] if want_logits else None, ws.next_ids[r],
                                  part=ws.part_lg)
            return ws
        ops.rmsnorm_qrow(x_cur, self.w.gf, self.abits, res_t, res_s, ws.xq, ws.s, clear=clear, x8=dx)
        if head.mode == "group":
            t_head = slot("head") if keep else ws.t_head
            self._lin(ws.xq, head, t_head, x8=dx)
            ops.logits_argmax(t_head, ws.s, ws.logits if want_logits else None, ws.next_ids, clear=clear,
                              part=ws.part_lg)
        else:
            # per-channel head: acc (the traced total), then the drop rule and M (exact_llm.py:89-96)
            acc = ops.linear_t(ws.xq, self.abits, head, slot("head") if keep else None)
            ops.requant_channel(acc, ws.s, head.M, head.Mbits, head.bias, out=ws.t_head)
            ops.logits_argmax(ws.t_head, ws.s28, ws.logits if want_logits else None, ws.next_ids, part=ws.part_lg)
        return ws

    def _moe(self, ws, L, dx=None, dh=None, x=None, routed=False, zero=None):
        """MoE block on m = ws.xq (scale ws.s), added into x (ws.x when None) (MoEInt.moe, moe_exact_kaggle.py:454-467):
        router (with the shared-expert gate logit in the same GEMV) -> isoftmax -> stable top-k -> experts grouped
        into chunks -> SwiGLU per (row, expert) pair -> combination weighted by the Q20 probabilities, plus the
        isig-gated shared expert. routed: the router totals ws.t_rt are already there (the norm-fused router GEMV);
        zero: an int64 tensor to clear on the way (the shared expert's down GEMV clears it, or a launch of its own)."""
        c, tab, k = self.cfg, self.tab, self.cfg.topk
        P = ws.R * k
        x = ws.x if x is None else x
        if not routed:
            self._lin(ws.xq, L["router"], ws.t_rt, x8=dx)
        grouped = P >= self.EXPERT_GEMM_MIN_PAIRS   # prefill: experts on the matrix cores, one tile per 128 pairs
        # decode: the SwiGLU in the expert gate|up GEMV's epilogue and the qrow in the expert down GEMV (chunks of 4 pairs)
        efuse = (self.EXPERT_SWIGLU and not grouped and self.abits == 15 and c.MI % 64 == 0
                 and c.MI // ops.SWIGLU_PART_COLS <= ops.XQ_PARTS_MAX)
        chunk = (ops.EXPERT_CHUNK[self.abits] if grouped else
                 ops.EXPERT_FUSE_CHUNK if efuse else ops.chunk_rows(self.abits))
        if self.MOE_ROUTE and c.NE <= ops.ROUTE_MAX and P <= ops.ROUTE_MAX:   # top-k and dispatch in one wave
            ops.moe_route(ws.t_rt, ws.s, tab.exp, k, ws.p_sel, ws.e_sel, chunk, ws.disp, clear=True, NE=c.NE,
                          gate_col=ws.gate_col, sig=tab.sig, gate=ws.gate)
        else:
            ops.router_topk(ws.t_rt, ws.s, tab.exp, k, ws.p_sel, ws.e_sel, clear=True, NE=c.NE, gate_col=ws.gate_col,
                            sig=tab.sig, gate=ws.gate)
            ops.moe_dispatch(ws.e_sel, ws.s, c.NE, k, chunk, ws.disp)
        sfuse = (self.SHARED_SWIGLU and not grouped and self.abits == 15 and ws.R <= ops.SWIGLU_GEMV_ROWS and c.SI % 64 == 0
                 and c.SI // ops.SWIGLU_PART_COLS <= ops.XQ_PARTS_MAX and L["sgu"].bias is None)
        if efuse and ws.eh is None:
            ws.eh = torch.zeros((P, c.MI), dtype=I64, device=self.dev)
            ws.part_eh = torch.zeros(P * (c.MI // ops.SWIGLU_PART_COLS), dtype=I32, device=self.dev)
        if sfuse and ws.hsh is None:
            ws.hsh = torch.zeros((ws.R, c.SI), dtype=I64, device=self.dev)
        if efuse and sfuse and self.MOE_PAIR and ws.R <= 2:
            # decode rows: the routed and the shared experts' SwiGLU GEMVs in one launch, their down GEMVs in another
            ops.moe_swiglu_pair(ws.xq, ws.disp["pair_row"], L["egu"], ws.disp, ws.disp["s_pair"], tab.silu, ws.eh,
                                ws.part_eh, L["sgu"], ws.s, ws.hsh, ws.part_sw)
            ops.moe_qrow_pair(ws.eh, ws.part_eh, c.MI // ops.SWIGLU_PART_COLS, L["edown"], ws.disp, ws.t_ed, ws.esh,
                              ws.hsh, ws.part_sw, c.SI // ops.SWIGLU_PART_COLS, L["sd"], ws.t_sd, ws.ssh, zero=zero)
            ops.moe_combine(x, ws.t_ed, ws.esh, ws.p_sel, ws.disp["pidx"], k, ws.t_sd, ws.ssh, ws.gate, clear=True)
            return
        if efuse:
            ops.gemv_experts_swiglu(ws.xq, ws.disp["pair_row"], L["egu"], ws.disp, ws.disp["s_pair"], tab.silu, ws.eh,
                                    ws.part_eh)
            ops.gemv_experts_qrow_acc(ws.eh, ws.part_eh, c.MI // ops.SWIGLU_PART_COLS, L["edown"], ws.disp, ws.t_ed,
                                      ws.esh)
        elif grouped:
            ops.gemm_experts(ws.xq, self.abits, ws.disp["pair_row"], L["egu"], ws.disp, ws.t_egu, P)
        else:
            ops.gemv_experts(ws.xq, self.abits, ws.disp["pair_row"], L["egu"], ws.disp, ws.t_egu)
        if not efuse:
            ops.swiglu_qrow(ws.t_egu, ws.disp["s_pair"], tab.silu, self.abits, ws.ehq, ws.esh, clear=not grouped,
                            part=ws.part_esw)
            if grouped:
                ops.gemm_experts(ws.ehq, self.abits, None, L["edown"], ws.disp, ws.t_ed, P)
            else:
                ops.gemv_experts(ws.ehq, self.abits, None, L["edown"], ws.disp, ws.t_ed)
        if sfuse:
            # decode rows: the shared expert's SwiGLU in its gate|up GEMV's epilogue, the down GEMV quantises h
            ops.gemv_swiglu(ws.xq, L["sgu"], ws.s, tab.silu, ws.hsh, ws.part_sw)
            ops.gemv_qrow_acc(ws.hsh, ws.part_sw, c.SI // ops.SWIGLU_PART_COLS, self.abits, L["sd"], ws.t_sd, ws.ssh,
                              zero=zero)
        else:
            self._lin(ws.xq, L["sgu"], ws.t_sgu, x8=dx)
            ops.swiglu_qrow(ws.t_sgu, ws.s, tab.silu, self.abits, ws.shq, ws.ssh, clear=True, part=ws.part_sw, x8=dh)
            self._lin(ws.shq, L["sd"], ws.t_sd, x8=dh)
            if zero is not None:
                ops.zero_(zero)
        ops.moe_combine(x, ws.t_ed, ws.esh, ws.p_sel, ws.disp["pidx"], k, ws.t_sd, ws.ssh, ws.gate, clear=True)

    # ---------------------------------------------------------------- reference-shaped API
    PREFILL_GRAPHS = 8   # captured prefill passes kept (least recently used dropped)

    def forward(self, ids, cache=None, last_only=False, slot=0, graph=False):
        """int64 Q16 logits (T, V) of the new tokens ids (a list) for cache slot `slot` (exact_torch.py:171-193).
        graph=True: the pass for this (length, cache, slot, start position) runs eagerly the first time and is
        captured as a HIP graph, which later calls with the same shape replay (one launch from the host instead
        of about 12 per layer); the prompt ids and positions are copied in before each replay."""
        if cache is None:
            cache = self.new_cache(B=1)
            slot = 0
        _check_slot(slot, cache)
        T = len(ids)
        p0 = cache.n[slot]
        if p0 + T > self.Smax:
            raise ExactError(f"sequence of {p0 + T} positions exceeds the cache ({self.Smax})")
        self._cache = cache
        ws = self.workspace(T)
        ws.ids.copy_(torch.tensor(ids, dtype=I32))
        ws.slot.fill_(slot)
        ws.pos.copy_(torch.arange(p0, p0 + T, dtype=I32))
        # the matrix-core attention for prefill chunks of PREFILL_MIN_ROWS[hd] rows or more (hd 64, 128); the row kernel otherwise
        ws.seq = (slot, p0 + T) if T >= self.PREFILL_MIN_ROWS.get(self.cfg.hd, 1 << 30) else None
        key = (T, id(cache), slot, p0, bool(last_only))
        g = self._graphs.get(key) if graph else None
        try:
            if g is not None:
                self._graphs.move_to_end(key)
                g[0].replay()
            else:
                self.forward_rows(ws, last_only=last_only)
                if graph:   # capture the same pass (capture records, it does not run the kernels again)
                    cg = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(cg):
                        self.forward_rows(ws, last_only=last_only)
                    self._graphs[key] = (cg, cache)   # the graph holds the cache's buffers
                    while len(self._graphs) > self.PREFILL_GRAPHS:
                        self._graphs.popitem(last=False)
        finally:
            ws.seq = None
        cache.n[slot] = p0 + T
        return ws.logits[-1:].clone() if last_only else ws.logits.clone()

    def forward_traced(self, ids, cache=None, slot=0):
        """forward() that also returns the trace of the pass: {name: (T, n) int64} with the reference's names
        L{i}.q, .k, .v, .o, .gate, .up, .down and head (gpu_engine_trace_verify_kaggle.py:790-792)."""
        if cache is None:
            cache = self.new_cache(B=1)
            slot = 0
        _check_slot(slot, cache)
        T = len(ids)
        layout = TraceLayout(self.w, T)
        buf = torch.empty(layout.total, dtype=I64, device=self.dev)
        p0 = cache.n[slot]
        if p0 + T > self.Smax:
            raise ExactError(f"sequence of {p0 + T} positions exceeds the cache ({self.Smax})")
        self._cache = cache
        ws = self.workspace(T)
        ws.ids.copy_(torch.tensor(ids, dtype=I32))
        ws.slot.fill_(slot)
        ws.pos.copy_(torch.arange(p0, p0 + T, dtype=I32))
        ws.seq = (slot, p0 + T) if T >= self.PREFILL_MIN_ROWS.get(self.cfg.hd, 1 << 30) else None
        try:
            self.forward_rows(ws, trace=(layout, buf))
        finally:
            ws.seq = None
        cache.n[slot] = p0 + T
        return ws.logits.clone(), layout.split(buf.cpu().numpy())

    def decode_rows(self, tokens, cache):
        """One decode step for B sequences (row r = cache slot r, at position cache.n[r])."""
        B = len(tokens)
        self._cache = cache
        ws = self.workspace(B)
        ws.ids.copy_(torch.tensor(tokens, dtype=I32))
        ws.slot.copy_(torch.arange(B, dtype=I32))
        ws.pos.copy_(torch.tensor(cache.n[:B], dtype=I32))
        if max(cache.n[:B]) >= self.Smax:
            raise ExactError("cache full")
        self.forward_rows(ws, independent=True)
        for r in range(B):
            cache.n[r] += 1
        return ws.logits.clone(), ws.next_ids.clone()


def step_hash(prev, lg_row):
    """Chained per-step receipt hash: sha256 of the previous hash and the int64 logits row, first 16 hex
    digits (exact_llm.py:260-261)."""
    return hashlib.sha256(prev.encode() + np.ascontiguousarray(lg_row, np.int64).tobytes()).hexdigest()[:16]


class _RowPipe:
    """Each decode step's logits row (and its sampled id) copied to pinned host memory behind the step on the same
    stream, two slots in turn: the host hashes step t while the device runs step t + 1. Stream order makes each copy
    read the decoder's buffers before the next step overwrites them."""

    def __init__(self, V):
        self.rows = [torch.empty(V, dtype=I64, pin_memory=True) for _ in range(2)]
        self.ids = [torch.empty(1, dtype=I32, pin_memory=True) for _ in range(2)]
        self.ev = [torch.cuda.Event(), torch.cuda.Event()]

    def push(self, t, lg_row, ids):
        k = t % 2
        self.rows[k].copy_(lg_row, non_blocking=True)
        self.ids[k].copy_(ids, non_blocking=True)
        self.ev[k].record()

    def pop(self, t):
        """(logits row, sampled id) of step t, once its copies have landed"""
        k = t % 2
        self.ev[k].synchronize()
        return self.rows[k].numpy(), int(self.ids[k][0])


def generate(tm, prompt_ids, n, seed, temp):
    """Sampled generation with a receipt (exact_llm.generate, exact_llm.py:262-268): the integer sampler runs on
    the device and its token stays there as the next step's input (one HIP-graph replay a step); each step's logits
    row comes to the host only for the receipt hash, copied behind the step and hashed while the next step runs.
    Uses the KV cache (the reference re-runs the whole sequence per step; the logits are identical by causality).
    Returns (receipt dict, greedy tokens)."""
    tnum = ops.temp_num(temp)
    cache = tm.new_cache(B=1)
    step = torch.zeros(1, dtype=I32, device=tm.dev)
    chain, toks, greedy = "start", [], []
    lg = tm.forward(list(prompt_ids), cache, last_only=True)
    pipe = _RowPipe(lg.shape[1])
    gd, ids = None, torch.zeros(1, dtype=I32, device=tm.dev)
    if n > 1:
        gd = GraphDecoder(tm, cache, 1)
        gd.load([0])
        ids = gd.ws.ids            # the sampled token is the next step's input, on the device
    for t in range(n):
        if t > 0:
            lg, _ = gd.step()       # consumes ids; its greedy ids are overwritten by the sample below
        step.fill_(t)
        ops.sample(lg, seed, step, tnum, tm.tab.exp, ids)
        pipe.push(t, lg[0], ids)
        if t == 0 and gd is not None:
            gd.capture()            # captured after the first sample: its warm-up step restores ids and positions
        if t > 0:
            row, tok = pipe.pop(t - 1)
            chain = step_hash(chain, row)
            toks.append(tok)
            greedy.append(int(row.argmax()))
    row, tok = pipe.pop(n - 1)
    chain = step_hash(chain, row)
    toks.append(tok)
    greedy.append(int(row.argmax()))
    return dict(prompt=list(prompt_ids), seed=seed, temp=temp, tokens=toks, chain=chain), greedy


def verify(tm, receipt):
    """Recompute a receipt (exact_llm.verify, exact_llm.py:269-276): (ok, first bad position, "chain" or None). The
    receipt's own tokens feed the steps (from the device); each step's sample is compared on the host one step
    behind, and the work queued past a mismatch is discarded."""
    tnum = ops.temp_num(receipt["temp"])
    rec = list(receipt["tokens"])
    n = len(rec)
    cache = tm.new_cache(B=1)
    step = torch.zeros(1, dtype=I32, device=tm.dev)
    samp = torch.zeros(1, dtype=I32, device=tm.dev)
    chain = "start"
    lg = tm.forward(list(receipt["prompt"]), cache, last_only=True)
    if n == 0:
        return chain == receipt["chain"], (None if chain == receipt["chain"] else "chain")
    pipe = _RowPipe(lg.shape[1])
    gd = None
    if n > 1:
        rec_dev = torch.tensor(rec, dtype=I32).to(tm.dev)
        gd = GraphDecoder(tm, cache, 1)
        gd.load([rec[0]])
        gd.capture()

    def check(t):
        row, tok = pipe.pop(t)
        return step_hash(chain, row), tok == rec[t]

    for t in range(n):
        if t > 0:
            gd.ws.ids.copy_(rec_dev[t - 1:t])
            lg, _ = gd.step()
        step.fill_(t)
        ops.sample(lg, receipt["seed"], step, tnum, tm.tab.exp, samp)
        pipe.push(t, lg[0], samp)
        if t > 0:
            chain, ok = check(t - 1)
            if not ok:
                torch.cuda.current_stream().synchronize()
                return False, t - 1
    chain, ok = check(n - 1)
    if not ok:
        return False, n - 1
    return chain == receipt["chain"], (None if chain == receipt["chain"] else "chain")


class GraphDecoder:
    """HIP-graph decode step for B sequences (speed_fair_kaggle.py:590-645): ids, slots and positions
    live on the device; one replay runs every kernel of a step, writes the logits and the greedy next
    ids, and advances the positions. step() = copy tokens (optional) + replay."""

    def __init__(self, tm, cache, B, trace=False):
        """trace=True: every step also leaves the totals of every linear in one of two static device buffers
        (step j in trace_bufs[j % 2], laid out by self.layout), one captured graph per buffer; attach a
        TraceRecorder with record() to copy and commit them."""
        self.tm, self.cache, self.B = tm, cache, B
        self.ws = tm.workspace(B)
        self.graph = None
        self.trace = trace
        self.nstep = 0
        self.recorder = None
        if trace:
            self.layout = TraceLayout(tm.w, B)
            self.trace_bufs = [torch.zeros(self.layout.total, dtype=I64, device=tm.dev) for _ in range(2)]
            self.graphs = [None, None]

    def record(self, mode="commit", keep=False):
        """Attach a TraceRecorder (modes "device", "host", "commit"); returns it."""
        if not self.trace:
            raise ExactError("this decoder was built without trace capture")
        self.recorder = TraceRecorder(self, mode, keep)
        return self.recorder

    def load(self, tokens):
        ws = self.ws
        ws.ids.copy_(torch.tensor(tokens, dtype=I32))
        ws.slot.copy_(torch.arange(self.B, dtype=I32))
        ws.pos.copy_(torch.tensor(self.cache.n[:self.B], dtype=I32))

    def _step(self, b=0):
        self.tm._cache = self.cache
        self.tm.forward_rows(self.ws, trace=(self.layout, self.trace_bufs[b]) if self.trace else None, independent=True)
        ops.advance(self.ws.pos)

    def capture(self):
        """Warm up once outside the graph (restoring positions), then capture one step (one per trace buffer)."""
        ws = self.ws
        pos0 = ws.pos.clone()
        ids0 = ws.ids.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self._step()
        torch.cuda.current_stream().wait_stream(s)
        ws.pos.copy_(pos0)
        ws.ids.copy_(ids0)
        torch.cuda.synchronize()
        for b in range(2 if self.trace else 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step(b)
            if self.trace:
                self.graphs[b] = g
            self.graph = g
        torch.cuda.synchronize()

    def step(self):
        """One decode step: returns (logits (B, V) view, next ids view). The greedy ids land in the step's input
        ids, so the next step consumes them directly on the device; a caller that chooses other tokens (sampling, say)
        loads them with load() before the next step. Both views alias the decoder's own buffers: the next step, and
        for the ids also load(), overwrite them (clone what must outlive that)."""
        if max(self.cache.n[:self.B]) >= self.tm.Smax:
            raise ExactError("cache full")
        b = self.nstep % 2
        if self.recorder is not None:
            self.recorder.before_step(b)
        if self.graph is None:
            self._step(b)
        elif self.trace:
            self.graphs[b].replay()
        else:
            self.graph.replay()
        if self.recorder is not None:
            self.recorder.after_step(b)
        self.nstep += 1
        for r in range(self.B):
            self.cache.n[r] += 1
        # next_ids is the ids buffer itself, so the greedy ids are already the next step's input
        return self.ws.logits, self.ws.next_ids
