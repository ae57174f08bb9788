"""Benchmark: exact integer decode of a Qwen2.5-7B-shape model, batch 1, on one MI355X.

value = tok/s of full-model decode steps (embedding, 28 layers of RMSNorm, group-128 int8 q|k|v, RoPE, exact integer
attention over the KV cache, o, RMSNorm, SwiGLU MLP, then the final RMSNorm, the lm_head and the greedy argmax), int16
activations as the spec's qrow, each step one HIP graph replay; roofline = the step's int8 weight + int16 scale bytes
over its time against the 8 TB/s HBM peak.
Also reported: the isolated 7B decode GEMV pass (int8 x, bs1 and bs8) with the gate|up kernel's roofline; the same
GEMVs through the reference's own op exact::gemv on its row-major tensors; the 2048-token prefill GEMMs and attention
layer (int8 MFMA TOPS); decode of the 0.5B (bs1), 14B (bs1, bs8) and MoE (bs1) configurations; the trace-capture cost;
and the numpy oracle (the reference's CPU algorithm) timed on the host cores for every configuration.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--cpu-full] [--no-prefill] [--no-model]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "exact-llm_amd"))

METRIC = "decode tok/s (7B-shape, bs1); GEMV HBM GB/s; prefill int8 MFMA TOPS"
HBM_PEAK_GBPS = 8000.0
# gate|up launch: 37888*3584 int8 weights + 37888*28*2 scale bytes + 3584 x bytes + 37888*8 output bytes
GATEUP_BYTES = 37888 * 3584 + 37888 * 28 * 2 + 3584 + 37888 * 8
# HBM bytes per gate|up launch from FETCH_SIZE / WRITE_SIZE counter runs, each scaled by the same counter on a
# 512 MiB device copy (profiles/gemv_gateup_7b_traffic.md): 137,998,602 read + 1,818,624 written
GATEUP_TRAFFIC_BYTES = 139_822_021
# HBM bytes of one 7B bs1 decode step (the headline's unit of work), measured the same way over the step's 146
# launches (profiles/decode_7b_bs1_step.md): 7,284.5 MB read + 124.4 MB written
STEP_TRAFFIC_BYTES = 7_408_900_000
INT8_PEAK_TOPS = 5000.0


def gemv_pass(args):
    import numpy as np
    import torch
    from exact_amd import ops, synth
    from exact_amd.ops import I8, I64, PackedLinear

    cfg = synth.CONFIGS["qwen2.5-7b"]
    dev = "cuda"
    D, I, NL = cfg.D, cfg.I, cfg.NL
    nqkv = (cfg.H + 2 * cfg.KV) * cfg.hd
    thr = torch.tensor(synth.thresholds().astype(np.int64)).to(torch.int32).to(dev)
    seed = 7

    def lin(name, N, K):
        wp, mp = PackedLinear.alloc(N, K, dev)
        ops.synth_linear(wp, mp, N, K, synth.key(seed, name + ".w"), synth.key(seed, name + ".m"), synth.M_LO, synth.M_HI, thr)
        return PackedLinear(wp, mp, N, K)

    shapes = {"qkv": (nqkv, D), "o": (D, cfg.H * cfg.hd), "gateup": (2 * I, D), "down": (D, I)}
    layers = [{k: lin(f"L{li}.{k}", *v) for k, v in shapes.items()} for li in range(NL)]
    head = lin("head", cfg.V, D)

    def nbytes(N, K, R=1):
        return N * K + N * (K // 128) * 2 + R * K + R * N * 8

    st = torch.cuda.current_stream()

    def measure(R):
        """The pass and its per-shape launches for R activation rows (R tokens per pass)."""
        g = torch.Generator(device="cpu").manual_seed(1)
        x_d = torch.randint(-127, 128, (R, D), generator=g, dtype=torch.int8).to(dev)
        x_i = torch.randint(-127, 128, (R, I), generator=g, dtype=torch.int8).to(dev)
        x_a = torch.randint(-127, 128, (R, cfg.H * cfg.hd), generator=g, dtype=torch.int8).to(dev)
        xin = {"qkv": x_d, "o": x_a, "gateup": x_d, "down": x_i}
        # every GEMV of the pass writes its own exact output: one buffer, zeroed once per step, sliced per launch
        nout = NL * sum(v[0] for v in shapes.values()) + cfg.V
        obuf = torch.zeros(R * nout, dtype=I64, device=dev)
        outs, off = [], 0
        for li in range(NL):
            o = {}
            for k, v in shapes.items():
                o[k] = obuf[off:off + R * v[0]].view(R, v[0])
                off += R * v[0]
            outs.append(o)
        out_head = obuf[off:off + R * cfg.V].view(R, cfg.V)
        pass_bytes = sum(nbytes(*shapes[k], R) for k in shapes) * NL + nbytes(cfg.V, D, R)

        def step():
            ops.zero_(obuf)
            for L, o in zip(layers, outs):
                for k in shapes:
                    ops.gemv_g128_acc(xin[k], 7, L[k], o[k])
            ops.gemv_g128_acc(x_d, 7, head, out_head)

        torch.cuda.synchronize()
        step()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(st)
        for _ in range(args.steps):
            graph.replay()
        e1.record(st)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_time(e1) / args.steps

        # per-shape launch durations: one HIP graph of NL launches over distinct weights (no cache reuse),
        # timed with HIP events on the launch stream
        per = {}
        for k, (N, K) in list(shapes.items()) + [("head", (cfg.V, D))]:
            def shape_step():
                if k == "head":
                    ops.gemv_g128_acc(x_d, 7, head, out_head)
                else:
                    for L, o in zip(layers, outs):
                        ops.gemv_g128_acc(xin[k], 7, L[k], o[k])
            sg = torch.cuda.CUDAGraph()
            with torch.cuda.graph(sg):
                shape_step()
            sg.replay()
            reps = 5
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record(st)
            for _ in range(reps):
                sg.replay()
            b.record(st)
            torch.cuda.synchronize()
            n = reps * (1 if k == "head" else NL)
            us = a.elapsed_time(b) * 1000.0 / n
            per[k] = dict(N=N, K=K, us=round(us, 2), GBps=round(nbytes(N, K, R) / us / 1e3, 1))
            del sg
        del graph, obuf
        return dict(ms=ms, wall=wall, pass_bytes=pass_bytes, per=per)

    r1 = measure(1)
    r8 = measure(8)
    r1["bs8"] = r8
    del layers, head
    torch.cuda.empty_cache()
    return r1


def active_bytes(cfg):
    """int8 weight + int16 scale bytes read per decode token (MoE: the top-k experts, the shared expert and the router)."""
    from exact_amd import synth
    if not cfg.moe:
        return synth.param_bytes(cfg)
    D = cfg.D
    lb = lambda N, K: N * K + N * (K // 128) * 2
    layer = (lb((cfg.H + 2 * cfg.KV) * cfg.hd, D) + lb(D, cfg.H * cfg.hd) + lb(cfg.NE, D) + lb(1, D)
             + cfg.topk * (lb(2 * cfg.MI, D) + lb(D, cfg.MI)) + lb(2 * cfg.SI, D) + lb(D, cfg.SI))
    return cfg.NL * layer + lb(cfg.V, D)


def model_decode(args, name="qwen2.5-7b", prompt_len=16, B=1):
    """Full integer decode steps of a model (embedding, per layer irms, fused q|k|v GEMV, RoPE, integer
    attention over the KV cache, o, SwiGLU or MoE, down, head + greedy argmax), A16 activations as in the
    spec, B sequences per step, one HIP graph per step. Prefill (each sequence's prompt) is timed too: replays of
    the captured prefill pass of each slot (new prompts of the same length), and the same passes launched eagerly."""
    import numpy as np
    import torch
    from exact_amd import synth
    from exact_amd.model import DeviceWeights, GraphDecoder, TModel
    cfg = synth.CONFIGS[name]
    tm = TModel(DeviceWeights.synthetic(cfg, 11, "cuda"), Smax=prompt_len + args.warmup + args.steps + 8, batch=B)
    rng = np.random.default_rng(0)
    st = torch.cuda.current_stream()
    cache = tm.new_cache()

    def prefill_all(graph):
        """prefill every slot's prompt from position 0; returns (ms per sequence, greedy first tokens)"""
        for s_ in range(B):
            cache.n[s_] = 0
        firsts = []
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(st)
        for s_ in range(B):
            lg = tm.forward(rng.integers(0, cfg.V, prompt_len).tolist(), cache, last_only=True, slot=s_, graph=graph)
            firsts.append(int(lg[-1].argmax()))
        b.record(st)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / B, firsts

    # untimed passes first: they allocate the prompt-sized workspace, load every kernel the prefill uses and capture
    # each slot's prefill graph (one-time set-up costs, like the decode graph capture below)
    prefill_all(False)
    prefill_all(True)
    eager_ms, _ = prefill_all(False)
    prefill_ms, first = prefill_all(True)      # replays of the captured prefill passes, new prompts
    tm._graphs.clear()
    tm._ws.pop(prompt_len, None)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gd = GraphDecoder(tm, cache, B)
    gd.load(first)
    gd.capture()
    for _ in range(args.warmup):
        gd.step()
    torch.cuda.synchronize()
    a.record(st)
    for _ in range(args.steps):
        gd.step()
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / args.steps
    wbytes = active_bytes(cfg)
    del gd, cache
    check = fixture_check(tm, name) if B == 1 else None
    del tm
    torch.cuda.empty_cache()
    res = {"model": name, "batch": B, "tok_s": round(1000.0 * B / ms, 2), "ms_per_step": round(ms, 4), "abits": 15,
           "weights_GB_per_step": round(wbytes / 1e9, 3), "GBps": round(wbytes / ms / 1e6, 1),
           "frac_hbm": round(wbytes / ms / 1e6 / HBM_PEAK_GBPS, 4), "prompt": prompt_len,
           "prefill_ms_per_sequence": round(prefill_ms, 3), "prefill_eager_ms_per_sequence": round(eager_ms, 3)}
    if check is not None:
        res["oracle_fixture"] = check
    return res


FIXTURES = {"qwen2.5-7b": "full_c2.json"}   # oracle fixtures of the benchmarked models (the same seed: 11)


def fixture_check(tm, name):
    """Untimed: the benchmarked model (same weights) decodes the fixture's first sequence, prefill then greedy steps in
    a HIP graph as timed above, and every logits row hash and token is compared with the oracle's
    (tests/golden/make_full_configs.py)."""
    import torch
    from exact_amd.model import GraphDecoder
    fn = FIXTURES.get(name)
    path = os.path.join(ROOT, "tests", "golden", fn) if fn else None
    if not path or not os.path.exists(path):
        return None
    import hashlib
    spec = json.load(open(path))
    if spec["seed"] != 11 or spec["config"] != name:
        return None
    sq = spec["sequences"][0]
    h = lambda row: hashlib.sha256(row.astype("<i8").tobytes()).hexdigest()[:16]
    cache = tm.new_cache()
    row = tm.forward(sq["prompt"], cache, last_only=True, slot=0)[-1].cpu().numpy()
    ok = h(row) == sq["hashes"][0] and int(row.argmax()) == sq["tokens"][0]
    gd = GraphDecoder(tm, cache, 1)
    gd.load([int(row.argmax())])
    gd.capture()
    n = min(spec["new_tokens"], tm.Smax - spec["prompt_len"])
    for i in range(1, n):
        lg, nid = gd.step()
        torch.cuda.synchronize()
        ok = ok and h(lg[0].cpu().numpy()) == sq["hashes"][i] and int(nid[0]) == sq["tokens"][i]
    del gd, cache
    return {"fixture": fn, "tokens": n, "equal": bool(ok)}


def trace_capture(args, name="qwen2.5-7b", prompt_len=16, steps=32, reps=3):
    """Cost of the trace commitment in graph decode (the reference's T0-T3, prover_commit_cost_gpu_kaggle.py:791-845),
    7B shape, bs1, A16: T0 plain graph decode; T1 + the totals of every linear left in a static device trace buffer
    by the graph; T2 + copy of each step's trace to pinned host memory on a side stream; T3 + SHA-256 commitment
    of each step's trace (4 leaves in 4 threads). Median of `reps` runs of `steps` steps after a prompt, each run
    re-prefilled; logits of the first 8 steps must equal T0's."""
    import numpy as np
    import torch
    from exact_amd import synth
    from exact_amd.model import DeviceWeights, GraphDecoder, TModel
    cfg = synth.CONFIGS[name]
    tm = TModel(DeviceWeights.synthetic(cfg, 11, "cuda"), Smax=prompt_len + steps + 8, batch=1)
    ids = np.random.default_rng(1).integers(0, cfg.V, prompt_len).tolist()
    res, base = {}, None
    for mode, rmode in (("T0", None), ("T1", "device"), ("T2", "host"), ("T3", "commit")):
        cache = tm.new_cache(B=1)
        first = int(tm.forward(ids, cache, last_only=True)[0].argmax())
        gd = GraphDecoder(tm, cache, 1, trace=rmode is not None)
        gd.load([first])
        gd.capture()
        times, rows, ndig = [], [], 0
        for rep in range(reps):
            cache.n[0] = 0
            tm.forward(ids, cache, last_only=True)
            gd.load([first])
            gd.nstep = 0
            rec = gd.record(rmode) if rmode else None
            got = []
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for j in range(steps):
                lg, _ = gd.step()
                if j < 8:
                    got.append(lg.clone())
            digests = rec.finish() if rec else None
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
            if rep == 0:
                rows = got
                ndig = len(digests) if digests is not None else 0
        res[mode + "_tok_s"] = round(steps / float(np.median(times)), 2)
        if base is None:
            base = rows
        else:
            res[mode + "_logits_equal_T0"] = all(torch.equal(a, b) for a, b in zip(rows, base))
        if mode == "T3":
            res["T3_digests_per_run"] = ndig
        if rmode:
            res["trace_ints_per_token"] = gd.layout.total
        del gd
    for mode in ("T1", "T2", "T3"):
        res[mode + "_overhead"] = round(res["T0_tok_s"] / res[mode + "_tok_s"] - 1, 4)
    res.update(model=name, batch=1, steps=steps, prompt=prompt_len, reps=reps)
    del tm
    torch.cuda.empty_cache()
    return res


def attention_prefill(args, S=2048, H=28, KV=4, hd=128):
    """Exact integer causal attention of one 2048-token prefill layer (by default the 7B's 28 q / 4 kv heads of
    hd 128) from the KV cache, on the matrix cores and on the row kernel: algorithmic ops 2*(S(S+1)/2)*hd*H for q.k
    and the same for p.v."""
    import torch
    from exact_amd import ops
    from exact_amd.tables import DeviceTables
    dev = "cuda"
    tab = DeviceTables(dev, S, hd, 1e6)
    g = torch.Generator(device="cpu").manual_seed(3)
    kq = torch.randint(-32767, 32768, (1, KV, S, hd), generator=g, dtype=torch.int16).to(dev)
    sk = torch.randint(0, 16, (1, KV, S), generator=g, dtype=torch.int32).to(dev)
    v = torch.randint(-(1 << 30), 1 << 30, (1, KV, S, hd), generator=g, dtype=torch.int64).to(dev)
    qq = torch.randint(-32767, 32768, (S, H, hd), generator=g, dtype=torch.int16).to(dev)
    sq = torch.randint(0, 16, (S, H), generator=g, dtype=torch.int32).to(dev)
    slot = torch.zeros(S, dtype=torch.int32, device=dev)
    pos = torch.arange(S, dtype=torch.int32, device=dev)
    out = torch.empty((S, H * hd), dtype=torch.int64, device=dev)
    ref = torch.empty((S, H * hd), dtype=torch.int64, device=dev)
    ws = ops.prefill_workspace(S, H, KV, hd, S, dev)
    run_rows = lambda: ops.attention(qq, sq, (kq, sk, v), slot, pos, tab.exp, ref, H, KV, hd, tab.inv)
    run_mfma = lambda: ops.attention_prefill(qq, sq, (kq, sk, v), 0, pos, S, tab.exp, out, H, KV, hd, tab.inv, ws)
    st = torch.cuda.current_stream()

    def timed(fn, reps=3):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(reps):
            fn()
        b.record(st)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1000.0 / reps

    us_rows = timed(run_rows)
    us = timed(run_mfma, 5)
    same = bool(torch.equal(out, ref))
    ops_ = 2 * 2 * (S * (S + 1) // 2) * hd * H
    del kq, sk, v, qq, out, ref, ws
    torch.cuda.empty_cache()
    return {"S": S, "H": H, "KV": KV, "hd": hd, "us": round(us, 1), "G_ops": round(ops_ / 1e9, 2),
            "TOPS": round(ops_ / us / 1e6, 3), "row_kernel_us": round(us_rows, 1), "equal_to_row_kernel": same}


def prefill_gemm(args):
    import torch
    import numpy as np
    from exact_amd import ops, synth
    from exact_amd.ops import PackedLinear
    dev = "cuda"
    thr = torch.tensor(synth.thresholds().astype(np.int64)).to(torch.int32).to(dev)
    res = {}
    for name, (M, K, N) in {"gateup_K3584_N18944": (2048, 3584, 18944), "down_K18944_N3584": (2048, 18944, 3584)}.items():
        wp, mp = PackedLinear.alloc(N, K, dev)
        ops.synth_linear(wp, mp, N, K, synth.key(9, name + ".w"), synth.key(9, name + ".m"), synth.M_LO, synth.M_HI, thr)
        lin = PackedLinear(wp, mp, N, K)
        out = torch.empty((M, N), dtype=torch.int64, device=dev)
        st = torch.cuda.current_stream()
        # int8 rows (the benchmark's A8), then int16 rows (the spec's qrow 15: the same GEMM on interleaved digit
        # rows, twice the matrix-core work for the same algorithmic ops)
        for abits, label in ((7, name), (15, name + "_a16")):
            lim = (1 << abits) - 1
            x = torch.randint(-lim, lim + 1, (M, K), dtype=torch.int8 if abits == 7 else torch.int16).to(dev)
            ops.gemm_g128(x, abits, lin, out)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 3
            a.record(st)
            for _ in range(reps):
                ops.gemm_g128(x, abits, lin, out)
            b.record(st)
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1000.0 / reps
            res[label] = dict(us=round(us, 1), TOPS=round(2.0 * M * K * N / us / 1e6, 2))
            del x
        del wp, mp, lin, out
    torch.cuda.empty_cache()
    return res


def _oracle_env():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import exact_c
    import exact_oracle as O
    from exact_amd import synth
    return O, exact_c, synth


def cpu_model_string():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def progress(msg):
    """A progress line on stderr (the result is the one JSON line on stdout)."""
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def _median_time(fn, n, label=None):
    import numpy as np
    ts = []
    for i in range(n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if label:
            progress(f"CPU baseline: {label} run {i + 1}/{n}: {ts[-1]:.2f} s")
    return float(np.median(ts))


def _oracle_lin(seed, name, N, K, bias=False):
    """A linear of the synthetic model (the same integers the GPU runs) from the oracle's C generator."""
    O, exact_c, synth = _oracle_env()
    key = lambda s_: synth.key(seed, name + s_)
    b = synth.vector_np(key(".b"), N, *synth.BIAS) if bias else None
    return O.Lin(exact_c.weights(key(".w"), synth.thresholds(), N, K),
                 exact_c.scales(key(".m"), N, K, synth.M_LO, synth.M_HI), b)


def cpu_layer_step(name, context, steps=3, seed=11):
    """Seconds of one KV-cached decode step through ONE decoder layer of `name` (its real synthetic integers; numpy
    oracle = the reference's CPU algorithm) after a `context`-token prompt, median of `steps`; and seconds of the
    lm_head GEMV of one row. A token of the full model costs NL * layer + head (+ two row norms, negligible)."""
    import numpy as np
    O, exact_c, synth = _oracle_env()
    cfg = synth.CONFIGS[name]
    L = dict(g1=synth.vector_np(synth.key(seed, "L0.g1"), cfg.D, *synth.GAIN),
             g2=synth.vector_np(synth.key(seed, "L0.g2"), cfg.D, *synth.GAIN))
    for lname, N, K, bias in synth.linear_specs(cfg, 0):
        L[lname.split(".", 1)[1]] = _oracle_lin(seed, lname, N, K, bias)
    if cfg.moe:
        L["experts"] = [(L.pop(f"e{e}.gate"), L.pop(f"e{e}.up"), L.pop(f"e{e}.down")) for e in range(cfg.NE)]
    rng = np.random.default_rng(seed)
    V_small = context + steps + 2          # stand-in vocabulary: the layer, not the embedding, is timed here
    emb = rng.integers(-(1 << 17), 1 << 17, (V_small, cfg.D))
    head = O.Lin(rng.integers(-127, 128, (cfg.D, 64), dtype=np.int8), rng.integers(8192, 24576, (cfg.D // 128, 64)))
    m = O.Model(dict(emb=emb, gf=L["g1"], layers=[L], head=head),
                dict(D=cfg.D, H=cfg.H, KV=cfg.KV, hd=cfg.hd, NL=1, theta=cfg.theta, T=V_small + 2, topk=cfg.topk))
    cache = m.new_cache()
    m(list(range(context)), cache)
    ts = []
    for j in range(steps):
        t0 = time.perf_counter()
        m([context + j], cache)
        ts.append(time.perf_counter() - t0)
    hw = exact_c.weights(synth.key(seed, "head.w"), synth.thresholds(), cfg.V, cfg.D)
    hM = exact_c.scales(synth.key(seed, "head.m"), cfg.V, cfg.D, synth.M_LO, synth.M_HI)
    x = rng.integers(-(1 << 20), 1 << 20, (1, cfg.D))
    t_head = _median_time(lambda: O.linear_group_t(x, hw, hM), 1)
    return float(np.median(ts)), t_head, cfg.NL


def cpu_baseline(full=False):
    """The reference's numpy CPU path (the oracle restates it: per-group float64 BLAS + rint, numpy integer
    elementwise ops, per-head attention) timed on this host for each configuration (BASELINE.md's CPU plan), with
    bounded samples unless full: value = Qwen2.5-7B-shape bs1 KV-cached decode tok/s, from one layer's decode step
    x 28 + the lm_head."""
    import numpy as np
    O, exact_c, synth = _oracle_env()
    reps = 3 if full else 1
    out = {"cores": os.cpu_count(), "cpu": cpu_model_string(), "kind": "port",
           "threads": "numpy/BLAS defaults (all cores)", "timing": "median of 3" if full else "one run per sample"}
    # 7B-shape decode (the headline workload)
    progress("CPU baseline: 7B layer")
    t_l, t_h, nl = cpu_layer_step("qwen2.5-7b", 16)
    tok7 = 1.0 / (nl * t_l + t_h)
    out["qwen2.5-7b_bs1"] = {"kv_cached_tok_s": round(tok7, 4), "layer_step_s": round(t_l, 3), "head_s": round(t_h, 3),
                             "sample": "one layer's KV-cached decode step at a 16-token context (median of 3) x 28 + head"}
    # C2: the 7B decode GEMVs, bs1 and bs8, A8 (per shape)
    rng = np.random.default_rng(0)
    c2 = {}
    for sname, (N, K) in {"qkv": (4608, 3584), "o": (3584, 3584), "gateup": (37888, 3584), "down": (3584, 18944),
                          "head": (152064, 3584)}.items():
        w = exact_c.weights(synth.key(5, sname), synth.thresholds(), N, K)
        M = exact_c.scales(synth.key(6, sname), N, K, synth.M_LO, synth.M_HI)
        row = {}
        for R in (1, 8):
            x = rng.integers(-127, 128, (R, K))
            t = _median_time(lambda: O.linear_group_t(x, w, M, abits=7), reps)
            row[f"bs{R}_ms"] = round(1e3 * t, 2)
            row[f"bs{R}_GBps"] = round((N * K + N * (K // 128) * 2) / t / 1e9, 2)
        c2[sname] = row
        del w, M
    out["C2_gemv_7b"] = c2
    progress("CPU baseline: C2 GEMVs done")
    # C3: the 2048-token prefill GEMMs (A8) and one attention layer
    c3 = {}
    for gname, (K, N) in {"gateup_K3584_N18944": (3584, 18944), "down_K18944_N3584": (18944, 3584)}.items():
        w = exact_c.weights(synth.key(7, gname), synth.thresholds(), N, K)
        M = exact_c.scales(synth.key(8, gname), N, K, synth.M_LO, synth.M_HI)
        run = lambda rows_: _median_time(lambda: O.linear_group_t(rng.integers(-127, 128, (rows_, K)), w, M, abits=7,
                                                                   n_chunk=2048), 1)
        if full:
            t = run(2048)
        else:   # a fixed cost per call (the weights' float64 conversion) plus a cost per row: a line through 128 and 256
            t128, t256 = run(128), run(256)
            t = t128 + (t256 - t128) * (2048 - 128) / 128
        c3[gname] = {"s": round(t, 2), "GOPS": round(2.0 * 2048 * K * N / t / 1e9, 1)}
        del w, M
    S, hd, H = 2048, 128, 28
    q = rng.integers(-(1 << 20), 1 << 20, (S, hd))
    k = rng.integers(-(1 << 20), 1 << 20, (S, hd))
    v = rng.integers(-(1 << 30), 1 << 30, (S, hd))
    valid = np.tril(np.ones((S, S), bool))
    heads = H if full else 1
    t = sum(_median_time(lambda: O.attention_head(q, k, v, valid, O.inv_sqrt_hd(hd)), 1) for _ in range(heads)) * (H / heads)
    c3["attention_S2048_H28"] = {"s": round(t, 2), "GOPS": round(2 * 2 * (S * (S + 1) // 2) * hd * H / t / 1e9, 2)}
    out["C3_prefill"] = c3
    progress("CPU baseline: C3 done")
    c3["sample"] = ("the full 2048 rows, every head" if full else
                    "GEMMs at 128 and 256 of the 2048 rows, extrapolated linearly in the rows; one of the 28 heads x 28")
    # C4 / C5: one layer's decode step x layers + head
    for key_, name, ctx in (("C4_qwen2.5-14b_bs1", "qwen2.5-14b", 128), ("C5_qwen1.5-moe-a2.7b_bs1", "qwen1.5-moe-a2.7b", 256)):
        t_l, t_h, nl = cpu_layer_step(name, ctx)
        progress(f"CPU baseline: {key_} layer done")
        out[key_] = {"kv_cached_s_per_token": round(nl * t_l + t_h, 3), "layer_step_s": round(t_l, 3),
                     "head_s": round(t_h, 3), "sample": f"one layer's KV-cached decode step at a {ctx}-token context "
                                                        f"(median of 3) x {nl} + head"}
    out["C1_qwen2.5-0.5b"] = cpu_model_c1(full)
    return out


def cpu_model_c1(full=False):
    """The oracle's whole-model decode (the reference's numpy CPU path, exact_llm.py:161-180, 262-268) for the
    Qwen2.5-0.5B-shape model of the C1 config, 16-token prompt + 64 greedy tokens, both variants of the reference's
    generate: KV-cached (one new row per step, run in full) and as-reference (the whole sequence recomputed every
    step: bounded runs time the steps at 17 and 80 positions and sum the 64 steps linearly between them)."""
    import numpy as np
    O, exact_c, synth = _oracle_env()
    cfg = synth.CONFIGS["qwen2.5-0.5b"]
    seed = 11
    t0 = time.perf_counter()
    layers = []
    for i in range(cfg.NL):
        L = dict(g1=synth.vector_np(synth.key(seed, f"L{i}.g1"), cfg.D, *synth.GAIN),
                 g2=synth.vector_np(synth.key(seed, f"L{i}.g2"), cfg.D, *synth.GAIN))
        for name, N, K, bias in synth.linear_specs(cfg, i):
            L[name.split(".", 1)[1]] = _oracle_lin(seed, name, N, K, bias)
        layers.append(L)
    thr = synth.thresholds()
    ew = exact_c.weights(synth.key(seed, "emb.w"), thr, cfg.V, cfg.D)
    eM = exact_c.scales(synth.key(seed, "emb.m"), cfg.V, cfg.D, synth.M_LO, synth.M_HI)
    m = O.Model(dict(emb=exact_c.embed(ew, eM), gf=synth.vector_np(synth.key(seed, "gf"), cfg.D, *synth.GAIN),
                     layers=layers, head=O.Lin(ew, eM)),
                dict(D=cfg.D, H=cfg.H, KV=cfg.KV, hd=cfg.hd, NL=cfg.NL, theta=cfg.theta, T=96, topk=0))
    build_s = time.perf_counter() - t0
    ids = np.random.default_rng(0).integers(0, cfg.V, 16).tolist()

    def cached_run():
        O.greedy_decode(m, ids, 64, cached=True)

    reps = 3 if full else 1
    if full:
        kv_s = _median_time(cached_run, reps, "C1 KV-cached 16 + 64")
    else:   # the prompt and 8 steps, the other 55 steps at the median step time
        cache = m.new_cache()
        t0 = time.perf_counter()
        tok = int(m(ids, cache)[-1].argmax())
        pre_s = time.perf_counter() - t0
        ts = []
        for _ in range(8):
            t0 = time.perf_counter()
            tok = int(m([tok], cache)[-1].argmax())
            ts.append(time.perf_counter() - t0)
        kv_s = pre_s + 63 * float(np.median(ts))
    res = {"cores": os.cpu_count(), "kind": "port", "model_build_s": round(build_s, 1),
           "kv_cached_s": round(kv_s, 2), "kv_cached_tok_s": round(64 / kv_s, 3)}
    if full:
        ar_s = _median_time(lambda: O.greedy_decode(m, ids, 64, cached=False), reps, "C1 as-reference 16 + 64")
        res.update(as_reference_s=round(ar_s, 2), as_reference_tok_s=round(64 / ar_s, 3),
                   sample="16 + 64 tokens, both variants in full, median of 3")
    else:
        t17 = _median_time(lambda: m(ids + [1]), 1)
        t80 = _median_time(lambda: m(ids + list(range(1, 65))), 1)
        ar_s = t17 + sum(t17 + (t80 - t17) * (n - 17) / 63.0 for n in range(18, 81))
        res.update(as_reference_s=round(ar_s, 2), as_reference_tok_s=round(64 / ar_s, 3),
                   as_reference_step_s_at_17=round(t17, 3), as_reference_step_s_at_80=round(t80, 3),
                   sample="16 + 64 tokens; KV-cached: the prompt and 8 steps timed, 63 steps at their median; "
                          "as-reference: its steps at 17 and 80 positions timed, linear in between")
    return res


def gemv_op_pass(args):
    """The reference's decode GEMVs through its own op, exact::gemv (speed_fair_kaggle.py:686-702, called per linear by
    TLinG), on its own tensors: per 7B layer q, k, v, o, gate, up (N x 3584) and down (3584 x 18944) + lm_head, wT int8
    (N, K) row-major, Mg int64 (N, K/128), x int16; one HIP graph of 28 layers + head over distinct weights. Bytes per
    call: N K + 8 N G + 2 K + 8 N."""
    import torch
    dev = "cuda"
    D, I, V = 3584, 18944, 152064
    shapes = {"q": (D, D), "k": (512, D), "v": (512, D), "o": (D, D), "gate": (I, D), "up": (I, D), "down": (D, I)}
    g = torch.Generator(device=dev).manual_seed(5)

    def mk(N, K):
        w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8, device=dev)
        return w, torch.randint(1, 1 << 27, (N, K // 128), generator=g, dtype=torch.int64, device=dev)

    layers = [{k: mk(*v) for k, v in shapes.items()} for _ in range(28)]
    head = mk(V, D)
    xd = torch.randint(-32767, 32768, (D,), generator=g, dtype=torch.int16, device=dev)
    xi = torch.randint(-32767, 32768, (I,), generator=g, dtype=torch.int16, device=dev)
    E = torch.ops.exact
    nbytes = lambda N, K: N * K + 8 * N * (K // 128) + 2 * K + 8 * N
    pass_bytes = 28 * sum(nbytes(*v) for v in shapes.values()) + nbytes(V, D)

    def step():
        for L in layers:
            for k, (w, M) in L.items():
                E.gemv(xi if k == "down" else xd, w, M)
        E.gemv(xd, *head)

    step()
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        step()
    gr.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    a.record(st)
    for _ in range(reps):
        gr.replay()
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    del gr, layers, head
    torch.cuda.empty_cache()
    return {"tok_s": round(1000.0 / ms, 2), "ms_per_pass": round(ms, 4), "GBps": round(pass_bytes / ms / 1e6, 1),
            "frac_hbm": round(pass_bytes / ms / 1e6 / HBM_PEAK_GBPS, 4), "GB_per_pass": round(pass_bytes / 1e9, 3),
            "calls_per_pass": 28 * 7 + 1}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-full", action="store_true",
                    help="the CPU baseline in full (every row and head, both C1 variants run whole, median of 3)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-model", action="store_true", help="skip the model runs other than the 7B headline")
    ap.add_argument("--no-gemv", action="store_true", help="skip the isolated GEMV passes")
    ap.add_argument("--models", default="c1,c4,c4b8,c5", help="other model decode runs: c1, c4, c4b8, c5")
    ap.add_argument("--no-trace", action="store_true", help="skip the trace-capture cost runs (7B decode T0-T3)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also copy 512 MiB on the device three times (calibrates the HBM traffic counters)")
    ap.add_argument("--cpu-only", action="store_true", help="only the CPU baseline (no GPU work); prints its JSON")
    ap.add_argument("--no-headline", action="store_true",
                    help="skip the 7B decode headline (for profiling the other parts); prints their JSON without a value")
    args = ap.parse_args()
    if args.cpu_only:
        print(json.dumps(cpu_baseline(full=args.cpu_full)), flush=True)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the exact path runs on a single MI355X here; runs over several GPUs "
              "(row blocks, KV heads or experts sharded, one int64 all-reduce per split linear) are not part of it.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    import exact_amd
    exact_amd.load()
    if args.copy_probe:
        src = torch.randint(0, 100, (512 << 20,), dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # the headline: full-model Qwen2.5-7B-shape decode, batch 1, int16 activations (the spec), timed over --steps steps
    mdl = None if args.no_headline else model_decode(args)
    if mdl is not None:
        progress(f"7B decode {mdl['tok_s']} tok/s")
    r = None if args.no_gemv else gemv_pass(args)
    progress("GEMV pass done")
    op = None if args.no_gemv else gemv_op_pass(args)
    progress("exact::gemv pass done")
    pre = {} if args.no_prefill else prefill_gemm(args)
    models, trc = None, None
    if not args.no_model:
        want = set(args.models.split(","))
        runs = {"C1_qwen2.5-0.5b_bs1": ("c1", "qwen2.5-0.5b", 16, 1), "C4_qwen2.5-14b_bs1": ("c4", "qwen2.5-14b", 128, 1),
                "C4_qwen2.5-14b_bs8": ("c4b8", "qwen2.5-14b", 128, 8),
                "C5_qwen1.5-moe-a2.7b_bs1": ("c5", "qwen1.5-moe-a2.7b", 256, 1)}
        models = {}
        for k, (tag, n, p_, b) in runs.items():
            if tag in want:
                models[k] = model_decode(args, n, p_, B=b)
                progress(f"{k} {models[k]['tok_s']} tok/s")
        trc = None if args.no_trace else trace_capture(args)
    att = None if args.no_prefill else attention_prefill(args)
    att64 = None if args.no_prefill else attention_prefill(args, H=14, KV=2, hd=64)   # the 0.5B's heads
    progress("prefill GEMM / attention / trace done")
    cpu = None if args.no_cpu else cpu_baseline(full=args.cpu_full)
    if mdl is None:   # a profiling run of the other parts: no headline value
        print(json.dumps({"metric": METRIC, "value": None, "headline": "skipped (--no-headline)", "gemv_c2": r,
                          "exact_gemv_op": op, "prefill_gemm": pre, "attention_prefill": att,
                          "attention_prefill_hd64": att64, "model_configs": models,
                          "trace_capture": trc, "cpu_baseline": cpu}, default=str), flush=True)
        return
    wbytes = mdl["weights_GB_per_step"] * 1e9
    step_gbps = wbytes / (mdl["ms_per_step"] * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": mdl["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": mdl["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Qwen2.5-7B-shape integer model (28 layers, hidden 3584, 28/4 heads, intermediate 18944, "
                               "vocab 152064), random-init seeded int8 weights with group-128 int16 scales, batch-1 greedy "
                               "decode after a 16-token prompt: embedding, per layer RMSNorm + q|k|v + RoPE + exact "
                               "integer attention + o + RMSNorm + SwiGLU MLP, final RMSNorm, lm_head, argmax; int16 "
                               "activations (the spec's qrow 15), one HIP graph per step",
                   "batch": 1, "abits": 15, "prompt": mdl["prompt"], "weights_GB_per_step": mdl["weights_GB_per_step"],
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(step_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(step_gbps / HBM_PEAK_GBPS, 4), "traffic": STEP_TRAFFIC_BYTES,
                     "algorithmic_bytes": int(wbytes), "unit_of_work": "one decode step (embedding to greedy token, one "
                                                                       "graph replay): int8 weights + int16 scales read"},
        "model_decode": mdl,
        "model_configs": models,
        "prefill_gemm": pre,
        "prefill_TOPS": (round(min(v["TOPS"] for k, v in pre.items() if not k.endswith("_a16")), 2) if pre else None),
        "prefill_TOPS_a16": (round(min(v["TOPS"] for k, v in pre.items() if k.endswith("_a16")), 2) if pre else None),
        "attention_prefill": att,
        "attention_prefill_hd64": att64,
        "trace_capture": trc,
        "exact_gemv_op": op,
        "cpu_baseline": None if cpu is None else dict(
            value=cpu["qwen2.5-7b_bs1"]["kv_cached_tok_s"], unit="tok/s", cores=cpu["cores"], kind="port",
            sample="Qwen2.5-7B-shape bs1 KV-cached decode on the numpy oracle (the reference's CPU algorithm): "
                   + cpu["qwen2.5-7b_bs1"]["sample"], per_config=cpu),
    }
    if r is not None:
        dom = r["per"]["gateup"]
        line["gemv_c2"] = {
            "workload": "Qwen2.5-7B-shape bs1 decode GEMV pass: 28 x (q|k|v 4608x3584, o 3584x3584, gate|up 37888x3584, "
                        "down 3584x18944) + lm_head 152064x3584, x int8 U[-127,127] (A8), group-128 int16 scales, "
                        "int64 outputs, one HIP graph",
            "tok_s": round(1000.0 / r["ms"], 2), "ms_per_pass": round(r["ms"], 4),
            "GBps": round(r["pass_bytes"] / (r["ms"] * 1e-3) / 1e9, 1), "GB_per_pass": round(r["pass_bytes"] / 1e9, 3),
            "per_shape": r["per"],
            "bs8": {"tok_s": round(8000.0 / r["bs8"]["ms"], 2), "ms_per_pass": round(r["bs8"]["ms"], 4),
                    "GBps": round(r["bs8"]["pass_bytes"] / (r["bs8"]["ms"] * 1e-3) / 1e9, 1), "per_shape": r["bs8"]["per"]},
            "roofline_kernel": {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                                "frac": round(dom["GBps"] / HBM_PEAK_GBPS, 4), "traffic": GATEUP_TRAFFIC_BYTES,
                                "algorithmic_bytes": GATEUP_BYTES,
                                "kernel": "k_gemv_g128<7,true,1,16> on gate|up 37888x3584, bs1 A8"},
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
