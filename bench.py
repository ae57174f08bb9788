"""Benchmark: Qwen2.5-7B-shape batch-1 decode GEMV pass on one MI355X.

One step = the exact group-128 int8 GEMVs of one 7B decode token over distinct weights resident in
HBM: 28 layers x {q|k|v (4608 x 3584), o (3584 x 3584), gate|up (37888 x 3584), down (3584 x 18944)}
plus lm_head (152064 x 3584) = 7.07 GB of int8 weights + 0.11 GB of int16 scales, x int8 uniform in
[-127, 127] (A8), int64 outputs, captured in one HIP graph. value = steps per second (tok/s).
Also reported: the pass's HBM rate, per-shape GEMV rates (HIP events on the launch stream), the
prefill GEMM rate (M = 2048, K = 3584 -> N = 18944 and K = 18944 -> N = 3584) and the numpy oracle
timed on the host cores as the CPU baseline.

Also: full-model decode (embedding to greedy token) of the 7B shape, the 0.5B (bs1), 14B (bs1, bs8) and
MoE (bs1) configurations, and the exact integer attention of a 2048-token prefill layer.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill] [--no-model]
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
# 512 MiB device copy (profiles/gemv_gateup_7b_traffic.md)
GATEUP_TRAFFIC_BYTES = 139_850_000
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
    del tm, gd, cache
    torch.cuda.empty_cache()
    return {"model": name, "batch": B, "tok_s": round(1000.0 * B / ms, 2), "ms_per_step": round(ms, 4), "abits": 15,
            "weights_GB_per_step": round(wbytes / 1e9, 3), "GBps": round(wbytes / ms / 1e6, 1),
            "frac_hbm": round(wbytes / ms / 1e6 / HBM_PEAK_GBPS, 4), "prompt": prompt_len,
            "prefill_ms_per_sequence": round(prefill_ms, 3), "prefill_eager_ms_per_sequence": round(eager_ms, 3)}


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
    """Exact integer causal attention of one 2048-token prefill layer (28 q / 4 kv heads, hd 128) from the
    KV cache: algorithmic ops 2*(S(S+1)/2)*hd*H for q.k and the same for p.v."""
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
        x = torch.randint(-127, 128, (M, K), dtype=torch.int8).to(dev)
        out = torch.empty((M, N), dtype=torch.int64, device=dev)
        ops.gemm_g128(x, 7, lin, out)
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 3
        a.record(st)
        for _ in range(reps):
            ops.gemm_g128(x, 7, lin, out)
        b.record(st)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1000.0 / reps
        res[name] = dict(us=round(us, 1), TOPS=round(2.0 * M * K * N / us / 1e6, 2))
        del wp, mp, lin, x, out
    torch.cuda.empty_cache()
    return res


def cpu_baseline():
    """The oracle's group-128 linear (float64 BLAS per group + int64 rescale, the reference's CPU
    algorithm) on one 7B layer's GEMVs + the head, bs1 A8, timed on this host; extrapolated to a token."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import exact_oracle as O
    rng = np.random.default_rng(0)
    shapes = {"q": (3584, 3584), "k": (512, 3584), "v": (512, 3584), "o": (3584, 3584), "gate": (18944, 3584),
              "up": (18944, 3584), "down": (3584, 18944)}
    t_layer = 0.0
    for name, (N, K) in shapes.items():
        w = rng.integers(-127, 128, (K, N), dtype=np.int8)
        M = rng.integers(8192, 24576, (K // 128, N))
        x = rng.integers(-127, 128, (1, K))
        t0 = time.perf_counter()
        O.linear_group_t(x, w, M, abits=7)
        t_layer += time.perf_counter() - t0
    N, K = 152064, 3584
    w = rng.integers(-127, 128, (K, N), dtype=np.int8)
    M = rng.integers(8192, 24576, (K // 128, N))
    x = rng.integers(-127, 128, (1, K))
    t0 = time.perf_counter()
    O.linear_group_t(x, w, M, abits=7)
    t_head = time.perf_counter() - t0
    tok_s = 1.0 / (28 * t_layer + t_head)
    return {"value": round(tok_s, 4), "unit": "tok/s", "cores": os.cpu_count(), "kind": "port",
            "sample": f"one 7B layer's 7 GEMVs ({t_layer:.2f} s) + lm_head ({t_head:.2f} s), bs1 A8, numpy oracle "
                      "(float64 BLAS per group), extrapolated as 28 layers + head"}


def cpu_model_c1():
    """The oracle's whole-model decode on the host (the reference's numpy CPU path, exact_llm.py:161-180, 262-268) for
    the Qwen2.5-0.5B-shape model of the C1 config, both variants of the reference's generate: KV-cached (one new row
    per step) and as-reference (the whole sequence recomputed every step). A bounded sample: a 16-token prompt, then
    2 cached decode steps and 1 uncached step at length 17."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import exact_c
    import exact_oracle as O
    from exact_amd import synth
    cfg = synth.CONFIGS["qwen2.5-0.5b"]
    seed = 11
    thr = synth.thresholds()
    t0 = time.perf_counter()

    def lin(name, N, K, bias):   # the synthetic model's integers, from the oracle's C generator
        key = lambda s_: synth.key(seed, name + s_)
        b = synth.vector_np(key(".b"), N, *synth.BIAS) if bias else None
        return O.Lin(exact_c.weights(key(".w"), thr, N, K), exact_c.scales(key(".m"), N, K, synth.M_LO, synth.M_HI), b)

    layers = []
    for i in range(cfg.NL):
        L = dict(g1=synth.vector_np(synth.key(seed, f"L{i}.g1"), cfg.D, *synth.GAIN),
                 g2=synth.vector_np(synth.key(seed, f"L{i}.g2"), cfg.D, *synth.GAIN))
        for name, N, K, bias in synth.linear_specs(cfg, i):
            L[name.split(".", 1)[1]] = lin(name, N, K, bias)
        layers.append(L)
    ew = exact_c.weights(synth.key(seed, "emb.w"), thr, cfg.V, cfg.D)
    eM = exact_c.scales(synth.key(seed, "emb.m"), cfg.V, cfg.D, synth.M_LO, synth.M_HI)
    m = O.Model(dict(emb=exact_c.embed(ew, eM), gf=synth.vector_np(synth.key(seed, "gf"), cfg.D, *synth.GAIN),
                     layers=layers, head=O.Lin(ew, eM)),
                dict(D=cfg.D, H=cfg.H, KV=cfg.KV, hd=cfg.hd, NL=cfg.NL, theta=cfg.theta, T=64, topk=0))
    build_s = time.perf_counter() - t0
    ids = np.random.default_rng(0).integers(0, cfg.V, 16).tolist()
    cache = m.new_cache()
    t0 = time.perf_counter()
    lg = m(ids, cache)
    prefill_s = time.perf_counter() - t0
    tok = int(lg[-1].argmax())
    t0 = time.perf_counter()
    for _ in range(2):
        tok = int(m([tok], cache)[-1].argmax())
    cached_s = (time.perf_counter() - t0) / 2
    t0 = time.perf_counter()
    m(ids + [tok])
    uncached_s = time.perf_counter() - t0
    return {"unit": "tok/s", "cores": os.cpu_count(), "kind": "port",
            "kv_cached_tok_s": round(1.0 / cached_s, 3), "as_reference_tok_s_at_17": round(1.0 / uncached_s, 3),
            "prefill_16_s": round(prefill_s, 2), "model_build_s": round(build_s, 1),
            "sample": "Qwen2.5-0.5B-shape integer model (24 layers, group-128 A16), numpy oracle: 16-token prompt, "
                      "2 KV-cached decode steps, 1 step recomputing all 17 positions"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-model", action="store_true")
    ap.add_argument("--no-gemv", action="store_true", help="skip the GEMV pass (profiling runs of the other parts)")
    ap.add_argument("--models", default="7b,c1,c4,c4b8,c5", help="model decode runs: 7b, c1, c4, c4b8, c5")
    ap.add_argument("--no-trace", action="store_true", help="skip the trace-capture cost runs (7B decode T0-T3)")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also copy 512 MiB on the device three times (calibrates the HBM traffic counters)")
    args = ap.parse_args()
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
    r = None if args.no_gemv else gemv_pass(args)
    pre = {} if args.no_prefill else prefill_gemm(args)
    mdl, models, trc = None, None, None
    if not args.no_model:
        want = set(args.models.split(","))
        mdl = model_decode(args) if "7b" in want else None
        runs = {"C1_qwen2.5-0.5b_bs1": ("c1", "qwen2.5-0.5b", 16, 1), "C4_qwen2.5-14b_bs1": ("c4", "qwen2.5-14b", 128, 1),
                "C4_qwen2.5-14b_bs8": ("c4b8", "qwen2.5-14b", 128, 8),
                "C5_qwen1.5-moe-a2.7b_bs1": ("c5", "qwen1.5-moe-a2.7b", 256, 1)}
        models = {k: model_decode(args, n, p, B=b) for k, (tag, n, p, b) in runs.items() if tag in want}
        trc = trace_capture(args) if "7b" in want and not args.no_trace else None
    att = None if args.no_prefill else attention_prefill(args)
    cpu = None if args.no_cpu else cpu_baseline()
    cpu_c1 = None if args.no_cpu else cpu_model_c1()
    if r is None:
        print(json.dumps({"metric": METRIC, "value": None, "model_decode": mdl, "model_configs": models,
                          "trace_capture": trc, "prefill_gemm": pre, "attention_prefill": att}), flush=True)
        return
    tok_s = 1000.0 / r["ms"]
    pass_gbps = r["pass_bytes"] / (r["ms"] * 1e-3) / 1e9
    dom = r["per"]["gateup"]
    line = {
        "metric": METRIC, "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(r["ms"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Qwen2.5-7B-shape bs1 decode GEMV pass: 28 x (q|k|v 4608x3584, o 3584x3584, "
                               "gate|up 37888x3584, down 3584x18944) + lm_head 152064x3584, group-128 int16 scales, "
                               "A8 x, int64 outputs, one HIP graph", "batch": 1, "abits": 7,
                   "weights_GB": round(r["pass_bytes"] / 1e9, 3), "parallelism": "single GPU"},
        "gemv_GBps": round(pass_gbps, 1),
        "gemv_per_shape": r["per"],
        "gemv_bs8": {"tok_s": round(8000.0 / r["bs8"]["ms"], 2), "ms_per_step": round(r["bs8"]["ms"], 4),
                     "GBps": round(r["bs8"]["pass_bytes"] / (r["bs8"]["ms"] * 1e-3) / 1e9, 1), "per_shape": r["bs8"]["per"]},
        "model_decode": mdl,
        "model_configs": models,
        "trace_capture": trc,
        "prefill_gemm": pre,
        "attention_prefill": att,
        "prefill_TOPS": (round(min(v["TOPS"] for v in pre.values()), 2) if pre else None),
        "roofline": {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dom["GBps"] / HBM_PEAK_GBPS, 4), "traffic": GATEUP_TRAFFIC_BYTES,
                     "algorithmic_bytes": GATEUP_BYTES,
                     "kernel": "k_gemv_g128<7,true,1,16> on gate|up 37888x3584, bs1 A8"},
        "cpu_baseline": cpu,
        "cpu_model_c1": cpu_c1,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
