"""Trace capture and commitment of the totals t = sum_g M_g (x_g . W_g) of every linear.

Prover side (the reference's fast GPU engine, experiments/prover_commit_cost_gpu_kaggle.py:727-845 and
experiments/gpu_engine_trace_verify_kaggle.py:776-798):
  T1  every linear's pre-rounding total t lands in a static trace buffer inside the decode graph;
  T2  the step's trace is copied to pinned host memory on a side stream;
  T3  each step's host trace is committed: SHA-256 of 4 equal chunks in parallel threads, then SHA-256 of the
      4 digests (a Merkle root over 4 leaves).
Here T1 costs no copy: the GEMVs accumulate straight into the trace buffer's slots, the consumer kernels read
them there without clearing them, and one fill kernel zeroes the buffer at the start of each pass. Device
buffers and pinned host buffers are both double-buffered, so step j's copy and hash overlap step j + 1
(TraceRecorder states the ordering rules).

The verifier side (the Freivalds keys and check of gpu_engine_trace_verify_kaggle.py:799-833) is not part of this
package; the tests hold a restatement of it to check captured traces.
"""
import hashlib
import queue
import threading
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from ._lib import ExactError

I64 = torch.int64


# ----------------------------------------------------------------------------- layout
class TraceLayout:
    """Where each linear's totals sit in one pass's trace of R rows: per layer q|k|v (R, nq), o (R, D),
    gate|up (R, 2I), down (R, D), then the head (R, V); each block row-major. With the fused parts adjacent
    (64-row aligned sizes, every model here), a row block holds the reference's q, k, v, o, gate, up, down
    values in the reference's call order (prover_commit_cost_gpu_kaggle.py:740-741)."""

    def __init__(self, weights, R):
        if weights.mode != "group" or weights.cfg.moe:
            raise ExactError("trace capture covers dense models with group-128 linears")
        self.R = R
        self.blocks = []   # (key, offset, N, parts): parts = [(reference name, column offset, width)]
        off = 0
        for li, L in enumerate(weights.layers):
            for key in ("qkv", "o", "gateup", "down"):
                lin = L[key]
                self.blocks.append((f"L{li}.{key}", off, lin.N, [(f"L{li}.{nm}", o, n) for nm, o, n in lin.parts]))
                off += R * lin.N
        head = weights.head
        self.blocks.append(("head", off, head.N, [("head", 0, head.N)]))
        off += R * head.N
        self.total = off
        self._index = {b[0]: b for b in self.blocks}

    def slot(self, buf, key):
        """(R, N) view of block `key` in a device or host trace buffer."""
        _, off, N, _ = self._index[key]
        return buf[off:off + self.R * N].view(self.R, N) if isinstance(buf, torch.Tensor) else \
            buf[off:off + self.R * N].reshape(self.R, N)

    def split(self, host):
        """{reference name: (R, n) int64 array} of a host trace (names L{i}.q ... L{i}.down, head)."""
        host = np.asarray(host)
        out = {}
        for key, off, N, parts in self.blocks:
            blk = host[off:off + self.R * N].reshape(self.R, N)
            for name, o, n in parts:
                out[name] = blk[:, o:o + n]
        return out


# ----------------------------------------------------------------------------- commitment
_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        _POOL = ThreadPoolExecutor(8)   # two commitments of 4 leaves at a time
    return _POOL


def commit(arr, leaves=4):
    """SHA-256 Merkle root over `leaves` equal chunks of an int64 array's little-endian bytes
    (prover_commit_cost_gpu_kaggle.py:803-806): sha256(sha256(chunk_0) || ... || sha256(chunk_{leaves-1})).
    hashlib releases the interpreter lock on large buffers, so the chunks hash in parallel; they are hashed in
    place (no bytes copy made while holding the lock)."""
    a = np.ascontiguousarray(arr, dtype="<i8")
    step = (len(a) + leaves - 1) // leaves
    parts = list(_pool().map(lambda i: hashlib.sha256(memoryview(a[i * step:(i + 1) * step]).cast("B")).digest(),
                             range(leaves)))
    return hashlib.sha256(b"".join(parts)).digest()


class TraceRecorder:
    """Trace capture for a GraphDecoder built with trace=True. mode:
      "device"  T1: the trace stays in the device buffers (the graphs write it; nothing more per step);
      "host"    T2: + copy of each step's trace to pinned host memory on a side stream;
      "commit"  T3: + the commitment of each step's host trace, by one worker thread per pinned buffer
                (two steps hash at once, each over 4 threads).
    GraphDecoder.step calls before_step(b) / after_step(b) around the replay that writes device buffer b;
    finish() copies the last step, drains the work and returns the digests (commit) or None. keep=True also
    keeps a host copy of every step's trace (for checks).

    Ordering without any GPU-side wait between streams (such waits stalled every step by about 12% on the
    7B decode): step j's copy is issued by the host once step j's completion event has fired, which it
    does while step j + 1 runs; the replay that overwrites a device buffer is issued only after that
    buffer's copy has finished (the host waits on the copy's event, about 0.23 ms for 12.3 MB, well within
    a step); a pinned buffer is refilled only after the worker has hashed it."""

    def __init__(self, gd, mode="commit", keep=False):
        if mode not in ("device", "host", "commit"):
            raise ExactError(f"trace mode {mode!r}")
        self.gd, self.mode, self.keep = gd, mode, keep
        n = gd.layout.total
        self.pins = [torch.empty(n, dtype=I64, pin_memory=True) for _ in range(2)] if mode != "device" else []
        self.side = torch.cuda.Stream() if mode != "device" else None
        self.step_ev = [None, None]       # completion of the last step that wrote device buffer i, not yet copied
        self.copy_ev = [None, None]       # completion of the last copy out of device buffer i
        self.free = [threading.Event(), threading.Event()]   # pinned buffer i may be overwritten
        for e in self.free:
            e.set()
        self._digests, self._kept = {}, {}
        self.ncopied = 0
        self.qs = [queue.Queue(), queue.Queue()]
        self.workers = []
        if mode == "commit" or (mode == "host" and keep):
            self.workers = [threading.Thread(target=self._work, args=(i,), daemon=True) for i in range(2)]
            for w in self.workers:
                w.start()

    def _work(self, i):
        while True:
            item = self.qs[i].get()
            if item is None:
                return
            j, ev = item
            ev.synchronize()
            arr = self.pins[i].numpy()
            if self.keep:
                self._kept[j] = arr.copy()
            if self.mode == "commit":
                self._digests[j] = commit(arr)
            self.free[i].set()

    @property
    def digests(self):
        return [self._digests[j] for j in sorted(self._digests)]

    @property
    def kept(self):
        return [self._kept[j] for j in sorted(self._kept)]

    def _copy(self, b):
        """Copy device buffer b (its step has finished) to pinned buffer b on the side stream."""
        self.step_ev[b].synchronize()
        self.step_ev[b] = None
        self.free[b].wait()
        self.free[b].clear()
        with torch.cuda.stream(self.side):
            self.pins[b].copy_(self.gd.trace_bufs[b], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.side)
        self.copy_ev[b] = ev
        j, self.ncopied = self.ncopied, self.ncopied + 1
        if self.workers:
            self.qs[b].put((j, ev))
        else:
            self.free[b].set()   # T2 alone: copies into one pinned buffer follow each other on the side stream

    def before_step(self, b):
        if self.mode == "device":
            return
        if self.step_ev[b] is not None:     # only when steps outran after_step's copies (not in GraphDecoder)
            self._copy(b)
        if self.copy_ev[b] is not None:
            self.copy_ev[b].synchronize()
            self.copy_ev[b] = None

    def after_step(self, b):
        if self.mode == "device":
            if self.keep:
                self._kept[len(self._kept)] = self.gd.trace_bufs[b].cpu().numpy()
            return
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream())
        self.step_ev[b] = ev
        if self.step_ev[1 - b] is not None:   # the previous step: finished by now or soon (this one is queued)
            self._copy(1 - b)

    def finish(self):
        for b in (0, 1):   # after after_step only the last step is still uncopied
            if self.step_ev[b] is not None:
                self._copy(b)
        for q in self.qs:
            q.put(None)
        for w in self.workers:
            w.join()
        self.workers = []
        if self.side is not None:
            self.side.synchronize()
        return self.digests if self.mode == "commit" else None
