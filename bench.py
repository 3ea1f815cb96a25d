#!/usr/bin/env python3
"""Benchmark of zwhisper's attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload N] [--only] [--dense-math x3|fp32]
                    [--extra NAME] [--no-cpu] [--no-parity]

A step is one pass of the attention path over one batch of synthetic input, already resident
in HBM.  The headline line (one JSON object on stdout) is workload 2, Whisper base.en encoder
self-attention over 16 windows x 1500 frames (8 heads x 64, K transposed), in TFLOP/s of
algorithmic work (4*d*H per visible (q, k) pair, src/bench.zig:76).  stdout carries only that
line, a few KB.  The other four workloads are measured too (unless --only): the headline line lists
each under "workloads" with its value, step time and roofline fraction, and stderr carries every
workload's full record, one "[bench-record] {...}" line each (src/bench.zig:51-78 likewise prints
one short line per measurement).  Each has its own roofline: 16-bit MFMA (2.5 PFLOP/s, f16 and bf16 alike) for the dense ones, whose kernel
computes each f32 product as three 16-bit products of hi/lo-split operands (ceiling: a third of
that peak), HBM (8 TB/s) for the decode ones.  Unless --only, the three dense workloads are also
run on the fp32-MFMA kernel ("*_fp32mfma", fp32 peak 157.3 TFLOP/s).  Every attention workload
carries "parity": its outputs against the f64 closed form, checked after the timed region, with
the bar of the arithmetic that ran.  The two encoder workloads also carry "dropin_host_buffers":
the host-pointer drop-in (zwg_attention_ex, H2D + kernels + D2H per window), which includes PCIe
and is never the headline value.

Timing: the card raises its clocks over the first tens of milliseconds of continuous load, so
each workload runs W untimed warm-up steps, K "cold" steps timed with one event pair (reported
as `cold`, the rate while the clocks ramp; never the value), untimed steps for 0.3 s, and then
exactly K steps bracketed by torch.cuda.synchronize() and by one pair of HIP events on the stream
the kernels run on: their wall time gives ms_per_step and `value`, the events' elapsed time over
K the kernel time used for the roofline (kernel_ms_mean) -- the rate a serving loop under steady
load sees.  K further steps, each between its own pair of events, give kernel_ms_median and
kernel_ms_min.  Decode workloads rotate between two copies of their inputs so no step finds its
K/V in the 256 MB last-level cache left by the previous one.
The CPU baseline is the C restatement of the reference's multithreaded attention (oracle/),
timed on this host's cores on a bounded sample of the same workload, on CPUs - 1 threads (the
reference's default pool) over the CPUs this job may use (affinity, cgroup quota and
OMP_NUM_THREADS; "host" in the line gives them and the CPU model), and on min(that, 4) threads for
decode (the reference's decode pool).

--extra NAME measures one of the workloads around the attention path alone; --workload N --only
[--dense-math fp32] one attention workload alone (the forms the rocprofv3 counter runs use).

Unless --only, the line also carries the device cache updates of three of the workloads (the K/V
rows of a step written into the HBM-resident caches, with rotary positions for Qwen2), as
"small_dec_kv_append_x32", "qwen15_kv_append_x64" and "qwen05_prefill_kv_append", each with an
HBM roofline and oracle/kv.py's update timed beside it, and the six linear layers of a base.en
encoder layer over the 16 windows ("base_enc_linear_x16", f16 weights on f16 MFMA) with the
oracle's ops.linear timed beside it, and three decode steps' linear layers over int8 block
weights (HBM-bound; "qwen15_logits_q8_x64", "qwen15_decode_q8_linear_x64",
"small_dec_q8_linear_x32") with the oracle's ops.linear over Q8 timed beside them, two decode
steps' q/k/v projections with the new K/V rows written into the device caches by the projections
themselves ("small_dec_qkv_cache_x32", "qwen15_qkv_cache_x64", with the unfused projections +
append timed beside them), one whole base.en encoder layer over the 16 windows
("base_enc_layer_x16") with the oracle's layer beside it, and the two callers' whole token steps
on the device, the Whisper small.en decoder over 32 windows ("small_dec_step_x32") and Qwen2.5-1.5B
over 64 sequences ("qwen15_step_x64"), each with the same step as separate calls and the oracle's
forward for one token beside it, and Qwen2.5-0.5B's 2048-token prompt in 8 forward batches of 256
("qwen05_prompt_2048", with the oracle's forward over the first batch beside it).

Each attention workload also carries "rate": windows/s for the encoders, tokens/s for the decoder
step, the prefill and the LLM decode step, at wall time per step.  The prefill's CPU baseline runs
as llm.prompt does (8 calls of 256 rows); "cpu_baseline_one_call" times it as one 2048-row call.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_MFMA_F32 = 157.3e12  # FLOP/s, MI355X dense fp32 matrix
PEAK_MFMA_F16 = 2500e12  # FLOP/s, MI355X dense fp16 matrix
PEAK_HBM = 8.0e12  # B/s, MI355X HBM3E


CPU_MIN_SECONDS = 2.0  # each CPU baseline repeats its sample for at least this long


def time_cpu(run, min_reps: int = 5) -> tuple[float, float, int]:
    """One warm-up call, then repeated calls until both `min_reps` runs and CPU_MIN_SECONDS have
    passed (src/bench.zig:69-75 takes the best of 5 after one warm-up).  Returns (best, mean, runs)."""
    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or time.perf_counter() - t_start < CPU_MIN_SECONDS:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return min(times), float(np.mean(times)), len(times)


def cpu_timing(best: float, mean: float, runs: int) -> str:
    return f"best of {runs} runs over {CPU_MIN_SECONDS:g}+ s after one warm-up (mean {1e3 * mean:.2f} ms)"


def _cgroup_cpus():
    """CPUs this process's cgroup may use (cpu.max quota / period), or None when unlimited."""
    for path in ("/sys/fs/cgroup/cpu.max",):
        try:
            with open(path) as f:
                quota, period = f.read().split()[:2]
            if quota != "max":
                return float(quota) / float(period)
        except (OSError, ValueError):
            pass
    return None


def host_cpus() -> dict:
    """The CPUs this process may use: the affinity mask (what `nproc` reports), bounded by the
    cgroup's CPU quota and by OMP_NUM_THREADS when set (the share a shared host grants this job),
    and the CPU model."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    quota = _cgroup_cpus()
    try:
        omp = int(os.environ.get("OMP_NUM_THREADS", "")) or None
    except ValueError:
        omp = None
    limits = [nproc]
    if quota is not None:
        limits.append(int(math.ceil(quota)))
    if omp is not None:
        limits.append(omp)
    cpus = min(limits)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": nproc, "cgroup_cpus": quota, "omp_num_threads": omp, "cpus": max(1, cpus), "cpu_model": model}


def host_threads() -> int:
    """The reference's default pool size, CPUs - 1 (src/main.zig:126, src/capi.zig:71), over the
    CPUs this process may use (host_cpus)."""
    return max(1, host_cpus()["cpus"] - 1)


class Workload:
    """Device inputs for one benchmark workload and a step that runs it."""

    def __init__(self, number: int, torch, ctx, copies: int):
        from zwhisper_amd import workloads as W

        self.W = W
        self.number = number
        self.spec = W.WORKLOADS[number]
        self.torch = torch
        self.ctx = ctx
        self.copies = copies
        self.lengths = W.kv_lengths(number)
        self.work = W.algorithmic_work(number, self.lengths)
        self.sets = []
        self._setup()

    # ---- inputs
    def _dev(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def _setup(self):
        from zwhisper_amd.ops import AttnShape

        W, w, n = self.W, self.spec, self.number
        t = self.torch
        if n in (1, 2, 4):
            kt = W.kt_stride_for(w.n_kv_cap) if n != 4 else w.n_kv_cap
            qs, ks, vs = [], [], []
            for item in range(w.n_items):
                q, kl, v = W.make_dense(n, item)
                qs.append(q)
                ks.append(W.to_kt(kl, kt))
                vs.append(v)
            q, k, v = np.stack(qs), np.stack(ks), np.stack(vs)
            self.shape = AttnShape(w.n_q, w.n_kv_cap, w.n_head, w.n_head_kv, w.d, w.n_head * w.d,
                                   w.n_head_kv * w.d, w.n_head * w.d, w.causal, kt)
            self.host = {"q": q, "k": k, "v": v}
            base = {"q": self._dev(q), "k": self._dev(k), "v": self._dev(v)}
            base["out"] = t.empty((w.n_items, w.n_q, w.n_head * w.d), dtype=t.float32, device="cuda")
            self.bstrides = (q[0].size, k[0].size, v[0].size, w.n_q * w.n_head * w.d)
            self.sets = [base] + [{kk: (vv.clone() if kk != "out" else vv) for kk, vv in base.items()}
                                  for _ in range(self.copies - 1)]
        elif n == 3:
            ns = w.n_head * w.d
            cap, n_cross = w.n_kv_cap, w.extra["cross_n_kv"]
            qs = np.zeros((w.n_items, ns), np.float32)
            qc = np.zeros((w.n_items, ns), np.float32)
            ks = np.zeros((w.n_items, cap, ns), np.float32)
            vs = np.zeros((w.n_items, cap, ns), np.float32)
            kc = np.zeros((w.n_items, n_cross, ns), np.float32)
            vc = np.zeros((w.n_items, n_cross, ns), np.float32)
            for i in range(w.n_items):
                s = W.make_decoder_step(i)
                qs[i], qc[i] = s["q_self"][0], s["q_cross"][0]
                ks[i, : s["n_self"]], vs[i, : s["n_self"]] = s["k_self"], s["v_self"]
                kc[i], vc[i] = s["k_cross"], s["v_cross"]
            self.shape_self = AttnShape(1, cap, w.n_head, w.n_head, w.d, ns, ns, ns, True, None)
            self.shape_cross = AttnShape(1, n_cross, w.n_head, w.n_head, w.d, ns, ns, ns, False, None)
            nkv = t.from_numpy(self.lengths.astype(np.int32)).cuda()
            for c in range(self.copies):
                self.sets.append({
                    "qs": self._dev(qs), "qc": self._dev(qc), "ks": self._dev(ks), "vs": self._dev(vs),
                    "kc": self._dev(kc), "vc": self._dev(vc), "nkv": nkv,
                    "os": t.empty((w.n_items, ns), dtype=t.float32, device="cuda"),
                    "oc": t.empty((w.n_items, ns), dtype=t.float32, device="cuda"),
                })
            self.host = {"qs": qs, "qc": qc, "ks": ks, "vs": vs, "kc": kc, "vc": vc}
        elif n == 5:
            cap, ns, kvw = w.n_kv_cap, w.n_head * w.d, w.n_head_kv * w.d
            q = np.zeros((w.n_items, ns), np.float32)
            kt = np.zeros((w.n_items, w.n_head_kv, w.d, cap), np.float32)
            v = np.zeros((w.n_items, cap, kvw), np.float32)
            for i in range(w.n_items):
                qi, kl, vi, n_kv = W.make_llm_decode(i)
                q[i] = qi[0]
                kt[i] = W.to_kt(kl, cap)
                v[i, :n_kv] = vi
            self.shape = AttnShape(1, cap, w.n_head, w.n_head_kv, w.d, ns, kvw, ns, True, cap)
            nkv = t.from_numpy(self.lengths.astype(np.int32)).cuda()
            for c in range(self.copies):
                self.sets.append({"q": self._dev(q), "k": self._dev(kt), "v": self._dev(v), "nkv": nkv,
                                  "out": t.empty((w.n_items, ns), dtype=t.float32, device="cuda")})
            self.bstrides = (ns, kt[0].size, v[0].size, ns)
            self.host = {"q": q, "k": kt, "v": v}

    # ---- one step
    def step(self, i: int):
        self.last = i
        s = self.sets[i % len(self.sets)]
        w, ctx = self.spec, self.ctx
        if self.number in (1, 2, 4):
            qb, kb, vb, ob = self.bstrides
            ctx.attention_batch_dev(s["q"], s["k"], s["v"], self.shape, s["out"], w.n_items, qb, kb, vb, ob)
        elif self.number == 3:
            ns = w.n_head * w.d
            cap, n_cross = w.n_kv_cap, w.extra["cross_n_kv"]
            ctx.attention_batch_dev(s["qs"], s["ks"], s["vs"], self.shape_self, s["os"], w.n_items, ns, cap * ns,
                                    cap * ns, ns, s["nkv"])
            ctx.attention_batch_dev(s["qc"], s["kc"], s["vc"], self.shape_cross, s["oc"], w.n_items, ns,
                                    n_cross * ns, n_cross * ns, ns)
        else:
            qb, kb, vb, ob = self.bstrides
            ctx.attention_batch_dev(s["q"], s["k"], s["v"], self.shape, s["out"], w.n_items, qb, kb, vb, ob, s["nkv"])

    def parity(self, x3: bool) -> dict:
        """The last step's outputs against the f64 closed form (oracle/naive.py), outside the timed
        region: max abs error and normwise relative error ||gpu - ref||_inf / ||ref||_inf, with the
        bar of the arithmetic that ran (x3 dense: 5e-5 and 3e-5; f32: 2e-4 and 1e-3)."""
        from oracle import naive
        from zwhisper_amd.ops import AttnShape

        self.torch.cuda.synchronize()
        w, n, W = self.spec, self.number, self.W
        s = self.sets[self.last % len(self.sets)]
        pairs = []  # (got, ref)
        if n in (1, 2, 4):
            out = s["out"].cpu().numpy()
            items = [0, 7, 15] if n == 2 else [0]
            for i in items:
                pairs.append((out[i], naive.attention_f64(self.host["q"][i], self.host["k"][i], self.host["v"][i],
                                                          self.shape)))
            what = f"items {items} of {w.n_items}, every output"
        elif n == 3:
            ns = w.n_head * w.d
            os_, oc = s["os"].cpu().numpy(), s["oc"].cpu().numpy()
            h = self.host
            for i in range(w.n_items):
                L = int(self.lengths[i])
                sh = AttnShape(1, L, w.n_head, w.n_head, w.d, ns, ns, ns, True, None)
                pairs.append((os_[i], naive.attention_f64(h["qs"][i], h["ks"][i, :L], h["vs"][i, :L], sh)))
                pairs.append((oc[i], naive.attention_f64(h["qc"][i], h["kc"][i], h["vc"][i], self.shape_cross)))
            what = f"all {w.n_items} windows, self and cross"
            x3 = False
        else:
            ns, kvw, cap = w.n_head * w.d, w.n_head_kv * w.d, w.n_kv_cap
            out = s["out"].cpu().numpy()
            h = self.host
            for i in range(w.n_items):
                L = int(self.lengths[i])
                sh = AttnShape(1, L, w.n_head, w.n_head_kv, w.d, ns, kvw, ns, True, cap)
                pairs.append((out[i], naive.attention_f64(h["q"][i], h["k"][i], h["v"][i], sh)))
            what = f"all {w.n_items} sequences"
            x3 = False
        err = max(float(np.abs(g.astype(np.float64).reshape(-1) - r).max()) for g, r in pairs)
        ref_max = max(float(np.abs(r).max()) for _, r in pairs)
        bar = {"max_abs": 5e-5, "normwise_rel": 3e-5} if x3 else {"max_abs": 2e-4, "normwise_rel": 1e-3}
        rel = err / max(ref_max, 1e-30)
        return {"vs": "f64 closed form (oracle/naive.py)", "checked": what, "max_abs": err, "normwise_rel": rel,
                "bar": bar, "within_bar": err <= bar["max_abs"] and rel <= bar["normwise_rel"]}

    def dropin(self, reps: int = 3) -> dict:
        """The host-pointer drop-in (zwg_attention_ex), what the unchanged callers bind: one
        synchronous call per window or sequence on pageable host buffers, H2D of q/k/v (the spans
        the reference reads), the kernels and D2H of out, timed on the host clock.
          encoders: src/encoder.zig:167, one call per window;
          decoder step: src/decoder.zig:184 (self, the window's cache rows 0..n_kv) and :191 (cross,
            the window's 1500 encoder rows), two calls per window;
          LLM decode step: src/llm.zig:191-202, one call per sequence over its transposed cache
            (n_ctx columns) and its V rows 0..n_kv.
        Includes PCIe: never the headline value."""
        from zwhisper_amd.ops import AttnShape

        w, n = self.spec, self.number
        h = self.host
        calls = []  # (q, k, v, shape, out, device output row to compare with)
        if n in (1, 2):
            for i in range(w.n_items):
                calls.append((np.ascontiguousarray(h["q"][i]).reshape(-1), np.ascontiguousarray(h["k"][i]).reshape(-1),
                              np.ascontiguousarray(h["v"][i]).reshape(-1), self.shape,
                              np.zeros(w.n_q * w.n_head * w.d, np.float32), ("out", i)))
        elif n == 3:
            ns = w.n_head * w.d
            for i in range(w.n_items):
                L = int(self.lengths[i])
                sh = AttnShape(1, L, w.n_head, w.n_head, w.d, ns, ns, ns, True, None)
                calls.append((h["qs"][i].copy(), np.ascontiguousarray(h["ks"][i, :L]).reshape(-1),
                              np.ascontiguousarray(h["vs"][i, :L]).reshape(-1), sh, np.zeros(ns, np.float32),
                              ("os", i)))
                calls.append((h["qc"][i].copy(), np.ascontiguousarray(h["kc"][i]).reshape(-1),
                              np.ascontiguousarray(h["vc"][i]).reshape(-1), self.shape_cross, np.zeros(ns, np.float32),
                              ("oc", i)))
        else:
            ns, kvw, cap = w.n_head * w.d, w.n_head_kv * w.d, w.n_kv_cap
            for i in range(w.n_items):
                L = int(self.lengths[i])
                sh = AttnShape(1, L, w.n_head, w.n_head_kv, w.d, ns, kvw, ns, True, cap)
                calls.append((h["q"][i].copy(), np.ascontiguousarray(h["k"][i]).reshape(-1),
                              np.ascontiguousarray(h["v"][i, :L]).reshape(-1), sh, np.zeros(ns, np.float32),
                              ("out", i)))

        def run():
            for q, k, v, sh, out, _ in calls:
                self.ctx.attention_ex_host(q, k, v, sh, out)

        best, mean, runs = time_cpu(run, reps)
        self.torch.cuda.synchronize()
        s = self.sets[self.last % len(self.sets)]
        dev = {key: s[key].cpu().numpy() for key in {c[5][0] for c in calls}}
        diff = max(float(np.abs(out - dev[key][i].reshape(-1)).max()) for _, _, _, _, out, (key, i) in calls)
        moved = sum(q.nbytes + k.nbytes + v.nbytes + out.nbytes for q, k, v, _, out, _ in calls)
        per = "window" if n in (1, 2, 3) else "sequence"
        res = {"ms_per_step": 1e3 * best, "ms_per_step_mean": 1e3 * mean, "calls_per_step": len(calls),
               "pcie_bytes_per_step": moved, "max_abs_vs_device_line": diff,
               "note": f"zwg_attention_ex per {per}" + (" (self and cross)" if n == 3 else "") +
                       " on pageable host buffers (H2D q/k/v + kernels + D2H out), synchronous; best of "
                       f"{runs} runs; a one-{per} call plans its own key split, so it can round differently "
                       "from the batched device call"}
        if w.bound == "mfma":
            res.update({"value": self.work / best / 1e12, "unit": "TFLOP/s"})
        else:
            res.update({"value": self.work / best / 1e9, "unit": "GB/s",
                        "tokens_per_s": w.n_items / best, "note_value": "the step's algorithmic bytes (the "
                        "device line's) over the drop-in's wall time; PCIe moves pcie_bytes_per_step"})
        return res

    def free(self):
        self.sets = []
        self.host = None


class PromptWorkload(Workload):
    """Workload 4 (the Qwen2.5-0.5B 2048-token prefill) as llm.prompt feeds it
    (src/llm.zig:258-266): one step is 8 zwg_attention_dev calls of 256 query rows, call i over the
    cache's first 256 (i + 1) keys of the transposed cache (2048 columns), each writing its rows of
    the output.  Same visible pairs, so the same algorithmic work and results as the one-call
    prefill; eight launches (and merges) instead of one."""

    name = "qwen05_prefill_8x256"
    calls = 8

    def __init__(self, torch, ctx):
        super().__init__(4, torch, ctx, 1)
        from zwhisper_amd.ops import AttnShape

        w = self.spec
        rows = w.n_q // self.calls
        self.rows = rows
        self.shapes = [AttnShape(rows, rows * (i + 1), w.n_head, w.n_head_kv, w.d, w.n_head * w.d,
                                 w.n_head_kv * w.d, w.n_head * w.d, True, w.n_kv_cap) for i in range(self.calls)]
        s = self.sets[0]
        ns = w.n_head * w.d
        self.views = [(s["q"][0].view(w.n_q, ns)[rows * i: rows * (i + 1)], s["out"][0][rows * i: rows * (i + 1)])
                      for i in range(self.calls)]

    def step(self, i: int):
        self.last = i
        s = self.sets[0]
        for sh, (q, out) in zip(self.shapes, self.views):
            self.ctx.attention_dev(q, s["k"][0], s["v"][0], sh, out)


class AppendWorkload:
    """A cache update of one step (zwg_kv_append / _batch): the new K/V rows (and q) of a step
    written into the device-resident caches, with rotary positions for the Qwen2 shapes.

    Algorithmic bytes: the k, v (and q) rows read, the cache rows written, q written back, and
    the cos/sin table rows read.  The sources and caches (1-20 MB) stay in the 256 MB last-level
    cache between steps, as they would in a decode loop; at one token per sequence the update is
    bound by launch and memory latency, not bandwidth.
    """

    def __init__(self, name: str, torch, ctx):
        import zwhisper_amd as z
        from zwhisper_amd import workloads as W

        self.name = name
        self.torch = torch
        rng = np.random.default_rng(0x5A57)
        f32 = np.float32
        if name == "qwen15_kv_append_x64":
            w = W.WORKLOADS[5]
            self.description = "Qwen2.5-1.5B decode-step cache update: 64 sequences x 1 token, rotary q/k, K^T scatter"
            n, h, hkv, d, n_ctx = w.n_items, w.n_head, w.n_head_kv, w.d, w.n_kv_cap
            self.kv = z.KVCache(ctx, 1, n, n_ctx, hkv, d, z.KV_KT, rope_base=1.0e6)
            self.pos = (W.kv_lengths(5) - 1).astype(np.int32)
            self.batch = True
        elif name == "qwen05_prefill_kv_append":
            w = W.WORKLOADS[4]
            self.description = "Qwen2.5-0.5B prefill cache update: 2048 tokens, rotary q/k, K^T scatter"
            n, h, hkv, d, n_ctx = w.n_q, w.n_head, w.n_head_kv, w.d, w.n_kv_cap
            self.kv = z.KVCache(ctx, 1, 1, n_ctx, hkv, d, z.KV_KT, rope_base=1.0e6)
            self.pos = np.arange(n, dtype=np.int32)
            self.batch = False
        else:
            w = W.WORKLOADS[3]
            self.description = "Whisper small.en decoder-step cache update: 32 windows x 1 token, row-major"
            n, h, hkv, d, n_ctx = w.n_items, w.n_head, w.n_head_kv, w.d, w.n_kv_cap
            self.kv = z.KVCache(ctx, 1, n, n_ctx, hkv, d, z.KV_ROW)
            self.pos = (W.kv_lengths(3) - 1).astype(np.int32)
            self.batch = True
        self.n, self.h, self.hkv, self.d, self.n_ctx = n, h, hkv, d, n_ctx
        self.rope = name != "small_dec_kv_append_x32"
        kvw, ne = hkv * d, h * d
        self.host = {"k": rng.standard_normal((n, kvw)).astype(f32), "v": rng.standard_normal((n, kvw)).astype(f32),
                     "q": rng.standard_normal((n, ne)).astype(f32)}
        self.dev = {k: torch.from_numpy(a).cuda() for k, a in self.host.items()}
        self.pos_dev = torch.from_numpy(self.pos).cuda()
        rows = 2 * n * kvw * 4 * 2  # k, v read and written
        if self.rope:
            rows += 2 * n * ne * 4 + 2 * n * (d // 2) * 4  # q read + written, cos/sin rows
        self.work = float(rows)

    def step(self, i: int):
        d = self.dev
        q = d["q"] if self.rope else None
        if self.batch:
            self.kv.append_batch(0, 0, self.pos_dev, d["k"], d["v"], q, self.h, self.h * self.d)
        else:
            self.kv.append(0, 0, 0, d["k"], d["v"], q, self.h, self.h * self.d)

    def device_time(self, steps: int) -> float:
        """Mean device time of one update, in ms: `steps` updates captured back to back in a HIP
        graph and replayed, so host launch overhead (larger than these kernels in this Python
        harness) does not count.  The replay rotates q again each step; the timing does not
        depend on the values."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step(0)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                self.step(i)
        g.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        best = float("inf")
        for _ in range(3):
            ev[0].record(stream)
            g.replay()
            ev[1].record(stream)
            torch.cuda.synchronize()
            best = min(best, ev[0].elapsed_time(ev[1]) / steps)
        del g
        return best

    def cpu_baseline(self) -> dict:
        """oracle/kv.py's vectorised update (the reference's loops of src/llm.zig:182-190 and
        src/decoder.zig:182-183, in numpy) on this host."""
        from oracle import kv as okv

        kvw = self.hkv * self.d
        kt = np.zeros(kvw * self.n_ctx, np.float32)
        cv = np.zeros(self.n_ctx * kvw, np.float32)
        cos, sin = okv.rope_tables(self.n_ctx, self.d, 1.0e6) if self.rope else (None, None)

        def run():
            if self.rope:
                # one sequence's cache stands in for each of the batch's, as each token writes its own
                okv.llm_append_vec(self.host["q"].copy(), self.host["k"], self.host["v"], self.pos, self.h, self.hkv,
                                   self.d, kt, cv, self.n_ctx, cos, sin)
            else:  # row-major self caches: k and v rows at their positions (src/decoder.zig:182-183)
                kt.reshape(self.n_ctx, kvw)[self.pos] = self.host["k"]
                cv.reshape(self.n_ctx, kvw)[self.pos] = self.host["v"]

        best, mean, runs = time_cpu(run)
        return {"value": self.work / best / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": "the whole update; oracle/kv.py llm_append_vec (numpy, one thread); "
                          + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.kv.close()
        self.dev = None


class LinearWorkload:
    """The six linear layers of one Whisper base.en encoder layer over 16 windows x 1500 frames
    (src/encoder.zig:164-174): q, k, v and out projections (512 -> 512), MLP up (512 -> 2048) and
    down (2048 -> 512), f16 weights, f32 activations and bias, through zwg_linear_dev.

    Algorithmic work: 2 m n k flops per layer, m = 24000 rows.  The kernels run on f16 MFMA with
    each f32 activation split into two f16 terms, so their ceiling is half the f16 peak.
    """

    name = "base_enc_linear_x16"
    description = ("Whisper base.en encoder layer projections, 16 windows x 1500 frames: q/k/v/o 512->512, "
                   "MLP 512->2048->512, f16 weights")

    def __init__(self, torch, ctx, windows: int = 16):
        self.torch = torch
        self.ctx = ctx
        self.m = windows * 1500
        d, f = 512, 2048
        self.layers = [(d, d)] * 4 + [(d, f), (f, d)]  # (k, n)
        g = torch.Generator(device="cuda").manual_seed(0x11EA)
        self.x = {kk: torch.randn(self.m, kk, device="cuda", generator=g) for kk in (d, f)}
        self.out = {nn: torch.empty(self.m, nn, device="cuda") for nn in (d, f)}
        self.w = [(torch.randn(n, k, device="cuda", generator=g) / np.sqrt(k)).half() for k, n in self.layers]
        self.b = [torch.randn(n, device="cuda", generator=g) for _, n in self.layers]
        self.work = float(sum(2 * self.m * n * k for k, n in self.layers))

    def step(self, i: int):
        for (k, n), w, b in zip(self.layers, self.w, self.b):
            self.ctx.linear_dev(self.x[k], self.m, k, w, b, n, self.out[n])

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's ops.linear with f16 weights (oracle/attn_oracle.c, the reference's ntBlock
        over its Pool) on one of the 16 windows."""
        import oracle

        rows = 1500
        xs = {kk: v[:rows].cpu().numpy() for kk, v in self.x.items()}
        ws = [w.cpu().numpy() for w in self.w]
        bs = [b.cpu().numpy() for b in self.b]
        outs = {nn: np.zeros(rows * nn, np.float32) for nn in self.out}
        o = oracle.Oracle(threads)

        def run():
            for (k, n), w, b in zip(self.layers, ws, bs):
                o.linear_f16(xs[k], rows, k, w, b, n, out=outs[n])

        best, mean, runs = time_cpu(run, 3)
        o.close()
        work = self.work * rows / self.m
        return {"value": work / best / 1e12, "unit": "TFLOP/s", "cores": o.threads, "kind": "port",
                "sample": "1 of 16 windows (1500 rows), all six layers; oracle/attn_oracle.c ora_linear_f16; "
                          + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.x = self.out = self.w = self.b = None


class EncoderLayerWorkload:
    """One Whisper base.en encoder layer over 16 windows x 1500 frames on the device
    (zwg_encoder_layer_dev: the loop body of src/encoder.zig:164-175): two layer norms, the q/k/v/o
    and MLP projections with f16 weights (GELU and the residual adds fused into their stores) and
    the 16 windows' self-attention (8 heads x 64).

    Algorithmic work: the projections' 2 m n k (24 m n_state^2 over all six) plus attention's 4 d H per
    (q, k) pair.  Roofline: the time both would take at their own MFMA peaks (f16 MFMA for the
    projections at two MFMAs per f32 x f16 product, fp32 MFMA for attention); the layer norms and
    the attention's row-major K read add no flops.
    """

    name = "base_enc_layer_x16"
    description = ("Whisper base.en encoder layer, 16 windows x 1500 frames: layer norms, q/k/v/o and MLP "
                   "(f16 weights, GELU and residuals fused), self-attention 8x64")

    def __init__(self, torch, ctx, windows: int = 16):
        import zwhisper_amd as z

        self.torch, self.ctx, self.windows = torch, ctx, windows
        self.n_ctx, self.ns, self.n_head = 1500, 512, 8
        ns = self.ns
        g = torch.Generator(device="cuda").manual_seed(0xE1)

        def f16(n, k):
            return (torch.randn(n, k, device="cuda", generator=g) / np.sqrt(k)).half()

        def vec(n):
            return torch.randn(n, device="cuda", generator=g) * 0.1

        self.w = {"attn_ln_w": 1 + vec(ns), "attn_ln_b": vec(ns), "q_w": f16(ns, ns), "q_b": vec(ns),
                  "k_w": f16(ns, ns), "v_w": f16(ns, ns), "v_b": vec(ns), "o_w": f16(ns, ns), "o_b": vec(ns),
                  "mlp_ln_w": 1 + vec(ns), "mlp_ln_b": vec(ns), "mlp0_w": f16(4 * ns, ns), "mlp0_b": vec(4 * ns),
                  "mlp1_w": f16(ns, 4 * ns), "mlp1_b": vec(ns)}
        rows = windows * self.n_ctx
        self.x0 = torch.randn(windows, self.n_ctx, ns, device="cuda", generator=g)
        self.x = self.x0.clone()
        self.scratch = torch.empty(z.ops.encoder_layer_scratch(rows, ns), device="cuda")
        self.lin_flops = 24.0 * rows * ns * ns
        self.attn_flops = 4.0 * self.n_ctx * self.n_ctx * ns * windows
        self.work = self.lin_flops + self.attn_flops
        self.ideal_s = self.lin_flops * 2 / PEAK_MFMA_F16 + self.attn_flops * 3 / PEAK_MFMA_F16

    def step(self, i: int):
        # the layer updates x in place, so successive steps apply it to its own output, as the
        # encoder's stack of layers does; every linear reads normalised rows, so magnitudes stay put
        self.ctx.encoder_layer_dev(self.x, self.windows, self.n_ctx, self.ns, self.n_head, self.w, self.scratch)

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's encoder layer (ops.layerNorm, ops.linear over f16, ops.attention, ops.gelu,
        ops.add restated in oracle/attn_oracle.c) on one of the 16 windows."""
        import oracle

        w = {k: v.cpu().numpy() for k, v in self.w.items()}
        x = self.x0[0].cpu().numpy()
        o = oracle.Oracle(threads)
        best, mean, runs = time_cpu(lambda: o.encoder_layer(x, self.n_ctx, self.ns, self.n_head, w), 3)
        o.close()
        return {"value": self.work / self.windows / best / 1e12, "unit": "TFLOP/s", "cores": o.threads,
                "kind": "port", "sample": "1 of 16 windows; oracle Oracle.encoder_layer (attn_oracle.c); "
                                          + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.w = self.x = self.x0 = self.scratch = None


class Q8LinearWorkload:
    """A decode step's linear layers over int8 block weights (gemm.Q8, src/gemm.zig:188-351), m rows
    (sequences or windows decoded in lockstep) per layer, with the weights resident in HBM in the
    packed device layout (zwg_q8w_create, done once as the reference builds its Q8 at load).  The
    layers that read the same x -- q/k/v, and the MLP's gate and up -- run as one
    zwg_linear_q8w_group_dev call (`groups`: how many consecutive layers each call takes), the
    others by zwg_linear_q8w_dev.

    Algorithmic bytes per step: for every layer its int8 weights (n k), f32 block scales (n k / 32 * 4),
    bias (n * 4, when it has one), the x rows read (m k * 4) and the out rows written (m n * 4): the
    weights are read once per step, which is what makes these layers HBM-bound at m <= 64.  `copies`
    sets of weights rotate so that no step finds its weights in the 256 MB last-level cache.
    A step is one replay of a HIP graph that holds the step's launches (captured once per weight
    set), as a serving loop would run it: the step's many small launches are then not paced by this
    Python harness.
    """

    def __init__(self, name: str, description: str, torch, ctx, m: int, layers, copies: int = 1,
                 cpu_layers: int = 0, groups=None):
        import zwhisper_amd as z

        self.name, self.description = name, description
        self.torch, self.ctx, self.m = torch, ctx, m
        self.layers = layers  # (k, n, has_bias)
        self.groups = list(groups) if groups else [1] * len(layers)
        assert sum(self.groups) == len(layers)
        g = torch.Generator(device="cuda").manual_seed(0x0808)
        dims = sorted({k for k, _, _ in layers} | {n for _, n, _ in layers})
        self.x = {d: torch.randn(m, d, device="cuda", generator=g) for d in dims}
        # outputs by (n, place in its call): the members of a grouped call write distinct buffers
        self.out = {(d, j): torch.empty(m, d, device="cuda") for d in dims for j in range(max(self.groups))}
        self.sets = []
        self.raw = []  # unpacked copies of the first layers, for the CPU baseline
        for c in range(copies):
            ws = []
            for li, (k, n, hb) in enumerate(layers):
                q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
                sc = torch.rand(n, k // 32, device="cuda", generator=g) * (2.0 / 127 / np.sqrt(k))
                b = torch.randn(n, device="cuda", generator=g) if hb else None
                ws.append((z.Q8(q, sc, n, k).resident(ctx), b))
                if c == 0 and li < cpu_layers:
                    self.raw.append((q.cpu().numpy(), sc.cpu().numpy(), None if b is None else b.cpu().numpy()))
                del q, sc
            self.sets.append(ws)
        torch.cuda.synchronize()
        self.work = float(sum(n * k + n * k // 32 * 4 + (n * 4 if hb else 0) + m * k * 4 + m * n * 4
                              for k, n, hb in layers))
        # one graph per weight set, captured after an eager warm-up
        for ws in self.sets:
            self._run(ws)
        torch.cuda.synchronize()
        self.graphs = []
        for ws in self.sets:
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                self._run(ws)
            self.graphs.append(gr)
        torch.cuda.synchronize()

    def _run(self, ws):
        i = 0
        for gsize in self.groups:
            (k, n, _), (w, b) = self.layers[i], ws[i]
            if gsize == 1:
                self.ctx.linear_q8w_dev(self.x[k], self.m, w, b, self.out[(n, 0)])
            else:
                mem = range(i, i + gsize)
                self.ctx.linear_q8w_group_dev(self.x[k], self.m, [ws[j][0] for j in mem], [ws[j][1] for j in mem],
                                              [self.out[(self.layers[j][1], j - i)] for j in mem])
            i += gsize

    def step(self, i: int):
        self.graphs[i % len(self.graphs)].replay()

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's ops.linear over Q8 (oracle/attn_oracle.c: ntBlockQ over the reference's Pool),
        on the first layers."""
        import oracle

        sample = self.layers[:len(self.raw)]
        xs = {d: v.cpu().numpy() for d, v in self.x.items()}
        outs = {d: np.zeros(self.m * d, np.float32) for d, _ in self.out}
        o = oracle.Oracle(threads)

        def run():
            for (k, n, _), (q, sc, b) in zip(sample, self.raw):
                o.linear_q8(xs[k], self.m, k, q, sc, b, n, out=outs[n])

        best, mean, runs = time_cpu(run, 3)
        o.close()
        work = float(sum(n * k + n * k // 32 * 4 + (n * 4 if hb else 0) + self.m * k * 4 + self.m * n * 4
                         for k, n, hb in sample))
        return {"value": work / best / 1e9, "unit": "GB/s", "cores": o.threads, "kind": "port",
                "sample": f"{len(sample)} of {len(self.layers)} layers at the full {self.m} rows; "
                          "oracle/attn_oracle.c ora_linear_q8; " + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.graphs = None
        for ws in self.sets or []:
            for w, _ in ws:
                w.close()
        self.x = self.out = self.sets = self.raw = None


class QkvCacheWorkload:
    """A decode step's q/k/v projections and cache writes over all layers, int8 resident weights:
    per layer one zwg_linear_q8w_qkv_kv_dev (the projections with the cache append in their final
    store: q rotated and written out, k and v rotated and scattered into the device cache at each
    sequence's position), replayed as one HIP graph per step.  Beside it the record times the same
    step as the two calls it replaces, zwg_linear_q8w_group_dev into rows and zwg_kv_append_batch,
    per layer ("unfused"): one launch more per layer.  Algorithmic bytes per layer: the three weight
    sets (int8, f32 block scales, biases), x read, q written, and the k and v rows written into the
    cache."""

    def __init__(self, name: str, description: str, torch, ctx, m: int, k: int, n_layer: int, n_head: int,
                 n_head_kv: int, d: int, kt: bool, rope: float, n_ctx: int, biases):
        import zwhisper_amd as z
        from zwhisper_amd import _lib

        self.name, self.description = name, description
        self.torch, self.ctx, self.m, self.k, self.n_layer = torch, ctx, m, k, n_layer
        g = torch.Generator(device="cuda").manual_seed(0x0909)
        ns = (n_head * d, n_head_kv * d, n_head_kv * d)
        self.layers = []
        self.raw = None
        for li in range(n_layer):
            rs, bs = [], []
            for n, hb in zip(ns, biases):
                q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
                sc = torch.rand(n, k // 32, device="cuda", generator=g) * (2.0 / 127 / np.sqrt(k))
                rs.append(z.Q8(q, sc, n, k).resident(ctx))
                bs.append(torch.randn(n, device="cuda", generator=g) if hb else None)
                if li == 0:
                    self.raw = (self.raw or []) + [(q.cpu().numpy(), sc.cpu().numpy(),
                                                    None if bs[-1] is None else bs[-1].cpu().numpy())]
            self.layers.append((rs, bs))
        self.kv = z.KVCache(ctx, n_layer, m, n_ctx, n_head_kv, d, _lib.KV_KT if kt else _lib.KV_ROW, rope)
        self.x = torch.randn(m, k, device="cuda", generator=g)
        self.q = torch.empty(m, n_head * d, device="cuda")
        self.k_rows = torch.empty(m, n_head_kv * d, device="cuda")
        self.v_rows = torch.empty(m, n_head_kv * d, device="cuda")
        self.pos = torch.randint(0, n_ctx, (m,), dtype=torch.int32, device="cuda", generator=g)
        self.n_head, self.rope = n_head, rope
        self.work = float(n_layer * (sum(n * k + n * k // 32 * 4 + (n * 4 if hb else 0) for n, hb in zip(ns, biases))
                                     + m * k * 4 + m * ns[0] * 4 + 2 * m * ns[1] * 4))
        self.graphs = {}
        for mode in ("fused", "unfused"):
            self._run(mode)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                self._run(mode)
            self.graphs[mode] = gr
        torch.cuda.synchronize()

    def _run(self, mode: str):
        for li, (rs, bs) in enumerate(self.layers):
            if mode == "fused":
                self.ctx.linear_q8w_qkv_kv_dev(self.x, self.m, rs, bs, self.q, self.kv, li, 0, self.pos)
            else:
                self.ctx.linear_q8w_group_dev(self.x, self.m, rs, bs, [self.q, self.k_rows, self.v_rows])
                self.kv.append_batch(li, 0, self.pos, self.k_rows, self.v_rows,
                                     q=self.q if self.rope > 0 else None, n_head=self.n_head,
                                     q_stride=self.q.shape[1])

    def step(self, i: int):
        self.graphs["fused"].replay()

    def extra_record(self, steps: int) -> dict:
        """The unfused step (group call + append per layer), timed as the fused one."""
        torch = self.torch
        for _ in range(5):
            self.graphs["unfused"].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            self.graphs["unfused"].replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        return {"unfused": {"kernel_ms_per_step": ms, "launches_per_layer": 3,
                            "note": "zwg_linear_q8w_group_dev into rows + zwg_kv_append_batch per layer, the "
                                    "same HIP-graph replay; the fused call takes 2 launches per layer"}}

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's ops.linear over Q8 (oracle/attn_oracle.c) for one layer's q, k and v."""
        import oracle

        x = self.x.cpu().numpy()
        outs = [np.zeros(self.m * q.shape[0], np.float32) for q, _, _ in self.raw]
        o = oracle.Oracle(threads)

        def run():
            for (q, sc, b), out in zip(self.raw, outs):
                o.linear_q8(x, self.m, self.k, q, sc, b, q.shape[0], out=out)

        best, mean, runs = time_cpu(run, 3)
        o.close()
        return {"value": self.work / self.n_layer / best / 1e9, "unit": "GB/s", "cores": o.threads, "kind": "port",
                "sample": "layer 0's q, k and v projections (the cache rows' copy not included); "
                          "oracle/attn_oracle.c ora_linear_q8; " + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.graphs = None
        for rs, _ in self.layers or []:
            for w in rs:
                w.close()
        if self.kv is not None:
            self.kv.close()
        self.layers = self.kv = self.x = self.q = self.raw = None


class DecoderStepWorkload:
    """The Whisper text decoder's token step on the device (zwg_decoder_step_dev: Decoder.forward,
    src/decoder.zig:165-205, one new token in each of m windows decoded in lockstep): embeddings,
    every layer's self-attention over the window's cache (k and v rows written at its position),
    cross-attention over its n_audio_ctx cross K/V, MLP, then the final norm and the logits over
    the vocabulary.  Random int8 block weights of the model's shapes, resident; the cross caches
    filled once by zwg_decoder_set_audio_dev from a random encoder output (setAudio, timed once
    and reported beside); window w decodes at position n_kv_w - 1 with the small.en step's seeded
    self lengths (n_kv ~ U[1, 448]).  A step is one replay of a HIP graph of the call.

    Algorithmic bytes per step: every layer's int8 weights, block scales, biases and norms read
    once, the token embedding once (the logits' weights), each window's self K/V rows 0..pos and
    its cross K/V read once per layer and its new k and v rows written, the positional rows read
    and the logits written.  Beside it the record times the same step composed of the separate
    calls ("unfused": layer norms, q/k/v + cache, attention, int8 linears with their epilogues),
    which gives the same results bit for bit."""

    dtype = ("f32 (projections: f32 x int8 block weights on f16 MFMA, x split into two f16 terms; attention: "
             "f32 FMA decode kernels)")

    def __init__(self, name: str, description: str, torch, ctx, m: int = 32, n_layer: int = 12, ns: int = 768,
                 n_head: int = 12, n_vocab: int = 51864, n_tctx: int = 448, n_actx: int = 1500):
        import zwhisper_amd as z
        from zwhisper_amd.workloads import kv_lengths

        self.name, self.description = name, description
        self.torch, self.ctx, self.m, self.ns, self.H = torch, ctx, m, ns, n_head
        self.n_layer, self.n_vocab, self.n_tctx, self.n_actx = n_layer, n_vocab, n_tctx, n_actx
        g = torch.Generator(device="cuda").manual_seed(0x0A0A)

        def q8(n, k):
            q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
            sc = torch.rand(n, k // 32, device="cuda", generator=g) * (2.0 / 127 / np.sqrt(k))
            return z.Q8(q, sc, n, k)

        def vec(n, base=0.0):
            return base + 0.1 * torch.randn(n, device="cuda", generator=g)

        layers = []
        for _ in range(n_layer):
            w = {nm: q8(ns, ns) for nm in ("q_w", "k_w", "v_w", "o_w", "cq_w", "ck_w", "cv_w", "co_w")}
            w["mlp0_w"], w["mlp1_w"] = q8(4 * ns, ns), q8(ns, 4 * ns)
            for nm in ("q_b", "v_b", "o_b", "cq_b", "cv_b", "co_b", "mlp1_b"):
                w[nm] = vec(ns)
            w["mlp0_b"] = vec(4 * ns)
            for ln in ("attn_ln", "cross_ln", "mlp_ln"):
                w[ln + "_w"], w[ln + "_b"] = vec(ns, 1.0), vec(ns)
            layers.append(w)
        te = q8(n_vocab, ns)
        pe = 0.5 * torch.randn(n_tctx, ns, device="cuda", generator=g)
        self.dec = z.Decoder(ctx, te, pe, vec(ns, 1.0), vec(ns), layers, n_head, n_tctx, n_actx, m)
        self.host = None  # host copies for the CPU baseline: one window's weights and cross K/V
        self._host_src = (te, pe, layers)
        enc = torch.randn(m, n_actx, ns, device="cuda", generator=g)
        self.dec.set_audio(enc, m, 0)  # first call: kernels loaded
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        self.dec.set_audio(enc, m, 0)
        e1.record()
        torch.cuda.synchronize()
        self.set_audio_ms = e0.elapsed_time(e1)
        self.enc0 = enc[0].cpu().numpy()
        n_kv = kv_lengths(3)[:m].astype(np.int64)
        self.pos = torch.from_numpy((n_kv - 1).astype(np.int32)).cuda()
        self.tok = torch.randint(0, n_vocab, (m,), dtype=torch.int32, device="cuda", generator=g)
        self.logits = torch.empty(m, n_vocab, device="cuda")
        wb = sum(w.n * w.k * 1.125 for lw in layers for nm, w in lw.items() if nm not in ("ck_w", "cv_w")
                 and isinstance(w, z.Q8))
        vb = 4.0 * sum(t.numel() for lw in layers for nm, t in lw.items() if not isinstance(t, z.Q8)
                       and nm not in ("cv_b",))
        kvb = 4.0 * ns * n_layer * (2 * float(n_kv.sum()) + 2 * m * n_actx + 2 * m)
        self.work = float(wb + vb + te.n * te.k * 1.125 + kvb + 4.0 * m * ns * 2 + 4.0 * m * n_vocab)
        self.n_kv = n_kv
        # the unfused step: the separate calls over the same weights, its own caches (cross K/V by
        # the same projections of the same encoder output)
        self.self_kv = z.KVCache(ctx, n_layer, m, n_tctx, n_head, ns // n_head)
        self.cross_kv = z.KVCache(ctx, n_layer, m, n_actx, n_head, ns // n_head)
        for li, L in enumerate(self.dec.layer_refs):
            k, v = self.cross_kv.ptrs(li, 0)
            ctx.linear_q8w_dev(enc, m * n_actx, L["ck_w"], None, k)
            ctx.linear_q8w_dev(enc, m * n_actx, L["cv_w"], L["cv_b"], v)
        del enc
        self.X, self.A, self.Q, self.T = (torch.empty(m, ns, device="cuda") for _ in range(4))
        self.Hd = torch.empty(m, 4 * ns, device="cuda")
        # the embedding rows te.row(tok) + pe[pos], f32 products and sums as the fused kernel's
        tl = self.tok.long()
        self.E = te.q[tl].float() * te.scales[tl].repeat_interleave(32, dim=1) + pe[self.pos.long()]
        self.n_kv_t = (self.pos + 1).to(torch.int32)
        self.graphs = {}
        for mode in ("fused", "unfused"):
            self._run(mode)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                self._run(mode)
            self.graphs[mode] = gr
        torch.cuda.synchronize()

    def _run(self, mode: str):
        import zwhisper_amd as z
        from zwhisper_amd import _lib

        if mode == "fused":
            self.dec.step(self.tok, self.pos, self.logits, 0)
            return
        ctx, dec, m, ns, H = self.ctx, self.dec, self.m, self.ns, self.H
        X, A, Q, T, Hd = self.X, self.A, self.Q, self.T, self.Hd
        X.copy_(self.E)
        L0 = dec.layer_refs[0]
        ctx.layer_norm_dev(X, m, ns, L0["attn_ln_w"], L0["attn_ln_b"], 1e-5, A)
        sh_s = z.AttnShape(1, self.n_tctx, H, H, ns // H, ns, ns, ns, False)
        sh_c = z.AttnShape(1, self.n_actx, H, H, ns // H, ns, ns, ns, False)
        ps, pc = self.self_kv.info.seq_stride, self.cross_kv.info.seq_stride
        for li, L in enumerate(dec.layer_refs):
            ctx.linear_q8w_qkv_kv_dev(A, m, [L["q_w"], L["k_w"], L["v_w"]], [L["q_b"], None, L["v_b"]], Q,
                                      self.self_kv, li, 0, self.pos)
            k, v = self.self_kv.ptrs(li, 0)
            ctx.attention_batch_dev(Q, k, v, sh_s, T, m, ns, ps, ps, ns, self.n_kv_t)
            ctx.linear_q8w_epi_dev(T, m, L["o_w"], L["o_b"], X, _lib.EPI_ADD)
            ctx.layer_norm_dev(X, m, ns, L["cross_ln_w"], L["cross_ln_b"], 1e-5, A)
            ctx.linear_q8w_dev(A, m, L["cq_w"], L["cq_b"], Q)
            k, v = self.cross_kv.ptrs(li, 0)
            ctx.attention_batch_dev(Q, k, v, sh_c, T, m, ns, pc, pc, ns)
            ctx.linear_q8w_epi_dev(T, m, L["co_w"], L["co_b"], X, _lib.EPI_ADD)
            ctx.layer_norm_dev(X, m, ns, L["mlp_ln_w"], L["mlp_ln_b"], 1e-5, A)
            ctx.linear_q8w_epi_dev(A, m, L["mlp0_w"], L["mlp0_b"], Hd, _lib.EPI_GELU)
            ctx.linear_q8w_epi_dev(Hd, m, L["mlp1_w"], L["mlp1_b"], X, _lib.EPI_ADD)
            last = li + 1 == self.n_layer
            ctx.layer_norm_dev(X, m, ns, dec.ln_w if last else dec.layer_refs[li + 1]["attn_ln_w"],
                               dec.ln_b if last else dec.layer_refs[li + 1]["attn_ln_b"], 1e-5, A)
        ctx.linear_q8w_dev(A, m, dec.te, None, self.logits_u)

    @property
    def logits_u(self):
        if not hasattr(self, "_lu"):
            self._lu = self.torch.empty_like(self.logits)
        return self._lu

    def step(self, i: int):
        self.graphs["fused"].replay()

    def extra_record(self, steps: int) -> dict:
        """The unfused step timed as the fused one, the bit-for-bit check of the two, tokens/s and
        the setAudio time."""
        torch = self.torch
        for _ in range(5):
            self.graphs["unfused"].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            self.graphs["unfused"].replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        self.graphs["fused"].replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(self.logits, self.logits_u))
        return {"unfused": {"kernel_ms_per_step": ms, "logits_equal_bitwise": same,
                            "note": "the same step as separate calls (layer norms, q/k/v + cache, attention, "
                                    "int8 linears with add / GELU epilogues), one HIP-graph replay per step"},
                "tokens_per_step": self.m,
                "set_audio_ms": self.set_audio_ms,
                "set_audio_note": f"cross K/V of {self.m} windows x {self.n_layer} layers from the encoder output "
                                  f"({self.m} x {self.n_actx} rows x 2 projections per layer), one call"}

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's Decoder.forward (Oracle.decoder_forward: ops.linear over Q8, layerNorm, gelu,
        attention, the reference's steps) for one window's token, all layers and the logits."""
        import oracle

        te, pe, layers = self._host_src
        w0 = 0
        hl = [{nm: ((t.q.cpu().numpy(), t.scales.cpu().numpy()) if hasattr(t, "scales") else t.cpu().numpy())
               for nm, t in lw.items()} for lw in layers]
        dec = {"te": (te.q.cpu().numpy(), te.scales.cpu().numpy()), "pe": pe.cpu().numpy(),
               "ln_w": self.dec.ln_w.cpu().numpy(), "ln_b": self.dec.ln_b.cpu().numpy(), "n_head": self.H,
               "layers": hl}
        o = oracle.Oracle(threads)
        cross = o.decoder_set_audio(self.enc0, self.n_actx, self.ns, hl)
        cache = {"k": np.zeros((self.n_layer, self.n_tctx, self.ns), np.float32),
                 "v": np.zeros((self.n_layer, self.n_tctx, self.ns), np.float32),
                 "ck": np.stack([c[0] for c in cross]), "cv": np.stack([c[1] for c in cross])}
        pos = int(self.n_kv[w0]) - 1
        tok = int(self.tok[w0].item())

        def run():
            o.decoder_forward(dec, cache, tok, pos)

        best, mean, runs = time_cpu(run, 3)
        o.close()
        # one window's token: all the weights, and that window's own cache rows
        kv_all = 4.0 * self.ns * self.n_layer * (2 * float(self.n_kv.sum()) + 2 * self.m * self.n_actx + 2 * self.m)
        kv_one = 4.0 * self.ns * self.n_layer * (2 * (pos + 1) + 2 * self.n_actx + 2)
        work1 = self.work - kv_all - 4.0 * self.m * (2 * self.ns + self.n_vocab) + kv_one + 4.0 * (2 * self.ns + self.n_vocab)
        return {"value": 1.0 / best, "unit": "tokens/s", "cores": o.threads, "kind": "port",
                "bytes_per_token": work1, "gb_per_s": work1 / best / 1e9,
                "sample": f"one window's token (position {pos}) through all {self.n_layer} layers and the logits, "
                          "as the reference decodes a window; oracle Decoder.forward over oracle/attn_oracle.c; "
                          + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.graphs = None
        self.dec.close()
        self.self_kv.close()
        self.cross_kv.close()
        self.dec = self.self_kv = self.cross_kv = self._host_src = None


class LlmStepWorkload:
    """Qwen2's decode step on the device (zwg_llm_step_dev: Model.forward, src/llm.zig:169-216, one
    new token in each of m sequences decoded in lockstep): the embedding rows, every layer's RMS
    norm, q/k/v projections with rotary positions and the cache writes (keys transposed), GQA
    attention over each sequence's cached keys, the output projection, the SwiGLU MLP, then the
    output norm and the logits over the vocabulary (tied to the embedding, as Qwen2.5-1.5B's).
    Random int8 block weights of the model's shapes, resident; sequence s decodes at position
    n_kv_s - 1 with the Qwen2.5-1.5B decode lengths (n_kv ~ U[1024, 4096]).  A step is one replay of
    a HIP graph of the call.

    Algorithmic bytes per step: every layer's int8 weights, block scales, biases and norms read
    once, the output weights once, each sequence's embedding row, its K/V rows 0..pos read once
    per layer and its new k and v rows written, and the logits written.  Beside it the record times
    the same step composed of the separate calls ("unfused": RMS norms, q/k/v + cache, attention,
    int8 linears with the add epilogue, the grouped gate/up call, SiLU-mul), which gives the same
    results bit for bit."""

    dtype = ("f32 (projections: f32 x int8 block weights on f16 MFMA, x split into two f16 terms; attention: "
             "f32 FMA decode kernels over the transposed keys)")

    def __init__(self, name: str, description: str, torch, ctx, m: int = 64, n_layer: int = 28, ne: int = 1536,
                 n_head: int = 12, n_head_kv: int = 2, n_ff: int = 8960, n_vocab: int = 151936, n_ctx: int = 4096,
                 rope_base: float = 1e6, eps: float = 1e-6):
        import zwhisper_amd as z
        from zwhisper_amd import _lib
        from zwhisper_amd.workloads import kv_lengths

        self.name, self.description = name, description
        self.torch, self.ctx, self.m, self.ne, self.H, self.Hk = torch, ctx, m, ne, n_head, n_head_kv
        self.n_layer, self.n_ff, self.n_vocab, self.n_ctx, self.eps = n_layer, n_ff, n_vocab, n_ctx, eps
        d = ne // n_head
        kvw = n_head_kv * d
        g = torch.Generator(device="cuda").manual_seed(0x0B0B)

        def q8(n, k):
            q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
            sc = torch.rand(n, k // 32, device="cuda", generator=g) * (2.0 / 127 / np.sqrt(k))
            return z.Q8(q, sc, n, k)

        def vec(n, base=0.0, scale=0.1):
            return base + scale * torch.randn(n, device="cuda", generator=g)

        layers = []
        for _ in range(n_layer):
            layers.append({"wq": q8(ne, ne), "wk": q8(kvw, ne), "wv": q8(kvw, ne), "wo": q8(ne, ne),
                           "w_gate": q8(n_ff, ne), "w_up": q8(n_ff, ne), "w_down": q8(ne, n_ff),
                           "bq": vec(ne, scale=0.3), "bk": vec(kvw, scale=0.3), "bv": vec(kvw),
                           "attn_norm": vec(ne, 1.0), "ffn_norm": vec(ne, 1.0)})
        embd = q8(n_vocab, ne)
        output_norm = vec(ne, 1.0)
        self.lm = z.LLM(ctx, embd, None, output_norm, layers, n_head, n_head_kv, n_ff, n_ctx, m, rope_base, eps)
        self._host_src = (embd, output_norm, layers)
        n_kv = kv_lengths(5)[:m].astype(np.int64)
        self.n_kv = n_kv
        self.pos = torch.from_numpy((n_kv - 1).astype(np.int32)).cuda()
        self.tok = torch.randint(0, n_vocab, (m,), dtype=torch.int32, device="cuda", generator=g)
        self.logits = torch.empty(m, n_vocab, device="cuda")
        self._lu = torch.empty_like(self.logits)
        wb = sum(w.n * w.k * 1.125 for lw in layers for w in lw.values() if isinstance(w, z.Q8))
        vb = 4.0 * sum(t.numel() for lw in layers for t in lw.values() if not isinstance(t, z.Q8))
        kvb = 4.0 * kvw * n_layer * (2 * float(n_kv.sum()) + 2 * m)
        self.work = float(wb + vb + embd.n * embd.k * 1.125 + 4.0 * ne + m * ne * 1.125 + kvb + 4.0 * m * n_vocab)
        # the unfused step: the separate calls over the same weights, its own cache
        self.kv = z.KVCache(ctx, n_layer, m, n_ctx, n_head_kv, d, _lib.KV_KT, rope_base)
        self.X, self.Hn, self.Q, self.T = (torch.empty(m, ne, device="cuda") for _ in range(4))
        self.G, self.U = torch.empty(m, n_ff, device="cuda"), torch.empty(m, n_ff, device="cuda")
        # the embedding rows embd.row(tok): f32 products as the fused kernel's
        tl = self.tok.long()
        self.E = embd.q[tl].float() * embd.scales[tl].repeat_interleave(32, dim=1)
        self.n_kv_t = (self.pos + 1).to(torch.int32)
        self.graphs = {}
        for mode in ("fused", "unfused"):
            self._run(mode)
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                self._run(mode)
            self.graphs[mode] = gr
        torch.cuda.synchronize()

    def _run(self, mode: str):
        import zwhisper_amd as z
        from zwhisper_amd import _lib

        if mode == "fused":
            self.lm.step(self.tok, self.pos, self.logits, 0)
            return
        ctx, lm, m, ne, nff = self.ctx, self.lm, self.m, self.ne, self.n_ff
        X, Hn, Q, T, G, U = self.X, self.Hn, self.Q, self.T, self.G, self.U
        X.copy_(self.E)
        ctx.rms_norm_dev(X, m, ne, lm.layer_refs[0]["attn_norm"], self.eps, Hn)
        d = ne // self.H
        sh = z.AttnShape(1, self.n_ctx, self.H, self.Hk, d, ne, self.Hk * d, ne, False, self.n_ctx)
        ps = self.kv.info.seq_stride
        for li, L in enumerate(lm.layer_refs):
            ctx.linear_q8w_qkv_kv_dev(Hn, m, [L["wq"], L["wk"], L["wv"]], [L["bq"], L["bk"], L["bv"]], Q, self.kv, li,
                                      0, self.pos)
            k, v = self.kv.ptrs(li, 0)
            ctx.attention_batch_dev(Q, k, v, sh, T, m, ne, ps, ps, ne, self.n_kv_t)
            ctx.linear_q8w_epi_dev(T, m, L["wo"], None, X, _lib.EPI_ADD)
            ctx.rms_norm_dev(X, m, ne, L["ffn_norm"], self.eps, Hn)
            ctx.linear_q8w_group_dev(Hn, m, [L["w_gate"], L["w_up"]], None, [G, U])
            ctx.silu_mul_dev(G, U)
            ctx.linear_q8w_epi_dev(G, m, L["w_down"], None, X, _lib.EPI_ADD)
            last = li + 1 == self.n_layer
            ctx.rms_norm_dev(X, m, ne, lm.output_norm if last else lm.layer_refs[li + 1]["attn_norm"], self.eps, Hn)
        ctx.linear_q8w_dev(Hn, m, lm.output, None, self._lu)

    def step(self, i: int):
        self.graphs["fused"].replay()

    def extra_record(self, steps: int) -> dict:
        """The unfused step timed as the fused one, the bit-for-bit check of the two and tokens/s."""
        torch = self.torch
        for _ in range(5):
            self.graphs["unfused"].replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            self.graphs["unfused"].replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        self.graphs["fused"].replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(self.logits, self._lu))
        return {"unfused": {"kernel_ms_per_step": ms, "logits_equal_bitwise": same,
                            "note": "the same step as separate calls (RMS norms, q/k/v + cache, attention, int8 "
                                    "linears with the add epilogue, grouped gate/up, SiLU-mul), one HIP-graph "
                                    "replay per step"},
                "tokens_per_step": self.m}

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's Model.forward (Oracle.llm_forward: ops.linear over Q8, rmsNorm, the rotary
        cache writes, attentionEx over the transposed cache, siluMul, the reference's steps) for
        one sequence's token, all layers and the logits."""
        import oracle
        from oracle import kv as kvo

        embd, output_norm, layers = self._host_src
        d = self.ne // self.H
        hl = [{nm: ((t.q.cpu().numpy(), t.scales.cpu().numpy()) if hasattr(t, "scales") else t.cpu().numpy())
               for nm, t in lw.items()} for lw in layers]
        e = (embd.q.cpu().numpy(), embd.scales.cpu().numpy())
        cos, sin = kvo.rope_tables(self.n_ctx, d, 1e6)
        lm = {"embd": e, "output": e, "output_norm": output_norm.cpu().numpy(), "n_head": self.H,
              "n_head_kv": self.Hk, "eps": self.eps, "cos": cos, "sin": sin, "layers": hl}
        cache = {"kt": np.zeros((self.n_layer, self.Hk * d * self.n_ctx), np.float32),
                 "v": np.zeros((self.n_layer, self.n_ctx, self.Hk * d), np.float32)}
        s0 = 0
        pos = int(self.n_kv[s0]) - 1
        tok = int(self.tok[s0].item())
        o = oracle.Oracle(threads)

        def run():
            o.llm_forward(lm, cache, tok, pos)

        best, mean, runs = time_cpu(run, 3)
        o.close()
        kvw = self.Hk * d
        kv_all = 4.0 * kvw * self.n_layer * (2 * float(self.n_kv.sum()) + 2 * self.m)
        kv_one = 4.0 * kvw * self.n_layer * (2 * (pos + 1) + 2)
        per_seq = self.ne * 1.125 + 4.0 * self.n_vocab
        work1 = self.work - kv_all - self.m * per_seq + kv_one + per_seq
        return {"value": 1.0 / best, "unit": "tokens/s", "cores": o.threads, "kind": "port",
                "bytes_per_token": work1, "gb_per_s": work1 / best / 1e9,
                "sample": f"one sequence's token (position {pos}) through all {self.n_layer} layers and the logits, "
                          "as the reference decodes a sequence; oracle Model.forward over oracle/attn_oracle.c; "
                          + cpu_timing(best, mean, runs), "seconds": best}

    def free(self):
        self.graphs = None
        self.lm.close()
        self.kv.close()
        self.lm = self.kv = self._host_src = None


class LlmPromptWorkload:
    """Qwen2's prompt on the device as llm.prompt feeds it (src/llm.zig:258-266): one step is a
    2048-token prompt of one sequence in 8 zwg_llm_forward_dev calls of 256 tokens (Model.forward,
    src/llm.zig:169-216, over a batch: RMS norms, the q/k/v projections, the rotary cache append,
    causal attention over the cache so far, o, the SwiGLU MLP, and the last token's logits), replayed
    as one HIP graph.  Qwen2.5-0.5B shapes (24 layers, 896 wide, 14q/2kv heads of 64, n_ff 4864,
    151936-token tied vocabulary), random int8 block weights, resident.

    Algorithmic work per step: 2 flops per weight per token for every projection, 4 d H per
    visible (query, key) pair for the attention (src/bench.zig:76), 2 flops per weight for the 8
    calls' logits.  Its roofline is composite, as the encoder layer's: the projections at half
    the 16-bit MFMA peak (two f16 products per f32 x int8 product), the attention at a third (x3)."""

    dtype = ("f32 (projections: f32 x int8 block weights on f16 MFMA, x split into two f16 terms; attention: x3 "
             "16-bit MFMA)")

    def __init__(self, name: str, description: str, torch, ctx, n_tok: int = 2048, calls: int = 8, n_layer: int = 24,
                 ne: int = 896, n_head: int = 14, n_head_kv: int = 2, n_ff: int = 4864, n_vocab: int = 151936,
                 n_ctx: int = 2048):
        import zwhisper_amd as z

        self.name, self.description = name, description
        self.torch, self.ctx = torch, ctx
        self.n_tok, self.calls, self.rows = n_tok, calls, n_tok // calls
        self.ne, self.H, self.Hk, self.n_ff, self.n_layer, self.n_vocab, self.n_ctx = (ne, n_head, n_head_kv, n_ff,
                                                                                         n_layer, n_vocab, n_ctx)
        d = ne // n_head
        kvw = n_head_kv * d
        g = torch.Generator(device="cuda").manual_seed(0x0C0C)

        def q8(n, k):
            q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g)
            sc = torch.rand(n, k // 32, device="cuda", generator=g) * (2.0 / 127 / np.sqrt(k))
            return z.Q8(q, sc, n, k)

        def vec(n, base=0.0, scale=0.1):
            return base + scale * torch.randn(n, device="cuda", generator=g)

        layers = []
        for _ in range(n_layer):
            layers.append({"wq": q8(ne, ne), "wk": q8(kvw, ne), "wv": q8(kvw, ne), "wo": q8(ne, ne),
                           "w_gate": q8(n_ff, ne), "w_up": q8(n_ff, ne), "w_down": q8(ne, n_ff),
                           "bq": vec(ne, scale=0.3), "bk": vec(kvw, scale=0.3), "bv": vec(kvw),
                           "attn_norm": vec(ne, 1.0), "ffn_norm": vec(ne, 1.0)})
        embd = q8(n_vocab, ne)
        output_norm = vec(ne, 1.0)
        self.lm = z.LLM(ctx, embd, None, output_norm, layers, n_head, n_head_kv, n_ff, n_ctx, 1)
        self._host_src = (embd, output_norm, layers)
        self.tok = torch.randint(0, n_vocab, (n_tok,), dtype=torch.int32, device="cuda", generator=g)
        self.logits = torch.empty(n_vocab, device="cuda")
        per_tok = 2.0 * sum(w.n * w.k for w in layers[0].values() if isinstance(w, z.Q8)) * n_layer
        self.linear_flops = per_tok * n_tok + calls * 2.0 * n_vocab * ne
        pairs = n_tok * (n_tok + 1) / 2
        self.attn_flops = 4.0 * d * n_head * pairs * n_layer
        self.work = self.linear_flops + self.attn_flops
        self.ideal_s = self.linear_flops / (PEAK_MFMA_F16 / 2) + self.attn_flops / (PEAK_MFMA_F16 / 3)
        self._run()
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._run()
        torch.cuda.synchronize()

    def _run(self):
        for c in range(self.calls):
            self.lm.forward(self.tok[c * self.rows:(c + 1) * self.rows], c * self.rows, self.logits, 0)

    def step(self, i: int):
        self.graph.replay()

    def extra_record(self, steps: int) -> dict:
        """The step's calls eagerly (no graph), the graph's logits against them, tokens/s."""
        torch = self.torch
        self.graph.replay()
        torch.cuda.synchronize()
        ref = self.logits.clone()
        t0 = time.perf_counter()
        for _ in range(3):
            self._run()
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) / 3 * 1e3
        return {"eager": {"ms_per_step": eager_ms, "logits_equal_bitwise": bool(torch.equal(ref, self.logits)),
                          "note": "the 8 calls launched from the host per step, no graph"},
                "tokens_per_step": self.n_tok, "calls_per_step": self.calls,
                "linear_flops": self.linear_flops, "attention_flops": self.attn_flops}

    def cpu_baseline(self, threads: int) -> dict:
        """The oracle's Model.forward (Oracle.llm_forward over a batch: ops.linear over Q8,
        rmsNorm, the rotary cache writes, attentionEx causal over the transposed cache, siluMul)
        for the prompt's first call of 256 tokens."""
        import oracle
        from oracle import kv as kvo

        embd, output_norm, layers = self._host_src
        d = self.ne // self.H
        hl = [{nm: ((t.q.cpu().numpy(), t.scales.cpu().numpy()) if hasattr(t, "scales") else t.cpu().numpy())
               for nm, t in lw.items()} for lw in layers]
        e = (embd.q.cpu().numpy(), embd.scales.cpu().numpy())
        cos, sin = kvo.rope_tables(self.n_ctx, d, 1e6)
        lm = {"embd": e, "output": e, "output_norm": output_norm.cpu().numpy(), "n_head": self.H,
              "n_head_kv": self.Hk, "eps": 1e-6, "cos": cos, "sin": sin, "layers": hl}
        cache = {"kt": np.zeros((self.n_layer, self.Hk * d * self.n_ctx), np.float32),
                 "v": np.zeros((self.n_layer, self.n_ctx, self.Hk * d), np.float32)}
        toks = self.tok[:self.rows].cpu().numpy()
        o = oracle.Oracle(threads)

        def run():
            o.llm_forward(lm, cache, toks, 0)

        best, mean, runs = time_cpu(run, 2)
        o.close()
        per_tok = self.linear_flops / self.n_tok
        work1 = per_tok * self.rows + 4.0 * d * self.H * self.rows * (self.rows + 1) / 2 * self.n_layer
        return {"value": self.rows / best, "unit": "tokens/s", "cores": o.threads, "kind": "port",
                "tflops": work1 / best / 1e12,
                "sample": f"the prompt's first call: {self.rows} tokens through all {self.n_layer} layers and the last "
                          "token's logits, oracle Model.forward over oracle/attn_oracle.c; " + cpu_timing(best, mean, runs),
                "seconds": best}

    def free(self):
        self.graph = None
        self.lm.close()
        self.lm = self._host_src = None


def q8_workloads(torch, ctx):
    """(name, constructor) of the int8 decode-step measurements."""
    qwen_layer = [(1536, 1536, True), (1536, 256, True), (1536, 256, True), (1536, 1536, False),
                  (1536, 8960, False), (1536, 8960, False), (8960, 1536, False)]  # src/llm.zig:179-207
    whisper_layer = [(768, 768, True), (768, 768, False), (768, 768, True), (768, 768, True),
                     (768, 768, True), (768, 768, True), (768, 3072, True), (3072, 768, True)]  # src/decoder.zig:181-201
    yield "qwen15_logits_q8_x64", lambda: Q8LinearWorkload(
        "qwen15_logits_q8_x64", "Qwen2.5-1.5B output projection over the 151936-token vocabulary, 64 sequences "
        "(src/llm.zig:214-216), int8 block weights", torch, ctx, 64, [(1536, 151936, False)], copies=2, cpu_layers=1)
    yield "qwen15_decode_q8_linear_x64", lambda: Q8LinearWorkload(
        "qwen15_decode_q8_linear_x64", "Qwen2.5-1.5B decode step, 64 sequences: q/k/v/o, gate/up/down of all "
        "28 layers (196 linear layers in 112 calls: q/k/v and gate/up grouped), int8 block weights", torch, ctx, 64,
        qwen_layer * 28, cpu_layers=7, groups=[3, 1, 2, 1] * 28)
    yield "small_dec_q8_linear_x32", lambda: Q8LinearWorkload(
        "small_dec_q8_linear_x32", "Whisper small.en decoder step, 32 windows: q/k/v/o, cross q/o, MLP of all "
        "12 layers and the 51864-token logits (97 linear layers in 73 calls: q/k/v grouped), int8 block weights",
        torch, ctx, 32, whisper_layer * 12 + [(768, 51864, False)], copies=2, cpu_layers=8,
        groups=[3, 1, 1, 1, 1, 1] * 12 + [1])
    yield "small_dec_qkv_cache_x32", lambda: QkvCacheWorkload(
        "small_dec_qkv_cache_x32", "Whisper small.en decoder step, 32 windows: self-attention q/k/v projections "
        "of all 12 layers with the new k and v rows written into the row-major device caches "
        "(src/decoder.zig:181-183), int8 block weights", torch, ctx, 32, 768, 12, 12, 12, 64, False, 0.0, 448,
        (True, False, True))
    yield "small_dec_step_x32", lambda: DecoderStepWorkload(
        "small_dec_step_x32", "Whisper small.en decoder token step, 32 windows in lockstep (src/decoder.zig:165-205): "
        "embeddings, 12 layers of self-attention over each window's cache (n_kv ~ U[1, 448]), cross-attention over "
        "1500 audio frames and MLP, int8 block weights, then the 51864-token logits", torch, ctx)
    yield "qwen15_qkv_cache_x64", lambda: QkvCacheWorkload(
        "qwen15_qkv_cache_x64", "Qwen2.5-1.5B decode step, 64 sequences: q/k/v projections of all 28 layers, "
        "q and k rotated (base 1e6), k scattered into the transposed device cache and v into its rows "
        "(src/llm.zig:179-190), int8 block weights", torch, ctx, 64, 1536, 28, 12, 2, 128, True, 1e6, 4096,
        (True, True, True))
    yield "qwen15_step_x64", lambda: LlmStepWorkload(
        "qwen15_step_x64", "Qwen2.5-1.5B decode token step, 64 sequences in lockstep (src/llm.zig:169-216): "
        "embeddings, 28 layers of RMS norm, q/k/v with rotary positions into the transposed cache, GQA attention "
        "(12q/2kv x 128) over each sequence's cache (n_kv ~ U[1024, 4096]) and the SwiGLU MLP, int8 block weights, "
        "then the 151936-token logits (tied output)", torch, ctx)


def time_workload(wl, steps: int, warmup: int) -> dict:
    """The card raises its clocks over the first tens of milliseconds of continuous load, so steps
    timed right after a few warm-up steps measure part of that ramp.  Order: W warm-up steps; K
    "cold" steps timed with one event pair (reported as `cold`, never as the value); untimed steps
    for SETTLE_S; then exactly K timed steps bracketed by torch.cuda.synchronize(), with one pair
    of HIP events on the stream the kernels run on around them: the wall time gives ms_per_step
    (and `value`), the events kernel_ms_mean, the device time per step with nothing inserted
    between the steps.  Afterwards (outside the timed region) K more steps each bracketed by their
    own events give the per-step median and minimum; an event pair between launches adds a short
    gap, so those run a little above the mean."""
    torch = wl.torch
    stream = torch.cuda.current_stream()
    i = 0
    for _ in range(warmup):
        wl.step(i)
        i += 1
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(steps):
        wl.step(i)
        i += 1
    c1.record(stream)
    torch.cuda.synchronize()
    cold_ms = c0.elapsed_time(c1) / steps
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(16):
            wl.step(i)
            i += 1
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        wl.step(i)
        i += 1
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms_mean = e0.elapsed_time(e1) / steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for k in range(steps):
        ev[k][0].record(stream)
        wl.step(i)
        i += 1
        ev[k][1].record(stream)
    torch.cuda.synchronize()
    kms = [a.elapsed_time(b) for a, b in ev]
    return {"wall_s": wall, "ms_per_step": 1e3 * wall / steps, "kernel_ms_mean": kernel_ms_mean,
            "kernel_ms_min": float(np.min(kms)), "kernel_ms_median": float(np.median(kms)),
            "cold_kernel_ms": cold_ms, "settle_s": settle_s}


SETTLE_S = 0.3  # untimed continuous load between the cold steps and the timed steps
TRAFFIC_SOURCE: dict = {}  # traffic_source(), set once in main()


def cold(r: dict, work: float, unit: str, peak: float, products: int = 1) -> dict:
    """The cold-start record of a workload (reported beside `value`, never as it): device time per
    step of the K steps timed right after the W warm-up steps, before the clocks settle."""
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    achieved = work / (r["cold_kernel_ms"] * 1e-3)
    out = {"kernel_ms_per_step": r["cold_kernel_ms"], "achieved": achieved / scale, "unit": unit,
           "frac": achieved / peak,
           "note": "device time per step of K steps right after the W warm-up steps, while the clocks ramp"}
    if products > 1:
        out["issued_frac"] = products * achieved / peak
    return out


def cpu_baseline(number: int, threads: int, decode_pool: bool = True, one_call: bool = False) -> dict:
    """The oracle (C restatement of ops.attentionEx + Pool) on a bounded sample of the workload.

    Decode workloads run on min(threads, 4) threads, the reference's decode pool (pool_dec,
    src/transcribe.zig:106, src/llm.zig:151), unless decode_pool is False (all threads: the
    stronger baseline).  The prefill runs as llm.prompt feeds it, 8 calls of 256 rows, unless
    one_call is True: then as one 2048-row call, for comparison."""
    import oracle
    from zwhisper_amd import workloads as W
    from zwhisper_amd.ops import AttnShape

    w = W.WORKLOADS[number]
    if number in (3, 5) and decode_pool:
        threads = min(threads, 4)
    o = oracle.Oracle(threads)
    calls = []  # (q, k, v, shape) of the sample
    if number in (1, 2):
        n_items = w.n_items
        for item in range(n_items):
            q, kl, v = W.make_dense(number, item)
            # encoder.zig:167 passes row-major K; attentionEx transposes it itself
            k = kl.reshape(w.n_kv_cap, -1)
            ns = w.n_head * w.d
            calls.append((q, k, v, AttnShape(w.n_q, w.n_kv_cap, w.n_head, w.n_head, w.d, ns, ns, ns, False, None)))
        sample = f"{n_items} of {w.n_items} window(s)"
        work = W.algorithmic_work(number) * n_items / w.n_items
    elif number == 4:
        q, kl, v = W.make_dense(4, 0)
        kt = W.to_kt(kl, w.n_kv_cap)
        ns, kvw = w.n_head * w.d, w.n_head_kv * w.d
        # llm.prompt feeds batches of 256 rows with kt_stride = n_ctx (src/llm.zig:258-266, :191-202)
        rows = w.n_q if one_call else 256
        for b0 in range(0, w.n_q, rows):
            calls.append((q[b0:b0 + rows], kt, v[: b0 + rows],
                          AttnShape(rows, b0 + rows, w.n_head, w.n_head_kv, w.d, ns, kvw, ns, True, w.n_kv_cap)))
        sample = "the whole prefill as one 2048-row call" if one_call else "the whole prefill as 8 calls of 256 rows"
        work = W.algorithmic_work(4)
    elif number == 3:
        ns = w.n_head * w.d
        n_items = w.n_items
        lengths = W.kv_lengths(3)
        for item in range(n_items):
            s = W.make_decoder_step(item)
            calls.append((s["q_self"], s["k_self"], s["v_self"],
                          AttnShape(1, s["n_self"], w.n_head, w.n_head, w.d, ns, ns, ns, True, None)))
            calls.append((s["q_cross"], s["k_cross"], s["v_cross"],
                          AttnShape(1, 1500, w.n_head, w.n_head, w.d, ns, ns, ns, False, None)))
        sample = f"{n_items} of {w.n_items} windows (self + cross each)"
        work = float(sum(2 * int(n) * ns * 4 + 2 * 1500 * ns * 4 + 4 * ns * 4 for n in lengths[:n_items]))
    else:
        ns, kvw = w.n_head * w.d, w.n_head_kv * w.d
        n_items = w.n_items
        lengths = W.kv_lengths(5)
        for item in range(n_items):
            q, kl, v, n_kv = W.make_llm_decode(item)
            kt = W.to_kt(kl, w.n_kv_cap)
            calls.append((q, kt, v, AttnShape(1, n_kv, w.n_head, w.n_head_kv, w.d, ns, kvw, ns, True, w.n_kv_cap)))
        sample = f"{n_items} of {w.n_items} sequences"
        work = float(sum(2 * int(n) * kvw * 4 + 2 * ns * 4 for n in lengths[:n_items]))
    prepared = []
    for q, k, v, sh in calls:
        out = np.zeros(sh.out_len(), dtype=np.float32)
        scratch = np.empty(oracle.scratch_floats(sh), dtype=np.float32)
        prepared.append((np.ascontiguousarray(q).reshape(-1), np.ascontiguousarray(k).reshape(-1),
                         np.ascontiguousarray(v).reshape(-1), sh, out, scratch))

    def run_all():
        for q, k, v, sh, out, scratch in prepared:
            o.attention_ex(q, k, v, sh, out=out, scratch=scratch)

    best, mean, runs = time_cpu(run_all)
    o.close()
    bound = W.WORKLOADS[number].bound
    value = work / best / (1e12 if bound == "mfma" else 1e9)
    return {"value": value, "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "cores": o.threads,
            "kind": "port", "sample": f"{sample}; oracle/attn_oracle.c; " + cpu_timing(best, mean, runs),
            "seconds": best}


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")


def kernel_sources_sha() -> str:
    """SHA-256 (first 16 hex digits) of the kernel sources (zwhisper_amd/csrc/*), in name order:
    the traffic figures of profiles/traffic.json record the sources they were measured on."""
    import hashlib

    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "zwhisper_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".hpp")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def _traffic_table() -> dict:
    try:
        with open(TRAFFIC_JSON) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def traffic_for(workload_name: str):
    """HBM bytes per step from the committed rocprofv3 counter summary, if one exists.  The
    figure is not measured in this run (counters need a run of their own under rocprofv3 --pmc);
    traffic_source() says where it comes from and whether the kernels have changed since."""
    return _traffic_table().get(workload_name)


def traffic_source() -> dict:
    """Where roofline.traffic comes from: profiles/traffic.json, two rocprofv3 --pmc passes
    (FETCH_SIZE, WRITE_SIZE) scaled by a device-copy calibration, measured on the kernel sources
    whose hash it records; `current` says whether those are the sources that ran here."""
    cal = _traffic_table().get("_calibration", {})
    measured = cal.get("sources_sha")
    now = kernel_sources_sha()
    return {"file": "profiles/traffic.json", "measured_in_this_run": False,
            "counters": "rocprofv3 --pmc FETCH_SIZE (x%.3f) + WRITE_SIZE (x%.3f), separate passes"
                        % (cal.get("fetch_factor", float("nan")), cal.get("write_factor", float("nan"))),
            "sources_sha_measured": measured, "sources_sha_now": now, "current": measured == now}


DENSE_DTYPE = ("x3: f32 inputs split into 16-bit hi + lo terms (f16 for Q.K^T and for P.V), three 16-bit MFMA "
               "products per product, f32 accumulation")


def step_rate(number: int, ms_per_step: float) -> dict:
    """Windows/s (encoders) or tokens/s (decoder and LLM) of a workload's steps, at wall time."""
    from zwhisper_amd import workloads as W

    w = W.WORKLOADS[number]
    per_s = 1e3 / ms_per_step
    if number in (1, 2):
        return {"value": w.n_items * per_s, "unit": "windows/s", "per_step": w.n_items}
    if number == 4:
        return {"value": w.n_q * per_s, "unit": "tokens/s", "per_step": w.n_q, "note": "prompt tokens"}
    return {"value": w.n_items * per_s, "unit": "tokens/s", "per_step": w.n_items,
            "note": "one new token per window or sequence"}


def dense_roofline(achieved: float, dense_math: int) -> dict:
    """MFMA roofline of a dense attention kernel at `achieved` algorithmic FLOP/s.

    The x3 kernel issues three 16-bit MFMA products (hi*hi + hi*lo + lo*hi) per algorithmic
    product, so it is priced against the f16/bf16 dense peak with a ceiling of frac 1/3; the
    fp32 kernel against the fp32 dense peak.
    """
    if dense_math == 0:
        return {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_MFMA_F16 / 1e12, "unit": "TFLOP/s",
                "frac": achieved / PEAK_MFMA_F16, "mfma_products_per_product": 3,
                "issued_frac": 3 * achieved / PEAK_MFMA_F16,
                "note": "f16/bf16 MFMA peak; three 16-bit products per algorithmic product, so the kernel's "
                        "ceiling is frac 1/3 and issued_frac is the share of the 16-bit MFMA peak issued"}
    return {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_MFMA_F32 / 1e12, "unit": "TFLOP/s",
            "frac": achieved / PEAK_MFMA_F32}


def _attention_line(wl: Workload, r: dict, dense_math: int) -> dict:
    """Result record of an attention workload: value at wall time per step, roofline at the
    kernels' event time per step."""
    spec = wl.spec
    per_step = wl.work
    achieved = per_step / (r["kernel_ms_mean"] * 1e-3)
    if spec.bound == "mfma":
        roof = dense_roofline(achieved, dense_math)
        value = per_step / (r["ms_per_step"] * 1e-3) / 1e12
        unit = "TFLOP/s"
        dtype = DENSE_DTYPE if dense_math == 0 else "f32 (fp32 MFMA)"
    else:
        roof = {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": achieved / PEAK_HBM}
        value = per_step / (r["ms_per_step"] * 1e-3) / 1e9
        unit = "GB/s"
        dtype = "f32"
    if spec.bound == "mfma":
        cold_rec = cold(r, per_step, "TFLOP/s", PEAK_MFMA_F16 if dense_math == 0 else PEAK_MFMA_F32,
                        3 if dense_math == 0 else 1)
    else:
        cold_rec = cold(r, per_step, "GB/s", PEAK_HBM)
    return {"workload": spec.name, "description": spec.description, "value": value, "unit": unit,
            "rate": step_rate(wl.number, r["ms_per_step"]), "ms_per_step": r["ms_per_step"],
            "kernel_ms_mean": r["kernel_ms_mean"], "kernel_ms_median": r["kernel_ms_median"],
            "kernel_ms_min": r["kernel_ms_min"], "algorithmic_work_per_step": per_step, "dtype": dtype,
            "roofline": roof, "cold": cold_rec, "settle_s": r["settle_s"]}


def _say(name: str, res: dict, peak_name: str) -> None:
    """One summary line and the workload's full record (one JSON object) on stderr.  stdout carries
    only the final headline line."""
    roof = res.get("roofline", {})
    if roof.get("traffic") is not None:
        roof["traffic_source"] = TRAFFIC_SOURCE
    cpu = res.get("cpu_baseline")
    par = res.get("parity")
    print(f"[bench] {name}: {res['value']:.2f} {res['unit']} ({res['ms_per_step']:.4f} ms/step, kernels "
          f"{res['kernel_ms_mean']:.4f} ms, {100 * res['roofline']['frac']:.1f}% of {peak_name})"
          + (f", cold {res['cold']['kernel_ms_per_step']:.4f} ms ({100 * res['cold']['frac']:.1f}%)"
             if "cold" in res else "")
          + (f", parity max abs {par['max_abs']:.2e} rel {par['normwise_rel']:.2e}" if par else "")
          + (f", cpu {cpu['value']:.3f} {cpu['unit']} on {cpu['cores']} threads" if cpu else ""),
          file=sys.stderr, flush=True)
    print("[bench-record] " + json.dumps({"workload": name, **{k: v for k, v in res.items() if k != "workload"}}),
          file=sys.stderr, flush=True)


EXTRAS = ("qwen05_prefill_8x256", "small_dec_kv_append_x32", "qwen15_kv_append_x64", "qwen05_prefill_kv_append",
          "base_enc_linear_x16",
          "base_enc_layer_x16", "qwen15_logits_q8_x64", "qwen15_decode_q8_linear_x64", "small_dec_q8_linear_x32",
          "small_dec_qkv_cache_x32", "qwen15_qkv_cache_x64", "small_dec_step_x32", "qwen15_step_x64",
          "qwen05_prompt_2048")


def run_extra(name: str, torch, ctx, args, threads: int) -> dict:
    """One of the measurements around the attention path (cache updates, projections, a whole
    encoder layer, int8 decode-step projections)."""
    if name == "qwen05_prefill_8x256":
        wl = PromptWorkload(torch, ctx)
        r = time_workload(wl, args.steps, args.warmup)
        res = _attention_line(wl, r, 0)
        res["workload"] = wl.name
        res["description"] = wl.spec.description + "; as llm.prompt feeds it: 8 calls of 256 rows over growing caches"
        res["calls_per_step"] = wl.calls
        res["roofline"]["traffic"] = traffic_for(wl.name)
        if not args.no_parity:
            res["parity"] = wl.parity(x3=True)
        res["cpu_baseline_note"] = "the qwen05_prefill line's cpu_baseline times the oracle in this same 8 x 256 form"
        wl.free()
        _say(name, res, "mfma peak")
        return res
    if name in ("small_dec_kv_append_x32", "qwen15_kv_append_x64", "qwen05_prefill_kv_append"):
        wl = AppendWorkload(name, torch, ctx)
        r = time_workload(wl, args.steps, args.warmup)
        dev_ms = wl.device_time(max(args.steps, 20))
        achieved = wl.work / (dev_ms * 1e-3)
        res = {"workload": name, "description": wl.description,
               "value": wl.work / (r["ms_per_step"] * 1e-3) / 1e9, "unit": "GB/s", "ms_per_step": r["ms_per_step"],
               "kernel_ms_mean": dev_ms, "kernel_ms_note": "device time per update, from a HIP graph of "
               "back-to-back updates; ms_per_step includes this Python harness's launch overhead",
               "algorithmic_work_per_step": wl.work,
               "roofline": {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                            "frac": achieved / PEAK_HBM, "traffic": None}}
        if not args.no_cpu:
            res["cpu_baseline"] = wl.cpu_baseline()
        wl.free()
        _say(name, res, "hbm peak")
        return res
    if name == "base_enc_linear_x16":
        wl = LinearWorkload(torch, ctx)
        r = time_workload(wl, args.steps, args.warmup)
        achieved = wl.work / (r["kernel_ms_mean"] * 1e-3)
        res = {"workload": wl.name, "description": wl.description,
               "value": wl.work / (r["ms_per_step"] * 1e-3) / 1e12, "unit": "TFLOP/s",
               "ms_per_step": r["ms_per_step"], "kernel_ms_mean": r["kernel_ms_mean"],
               "kernel_ms_median": r["kernel_ms_median"], "kernel_ms_min": r["kernel_ms_min"],
               "algorithmic_work_per_step": wl.work,
               "dtype": "f32 activations x f16 weights, f32 accumulation (f16 MFMA, x split into two f16 terms)",
               "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_MFMA_F16 / 1e12,
                            "unit": "TFLOP/s", "frac": achieved / PEAK_MFMA_F16, "traffic": traffic_for(wl.name),
                            "note": "two f16 MFMAs per f32 x f16 product: the kernels' ceiling is frac 0.5"},
               "cold": cold(r, wl.work, "TFLOP/s", PEAK_MFMA_F16, 2)}
        if not args.no_cpu:
            res["cpu_baseline"] = wl.cpu_baseline(threads)
        wl.free()
        _say(name, res, "f16 mfma peak")
        return res
    if name == "base_enc_layer_x16":
        wl = EncoderLayerWorkload(torch, ctx)
        r = time_workload(wl, args.steps, args.warmup)
        achieved = wl.work / (r["kernel_ms_mean"] * 1e-3)
        peak = wl.work / wl.ideal_s
        res = {"workload": wl.name, "description": wl.description,
               "value": wl.work / (r["ms_per_step"] * 1e-3) / 1e12, "unit": "TFLOP/s",
               "ms_per_step": r["ms_per_step"], "kernel_ms_mean": r["kernel_ms_mean"],
               "kernel_ms_median": r["kernel_ms_median"], "kernel_ms_min": r["kernel_ms_min"],
               "algorithmic_work_per_step": wl.work,
               "dtype": "f32 (projections: f32 x f16 on f16 MFMA with x split into two f16 terms; attention: x3 "
                        "16-bit MFMA)",
               "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                            "frac": achieved / peak, "traffic": traffic_for(wl.name),
                            "note": "peak = the layer's flops over the time they take at their own peaks: "
                                    "projections at half the f16 MFMA peak, attention at a third of the 16-bit MFMA "
                                    "peak"},
               "cold": cold(r, wl.work, "TFLOP/s", peak)}
        if not args.no_cpu:
            res["cpu_baseline"] = wl.cpu_baseline(threads)
        wl.free()
        _say(name, res, "the layer's mfma roofline")
        return res
    if name == "qwen05_prompt_2048":
        wl = LlmPromptWorkload(name, "Qwen2.5-0.5B 2048-token prompt as llm.prompt feeds it (src/llm.zig:258-266): 8 "
                               "zwg_llm_forward_dev calls of 256 tokens, each through 24 layers (RMS norms, int8 "
                               "q/k/v with rotary positions into the transposed cache, causal GQA attention 14q/2kv "
                               "x 64 over the cache so far, o, SwiGLU MLP) and the last token's logits over the "
                               "151936-token vocabulary", torch, ctx)
        r = time_workload(wl, args.steps, args.warmup)
        achieved = wl.work / (r["kernel_ms_mean"] * 1e-3)
        peak = wl.work / wl.ideal_s
        res = {"workload": wl.name, "description": wl.description,
               "value": wl.work / (r["ms_per_step"] * 1e-3) / 1e12, "unit": "TFLOP/s",
               "ms_per_step": r["ms_per_step"], "kernel_ms_mean": r["kernel_ms_mean"],
               "kernel_ms_median": r["kernel_ms_median"], "kernel_ms_min": r["kernel_ms_min"],
               "algorithmic_work_per_step": wl.work, "dtype": wl.dtype,
               "roofline": {"bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                            "frac": achieved / peak, "traffic": traffic_for(wl.name),
                            "note": "peak = the step's flops over the time they take at their own peaks: projections "
                                    "at half the f16 MFMA peak, attention at a third of the 16-bit MFMA peak"},
               "cold": cold(r, wl.work, "TFLOP/s", peak)}
        res.update(wl.extra_record(args.steps))
        res["tokens_per_s"] = wl.n_tok / (r["ms_per_step"] * 1e-3)
        if not args.no_cpu:
            res["cpu_baseline"] = wl.cpu_baseline(threads)
        wl.free()
        torch.cuda.empty_cache()
        _say(name, res, "the step's mfma roofline")
        return res
    for q8_name, make in q8_workloads(torch, ctx):
        if q8_name != name:
            continue
        wl = make()
        r = time_workload(wl, args.steps, args.warmup)
        achieved = wl.work / (r["kernel_ms_mean"] * 1e-3)
        res = {"workload": wl.name, "description": wl.description,
               "value": wl.work / (r["ms_per_step"] * 1e-3) / 1e9, "unit": "GB/s",
               "ms_per_step": r["ms_per_step"], "kernel_ms_mean": r["kernel_ms_mean"],
               "kernel_ms_median": r["kernel_ms_median"], "kernel_ms_min": r["kernel_ms_min"],
               "algorithmic_work_per_step": wl.work,
               "dtype": getattr(wl, "dtype", None) or "f32 activations x int8 block weights, f32 accumulation (f16 MFMA, x split into two "
                        "f16 terms, block sums scaled in f32)",
               "roofline": {"bound": "hbm", "achieved": achieved / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                            "frac": achieved / PEAK_HBM, "traffic": traffic_for(wl.name)},
               "cold": cold(r, wl.work, "GB/s", PEAK_HBM)}
        if hasattr(wl, "extra_record"):
            res.update(wl.extra_record(args.steps))
        if "tokens_per_step" in res:
            res["tokens_per_s"] = res["tokens_per_step"] / (r["ms_per_step"] * 1e-3)
        if not args.no_cpu:
            res["cpu_baseline"] = wl.cpu_baseline(threads)
        wl.free()
        torch.cuda.empty_cache()
        _say(name, res, "hbm peak")
        return res
    raise ValueError(f"unknown workload {name}")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", type=int, default=2, choices=[1, 2, 3, 4, 5], help="headline workload")
    ap.add_argument("--only", action="store_true", help="measure the headline workload only")
    ap.add_argument("--dense-math", choices=["x3", "fp32"], default="x3",
                    help="arithmetic of the dense kernel for the headline workload")
    ap.add_argument("--extra", choices=EXTRAS, default=None,
                    help="measure only this workload around the attention path (no attention workloads)")
    ap.add_argument("--skip-extra", choices=EXTRAS, action="append", default=[],
                    help="leave this workload around the attention path out of the full run (repeatable)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-parity", action="store_true", help="skip the f64 parity checks of the outputs")
    ap.add_argument("--calibrate-copy", type=int, metavar="MIB", default=0,
                    help="only run a plain device copy of MIB MiB five times (the reference kernel that "
                         "scales rocprofv3's FETCH_SIZE/WRITE_SIZE counters to bytes)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}).", file=sys.stderr)
        return 2

    import torch

    import zwhisper_amd as z
    from zwhisper_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "launches": 5}), flush=True)
        return 0
    global TRAFFIC_SOURCE
    TRAFFIC_SOURCE = traffic_source()
    host = host_cpus()
    threads = host_threads()
    print(f"[bench] host: {host['cpu_model']}, nproc {host['nproc']}, CPUs for this job {host['cpus']}, "
          f"CPU baselines on {threads} threads (4 for decode)", file=sys.stderr, flush=True)
    head_math = z.DENSE_FP32 if args.dense_math == "fp32" else z.DENSE_X3
    ctx = z.Context(0)
    results = {}
    if args.extra:
        res = run_extra(args.extra, torch, ctx, args, threads)
        ctx.close()
        if "cpu_baseline" in res:
            res["cpu_baseline"].update({"nproc": host["nproc"], "cpus_for_job": host["cpus"],
                                        "cpu_model": host["cpu_model"]})
        line = {"metric": res["workload"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
                "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
                "higher_is_better": True, "host": host, "result": res}
        print(json.dumps(line), flush=True)
        return 0

    numbers = [args.workload] + ([] if args.only else [n for n in (1, 2, 3, 4, 5) if n != args.workload])
    head_ctx = z.Context(0, dense_math=head_math) if head_math != z.DENSE_X3 else ctx
    for n in numbers:
        spec = W.WORKLOADS[n]
        copies = 2 if spec.bound == "hbm" else 1
        c = head_ctx if n == args.workload else ctx
        dm = head_math if n == args.workload else z.DENSE_X3
        wl = Workload(n, torch, c, copies)
        r = time_workload(wl, args.steps, args.warmup)
        res = _attention_line(wl, r, dm)
        res["roofline"]["traffic"] = traffic_for(spec.name if dm == z.DENSE_X3 else spec.name + "_fp32mfma")
        if not args.no_parity:
            res["parity"] = wl.parity(x3=dm == z.DENSE_X3)
        if not args.only and dm == z.DENSE_X3 and n != 4:
            res["dropin_host_buffers"] = wl.dropin()
        if not args.no_cpu:
            res["cpu_baseline"] = cpu_baseline(n, threads)
            if n in (3, 5):
                res["cpu_baseline_all_threads"] = cpu_baseline(n, threads, decode_pool=False)
            if n == 4:
                res["cpu_baseline_one_call"] = cpu_baseline(n, threads, one_call=True)
        results[n] = res
        _say(spec.name, res, f"{spec.bound} peak")
        wl.free()
        del wl
        torch.cuda.empty_cache()
    if head_ctx is not ctx:
        head_ctx.close()
    if not args.only:
        # the dense workloads again on the fp32-MFMA kernel (ZWG_DENSE_FP32), for comparison
        ctx32 = z.Context(0, dense_math=z.DENSE_FP32)
        for n in (2, 1, 4):
            spec = W.WORKLOADS[n]
            wl = Workload(n, torch, ctx32, 1)
            r = time_workload(wl, args.steps, args.warmup)
            name = spec.name + "_fp32mfma"
            res = _attention_line(wl, r, z.DENSE_FP32)
            res["workload"] = name
            res["description"] = spec.description + "; fp32 MFMA kernel (ZWG_DENSE_FP32)"
            res["roofline"]["traffic"] = traffic_for(name)
            if not args.no_parity:
                res["parity"] = wl.parity(x3=False)
            results[name] = res
            _say(name, res, "fp32 mfma peak")
            wl.free()
            del wl
            torch.cuda.empty_cache()
        ctx32.close()
        for name in EXTRAS:
            if name not in args.skip_extra:
                results[name] = run_extra(name, torch, ctx, args, threads)
    ctx.close()
    # every CPU baseline states the host it ran on
    for res in results.values():
        for key, val in res.items():
            if key.startswith("cpu_baseline") and isinstance(val, dict):
                val.update({"nproc": host["nproc"], "cpus_for_job": host["cpus"], "cpu_model": host["cpu_model"]})

    head = results[args.workload]
    spec = W.WORKLOADS[args.workload]
    line = {
        "metric": "encoder/prefill attn TFLOP/s + decode-attn HBM GB/s on 1 MI355X, % roofline",
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded N(0,1), SplitMix64 + Box-Muller)",
        "config": {"workload": spec.name, "items": spec.n_items, "n_q": spec.n_q, "n_kv": spec.n_kv_cap,
                   "n_head": spec.n_head, "n_head_kv": spec.n_head_kv, "head_dim": spec.d, "causal": spec.causal,
                   "k_layout": "transposed" if spec.kt else "row-major", "parallelism": "single GPU"},
        "roofline": head["roofline"],
        "cold": head["cold"],
        "rate": head["rate"],
        "kernel_ms_median": head["kernel_ms_median"],
        "parity": head.get("parity"),
        "host": {k: host[k] for k in ("cpu_model", "nproc", "cpus")},
        "cpu_baseline": head.get("cpu_baseline"),
        # the other workloads, one short entry each; their full records are the "[bench-record]"
        # lines on stderr
        "workloads": {r["workload"]: _brief(r) for n, r in results.items() if n != args.workload},
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


def _brief(res: dict) -> dict:
    """A workload's entry on the headline line: value, step time and roofline fraction."""
    out = {"value": round(res["value"], 4), "unit": res["unit"], "ms_per_step": round(res["ms_per_step"], 5),
           "frac": round(res["roofline"]["frac"], 4), "bound": res["roofline"]["bound"]}
    if "parity" in res and res["parity"] is not None:
        out["parity_ok"] = res["parity"]["within_bar"]
    return out


if __name__ == "__main__":
    sys.exit(main())
