#!/usr/bin/env python3
"""Benchmark of the paged KV-cache hot path on one MI355X.

Default workload (the headline metric): Qwen2.5-7B attention
geometry (28 query heads, 4 kv heads, head_dim 128, 28 layers), fp16 K/V in
16-token pages, 16 sessions with context lengths uniform in [512, 8192]
(seeded), pages scattered by a seeded shuffle of a shared pool.  One step =
plan the batch partition once (launch_attn_decode_plan), then for each of the
28 layers: append 1 token per session and run split-K paged attention for all
sessions in one fused call (launch_attn_decode_paged_planned with k_new/v_new:
split kernel + combine kernel), the whole step replayed from a HIP graph.  Inputs (pool, tables, Q, new K/V for every layer) are
resident in HBM before timing starts.  The appended position is the same each
step (slot ctx_i of session i is rewritten), so every step does identical work.

Output: one JSON line (metric = KV GB/s; ms_per_step; roofline of the decode
kernel measured with HIP events; cpu_baseline = oracle/cpu_baseline.c, a
vectorised, threaded host restatement, on the host cores over one layer of the
same workload).

Other workloads (--workload): single1p5b (config 1), cow (config 3),
longctx14b (config 4), prefill (config 5), rope (RoPE fused with the append,
config-5 chunk shape), gemv (Q4_K projections of one 7B decode layer).  They
print their own JSON line.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "conflux-nova_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import nova_amd  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E vendor peak
FP16_MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA vendor peak



CPU_SAMPLE_S = 10.0     # host seconds per CPU baseline: the sample call is repeated up to this


def timed_repeat(fn, min_s=CPU_SAMPLE_S, max_reps=10000):
    """Calls fn until min_s seconds have passed (at least once); returns
    (seconds per call, the first call's result, number of calls)."""
    t0 = time.perf_counter()
    first = fn()
    n = 1
    while time.perf_counter() - t0 < min_s and n < max_reps:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, first, n


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode7b",
                    choices=["decode7b", "single1p5b", "cow", "longctx14b", "prefill", "rope", "gemv", "copycal"])
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--main-only", action="store_true",
                    help="decode workloads: time the batched step only (no per-session or fused-RoPE comparison legs)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = all host cores")
    ap.add_argument("--configs", default="all", choices=["all", "main"],
                    help="decode7b: 'all' adds configs 1, 3, 4 and 5 (their own timing, roofline, CPU baseline "
                         "and parity) under the line's 'configs' key; 'main' times config 2 only")
    return ap.parse_args()


def cpu_threads(args) -> int:
    if args.cpu_threads:
        return args.cpu_threads
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


class Timer:
    """HIP events on a given stream."""

    def __init__(self, nova, stream):
        self.n, self.s = nova, stream
        self.a, self.b = nova.dev_event_create(), nova.dev_event_create()

    def start(self):
        self.n.dev_event_record(self.a, self.s)

    def stop(self) -> float:
        self.n.dev_event_record(self.b, self.s)
        return self.n.dev_event_elapsed_ms(self.a, self.b)


def decode_bytes(n_keys, nkv, hd, nh, layers) -> int:
    """Algorithmic HBM bytes of append + decode (per step, all layers)."""
    n_keys = np.asarray(n_keys, np.int64)
    per_layer = (n_keys * nkv * hd * 2 * 2            # K + V rows read (fp16)
                 + nkv * hd * 2 * 2                   # appended K + V row written
                 + 4 * ((n_keys + 15) // 16)          # block-table entries
                 + nh * hd * 4 * 2)                   # Q read, O written (fp32)
    return int(per_layer.sum()) * layers


class DecodeWorkload:
    """Ragged batched decode: pool, tables, per-layer Q / new K/V, graph."""

    def __init__(self, nova, ctx, seed, stream, layers=None):
        self.nova, self.s = nova, stream
        self.layers = layers or nova.n_layers
        rng = np.random.default_rng(seed)
        self.ctx = np.asarray(ctx, np.int32)
        self.n = len(ctx)
        self.n_keys = (self.ctx + 1).astype(np.int32)          # append at pos ctx, attend ctx+1 keys
        pages = (self.n_keys + 15) // 16
        self.max_pages = int(pages.max())
        self.nb = int(pages.sum()) + 8
        perm = rng.permutation(self.nb).astype(np.int32)
        tables = np.zeros((self.n, self.max_pages), np.int32)
        off = 0
        for i in range(self.n):
            tables[i, :pages[i]] = perm[off:off + pages[i]]
            off += pages[i]
        self.tables_h = tables
        page_halves = nova.kb * nova.kvw
        self.layer_halves = self.nb * page_halves
        per_pool = nova.n_layers * self.layer_halves
        self.k = nova.alloc(per_pool * 2)
        self.v = nova.alloc(per_pool * 2)
        nova.testkit_fill_normal_f16(self.k.ptr, per_pool, seed * 7 + 1, 1.0, stream)
        nova.testkit_fill_normal_f16(self.v.ptr, per_pool, seed * 7 + 2, 1.0, stream)
        self.tables = nova.upload(tables)
        self.nk = nova.upload(self.n_keys)
        L = self.layers
        self.q_h = rng.standard_normal((L, self.n, nova.nh, nova.hd)).astype(np.float32)
        self.knew_h = rng.standard_normal((L, self.n, nova.nkv, nova.hd)).astype(np.float16).view(np.uint16)
        self.vnew_h = rng.standard_normal((L, self.n, nova.nkv, nova.hd)).astype(np.float16).view(np.uint16)
        self.q = nova.upload(self.q_h)
        self.knew = nova.upload(self.knew_h)
        self.vnew = nova.upload(self.vnew_h)
        self.o = nova.alloc(L * self.n * nova.nh * nova.hd * 4)
        self.ws = nova.alloc(nova.attn_decode_batch_workspace_bytes(self.n))
        nova.dev_zero(self.ws.ptr, self.ws.nbytes, stream)
        nova.dev_stream_sync(stream)
        self.graph = None

    def plan(self):
        # n_keys and the block tables are the same in every layer of a step
        self.nova.launch_attn_decode_plan(self.tables.ptr, self.max_pages, self.nk.ptr, self.n, self.ws.ptr, self.s)

    def launch_layer(self, l):
        nv = self.nova
        qs = self.n * nv.nh * nv.hd
        kvs = self.n * nv.kvw
        nv.launch_attn_decode_paged_planned(
            self.q.ptr + l * qs * 4, self.k.ptr, self.v.ptr, self.tables.ptr, self.max_pages, self.n, l, self.nb,
            self.knew.ptr + l * kvs * 2, self.vnew.ptr + l * kvs * 2, self.o.ptr + l * qs * 4, self.ws.ptr, self.s)

    def step_eager(self):
        self.plan()
        for l in range(self.layers):
            self.launch_layer(l)

    def capture(self):
        nv = self.nova
        nv.dev_graph_begin(self.s)
        self.step_eager()
        self.graph = nv.dev_graph_end(self.s)

    def step(self):
        self.nova.dev_graph_launch(self.graph, self.s)

    def bytes_per_step(self) -> int:
        nv = self.nova
        return decode_bytes(self.n_keys, nv.nkv, nv.hd, nv.nh, self.layers)

    def kernel_times(self, reps=20):
        """Average duration (ms) of one layer's decode launch pair (split +
        combine: one launch_attn_decode_paged_planned call), of the split
        kernel alone (testkit_attn_decode_split_only) and of the stream floor
        (testkit_decode_stream_floor: the same grid reading the same pages
        with no arithmetic), each from a HIP graph of
        the 28 layers' launches replayed `reps` times and timed with events on
        the stream the kernels run on -- the same replay as the timed step,
        minus the once-per-step plan kernel."""
        nv, s, L = self.nova, self.s, self.layers
        qs, kvs = self.n * nv.nh * nv.hd, self.n * nv.kvw

        def split_only(l):
            nv.testkit_attn_decode_split_only(
                self.q.ptr + l * qs * 4, self.k.ptr, self.v.ptr, self.tables.ptr, self.max_pages, self.n, l, self.nb,
                self.knew.ptr + l * kvs * 2, self.vnew.ptr + l * kvs * 2, self.ws.ptr, s)

        def floor(l):
            nv.testkit_decode_stream_floor(self.k.ptr, self.v.ptr, self.tables.ptr, self.max_pages, self.n, l,
                                           self.nb, self.ws.ptr, s)

        # contiguous floor: the layer's algorithmic bytes as one contiguous
        # non-temporal grid-stride read by two 256-thread workgroups per CU
        # (no pages, no table; the fastest streaming shape measured); layers
        # take disjoint ranges (K pool for the first half of the layers, V
        # pool for the rest), so nothing is read twice per step
        half = (L + 1) // 2
        nbytes = min(self.bytes_per_step() // L, nv.n_layers * self.layer_halves * 2 // half) // 16 * 16
        self.contig_bytes = nbytes
        cus = nv.dev_cu_count()
        sink = nv.alloc(cus * 512 * 4)

        def contig(l):
            src = (self.k.ptr if l < half else self.v.ptr) + (l % half) * nbytes
            nv.testkit_stream_read(src, nbytes, 2 * cus, sink.ptr, s)

        out = {}
        for name, fn in (("pair", self.launch_layer), ("split", split_only), ("floor", floor),
                         ("contig", contig)):
            nv.dev_graph_begin(s)
            for l in range(L):
                fn(l)
            g = nv.dev_graph_end(s)
            for _ in range(3):
                nv.dev_graph_launch(g, s)
            t = Timer(nv, s)
            t.start()
            for _ in range(reps):
                nv.dev_graph_launch(g, s)
            out[name] = t.stop() / (reps * L)
            nv.dev_graph_destroy(g)
        return out["pair"], out["split"], out["floor"], out["contig"]

    def solo_ms(self, steps, warmup):
        """The same step through launch_attn_decode_paged_solo: one launch per
        layer (one workgroup per (kv head, session) streams the session's
        pages, merges on chip and writes O; fused append), no plan, no
        partials, no combine; from a HIP graph, ms per step."""
        nv, s, L = self.nova, self.s, self.layers
        qs, kvs = self.n * nv.nh * nv.hd, self.n * nv.kvw
        nv.dev_graph_begin(s)
        for l in range(L):
            nv.launch_attn_decode_paged_solo(
                self.q.ptr + l * qs * 4, self.k.ptr, self.v.ptr, self.tables.ptr, self.max_pages, self.nk.ptr,
                self.n, l, self.nb, self.knew.ptr + l * kvs * 2, self.vnew.ptr + l * kvs * 2,
                self.o.ptr + l * qs * 4, s)
        g = nv.dev_graph_end(s)
        for _ in range(warmup):
            nv.dev_graph_launch(g, s)
        t = Timer(nv, s)
        t.start()
        for _ in range(steps):
            nv.dev_graph_launch(g, s)
        ms = t.stop() / steps
        nv.dev_graph_destroy(g)
        nv.dev_stream_sync(s)
        return ms

    def per_session_ms(self, steps, warmup):
        """The reference's call pattern for the same step (Engine::decode_batch,
        src/model.cpp:282-289): per layer and session one launch_kv_store_paged
        of the new token and one launch_attn_decode_paged, 2N launches per
        layer, replayed from a HIP graph; ms per step."""
        nv, s, L, n = self.nova, self.s, self.layers, self.n
        scratch = nv.alloc(nv.nh * 32 * (nv.hd + 2) * 4)
        tab = [self.tables.ptr + i * self.max_pages * 4 for i in range(n)]
        qs, kvs = n * nv.nh * nv.hd, n * nv.kvw

        def step():
            for l in range(L):
                for i in range(n):
                    nv.launch_kv_store_paged(self.k.ptr, self.v.ptr, tab[i], l, self.nb, 1, int(self.ctx[i]),
                                             self.knew.ptr + (l * kvs + i * nv.kvw) * 2,
                                             self.vnew.ptr + (l * kvs + i * nv.kvw) * 2, s)
                    nv.launch_attn_decode_paged(self.q.ptr + (l * qs + i * nv.nh * nv.hd) * 4, self.k.ptr, self.v.ptr,
                                                tab[i], l, self.nb, int(self.n_keys[i]),
                                                self.o.ptr + (l * qs + i * nv.nh * nv.hd) * 4, scratch.ptr, s)

        nv.dev_graph_begin(s)
        step()
        g = nv.dev_graph_end(s)
        for _ in range(warmup):
            nv.dev_graph_launch(g, s)
        t = Timer(nv, s)
        t.start()
        for _ in range(steps):
            nv.dev_graph_launch(g, s)
        ms = t.stop() / steps
        nv.dev_graph_destroy(g)
        return ms

    def rope_compare(self, steps, warmup):
        """The decode step with RoPE in front of it (a real model's step): the
        separate launch_rope_kv_store_paged_batch + planned decode per layer,
        against launch_attn_decode_paged_rope_planned (one launch pair per
        layer).  Both from HIP graphs; us per step for each."""
        nv, s, L = self.nova, self.s, self.layers
        rows = int(self.n_keys.max())
        half = nv.hd // 2
        cs, sn = nv.alloc(rows * half * 4), nv.alloc(rows * half * 4)
        nv.launch_rope_table_rows(cs.ptr, sn.ptr, rows, s)
        rng = np.random.default_rng(5)
        k32 = nv.upload(rng.standard_normal((L, self.n, nv.nkv, nv.hd)).astype(np.float32))
        v32 = nv.upload(rng.standard_normal((L, self.n, nv.nkv, nv.hd)).astype(np.float32))
        qsep = nv.upload(self.q_h)
        pos = nv.upload(self.ctx)
        qs, kvs = self.n * nv.nh * nv.hd, self.n * nv.kvw

        def separate():
            self.plan()
            for l in range(L):
                nv.launch_rope_kv_store_paged_batch(qsep.ptr + l * qs * 4, k32.ptr + l * kvs * 4,
                                                    v32.ptr + l * kvs * 4, cs.ptr, sn.ptr, self.k.ptr, self.v.ptr,
                                                    self.tables.ptr, self.max_pages, pos.ptr, self.n, 1, l,
                                                    self.nb, s)
                nv.launch_attn_decode_paged_planned(qsep.ptr + l * qs * 4, self.k.ptr, self.v.ptr, self.tables.ptr,
                                                    self.max_pages, self.n, l, self.nb, None, None,
                                                    self.o.ptr + l * qs * 4, self.ws.ptr, s)

        def fused():
            self.plan()
            for l in range(L):
                nv.launch_attn_decode_paged_rope_planned(self.q.ptr + l * qs * 4, k32.ptr + l * kvs * 4,
                                                         v32.ptr + l * kvs * 4, cs.ptr, sn.ptr, self.k.ptr,
                                                         self.v.ptr, self.tables.ptr, self.max_pages, self.n, l,
                                                         self.nb, self.o.ptr + l * qs * 4, self.ws.ptr, s)

        out = {}
        for name, fn in (("separate_us_per_step", separate), ("fused_us_per_step", fused)):
            nv.dev_graph_begin(s)
            fn()
            g = nv.dev_graph_end(s)
            for _ in range(warmup):
                nv.dev_graph_launch(g, s)
            t = Timer(nv, s)
            t.start()
            for _ in range(steps):
                nv.dev_graph_launch(g, s)
            out[name] = round(t.stop() / steps * 1e3, 2)
            nv.dev_graph_destroy(g)
        nv.dev_stream_sync(s)
        return out

    def cpu_sample(self, layer, threads):
        """Run the CPU baseline (oracle/cpu_baseline.c: AVX2/F16C, a thread
        pool over (session, kv head, 64-page split) units) on the host over
        one layer; returns (seconds, outputs).  The appended token goes in
        with the C oracle's append first (untimed)."""
        from oracle_py import CpuBaseline, Oracle
        nv = self.nova
        orc = Oracle()
        cpub = CpuBaseline()
        shape = (self.nb, nv.kb, nv.nkv, nv.hd)
        off = layer * self.layer_halves * 2
        pk = nv.download(self.k.ptr + off, shape, np.uint16)
        pv = nv.download(self.v.ptr + off, shape, np.uint16)
        # the appended token is part of the layer's keys
        for i in range(self.n):
            orc.kv_store_paged(nv.model, pk, pv, np.ascontiguousarray(self.tables_h[i]), 0, self.nb, 1,
                               int(self.ctx[i]), np.ascontiguousarray(self.knew_h[layer, i]),
                               np.ascontiguousarray(self.vnew_h[layer, i]))
        q = np.ascontiguousarray(self.q_h[layer])
        secs, out, reps = timed_repeat(
            lambda: cpub.attn_decode_batch(nv.model, q, pk, pv, self.tables_h, self.n_keys, 0, self.nb, threads))
        self.cpu_reps = reps
        return secs, out


def ragged_ctx(seed, n, lo, hi):
    return np.random.default_rng(seed).integers(lo, hi + 1, n).astype(np.int32)


def load_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("traffic_bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


def run_decode(args, model, ctx, workload_name, metric_cfg, cpu_scale_note):
    nova = nova_amd.load(model)
    s = nova.dev_stream_create()
    wl = DecodeWorkload(nova, ctx, args.seed, s)
    print("[leg] batched step", file=sys.stderr, flush=True)
    wl.step_eager()            # first touch, check launches
    nova.dev_stream_sync(s)
    wl.capture()
    for _ in range(args.warmup):
        wl.step()
    nova.dev_stream_sync(s)
    t = Timer(nova, s)
    nova.dev_sync()
    t.start()
    for _ in range(args.steps):
        wl.step()
    ms = t.stop() / args.steps
    nova.dev_sync()
    bytes_step = wl.bytes_per_step()
    gbs = bytes_step / (ms * 1e-3) / 1e9
    pair_ms, split_ms, floor_ms, contig_ms = wl.kernel_times()
    bytes_launch = bytes_step / wl.layers
    split_gbs = bytes_launch / (split_ms * 1e-3) / 1e9
    pair_gbs = bytes_launch / (pair_ms * 1e-3) / 1e9
    traffic = load_traffic(workload_name)
    roof = {"bound": "hbm", "achieved": round(split_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(split_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": "decode_split_kernel alone (one layer of all sessions; the split + combine pair "
                      "that callers run is launch_pair_*)",
            "kernel_us": round(split_ms * 1e3, 2), "bytes_per_launch": bytes_launch,
            "launch_pair_us": round(pair_ms * 1e3, 2),
            "launch_pair_frac": round(pair_gbs / HBM_PEAK_GBS, 4),
            "step_frac": round(gbs / HBM_PEAK_GBS, 4),
            "stream_floor_us": round(floor_ms * 1e3, 2),
            "stream_floor_frac": round(bytes_launch / (floor_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "contig_floor_us": round(contig_ms * 1e3, 2),
            "contig_floor_frac": round(wl.contig_bytes / (contig_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "contig_floor_bytes": wl.contig_bytes,
            "timing": "HIP events around graph replays of the 28 layers' launches: split kernel alone "
                      "(testkit_attn_decode_split_only), the split + combine pair "
                      "(launch_attn_decode_paged_planned) and the stream floor (testkit_decode_stream_floor: "
                      "the split grid reading the same pages with the same loads, no arithmetic), the contiguous "
                      "floor (testkit_stream_read: the same bytes as one contiguous grid-stride read, two workgroups per CU); "
                      "step_frac = the timed step incl. the plan kernel"}
    # the one-launch solo path (one CU per session and kv head): timed where
    # its sessions are short enough to finish in minutes at this step count
    got_split = nova.download(wl.o, (wl.n, nova.nh, nova.hd), np.float32)
    solo_ms = None
    if wl.max_pages <= 128:
        print("[leg] solo step", file=sys.stderr, flush=True)
        solo_ms = wl.solo_ms(args.steps, args.warmup)
    got_solo = nova.download(wl.o, (wl.n, nova.nh, nova.hd), np.float32) if solo_ms else None
    cpu = None
    parity = None
    if not args.no_cpu:
        th = cpu_threads(args)
        secs, out = wl.cpu_sample(0, th)
        # parity at full size on layer 0 (GPU output of the last replay of each path)
        err = float(np.abs(got_split - out).max())
        parity = {"layer0_max_abs_err": err, "ok": err <= 2e-3}
        if got_solo is not None:
            err_solo = float(np.abs(got_solo - out).max())
            parity["solo_layer0_max_abs_err"] = err_solo
            parity["ok"] = parity["ok"] and err_solo <= 2e-3
            err = max(err, err_solo)
        if not parity["ok"]:
            print(f"bench: PARITY FAILURE on layer 0: max|gpu-cpu| = {err:.3e}", file=sys.stderr, flush=True)
        cpu_gbs = (bytes_step / wl.layers) / secs / 1e9
        cpu = {"value": round(cpu_gbs, 3), "unit": "GB/s", "cores": th, "kind": "port",
               "sample": f"1 of {wl.layers} layers ({cpu_scale_note}); cb_attn_decode_batch "
                         f"(oracle/cpu_baseline.c: AVX2/F16C, {th} threads), "
                         f"{secs * 1e3:.3f} ms per call (mean of {wl.cpu_reps}, warm host caches); max|gpu-cpu| on that layer {err:.2e}",
               "us_per_step_equiv": round(secs * wl.layers * 1e6, 1)}
    # after the parity leg above: they rewrite the outputs and the appended slots
    per_session = rope = None
    if not getattr(args, "main_only", False):
        print("[leg] per-session launches", file=sys.stderr, flush=True)
        per_session = wl.per_session_ms(args.steps, args.warmup)
        if model == "qwen25_7b":
            print("[leg] rope in step", file=sys.stderr, flush=True)
            rope = wl.rope_compare(args.steps, args.warmup)
    line = {
        "metric": metric_cfg["metric"], "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "us_per_step": round(ms * 1e3, 2), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16 KV / f32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V, Q; seeded ragged contexts and page shuffle)",
        "config": metric_cfg["config"], "roofline": roof, "cpu_baseline": cpu,
    }
    if solo_ms is not None:
        solo = {"ms_per_step": round(solo_ms, 4), "GBs": round(bytes_step / (solo_ms * 1e-3) / 1e9, 1),
                "pct_hbm_peak": round(100 * bytes_step / (solo_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                "us_per_layer": round(solo_ms * 1e3 / wl.layers, 2),
                "what": "the same step through launch_attn_decode_paged_solo: one launch per layer, one "
                        "workgroup per (kv head, session) streaming the session's pages, output written by the "
                        "split kernel (no plan, no partials, no combine launch), fused append"}
        if solo_ms < ms:
            # the faster path leads the line; the planned split path stays beside it
            split = {"ms_per_step": line["ms_per_step"], "GBs": line["value"], "pct_hbm_peak": line["pct_hbm_peak"],
                     "what": "plan + 28 x launch_attn_decode_paged_planned (split + combine), from a HIP graph",
                     "roofline": roof}
            sgbs = bytes_step / (solo_ms * 1e-3) / 1e9
            line.update({"value": round(sgbs, 2), "ms_per_step": round(solo_ms, 4),
                         "us_per_step": round(solo_ms * 1e3, 2), "pct_hbm_peak": round(100 * sgbs / HBM_PEAK_GBS, 2),
                         "path": "solo (launch_attn_decode_paged_solo)", "split_path": split})
            line["roofline"] = {"bound": "hbm", "achieved": round(sgbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(sgbs / HBM_PEAK_GBS, 4), "traffic": load_traffic(workload_name + "_solo"),
                                "kernel": "decode_split_kernel<solo> (one launch per layer: the whole step's work)",
                                "kernel_us": round(solo_ms * 1e3 / wl.layers, 2), "bytes_per_launch": bytes_launch,
                                "timing": "HIP events around graph replays of the step's 28 solo launches"}
        else:
            line["solo_path"] = solo
    if parity:
        line["parity"] = parity
    if per_session:
        line["per_session_launches"] = {
            "ms_per_step": round(per_session, 4), "GBs": round(bytes_step / (per_session * 1e-3) / 1e9, 1),
            "what": "the same step as the reference calls it: per layer and session launch_kv_store_paged + "
                    "launch_attn_decode_paged (2N launches per layer), from a HIP graph"}
    if rope:
        line["rope_in_step"] = dict(rope, note="the same step with RoPE of q and the new k in front of each layer: "
                                               "launch_rope_kv_store_paged_batch + planned decode, against "
                                               "launch_attn_decode_paged_rope_planned (RoPE and append inside the "
                                               "decode launch)")
    return line


# ---------------------------------------------------------------------------
# config 3: copy-on-write prefix sharing
# ---------------------------------------------------------------------------
VOCAB = 151936
ROOT_LEN = 2048
FORK = 2047           # unaligned fork point: with 16-token pages a 2048-token fork never COWs
N_ROOTS, PER_ROOT = 4, 16


def run_cow(args):
    """4 roots x 2048 seeded token ids, 64 children forked at 2047 tokens, each
    appending a divergent suffix of U[0,1024] tokens token by token.  The first
    append of every child copies the shared, half-filled tail page (all 28
    layers, K and V); the timed figure is that batched COW copy.  Block tables,
    refcounts, free list, cow_count and the kv_block IDs are compared with the C
    oracle driven by the same calls."""
    import ctypes as C
    from oracle_py import Oracle
    nova = nova_amd.load("qwen25_7b")
    orc = Oracle()
    rng = np.random.default_rng(args.seed)
    n_child = N_ROOTS * PER_ROOT
    suffix = rng.integers(0, 1025, n_child)
    order = np.argsort(-suffix, kind="stable")          # children created longest-suffix first
    suffix = suffix[order]
    ctx = ROOT_LEN + 1024
    n_slices = N_ROOTS + n_child + 4                     # 4 spare slices feed alloc_block
    h = nova.nova_paged_new(n_slices, ctx)
    pool = nova.nova_paged_pool(h)
    nb = nova.nova_paged_nb(h)
    nblocks = nova.nova_kvpool_nblocks(pool)
    st = nova.nova_paged_stream(h)
    kp, vp = nova.nova_paged_pool_k(h), nova.nova_paged_pool_v(h)
    oh = orc.pool.new(n_slices, ctx)
    sess = [nova.nova_paged_create_session(h, 1) for _ in range(N_ROOTS + n_child)]
    osess = [orc.pool.acquire(oh) for _ in range(N_ROOTS + n_child)]
    assert sess == osess
    per_pool = nova.n_layers * nb * nova.kb * nova.kvw
    nova.testkit_fill_normal_f16(kp, per_pool, args.seed * 3 + 1, 1.0, st)
    nova.testkit_fill_normal_f16(vp, per_pool, args.seed * 3 + 2, 1.0, st)
    nova.dev_stream_sync(st)
    # kv_block IDs: prefix = hash(root prompt up to the fork), suffix = hash(child ids) ^ 1
    root_ids = rng.integers(0, VOCAB, (N_ROOTS, ROOT_LEN)).astype(np.int32)
    child_ids = [rng.integers(0, VOCAB, int(L)).astype(np.int32) for L in suffix]

    def nova_hash(ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        return nova.nova_kv_hash_ids(a.ctypes.data_as(C.POINTER(C.c_int)), len(a))

    ids_ok = True
    reg, oreg = nova.nova_registry_new(), orc.registry.new()
    for c in range(n_child):
        root = c % N_ROOTS
        p1, p2 = nova_hash(root_ids[root][:FORK]), orc.kv_hash_ids(root_ids[root][:FORK].tolist())
        s1, s2 = nova_hash(child_ids[c]) ^ 1, orc.kv_hash_ids(child_ids[c].tolist()) ^ 1
        ids_ok &= (p1 == p2) and (s1 == s2)
        nova.nova_registry_put(reg, p1, s1, N_ROOTS + c, 1, FORK, FORK + int(suffix[c]))
        orc.registry.put(oreg, p2, s2, N_ROOTS + c, 1, FORK, FORK + int(suffix[c]))
    ids_ok &= nova.nova_registry_live(reg) == orc.registry.live(oreg)
    # fork
    layer0 = (nb, nova.kb, nova.nkv, nova.hd)
    before_k = nova.download(kp, layer0, np.uint16)
    for c in range(n_child):
        child, root = N_ROOTS + c, c % N_ROOTS
        nova.nova_paged_attach_prefix(h, child, root, FORK)
        orc.pool.attach_prefix(oh, child, root, FORK)
    # first append of every child: one batched COW (decisions in session order)
    ids = (C.c_int * n_child)(*range(N_ROOTS, N_ROOTS + n_child))
    pos = (C.c_int64 * n_child)(*([FORK] * n_child))
    one = (C.c_int * n_child)(*([1] * n_child))
    t = Timer(nova, st)
    t.start()
    copies = nova.nova_paged_cow_batch(h, ids, pos, one, n_child, st)
    first_ms = t.stop()
    for c in range(n_child):
        orc.pool.cow_slice(oh, N_ROOTS + c, FORK)
    # the same 64 page copies, repeated, for a stable per-launch time
    lb = FORK >> 4
    ops = (nova_amd.CowOp * n_child)()
    for c in range(n_child):
        child, root = N_ROOTS + c, c % N_ROOTS
        ops[c].src = orc.pool.table_arr(oh, root)[lb]
        ops[c].dst = orc.pool.table_arr(oh, child)[lb]
        ops[c].table_index = child * nblocks + lb
    for _ in range(args.warmup):
        nova.launch_kv_cow_apply(kp, vp, nb, nova.nova_paged_tables(h), ops, n_child, st)
    t.start()
    for _ in range(args.steps):
        nova.launch_kv_cow_apply(kp, vp, nb, nova.nova_paged_tables(h), ops, n_child, st)
    cow_ms = t.stop() / args.steps
    page_bytes = nova.n_layers * 2 * nova.kb * nova.kvw * 2
    cow_bytes = n_child * 2 * page_bytes                 # read + write of every copied page
    # suffix appends, token by token, all layers (children sorted: active ones are a prefix)
    maxL = int(suffix.max())
    kvn = nova.alloc(nova.n_layers * max(maxL, 1) * n_child * nova.kvw * 2 * 2)
    nova.testkit_fill_normal_f16(kvn.ptr, nova.n_layers * max(maxL, 1) * n_child * nova.kvw * 2,
                                 args.seed * 3 + 3, 1.0, st)
    posbuf = nova.upload(np.full(n_child, FORK, np.int32))
    tables_child = nova.nova_paged_tables(h) + N_ROOTS * nblocks * 4
    extra_cow = 0
    t.start()
    for step in range(maxL):
        active = int((suffix > step).sum())
        act = (C.c_int * active)(*range(N_ROOTS, N_ROOTS + active))
        ps = (C.c_int64 * active)(*([FORK + step] * active))
        ns = (C.c_int * active)(*([1] * active))
        extra_cow += nova.nova_paged_cow_batch(h, act, ps, ns, active, st)
        for c in range(active):
            orc.pool.cow_slice(oh, N_ROOTS + c, FORK + step)
        pv = np.full(active, FORK + step, np.int32)
        nova.dev_upload_async(posbuf.ptr, pv.ctypes.data, pv.nbytes, st)
        nova.dev_stream_sync(st)
        for l in range(nova.n_layers):
            base = kvn.ptr + ((l * maxL + step) * n_child) * nova.kvw * 2 * 2
            nova.launch_kv_store_paged_batch(kp, vp, tables_child, nblocks, posbuf.ptr, active, l, nb, 1,
                                             base, base + n_child * nova.kvw * 2, st)
    append_ms = t.stop()
    nova.dev_stream_sync(st)
    # ---- parity ----
    from ctypes import c_int32
    def prod_table(s_):
        n = nova.nova_kvpool_table(pool, s_, None, 0)
        buf = (c_int32 * n)()
        nova.nova_kvpool_table(pool, s_, buf, n)
        return list(buf)
    def prod_free():
        n = nova.nova_kvpool_free_list(pool, None, 0)
        buf = (C.c_int * max(n, 1))()
        nova.nova_kvpool_free_list(pool, buf, n)
        return list(buf[:n])
    tables_ok = all(prod_table(s_) == orc.pool.table_arr(oh, s_) for s_ in sess)
    refcnt_ok = [nova.nova_kvpool_refcnt(pool, b) for b in range(nb)] == orc.pool.refcnt_arr(oh)
    free_ok = prod_free() == orc.pool.free_list_arr(oh)
    cow_ok = (copies == n_child and extra_cow == 0 and
              nova.nova_kvpool_cow_count(pool) == orc.pool.cow_count(oh) == n_child)
    dev_tables = nova.download(nova.nova_paged_tables(h), (n_slices, nblocks), np.int32)
    dev_ok = all(dev_tables[s_].tolist() == orc.pool.table_arr(oh, s_) for s_ in sess)
    # data: children see the donor prefix then their own suffix; donors untouched
    after_k = nova.download(kp, layer0, np.uint16)
    data_ok = True
    kv_h = None
    for c in (0, n_child // 2, n_child - 1):
        child, root = N_ROOTS + c, c % N_ROOTS
        L = int(suffix[c])
        got = orc.kv_gather_paged("qwen25_7b", after_k, np.asarray(orc.pool.table_arr(oh, child), np.int32), 0, nb,
                                  FORK + L)
        want_prefix = orc.kv_gather_paged("qwen25_7b", before_k, np.asarray(orc.pool.table_arr(oh, root), np.int32),
                                          0, nb, FORK)
        data_ok &= np.array_equal(got[:FORK], want_prefix)
        if L:
            if kv_h is None:
                # layer 0 block of each step: [K rows of all children][V rows of all children]
                kv_h = nova.download(kvn, (maxL, 2, n_child, nova.nkv, nova.hd), np.uint16)
            data_ok &= np.array_equal(got[FORK:], kv_h[:L, 0, c])
    donor_ok = all(np.array_equal(after_k[p], before_k[p])
                   for r_ in range(N_ROOTS) for p in orc.pool.table_arr(oh, r_)[:lb + 1])
    # the same launch with 64 distinct donor pages (after the parity checks: it
    # overwrites pages and table entries nothing reads afterwards): every
    # copied byte comes from HBM, so this is the kernel's HBM rate
    ops2 = (nova_amd.CowOp * n_child)()
    base = nb - 2 * n_child
    for c in range(n_child):
        ops2[c].src, ops2[c].dst, ops2[c].table_index = base + c, base + n_child + c, c
    for _ in range(args.warmup):
        nova.launch_kv_cow_apply(kp, vp, nb, nova.nova_paged_tables(h), ops2, n_child, st)
    t.start()
    for _ in range(args.steps):
        nova.launch_kv_cow_apply(kp, vp, nb, nova.nova_paged_tables(h), ops2, n_child, st)
    distinct_ms = t.stop() / args.steps
    nova.dev_stream_sync(st)
    nova.nova_paged_delete(h)
    gbs = cow_bytes / (cow_ms * 1e-3) / 1e9
    hbm_gbs = cow_bytes / (distinct_ms * 1e-3) / 1e9
    # CPU baseline: the same 64 page copies (every layer, K and V) with the C
    # oracle's or_cow_copy on a host pool of the 4 donor pages + 64 fresh pages
    # (a bounded stand-in for the full pool, which is not mirrored on the host)
    hp_k = np.zeros((nova.n_layers, N_ROOTS + n_child, nova.kb, nova.nkv, nova.hd), np.uint16)
    hp_v = np.zeros_like(hp_k)
    hp_k[:, :N_ROOTS] = 1
    hp_v[:, :N_ROOTS] = 2
    def cow_all():
        for c in range(n_child):
            orc.cow_copy("qwen25_7b", hp_k, hp_v, nova.n_layers, N_ROOTS + n_child, c % N_ROOTS, N_ROOTS + c)
    cpu_secs, _, cpu_reps = timed_repeat(cow_all)
    cpu_ok = bool(np.all(hp_k[:, N_ROOTS:] == 1) and np.all(hp_v[:, N_ROOTS:] == 2))
    return {
        # value: the 64-copy launch's HBM rate (64 distinct donor pages, every
        # copied byte read from and written to HBM); config 3's own launch,
        # whose 4 shared donor pages are read from cache, is shared_donors
        "metric": "COW fork page copy GB/s (config 3, Qwen2.5-7B)", "value": round(hbm_gbs, 1), "unit": "GB/s",
        "us_per_launch": round(distinct_ms * 1e3, 2), "pct_hbm_peak": round(100 * hbm_gbs / HBM_PEAK_GBS, 2),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
        "dtype": "f16 KV (byte copy)", "data": "synthetic (seeded token ids, N(0,1) K/V)",
        "config": {"workload": "config3: 4 roots x 2048 tokens, 64 children forked at 2047 tokens "
                               "(unaligned, so the half-filled tail page is shared), suffix U[0,1024] "
                               "appended token by token", "fork_tokens": FORK, "children": n_child,
                   "suffix_tokens_total": int(suffix.sum())},
        # the roofline is the kernel's HBM rate: the same 64-copy launch with 64
        # distinct donor pages, every byte from HBM.  Config 3's own launch
        # copies 4 donor pages 16 times each; its reads come from cache, so its
        # rate (shared_donors) exceeds the HBM peak and is no HBM figure.
        "roofline": {"bound": "hbm", "achieved": round(hbm_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(hbm_gbs / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": "cow_apply_kernel (launch_kv_cow_apply), 64 copies from 64 distinct donor pages",
                     "kernel_us": round(distinct_ms * 1e3, 2), "bytes_per_launch": cow_bytes},
        "shared_donors": {"us": round(cow_ms * 1e3, 2), "GBs": round(gbs, 1),
                          "traffic": load_traffic("cow"),
                          "what": "config 3's own launch: 64 copies of 4 donor pages (16 children per donor), "
                                  "the donor reads served from cache; traffic = measured HBM bytes per launch"},
        "first_cow_batch_us": round(first_ms * 1e3, 2),
        "append_ms_total": round(append_ms, 1), "append_steps": maxL,
        "parity": {"tables": tables_ok, "device_tables": dev_ok, "refcounts": refcnt_ok, "free_list": free_ok,
                   "cow_once_per_child": cow_ok, "kv_block_ids": bool(ids_ok), "data": bool(data_ok),
                   "donor_untouched": bool(donor_ok)},
        "cpu_baseline": {"value": round(cow_bytes / cpu_secs / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"the same 64 COW page copies (28 layers, K and V) with the C oracle's "
                                   f"or_cow_copy on a host pool of 68 pages, single-threaded, "
                                   f"{cpu_secs * 1e3:.1f} ms per call (mean of {cpu_reps}); copies verified: {cpu_ok}"},
    }


# ---------------------------------------------------------------------------
# config 5: chunked prefill append + causal paged attention (MFMA)
# ---------------------------------------------------------------------------
def prefill_flops(n_past, n_q, nh, hd) -> int:
    n_past = np.asarray(n_past, np.int64)
    keys = n_past * n_q + n_q * (n_q + 1) // 2          # sum over q of (P + q + 1)
    return int((keys * nh * 4 * hd).sum())


def run_prefill(args):
    nova = nova_amd.load("qwen25_7b")
    s = nova.dev_stream_create()
    rng = np.random.default_rng(args.seed)
    n_sess, n_q = 8, 512
    n_past = rng.integers(0, 4097, n_sess).astype(np.int32)
    pages = (n_past + n_q + 15) // 16
    nb = int(pages.sum()) + 8
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((n_sess, int(pages.max())), np.int32)
    off = 0
    for i in range(n_sess):
        tables[i, :pages[i]] = perm[off:off + pages[i]]
        off += pages[i]
    L = nova.n_layers
    per_pool = L * nb * nova.kb * nova.kvw
    k, v = nova.alloc(per_pool * 2), nova.alloc(per_pool * 2)
    nova.testkit_fill_normal_f16(k.ptr, per_pool, args.seed + 11, 1.0, s)
    nova.testkit_fill_normal_f16(v.ptr, per_pool, args.seed + 12, 1.0, s)
    chunk_elems = n_sess * n_q * nova.kvw
    kc, vc = nova.alloc(L * chunk_elems * 2), nova.alloc(L * chunk_elems * 2)
    nova.testkit_fill_normal_f16(kc.ptr, L * chunk_elems, args.seed + 13, 1.0, s)
    nova.testkit_fill_normal_f16(vc.ptr, L * chunk_elems, args.seed + 14, 1.0, s)
    q_h = rng.standard_normal((n_sess, n_q, nova.nh, nova.hd)).astype(np.float32)   # one layer's Q
    q = nova.upload(q_h)
    o = nova.alloc(L * q_h.nbytes)
    dt, dp = nova.upload(tables), nova.upload(n_past)
    stride = tables.shape[1]

    def layer_ops(l):
        nova.launch_kv_store_paged_batch(k.ptr, v.ptr, dt.ptr, stride, dp.ptr, n_sess, l, nb, n_q,
                                         kc.ptr + l * chunk_elems * 2, vc.ptr + l * chunk_elems * 2, s)
        nova.launch_attn_prefill_paged_batch(q.ptr, k.ptr, v.ptr, dt.ptr, stride, dp.ptr, n_sess, n_q, l, nb,
                                             o.ptr + l * q_h.nbytes, s)

    for l in range(L):
        layer_ops(l)
    nova.dev_stream_sync(s)
    nova.dev_graph_begin(s)
    for l in range(L):
        layer_ops(l)
    g = nova.dev_graph_end(s)
    for _ in range(args.warmup):
        nova.dev_graph_launch(g, s)
    t = Timer(nova, s)
    t.start()
    for _ in range(args.steps):
        nova.dev_graph_launch(g, s)
    ms = t.stop() / args.steps
    # attention kernel alone: a graph of the 28 layers' prefill launches,
    # replayed, HIP events on the stream they run on
    nova.dev_graph_begin(s)
    for l in range(L):
        nova.launch_attn_prefill_paged_batch(q.ptr, k.ptr, v.ptr, dt.ptr, stride, dp.ptr, n_sess, n_q, l, nb,
                                             o.ptr + l * q_h.nbytes, s)
    ga = nova.dev_graph_end(s)
    nova.dev_graph_launch(ga, s)
    reps = max(args.steps, 5)
    t.start()
    for _ in range(reps):
        nova.dev_graph_launch(ga, s)
    k_ms = t.stop() / (reps * L)
    nova.dev_graph_destroy(ga)
    # the reference's call pattern: one launch_attn_prefill_paged per session
    t.start()
    for l in range(L):
        for i in range(n_sess):
            nova.launch_attn_prefill_paged(q.ptr + i * n_q * nova.nh * nova.hd * 4, k.ptr, v.ptr,
                                           dt.ptr + i * stride * 4, l, nb, n_q, int(n_past[i]),
                                           o.ptr + l * q_h.nbytes + i * n_q * nova.nh * nova.hd * 4, s)
    single_ms = t.stop() / L
    flops = prefill_flops(n_past, n_q, nova.nh, nova.hd)
    tflops = flops / (k_ms * 1e-3) / 1e12
    cpu = parity = None
    if not args.no_cpu:
        from oracle_py import CpuBaseline
        cpub = CpuBaseline()
        th = cpu_threads(args)
        shape = (nb, nova.kb, nova.nkv, nova.hd)
        pk = nova.download(k, shape, np.uint16)          # layer 0 (chunk already appended)
        pv = nova.download(v, shape, np.uint16)
        q4 = np.ascontiguousarray(q_h.reshape(n_sess, n_q, nova.nh, nova.hd))
        secs, ref, reps = timed_repeat(lambda: cpub.attn_prefill_batch(
            "qwen25_7b", q4, pk, pv, tables, n_past, n_q, 0, nb, th))
        got = nova.download(o, (n_sess, n_q, nova.nh, nova.hd), np.float32)
        perr = float(np.abs(got - ref).max())
        cpu = {"value": round(flops / secs / 1e12, 6), "unit": "TFLOP/s", "cores": th, "kind": "port",
               "sample": f"layer 0 of 28, all 8 sessions; cb_attn_prefill_batch (oracle/cpu_baseline.c: "
                         f"AVX2/F16C, {th} threads), {secs * 1e3:.1f} ms per call (mean of {reps}); "
                         f"max|gpu-cpu| {perr:.2e}"}
        parity = {"layer0_max_abs_err": perr, "ok": perr <= 2e-3}
        if not parity["ok"]:
            print(f"bench: PARITY FAILURE on prefill: max|gpu-cpu| = {perr:.3e}", file=sys.stderr, flush=True)
    return {
        "metric": "chunked-prefill causal paged attention TFLOP/s (config 5, Qwen2.5-7B)",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "us_per_layer": round(ms * 1e3 / L, 2), "higher_is_better": True,
        "dtype": "f16 MFMA / f32 accumulate", "data": "synthetic (seeded N(0,1) Q/K/V, prefix U[0,4096])",
        "config": {"workload": "config5: 8 sessions, 512-token chunk appended then causal attention over "
                               "prefix U[0,4096] + chunk, 28 layers", "n_past": n_past.tolist(), "chunk": n_q},
        "per_session_launches": {"us_per_layer": round(single_ms * 1e3, 2),
                                 "tflops": round(flops / (single_ms * 1e-3) / 1e12, 2),
                                 "what": "the same layer as 8 launch_attn_prefill_paged calls (the reference's "
                                         "one-session-per-call pattern, src/model.cpp AttnOp)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": load_traffic("prefill"),
                     "kernel": "prefill_kernel (launch_attn_prefill_paged_batch)",
                     "kernel_us": round(k_ms * 1e3, 2), "flops_per_launch": flops},
        "cpu_baseline": cpu,
        **({"parity": parity} if parity else {}),
    }


def rope_bytes(n_tok, nh, nkv, hd) -> int:
    """Algorithmic bytes of RoPE + fp16 append per token: q read and written
    (fp32), k and v read (fp32), the cos/sin row read, k and v written (fp16)."""
    return n_tok * (2 * nh * hd * 4 + 2 * nkv * hd * 4 + 2 * (hd // 2) * 4 + 2 * nkv * hd * 2)


def run_rope(args):
    """RoPE fused with the paged append (launch_rope_kv_store_paged_batch),
    the step before the attention path (RopeKvOp, code/graph/dense.h:75-83):
    a config-5-shaped prefill chunk (8 sessions x 512 tokens at n_past
    U[0,4096]) is the measured launch; a decode step (16 sessions x 1 token)
    is timed beside it."""
    nova = nova_amd.load("qwen25_7b")
    s = nova.dev_stream_create()
    rng = np.random.default_rng(args.seed)
    nh, nkv, hd = nova.nh, nova.nkv, nova.hd
    rows = 16384
    cs, sn = nova.alloc(rows * hd // 2 * 4), nova.alloc(rows * hd // 2 * 4)
    nova.launch_rope_table_rows(cs.ptr, sn.ptr, rows, s)

    def setup(n_sess, n, n_past):
        pages = (n_past + n + 15) // 16
        nb = int(pages.sum()) + 8
        perm = rng.permutation(nb).astype(np.int32)
        tables = np.zeros((n_sess, int(pages.max())), np.int32)
        off = 0
        for i in range(n_sess):
            tables[i, :pages[i]] = perm[off:off + pages[i]]
            off += pages[i]
        pk, pv = nova.alloc(nb * nova.kb * nova.kvw * 2), nova.alloc(nb * nova.kb * nova.kvw * 2)
        q = rng.standard_normal((n_sess, n, nh, hd)).astype(np.float32)
        k = rng.standard_normal((n_sess, n, nkv, hd)).astype(np.float32)
        v = rng.standard_normal((n_sess, n, nkv, hd)).astype(np.float32)
        bufs = dict(q=nova.upload(q), k=nova.upload(k), v=nova.upload(v), t=nova.upload(tables),
                    p=nova.upload(n_past.astype(np.int32)), pk=pk, pv=pv)
        call = lambda: nova.launch_rope_kv_store_paged_batch(  # noqa: E731
            bufs["q"].ptr, bufs["k"].ptr, bufs["v"].ptr, cs.ptr, sn.ptr, pk.ptr, pv.ptr, bufs["t"].ptr,
            tables.shape[1], bufs["p"].ptr, n_sess, n, 0, nb, s)
        return call, (q, k, v, tables, nb, bufs)

    def timed(call, steps):
        for _ in range(args.warmup):
            call()
        t = Timer(nova, s)
        t.start()
        for _ in range(steps):
            call()
        return t.stop() / steps

    n_past = rng.integers(0, 4097, 8).astype(np.int32)
    chunk, (q, k, v, tables, nb, bufs) = setup(8, 512, n_past)
    ms = timed(chunk, max(args.steps, 20))
    nbytes = rope_bytes(8 * 512, nh, nkv, hd)
    ctx = ragged_ctx(args.seed, 16, 512, 8192)
    dec, _ = setup(16, 1, ctx)
    dec_ms = timed(dec, max(args.steps, 50))
    gbs = nbytes / (ms * 1e-3) / 1e9
    # parity of session 0's chunk against the oracle, on fresh inputs
    from oracle_py import Oracle
    orc = Oracle()
    q0 = rng.standard_normal((8, 512, nh, hd)).astype(np.float32)
    nova.dev_upload(bufs["q"].ptr, q0.ctypes.data, q0.nbytes)
    chunk()
    nova.dev_stream_sync(s)
    hcs = nova.download(cs, (rows, hd // 2), np.float32)
    hsn = nova.download(sn, (rows, hd // 2), np.float32)
    got_q = nova.download(bufs["q"], q0.shape, np.float32)
    shape = (nb, nova.kb, nkv, hd)
    gk = nova.download(bufs["pk"], shape, np.uint16)
    gv = nova.download(bufs["pv"], shape, np.uint16)
    hk, hv = np.zeros(shape, np.uint16), np.zeros(shape, np.uint16)
    secs, rq, reps = timed_repeat(lambda: orc.rope_kv_store_paged(
        "qwen25_7b", q0[0], k[0], v[0], hcs, hsn, hk, hv, np.ascontiguousarray(tables[0]), 0, nb, int(n_past[0])))
    rows0 = orc.kv_gather_paged("qwen25_7b", hk, tables[0], 0, nb, int(n_past[0]) + 512)[int(n_past[0]):]
    got0 = orc.kv_gather_paged("qwen25_7b", gk, tables[0], 0, nb, int(n_past[0]) + 512)[int(n_past[0]):]
    rv0 = orc.kv_gather_paged("qwen25_7b", hv, tables[0], 0, nb, int(n_past[0]) + 512)[int(n_past[0]):]
    gv0 = orc.kv_gather_paged("qwen25_7b", gv, tables[0], 0, nb, int(n_past[0]) + 512)[int(n_past[0]):]
    parity = bool(np.array_equal(got_q[0], rq) and np.array_equal(got0, rows0) and np.array_equal(gv0, rv0))
    cpu_bytes = rope_bytes(512, nh, nkv, hd)
    return {
        "metric": "RoPE + paged fp16 append GB/s (config-5 chunk, Qwen2.5-7B)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": max(args.steps, 20), "warmup": args.warmup,
        "higher_is_better": True, "vs_baseline": None, "dtype": "f32 rotate / f16 store",
        "data": "synthetic (seeded N(0,1) q, k, v; prefix U[0,4096]; seeded page shuffle)",
        "config": {"workload": "8 sessions x 512-token chunk at n_past U[0,4096]: rotate q in place, rotate k "
                               "and append k, v as fp16 through the block tables, one launch",
                   "n_past": n_past.tolist(), "chunk": 512},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic("rope"),
                     "kernel": "rope_kernel<true> (launch_rope_kv_store_paged_batch)",
                     "kernel_us": round(ms * 1e3, 2), "bytes_per_launch": nbytes},
        "decode_step_us": round(dec_ms * 1e3, 2),
        "decode_step": "16 sessions x 1 token (ctx U[512,8192]), one launch",
        "parity": {"session0_q_k_v_bit_exact": parity},
        "cpu_baseline": {"value": round(cpu_bytes / secs / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"session 0's 512-token chunk, C oracle or_rope_kv_store_paged "
                                   f"single-threaded, {secs * 1e3:.2f} ms per call (mean of {reps})"},
    }


def run_gemv(args):
    """One Qwen2.5-7B decode layer's Q4_K projections for one token (the
    reference's decode path, src/model.cpp + code/graph/dense.h): quantise
    the normed hidden state, q/k/v projections, quantise the attention output,
    o projection, quantise, gate and up, quantise the FFN activation, down.
    Weights are random bytes with realistic fp16 super-block scales; all
    resident in HBM.  The measured figure is weight + activation bytes over
    the sequence's time; the gate projection (38 MB) is the dominant kernel."""
    nova = nova_amd.load("qwen25_7b")
    s = nova.dev_stream_create()
    rng = np.random.default_rng(args.seed)
    D, FFN, QO, KV = 3584, 18944, 28 * 128, 4 * 128
    shapes = {"q": (QO, D), "k": (KV, D), "v": (KV, D), "o": (D, QO), "gate": (FFN, D), "up": (FFN, D),
              "down": (D, FFN)}
    W = {}
    for name, (rows, cols) in shapes.items():
        b = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
        b[..., 0:2] = rng.uniform(2e-4, 4e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
        b[..., 2:4] = rng.uniform(1e-4, 2e-3, (rows, cols // 256, 1)).astype(np.float16).view(np.uint8)
        W[name] = (nova.upload(b), b)
    acts = {k: nova.upload(rng.standard_normal(n).astype(np.float32)) for k, n in (("x", D), ("ffn", FFN))}
    q8 = {k: (nova.alloc(n), nova.alloc(n // 8), nova.alloc(n // 4)) for k, n in (("x", D), ("ffn", FFN))}
    outs = {name: nova.alloc(rows * 4) for name, (rows, cols) in shapes.items()}

    def gemv(name, act):
        rows, cols = shapes[name]
        qs, d, sm = q8[act]
        nova.launch_gemv_q4k(W[name][0].ptr, rows, cols, qs.ptr, d.ptr, sm.ptr, outs[name].ptr, s)

    def quant(act, n):
        qs, d, sm = q8[act]
        nova.launch_quant_q8(qs.ptr, d.ptr, sm.ptr, acts[act].ptr, 1, n, s)

    def layer_separate():
        """the reference's sequence: quantise, then one GEMV per projection"""
        quant("x", D)
        for name in ("q", "k", "v"):
            gemv(name, "x")
        quant("x", D)
        gemv("o", "x")
        quant("x", D)
        gemv("gate", "x")
        gemv("up", "x")
        quant("ffn", FFN)
        gemv("down", "ffn")

    def fused(names, act):
        n = len(names)
        bl = (C.c_void_p * n)(*[W[m][0].ptr for m in names])
        rw = (C.c_int64 * n)(*[shapes[m][0] for m in names])
        ou = (C.c_void_p * n)(*[outs[m].ptr for m in names])
        nova.launch_gemv_q4k_f32(bl, rw, ou, n, shapes[names[0]][1], acts[act].ptr, s)

    def layer():
        """quantisation inside the GEMV launch for the 3584-wide activation, q/k/v
        and gate/up as one launch each; the 18944-wide FFN activation is
        quantised once by its own launch (inside the launch every workgroup
        would re-quantise it: measured 21.9 vs 12.1 + 3.0 us), as the
        reference does in its producer (launch_swiglu, norm.cu:83-87)"""
        fused(("q", "k", "v"), "x")
        fused(("o",), "x")
        fused(("gate", "up"), "x")
        quant("ffn", FFN)
        gemv("down", "ffn")

    def graph_of(fn, reps=1):
        fn()                                       # eager once: argument checks
        nova.dev_stream_sync(s)
        nova.dev_graph_begin(s)
        for _ in range(reps):
            fn()
        return nova.dev_graph_end(s)

    def time_graph(g, n):
        nova.dev_graph_launch(g, s)
        for _ in range(args.warmup):
            nova.dev_graph_launch(g, s)
        t = Timer(nova, s)
        t.start()
        for _ in range(n):
            nova.dev_graph_launch(g, s)
        return t.stop() / n

    steps = max(args.steps, 50)
    g_layer, g_sep = graph_of(layer), graph_of(layer_separate)
    ms = time_graph(g_layer, steps)
    sep_ms = time_graph(g_sep, steps)
    wbytes = sum(r * c // 256 * 144 for r, c in shapes.values())
    # activation read once per launch (fp32), outputs written
    abytes = 3 * D * 4 + FFN * 4 + (FFN + FFN // 32 * 4 + FFN // 16 * 4) * 2 + sum(r * 4 for r, c in shapes.values())
    gbs = (wbytes + abytes) / (ms * 1e-3) / 1e9
    # the dominant kernel alone: the gate + up launch, 20 per graph replay
    g_gu = graph_of(lambda: fused(("gate", "up"), "x"), 20)
    gate_ms = time_graph(g_gu, steps) / 20

    # Engine::decode_batch's form (model.cpp:262-303): four tokens through the
    # layer, each projection one launch_gemv4_q4k reading its weights once
    x4 = {k: nova.upload(rng.standard_normal((4, n)).astype(np.float32)) for k, n in (("x", D), ("ffn", FFN))}
    q84 = {k: (nova.alloc(4 * n), nova.alloc(4 * n // 8), nova.alloc(4 * n // 4)) for k, n in (("x", D), ("ffn", FFN))}
    outs4 = {name: nova.alloc(4 * rows * 4) for name, (rows, cols) in shapes.items()}

    def quant4(act, n):
        qs, d, sm = q84[act]
        nova.launch_quant_q8(qs.ptr, d.ptr, sm.ptr, x4[act].ptr, 4, n, s)

    def gemv4(name, act):
        rows, cols = shapes[name]
        qs, d, sm = q84[act]
        nova.launch_gemv4_q4k(W[name][0].ptr, rows, cols, qs.ptr, d.ptr, sm.ptr, outs4[name].ptr, s)

    def layer4():
        quant4("x", D)
        for name in ("q", "k", "v"):
            gemv4(name, "x")
        quant4("x", D)
        gemv4("o", "x")
        quant4("x", D)
        gemv4("gate", "x")
        gemv4("up", "x")
        quant4("ffn", FFN)
        gemv4("down", "ffn")

    g_l4 = graph_of(layer4)
    l4_ms = time_graph(g_l4, steps)
    for g in (g_layer, g_sep, g_gu, g_l4):
        nova.dev_graph_destroy(g)
    rows, cols = shapes["gate"]
    gate_bytes = 2 * rows * cols // 256 * 144 + cols * 4 + 2 * rows * 4
    gate_gbs = gate_bytes / (gate_ms * 1e-3) / 1e9
    # parity on the gate projection (sampled rows) and CPU baseline
    from oracle_py import Oracle
    orc = Oracle()
    x = nova.download(acts["x"], (1, D), np.float32)
    xq, xd, xs = orc.quant_q8(x)
    got = nova.download(outs["gate"], (rows,), np.float32)
    sample = 512
    wsample = np.ascontiguousarray(W["gate"][1][:sample])
    secs, ref, reps = timed_repeat(lambda: orc.gemv_q4k(wsample, sample, cols, xq, xd, xs))
    err = float(np.max(np.abs(got[:sample] - ref) / (np.abs(ref) + 1e-3)))
    cpu_bytes = sample * cols // 256 * 144
    return {
        "metric": "Q4_K decode GEMV GB/s, one Qwen2.5-7B layer's projections (q,k,v,o,gate,up,down)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "us_per_layer": round(ms * 1e3, 2), "higher_is_better": True, "vs_baseline": None,
        "separate_launches": {"us_per_layer": round(sep_ms * 1e3, 2),
                              "note": "the reference's call sequence: 4 launch_quant_q8 + 7 launch_gemv_q4k"},
        "four_tokens": {"us_per_layer": round(l4_ms * 1e3, 2), "us_per_token": round(l4_ms * 1e3 / 4, 2),
                        "weight_GBs": round(wbytes / (l4_ms * 1e-3) / 1e9, 1),
                        "note": "Engine::decode_batch's form: 4 launch_quant_q8 (4 rows) + 7 launch_gemv4_q4k"},
        "dtype": "q4_K weights x int8 activations, f32 accumulate",
        "data": "synthetic (seeded random Q4_K blocks with fp16 scales in [1e-4, 4e-3]; N(0,1) activations)",
        "config": {"workload": "one decode token through a Qwen2.5-7B layer's 7 Q4_K projections: "
                               "launch_gemv_q4k_f32 for q/k/v, o and gate/up (each quantising its activation), "
                               "launch_quant_q8 + launch_gemv_q4k for down",
                   "weight_bytes": wbytes, "shapes": shapes},
        "roofline": {"bound": "hbm", "achieved": round(gate_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gate_gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic("gemv"),
                     "kernel": "gemv_fixed_kernel<2, true> (launch_gemv_q4k_f32), gate + up projections, 2 x 18944 x 3584",
                     "kernel_us": round(gate_ms * 1e3, 2), "bytes_per_launch": gate_bytes},
        "parity": {"gate_rows_checked": sample, "max_rel_err": err},
        "cpu_baseline": {"value": round(cpu_bytes / secs / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                         "sample": f"{sample} rows of the gate projection, C oracle or_gemv_q4k (dequantise + "
                                   f"double dot) single-threaded, {secs * 1e3:.2f} ms per call (mean of {reps})"},
    }


def run_copycal(args):
    """Plain copy of 1 GiB (testkit_copy): the known-traffic kernel used to
    calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE (each launch reads and writes
    exactly 1 GiB)."""
    nova = nova_amd.load("qwen25_7b")
    s = nova.dev_stream_create()
    nbytes = 1 << 30
    a, b = nova.alloc(nbytes), nova.alloc(nbytes)
    nova.testkit_fill_normal_f16(a.ptr, nbytes // 2, 1, 1.0, s)
    for _ in range(args.warmup):
        nova.testkit_copy(b.ptr, a.ptr, nbytes, s)
    t = Timer(nova, s)
    t.start()
    for _ in range(args.steps):
        nova.testkit_copy(b.ptr, a.ptr, nbytes, s)
    ms = t.stop() / args.steps
    return {"metric": "plain copy GB/s (read + write)", "value": round(2 * nbytes / ms / 1e6, 1), "unit": "GB/s",
            "bytes_read_per_launch": nbytes, "bytes_written_per_launch": nbytes, "kernel_us": round(ms * 1e3, 2)}


def single1p5b_cfg():
    return np.array([1024], np.int32), {
        "metric": "paged decode step, Qwen2.5-1.5B single session",
        "config": {"workload": "config1: 1 session ctx 1024, Qwen2.5-1.5B attention (12q/2kv, 28 layers)",
                   "sessions": 1, "ctx": 1024, "layers": 28}}


def longctx14b_cfg():
    return np.full(8, 32767, np.int32), {
        "metric": "paged flash-decode KV GB/s, Qwen2.5-14B long context",
        "config": {"workload": "config4: 8 sessions x 32768 tokens, Qwen2.5-14B attention "
                               "(40q/8kv, hd128, 48 layers), ~51.5 GB KV resident",
                   "sessions": 8, "ctx": 32768, "layers": 48}}


# keys of a workload's line that the configs sub-objects leave out (the top
# level states them once)
_SUB_DROP = ("n_gpus", "steps", "warmup", "higher_is_better", "scaling", "vs_baseline", "data")


def other_configs(args):
    """Configs 1, 3, 4 and 5 of BASELINE.json, each with its own timing,
    roofline, CPU baseline and parity, for the default line (config 2 is the
    line itself).  Decode configs time the batched step only."""
    import copy
    sub = copy.copy(args)
    sub.main_only = True
    out = {}
    legs = [("config1", lambda: run_decode(sub, "qwen25_1p5b", single1p5b_cfg()[0], "single1p5b",
                                           single1p5b_cfg()[1], "Qwen2.5-1.5B, 1 session")),
            ("config3", lambda: run_cow(sub)),
            ("config4", lambda: run_decode(sub, "qwen25_14b", longctx14b_cfg()[0], "longctx14b",
                                           longctx14b_cfg()[1], "Qwen2.5-14B, 8 x 32K")),
            ("config5", lambda: run_prefill(sub))]
    for name, fn in legs:
        print(f"[leg] {name}", file=sys.stderr, flush=True)
        r = fn()
        out[name] = {k: v for k, v in r.items() if k not in _SUB_DROP}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU figures are not produced "
                                   "(sessions would shard by GPU with no exchange during decode)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.workload == "decode7b":
        ctx = ragged_ctx(args.seed, 16, 512, 8192)
        cfg = {"metric": "paged flash-decode KV GB/s (% HBM peak) + us/decode step, Qwen2.5-7B shape",
               "config": {"workload": "config2: batched ragged paged flash-decode, Qwen2.5-7B attention "
                                      "(28q/4kv heads, hd128, 28 layers), fp16 KV, 16-token pages, "
                                      "16 sessions ctx U[512,8192], 1-token append + split-K attention per layer",
                          "sessions": 16, "ctx": ctx.tolist(), "layers": 28, "page_tokens": 16}}
        line = run_decode(args, "qwen25_7b", ctx, "decode7b", cfg, "Qwen2.5-7B, 16 sessions")
        if args.configs == "all":
            line["configs"] = other_configs(args)
    elif args.workload == "longctx14b":
        ctx, cfg = longctx14b_cfg()
        line = run_decode(args, "qwen25_14b", ctx, "longctx14b", cfg, "Qwen2.5-14B, 8 x 32K")
    elif args.workload == "single1p5b":
        ctx, cfg = single1p5b_cfg()
        line = run_decode(args, "qwen25_1p5b", ctx, "single1p5b", cfg, "Qwen2.5-1.5B, 1 session")
    elif args.workload == "copycal":
        line = run_copycal(args)
    elif args.workload == "cow":
        line = run_cow(args)
    elif args.workload == "rope":
        line = run_rope(args)
    elif args.workload == "gemv":
        line = run_gemv(args)
    else:
        line = run_prefill(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
