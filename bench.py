#!/usr/bin/env python3
"""Decode-step benchmark of libmx at the Qwen3-0.6B shape (one MI355X).

A step is one decode token's pass of the hot path at the Qwen3-0.6B shape (the Qwen3-TTS 0.6B talker / Qwen3-ASR 0.6B
text decoder): GET_ROWS of the token's row of the tied 151936 x 1024 Q8_0 embedding, then per layer (28) the q/k/v,
attn_o, gate/up and down Q8_0 mat-vecs, then the 151936-row Q8_0 lm_head mat-vec -- 197 mat-vecs reading
633,233,408 bytes of weights per token. Every weight tensor is distinct and lives in HBM; q/k/v and gate/up each run
as one launch (they share their input). The ops between them (RMSNorm, RoPE, attention over the f16 KV cache, SwiGLU,
argmax) stay on ggml's CPU backend in this design, so each mat-vec reads a synthetic N(0,1) activation vector resident
in HBM. The step is recorded once as a graph and replayed.

Prints one JSON line. --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
METRIC = "quant mat-vec weight GB/s (% HBM peak); decode tok/s at Qwen3-0.6B shape"
HBM_PEAK_GBPS = 8000.0

# Qwen3-0.6B shape
LAYERS, HIDDEN, FFN, NQ, NKV, HEAD_DIM, VOCAB = 28, 1024, 3072, 16, 8, 128, 151936
Q8_0_ROW = lambda k: k // 32 * 34  # noqa: E731


def load_mx():
    name = "speech_cpp_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg = ROOT / "speech.cpp_amd"
    spec = importlib.util.spec_from_file_location(name, pkg / "__init__.py", submodule_search_locations=[str(pkg)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def layer_shapes():
    """(name, K, N) of one layer's linears, ggml order: W [K, N]."""
    q, kv = NQ * HEAD_DIM, NKV * HEAD_DIM
    return [("q", HIDDEN, q), ("k", HIDDEN, kv), ("v", HIDDEN, kv), ("o", q, HIDDEN), ("gate", HIDDEN, FFN),
            ("up", HIDDEN, FFN), ("down", FFN, HIDDEN)]


def weight_seed(layer: int, idx: int) -> int:
    return 0x5EED0000 + 2 * 16 + layer * 16 + idx


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Model:
    """The decode step's tensors on the device, built from seeded synthetic weights."""

    def __init__(self, mx, be, threads: int):
        self.mx, self.be = mx, be
        t0 = time.time()
        self.host = {}
        self.layers = []
        for l in range(LAYERS):
            ws = {}
            for i, (name, K, N) in enumerate(layer_shapes()):
                q = mx.quantize_normal(mx.Q8_0, weight_seed(l, i), N, K, 0.02, nthreads=threads)
                ws[name] = be.tensor(mx.Q8_0, (K, N), q)
                self.host[(l, name)] = q
            self.layers.append(ws)
        head = mx.quantize_normal(mx.Q8_0, weight_seed(LAYERS, 0), VOCAB, HIDDEN, 0.02, nthreads=threads)
        self.embd = be.tensor(mx.Q8_0, (HIDDEN, VOCAB), head)
        self.host["embd"] = head
        log(f"weights generated and uploaded in {time.time() - t0:.1f} s")
        # activations: the token id, its embedding row, and one synthetic input per mat-vec of every layer
        self.ids = be.tensor(mx.I32, (1,), np.array([4242], np.int32))
        self.x0 = be.tensor(mx.F32, (HIDDEN, 1))
        self.acts = []
        for l in range(LAYERS):
            a = {}
            for j, (name, K) in enumerate([("attn_out", NQ * HEAD_DIM), ("ffn_in", HIDDEN), ("ffn_act", FFN),
                                           ("final", HIDDEN)]):
                a[name] = be.tensor(mx.F32, (K, 1), mx.fill_normal(0xAC700002 + 16 * l + j, 1, K))
            self.acts.append(a)
        self.outs = []
        for l in range(LAYERS):
            self.outs.append({name: be.tensor(mx.F32, (N, 1)) for name, K, N in layer_shapes()})
        self.logits = be.tensor(mx.F32, (VOCAB, 1))

    def launches(self):
        """The step as a list of (label, K, weight bytes, callable)."""
        be, L = self.be, []
        L.append(("get_rows", HIDDEN, Q8_0_ROW(HIDDEN), lambda: be.get_rows(self.embd, self.ids, self.x0)))
        for l in range(LAYERS):
            w, o, a = self.layers[l], self.outs[l], self.acts[l]
            x_in = self.x0 if l == 0 else a["final"]  # layer 0 reads the embedding row GET_ROWS produced
            L.append(("qkv", HIDDEN, sum(Q8_0_ROW(w[n].ne[0]) * w[n].ne[1] for n in ("q", "k", "v")),
                      lambda w=w, o=o, x=x_in: be.mul_mat_group([w["q"], w["k"], w["v"]], x, [o["q"], o["k"], o["v"]])))
            L.append(("attn_o", NQ * HEAD_DIM, Q8_0_ROW(w["o"].ne[0]) * w["o"].ne[1],
                      lambda w=w, o=o, a=a: be.mul_mat(w["o"], a["attn_out"], o["o"])))
            L.append(("gate_up", HIDDEN, sum(Q8_0_ROW(w[n].ne[0]) * w[n].ne[1] for n in ("gate", "up")),
                      lambda w=w, o=o, a=a: be.mul_mat_group([w["gate"], w["up"]], a["ffn_in"], [o["gate"], o["up"]])))
            L.append(("down", FFN, Q8_0_ROW(w["down"].ne[0]) * w["down"].ne[1],
                      lambda w=w, o=o, a=a: be.mul_mat(w["down"], a["ffn_act"], o["down"])))
        L.append(("lm_head", HIDDEN, Q8_0_ROW(HIDDEN) * VOCAB,
                  lambda: be.mul_mat(self.embd, self.acts[LAYERS - 1]["final"], self.logits)))
        return L


def per_label_pass(be, launches, reps: int):
    """Mean kernel time (ms) per launch of each label: each label's launches (the 28 layers' instances, distinct
    weights) are recorded as a graph of their own and replayed, so no event sits between two kernels. All graphs are
    recorded first and freed last."""
    labels = []
    for lab, _, _, _ in launches:
        if lab not in labels:
            labels.append(lab)
    graphs = {}
    for lab in labels:
        be.graph_begin()
        for l, _, _, fn in launches:
            if l == lab:
                fn()
        graphs[lab] = be.graph_end()
    out = {}
    e0, e1 = be.event(), be.event()
    for lab in labels:
        count = sum(1 for l, _, _, _ in launches if l == lab)
        for _ in range(3):
            be.graph_launch(graphs[lab])
        be.sync()
        be.record(e0)
        for _ in range(reps):
            be.graph_launch(graphs[lab])
        be.record(e1)
        be.sync()
        out[lab] = be.elapsed_ms(e0, e1) / (reps * count)
    be.event_free(e0)
    be.event_free(e1)
    for g in graphs.values():
        be.graph_free(g)
    return out


def cpu_baseline(mx, model, seconds: float):
    """The oracle's AVX2 multi-threaded port of ggml's CPU mul_mat on the same weights, one token at a time."""
    sys.path.insert(0, str(ROOT))
    import oracle as O

    threads = O.physical_cores()
    x = {K: mx.fill_normal(0xAC700002 + K, 1, K) for K in (HIDDEN, NQ * HEAD_DIM, FFN)}
    shapes = layer_shapes()
    ids = np.array([4242], np.int32)

    def token():
        O.get_rows(O.TYPE_Q8_0, model.host["embd"][4242:4243], HIDDEN, np.array([0], np.int32))
        for l in range(LAYERS):
            for name, K, N in shapes:
                O.cpu_fast_mul_mat(O.TYPE_Q8_0, model.host[(l, name)], x[K], threads)
        O.cpu_fast_mul_mat(O.TYPE_Q8_0, model.host["embd"], x[HIDDEN], threads)

    del ids
    token()  # first run excluded
    n, t0 = 0, time.perf_counter()
    while True:
        token()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": n / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} full decode tokens (1 GET_ROWS + 197 Q8_0 mat-vecs, 633 MB of weights each) after one "
                      f"untimed token, {el:.1f} s, AVX2 int8 dots, src1 quantized once per product, rows split "
                      f"across {threads} threads"}


COPY_BYTES = 256 << 20  # the plain copy the counters are calibrated on
TRAFFIC_FILE = ROOT / "profiles" / "k_matvec_q8_0_qwen3-0.6b_decode.traffic.txt"


def summarize_pmc(fetch_csv: str, write_csv: str) -> str:
    """Per-dispatch HBM traffic of the step's mat-vecs from two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE,
    KiB per dispatch), each scaled by what the counter reads for the run's plain 256 MiB device copy."""
    import csv
    import statistics

    def per_kernel(path, counter):
        vals = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return vals

    f = per_kernel(fetch_csv, "FETCH_SIZE")
    w = per_kernel(write_csv, "WRITE_SIZE")
    copy = [k for k in f if "copyBuffer" in k]
    f_cal = max(max(f[k]) for k in copy) * 1024 / COPY_BYTES   # counter bytes per byte actually read
    w_cal = max(max(w[k]) for k in copy if k in w) * 1024 / COPY_BYTES
    mv = [k for k in f if "k_matvec" in k]
    fetch = [v for k in mv for v in f[k]]
    write = [v for k in mv for v in w.get(k, [])]
    fb = statistics.mean(fetch) * 1024 / f_cal
    wb = statistics.mean(write) * 1024 / w_cal if write else 0.0
    lines = [f"kernel family: k_matvec<Q8_0,1,*> ({len(fetch)} dispatches)",
             f"copy calibration: FETCH_SIZE reads {f_cal:.4f} x and WRITE_SIZE {w_cal:.4f} x the bytes of a "
             f"{COPY_BYTES >> 20} MiB device copy",
             f"fetch_bytes_per_launch: {fb:.0f}", f"write_bytes_per_launch: {wb:.0f}",
             f"traffic_bytes_per_launch: {fb + wb:.0f}"]
    return "\n".join(lines)


def read_traffic():
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":")[1]))
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU-baseline sample (0 skips it)")
    ap.add_argument("--no-graph", action="store_true", help="replay the step eagerly instead of as a graph")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic summary of two rocprofv3 --pmc runs of this benchmark and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc))
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported by this build", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    mx = load_mx()
    if mx.device_count() < 1:
        print("no GPU visible to libmx", file=sys.stderr)
        sys.exit(1)
    be = mx.Backend(0)
    threads = max(1, len(os.sched_getaffinity(0)))
    model = Model(mx, be, threads)
    launches = model.launches()
    weight_bytes = sum(b for _, _, b, _ in launches)
    act_bytes = (HIDDEN * 4 + LAYERS * 4 * (HIDDEN + NQ * HEAD_DIM + HIDDEN + FFN) +
                 4 * (LAYERS * sum(N for _, _, N in layer_shapes()) + VOCAB + HIDDEN))

    def step_eager():
        for _, _, _, fn in launches:
            fn()

    step_eager()
    be.sync()
    graph = None
    if not args.no_graph:
        be.graph_begin()
        step_eager()
        graph = be.graph_end()
    step = (lambda: be.graph_launch(graph)) if graph else step_eager

    # A plain device copy of known size: the reference the HBM traffic counters are calibrated on.
    cp_src, cp_dst = be.tensor(mx.F32, (COPY_BYTES // 4,)), be.tensor(mx.F32, (COPY_BYTES // 4,))
    mx.check(mx.lib().mx_tensor_copy(be.h, cp_src.ref(), cp_dst.ref()))
    be.sync()
    cp_src.free()
    cp_dst.free()

    for _ in range(args.warmup):
        step()
    be.sync()
    e0, e1 = be.event(), be.event()
    t0 = time.perf_counter()
    be.record(e0)
    for _ in range(args.steps):
        step()
    be.record(e1)
    be.sync()
    wall = time.perf_counter() - t0
    ms_events = be.elapsed_ms(e0, e1)
    ms_per_step = ms_events / args.steps
    log(f"timed {args.steps} steps: {ms_events:.2f} ms by events, {wall * 1e3:.2f} ms by wall clock")

    # Roofline of the dominant kernel: k_matvec over Q8_0 at batch 1 (every launch of the step but the one GET_ROWS;
    # the template is instantiated per lanes-per-row, all the same code).
    per_ms = per_label_pass(be, launches, reps=20)
    by_label = {}
    for label, K, b, _ in launches:
        d = by_label.setdefault(label, [0, 0])
        d[0] += 1
        d[1] += b
    for label, (n, b) in by_label.items():
        ms = per_ms[label]
        log(f"{label:8s} {n:3d} launches  {ms * 1e3:8.2f} us each  {b / n / 1e6:8.2f} MB each  "
            f"{b / n / (ms * 1e-3) / 1e9:8.1f} GB/s")
    mv = [lab for lab in by_label if lab != "get_rows"]
    mv_launches = sum(by_label[lab][0] for lab in mv)
    mv_bytes = sum(by_label[lab][1] for lab in mv)
    mv_ms = sum(per_ms[lab] * by_label[lab][0] for lab in mv)
    dom_name = "k_matvec<Q8_0, NC=1>"
    per_launch_bytes = mv_bytes / mv_launches
    per_launch_ms = mv_ms / mv_launches
    achieved = per_launch_bytes / (per_launch_ms * 1e-3) / 1e9
    dom = {"launches": mv_launches}

    traffic = read_traffic()

    tok_s = 1e3 / ms_per_step
    step_gbps = weight_bytes / (ms_per_step * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized by quantize_row_q8_0_ref; N(0,1) activations)",
        "config": {"workload": "qwen3-0.6b-shape decode step, batch 1", "layers": LAYERS, "hidden": HIDDEN,
                   "ffn": FFN, "q_heads": NQ, "kv_heads": NKV, "head_dim": HEAD_DIM, "vocab": VOCAB,
                   "weights": "Q8_0", "ops_per_step": "1 GET_ROWS + 197 MUL_MAT in 114 launches",
                   "graph": graph is not None},
        "weight_bytes_per_step": weight_bytes,
        "weight_GBps": round(step_gbps, 1),
        "hbm_frac_step": round(step_gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "launches_per_step": dom["launches"], "bytes_per_launch": int(per_launch_bytes),
                     "us_per_launch": round(per_launch_ms * 1e3, 3)},
    }
    del act_bytes
    if graph:
        be.graph_free(graph)
    be.event_free(e0)
    be.event_free(e1)
    if rank == 0 and args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_baseline(mx, model, args.cpu_seconds)
    be.close()
    if rank == 0:
        print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
