#!/usr/bin/env python3
"""Benchmarks of libmx's quantized products on one MI355X.

Default workload (`--workload decode`): the decode step at the Qwen3-0.6B shape (the Qwen3-TTS 0.6B talker / Qwen3-ASR
0.6B text decoder). GET_ROWS of the token's row of the tied 151936 x 1024 Q8_0 embedding, then per layer (28) the
q/k/v, attn_o, gate/up and down Q8_0 mat-vecs, then the 151936-row Q8_0 lm_head mat-vec -- 197 mat-vecs reading
633,233,408 bytes of weights per token. Every weight tensor is distinct and lives in HBM; q/k/v and gate/up each run
as one launch (they share their input). The ops between them (RMSNorm, RoPE, attention over the f16 KV cache, SwiGLU,
argmax) are not part of this workload, so each mat-vec reads a synthetic N(0,1) activation vector resident in HBM.
The step is recorded once as a graph and replayed.

Other workloads (one JSON line each, same keys):
  decode-full  the same decode step with every op on the device, as Qwen3Decoder::layers builds it: RMSNorm (norm
               weight fused), q/k/v, per-head q/k RMSNorm, NEOX RoPE, SET_ROWS into the f16 KV cache, flash attention
               over the cache prefilled with N(0,1) to 1024 positions (1088 read as 17 blocks of 64, the new token at
               1024), attn_o, residual add, RMSNorm, gate/up, SwiGLU, down, add; final RMSNorm, lm_head, ARGMAX
  matvec       one Q8_0 MUL_MAT 3072 x 1024 at batch 1, rotated over 160 distinct copies of the weight (535 MB)
  prefill-q4k  Qwen3-1.7B-shape talker prefill: 28 layers of Q4_K linears (Q6_K down), M = 512 rows
  asr-1.7b     Qwen3-ASR-1.7B-shape Q8_0 prefill of 1564 rows in blocks {512, 512, 512, 28}, the head on the last
               row, then 32 batch-1 decode tokens
  moe          one Drama3-like MoE FFN layer (gate, up, down MUL_MAT_ID; 64 Q4_K experts, top-4 of a softmax router)
               at token batches of 1, 16 and 256

Prints one JSON line. --gpus N > 1 exits: one GPU is measured.
"""
from __future__ import annotations

import argparse
import gc
import subprocess
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
INT8_PEAK_TOPS = 5000.0   # dense int8 MFMA, MI355X
FP16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLCK = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TSIZE = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
NAME = {Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}
TYPE_OF = {v: k for k, v in NAME.items()}


def row_bytes(t: int, k: int) -> int:
    return k // BLCK[t] * TSIZE[t]


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


def load_oracle():
    sys.path.insert(0, str(ROOT))
    import oracle as O
    return O


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_seed(config: int, layer: int, idx: int) -> int:
    return 0x5EED0000 + config * 16 + layer * 16 + idx


class Launch:
    """One call into libmx: a label (launches of one label share a kernel and a shape class), its algorithmic bytes
    (weights + activations read + outputs written) and int8 ops, and the call."""

    def __init__(self, label, nbytes, ops, fn, weight_bytes=None):
        self.label, self.nbytes, self.ops, self.fn = label, nbytes, ops, fn
        self.weight_bytes = nbytes if weight_bytes is None else weight_bytes


# A read of 2 x EVICT_BYTES through the backend's stream pushes every earlier line out of the 256 MB last-level cache
# (and the L2s), leaving clean lines behind (a copy would leave dirty ones, whose write-back the next kernel would
# pay for); set up by main() once the backend exists.
EVICT_BYTES = 256 << 20
EVICT = None


def make_evictor(mx, be):
    buf = be.tensor(mx.F32, (2 * EVICT_BYTES // 4,))
    mx.check(mx.lib().mx_tensor_memset(be.h, buf.ref(), 0, 0, 2 * EVICT_BYTES))

    def evict():
        be.peak_read(buf, 8192, 16)
    evict()  # sizes the backend's scratch now, before any graph is recorded
    be.sync()
    return evict


def per_label_pass(be, launches, reps: int, use_graph: bool = True):
    """Mean time (ms) per launch of each label: each label's launches are recorded as a graph of their own and
    replayed, so no event sits between two kernels. A label of few small launches repeats them inside its graph (up to
    32 launches), so the graph's own launch cost does not swamp them; launches of 16 MB and more are recorded once, as
    a repeat would find them in the 256 MB last-level cache. A label whose distinct weights total less than twice that
    cache is timed one replay at a time with the caches flushed before each (a 512 MB read outside the events), so
    its replays read their weights from HBM as the step does. All graphs are recorded first and freed last. Without
    graphs the same launches are issued eagerly between the events."""
    labels = []
    for L in launches:
        if L.label not in labels:
            labels.append(L.label)
    graphs, counts, runs = {}, {}, {}
    for lab in labels:
        mine = [L for L in launches if L.label == lab]
        rep = 1 if max(L.nbytes for L in mine) >= (16 << 20) else max(1, 32 // len(mine))

        def run(mine=mine, rep=rep):
            for _ in range(rep):
                for L in mine:
                    L.fn()
        if use_graph:
            be.graph_begin()
            run()
            graphs[lab] = be.graph_end()
            runs[lab] = (lambda g=graphs[lab]: be.graph_launch(g))
        else:
            runs[lab] = run
        counts[lab] = rep * len(mine)
    out = {}
    e0, e1 = be.event(), be.event()
    for lab in labels:
        count = counts[lab]
        for _ in range(3):
            runs[lab]()
        be.sync()
        distinct = sum(L.weight_bytes for L in launches if L.label == lab)
        if EVICT is not None and distinct < 2 * EVICT_BYTES:
            total = 0.0
            for _ in range(reps):
                EVICT()
                be.record(e0)
                runs[lab]()
                be.record(e1)
                be.sync()
                total += be.elapsed_ms(e0, e1)
            out[lab] = total / (reps * count)
            continue
        be.record(e0)
        for _ in range(reps):
            runs[lab]()
        be.record(e1)
        be.sync()
        out[lab] = be.elapsed_ms(e0, e1) / (reps * count)
    be.event_free(e0)
    be.event_free(e1)
    for g in graphs.values():
        be.graph_free(g)
    return out


def label_table(launches, per_ms):
    """{label: (launches, bytes, ops, ms per launch)} and a log line per label."""
    by = {}
    for L in launches:
        d = by.setdefault(L.label, [0, 0, 0])
        d[0] += 1
        d[1] += L.nbytes
        d[2] += L.ops
    out = {}
    for lab, (n, b, ops) in by.items():
        ms = per_ms[lab]
        out[lab] = (n, b, ops, ms)
        extra = f"  {ops / n / (ms * 1e-3) / 1e12:8.1f} TOP/s" if ops else ""
        log(f"{lab:10s} {n:4d} launches  {ms * 1e3:9.2f} us each  {b / n / 1e6:9.2f} MB each  "
            f"{b / n / (ms * 1e-3) / 1e9:8.1f} GB/s{extra}")
    return out


def time_graph(be, launches, steps: int, warmup: int, use_graph: bool = True, rounds: int = 3):
    """Runs the launches once eagerly (sizes the scratch), records them as one graph, then after `warmup` untimed
    replays times `rounds` rounds of exactly `steps` replays each between HIP events on the backend's stream (the
    device synchronized before and after each). Returns the median round's ms per step."""
    def eager():
        for L in launches:
            L.fn()

    eager()
    be.sync()
    graph = None
    if use_graph:
        be.graph_begin()
        eager()
        graph = be.graph_end()
        log(f"step graph: {len(launches)} launches recorded as {be.graph_nodes(graph)} kernel nodes")
    step = (lambda: be.graph_launch(graph)) if graph else eager
    for _ in range(warmup):
        step()
    be.sync()
    e0, e1 = be.event(), be.event()
    per = []
    for r in range(rounds):
        be.sync()
        t0 = time.perf_counter()
        be.record(e0)
        for _ in range(steps):
            step()
        be.record(e1)
        be.sync()
        wall = time.perf_counter() - t0
        ms = be.elapsed_ms(e0, e1)
        per.append(ms / steps)
        log(f"round {r + 1}: timed {steps} steps: {ms:.2f} ms by events, {wall * 1e3:.2f} ms by wall clock")
    be.event_free(e0)
    be.event_free(e1)
    if graph:
        be.graph_free(graph)
    return sorted(per)[len(per) // 2]


def hbm_roofline(kernel, table, labels):
    """Algorithmic bytes per launch over the labels' mean launch time."""
    n = sum(table[l][0] for l in labels)
    b = sum(table[l][1] for l in labels)
    ms = sum(table[l][3] * table[l][0] for l in labels)
    achieved = (b / n) / (ms / n * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "launches_per_step": n, "bytes_per_launch": int(b / n),
            "us_per_launch": round(ms / n * 1e3, 3)}


def step_hbm_roofline(kernel, launches, ms_step, ms_other=0.0):
    """Algorithmic bytes per launch of `launches` over their mean duration inside the timed step: the step's time less
    `ms_other` (the step's other kernels) split over the launches. The step streams more weights than the 256 MB
    last-level cache holds, so no launch finds its weights there, and the gaps between kernels in the graph count as
    part of each launch."""
    n = len(launches)
    b = sum(L.nbytes for L in launches)
    ms = (ms_step - ms_other) / n
    achieved = (b / n) / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": kernel, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "launches_per_step": n, "bytes_per_launch": int(b / n),
            "us_per_launch": round(ms * 1e3, 3)}


def mfma_roofline(kernel, table, labels, peak=INT8_PEAK_TOPS, unit="TOP/s"):
    """Algorithmic multiply-adds x 2 per launch over the labels' mean launch time, against the dense MFMA peak of the
    arithmetic the kernel issues (int8 for the Q8_K/Q8_1 GEMMs, fp16 for the dequantizing Q8_0 GEMM)."""
    n = sum(table[l][0] for l in labels)
    ops = sum(table[l][2] for l in labels)
    ms = sum(table[l][3] * table[l][0] for l in labels)
    achieved = ops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": kernel, "achieved": round(achieved, 1), "peak": peak,
            "unit": unit, "frac": round(achieved / peak, 4), "launches_per_step": n,
            "ops_per_launch": int(ops / n), "us_per_launch": round(ms / n * 1e3, 3)}


def base_result(args, value, unit, ms_per_step, dtype, config, higher=True):
    return {"metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms_per_step, 5), "higher_is_better": higher, "scaling": "weak", "vs_baseline": None,
            "dtype": dtype, "data": "synthetic (seeded N(0,0.02) weights quantized by ggml's reference quantizers; "
                                    "N(0,1) activations)", "config": config}


def host_info():
    """The host the CPU baseline ran on: what lscpu and nproc report, the cores the port used, and the instruction set
    of its Q8_0 dot."""
    info = {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        keep = ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "NUMA node(s)", "CPU max MHz",
                "L3 cache")
        info["lscpu"] = {k.strip(): v.strip() for k, v in (l.split(":", 1) for l in out.splitlines() if ":" in l)
                         if k.strip() in keep}
        flags = next((l.split(":", 1)[1].split() for l in out.splitlines() if l.startswith("Flags")), [])
        info["avx2"], info["avx512_vnni"] = "avx2" in flags, "avx512_vnni" in flags
    except (OSError, subprocess.SubprocessError, StopIteration):
        info["lscpu"] = None
    O = load_oracle()
    info["physical_cores"] = O.physical_cores()
    info["q8_0_dot"] = {2: "AVX512-VNNI vpdpbusd", 1: "AVX2 maddubs"}[O.fast().cpf_q8_0_isa()]
    return info


def cpu_result(many, one):
    """A CPU baseline measured on the physical cores (`many`) with its one-thread twin (`one`) and the host."""
    out = dict(many)
    out["value_1thread"], out["sample_1thread"] = one["value"], one["sample"]
    out["host"] = host_info()
    return out


def timed_sample(fn, seconds: float, rounds: int = 3):
    """Runs fn once untimed, then in `rounds` timed rounds of about seconds / rounds each; returns (runs, elapsed s) of
    the round with the median rate (every round's rate is logged)."""
    fn()
    out = []
    for _ in range(rounds):
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds / rounds:
                break
        out.append((n / el, n, el))
    out.sort()
    log("cpu sample rounds: " + ", ".join(f"{r:.4g}/s" for r, _, _ in out) + " (median reported)")
    _, n, el = out[len(out) // 2]
    return n, el


# ---------------------------------------------------------------------------------------------- decoder shapes
def decoder_shapes(hidden, ffn, nq, nkv, head_dim):
    """(name, K, N) of one layer's linears, ggml order: W [K, N]."""
    q, kv = nq * head_dim, nkv * head_dim
    return [("q", hidden, q), ("k", hidden, kv), ("v", hidden, kv), ("o", q, hidden), ("gate", hidden, ffn),
            ("up", hidden, ffn), ("down", ffn, hidden)]


class Decoder:
    """A decoder's linears on the device, built from seeded synthetic weights: per layer q, k, v, o, gate, up, down,
    plus the tied embedding / lm_head table."""

    def __init__(self, mx, be, config, layers, hidden, ffn, nq, nkv, head_dim, vocab, types, threads, keep_host):
        self.mx, self.be = mx, be
        self.layers_n, self.hidden, self.ffn, self.vocab = layers, hidden, ffn, vocab
        self.shapes = decoder_shapes(hidden, ffn, nq, nkv, head_dim)
        self.types = types  # name -> weight type
        t0 = time.time()
        self.host = {}
        self.layers = []
        for l in range(layers):
            ws = {}
            for i, (name, K, N) in enumerate(self.shapes):
                t = types[name]
                q = mx.quantize_normal(t, weight_seed(config, l, i), N, K, 0.02, nthreads=threads)
                ws[name] = be.tensor(t, (K, N), q)
                if keep_host:
                    self.host[(l, name)] = q
            self.layers.append(ws)
        self.embd = None
        if vocab:
            head = mx.quantize_normal(Q8_0, weight_seed(config, layers, 0), vocab, hidden, 0.02, nthreads=threads)
            self.embd = be.tensor(Q8_0, (hidden, vocab), head)
            if keep_host:
                self.host["embd"] = head
        log(f"weights generated and uploaded in {time.time() - t0:.1f} s")

    def wbytes(self, l, names):
        return sum(row_bytes(self.layers[l][n].type, self.layers[l][n].ne[0]) * self.layers[l][n].ne[1] for n in names)

    def layer_bytes(self):
        return sum(self.wbytes(l, [n for n, _, _ in self.shapes]) for l in range(self.layers_n))

    def head_bytes(self):
        return row_bytes(Q8_0, self.hidden) * self.vocab if self.vocab else 0


class DecodeActs:
    """Per-layer synthetic activations and outputs of a batch-`M` pass (distinct tensors per layer when
    `per_layer`, else one set shared by every layer)."""

    def __init__(self, mx, be, dec, M, seed, per_layer):
        q_dim = [K for n, K, _ in dec.shapes if n == "o"][0]
        self.M = M
        sets = dec.layers_n if per_layer else 1
        self.acts, self.outs = [], []
        for l in range(sets):
            a = {}
            for j, (name, K) in enumerate([("attn_out", q_dim), ("ffn_in", dec.hidden), ("ffn_act", dec.ffn),
                                           ("final", dec.hidden)]):
                a[name] = be.tensor(mx.F32, (K, M), mx.fill_normal(seed + 16 * l + j, M, K))
            self.acts.append(a)
            self.outs.append({name: be.tensor(mx.F32, (N, M)) for name, K, N in dec.shapes})
        self.per_layer = per_layer

    def at(self, l):
        i = l if self.per_layer else 0
        return self.acts[i], self.outs[i]


def layer_launches(be, dec, acts, l, x_in, label_of):
    """One layer's products as four launches: q/k/v (shared input), attn_o, gate/up (shared input), down."""
    w = dec.layers[l]
    a, o = acts.at(l)
    M = acts.M
    x_in = a["final"] if x_in is None else x_in
    out = []

    def mk(label, names, x, K):
        b = dec.wbytes(l, names)
        N = sum(w[n].ne[1] for n in names)
        ops = 2 * M * K * N if M > 1 else 0
        nbytes = b + 4 * M * (K + N)
        if len(names) == 1:
            fn = lambda: be.mul_mat(w[names[0]], x, o[names[0]])  # noqa: E731
        else:
            fn = lambda: be.mul_mat_group([w[n] for n in names], x, [o[n] for n in names])  # noqa: E731
        out.append(Launch(label_of(label, w[names[0]].type), nbytes, ops, fn, weight_bytes=b))

    mk("qkv", ["q", "k", "v"], x_in, dec.hidden)
    mk("attn_o", ["o"], a["attn_out"], w["o"].ne[0])
    mk("gate_up", ["gate", "up"], a["ffn_in"], dec.hidden)
    mk("down", ["down"], a["ffn_act"], dec.ffn)
    return out


# ---------------------------------------------------------------------------------------------- decode (default)
QWEN3_06B = dict(layers=28, hidden=1024, ffn=3072, nq=16, nkv=8, head_dim=128, vocab=151936)
COPY_BYTES = 256 << 20  # the plain copy the counters are calibrated on
# HBM traffic per launch of each workload's dominant kernel, from two rocprofv3 --pmc passes over the workload
# (FETCH_SIZE, then WRITE_SIZE), summarized by --summarize-pmc: workload -> (summary file, kernel name substring)
TRAFFIC = {"decode": ("k_matvec_q8_0_qwen3-0.6b_decode.traffic.txt", "k_matvec"),
           "matvec": ("k_matvec_q8_0_3072x1024_rotated.traffic.txt", "k_matvec"),
           "prefill-q4k": ("k_gemm_q4k_qwen3-1.7b_prefill.traffic.txt", "k_gemm_q4k<"),
           "asr-1.7b": ("k_gemm_q8_0_i8_qwen3-asr-1.7b_prefill.traffic.txt", "k_gemm_q8_0_i8<"),
           "moe": ("k_mmid_q4k_drama3_moe.traffic.txt", "k_mmid_q4k")}


def calibration_copy(mx, be):
    """A plain device copy of known size: the reference the HBM traffic counters are calibrated on."""
    cp_src, cp_dst = be.tensor(mx.F32, (COPY_BYTES // 4,)), be.tensor(mx.F32, (COPY_BYTES // 4,))
    mx.check(mx.lib().mx_tensor_copy(be.h, cp_src.ref(), cp_dst.ref()))
    be.sync()
    cp_src.free()
    cp_dst.free()


def decode_token_launches(be, mx, dec, acts, ids, x0, logits):
    L = [Launch("get_rows", row_bytes(Q8_0, dec.hidden) + 4 + 4 * dec.hidden, 0,
                lambda: be.get_rows(dec.embd, ids, x0))]
    for l in range(dec.layers_n):
        L += layer_launches(be, dec, acts, l, x0 if l == 0 else None, lambda lab, t: lab)
    final = acts.at(dec.layers_n - 1)[0]["final"]
    L.append(Launch("lm_head", dec.head_bytes() + 4 * (dec.hidden + dec.vocab), 0,
                    lambda: be.mul_mat(dec.embd, final, logits), weight_bytes=dec.head_bytes()))
    return L


def run_decode(args, mx, be, threads):
    S = QWEN3_06B
    dec = Decoder(mx, be, 2, S["layers"], S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"], S["vocab"],
                  {n: Q8_0 for n, _, _ in decoder_shapes(S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"])},
                  threads, keep_host=True)
    acts = DecodeActs(mx, be, dec, 1, 0xAC700002, per_layer=True)
    ids = be.tensor(mx.I32, (1,), np.array([4242], np.int32))
    x0 = be.tensor(mx.F32, (S["hidden"], 1))
    logits = be.tensor(mx.F32, (S["vocab"], 1))
    launches = decode_token_launches(be, mx, dec, acts, ids, x0, logits)
    weight_bytes = sum(L.weight_bytes for L in launches)

    ms_per_step = time_graph(be, launches, args.steps, args.warmup, not args.no_graph)
    # Roofline of the dominant kernel: k_matvec over Q8_0 at batch 1 (every launch of the step but the one GET_ROWS;
    # the template is instantiated per lanes-per-row, all the same code), timed inside the step.
    table = label_table(launches, per_label_pass(be, launches, reps=20, use_graph=not args.no_graph))
    roof = step_hbm_roofline("k_matvec<Q8_0, NC=1>", [L for L in launches if L.label != "get_rows"], ms_per_step,
                             ms_other=table["get_rows"][3])
    roof["traffic"] = read_traffic("decode")
    tok_s = 1e3 / ms_per_step
    step_gbps = weight_bytes / (ms_per_step * 1e-3) / 1e9
    result = base_result(args, round(tok_s, 2), "tok/s", ms_per_step, "int8", {
        "workload": "qwen3-0.6b-shape decode step, batch 1", **S, "weights": "Q8_0",
        "ops_per_step": "1 GET_ROWS + 197 MUL_MAT in 114 launches", "graph": not args.no_graph})
    result.update({"weight_bytes_per_step": weight_bytes, "weight_GBps": round(step_gbps, 1),
                   "hbm_frac_step": round(step_gbps / HBM_PEAK_GBPS, 4), "roofline": roof})
    if args.full_step:
        result.update(decode_full_extra(args, mx, be, dec))
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_result(cpu_decode(dec, args.cpu_seconds),
                                            cpu_decode(dec, args.cpu_seconds / 3, threads=1))
    return result


def decode_full_extra(args, mx, be, dec):
    """The whole decode step on the same weights (every op on the device, fused, KV cache at KV_PAST positions), timed
    as the decode-full workload times it: its tokens per second beside the products-only step."""
    S = QWEN3_06B
    st = full_step_state(mx, be, dec, S["nq"], S["nkv"], S["head_dim"], 1)
    ids = be.tensor(mx.I32, (1,), np.array([4242], np.int32))
    launches = full_step_launches(be, mx, dec, st, ids, S["nq"], S["nkv"], S["head_dim"], fused=True)
    steps, warmup = DEFAULT_STEPS["decode-full"]
    ms = time_graph(be, launches, steps, warmup, not args.no_graph)
    return {"decode_full_tok_s": round(1e3 / ms, 2), "decode_full_ms_per_token": round(ms, 5),
            "decode_full_launches": len(launches)}


def cpu_decode(dec, seconds, threads=None):
    """The oracle's multi-threaded port of ggml's CPU mul_mat on the same weights, one token at a time."""
    O = load_oracle()
    threads = threads or O.physical_cores()
    x = {K: O.fill_normal(0xAC700002 + K, 1, K) for K in {K for _, K, _ in dec.shapes}}

    def token():
        O.get_rows(O.TYPE_Q8_0, dec.host["embd"][4242:4243], dec.hidden, np.array([0], np.int32))
        for l in range(dec.layers_n):
            for name, K, N in dec.shapes:
                O.cpu_fast_mul_mat(dec.types[name], dec.host[(l, name)], x[K], threads)
        O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host["embd"], x[dec.hidden], threads)

    n, el = timed_sample(token, seconds)
    return {"value": round(n / el, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} full decode tokens (1 GET_ROWS + 197 Q8_0 mat-vecs, 633 MB of weights each) after one "
                      f"untimed token, {el:.1f} s (the median of three rounds), int8 dots, src1 quantized once per product, rows split "
                      f"across {threads} threads"}


def summarize_pmc(fetch_csv: str, write_csv: str, kernel: str) -> str:
    """Per-dispatch HBM traffic of the kernels whose name holds `kernel`, from two rocprofv3 --pmc runs (FETCH_SIZE,
    then WRITE_SIZE, KiB per dispatch), each scaled by what the counter reads for the run's plain 256 MiB device
    copy."""
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
    mv = [k for k in f if kernel in k]
    fetch = [v for k in mv for v in f[k]]
    write = [v for k in mv for v in w.get(k, [])]
    fb = statistics.mean(fetch) * 1024 / f_cal
    wb = statistics.mean(write) * 1024 / w_cal if write else 0.0
    lines = [f"kernels matching '{kernel}': {len(fetch)} dispatches",
             f"copy calibration: FETCH_SIZE reads {f_cal:.4f} x and WRITE_SIZE {w_cal:.4f} x the bytes of a "
             f"{COPY_BYTES >> 20} MiB device copy",
             f"fetch_bytes_per_launch: {fb:.0f}", f"write_bytes_per_launch: {wb:.0f}",
             f"traffic_bytes_per_launch: {fb + wb:.0f}"]
    return "\n".join(lines)


def summarize_busy(csv_path: str, kernel: str, clock_mhz: float) -> str:
    """Per-dispatch time of the kernels whose name holds `kernel`, from one rocprofv3 --pmc GRBM_GUI_ACTIVE run, two
    ways: the dispatch's own start and end timestamps, and its GPU-busy clock cycles (counted over the dispatch, summed
    over the 8 XCDs) at the shader clock. Both carry the profiler's per-dispatch cost; the one-workgroup GET_ROWS of
    the same run (1 KB read) measures that floor, and the 512 MB cache-flush reads (k_peak_read) check the cycle
    scale against their known duration."""
    import csv
    import statistics
    busy, span = {}, {}
    for r in csv.DictReader(open(csv_path)):
        if r["Counter_Name"] != "GRBM_GUI_ACTIVE":
            continue
        busy.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]) / 8 / clock_mhz)
        span.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    med = statistics.median
    lines = [f"per dispatch, us: timestamps (end - start) and GRBM_GUI_ACTIVE / 8 XCDs / {clock_mhz:.0f} MHz"]
    floor = [name for name in busy if "k_get_rows" in name]
    for name in sorted(busy):
        if kernel in name or "k_peak_read" in name or "k_get_rows" in name:
            lines.append(f"{name[:56]:56s} dispatches {len(busy[name]):5d}  timestamps median {med(span[name]):8.3f}"
                         f"  busy median {med(busy[name]):8.3f}")
    mv_span = [v for name in span if kernel in name for v in span[name]]
    mv_busy = [v for name in busy if kernel in name for v in busy[name]]
    lines.append(f"{kernel}: {len(mv_span)} dispatches, timestamps mean {statistics.mean(mv_span):.3f} us, "
                 f"busy mean {statistics.mean(mv_busy):.3f} us")
    if floor:
        fs = med([v for name in floor for v in span[name]])
        fb = med([v for name in floor for v in busy[name]])
        lines.append(f"one-workgroup floor (k_get_rows): timestamps {fs:.3f} us, busy {fb:.3f} us")
        lines.append(f"{kernel} above the floor: timestamps {statistics.mean(mv_span) - fs:.3f} us, "
                     f"busy {statistics.mean(mv_busy) - fb:.3f} us")
    return "\n".join(lines)


def read_traffic(workload):
    path = ROOT / "profiles" / TRAFFIC[workload][0]
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":")[1]))
    return None


# ---------------------------------------------------------------------------------------------- decode-full
KV_PAST = 1024       # the f16 KV cache is prefilled with N(0,1) values to 1024 positions; the new token is the 1025th
ATT_BLOCK = 64       # flash attention reads whole blocks of 64 positions (qwen3-decoder.cpp kAttentionBlock)
RMS_EPS, ROPE_THETA = 1e-6, 1e6


def full_step_launches(be, mx, dec, st, ids, nq, nkv, hd, fused=True):
    """The decode step's launches, in Qwen3Decoder::layers order (qwen3-decoder.cpp:350-412, outputs :422-438). Fused:
    norm + q/k/v, q/k norm + RoPE + KV stores + attention, attn_o + residual, norm + gate/up, SwiGLU + down + residual
    (each fusion computes what the separate ops compute); unfused: one launch per ggml node."""
    H, kv_dim, n_kv = dec.hidden, nkv * hd, st["n_kv"]
    L = []
    x, h, pos, mask = st["x"], st["h"], st["pos"], st["mask"]
    L.append(Launch("get_rows", row_bytes(Q8_0, H) + 4 + 4 * H, 0, lambda: be.get_rows(dec.embd, ids, x)))
    for l in range(dec.layers_n):
        w, nw, c = dec.layers[l], st["norms"][l], st["cache"][l]
        o = st["outs"]
        qv = o["q"].view((hd, nq, 1), (4, hd * 4, nq * hd * 4))
        kv = o["k"].view((hd, nkv, 1), (4, hd * 4, nkv * hd * 4))
        vv = o["v"].view((hd, nkv, 1), (4, hd * 4, nkv * hd * 4))
        qh = st["qr"].view((hd, 1, nq), (4, nq * hd * 4, hd * 4))
        kh = c["k"].view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2))
        vh = c["v"].view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2))
        kr_rows = st["kr"].view((kv_dim, 1), (4, kv_dim * 4))
        wq, wo, wg, wd = (dec.wbytes(l, n) for n in (["q", "k", "v"], ["o"], ["gate", "up"], ["down"]))
        attention = Launch("attention", 2 * 2 * (KV_PAST + 1) * kv_dim + 8 * nq * hd, 0,
                           lambda qh=qh, kh=kh, vh=vh: be.flash_attn_ext(qh, kh, vh, mask, st["att"], 1.0 / np.sqrt(hd)))
        if fused:
            L += [Launch("qkv", wq + 4 * (H + (nq + 2 * nkv) * hd), 0,
                         lambda w=w, nw=nw: be.mul_mat_fused([w["q"], w["k"], w["v"]], x, [o["q"], o["k"], o["v"]],
                                                             norm_w=nw["attn"], eps=RMS_EPS), weight_bytes=wq),
                  # q / k norms, RoPE and the KV stores ride in the attention launch (mx_attn_decode)
                  Launch("attention", attention.nbytes + 4 * (nq * hd + 2 * kv_dim) + 2 * 2 * kv_dim, 0,
                         lambda qv=qv, kv=kv, vv=vv, nw=nw, c=c, kh=kh, vh=vh: be.attn_decode(
                             qv, kv, vv, nw["q"], nw["k"], pos, c["k"], c["v"], kh, vh, mask, st["att"], RMS_EPS,
                             ROPE_THETA, 1.0 / np.sqrt(hd))),
                  Launch("attn_o", wo + 4 * (nq * hd + 2 * H), 0,
                         lambda w=w: be.mul_mat_fused([w["o"]], st["att_rows"], [x], residual=[x]), weight_bytes=wo),
                  Launch("gate_up", wg + 4 * (H + 2 * dec.ffn), 0,
                         lambda w=w, nw=nw: be.mul_mat_fused([w["gate"], w["up"]], x, [o["gate"], o["up"]],
                                                             norm_w=nw["ffn"], eps=RMS_EPS), weight_bytes=wg),
                  Launch("down", wd + 4 * (2 * dec.ffn + 2 * H), 0,
                         lambda w=w: be.mul_mat_fused([w["down"]], o["gate"], [x], glu_b=o["up"], residual=[x]),
                         weight_bytes=wd)]
            continue
        L += [Launch("norm", 8 * H, 0, lambda nw=nw: be.rms_norm(x, h, RMS_EPS, nw["attn"])),
              Launch("qkv", wq + 4 * (H + (nq + 2 * nkv) * hd), 0,
                     lambda w=w: be.mul_mat_group([w["q"], w["k"], w["v"]], h, [o["q"], o["k"], o["v"]]),
                     weight_bytes=wq),
              Launch("qk_norm", 8 * nq * hd, 0, lambda qv=qv, nw=nw: be.rms_norm(qv, st["qn"], RMS_EPS, nw["q"])),
              Launch("qk_norm", 8 * nkv * hd, 0, lambda kv=kv, nw=nw: be.rms_norm(kv, st["kn"], RMS_EPS, nw["k"])),
              Launch("set_rows", 6 * kv_dim, 0, lambda c=c: be.set_rows(o["v"], pos, c["v"])),
              Launch("rope", 8 * nq * hd, 0, lambda: be.rope(st["qn"], pos, st["qr"], hd, ROPE_THETA)),
              Launch("rope", 8 * nkv * hd, 0, lambda: be.rope(st["kn"], pos, st["kr"], hd, ROPE_THETA)),
              Launch("set_rows", 6 * kv_dim, 0, lambda c=c, kr_rows=kr_rows: be.set_rows(kr_rows, pos, c["k"])),
              attention,
              Launch("attn_o", wo + 4 * (nq * hd + H), 0,
                     lambda w=w: be.mul_mat(w["o"], st["att_rows"], o["o"]), weight_bytes=wo),
              Launch("add", 12 * H, 0, lambda: be.add(x, o["o"], x)),
              Launch("norm", 8 * H, 0, lambda nw=nw: be.rms_norm(x, h, RMS_EPS, nw["ffn"])),
              Launch("gate_up", wg + 4 * (H + 2 * dec.ffn), 0,
                     lambda w=w: be.mul_mat_group([w["gate"], w["up"]], h, [o["gate"], o["up"]]), weight_bytes=wg),
              Launch("swiglu", 12 * dec.ffn, 0, lambda: be.swiglu(o["gate"], o["up"], st["act"])),
              Launch("down", wd + 4 * (dec.ffn + H), 0,
                     lambda w=w: be.mul_mat(w["down"], st["act"], o["down"]), weight_bytes=wd),
              Launch("add", 12 * H, 0, lambda: be.add(x, o["down"], x))]
    # the head keeps its norm apart: fused, each of its 9,496 workgroups would redo the norm's reduction
    L += [Launch("norm", 8 * H, 0, lambda: be.rms_norm(x, h, RMS_EPS, st["final_norm"])),
          Launch("lm_head", dec.head_bytes() + 4 * (H + dec.vocab), 0,
                 lambda: be.mul_mat(dec.embd, h, st["logits"]), weight_bytes=dec.head_bytes())]
    L.append(Launch("argmax", 4 * dec.vocab + 4, 0, lambda: be.argmax(st["logits"], st["pick"])))
    return L


def full_step_state(mx, be, dec, nq, nkv, hd, threads):
    """Norm weights N(1, 0.1), the f16 KV caches (N(0,1) to KV_PAST positions), position and mask inputs, buffers."""
    H, kv_dim = dec.hidden, nkv * hd
    n_kv = (KV_PAST + 1 + ATT_BLOCK - 1) // ATT_BLOCK * ATT_BLOCK
    st = {"n_kv": n_kv, "norms": [], "cache": []}
    for l in range(dec.layers_n):
        st["norms"].append({n: be.tensor(mx.F32, (k,), mx.fill_normal(0x7077 + 16 * l + i, 1, k, 1.0, 0.1))
                            for i, (n, k) in enumerate([("attn", H), ("ffn", H), ("q", hd), ("k", hd)])})
        c = {}
        for j, n in enumerate(("k", "v")):
            vals = np.zeros((n_kv, kv_dim), np.float16)
            vals[:KV_PAST] = mx.fill_normal(0xCAC4E000 + 2 * l + j, KV_PAST, kv_dim).astype(np.float16)
            c[n] = be.tensor(mx.F16, (kv_dim, n_kv), vals.view(np.uint16))
        st["cache"].append(c)
    st["final_norm"] = be.tensor(mx.F32, (H,), mx.fill_normal(0x7077F, 1, H, 1.0, 0.1))
    st["x"], st["h"] = be.tensor(mx.F32, (H, 1)), be.tensor(mx.F32, (H, 1))
    st["outs"] = {n: be.tensor(mx.F32, (N, 1)) for n, _, N in dec.shapes}
    st["qn"], st["qr"] = be.tensor(mx.F32, (hd, nq, 1)), be.tensor(mx.F32, (hd, nq, 1))
    st["kn"], st["kr"] = be.tensor(mx.F32, (hd, nkv, 1)), be.tensor(mx.F32, (hd, nkv, 1))
    st["att"] = be.tensor(mx.F32, (hd, nq, 1))
    st["att_rows"] = st["att"].view((nq * hd, 1), (4, nq * hd * 4))
    st["act"] = be.tensor(mx.F32, (dec.ffn, 1))
    st["logits"], st["pick"] = be.tensor(mx.F32, (dec.vocab, 1)), be.tensor(mx.I32, (1,))
    st["pos"] = be.tensor(mx.I32, (1,), np.array([KV_PAST], np.int32))
    m = np.zeros(n_kv, np.float32)
    m[KV_PAST + 1:] = -np.inf
    st["mask"] = be.tensor(mx.F16, (n_kv, 1), m.astype(np.float16).view(np.uint16))
    return st


def run_decode_full(args, mx, be, threads):
    S = QWEN3_06B
    nq, nkv, hd = S["nq"], S["nkv"], S["head_dim"]
    dec = Decoder(mx, be, 2, S["layers"], S["hidden"], S["ffn"], nq, nkv, hd, S["vocab"],
                  {n: Q8_0 for n, _, _ in decoder_shapes(S["hidden"], S["ffn"], nq, nkv, hd)}, threads,
                  keep_host=args.cpu_seconds > 0)
    st = full_step_state(mx, be, dec, nq, nkv, hd, threads)
    ids = be.tensor(mx.I32, (1,), np.array([4242], np.int32))
    launches = full_step_launches(be, mx, dec, st, ids, nq, nkv, hd, fused=not args.unfused)
    weight_bytes = sum(L.weight_bytes for L in launches if L.label in ("qkv", "attn_o", "gate_up", "down", "lm_head"))
    kv_bytes = dec.layers_n * 2 * 2 * (KV_PAST + 1) * nkv * hd
    ms_per_step = time_graph(be, launches, args.steps, args.warmup, not args.no_graph)
    table = label_table(launches, per_label_pass(be, launches, reps=10, use_graph=not args.no_graph))
    tok_s = 1e3 / ms_per_step
    mv = [L for L in launches if L.label in ("qkv", "attn_o", "gate_up", "down", "lm_head")]
    ms_mv = sum(table[lab][3] * table[lab][0] for lab in ("qkv", "attn_o", "gate_up", "down", "lm_head"))
    roof = hbm_roofline("k_matvec<Q8_0, NC=1>", table, ["qkv", "attn_o", "gate_up", "down", "lm_head"])
    roof["traffic"] = read_traffic("decode")
    att = hbm_roofline("k_fa_gqa<2> + k_fa_merge<128>", table, ["attention"])
    result = base_result(args, round(tok_s, 2), "tok/s", ms_per_step, "int8", {
        "workload": "qwen3-0.6b-shape decode step, batch 1, every op on the device, KV cache at 1024 positions",
        **S, "weights": "Q8_0", "kv_cache": "f16", "kv_past": KV_PAST, "kv_read": st["n_kv"],
        "launches_per_step": len(launches), "fused": not args.unfused, "graph": not args.no_graph})
    result.update({"weight_bytes_per_step": weight_bytes, "kv_bytes_per_step": kv_bytes,
                   "GBps_step": round((weight_bytes + kv_bytes) / (ms_per_step * 1e-3) / 1e9, 1),
                   "hbm_frac_step": round((weight_bytes + kv_bytes) / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                   "matvec_ms_per_step": round(ms_mv, 4), "roofline": roof, "attention_roofline": att})
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_result(cpu_decode_full(dec, st, args.cpu_seconds, nq, nkv, hd),
                                            cpu_decode_full(dec, st, args.cpu_seconds / 3, nq, nkv, hd, threads=1))
    return result


def cpu_decode_full(dec, st, seconds, nq, nkv, hd, threads=None):
    """The full step on the host: the port's mat-vecs and flash attention (ggml-cpu's loop, its (row, head) pairs over
    the threads) on the physical cores, the oracle's norms, RoPE and SwiGLU over the step's small vectors on one
    thread, over host copies of the same weights and caches."""
    O = load_oracle()
    threads = threads or O.physical_cores()
    H, n_kv, kv_dim = dec.hidden, st["n_kv"], nkv * hd
    # host caches as the oracle's attention reads them: [kv head, position, channel]
    caches = [{n: np.ascontiguousarray(np.frombuffer(c[n].get_bytes().tobytes(), np.uint16)
                                       .reshape(n_kv, nkv, hd).transpose(1, 0, 2)) for n in ("k", "v")}
              for c in st["cache"]]
    norms = [{n: t.numpy().reshape(-1) for n, t in nw.items()} for nw in st["norms"]]
    fin = st["final_norm"].numpy().reshape(-1)
    mask = np.zeros((1, n_kv), np.float32)
    mask[0, KV_PAST + 1:] = -np.inf
    mask = mask.astype(np.float16).view(np.uint16)
    pos = np.array([KV_PAST], np.int32)

    def token():
        x = O.get_rows(O.TYPE_Q8_0, dec.host["embd"][4242:4243], H, np.array([0], np.int32))
        for l in range(dec.layers_n):
            hv = O.binary("mul", O.rms_norm(x, RMS_EPS), norms[l]["attn"])
            q, k, v = (O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host[(l, n)], hv, threads) for n in ("q", "k", "v"))
            q = O.binary("mul", O.rms_norm(q.reshape(1, nq, hd), RMS_EPS), norms[l]["q"])
            k = O.binary("mul", O.rms_norm(k.reshape(1, nkv, hd), RMS_EPS), norms[l]["k"])
            q, k = O.rope_neox(q, pos, hd, ROPE_THETA), O.rope_neox(k, pos, hd, ROPE_THETA)
            # SET_ROWS: the new position's keys and values into the f16 caches
            caches[l]["k"][:, KV_PAST] = k.reshape(nkv, hd).astype(np.float16).view(np.uint16)
            caches[l]["v"][:, KV_PAST] = v.reshape(nkv, hd).astype(np.float16).view(np.uint16)
            att = O.cpu_fast_flash_attn_ext(q.transpose(1, 0, 2), caches[l]["k"], caches[l]["v"], mask,
                                            1.0 / np.sqrt(hd), threads)
            x = O.binary("add", x, O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host[(l, "o")], att.reshape(1, -1), threads))
            hv = O.binary("mul", O.rms_norm(x, RMS_EPS), norms[l]["ffn"])
            g, u = (O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host[(l, n)], hv, threads) for n in ("gate", "up"))
            x = O.binary("add", x, O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host[(l, "down")], O.swiglu(g, u), threads))
        hv = O.binary("mul", O.rms_norm(x, RMS_EPS), fin)
        return O.argmax(O.cpu_fast_mul_mat(O.TYPE_Q8_0, dec.host["embd"], hv, threads))

    n, el = timed_sample(token, seconds)
    return {"value": round(n / el, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{n} full decode tokens after one untimed token, {el:.1f} s (the median of three rounds): "
                      f"mat-vecs and flash attention (ggml-cpu's loop over 1025 positions, F16C, its (row, head) "
                      f"pairs split across threads) in the port on {threads} threads; norms / RoPE / SET_ROWS / "
                      f"SwiGLU over 1-4 KB vectors in the oracle on one thread"}


# ---------------------------------------------------------------------------------------------- matvec
MATVEC_COPIES = 160  # 160 x 3,342,336 B = 535 MB of distinct weight copies, larger than the 256 MB last-level cache


def run_matvec(args, mx, be, threads):
    K, N = 1024, 3072
    w = mx.quantize_normal(Q8_0, weight_seed(1, 0, 0), N, K, 0.02, nthreads=threads)
    x = mx.fill_normal(0xAC700001, 1, K)
    W = [be.tensor(Q8_0, (K, N), w) for _ in range(MATVEC_COPIES)]
    X = be.tensor(mx.F32, (K, 1), x)
    Y = be.tensor(mx.F32, (N, 1))
    nbytes = row_bytes(Q8_0, K) * N + 4 * K + 4 * N
    launches = [Launch("matvec", nbytes, 0, lambda Wi=Wi: be.mul_mat(Wi, X, Y)) for Wi in W]
    ms_per_step = time_graph(be, launches, args.steps, args.warmup, not args.no_graph)
    roof = step_hbm_roofline("k_matvec<Q8_0, NC=1>", launches, ms_per_step)
    roof["traffic"] = read_traffic("matvec")
    gbps = nbytes * MATVEC_COPIES / (ms_per_step * 1e-3) / 1e9
    result = base_result(args, round(gbps, 1), "GB/s", ms_per_step, "int8", {
        "workload": "single Q8_0 MUL_MAT 3072x1024 at batch 1, rotated over 160 weight copies",
        "K": K, "N": N, "copies": MATVEC_COPIES, "bytes_per_product": nbytes, "graph": not args.no_graph})
    result.update({"hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "us_per_product":
                   round(ms_per_step / MATVEC_COPIES * 1e3, 3), "roofline": roof})
    if args.cpu_seconds > 0:
        O = load_oracle()
        cores = O.physical_cores()
        host = np.ascontiguousarray(np.broadcast_to(w, (MATVEC_COPIES,) + w.shape))
        i = [0]

        runs = []
        for c, sec in ((cores, args.cpu_seconds), (1, args.cpu_seconds / 3)):
            cores_now = c

            def one_c(c=cores_now):
                O.cpu_fast_mul_mat(O.TYPE_Q8_0, host[i[0] % MATVEC_COPIES], x, c)
                i[0] += 1
            n, el = timed_sample(one_c, sec)
            runs.append({"value": round(n * nbytes / el / 1e9, 2), "unit": "GB/s", "cores": c, "kind": "port",
                         "sample": f"{n} products over {MATVEC_COPIES} rotated host copies, {el:.1f} s (the median of three rounds), {c} threads"})
        result["cpu_baseline"] = cpu_result(runs[0], runs[1])
    return result


# ---------------------------------------------------------------------------------------------- prefill
QWEN3_17B = dict(layers=28, hidden=2048, ffn=6144, nq=16, nkv=8, head_dim=128)


def prefill_launches(be, dec, acts, label_of):
    L = []
    for l in range(dec.layers_n):
        L += layer_launches(be, dec, acts, l, None, label_of)
    return L


def cpu_prefill(dec, M, seconds, types, cores=None):
    """The port of ggml's CPU mul_mat on the same weights at M rows, layer by layer, bounded by `seconds`."""
    O = load_oracle()
    cores = cores or O.physical_cores()
    x = {K: O.fill_normal(0xAC700300 + K, M, K) for K in {K for _, K, _ in dec.shapes}}
    ops_per_layer = sum(2 * M * K * N for _, K, N in dec.shapes)
    state = {"l": 0}

    def layer():
        l = state["l"] % dec.layers_n
        for name, K, N in dec.shapes:
            O.cpu_fast_mul_mat(types[name], dec.host[(l, name)], x[K], cores)
        state["l"] += 1

    n, el = timed_sample(layer, seconds)
    return {"value": round(ops_per_layer * n / el / 1e12, 4), "unit": "TOP/s", "cores": cores, "kind": "port",
            "sample": f"{n} layers' 7 products at M = {M} after one untimed layer, {el:.1f} s (the median of three "
                      f"rounds), int8 dots, {cores} threads"}


def run_prefill_q4k(args, mx, be, threads):
    S = QWEN3_17B
    M = 512
    types = {n: (Q6_K if n == "down" else Q4_K) for n, _, _ in
             decoder_shapes(S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"])}
    dec = Decoder(mx, be, 3, S["layers"], S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"], 0, types, threads,
                  keep_host=args.cpu_seconds > 0)
    acts = DecodeActs(mx, be, dec, M, 0xAC700003, per_layer=False)
    launches = prefill_launches(be, dec, acts, lambda lab, t: f"{lab}:{NAME[t]}")
    ops = sum(L.ops for L in launches)
    ms_per_step = time_graph(be, launches, args.steps, args.warmup, not args.no_graph)
    table = label_table(launches, per_label_pass(be, launches, reps=5, use_graph=not args.no_graph))
    roof = mfma_roofline("k_gemm_q4k (with its Q8_K activation pass)", table,
                         [l for l in table if l.endswith(":Q4_K")])
    roof["traffic"] = read_traffic("prefill-q4k")
    tops = ops / (ms_per_step * 1e-3) / 1e12
    result = base_result(args, round(tops, 2), "TOP/s", ms_per_step, "int8", {
        "workload": "qwen3-1.7b-shape talker prefill, M = 512", **S, "M": M, "weights": "Q4_K, Q6_K down",
        "graph": not args.no_graph})
    wb = dec.layer_bytes()
    result.update({"int8_frac": round(tops / INT8_PEAK_TOPS, 4), "ops_per_step": ops, "weight_bytes": wb,
                   "tok_s": round(M / (ms_per_step * 1e-3), 1), "roofline": roof,
                   "q6_k_down": (mfma_roofline("k_gemm_dq<Q6_K> (with its Q8_K activation pass)", table, ["down:Q6_K"],
                                               FP16_PEAK_TFLOPS, "TFLOP/s")
                                 if be.get_option("gemm_kquant") == 0 else
                                 mfma_roofline("k_gemm_kq<Q6_K>", table, ["down:Q6_K"]))})
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_result(cpu_prefill(dec, M, args.cpu_seconds, types),
                                            cpu_prefill(dec, M, args.cpu_seconds / 3, types, cores=1))
    return result


ASR_BLOCKS = (512, 512, 512, 28)   # 1500 audio rows + 64 text rows, in speech.cpp's 512-row prefill blocks
ASR_DECODE_TOKENS = 32


def run_asr(args, mx, be, threads):
    S = dict(QWEN3_17B, vocab=151936)
    types = {n: Q8_0 for n, _, _ in decoder_shapes(S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"])}
    dec = Decoder(mx, be, 4, S["layers"], S["hidden"], S["ffn"], S["nq"], S["nkv"], S["head_dim"], S["vocab"], types,
                  threads, keep_host=args.cpu_seconds > 0)
    blocks = tuple(args.blocks or ASR_BLOCKS)
    acts = {M: DecodeActs(mx, be, dec, M, 0xAC700004 + M * 256, per_layer=False) for M in sorted(set(blocks))}
    dacts = DecodeActs(mx, be, dec, 1, 0xAC700004, per_layer=True)
    logits = be.tensor(mx.F32, (S["vocab"], 1))
    ids = be.tensor(mx.I32, (1,), np.array([4242], np.int32))
    x0 = be.tensor(mx.F32, (S["hidden"], 1))
    pre = []
    for M in blocks:
        pre += prefill_launches(be, dec, acts[M], lambda lab, t, M=M: f"prefill_M{M}")
    last = acts[blocks[-1]].acts[0]["final"]
    head_x = be.tensor(mx.F32, (S["hidden"], 1), last.numpy().reshape(blocks[-1], S["hidden"])[-1:])
    pre.append(Launch("head_last_row", dec.head_bytes(), 0, lambda: be.mul_mat(dec.embd, head_x, logits)))
    tok = decode_token_launches(be, mx, dec, dacts, ids, x0, logits)
    pre_ops = sum(L.ops for L in pre)
    ms_pre = time_graph(be, pre, max(1, args.steps), args.warmup, not args.no_graph)
    ms_tok = time_graph(be, tok, max(1, args.steps) * ASR_DECODE_TOKENS, args.warmup, not args.no_graph)
    ms_step = ms_pre + ASR_DECODE_TOKENS * ms_tok
    table = label_table(pre + tok, per_label_pass(be, pre + tok, reps=3, use_graph=not args.no_graph))
    # the prefill GEMM multiplies Q8_0 weights and Q8_0-quantized activations on int8 MFMA, block by block (--opt
    # gemm_q8_0=2 selects the fp16 dequantizing GEMM instead); the decode mat-vecs use int8 dot products
    dq = be.get_option("gemm_q8_0") == 2
    big = [l for l in table if l == f"prefill_M{max(blocks)}"]  # the largest block's products (512 rows as run)
    roof = (mfma_roofline("k_gemm_dq<Q8_0> (with its activation pass)", table, big, FP16_PEAK_TFLOPS, "TFLOP/s")
            if dq else mfma_roofline("k_gemm_q8_0_i8 (with its activation pass)", table, big))
    roof["traffic"] = read_traffic("asr-1.7b") if not dq and max(blocks) == 512 else None  # measured on 512-row blocks
    tops = pre_ops / (ms_pre * 1e-3) / 1e12
    tok_w = sum(L.weight_bytes for L in tok)
    result = base_result(args, round(tops, 2), "TOP/s", ms_step, "fp16" if dq else "int8", {
        "workload": "qwen3-asr-1.7b-shape Q8_0 prefill of 1564 rows + 32 decode tokens", **S,
        "blocks": list(blocks), "decode_tokens": ASR_DECODE_TOKENS, "weights": "Q8_0", "graph": not args.no_graph})
    result.update({"mfma_frac": round(tops / (FP16_PEAK_TFLOPS if dq else INT8_PEAK_TOPS), 4),
                   "decode_dtype": "int8", "prefill_ms": round(ms_pre, 4),
                   "prefill_ops": pre_ops, "decode_ms_per_token": round(ms_tok, 5),
                   "decode_tok_s": round(1e3 / ms_tok, 2), "decode_weight_bytes_per_token": tok_w,
                   "decode_hbm_frac": round(tok_w / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "roofline": roof,
                   "decode_roofline": step_hbm_roofline("k_matvec<Q8_0, NC=1>",
                                                        [L for L in tok if L.label != "get_rows"], ms_tok,
                                                        ms_other=table["get_rows"][3])})
    if args.cpu_seconds > 0:
        result["cpu_baseline"] = cpu_result(cpu_prefill(dec, 512, args.cpu_seconds, types),
                                            cpu_prefill(dec, 512, args.cpu_seconds / 3, types, cores=1))
    return result


# ---------------------------------------------------------------------------------------------- moe
MOE_E, MOE_K, MOE_H, MOE_F = 64, 4, 2048, 1536
MOE_BATCHES = (1, 16, 256)
MOE_LAYERS = 16  # distinct copies of the expert tensors: 5.4 GB, so no layer finds its experts in the 256 MB cache


def router_ids(T, seed):
    """top-4 of softmax(N(0,1) logits) per token (softmax is monotone, so the top-4 of the logits)."""
    mx = load_mx()
    logits = mx.fill_normal(seed, T, MOE_E).astype(np.float64)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return np.argsort(-p, axis=1, kind="stable")[:, :MOE_K].astype(np.int32)


def run_moe(args, mx, be, threads):
    t0 = time.time()
    WT = TYPE_OF[args.moe_weights]  # Q4_K as the configuration names it; the other types measure their own paths
    specs = [("gate", MOE_H, MOE_F), ("up", MOE_H, MOE_F), ("down", MOE_F, MOE_H)]
    host = {}
    for i, (name, K, N) in enumerate(specs):
        host[name] = mx.quantize_normal(WT, weight_seed(5, 0, i), MOE_E * N, K, 0.02, nthreads=threads)
    layers = [{name: be.tensor(WT, (K, N, MOE_E), host[name]) for name, K, N in specs} for _ in range(MOE_LAYERS)]
    log(f"expert weights generated and uploaded ({MOE_LAYERS} layer copies) in {time.time() - t0:.1f} s")
    per_expert = sum(row_bytes(WT, K) * N for _, K, N in specs)
    per_batch, all_launches, ms_total = [], [], 0.0
    for T in args.batches or MOE_BATCHES:
        launches, wbytes, distinct = [], 0, []
        xb = be.tensor(mx.F32, (MOE_H, 1, T), mx.fill_normal(0xAC700005 + T, T, MOE_H))
        xa = be.tensor(mx.F32, (MOE_F, MOE_K, T), mx.fill_normal(0xAC700105 + T, T * MOE_K, MOE_F))
        yg = be.tensor(mx.F32, (MOE_F, MOE_K, T))
        yu = be.tensor(mx.F32, (MOE_F, MOE_K, T))
        yd = be.tensor(mx.F32, (MOE_H, MOE_K, T))
        for l, E in enumerate(layers):
            ids = router_ids(T, 0x70E70005 + 1000 * T + l)
            d = len(np.unique(ids))
            distinct.append(d)
            I = be.tensor(mx.I32, (MOE_K, T), ids)
            wgu = d * row_bytes(WT, MOE_H) * MOE_F
            wdn = d * row_bytes(WT, MOE_F) * MOE_H
            ops = 2 * T * MOE_K * MOE_H * MOE_F
            # gate and up read the same rows and ids (TextModel::experts): one MUL_MAT_ID group, one prep
            gu_bytes = 2 * wgu + 4 * T * (MOE_H + 2 * MOE_K * MOE_F + MOE_K)
            launches.append(Launch(f"T{T}", gu_bytes, 2 * ops,
                                   lambda E=E, I=I: be.mul_mat_id_group([E["gate"], E["up"]], xb, I, [yg, yu]),
                                   weight_bytes=2 * wgu))
            launches.append(Launch(f"T{T}", wdn + 4 * T * (MOE_K * MOE_F + MOE_K * MOE_H + MOE_K), ops,
                                   lambda E=E, I=I: be.mul_mat_id(E["down"], xa, I, yd), weight_bytes=wdn))
            wbytes += d * per_expert
        log(f"T = {T}: distinct experts per layer {min(distinct)}..{max(distinct)} (mean {np.mean(distinct):.1f})")
        ms = time_graph(be, launches, args.steps, args.warmup, not args.no_graph)
        ms_total += ms
        b = sum(L.nbytes for L in launches)
        per_batch.append({"T": T, "distinct_experts_mean": round(float(np.mean(distinct)), 2),
                          "weight_bytes_per_layer": int(wbytes / MOE_LAYERS),
                          "us_per_layer": round(ms / MOE_LAYERS * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
                          "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                          "TOPs": round(sum(L.ops for L in launches) / (ms * 1e-3) / 1e12, 2)})
        all_launches.append((T, launches, ms))
    total_b = sum(L.nbytes for _, ls, _ in all_launches for L in ls)
    gbps = total_b / (ms_total * 1e-3) / 1e9
    T_dom, l_dom, ms_dom = all_launches[-1]
    kern = (f"k_mmid_q4k at T = {T_dom} (with its bucket and Q8_K pass)" if WT == Q4_K else
            f"k_gemm_dq over expert chunks at T = {T_dom} (with its bucket and fp16 row pass)")
    roof = step_hbm_roofline(kern, l_dom, ms_dom)
    roof["traffic"] = read_traffic("moe") if WT == Q4_K else None
    result = base_result(args, round(gbps, 1), "GB/s", ms_total, "int8", {
        "workload": "drama3-like MoE FFN layer via MUL_MAT_ID, token batches 1, 16, 256", "experts": MOE_E,
        "top_k": MOE_K, "hidden": MOE_H, "expert_ffn": MOE_F, "weights": args.moe_weights, "layer_copies": MOE_LAYERS,
        "graph": not args.no_graph})
    result.update({"hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "per_batch": per_batch, "roofline": roof})
    if args.cpu_seconds > 0 and WT != Q5_K:  # the CPU port has no Q5_K dot
        O = load_oracle()
        cores = O.physical_cores()
        T = 16
        ids = router_ids(T, 0x70E70005 + 1000 * T)
        xb = O.fill_normal(0xAC700005 + T, T, MOE_H)
        xa = O.fill_normal(0xAC700105 + T, T * MOE_K, MOE_F).reshape(T, MOE_K, MOE_F)
        hw = {name: host[name].reshape(MOE_E, N, -1) for name, _, N in specs}

        def layer(c):
            for name in ("gate", "up"):
                for e in np.unique(ids):
                    rows = np.nonzero((ids == e).any(axis=1))[0]
                    O.cpu_fast_mul_mat(WT, hw[name][e], xb[rows], c)
            for e in np.unique(ids):
                t_idx, s_idx = np.nonzero(ids == e)
                O.cpu_fast_mul_mat(WT, hw["down"][e], xa[t_idx, s_idx], c)

        wb = len(np.unique(ids)) * per_expert
        runs = []
        for c, sec in ((cores, args.cpu_seconds), (1, args.cpu_seconds / 3)):
            n, el = timed_sample(lambda c=c: layer(c), sec)
            runs.append({"value": round(n * wb / el / 1e9, 2), "unit": "GB/s", "cores": c, "kind": "port",
                         "sample": f"{n} MoE layers at T = {T} ({len(np.unique(ids))} distinct experts), "
                                   f"per-expert AVX2 products over the routed rows, {el:.1f} s (the median of three rounds), "
                                   f"{c} threads"})
        result["cpu_baseline"] = cpu_result(runs[0], runs[1])
    return result


def run_peaks(args, mx, be, threads):
    """Practical ceilings of this device, measured with the products' own launch path: a streaming read of a 4 GiB
    buffer (16 times the last-level cache) swept over loads in flight, plain / nontemporal loads and grid sizes; and
    int8 / fp16 MFMA issue from register operands. The products' roofline fractions stay quoted against the published
    peaks; these say how much of each peak a kernel can reach at all."""
    nbytes = 4 << 30
    buf = be.tensor(mx.F32, (nbytes // 4,))
    mx.check(mx.lib().mx_tensor_memset(be.h, buf.ref(), 0, 0, nbytes))
    e0, e1 = be.event(), be.event()

    def timed(fn, reps):
        fn()
        be.sync()
        be.record(e0)
        for _ in range(reps):
            fn()
        be.record(e1)
        be.sync()
        return be.elapsed_ms(e0, e1) / reps

    sweep = []
    for loads in (4, 8, 16):
        for nt in (False, True):
            for wgs in (1024, 2048, 4096, 8192, 16384):
                ms = timed(lambda: be.peak_read(buf, wgs, loads, nt), args.steps)
                gbps = nbytes / (ms * 1e-3) / 1e9
                sweep.append({"loads": loads, "nontemporal": nt, "workgroups": wgs, "us": round(ms * 1e3, 2),
                              "GBps": round(gbps, 1)})
                log(f"read loads={loads:2d} nt={int(nt)} wgs={wgs:5d}: {ms * 1e3:8.1f} us  {gbps:7.1f} GB/s")
    best = max(sweep, key=lambda r: r["GBps"])
    mfma = {}
    for kind, name, per, peak in ((0, "int8", 65536, INT8_PEAK_TOPS), (1, "fp16", 32768, FP16_PEAK_TFLOPS)):
        rows = []
        for wgs in (256, 1024, 2048):
            iters = 20000
            ms = timed(lambda: be.peak_mfma(kind, wgs, iters), 3)
            t = wgs * 4 * iters * 8 * per / (ms * 1e-3) / 1e12
            rows.append({"workgroups": wgs, "iters": iters, "ms": round(ms, 3), "T_per_s": round(t, 1),
                         "frac": round(t / peak, 4)})
            log(f"mfma {name} wgs={wgs:5d}: {ms:8.3f} ms  {t:8.1f} T/s  ({t / peak:.3f} of {peak:.0f})")
        mfma[name] = {"best": max(rows, key=lambda r: r["T_per_s"]), "sweep": rows, "peak": peak,
                      "unit": "TOP/s" if kind == 0 else "TFLOP/s"}
    be.event_free(e0)
    be.event_free(e1)
    buf.free()
    result = base_result(args, best["GBps"], "GB/s", best["us"] * 1e-3, "u8", {
        "workload": "peak micro-benchmarks: 4 GiB streaming read; int8 and fp16 MFMA issue", "read_bytes": nbytes})
    result.update({"hbm_read_best": best, "hbm_read_frac_of_published": round(best["GBps"] / HBM_PEAK_GBPS, 4),
                   "hbm_read_sweep": sweep, "mfma": mfma})
    return result


# The prefill products' shapes (M = 512 blocks of configs 3 and 4: q/k/v, attn_o, gate/up, down; and a larger M)
VENDOR_SHAPES = ((512, 2048, 4096), (512, 2048, 2048), (512, 2048, 12288), (512, 6144, 2048), (1536, 2048, 12288),
                 (4096, 4096, 4096))


def run_vendor_gemm(args, mx, be, threads):
    """The vendor library's GEMMs on plain operands at the prefill products' shapes, for scale: int8 x int8 -> int32
    (torch._int_mm, hipBLASLt) and fp16 x fp16 -> fp16 (torch.matmul, hipBLASLt), operands resident, timed with torch
    events on torch's stream. No per-block scales and no dequantization: what a Q8_0 product would take if it were a
    plain int8 GEMM. Not a product path of this library; its ceiling for comparison."""
    import torch
    dev = "cuda"

    def timed(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    rows = []
    for M, K, N in VENDOR_SHAPES:
        g = torch.Generator(device=dev).manual_seed(M * 7 + K * 5 + N)
        a8 = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
        b8 = torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev, generator=g)
        ah = torch.randn(M, K, dtype=torch.float16, device=dev, generator=g)
        bh = torch.randn(K, N, dtype=torch.float16, device=dev, generator=g)
        ops = 2 * M * N * K
        ms8 = timed(lambda: torch._int_mm(a8, b8), args.steps)
        ms16 = timed(lambda: ah @ bh, args.steps)
        r = {"M": M, "K": K, "N": N, "int8_us": round(ms8 * 1e3, 2), "int8_TOPs": round(ops / (ms8 * 1e-3) / 1e12, 1),
             "int8_frac": round(ops / (ms8 * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4), "fp16_us": round(ms16 * 1e3, 2),
             "fp16_TFLOPs": round(ops / (ms16 * 1e-3) / 1e12, 1),
             "fp16_frac": round(ops / (ms16 * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4)}
        rows.append(r)
        log(f"M={M} K={K} N={N}: int8 {r['int8_us']:7.1f} us {r['int8_TOPs']:7.1f} TOP/s ({r['int8_frac']:.3f}); "
            f"fp16 {r['fp16_us']:7.1f} us {r['fp16_TFLOPs']:7.1f} TFLOP/s ({r['fp16_frac']:.3f})")
        del a8, b8, ah, bh
    m512 = [r for r in rows if r["M"] == 512]
    ops = sum(2 * r["M"] * r["N"] * r["K"] for r in m512)
    us = sum(r["int8_us"] for r in m512)
    result = base_result(args, round(ops / (us * 1e-6) / 1e12, 1), "TOP/s", us * 1e-3, "int8", {
        "workload": "vendor int8 / fp16 GEMM (hipBLASLt through torch) at the prefill products' shapes",
        "shapes": [list(s) for s in VENDOR_SHAPES]})
    result["data"] = "synthetic (seeded uniform int8 and N(0,1) fp16 operands)"
    result.update({"m512_block_int8_frac": round(ops / (us * 1e-6) / 1e12 / INT8_PEAK_TOPS, 4), "per_shape": rows})
    return result


WORKLOADS = {"decode": run_decode, "decode-full": run_decode_full, "matvec": run_matvec, "prefill-q4k": run_prefill_q4k, "asr-1.7b": run_asr,
             "moe": run_moe, "peaks": run_peaks, "vendor-gemm": run_vendor_gemm}
DEFAULT_STEPS = {"decode": (300, 20), "decode-full": (100, 10), "matvec": (50, 5), "prefill-q4k": (20, 3), "asr-1.7b": (3, 1), "moe": (20, 3), "peaks": (5, 1),
                 "vendor-gemm": (50, 3)}


def other_configs(args, mx, be, threads):
    """The other benchmark configurations, each at its default steps with a CPU sample of half the decode step's
    length, summarized for the default line: value, unit, time per step, the dominant kernel's roofline fraction and
    the CPU baseline (one after another on this backend; each workload's tensors are freed before the next)."""
    out = {}
    for w in ("matvec", "prefill-q4k", "asr-1.7b", "moe"):
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup = DEFAULT_STEPS[w]
        sub.cpu_seconds, sub.blocks, sub.batches = args.cpu_seconds / 2, None, None
        sub.moe_weights = "Q4_K"  # the configuration's experts
        log(f"configs: {w}")
        r = WORKLOADS[w](sub, mx, be, threads)
        roof = r.get("roofline") or {}
        out[w] = {"value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
                  "workload": r["config"]["workload"], "roofline_frac": roof.get("frac"), "bound": roof.get("bound"),
                  "kernel": roof.get("kernel")}
        if "cpu_baseline" in r:
            c = r["cpu_baseline"]
            out[w]["cpu_baseline"] = {k: c[k] for k in ("value", "unit", "cores", "kind", "sample", "value_1thread")
                                      if k in c}
        for k in ("hbm_frac", "decode_tok_s", "decode_hbm_frac", "prefill_ms"):
            if k in r:
                out[w][k] = r[k]
        if "per_batch" in r:
            out[w]["per_batch"] = [{"T": b["T"], "us_per_layer": b["us_per_layer"], "hbm_frac": b["hbm_frac"]}
                                   for b in r["per_batch"]]
        del r
        gc.collect()
        be.sync()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="decode")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU-baseline sample (0 skips it)")
    ap.add_argument("--no-graph", action="store_true",
                    help="replay the step (and each label's launches) eagerly instead of as graphs")
    ap.add_argument("--unfused", action="store_true", help="decode-full: one launch per ggml node, no fusions")
    ap.add_argument("--no-full-step", dest="full_step", action="store_false",
                    help="decode: skip timing the whole step (decode_full_tok_s) beside the products")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="decode: skip the other configurations' summaries (matvec, prefill-q4k, asr-1.7b, moe) that "
                         "the default line carries under 'configs'")
    ints = lambda v: [int(t) for t in v.split(",")]
    ap.add_argument("--blocks", type=ints, default=None,
                    help="asr-1.7b: prefill block rows (default 512,512,512,28; counter passes use 512,512,512)")
    ap.add_argument("--moe-weights", choices=sorted(TYPE_OF), default="Q4_K",
                    help="moe: the experts' type (default Q4_K, as the configuration names it)")
    ap.add_argument("--batches", type=ints, default=None,
                    help="moe: token batches (default 1,16,256; counter passes use 256)")
    ap.add_argument("--opt", action="append", default=[], metavar="NAME=VALUE",
                    help="a kernel choice of the backend (mx_backend_set_option), e.g. gemm_q8_0=2; repeatable")
    ap.add_argument("--pmc-kernel", default=None,
                    help="with --summarize-pmc: the kernel-name substring to sum (default: the workload's own)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic summary of two rocprofv3 --pmc runs of --workload's benchmark and exit")
    ap.add_argument("--summarize-busy", nargs=2, metavar=("GRBM_CSV", "CLOCK_MHZ"),
                    help="print the per-dispatch busy time of a rocprofv3 --pmc GRBM_GUI_ACTIVE run of --workload's "
                         "benchmark at the given shader clock and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc, args.pmc_kernel or TRAFFIC[args.workload][1]))
        return
    if args.summarize_busy:
        print(summarize_busy(args.summarize_busy[0], TRAFFIC[args.workload][1], float(args.summarize_busy[1])))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    steps, warmup = DEFAULT_STEPS[args.workload]
    args.steps = steps if args.steps is None else args.steps
    args.warmup = warmup if args.warmup is None else args.warmup
    rank = int(os.environ.get("RANK", "0"))
    if rank != 0:
        args.cpu_seconds = 0

    if args.workload == "vendor-gemm":  # torch's own HIP runtime: initialised before (and without) libmx's
        result = run_vendor_gemm(args, None, None, 1)
        print(json.dumps(result), flush=True)
        return
    mx = load_mx()
    if mx.device_count() < 1:
        print("no GPU visible to libmx", file=sys.stderr)
        sys.exit(1)
    be = mx.Backend(0)
    for kv in args.opt:
        name, value = kv.split("=", 1)
        be.set_option(name, int(value))
    calibration_copy(mx, be)
    global EVICT
    EVICT = make_evictor(mx, be)
    threads = max(1, len(os.sched_getaffinity(0)))
    result = WORKLOADS[args.workload](args, mx, be, threads)
    if args.workload == "decode" and args.configs:
        result["configs"] = other_configs(args, mx, be, threads)
    be.close()
    if rank == 0:
        print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
