"""Benchmark of the gfx950 quantized-weight path (one GPU).

Workload: every SmolLM2-135M-shaped linear layer
in Q4_0 as a matvec -- 30 layers x {q, k, v, o, gate, up, down} plus the tied
49152x576 lm_head, 211 products per step, batch 1.  One step is one pass over
all of them with synthetic activations; weights are synthetic (synth-v1,
N(0, 0.02)) and quantized on the GPU.  A step reads a different copy of the
whole weight set (rotating copies totalling >= 1 GiB), so no step finds its
weights in the 256 MB Infinity Cache.

The 211 products of a step run as one grouped launch (llmi_hip_group), so
the step is one kernel.  `value` = algorithmic bytes per step (packed codes
+ fp32 scales + x + y, each once) x steps / the time between two HIP events
around the back-to-back launches; `roofline` is that same kernel.  `cpu_baseline` times the reference's
threaded CPU quant::matmul on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "llm-inference-cpp_amd"))

import llmi_hip as H  # noqa: E402
import synth  # noqa: E402
import workloads as W  # noqa: E402

METRIC = "Q4_0/Q8_0 GEMV achieved HBM GB/s (% of peak); decode tokens/s, 1 GPU"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1 << 30
# The rocprofv3 summary that holds the measured HBM traffic of the headline
# kernel (FETCH_SIZE and WRITE_SIZE passes over this script, scaled by a
# plain copy kernel's readings).
TRAFFIC_PROFILE = os.path.join("profiles", "qgemv_group_smollm2_q4_b1.md")
HEADLINE_KERNEL = "qgemv_group<2, 1>"


def profiled_traffic(kernel: str = HEADLINE_KERNEL, path: str = TRAFFIC_PROFILE):
    """HBM bytes per launch of `kernel` from the traffic table of a committed
    rocprofv3 summary: the row whose first cell is the kernel's name, the
    column headed "HBM bytes (scaled)".  None when the summary has no such
    row."""
    try:
        with open(os.path.join(ROOT, path)) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    header = None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if "HBM bytes (scaled)" in cells:
            header = cells
            continue
        if header is not None and cells and cells[0].strip("`") == kernel and len(cells) == len(header):
            try:
                return int(cells[header.index("HBM bytes (scaled)")].replace(",", ""))
            except ValueError:
                return None
    return None


SMOL_LAYER = W.SMOL_LAYER
SMOL_HEAD = W.SMOL_HEAD
N_LAYERS = 30
QWEN_TARGETS = [("lm_head", 151936, 896, H.Q4_0), ("lm_head", 151936, 896, H.Q8_0),
                ("gate_proj", 4864, 896, H.Q4_0), ("down_proj", 896, 4864, H.Q4_0)]


algo_bytes = W.algo_bytes


def step_shapes():
    shapes = [s for _ in range(N_LAYERS) for s in SMOL_LAYER]
    shapes.append(SMOL_HEAD)
    return shapes


class WeightSet:
    """`copies` independent device copies of a list of (name, out, in)."""

    def __init__(self, shapes, qt, copies, seed0):
        self.shapes = shapes
        self.copies = []
        biggest = max(o * i for _, o, i in shapes)
        stage = H.DeviceBuffer(biggest * 4)
        for c in range(copies):
            ws = []
            for j, (_, out, n_in) in enumerate(shapes):
                H.synth_normal_dev(stage, out * n_in, seed0 + 1000003 * c + j, 0.0, 0.02)
                ws.append(H.Weight.quantize_dev(stage.ptr, out, n_in, qt))
            self.copies.append(ws)
        stage.free()

    def free(self):
        for ws in self.copies:
            for w in ws:
                w.free()


def run_step(ws, xs, ys, batch):
    for w, x, y in zip(ws, xs, ys):
        w.matmul_dev(x.ptr, batch, None, y.ptr)


def activations(shapes, batch, seed):
    xs, ys = [], []
    cache = {}
    for _, out, n_in in shapes:
        if (out, n_in) not in cache:
            xb = H.DeviceBuffer(batch * n_in * 4)
            H.synth_normal_dev(xb, batch * n_in, seed + n_in, 0.0, 1.0)
            cache[(out, n_in)] = (xb, H.DeviceBuffer(batch * out * 4))
        xs.append(cache[(out, n_in)][0])
        ys.append(cache[(out, n_in)][1])
    return xs, ys, cache


def time_steps(wset, batch, steps, warmup, mode="group", sustain=0):
    """GPU time of `steps` passes over the rotating weight copies (with
    sustain > 0: a pair (ms, sustain_ms), the first `sustain` passes timed
    on their own right before the warm-up, on the same launches).

    mode "group": each pass is ONE llmi_hip_group launch holding its copy's
    211 products; "tol": the same products as one tolerance-mode group
    (llmi_hip_tol_group: the activation split kernel + one product launch);
    "graph": one HIP graph replay of 211 single-matrix launches; "plain": 211
    single-matrix launches from Python."""
    xs, ys, keep = activations(wset.shapes, batch, 77)
    n = len(wset.copies)
    if mode in ("group", "tol"):
        kind = H.Group if mode == "group" else H.TolGroup
        gs = [kind([(w, x.ptr, y.ptr, batch) for w, x, y in zip(ws, xs, ys)]) for ws in wset.copies]
        run = lambda i: gs[i % n].launch()  # noqa: E731
    elif mode == "graph":
        gs = [H.Graph(lambda ws=ws: run_step(ws, xs, ys, batch)) for ws in wset.copies]
        run = lambda i: gs[i % n].launch()  # noqa: E731
    else:
        run = lambda i: run_step(wset.copies[i % n], xs, ys, batch)  # noqa: E731
    sus_ms = None
    if sustain > 0:
        t = H.Timer()
        t.start()
        for i in range(sustain):
            run(i)
        sus_ms = t.stop()
    for i in range(warmup):
        run(sustain + i)
    H.synchronize()
    t = H.Timer()
    t.start()
    for i in range(steps):
        run(sustain + warmup + i)
    ms = t.stop()
    H.synchronize()
    del keep
    return ms if sustain <= 0 else (ms, sus_ms)


def tolerance_check(wset):
    """Largest |y_tol - y_exact| / max|y_exact| over the 211 products of one
    copy, batch 1 and 8 (the exact kernel's outputs equal the reference's)."""
    worst = 0.0
    ws = wset.copies[0]
    for batch in (1, 8):
        xs, ys, keep = activations(wset.shapes, batch, 77)
        yt = {id(w): H.DeviceBuffer(batch * out * 4) for (_, out, _), w in zip(wset.shapes, ws)}
        gt = H.TolGroup([(w, x.ptr, yt[id(w)].ptr, batch) for w, x in zip(ws, xs)])
        gt.launch()
        H.synchronize()
        # The exact group's products of one shape share a y buffer, so each
        # product's exact output comes from a launch of its own.
        for (_, out, _), w, x in zip(wset.shapes, ws, xs):
            ye = H.DeviceBuffer(batch * out * 4)
            w.matmul_dev(x.ptr, batch, None, ye.ptr)
            H.synchronize()
            a = ye.download(np.float32, batch * out).astype(np.float64)
            b = yt[id(w)].download(np.float32, batch * out).astype(np.float64)
            worst = max(worst, float(np.abs(a - b).max() / max(np.abs(a).max(), 1e-30)))
            ye.free()
        gt.free()
        for b in yt.values():
            b.free()
        del keep
    return worst


def time_launches(weights, batch, launches, tol=False):
    """Mean GPU time per launch of `launches` back-to-back launches (cycling
    through the rotating weight copies) between one pair of HIP events on
    the library stream.  Includes the ~2 us stream dispatch gap between
    kernels; an event pair around each single launch would add ~6 us more."""
    n_in, out = weights[0].n_in, weights[0].out
    xb = H.DeviceBuffer(batch * n_in * 4)
    H.synth_normal_dev(xb, batch * n_in, 5, 0.0, 1.0)
    yb = H.DeviceBuffer(batch * out * 4)
    call = (lambda w: w.matmul_tol_dev(xb.ptr, batch, None, yb.ptr)) if tol else \
        (lambda w: w.matmul_dev(xb.ptr, batch, None, yb.ptr))
    call(weights[0])  # warm-up (code load)
    H.synchronize()
    t = H.Timer()
    t.start()
    for i in range(launches):
        call(weights[(i + 1) % len(weights)])
    ms = t.stop()
    H.synchronize()
    return ms / launches


def target_shapes():
    """Per-launch GB/s of the Qwen2.5-0.5B shapes the north star targets
    (>= 70% of HBM peak), cold cache via rotating copies."""
    res = {}
    stage = None
    for name, out, n_in, qt in QWEN_TARGETS:
        nbytes = out * H.row_bytes(n_in, qt) + 4 * out * H.nblocks(n_in)
        copies = max(2, min(400, -(-ROTATE_BYTES // nbytes)))
        if stage is None or stage.nbytes < out * n_in * 4:
            stage = H.DeviceBuffer(max(out * n_in * 4, 151936 * 896 * 4))
        ws = []
        for c in range(copies):
            H.synth_normal_dev(stage, out * n_in, 900 + c, 0.0, 0.02)
            ws.append(H.Weight.quantize_dev(stage.ptr, out, n_in, qt))
        ms = time_launches(ws, 1, min(200, 2 * copies))
        gbs = algo_bytes(out, n_in, qt, 1) / (ms * 1e-3) / 1e9
        res[f"qwen_{name}_{H.TYPE_NAMES[qt]}_{out}x{n_in}"] = dict(us=round(ms * 1e3, 2), gbs=round(gbs, 1),
                                                                  pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 1))
        if qt == H.Q4_0:
            ms = time_launches(ws, 1, min(200, 2 * copies), tol=True)
            gbs = algo_bytes(out, n_in, qt, 1) / (ms * 1e-3) / 1e9
            res[f"qwen_{name}_{H.TYPE_NAMES[qt]}_{out}x{n_in}_tolerance_mode"] = dict(
                us=round(ms * 1e3, 2), gbs=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 1))
        for w in ws:
            w.free()
    if stage is not None:
        stage.free()
    res.update(grouped_mlp_targets())
    return res


def grouped_mlp_targets(steps=50):
    """The Qwen2.5-0.5B MLP matrices at streaming scale: all 24 layers' gate,
    up (4864x896) and down (896x4864) as one grouped launch per step, batch 1,
    rotating copies (>= 1 GiB).  A single launch of one of these 2.7 MB
    matrices is bound by launch latency, not bandwidth."""
    res = {}
    shapes = [s for _ in range(24) for s in (("gate_proj", 4864, 896), ("up_proj", 4864, 896), ("down_proj", 896, 4864))]
    for qt in (H.Q4_0, H.Q8_0):
        wb = sum(o * H.row_bytes(i, qt) + 4 * o * H.nblocks(i) for _, o, i in shapes)
        wset = WeightSet(shapes, qt, max(2, -(-ROTATE_BYTES // wb)), 31)
        for mode in ("group", "tol") if qt == H.Q4_0 else ("group",):
            ms = time_steps(wset, 1, steps, 5, mode=mode)
            us = ms / steps * 1e3
            gbs = sum(algo_bytes(o, i, qt, 1) for _, o, i in shapes) / (us * 1e-6) / 1e9
            key = f"qwen_mlp_24_layers_grouped_{H.TYPE_NAMES[qt]}" + ("_tolerance_mode" if mode == "tol" else "")
            res[key] = dict(us=round(us, 2), gbs=round(gbs, 1), pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 1))
            print(f"[bench] Qwen MLP x24 grouped {H.TYPE_NAMES[qt]} {mode}: {us:.1f} us, {gbs:.0f} GB/s",
                  file=sys.stderr, flush=True)
        wset.free()
    return res


# The reference's per-shape decode table (tools/bench_apple_silicon.cpp:96-146):
# each SmolLM2-135M shape alone at rows = 1, (name, out, in).
REF_SHAPES = [("attn_qkv_o", 576, 576), ("mlp_up_gate", 1536, 576), ("mlp_down", 576, 1536), ("lm_head", 49152, 576)]
PER_SHAPE_ROTATE = 512 << 20


def weight_bytes_of(out: int, n_in: int, qt: int) -> int:
    """Device bytes of one matrix: fp32 values, or packed codes + fp32 scales."""
    if qt == H.F32:
        return 4 * out * n_in
    return out * H.row_bytes(n_in, qt) + 4 * out * H.nblocks(n_in)


def per_shape_gpu():
    """Each of the reference's per-shape rows on the GPU: F32, Q8_0 and Q4_0,
    batch 1 and 8, as back-to-back single launches (llmi_hip_matmul_dev)
    cycling over rotating copies of >= 512 MB (more than the 256 MB Infinity
    Cache) or 2000 copies.  us = mean per launch between one pair of HIP
    events (includes the ~2 us dispatch gap); gbs = algorithmic bytes
    (weights + x + y) / us; weight_gbs = weight bytes / us, the reference
    table's GB/s."""
    res = {}
    stage = H.DeviceBuffer(max(o * i for _, o, i in REF_SHAPES) * 4)
    for name, out, n_in in REF_SHAPES:
        row = {}
        for qt in (H.F32, H.Q8_0, H.Q4_0):
            wb = weight_bytes_of(out, n_in, qt)
            copies = max(2, min(2000, -(-PER_SHAPE_ROTATE // wb)))
            ws = []
            for c in range(copies):
                H.synth_normal_dev(stage, out * n_in, 700 + c, 0.0, 0.02)
                ws.append(H.Weight.quantize_dev(stage.ptr, out, n_in, qt))
            entry = {"copies": copies, "weight_bytes": wb}
            for batch in (1, 8):
                us = time_launches(ws, batch, max(200, min(4000, 2 * copies))) * 1e3
                algo = wb + 4 * batch * (n_in + out)
                gbs = algo / (us * 1e-6) / 1e9
                entry[f"b{batch}"] = dict(us=round(us, 3), gbs=round(gbs, 1),
                                          weight_gbs=round(wb / (us * 1e-6) / 1e9, 1),
                                          pct_hbm_peak=round(100 * gbs / HBM_PEAK_GBS, 1))
            for w in ws:
                w.free()
            row[H.TYPE_NAMES[qt]] = entry
        res[f"{name}_{out}x{n_in}"] = row
    stage.free()
    b1 = res["mlp_up_gate_1536x576"]["q8_0"]["b1"]
    print(f"[bench] per-shape: C1 q8_0 1536x576 b1 {b1['us']} us {b1['gbs']} GB/s", file=sys.stderr, flush=True)
    return res


QWEN_LAYER = W.QWEN_LAYER
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32 vector (packed); this build issues non-packed FMAs only


def gguf_upload(reps=3):
    """GGUF -> device: the raw ggml blocks of a Qwen2.5
    lm_head-shaped tensor (151936x896) -> device weight through
    llmi_hip_weight_from_gguf, Q4_0 and Q8_0.  Wall time of the call: the
    host-to-device copy of the raw blocks (pageable memory) plus the
    conversion kernel; best of `reps`."""
    out, n_in = 151936, 896
    nb = out * n_in // 32
    rng = np.random.default_rng(5)
    res = {"tensor": f"{out}x{n_in}", "timing": "wall clock of the call, PCIe copy included"}
    for gt, name, qb in ((H.GGUF_Q4_0, "q4_0", 16), (H.GGUF_Q8_0, "q8_0", 32)):
        raw = rng.integers(0, 256, size=(nb, 2 + qb), dtype=np.uint8)
        sc = np.abs(rng.normal(0.0, 0.002, nb)).astype(np.float16).view(np.uint16)
        raw[:, 0] = (sc & 0xFF).astype(np.uint8)
        raw[:, 1] = (sc >> 8).astype(np.uint8)
        raw = raw.reshape(-1)
        best = float("inf")
        for _ in range(reps):
            H.synchronize()
            t0 = time.perf_counter()
            w = H.Weight.from_gguf(raw, out, n_in, gt)
            best = min(best, time.perf_counter() - t0)
            w.free()
        res[name] = {"raw_bytes": int(raw.nbytes), "ms": round(best * 1e3, 2),
                     "gbs": round(raw.nbytes / best / 1e9, 2)}
    return res


def prefill_gemm(steps=20, warmup=3):
    """M=512 tokens of fp32 activations against
    every Qwen2.5-0.5B linear layer (24 layers x 7 products) in Q8_0, on the
    bf16-MFMA GEMM, each layer with its own activations
    (workloads.PrefillProducts, the same products
    tests/test_gpu_gemm.py checks).  "per_layer" runs them as 24 launches of
    one layer's 7 products -- the realistic schedule, since a layer's input
    is the previous layer's output; "one_launch" runs all 168 in one grouped
    launch (independent products, an upper bound on the kernel)."""
    prods = W.PrefillProducts(M=512, layers=24, qt=H.Q8_0)
    flops = prods.flops()
    wbytes = sum(w.byte_size for w in prods.weights)
    res = {}
    for mode, groups in (("per_layer", [H.GemmGroup(li) for li in prods.per_layer]),
                         ("one_launch", [H.GemmGroup(prods.items)])):
        for _ in range(warmup):
            for g in groups:
                g.launch()
        H.synchronize()
        t = H.Timer()
        t.start()
        for _ in range(steps):
            for g in groups:
                g.launch()
        ms = t.stop() / steps
        H.synchronize()
        tf = flops / (ms * 1e-3) / 1e12
        res[mode] = dict(ms=round(ms, 4), tflops=round(tf, 1), frac_of_mfma_peak=round(tf / MFMA_PEAK_TFLOPS, 4),
                         launches=len(groups))
        for g in groups:
            g.free()
    prods.free()
    res.update(workload="24 layers x {q,k,v,o 896/128 x 896; gate,up 4864x896; down 896x4864} Q8_0, M=512, fp32 "
                        "in/out, distinct activations per layer",
               gflop=round(flops / 1e9, 2), weight_bytes=wbytes, precision="bf16 operands, fp32 accumulate (tolerance 2e-2)")
    print(f"[bench] c5 prefill GEMM: {res['per_layer']['tflops']} TFLOP/s per-layer, "
          f"{res['one_launch']['tflops']} one launch", file=sys.stderr, flush=True)
    return res


DECODE_RUNS = [  # (key, golden fixture, model config, weight type): BASELINE.json configs[2], configs[3]
    ("c3_smollm2_135m_q8_0", "c3_smollm2_q8", synth.SMOLLM2_135M, H.Q8_0),
    ("c4_qwen25_05b_q4_0", "c4_qwen25_q4", synth.QWEN25_05B, H.Q4_0),
]


def prefill_flops(cfg, T):
    """Floating-point operations of the exact prefill of T tokens: every
    projection at T rows, the lm_head on the last row, and causal attention
    (scores and P.V, 2 flops per multiply-add each)."""
    H, L, nh = cfg["hidden_size"], cfg["num_layers"], cfg["num_heads"]
    hd = H // nh
    kv = cfg["num_kv_heads"] * hd
    per_layer = H * H + 2 * kv * H + H * H + 3 * cfg["intermediate_size"] * H
    attn = L * nh * hd * 4 * T * (T + 1) // 2
    return 2 * T * L * per_layer + 2 * cfg["vocab_size"] * H + attn


def decode_runs(max_steps: int | None = None, greedy_only: bool = False, graphs: bool = True):
    """Full-model greedy decode on the synthetic models: prefill the prompt,
    then the configured number of greedy steps (at most max_steps, for
    profiling runs); ids are checked against the reference's (tests/golden),
    a shortened run against their prefix.  Then the sampled decode and the
    perplexity chunk, unless greedy_only (profiling passes).  graphs: the
    tolerance-mode greedy steps replay one captured graph (off for profilers
    that do not follow graphs)."""
    res = {}
    for key, golden, cfg, qt in DECODE_RUNS:
        with open(os.path.join(ROOT, "tests", "golden", golden + ".json")) as f:
            rec = json.load(f)
        if max_steps is not None and max_steps < rec["n_steps"]:
            rec = dict(rec, n_steps=max_steps, ids=rec["ids"][:max_steps])
        H.synchronize()
        t0 = time.perf_counter()
        m = H.synthetic_model_dev(cfg, rec["seed"], qt, rec["convention"])
        m.set_decode_graph(graphs)
        H.synchronize()
        load_s = time.perf_counter() - t0
        prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])
        m.generate_greedy(prompt, 4)  # warm-up at the real prompt length (code objects, workspace)
        t0 = time.perf_counter()
        ids = m.generate_greedy(prompt, rec["n_steps"])
        gen_s = time.perf_counter() - t0
        pre_ms, dec_ms = m.last_timing()
        wb = m.weight_bytes()
        n_kv = cfg["num_layers"] * cfg["num_kv_heads"] * (cfg["hidden_size"] // cfg["num_heads"]) * 4 * 2
        mean_ctx = rec["n_prompt"] + rec["n_steps"] / 2.0
        bytes_per_token = wb + n_kv * mean_ctx
        tok_s = rec["n_steps"] / (dec_ms * 1e-3)
        pre_tf = prefill_flops(cfg, rec["n_prompt"]) / (pre_ms * 1e-3) / 1e12
        roof = HBM_PEAK_GBS * 1e9 / bytes_per_token
        res[key] = dict(prompt=rec["n_prompt"], steps=rec["n_steps"], weights=H.TYPE_NAMES[qt],
                        prefill_ms=round(pre_ms, 2), prefill_tok_s=round(rec["n_prompt"] / (pre_ms * 1e-3), 1),
                        prefill_tflops=round(pre_tf, 2), prefill_frac_of_fp32_peak=round(pre_tf / FP32_PEAK_TFLOPS, 4),
                        decode_ms=round(dec_ms, 2), decode_tok_s=round(tok_s, 1),
                        bytes_per_token=int(bytes_per_token), roofline_tok_s=round(roof, 1),
                        frac_of_roofline=round(tok_s / roof, 4),
                        ids_match_reference=bool(np.array_equal(ids, np.array(rec["ids"], np.int32))))
        # llmi-generate --json's record (apps/llmi-generate/main.cpp:339-345); load = synthesising the
        # fp32 weights on the device and quantizing them there (no checkpoint file exists here).
        res[key]["generate_json"] = dict(prompt_ids=[int(i) for i in prompt], generated_ids=[int(i) for i in ids],
                                         load_seconds=round(load_s, 3), generate_seconds=round(gen_s, 3),
                                         weight_bytes=int(wb))
        print(f"[bench] {key}: prefill {pre_ms:.1f} ms, decode {tok_s:.1f} tok/s, ids match "
              f"{res[key]['ids_match_reference']}", file=sys.stderr, flush=True)
        # The same greedy run with the tolerance-mode decode step
        # (llmi_hip_model_set_decode_mode): position-chunked attention merged
        # in o_proj, the products split over K with atomic adds; logits
        # within the fp32 tolerance, not bit-identical.
        m.set_decode_mode(H.DECODE_TOLERANCE)
        m.generate_greedy(prompt, 4)
        ids_t = m.generate_greedy(prompt, rec["n_steps"])
        _, dec_t = m.last_timing()
        m.set_decode_mode(H.DECODE_EXACT)
        tok_t = rec["n_steps"] / (dec_t * 1e-3)
        want = np.array(rec["ids"], np.int32)
        res[key]["tolerance_mode"] = dict(
            decode_tok_s=round(tok_t, 1), frac_of_roofline=round(tok_t / roof, 4),
            ids_match_first64=bool(np.array_equal(ids_t[:64], want[:64])),
            ids_match_reference=bool(np.array_equal(ids_t, want)),
            what="attention split over position chunks (softmax per chunk, merged in the o_proj launch); each "
                 "matmul split over K into ~1k one-wavefront workgroups whose partial sums (the exact block "
                 "chains within a split) meet by atomic adds; logits within 1e-4 * max|logit| of the exact step "
                 "(tests)")
        print(f"[bench] {key}: tolerance-mode decode {tok_t:.1f} tok/s, first 64 ids match "
              f"{res[key]['tolerance_mode']['ids_match_first64']}", file=sys.stderr, flush=True)
        if not greedy_only:
            res[key]["sampled"] = sampled_decode(m, prompt, rec, cfg)
        if cfg["vocab_size"] > 100000 and not greedy_only:
            res[key]["perplexity_chunk"] = perplexity_chunk(m, prompt, cfg)
        m.free()
    return res


SAMPLING_CFG = (0.8, 40, 0.9)  # llmi-chat's documented sampling example (docs/sampling.md)


def sampling_targets(n: int) -> np.ndarray:
    """Uniform [0, 1) doubles standing in for sample()'s draws (the CPU leg
    replays the same numbers)."""
    return np.random.default_rng(2024).random(n)


def sampled_decode(m, prompt, rec, cfg):
    """The same decode with sample() per step on the device
    (llmi_hip_model_generate_sampled): temperature 0.8, top-k 40, top-p 0.9,
    and unfiltered temperature 1.0; plus the cost of one sampling call alone
    on device-resident logits of this vocabulary (greedy / unfiltered /
    filtered), each call synchronous as in the serving loop."""
    n = rec["n_steps"]
    targets = sampling_targets(n)
    out = {}
    for name, sc in (("t0.8_k40_p0.9", SAMPLING_CFG), ("t1.0", (1.0, 0, 1.0))):
        m.generate_sampled(prompt[:8], 4, H.Sampling(*sc), targets[:4])  # warm-up
        ids = m.generate_sampled(prompt, n, H.Sampling(*sc), targets)
        _, dec_ms = m.last_timing()
        out[name] = {"decode_tok_s": round(len(ids) / (dec_ms * 1e-3), 1), "steps": int(len(ids)),
                     "redrawn_steps": m.last_redraws()}
        if name == "t0.8_k40_p0.9":
            out["ids_first16"] = [int(i) for i in ids[:16]]
    V = cfg["vocab_size"]
    buf = H.DeviceBuffer(V * 4)
    H.synth_normal_dev(buf, V, 77, 0.0, 3.0)
    H.synchronize()
    calls = {}
    for name, sc in (("greedy", (0.0, 0, 1.0)), ("t1.0", (1.0, 0, 1.0)), ("t0.8_k40_p0.9", SAMPLING_CFG)):
        c = H.Sampling(*sc)
        for t in targets[:3]:
            H.sample_dev(buf, V, c, t)
        reps = 50
        t0 = time.perf_counter()
        for t in targets[:reps]:
            H.sample_dev(buf, V, c, t)
        calls[name] = round((time.perf_counter() - t0) / reps * 1e6, 1)
    buf.free()
    out["call_us"] = calls
    print(f"[bench] sampled decode {out['t0.8_k40_p0.9']['decode_tok_s']} tok/s (t0.8 k40 p0.9), "
          f"{out['t1.0']['decode_tok_s']} tok/s (t1.0); one call {calls} us", file=sys.stderr, flush=True)
    return out


def perplexity_chunk(m, prompt, cfg, reps=3):
    """llmi-perplexity's scoring of one 512-token chunk from position 256
    (the app's default), through llmi_hip_model_chunk_nll: exact, with the
    bf16-MFMA lm_head, and with every linear on the bf16-MFMA GEMM; wall
    clock per chunk, scored tokens/s, and each fast mode's largest per-token
    NLL difference from the exact one."""
    n, first = 512, 256
    ids = prompt[:n] if len(prompt) >= n else synth.uniform_ids(9, n, cfg["vocab_size"])
    out = {"tokens": n, "scored": n - 1 - first}
    nll = {}
    for name, head in (("exact", H.SCORE_EXACT), ("mfma_head", H.SCORE_MFMA_HEAD), ("mfma", H.SCORE_MFMA)):
        m.chunk_nll(ids, first, head)  # warm-up
        best = float("inf")
        for _ in range(reps):
            t0 = time.perf_counter()
            nll[name] = m.chunk_nll(ids, first, head)
            best = min(best, time.perf_counter() - t0)
        out[name] = {"ms": round(best * 1e3, 2), "scored_tok_s": round((n - 1 - first) / best, 1),
                     "mean_nll": round(float(nll[name].mean()), 6)}
    for name in ("mfma_head", "mfma"):
        out[name]["max_abs_nll_diff"] = round(float(np.abs(nll[name] - nll["exact"]).max()), 6)
    print(f"[bench] perplexity chunk: exact {out['exact']['ms']} ms, mfma head {out['mfma_head']['ms']} ms, "
          f"all-mfma {out['mfma']['ms']} ms", file=sys.stderr, flush=True)
    return out


def cpu_decode(runs, max_prompt: int = 128, steps: int = 16):
    """The reference's own forward_cached (oracle/_ref) on the same synthetic
    models, as a bounded sample: the first min(prompt, max_prompt) prompt ids,
    then `steps` greedy steps (checked against the reference's ids when the
    whole prompt fits); adds cpu_* fields to each run's entry."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    ref = O.reference()
    use_ref = ref is not None and ref.pool_workers() + 1 <= 16
    cpu = ref if use_ref else O.oracle()
    if not use_ref:
        cpu.set_pool_workers(15)
    for key, golden, cfg, qt in DECODE_RUNS:
        with open(os.path.join(ROOT, "tests", "golden", golden + ".json")) as f:
            rec = json.load(f)
        tensors = synth.make_tensors(cfg, rec["seed"], rec["convention"])
        t0 = time.perf_counter()
        cm = O.CpuModel(cpu, cfg, tensors, qt)
        load_s = time.perf_counter() - t0
        del tensors
        prompt_len = min(rec["n_prompt"], max_prompt)
        cm.new_cache(prompt_len + steps + 1)
        prompt = synth.uniform_ids(rec["prompt_seed"], rec["n_prompt"], cfg["vocab_size"])[:prompt_len]
        t0 = time.perf_counter()
        logits = cm.forward_cached(prompt)
        t1 = time.perf_counter()
        ids = []
        for _ in range(steps):
            nxt = int(np.argmax(logits))
            ids.append(nxt)
            logits = cm.forward_cached(np.array([nxt], np.int32))
        t2 = time.perf_counter()
        same = ids == list(rec["ids"][:steps]) if prompt_len == rec["n_prompt"] else None
        sampled_same = None
        want = runs[key].get("sampled", {}).get("ids_first16")
        if prompt_len == rec["n_prompt"] and want is not None:
            # The same 16 sampled steps on the CPU: forward_cached, then the
            # restated sample() with the GPU run's draws.
            cm.new_cache(prompt_len + steps + 1)
            targets = sampling_targets(rec["n_steps"])
            logits = cm.forward_cached(prompt)
            got = []
            for i in range(min(steps, len(want))):
                nxt = O.oracle().sample_target(logits, *SAMPLING_CFG, targets[i])
                got.append(nxt)
                logits = cm.forward_cached(np.array([nxt], np.int32))
            sampled_same = got == want[: len(got)]
        cm.close()
        runs[key].update(cpu_kind="reference" if use_ref else "port", cpu_threads=cpu.pool_workers() + 1,
                         cpu_sample=f"prompt {prompt_len} ids, {steps} greedy steps (load/quantize {load_s:.1f} s)",
                         cpu_prefill_tok_s=round(prompt_len / (t1 - t0), 1),
                         cpu_decode_tok_s=round(steps / (t2 - t1), 2), cpu_ids_match=same,
                         cpu_sampled_ids_match=sampled_same)
        print(f"[bench] {key} CPU: decode {steps / (t2 - t1):.2f} tok/s", file=sys.stderr, flush=True)


def pick_cpu(max_threads: int = 16):
    """The CPU implementation timed beside the GPU: the reference compiled
    from its sources (oracle/_ref) when its pool (hardware_concurrency() - 1
    workers, thread_pool.cpp) stays within `max_threads`, else the oracle's
    restatement with a pool of max_threads - 1 workers."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    ref = O.reference()
    if ref is not None and ref.pool_workers() + 1 <= max_threads:
        return O, ref, "reference"
    cpu = O.oracle()
    cpu.set_pool_workers(max_threads - 1)
    return O, cpu, "port"


def host_info():
    """The CPU the baselines ran on: model string, os.cpu_count(), the CPUs
    this process may run on, and std::thread::hardware_concurrency() (the
    reference's pool size + 1)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    ref = O.reference()
    return dict(cpu_model=model, os_cpu_count=os.cpu_count(), affinity_cpus=len(os.sched_getaffinity(0)),
                hardware_concurrency=None if ref is None else ref.pool_workers() + 1,
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def timed_calls(fn, seconds: float, min_calls: int = 3) -> float:
    """Seconds per call of fn() over at least `seconds` and `min_calls`."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds and n >= min_calls:
            return dt / n


def cpu_per_shape(seconds_per_leg: float = 0.25):
    """The reference's quant::matmul (a QuantizedMatrix kept alive between
    calls) on each per-shape row, Q8_0 and Q4_0, batch 1 and 8; and C5's
    dominant shape, gate_proj 4864x896 Q8_0 at M = 512."""
    O, cpu, kind = pick_cpu()
    res = {"kind": kind, "threads": cpu.pool_workers() + 1}
    for name, out, n_in in REF_SHAPES:
        row = {}
        for qt in (H.Q8_0, H.Q4_0):
            data, scales = cpu.quantize(synth.normal(600 + out, out * n_in, 0.0, 0.02), out, n_in, qt)
            qm = cpu.qmatrix(data, scales, out, n_in, qt)
            wb = weight_bytes_of(out, n_in, qt)
            entry = {}
            for batch in (1, 8):
                x = synth.normal(601 + batch, batch * n_in, 0.0, 1.0)
                y = np.zeros(batch * out, np.float32)
                sec = timed_calls(lambda: qm.matmul(x, batch, y), seconds_per_leg)
                entry[f"b{batch}"] = dict(us=round(sec * 1e6, 2),
                                          gbs=round((wb + 4 * batch * (n_in + out)) / sec / 1e9, 2),
                                          weight_gbs=round(wb / sec / 1e9, 2))
            qm.close()
            row[H.TYPE_NAMES[qt]] = entry
        res[f"{name}_{out}x{n_in}"] = row
    out, n_in, M = 4864, 896, 512
    data, scales = cpu.quantize(synth.normal(602, out * n_in, 0.0, 0.02), out, n_in, H.Q8_0)
    qm = cpu.qmatrix(data, scales, out, n_in, H.Q8_0)
    x = synth.normal(603, M * n_in, 0.0, 1.0)
    y = np.zeros(M * out, np.float32)
    sec = timed_calls(lambda: qm.matmul(x, M, y), 1.0, min_calls=2)
    qm.close()
    res["c5_gate_proj_4864x896_q8_0_m512"] = dict(ms=round(sec * 1e3, 2),
                                                  gflops=round(2.0 * M * out * n_in / sec / 1e9, 2))
    return res


def cpu_baseline(seconds_budget: float = 12.0, max_threads: int = 16):
    """The reference's threaded CPU quant::matmul (oracle/_ref, built from the
    reference sources) -- or, where its pool would exceed `max_threads`, the
    oracle's restatement with a pool of that size -- on full passes over the
    same SmolLM2 Q4_0 linear layers at batch 1, each matrix wrapped once
    (a QuantizedMatrix kept alive) so a pass times quant::matmul alone."""
    O, cpu, kind = pick_cpu(max_threads)
    shapes = SMOL_LAYER + [SMOL_HEAD]
    mats = []
    for j, (_, out, n_in) in enumerate(shapes):
        w = synth.normal(4000 + j, out * n_in, 0.0, 0.02)
        data, scales = cpu.quantize(w, out, n_in, O.Q4_0)
        x = synth.normal(5000 + j, n_in, 0.0, 1.0)
        mats.append((cpu.qmatrix(data, scales, out, n_in, O.Q4_0), x, np.zeros(out, np.float32)))
    layer_bytes = sum(algo_bytes(o, i, H.Q4_0, 1) for _, o, i in SMOL_LAYER)
    head_bytes = algo_bytes(SMOL_HEAD[1], SMOL_HEAD[2], H.Q4_0, 1)

    def one_pass():
        for _ in range(N_LAYERS):
            for qm, x, y in mats[:-1]:
                qm.matmul(x, 1, y)
        qm, x, y = mats[-1]
        qm.matmul(x, 1, y)

    one_pass()  # warm-up
    t0 = time.perf_counter()
    passes = 0
    while True:
        one_pass()
        passes += 1
        if time.perf_counter() - t0 >= seconds_budget:
            break
    dt = time.perf_counter() - t0
    for qm, _, _ in mats:
        qm.close()
    step_bytes = N_LAYERS * layer_bytes + head_bytes
    threads = cpu.pool_workers() + 1
    return dict(value=round(passes * step_bytes / dt / 1e9, 3), unit="GB/s", cores=threads, kind=kind,
                sample=f"{passes} full passes of the 211 SmolLM2 Q4_0 matvecs (batch 1), {dt:.1f} s",
                ms_per_step=round(1e3 * dt / passes, 2))


def cpu_leg_8():
    """The cpu_baseline workload on CPUs 0-7 only (as `taskset -c 0-7`), 8
    threads: comparable with the 8-CPU container the reference's fixtures
    were recorded in.  Runs in a child process started before this process
    touches the GPU."""
    cpus = {c for c in range(8) if c in os.sched_getaffinity(0)}
    os.sched_setaffinity(0, cpus)
    r = cpu_baseline(seconds_budget=6.0, max_threads=8)
    r["affinity"] = sorted(cpus)
    print(json.dumps(r), flush=True)


def cpu_legs_before_gpu():
    """Every CPU leg that needs no GPU result, run before this process
    initialises the GPU (the 8-CPU leg is a child process)."""
    import subprocess

    res = {"host": host_info()}
    try:
        child = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg-8"], capture_output=True,
                               text=True, timeout=300)
        res["taskset_0_7"] = json.loads(child.stdout.strip().splitlines()[-1]) if child.returncode == 0 else {
            "error": child.stderr[-300:]}
    except (subprocess.SubprocessError, ValueError, IndexError) as e:
        res["taskset_0_7"] = {"error": str(e)}
    res["per_shape"] = cpu_per_shape()
    res["baseline"] = cpu_baseline()
    print(f"[bench] CPU: {res['baseline']['value']} GB/s ({res['baseline']['cores']} threads), 8 CPUs "
          f"{res['taskset_0_7'].get('value')} GB/s", file=sys.stderr, flush=True)
    return res


LINE_LIMIT = 4096  # characters of the final stdout line


def _pick(d, *keys):
    """The entries of dict d named by keys (those present)."""
    return {k: d[k] for k in keys if isinstance(d, dict) and k in d}


def ids_sha256(ids) -> str:
    """SHA-256 of a token-id list as little-endian int32 (the golden fixtures'
    convention for id lists)."""
    import hashlib

    return hashlib.sha256(np.asarray(ids, dtype="<i4").tobytes()).hexdigest()


def compact_line(full: dict, full_path: str | None = None) -> dict:
    """The one JSON line bench.py prints: the contract's fields, the roofline
    and CPU baseline, and one summary per measured workload.  The per-shape
    table, id lists and sampling detail stay in the full record (written to
    `full_path`), so the line stays under LINE_LIMIT characters."""
    cfg = full.get("config", {})
    line = {k: full[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                                 "higher_is_better", "scaling", "vs_baseline", "dtype", "data") if k in full}
    line["config"] = dict(_pick(cfg, "workload", "weights", "batch", "algorithmic_bytes_per_step",
                                "rotating_weight_copies", "pct_hbm_peak"),
                          sustained_b1=_pick(cfg.get("sustained_b1") or {}, "seconds", "us_per_step", "gbs"),
                          batch8=cfg.get("batch8"),
                          lm_head_single_launch=cfg.get("lm_head_single_launch"))
    line["roofline"] = _pick(full.get("roofline", {}), "kernel", "bound", "achieved", "peak", "unit", "frac",
                             "traffic", "algorithmic_bytes_per_launch", "mean_launch_us")
    cpu = full.get("cpu_baseline")
    line["cpu_baseline"] = None if cpu is None else dict(
        _pick(cpu, "value", "unit", "cores", "kind", "sample"),
        cpu_model=(cpu.get("host") or {}).get("cpu_model"),
        taskset_0_7_gbs=(cpu.get("taskset_0_7") or {}).get("value"))
    c1 = full.get("c1_q8_0_1536x576")
    if c1:
        line["c1_q8_0_1536x576_b1"] = dict(_pick(c1.get("b1", {}), "us", "gbs", "pct_hbm_peak"),
                                          cpu_us=(c1.get("cpu") or {}).get("b1", {}).get("us"))
    tol = full.get("tolerance_mode") or {}
    if tol:
        line["tolerance_mode_c2"] = dict(b1_pct=tol.get("c2_b1", {}).get("pct_hbm_peak"),
                                         b8_pct=tol.get("c2_b8", {}).get("pct_hbm_peak"),
                                         max_rel_error=tol.get("max_rel_error_vs_exact"))
    tq = full.get("targets_qwen25") or {}
    if tq:
        line["targets_qwen25_pct_hbm_peak"] = {k.replace("qwen_", ""): v.get("pct_hbm_peak") for k, v in tq.items()}
    dec = {}
    for key, r in (full.get("decode") or {}).items():
        gj = r.get("generate_json") or {}
        dec[key] = dict(_pick(r, "decode_tok_s", "frac_of_roofline", "ids_match_reference", "prefill_ms",
                              "cpu_decode_tok_s", "cpu_kind", "cpu_threads"),
                        generated_ids_sha256=ids_sha256(gj["generated_ids"]) if "generated_ids" in gj else None)
        smp = (r.get("sampled") or {}).get("t0.8_k40_p0.9")
        if smp:
            dec[key]["sampled_tok_s"] = smp.get("decode_tok_s")
    if dec:
        line["decode"] = dec
    dtol = full.get("decode_tolerance_mode") or {}
    if dtol:
        line["decode_tolerance_mode"] = {k: _pick(r, "decode_tok_s", "frac_of_roofline", "ids_match_first64",
                                                  "ids_match_reference", "max_rel_logit_err")
                                         for k, r in dtol.items()}
    g = full.get("prefill_gemm_c5") or {}
    if g:
        line["prefill_gemm_c5"] = {m: _pick(g[m], "ms", "tflops", "frac_of_mfma_peak") for m in ("per_layer", "one_launch")
                                   if m in g}
    if full_path:
        line["full_record"] = os.path.relpath(os.path.abspath(full_path), ROOT)
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-targets", action="store_true", help="skip the Qwen2.5 shape table")
    ap.add_argument("--no-decode", action="store_true", help="skip the full-model decode runs")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM (configs[4])")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one plain 256 MiB device-to-device copy, the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--no-graphs", action="store_true",
                    help="plain launches only: the linear pass's graph leg and the tolerance-mode greedy decode's "
                         "graph replay are skipped (for profilers that do not follow graphs)")
    ap.add_argument("--no-shapes", action="store_true", help="skip the per-shape table (C1, C2 shapes)")
    ap.add_argument("--decode-steps", type=int, default=None,
                    help="cap the greedy decode runs at this many steps (profiling; ids checked as a prefix)")
    ap.add_argument("--sustain-seconds", type=float, default=5.0,
                    help="run the headline launches back to back for about this long before the timed steps, "
                         "reported as config.sustained_b1 (0: skip)")
    ap.add_argument("--greedy-only", action="store_true",
                    help="decode runs without the sampled decode and the perplexity chunk (profiling)")
    ap.add_argument("--full-record", default=os.path.join(ROOT, "gpurun_out", "bench_full.json"),
                    help="where to write the full record (per-shape table, id lists, sampling detail); '' to skip")
    ap.add_argument("--cpu-leg-8", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_leg_8:
        cpu_leg_8()
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "it has no multi-GPU path to measure", file=sys.stderr)
        sys.exit(2)

    cpu_early = None if args.no_cpu else cpu_legs_before_gpu()
    H.init(0)
    shapes = step_shapes()
    bytes_b1 = sum(algo_bytes(o, i, H.Q4_0, 1) for _, o, i in shapes)
    bytes_b8 = sum(algo_bytes(o, i, H.Q4_0, 8) for _, o, i in shapes)
    weight_bytes = sum(o * H.row_bytes(i, H.Q4_0) + 4 * o * H.nblocks(i) for _, o, i in shapes)
    copies = max(2, -(-ROTATE_BYTES // weight_bytes))
    print(f"[bench] building {copies} copies of the SmolLM2 Q4_0 linears ({weight_bytes / 1e6:.1f} MB each)",
          file=sys.stderr, flush=True)
    wset = WeightSet(shapes, H.Q4_0, copies, 1)

    # The headline's W + K launches follow a sustained run of the same
    # launches (~sustain_seconds of GPU time, its own rate reported beside
    # `value`): the K steps are then timed at the clocks a busy GPU runs at,
    # not on a GPU just woken from idle.
    sustained = None
    if args.sustain_seconds > 0:
        probe = time_steps(wset, 1, 50, 5, mode="group") / 50
        n_sus = max(1, int(args.sustain_seconds / (probe * 1e-3)))
        ms_b1, sus_ms = time_steps(wset, 1, args.steps, args.warmup, mode="group", sustain=n_sus)
        sus_us = sus_ms / n_sus * 1e3
        sustained = {"steps": n_sus, "seconds": round(sus_ms * 1e-3, 2), "us_per_step": round(sus_us, 3),
                     "gbs": round(bytes_b1 / (sus_us * 1e-6) / 1e9, 1),
                     "launches_before_headline": 55 + n_sus}  # the 5 + 50 probe launches, then the sustained
        print(f"[bench] sustained b1 over {sustained['seconds']} s: {sus_us:.2f} us/step, {sustained['gbs']} GB/s",
              file=sys.stderr, flush=True)
    else:
        ms_b1 = time_steps(wset, 1, args.steps, args.warmup, mode="group")
    ms_b8 = time_steps(wset, 8, max(1, args.steps // 4), args.warmup, mode="group")
    ms_b1_tol = time_steps(wset, 1, args.steps, args.warmup, mode="tol")
    ms_b8_tol = time_steps(wset, 8, max(1, args.steps // 4), args.warmup, mode="tol")
    n_single = max(1, args.steps // 10)
    ms_b1_graph = None if args.no_graphs else time_steps(wset, 1, n_single, 2, mode="graph")
    ms_b1_plain = time_steps(wset, 1, n_single, 2, mode="plain")
    step_ms = ms_b1 / args.steps
    value = bytes_b1 / (step_ms * 1e-3) / 1e9
    b8_step_ms = ms_b8 / max(1, args.steps // 4)
    print(f"[bench] grouped b1 {step_ms * 1e3:.1f} us/step {value:.1f} GB/s; b8 {b8_step_ms * 1e3:.1f} us/step",
          file=sys.stderr, flush=True)

    tol_b1_us = ms_b1_tol / args.steps * 1e3
    tol_b8_us = ms_b8_tol / max(1, args.steps // 4) * 1e3
    print(f"[bench] tolerance mode b1 {tol_b1_us:.1f} us/step; b8 {tol_b8_us:.1f} us/step", file=sys.stderr, flush=True)
    tol_err = tolerance_check(wset)

    heads = [ws[-1] for ws in wset.copies]
    head_ms = time_launches(heads, 1, 2 * len(heads) * 4)
    head_bytes = algo_bytes(SMOL_HEAD[1], SMOL_HEAD[2], H.Q4_0, 1)
    wset.free()

    if args.calibrate_copy:
        nbytes = 256 << 20
        src, dst = H.DeviceBuffer(nbytes), H.DeviceBuffer(nbytes)
        H.synth_normal_dev(src, nbytes // 4, 1, 0.0, 1.0)
        H.synchronize()
        H.check(H.init().llmi_hip_memcpy_d2d(dst.ptr, src.ptr, nbytes, None))
        H.synchronize()
        print(f"[bench] calibration copy: {nbytes} bytes read and written", file=sys.stderr, flush=True)
        src.free()
        dst.free()

    per_shape = {} if args.no_shapes else per_shape_gpu()
    targets = {} if args.no_targets else target_shapes()
    decode = {} if args.no_decode else decode_runs(args.decode_steps, args.greedy_only, not args.no_graphs)
    decode_tol = {k: r.pop("tolerance_mode") for k, r in decode.items() if "tolerance_mode" in r}
    gemm = {} if args.no_gemm else prefill_gemm()
    gguf = gguf_upload()
    cpu = None
    if cpu_early is not None:
        cpu = dict(cpu_early["baseline"], host=cpu_early["host"], taskset_0_7=cpu_early["taskset_0_7"])
        for key, row in cpu_early["per_shape"].items():
            if key in per_shape:
                for t, entry in row.items():
                    per_shape[key].setdefault(t, {})["cpu"] = entry
        per_shape["cpu_kind"] = cpu_early["per_shape"]["kind"]
        per_shape["cpu_threads"] = cpu_early["per_shape"]["threads"]
        if gemm:
            gemm["cpu_gate_proj_m512"] = cpu_early["per_shape"]["c5_gate_proj_4864x896_q8_0_m512"]
    if decode and not args.no_cpu:
        cpu_decode(decode)
    c1 = per_shape.get("mlp_up_gate_1536x576", {}).get("q8_0")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (synth-v1 N(0,0.02) weights quantized on the GPU, N(0,1) activations)",
        "config": {
            "workload": "BASELINE.json configs[1]: all SmolLM2-135M-shaped linear layers (30x q,k,v,o,gate,up,down "
                        "+ tied 49152x576 lm_head) as Q4_0 matvec, batch 1; the 211 products of a step run as one "
                        "grouped launch (llmi_hip_group)",
            "weights": "q4_0",
            "batch": 1,
            "algorithmic_bytes_per_step": bytes_b1,
            "rotating_weight_copies": copies,
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "sustained_b1": sustained,
            "batch8": {"us_per_step": round(b8_step_ms * 1e3, 2),
                       "gbs": round(bytes_b8 / (b8_step_ms * 1e-3) / 1e9, 2)},
            "single_launches_b1": {
                "graph_us_per_step": None if ms_b1_graph is None else round(ms_b1_graph / n_single * 1e3, 2),
                "plain_us_per_step": round(ms_b1_plain / n_single * 1e3, 2),
            },
            "lm_head_single_launch": {"us": round(head_ms * 1e3, 3),
                                      "gbs": round(head_bytes / (head_ms * 1e-3) / 1e9, 1)},
        },
        "c1_q8_0_1536x576": None if c1 is None else dict(
            c1, workload="BASELINE.json configs[0]: one Q8_0 1536x576 matvec (SmolLM2 up/gate), batch 1; "
                         "b8 = the same at batch 8"),
        "per_shape": per_shape,
        "roofline": {
            "kernel": "qgemv_group (one launch = the 211 SmolLM2 Q4_0 matvecs of a step), batch 1",
            "bound": "hbm",
            "achieved": round(value, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "traffic_source": f"rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE of {HEADLINE_KERNEL}, {TRAFFIC_PROFILE}",
            "algorithmic_bytes_per_launch": bytes_b1,
            "mean_launch_us": round(step_ms * 1e3, 3),
        },
        "tolerance_mode": {
            "what": "the same products through llmi_hip_tol_group (Q4_0 on the matrix cores, another summation "
                    "order): the fp32-accumulate contract max|y - y_ref| <= 1e-4 * max|y_ref|, not bit-exact; the "
                    "exact path above stays the default and the value of this line",
            "c2_b1": {"us_per_step": round(tol_b1_us, 2), "gbs": round(bytes_b1 / tol_b1_us / 1e3, 1),
                      "pct_hbm_peak": round(100 * bytes_b1 / tol_b1_us / 1e3 / HBM_PEAK_GBS, 1)},
            "c2_b8": {"us_per_step": round(tol_b8_us, 2), "gbs": round(bytes_b8 / tol_b8_us / 1e3, 1),
                      "pct_hbm_peak": round(100 * bytes_b8 / tol_b8_us / 1e3 / HBM_PEAK_GBS, 1)},
            "max_rel_error_vs_exact": tol_err,
            "roofline": {"kernel": "qgemv_tol_small<1> (the 211 products of a step), batch 1", "bound": "hbm",
                         "achieved": round(bytes_b1 / tol_b1_us / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(bytes_b1 / tol_b1_us / 1e3 / HBM_PEAK_GBS, 4)},
        },
        "targets_qwen25": targets,
        "decode": decode,
        "prefill_gemm_c5": gemm,
        "gguf_to_device": gguf,
        "cpu_baseline": cpu,
    }
    line["decode_tolerance_mode"] = decode_tol
    path = args.full_record
    if path:
        os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
        with open(path, "w") as f:
            json.dump(line, f, indent=1)
        print(f"[bench] full record written to {path}", file=sys.stderr, flush=True)
    print(json.dumps(compact_line(line, path)), flush=True)


if __name__ == "__main__":
    main()
