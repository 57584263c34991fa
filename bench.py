#!/usr/bin/env python3
"""MoE-layer throughput on one MI355X.

Workload (the single-layer decode configuration): one MoE layer, T=1 token
per step, hidden 2048, 512 experts, top-10 + shared expert, Q2 experts
(64-weight fp16-scale groups, 884,736-byte blobs), f32 activations,
RMSNorm'd N(0,1) inputs. 48 independent layers (21.7 GB of expert blobs) stay
resident in HBM and successive steps rotate through them, so a step never
finds its weights in the 256 MB Infinity Cache. A step is one token through
one layer: device routing, gate/up, down and combine, no host round trip.

Timing: W untimed warm-up steps, then exactly K steps (K/48 replays of a HIP
graph holding 48 steps, plus a partial graph if K is not a multiple of 48),
bracketed by a device synchronisation on both sides; value = K / seconds.

roofline: the dominant decode kernel's algorithmic bytes per launch divided by
its average duration, from graphs that run only that stage (HIP events on the
library's stream around the replays); peak = 8 TB/s HBM. traffic (HBM bytes
per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated) is
read from profiles/traffic.json when present.

prefill: T=512 (uniform routing) and T=2048 (Zipf(1.1) router prior) through
the grouped-MFMA path, per-stage times from events, reported beside the main
line. stack: the 48 resident layers chained (RMSNorm, MoE layer, residual) for
128 steps at batch 1 and batch 32, one HIP graph per step. real_model: the
real model's geometry (hidden 2560, ff 640) through the same kernels, decode
T=1 over 16 rotated resident layers and prefill T=512 / T=2048 (Zipf).
cpu_baseline: the CPU oracle (a restatement of the reference kernels in
their operation order, OpenMP over workgroups) on the host cores, T=1 decode
of a bounded token sample of the same layer.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer tok/s (T=1 decode, T=512 prefill); % HBM GB/s / % MFMA roofline"
PEAK_HBM = 8.0e12         # bytes/s, MI355X HBM3E
PEAK_MFMA_F16 = 2.5e15    # dense fp16/bf16 MFMA FLOP/s


def decode_kernel_bytes(W, F, E, K):
    """Algorithmic bytes per launch of each decode kernel (weights streamed +
    inputs read + outputs written; logits/hidden intermediates excluded)."""
    gu_blob = 2 * F * W // 4 + 2 * F * (W // 64) * 2
    dn_blob = W * F // 4 + W * (F // 64) * 2
    xq = (W // 64) * 256                                            # fixed-point activations
    return {
        "decode_route": E * W * 4 + W * 4 + W * 4 + xq + 4,              # W_r, w_sg, x; x records, gate
        "decode_gate_up": (K + 1) * gu_blob + xq + K * 8,                # 10 routed + shared gate/up planes
        "decode_down_combine": (K + 1) * dn_blob + W * 4 + K * 8,        # 11 down planes; y; ids, weights
    }


def layer_bytes(W, F, E, K, T, distinct):
    """Algorithmic bytes of one layer launch: distinct expert blobs touched +
    shared blob + router and gate weights + inputs and outputs."""
    blob = 2 * F * W // 4 + W * F // 4 + 2 * F * (W // 64) * 2 + W * (F // 64) * 2
    return distinct * blob + blob + E * W * 4 + W * 4 + 2 * T * W * 4


def layer_flops(W, F, E, K, T):
    return T * ((K + 1) * 3 * 2 * W * F + 2 * E * W)


def real_model(be, wl, np, capture, replay, release, layers=16, steps=960, prefill_reps=4, prefetch=True):
    """The real model's geometry (hidden 2560, expert ff 640, 512 experts,
    top-10 + shared, 1,382,400-byte Q2 blobs) through the same kernels:
    decode T=1 rotating through `layers` resident layers (HIP graphs), the
    decode kernels one stage at a time, and prefill T=512 / T=2048 (Zipf)."""
    W, F, E, K = 2560, 640, 512, 10
    lays = [wl.DeviceLayer(be, l, width=W, ff=F, experts=E, base_seed=wl.BASE_SEED + 1) for l in range(layers)]
    slots = []
    for i in range(layers):
        x = be.alloc(W, zero=False)
        be.synth_normal(x, W, lays[i].seed + 99, wl.STREAM_INPUT, 1.0)
        slots.append({"x": x, "y": be.alloc(W), "ids": be.alloc(K, "i32"), "w": be.alloc(K),
                      "ws": be.alloc_bytes(be.moe_workspace_bytes(1, W, F, E, K))})

    def step(i):
        s, lay = slots[i], lays[i]
        if prefetch:
            be.prefetch_router(lays[(i + 1) % layers].Wr, E, W)
        be.moe_layer(s["x"], 1, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, s["y"], s["ids"],
                     s["w"], s["ws"])

    def all_layers():
        for i in range(layers):
            step(i)

    all_layers()
    be.sync()
    g = capture(all_layers)
    replay(g)
    be.sync()
    be.event_record(8)
    for _ in range(steps // layers):
        replay(g)
    be.event_record(9)
    be.sync()
    release(g)
    us = be.event_elapsed_ms(8, 9) * 1e3 / (steps // layers * layers)
    step_bytes = layer_bytes(W, F, E, K, 1, K)
    out = {"workload": "single MoE layer, hidden 2560, ff 640, 512 experts, top-10 + shared, Q2 (1,382,400-byte "
                       "blobs), %d resident layers rotated" % layers,
           "decode_T1": {"tokens_per_s": round(1e6 / us, 1), "us_per_step": round(us, 3),
                         "execution": "one k_decode_fused launch per layer (kernels: the three-kernel path's stages, "
                                      "each alone)",
                         "hbm": {"bytes_per_step": step_bytes, "frac": round(step_bytes / (us * 1e-6) / PEAK_HBM, 4)}}}
    kb = decode_kernel_bytes(W, F, E, K)
    kern = {}
    for stage, name in enumerate(["decode_route", "decode_gate_up", "decode_down_combine"]):
        be.stage_select(1 << stage)
        gid = capture(all_layers)
        be.stage_select()
        be.stage_select(1 << stage)
        replay(gid)
        be.sync()
        be.event_record(8)
        for _ in range(20):
            replay(gid)
        be.event_record(9)
        be.sync()
        be.stage_select()
        kus = be.event_elapsed_ms(8, 9) * 1e3 / (20 * layers)
        kern[name] = {"avg_us": round(kus, 3), "frac_hbm": round(kb[name] / (kus * 1e-6) / PEAK_HBM, 4)}
        release(gid)
    out["decode_T1"]["kernels"] = kern
    for T, zipf in [(512, False), (2048, True)]:
        X = be.alloc(T * W, zero=False)
        be.synth_normal(X, T * W, wl.BASE_SEED + 5 + T, wl.STREAM_INPUT, 1.0)
        bias = be.alloc(wl.zipf_bias(E, lays[0].seed)) if zipf else None
        Y, ids, w = be.alloc(T * W), be.alloc(T * K, "i32"), be.alloc(T * K)
        ws = be.alloc_bytes(be.moe_workspace_bytes(T, W, F, E, K))

        def run(j):
            lay = lays[j % layers]
            be.moe_layer(X, T, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, Y, ids, w, ws,
                         bias=bias)

        for j in range(2):
            run(j)
        be.sync()
        gp = capture(lambda: [run(j) for j in range(prefill_reps)])
        replay(gp)
        be.sync()
        be.event_record(8)
        replay(gp)
        be.event_record(9)
        be.sync()
        release(gp)
        ms = be.event_elapsed_ms(8, 9) / prefill_reps
        distinct = len(np.unique(be.read(ids)))
        lb, lf = layer_bytes(W, F, E, K, T, distinct), layer_flops(W, F, E, K, T)
        cert = be.route_stats(ws, T, W, F, E, K)
        out["prefill T=%d%s" % (T, " zipf" if zipf else "")] = {
            "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_layer": round(ms, 4), "distinct_experts": int(distinct),
            "hbm_frac": round(lb / (ms * 1e-3) / PEAK_HBM, 4), "mfma_layer_frac": round(lf / (ms * 1e-3) / PEAK_MFMA_F16, 4),
            "route_candidates_per_token": round(cert[0] / T, 2) if cert else None,
            "route_fallback_tokens": cert[1] if cert else None}
        for b in (X, Y, ids, w, ws) + ((bias,) if bias is not None else ()):
            be.free(b)
    for s_ in slots:
        for b in s_.values():
            be.free(b)
    for lay in lays:
        lay.free()
    return out


def dense_formats(be, np, capture, replay, release, cols=2560, rows=10240, reps=200):
    """Dense-format projections at the real model's width, one token (GEMV):
    strata_bf16_project and strata_quant_gemv (S4, S8; group 32, offsets),
    each over enough distinct weight copies (> 256 MiB) that every launch
    reads its weights from HBM. Algorithmic bytes: the weights (codes +
    scales + offsets) + x + y."""
    out = {}
    rng = np.random.default_rng(7)
    x = be.alloc(rng.normal(0, 1, cols).astype(np.float32))
    y = be.alloc(rows)
    w = rng.normal(0, 0.05, rows * cols).astype(np.float32)
    hi = (w.view(np.uint32) >> 16).astype(np.uint32)
    del w
    bf16 = (hi[0::2] | (hi[1::2] << 16)).astype(np.uint32)
    del hi
    gs = 32
    cases = [("bf16_project", "strata_bf16_project", bf16, None)]
    for bits in (4, 8):
        codes = rng.integers(0, 2 ** 32, rows * cols * bits // 32, dtype=np.uint64).astype(np.uint32)
        cases.append(("quant_gemv_s%d" % bits, "strata_quant_gemv", codes, bits))
    for label, kernel, codes, bits in cases:
        wbytes = codes.nbytes + (0 if bits is None else 2 * 4 * rows * cols // gs)
        copies = max(2, -(-(320 << 20) // wbytes))
        bufs = []
        for _ in range(copies):
            if bits is None:
                bufs.append({"Codes": be.alloc(codes, "u32")})
            else:
                bufs.append({"Codes": be.alloc(codes, "u32"),
                             "Scales": be.alloc(rng.normal(0, 0.02, rows * cols // gs).astype(np.float32)),
                             "Offsets": be.alloc(rng.normal(0, 0.01, rows * cols // gs).astype(np.float32))})

        def launch(i, b=bufs, kernel=kernel, bits=bits):
            a = dict(b[i % len(b)], X=x, Y=y, cols=cols, rows=rows)
            if bits is None:
                a.update(tokens=1, outputStride=rows, outputOffset=0)
                be.run(kernel, a, [rows, 1, 1])
            else:
                a.update(bits=bits, groupSize=gs, bias=-(1 << (bits - 1)), codebook=0, hasOffset=1)
                be.run(kernel, a, [rows, 1, 1])

        gid = capture(lambda: [launch(i) for i in range(reps)])
        replay(gid)
        be.sync()
        be.event_record(8)
        for _ in range(3):
            replay(gid)
        be.event_record(9)
        be.sync()
        us = be.event_elapsed_ms(8, 9) * 1e3 / (3 * reps)
        nbytes = wbytes + cols * 4 + rows * 4
        out[label] = {"cols": cols, "rows": rows, "avg_us": round(us, 3), "bytes_per_launch": nbytes,
                      "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac_hbm": round(nbytes / (us * 1e-6) / PEAK_HBM, 4),
                      "weight_copies": copies}
        release(gid)
        for b in bufs:
            for v in b.values():
                be.free(v)
    be.free(x)
    be.free(y)
    return out


def prompt_kernels(be, np, capture, replay, release, tokens=16, reps=50):
    """The prompt-batch kernels at production shapes for one chunk of 16
    tokens: GDN state update (128-wide keys, 16 key / 48 value heads), the
    causal attention of the chunk at cells 2032-2047 (24 heads of 256, 2 KV
    heads) and the 4-tap convolution over the GDN projection's 10240 channels.
    Algorithmic bytes: state or cache read (and state written) once, plus
    the chunk's inputs and outputs. Each launch reuses the same few MB, so
    they are served from the 256 MiB Infinity Cache; frac_hbm only scales
    the rate against the HBM peak."""
    out = {}
    rng = np.random.default_rng(5)
    T = tokens
    dim, kh, vh = 128, 16, 48
    state = be.alloc(rng.normal(0, 0.1, dim * vh * dim).astype(np.float32))
    q = be.alloc((rng.normal(0, 1, T * kh * dim) / np.sqrt(dim)).astype(np.float32))
    k = be.alloc((rng.normal(0, 1, T * kh * dim) / np.sqrt(dim)).astype(np.float32))
    v = be.alloc(rng.normal(0, 1, T * vh * dim).astype(np.float32))
    dec = be.alloc(np.full(T * vh, 0.97, np.float32))
    beta = be.alloc(np.full(T * vh, 0.5, np.float32))
    y = be.alloc(T * vh * dim)
    gdn = lambda: be.run("strata_gdn_batch", {"State": state, "Q": q, "K": k, "V": v, "Decay": dec, "Beta": beta,
                                              "Y": y, "dim": dim, "keyHeads": kh, "valueHeads": vh, "tokens": T},
                         [(vh * dim + 63) // 64, 1, 1])
    gdn_bytes = 2 * dim * vh * dim * 4 + T * (2 * kh * dim + 2 * vh * dim + 2 * vh) * 4
    ad, heads, kvh, pos = 256, 24, 2, 2048 - T
    keys = be.alloc(rng.normal(0, 1, 2048 * kvh * ad).astype(np.float32))
    values = be.alloc(rng.normal(0, 1, 2048 * kvh * ad).astype(np.float32))
    aq = be.alloc(rng.normal(0, 1, T * heads * ad).astype(np.float32))
    ay = be.alloc(T * heads * ad)
    att = lambda: be.run("strata_attention_batch", {"Q": aq, "Keys": keys, "Values": values, "Y": ay, "dim": ad,
                                                    "heads": heads, "kvHeads": kvh, "position": pos,
                                                    "scale": 1 / 16.0}, [heads, ad // 64, T])
    att_bytes = 2 * 2048 * kvh * ad * 4 + 2 * T * heads * ad * 4
    ch = 2 * kh * dim + vh * dim
    hist = be.alloc(ch * 3)
    cx = be.alloc(rng.normal(0, 1, T * ch).astype(np.float32))
    cw = be.alloc(rng.normal(0, 0.5, ch * 4).astype(np.float32))
    cy = be.alloc(T * ch)
    conv = lambda: be.run("strata_conv_batch", {"History": hist, "X": cx, "W": cw, "Y": cy, "channels": ch, "taps": 4,
                                                "dilation": 1, "activation": 1, "tokens": T}, [(ch + 63) // 64, 1, 1])
    conv_bytes = 2 * ch * 3 * 4 + 2 * T * ch * 4 + ch * 4 * 4
    for label, fn, nbytes in (("gdn_batch", gdn, gdn_bytes), ("attention_batch", att, att_bytes),
                              ("conv_batch", conv, conv_bytes)):
        gid = capture(lambda: [fn() for _ in range(reps)])
        replay(gid)
        be.sync()
        be.event_record(8)
        for _ in range(3):
            replay(gid)
        be.event_record(9)
        be.sync()
        us = be.event_elapsed_ms(8, 9) * 1e3 / (3 * reps)
        out[label] = {"tokens": T, "avg_us": round(us, 3), "bytes_per_launch": nbytes,
                      "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                      "frac_hbm": round(nbytes / (us * 1e-6) / PEAK_HBM, 4)}
        release(gid)
    for b in (state, q, k, v, dec, beta, y, keys, values, aq, ay, hist, cx, cw, cy):
        be.free(b)
    return out


def prompt_orchestration(timeout=300):
    """The fixture prompt (24 tokens) through StrataEngine.prefill in chunks
    and through step() token by token, in a Node.js child process."""
    import shutil
    import subprocess
    node = shutil.which("node")
    if node is None:
        return {"skipped": "node not found"}
    here = os.path.dirname(os.path.abspath(__file__))
    r = subprocess.run([node, os.path.join(here, "stratacuda_amd", "src", "bench_prompt.js"), "24", "5"],
                       cwd=here, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError("bench_prompt.js failed:\n" + r.stdout[-2000:])
    return json.loads(r.stdout.strip().splitlines()[-1])


def read_traffic(kernel):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        data = json.load(open(path))
        return data.get(kernel)
    except (OSError, ValueError):
        return None


def cpu_info():
    """CPU model and the cores this process may use."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"model": model, "logical_cpus": os.cpu_count(), "usable_cpus": usable}


def cpu_baseline(oracle, wl, seconds, prefill=True):
    """The CPU oracle (the reference kernels restated in C in their f32
    operation order, OpenMP over workgroups) on the host cores, at the
    reference pool's default of 4 threads (src/backend.js:125) and its limit
    of 8 (vendor/webcuda/src/wasm/thread-pool.hpp:49-50): T=1 decode over a
    bounded token sample, one full T=512 layer at both counts and one full
    T=2048 (Zipf) layer at 8 threads. ``value`` is the 8-thread T=1 rate."""
    import numpy as np
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    host = wl.host_layer(oracle, 0)
    ones = np.ones(W, np.float32)
    args = (host["Wr"], host["arena"], host["stride"], host["shared"], host["Wsg"], W, F, E, K)
    legs = {}
    for threads in (8, 4):
        oracle.set_threads(threads)
        n, t0 = 0, time.perf_counter()
        while True:
            z = oracle.synth_normal(W, host["seed"] + 5000 + n, wl.STREAM_INPUT, 1.0)
            oracle.moe_layer(oracle.norm(z, ones, W, 1), 1, *args)
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds / 2 or n >= 4096:
                break
        legs["decode_T1_threads%d" % threads] = {"tokens_per_s": round(n / el, 2), "tokens": n,
                                                 "seconds": round(el, 2)}
    if prefill:
        cases = [(512, False, 8), (512, False, 4), (2048, True, 8)]
        for T, zipf, threads in cases:
            oracle.set_threads(threads)
            X = oracle.synth_normal(T * W, wl.layer_seed(0) + 7 + T, wl.STREAM_INPUT, 1.0)
            bias = wl.zipf_bias(E, host["seed"]) if zipf else None
            t0 = time.perf_counter()
            oracle.moe_layer(X, T, *args, bias=bias)
            el = time.perf_counter() - t0
            legs["prefill_T%d%s_threads%d" % (T, "_zipf" if zipf else "", threads)] = {
                "tokens_per_s": round(T / el, 2), "seconds": round(el, 2)}
    info = cpu_info()
    t1 = legs["decode_T1_threads8"]
    return {"value": t1["tokens_per_s"], "unit": "tokens/s", "cores": 8, "kind": "port",
            "sample": "%d single-token decodes (T=1) of one full-geometry MoE layer (hidden 2048, 512 experts, "
                      "top-10 + shared, Q2) in %.1f s at 8 OpenMP threads; the C restatement of the reference "
                      "kernels in their f32 operation order (the reference's threaded-WASM build cannot be made "
                      "here: it needs Emscripten and a Node >= 22 code generator)" % (t1["tokens"], t1["seconds"]),
            "threads": {"value": 8, "reference_default": 4, "reference_pool_limit": 8},
            "cpu": info, "legs": legs}


PROFILE_CMDS = {
    "trace": "rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/trace -o decode -- "
             "python3 -u bench.py --no-cpu --eager --no-stack --no-pack --no-prompt --steps 960",
    "fetch": "rocprofv3 --pmc FETCH_SIZE -f csv -d gpurun_out/pmc_fetch -o decode -- "
             "python3 -u bench.py --no-cpu --eager --no-prefill --no-stack --no-real --no-dense --no-pack --no-prompt "
             "--layers 8 --steps 16 --warmup 8",
    "write": "rocprofv3 --pmc WRITE_SIZE -f csv -d gpurun_out/pmc_write -o decode -- "
             "python3 -u bench.py --no-cpu --eager --no-prefill --no-stack --no-real --no-dense --no-pack --no-prompt "
             "--layers 8 --steps 16 --warmup 8",
    "cal_fetch": "rocprofv3 --pmc FETCH_SIZE -f csv -d gpurun_out/pmc_cal_fetch -o cal -- python3 -u bench.py --calibrate",
    "cal_write": "rocprofv3 --pmc WRITE_SIZE -f csv -d gpurun_out/pmc_cal_write -o cal -- python3 -u bench.py --calibrate",
}
for _case in ("512", "2048zipf"):
    PROFILE_CMDS["mfma_" + _case] = (
        "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_BUSY_CYCLES GRBM_GUI_ACTIVE "
        "-f csv -d gpurun_out/pmc_mfma_%s -o prefill -- python3 -u bench.py --no-cpu --eager --no-stack --no-real "
        "--no-dense --no-pack --no-prompt --layers 2 "
        "--steps 2 --warmup 2 --prefill-reps 4 --prefill-cases %s" % (_case, _case))
# FLOPs per MFMA instruction: v_mfma_f32_32x32x16_f16 (64-row and register-B
# kernels), v_mfma_f32_16x16x32_f16 (16-row kernels).
MFMA_FLOP_32 = 2 * 32 * 32 * 16
MFMA_FLOP_16 = 2 * 16 * 16 * 32
SIMDS = 256 * 4
DECODE_KERNELS = ["k_decode_fused", "k_decode_route", "k_decode_gate_up", "k_decode_down"]


def _csv_rows(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def _kernel_key(name):
    for k in DECODE_KERNELS + ["k_prefill_gate_up", "k_prefill_down", "k_prefill_route", "k_dispatch",
                               "k_prefill_combine", "k_elementwise", "strata_elementwise"]:
        if "::" + k + "(" in name or name.startswith(k + "(") or ("::" + k + "<") in name:
            return k
    return None


def _pmc_mean(path, counter, kernel):
    vals = [float(r["Counter_Value"]) for r in _csv_rows(path)
            if r["Counter_Name"] == counter and _kernel_key(r["Kernel_Name"]) == kernel]
    return sum(vals) / len(vals) if vals else None, len(vals)


def _gemm_label(name):
    """Readable name of a prefill kernel from its (possibly mangled) symbol."""
    import re
    m = re.search(r"k_moe_gemm_streamILb(\d)ELi(\d)ELi(\d)ELi(\d+)E", name)
    if m:
        return "k_moe_gemm_stream<%s, %d x %d tile, K/64 = %s>" % (
            "gate_up" if m.group(1) == "1" else "down", 32 * int(m.group(2)), 128 * int(m.group(3)), m.group(4))
    # 16-row kernels: weight rows per block 64 x NT (the rows16 kernel's third
    # template argument, 4 when absent), mangled or demangled
    m = re.search(r"k_moe_gemm_(stream16|rows16)ILb(\d)ELi(\d+)E(?:Li(\d)E)?", name)
    g = (m.group(1), m.group(2) == "1", m.group(3), m.group(4)) if m else None
    if not m:
        m = re.search(r"k_moe_gemm_(stream16|rows16)<(true|false), (\d+)(?:, (\d))?>", name)
        g = (m.group(1), m.group(2) == "true", m.group(3), m.group(4)) if m else None
    if g:
        return "k_moe_gemm_%s<%s, 16 x %d tile, K/64 = %s>" % (g[0], "gate_up" if g[1] else "down",
                                                              64 * int(g[3] or 4), g[2])
    m = re.search(r"k_split_hilo", name)
    if m:
        return "k_split_hilo"
    # a symbol the profiler left mangled (an anonymous-namespace kernel with
    # integer / bool template arguments): its name and arguments
    m = re.match(r"_ZN12_GLOBAL__N_1(\d+)", name)
    if m:
        rest = name[m.end():]
        base = rest[:int(m.group(1))]
        targs = re.match(r"I((?:L[ib]\d+E)+)E", rest[int(m.group(1)):])
        if targs:
            vals = re.findall(r"L([ib])(\d+)E", targs.group(1))
            base += "<%s>" % ", ".join(("true" if v == "1" else "false") if k == "b" else v for k, v in vals)
        return base
    return name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]


def summarize_mfma(path, case, dest):
    """MFMA use of the prefill kernels from one --pmc run: per kernel the
    dispatches, mean duration (dispatch timestamps), MFMA instructions, the
    FLOP/s they issue and SQ_VALU_MFMA_BUSY_CYCLES over all SIMDs at 2.4 GHz."""
    import collections
    per = collections.defaultdict(dict)
    for r in _csv_rows(path):
        d = per[r["Dispatch_Id"]]
        d["name"] = r["Kernel_Name"]
        d["ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        d[r["Counter_Name"]] = float(r["Counter_Value"])
    agg = collections.OrderedDict()
    for d in per.values():
        if "gemm" not in d["name"] and "k_combine" not in d["name"] and "dispatch" not in d["name"] \
                and "split_hilo" not in d["name"]:
            continue
        agg.setdefault(_gemm_label(d["name"]), []).append(d)
    lines = ["# MFMA use of the prefill kernels, T=%s" % case.replace("zipf", " (Zipf-biased router)"), "",
             "Command (from the repository root):", "", "    " + PROFILE_CMDS["mfma_" + case], "",
             "Issued rate = SQ_INSTS_MFMA x FLOP per instruction (%d for the 32x32x16 MFMA of the 64-row tiles, "
             "%d for the 16x16x32 MFMA of the 16-row tiles) / duration; each algorithmic product runs twice, "
             "once for the high and once for the low fp16 half of the activations, so the algorithmic rate is half "
             "of it. Busy = SQ_VALU_MFMA_BUSY_CYCLES / (%d SIMDs x duration x 2.4 GHz). Peak: 2.5 PFLOP/s dense fp16."
             % (MFMA_FLOP_32, MFMA_FLOP_16, SIMDS), "",
             "| kernel | dispatches | avg us | MFMA insts | issued TFLOP/s | issued / peak | MFMA busy | VALU insts |",
             "|---|---|---|---|---|---|---|---|"]
    for name, ds in agg.items():
        n = len(ds)
        us = sum(d["ns"] for d in ds) / n / 1e3
        mf = sum(d.get("SQ_INSTS_MFMA", 0) for d in ds) / n
        busy = sum(d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) for d in ds) / n
        va = sum(d.get("SQ_INSTS_VALU", 0) for d in ds) / n
        rate = mf * (MFMA_FLOP_16 if "16<" in name else MFMA_FLOP_32) / (us * 1e-6) / 1e12 if us else 0.0
        lines.append("| %s | %d | %.1f | %.0f | %.1f | %.3f | %.3f | %.0f |" % (
            name, n, us, mf, rate, rate * 1e12 / PEAK_MFMA_F16, busy / (SIMDS * us * 1e-6 * 2.4e9) if us else 0.0,
            va))
    open(dest, "w").write("\n".join(lines) + "\n")


def summarize(out_dir):
    """Turns the rocprofv3 CSVs of the profiling commands (PROFILE_CMDS, run
    with their output under out_dir) into the text summaries under profiles/:
    kernel durations, and HBM traffic per launch from FETCH_SIZE / WRITE_SIZE
    (KiB per dispatch) scaled by what the same counters read for the copy
    kernel of known size."""
    import glob
    prof = os.path.join(ROOT, "profiles")
    os.makedirs(prof, exist_ok=True)
    stats = glob.glob(os.path.join(out_dir, "trace", "*kernel_stats.csv"))
    lines = ["# Kernel durations: decode T=1 (48 rotated layers), prefill T=512 / T=2048, the real model's "
             "geometry (hidden 2560, ff 640) and the dense-format projections (2560 x 10240)", "",
             "Command (from the repository root):", "", "    " + PROFILE_CMDS["trace"], "",
             "| kernel | calls | avg us | min us | max us | share |", "|---|---|---|---|---|---|"]
    for r in _csv_rows(stats[0]):
        name = _gemm_label(r["Name"])
        lines.append("| %s | %s | %.3f | %.3f | %.3f | %s%% |" % (
            name, r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3,
            r["Percentage"]))
    open(os.path.join(prof, "kernel_stats_moe_layer.md"), "w").write("\n".join(lines) + "\n")
    cal_f, _ = _pmc_mean(glob.glob(os.path.join(out_dir, "pmc_cal_fetch", "*counter_collection.csv"))[0],
                         "FETCH_SIZE", "k_elementwise")
    cal_w, _ = _pmc_mean(glob.glob(os.path.join(out_dir, "pmc_cal_write", "*counter_collection.csv"))[0],
                         "WRITE_SIZE", "k_elementwise")
    copy_bytes = 64 * 1024 * 1024 * 4
    f_fac, w_fac = copy_bytes / (cal_f * 1024), copy_bytes / (cal_w * 1024)
    W, F, E, K = 2048, 512, 512, 10
    algo = decode_kernel_bytes(W, F, E, K)
    algo_by_kernel = {"k_decode_fused": sum(algo.values()), "k_decode_route": algo["decode_route"],
                      "k_decode_gate_up": algo["decode_gate_up"], "k_decode_down": algo["decode_down_combine"]}
    traffic, md = {}, ["# HBM traffic per launch: decode T=1 kernels (8 rotated layers: the single-launch "
                       "layer k_decode_fused and the three-kernel path; L2-miss bytes, durations not used)", "",
                       "Commands (from the repository root):", ""]
    md += ["    " + PROFILE_CMDS[k] for k in ("fetch", "write", "cal_fetch", "cal_write")]
    md += ["", "Calibration: the copy kernel (strata_elementwise, 256 MiB read + 256 MiB written per launch) "
           "reads FETCH_SIZE %.0f KiB and WRITE_SIZE %.0f KiB per dispatch, so FETCH_SIZE is scaled by %.3f and "
           "WRITE_SIZE by %.3f." % (cal_f, cal_w, f_fac, w_fac), "",
           "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic bytes | algorithmic bytes | ratio |",
           "|---|---|---|---|---|---|---|"]
    for k in DECODE_KERNELS:
        fk, n = _pmc_mean(glob.glob(os.path.join(out_dir, "pmc_fetch", "*counter_collection.csv"))[0],
                          "FETCH_SIZE", k)
        wk, _ = _pmc_mean(glob.glob(os.path.join(out_dir, "pmc_write", "*counter_collection.csv"))[0],
                          "WRITE_SIZE", k)
        if fk is None or wk is None:
            continue
        t = int(round(fk * 1024 * f_fac + wk * 1024 * w_fac))
        traffic[k] = t
        md.append("| %s | %d | %.1f | %.1f | %d | %d | %.2f |" % (k, n, fk, wk, t, algo_by_kernel[k],
                                                                 t / algo_by_kernel[k]))
    json.dump(traffic, open(os.path.join(prof, "traffic.json"), "w"), indent=1)
    for case in ("512", "2048zipf"):
        found = glob.glob(os.path.join(out_dir, "pmc_mfma_" + case, "*counter_collection.csv"))
        if found:
            summarize_mfma(found[0], case, os.path.join(prof, "mfma_prefill_T%s.md" % case))
    open(os.path.join(prof, "traffic_decode_T1.md"), "w").write("\n".join(md) + "\n")
    print(json.dumps({"summaries": sorted(os.listdir(prof)), "traffic": traffic}))


def routing_problems(be, slots, E, K, np):
    """Slots whose routed IDs are not K distinct experts in [0, E) or whose
    output holds a non-finite value."""
    bad = []
    for i, s in enumerate(slots):
        ids = be.read(s["ids"])
        if not (ids.min() >= 0 and ids.max() < E and len(set(ids.tolist())) == K) or \
                not np.all(np.isfinite(be.read(s["y"]))):
            bad.append(i)
    return bad


def warm_and_check(be, step, slots, warmup, capture, replay, E, K, np):
    """`warmup` untimed steps (rotating over the layers), then one untimed
    replay of the graph that runs every layer once, and only then the check
    of every slot's routing: a slot is checked after it has run."""
    L = len(slots)
    for s in range(warmup):
        step(s % L)
    g_full = capture(lambda: [step(i) for i in range(L)])
    replay(g_full)
    be.sync()
    bad = routing_problems(be, slots, E, K, np)
    if bad:
        raise RuntimeError("invalid routing or non-finite output in layer slots %s" % bad[:8])
    return g_full


def replay_times(be, replay, g, reps):
    """Durations in ms of `reps` replays of g, each between two events on the
    library's stream (event slots 10 .. 10 + reps)."""
    assert reps + 11 <= 64
    be.event_record(10)
    for i in range(reps):
        replay(g)
        be.event_record(11 + i)
    be.sync()
    return [be.event_elapsed_ms(10 + i, 11 + i) for i in range(reps)]


def flat_prefill(case, r, W, F, E, K):
    """One prefill case as a flat object of scalars (tokens/s, ms per layer,
    the layer's HBM and MFMA rooflines, per-stage times)."""
    T = int(case.split("=")[1].split()[0])
    stage = r.get("stage_us", {})
    hbm, mfma = r.get("hbm", {}), r.get("mfma", {})
    zipf = "zipf" in case
    bound = "mfma" if T >= 2048 else "hbm"
    flat = {"workload": "MoE layer prefill T=%d%s: hidden %d, %d experts, top-%d + shared, Q2" %
                        (T, " (Zipf(1.1)-biased router)" if zipf else "", W, E, K),
            "tokens": T, "tokens_per_s": r["tokens_per_s"], "ms_per_layer": r["ms_per_layer"],
            "distinct_experts": r.get("distinct_experts"),
            "roofline_bound": bound,
            "roofline_achieved": mfma.get("layer_flops", 0) / (r["ms_per_layer"] * 1e-3) / 1e12 if bound == "mfma"
            else hbm.get("achieved_GBs"),
            "roofline_peak": PEAK_MFMA_F16 / 1e12 if bound == "mfma" else PEAK_HBM / 1e9,
            "roofline_unit": "TFLOP/s" if bound == "mfma" else "GB/s",
            "roofline_frac": mfma.get("layer_frac") if bound == "mfma" else hbm.get("frac"),
            "hbm_frac": hbm.get("frac"), "mfma_frac": mfma.get("layer_frac"),
            "route_us": stage.get("prefill_route"), "dispatch_us": stage.get("prefill_dispatch"),
            "gate_up_us": stage.get("prefill_gate_up_gemm"), "down_us": stage.get("prefill_down_gemm"),
            "combine_us": stage.get("prefill_combine")}
    if flat["roofline_achieved"] is not None:
        flat["roofline_achieved"] = round(flat["roofline_achieved"], 1)
    for k in ("router", "route_fallback_tokens", "route_candidates_per_token"):
        if k in r:
            flat[k] = r[k]
    return flat


def guarded(out, name, fn):
    """out[name] = fn(), or {"error": ...} when it raises, so that an optional
    section cannot take the headline with it."""
    t0 = time.perf_counter()
    print("bench: section %s" % name, file=sys.stderr, flush=True)
    try:
        out[name] = fn()
        print("bench: section %s done in %.1f s" % (name, time.perf_counter() - t0), file=sys.stderr, flush=True)
    except Exception as e:  # noqa: BLE001 - reported in the JSON line
        out[name] = {"error": "%s: %s" % (type(e).__name__, str(e)[:400])}
        print("bench: section %s failed: %s" % (name, e), file=sys.stderr, flush=True)


def under_profiler(environ=None):
    """True when rocprofv3's tracer is loaded into this process (its library in
    LD_PRELOAD, or the ROCPROF* settings it exports to the program)."""
    env = os.environ if environ is None else environ
    if "rocprof" in env.get("LD_PRELOAD", "").lower():
        return True
    return any(k.upper().startswith("ROCPROF") for k in env)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4800)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the 48-layer stack runs")
    ap.add_argument("--stack-steps", type=int, default=128)
    ap.add_argument("--no-pack", action="store_true", help="skip the pack-loading measurement")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense-format projection measurement")
    ap.add_argument("--no-prompt", action="store_true", help="skip the fixture prompt measurement (Node.js)")
    ap.add_argument("--no-real", action="store_true",
                    help="skip the real model's geometry (hidden 2560, ff 640) runs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="issue every step directly instead of replaying HIP graphs (for profilers)")
    ap.add_argument("--no-prefetch-router", action="store_true",
                    help="no next-layer router prefetch: by default each decode step names the next step's router "
                         "matrix (sm_prefetch_router), which its launch pulls into L2")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="seconds of T=1 CPU decodes (split over the 8- and 4-thread runs)")
    ap.add_argument("--cpu-quick", action="store_true", help="CPU baseline: T=1 only (no full prefill layers)")
    ap.add_argument("--prefill-reps", type=int, default=10)
    ap.add_argument("--prefill-cases", default="512,2048zipf",
                    help="comma-separated prefill cases: token count, 'zipf' for the Zipf-biased router")
    ap.add_argument("--summarize", metavar="DIR",
                    help="write the profiles/ summaries from rocprofv3 CSVs under DIR (no GPU needed)")
    ap.add_argument("--calibrate", action="store_true",
                    help="only run the copy kernel used to calibrate rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.summarize:
        return summarize(args.summarize)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs the MoE layer on a single MI355X (no multi-GPU path); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0 or args.layers < 1:
        sys.exit("steps >= 1, warmup >= 0, layers >= 1")
    if not args.eager and not args.calibrate and under_profiler():
        # rocprofv3 1.1.0's kernel tracing crashed inside hipGraphLaunch on
        # this benchmark's graph replays (SIGSEGV in the profiler's frames, twice):
        # profile the same work issued directly instead.
        print("bench.py: running under rocprofv3; graph replays are not profiled here, add --eager",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import stratacuda_amd as sm
    from stratacuda_amd import workload as wl

    be = sm.Backend(0)
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK

    if args.calibrate:
        n = 64 * 1024 * 1024  # 256 MiB read + 256 MiB written per launch
        a, b = be.alloc(n, zero=True), be.alloc(n)
        for _ in range(5):
            be.run("strata_elementwise", {"A": a, "B": a, "Y": b, "n": n, "mode": 0, "scale": 1.0}, [n // 64, 1, 1])
        be.sync()
        print(json.dumps({"calibration": "strata_elementwise copy", "bytes_read": n * 4, "bytes_written": n * 4}))
        return

    L = args.layers
    print("bench: building %d resident layers (%.1f GB of expert blobs)" % (L, L * E * wl.blob_stride() / 1e9),
          file=sys.stderr, flush=True)
    layers = [wl.DeviceLayer(be, l) for l in range(L)]
    ones = be.alloc(np.ones(W, np.float32))
    slots = []
    for i in range(L):
        z = be.alloc(W, zero=False)
        be.synth_normal(z, W, wl.layer_seed(i) + 99, wl.STREAM_INPUT, 1.0)
        x = be.alloc(W, zero=False)
        be.run("strata_norm", {"X": z, "W": ones, "Y": x, "cols": W, "rows": 1, "weightRows": 1, "mode": 0,
                               "epsilon": 1e-6, "scale": 1.0}, [1, 1, 1])
        slots.append({"x": x, "y": be.alloc(W), "ids": be.alloc(K, "i32"), "w": be.alloc(K),
                      "ws": be.alloc_bytes(be.moe_workspace_bytes(1, W, F, E, K))})

    def step(i):
        s, lay = slots[i], layers[i]
        if not args.no_prefetch_router:
            # the router matrix of the step after this one (the next layer of
            # the rotation), pulled into L2 by this step's launch
            be.prefetch_router(layers[(i + 1) % L].Wr, E, W)
        be.moe_layer(s["x"], 1, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, s["y"], s["ids"],
                     s["w"], s["ws"])

    def capture(fn):
        """A graph of what fn issues, or fn itself with --eager."""
        if args.eager:
            return fn
        be.graph_begin()
        fn()
        return be.graph_end()

    def replay(g):
        if args.eager:
            g()
        else:
            be.graph_launch(g)

    def release(g):
        if not args.eager:
            be.graph_free(g)

    def all_layers(count=L):
        for i in range(count):
            step(i)

    g_full = warm_and_check(be, step, slots, args.warmup, capture, replay, E, K, np)
    rem = args.steps % L
    g_rem = capture(lambda: all_layers(rem)) if rem else None
    if g_rem is not None:
        # its first launch (the graph's upload to the device) stays out of
        # the timed region, as the full graph's did in warm_and_check
        replay(g_rem)
        be.sync()

    def run_steps():
        for _ in range(args.steps // L):
            replay(g_full)
        if g_rem is not None:
            replay(g_rem)

    # ---- timed region: exactly K steps from graph replays, a device
    # synchronisation on both sides (nothing else inside)
    be.sync()
    t0 = time.perf_counter()
    run_steps()
    be.sync()
    t1 = time.perf_counter()
    wall = t1 - t0
    # the same K steps again between two events on the library's stream
    # (GPU time, reported beside the wall-clock value)
    be.event_record(0)
    run_steps()
    be.event_record(1)
    be.sync()
    gpu_ms = be.event_elapsed_ms(0, 1)
    ms_per_step = wall * 1e3 / args.steps
    # median over 50 separately timed replays of the 48-step graph
    rep_ms = sorted(replay_times(be, replay, g_full, 50))
    median_us = rep_ms[len(rep_ms) // 2] * 1e3 / L
    mean_us = sum(rep_ms) * 1e3 / (len(rep_ms) * L)

    # ---- per-kernel durations. One token at this geometry runs the single-
    # launch layer (k_decode_fused): its duration per launch is the step time
    # of the 48-step graph. The three-kernel decode path (stage 8 off) is
    # timed beside it, stage by stage, from graphs that run one stage each.
    kernel_bytes = decode_kernel_bytes(W, F, E, K)
    step_bytes = layer_bytes(W, F, E, K, 1, K)
    fused = W == 2048 and F == 512 and K <= 10 and E <= 512
    three_kernels = 0xffffffff & ~(1 << 8)
    kernels = {}
    reps = max(1, min(50, 2400 // L))

    def timed_graph(mask, ev0, ev1):
        be.stage_select(mask)
        gid = capture(all_layers)
        if not args.eager:
            be.stage_select()
        replay(gid)
        be.sync()
        be.event_record(ev0)
        for _ in range(reps):
            replay(gid)
        be.event_record(ev1)
        be.sync()
        be.stage_select()
        release(gid)
        return be.event_elapsed_ms(ev0, ev1) * 1e3 / (reps * L)

    if fused:
        gbs = step_bytes / (mean_us * 1e-6) / 1e9
        kernels["decode_fused"] = {"avg_us": round(mean_us, 3), "median_us": round(median_us, 3),
                                   "bytes_per_launch": step_bytes, "GB/s": round(gbs, 1),
                                   "frac_hbm": round(gbs * 1e9 / PEAK_HBM, 4),
                                   "note": "one launch per step: the per-launch time includes the dispatch gap "
                                           "between dependent launches in the graph"}
    three = {}
    for stage, name in enumerate(["decode_route", "decode_gate_up", "decode_down_combine"]):
        us = timed_graph(1 << stage, 2, 3)
        gbs = kernel_bytes[name] / (us * 1e-6) / 1e9
        three[name] = {"avg_us": round(us, 3), "bytes_per_launch": kernel_bytes[name], "GB/s": round(gbs, 1),
                       "frac_hbm": round(gbs * 1e9 / PEAK_HBM, 4)}
    three["layer_us"] = round(timed_graph(three_kernels, 2, 3), 3)
    if fused:
        kernels["three_kernel_path"] = three
        dom, hip_kernel = "decode_fused", "k_decode_fused"
        dk = kernels[dom]
    else:
        kernels.update(three)
        dom = max(("decode_route", "decode_gate_up", "decode_down_combine"), key=lambda k: three[k]["avg_us"])
        hip_kernel = {"decode_route": "k_decode_route", "decode_gate_up": "k_decode_gate_up",
                      "decode_down_combine": "k_decode_down"}[dom]
        dk = three[dom]
    roofline = {"bound": "hbm", "kernel": hip_kernel, "achieved": dk["GB/s"], "peak": PEAK_HBM / 1e9,
                "unit": "GB/s", "frac": dk["frac_hbm"], "traffic": read_traffic(hip_kernel),
                "bytes_per_launch": dk["bytes_per_launch"], "avg_us": dk["avg_us"],
                "traffic_source": "profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per launch, copy-kernel calibrated, "
                                  "measured without the next-layer router prefetch (with it a launch also fetches "
                                  "the next layer's W_r into L2; profiles/traffic_decode_T1.md)"}
    # whole step against the per-token algorithmic bytes
    step_s = gpu_ms * 1e-3 / args.steps
    layer_roof = {"bound": "hbm", "bytes_per_step": step_bytes, "achieved": round(step_bytes / step_s / 1e9, 1),
                  "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": round(step_bytes / step_s / PEAK_HBM, 4),
                  "gpu_us_per_step": round(step_s * 1e6, 3)}

    def section_prefill():
        """Prefill through the grouped-MFMA path."""
        prefill = {}
        cases = [(int(c.replace("zipf", "")), "zipf" in c) for c in args.prefill_cases.split(",") if c]
        for T, zipf in cases:
            Xs = []
            for j in range(2):
                X = be.alloc(T * W, zero=False)
                be.synth_normal(X, T * W, wl.layer_seed(j) + 7 + T, wl.STREAM_INPUT, 1.0)
                Xs.append(X)
            bias = be.alloc(wl.zipf_bias(E, wl.layer_seed(0))) if zipf else None
            Y, ids, w = be.alloc(T * W), be.alloc(T * K, "i32"), be.alloc(T * K)
            ws = be.alloc_bytes(be.moe_workspace_bytes(T, W, F, E, K))

            def run(j):
                lay = layers[j % L]
                be.moe_layer(Xs[j % 2], T, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, Y, ids,
                             w, ws, bias=bias)

            for j in range(3):
                run(j)
            be.sync()
            # per-stage times: events between the stages of eager calls
            be.stage_timing(True)
            for j in range(args.prefill_reps):
                run(j)
            be.sync()
            rep = be.stage_report()
            be.stage_timing(False)
            # the layer time: prefill_reps calls replayed from one graph
            # (issued directly with --eager)
            g = capture(lambda: [run(j) for j in range(args.prefill_reps)])
            replay(g)
            be.sync()
            be.event_record(4)
            replay(g)
            be.event_record(5)
            be.sync()
            release(g)
            ms = be.event_elapsed_ms(4, 5) / args.prefill_reps
            got = be.read(ids)
            distinct = len(np.unique(got))
            # the certified batch router's last call on this workspace: its
            # candidate experts per token and the tokens it sent to the exact
            # fallback (None below the router's 512 tokens)
            cert = be.route_stats(ws, T, W, F, E, K)
            counts = np.sort(np.bincount(got, minlength=E))[::-1]
            M = T * (K + 1)
            stages = {k: round(v[0] / max(1, v[1]) * 1e3, 2) for k, v in rep.items() if v[1]}
            gu_us, dn_us = stages.get("prefill_gate_up_gemm", 0.0), stages.get("prefill_down_gemm", 0.0)
            gu_fl, dn_fl = 2.0 * M * 2 * F * W, 2.0 * M * W * F
            lb = layer_bytes(W, F, E, K, T, distinct)
            lf = layer_flops(W, F, E, K, T)
            prefill["T=%d%s" % (T, " zipf" if zipf else "")] = {
                "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_layer": round(ms, 4),
                "distinct_experts": int(distinct), "top20_share": round(float(counts[:20].sum() / got.size), 3),
                "router": "certified (fp16 MFMA bound + exact boundary)" if cert else "exact reference order",
                "stage_us": stages,
                "execution": ("%d layer calls issued directly" % args.prefill_reps if args.eager else
                              "HIP graph of %d layer calls (stage_us: eager calls with events between the stages)"
                              % args.prefill_reps),
                "hbm": {"bytes": lb, "achieved_GBs": round(lb / (ms * 1e-3) / 1e9, 1),
                        "frac": round(lb / (ms * 1e-3) / PEAK_HBM, 4)},
                "mfma": {"layer_flops": lf, "layer_frac": round(lf / (ms * 1e-3) / PEAK_MFMA_F16, 4),
                         "gate_up_gemm_TFLOPs": round(gu_fl / (gu_us * 1e-6) / 1e12, 1) if gu_us else None,
                         "gate_up_gemm_frac": round(gu_fl / (gu_us * 1e-6) / PEAK_MFMA_F16, 4) if gu_us else None,
                         "down_gemm_frac": round(dn_fl / (dn_us * 1e-6) / PEAK_MFMA_F16, 4) if dn_us else None,
                         "peak": "2.5 PFLOP/s dense fp16/bf16"},
                "dtype": "f32 in/out; experts on fp16 MFMA (exact fp16 weights, activations split hi+lo), f32 accumulate",
            }
            if cert:
                prefill["T=%d%s" % (T, " zipf" if zipf else "")].update(
                    route_candidates_per_token=round(cert[0] / T, 2), route_fallback_tokens=cert[1])
        return prefill

    def section_stack():
        """Config 5: the 48-layer stack, token by token (batch 1) and batch 32."""
        stack = {}
        blob = 2 * F * W // 4 + W * F // 4 + 2 * F * (W // 64) * 2 + W * (F // 64) * 2
        for T in (1, 32):
            st = wl.DeviceStack(be, layers=layers, tokens=T, trace=True, prefetch=not args.no_prefetch_router)
            S = args.stack_steps
            inputs = be.alloc(S * T * W, zero=False)
            be.synth_normal(inputs, S * T * W, wl.BASE_SEED + 31 * T, wl.STREAM_INPUT, 1.0)
            gid = capture(st.step)
            for s in range(2):
                be.copy(inputs, st.H[0], T * W, s * T * W, 0)
                replay(gid)
            be.sync()
            be.event_record(6)
            for s in range(S):
                be.copy(inputs, st.H[0], T * W, s * T * W, 0)
                replay(gid)
            be.event_record(7)
            be.sync()
            ms = be.event_elapsed_ms(6, 7) / S
            distinct = [len(np.unique(be.read(st.ids[l]))) for l in range(st.L)]
            step_bytes = sum(d * blob + blob + E * W * 4 + 3 * W * 4 + 4 * T * W * 4 for d in distinct)
            stack["batch%d" % T] = {
                "tokens_per_s": round(T / (ms * 1e-3), 1), "ms_per_step": round(ms, 4), "layers": st.L,
                "steps": S, "distinct_experts_per_layer": round(sum(distinct) / len(distinct), 1),
                "hbm": {"bytes_per_step": step_bytes, "achieved_GBs": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                        "frac": round(step_bytes / (ms * 1e-3) / PEAK_HBM, 4)},
                "execution": "one HIP graph per step: per layer RMSNorm, MoE layer, residual add",
            }
            release(gid)
            be.free(inputs)
            st.free()
        return stack

    def section_pack():
        """Pack loading: layer 0 written as a pack, then streamed back into HBM."""
        pack = None
        import shutil
        import tempfile
        d = tempfile.mkdtemp(prefix="strata-pack-")
        try:
            lay = layers[0]
            host = {"arena": be.read_bytes(lay.arena), "stride": lay.stride, "shared": be.read_bytes(lay.shared),
                    "Wr": be.read(lay.Wr), "Wsg": be.read(lay.Wsg), "gamma": be.read(lay.gamma)}
            wl.write_pack(d, W, F, E, K, [host])
            reader = wl.PackReader(d)
            reader.load_layer(be, 0).free()  # page cache warm
            t0 = time.perf_counter()
            loaded = reader.load_layer(be, 0)
            be.sync()
            dt = time.perf_counter() - t0
            same = bool(np.array_equal(be.read_bytes(loaded.arena), host["arena"]))
            loaded.free()
            nbytes = (E + 1) * reader.blob_bytes
            pack = {"what": "one layer's 513 Q2 blobs from experts.bin (page cache) into the HBM arena, with the "
                            "device scale check, plus its dense vectors", "bytes": nbytes, "seconds": round(dt, 4),
                    "GB_per_s": round(nbytes / dt / 1e9, 2), "arena_bit_exact": same}
        finally:
            shutil.rmtree(d, ignore_errors=True)
        return pack

    def section_prompt():
        prompt = prompt_orchestration()
        prompt["kernels"] = prompt_kernels(be, np, capture, replay, release)
        return prompt

    def section_cpu():
        import oracle
        return cpu_baseline(oracle, wl, args.cpu_seconds, prefill=not args.cpu_quick)

    out = {
        "metric": METRIC,
        "value": round(args.steps / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded counter-based generator (SplitMix64); normals are Irwin-Hall sums of 12 "
                "uniforms (variance 1, |n| <= 6); random-init Q2 experts of the reference layout",
        "config": {"workload": "single MoE layer decode, T=1: hidden 2048, 512 experts, top-10 + shared, Q2 "
                               "(64-weight fp16-scale groups), 48 resident layers rotated per step",
                   "tokens_per_step": 1, "layers_rotated": L,
                   "router_prefetch": ("each step names the next step's router matrix; its launch pulls those rows "
                                       "into L2 while it waits (sm_prefetch_router)" if not args.no_prefetch_router
                                       else None),
                   "execution": "HIP graph of 48 steps, one launch per step (k_decode_fused)" if fused else
                                "HIP graph of 48 steps, three launches per step",
                   "gpu_us_per_step": round(gpu_ms * 1e3 / args.steps, 3),
                   "median_us_per_step": round(median_us, 3), "mean_us_per_step_50_replays": round(mean_us, 3),
                   "timing": "value = steps / wall time of the timed region (graph launches between two device "
                             "synchronisations); gpu_us_per_step from the same steps run again between HIP events; "
                             "median and mean over 50 separately timed replays of the 48-step graph (HIP events "
                             "on the library's stream)"},
        "roofline": roofline,
        "cpu_baseline": None,
        "layer_roofline": layer_roof,
        "kernels": kernels,
    }
    if not args.no_cpu:
        guarded(out, "cpu_baseline", section_cpu)
    if not args.no_prefill:
        # The nested per-case results under prefill_detail; flat objects of
        # scalars (the first case as `prefill`, the others beside it) so that
        # a reader keeping only scalar fields still sees them.
        guarded(out, "prefill_detail", section_prefill)
        detail = out.get("prefill_detail") or {}
        for i, (case, r) in enumerate((k, v) for k, v in detail.items() if isinstance(v, dict) and "ms_per_layer" in v):
            key = "prefill" if i == 0 else "prefill_" + case.replace("=", "").replace(" ", "_")
            out[key] = flat_prefill(case, r, W, F, E, K)
    for flag, name, fn in ((args.no_stack, "stack", section_stack),
                           (args.no_real, "real_model",
                            lambda: real_model(be, wl, np, capture, replay, release, prefetch=not args.no_prefetch_router)),
                           (args.no_dense, "dense_formats", lambda: dense_formats(be, np, capture, replay, release)),
                           (args.no_pack, "pack_load", section_pack), (args.no_prompt, "prompt", section_prompt)):
        out[name] = None
        if not flag:
            guarded(out, name, fn)
    print(json.dumps(out))
    be.dispose()


if __name__ == "__main__":
    main()
