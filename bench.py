#!/usr/bin/env python3
"""Benchmark of the routed int4 MoE layer on one MI355X (the metric and configurations of BASELINE.json).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only WORKLOAD]

Headline (`value`): the 16-row decode step (8 requests + 8 draft rows, Zipf(1.1) expert popularity): one MoE layer
(router + routed int4 experts + shared expert + bf16 output) per step, in tokens/s, the steps captured in one hipGraph
and replayed (eager launches reported beside it). Steps cycle over 6 seeded
layers and 64 seeded inputs so consecutive steps stream different weights (the working set of a step is far above
the 256 MB last-level cache, as in a real decode pass through 75+ layers). Extras: decode at 1 and 8 rows, the
2048-token prefill chunk, the 176-resident partial tier at 1/4/8 rows, the same split with the other 80 experts on the
host-CPU tier, and the 16-layer hipGraph step at 4 rows.
One JSON line on stdout; progress on stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0                  # MI355X HBM3E
MFMA_PEAK_TFLOPS = 2500.0              # MI355X dense fp16 / bf16
EXPERT_BYTES = 19_464_192              # int4 codes + bf16 g128 scales of gate, up, down
GU_EXPERT_BYTES = 2 * (6_291_456 + 196_608)
DOWN_EXPERT_BYTES = 6_291_456 + 196_608
SHARED_BYTES = 75_497_472              # bf16-sized shared expert (held as f16)
SHARED_GU_BYTES, SHARED_DOWN_BYTES = 50_331_648, 25_165_824
ROUTER_BYTES = 6_291_456 + 1_024       # fp32 W_g + bias
H = 6144


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def metric_name():
    try:
        with open(os.path.join(ROOT, "BASELINE.json")) as f:
            return json.load(f)["metric"]
    except Exception:
        return "MoE layer µs/token + HBM GB/s at B=1,8; prefill tok/s at 2048 tokens"


def timed(torch, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def timed_graph(torch, fn, steps, warmup):
    """the same steps captured in one hipGraph and replayed, as a decode loop runs its per-row-count step (the
    reference captures its decode step once per row count, rtx_graph.py:6-8); the timed region is one replay"""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    g.replay()                                          # (first replay uploads the graph)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    del g
    return el


def decode_layers(torch, synth, R, n_layers, zipf, dev):
    import numpy as np
    layers = []
    for l in range(n_layers):
        bias = synth.zipf_bias(layer=l) if zipf else None
        layers.append(synth.make_layer(l, dev, bias=bias))
    torch.cuda.synchronize()
    return layers


def decode_workload(torch, synth, R, steps, warmup, zipf, dev, n_layers=6, n_x=64, tag0=0):
    """per step: layers[i % L].decode(x[i % P]) (router, routed + shared experts, bf16 out)"""
    import numpy as np
    t0 = time.perf_counter()
    layers = decode_layers(torch, synth, R, n_layers, zipf, dev)
    xs = [synth.gen_x(tag0 + i, R, dev) for i in range(n_x)]
    log(f"[bench] decode R={R}: {n_layers} layers ({sum(l.bank.nbytes for l in layers) / 1e9:.1f} GB) ready in "
        f"{time.perf_counter() - t0:.1f} s")
    L, P = len(layers), len(xs)
    el_eager = timed(torch, lambda i: layers[i % L].decode(xs[i % P]), steps, warmup)
    el = timed_graph(torch, lambda i: layers[i % L].decode(xs[i % P]), steps, warmup)
    # per-kernel timing of the same steps with HIP events on the launch stream: A (router logits), B (shared + routed
    # gate/up + SwiGLU, gu7_kernel), C (shared + routed down, dn6_kernel), D (ordered reduce + bf16 out)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    for i in range(steps):
        lay, x = layers[i % L], xs[i % P]
        evs[i][0].record()
        for k, ph in enumerate((1, 2, 4, 8)):
            lay.decode(x, phases=ph)
            evs[i][k + 1].record()
    torch.cuda.synchronize()
    kus = [float(np.mean([e[k].elapsed_time(e[k + 1]) for e in evs])) * 1e3 for k in range(4)]
    # distinct experts of every timed step (deterministic: same layer / input pairs)
    U = []
    for i in range(steps):
        lay = layers[i % L]
        lay.decode(xs[i % P], phases=2)
        U.append(len(torch.unique(lay.sel[:R])))
    U = np.array(U, np.float64)
    step_s = el / steps
    bytes_step = float(np.mean(U * EXPERT_BYTES + SHARED_BYTES + ROUTER_BYTES + R * 2 * H * 2))
    kbytes = [ROUTER_BYTES + R * H * 2,
              float(np.mean(U * GU_EXPERT_BYTES + SHARED_GU_BYTES + R * H * 2)),
              float(np.mean(U * DOWN_EXPERT_BYTES + SHARED_DOWN_BYTES + (U + 1) * R * 2048 * 2)),
              0.0]
    names = ["A_router", "B_gate_up", "C_down", "D_reduce_out"]
    res = {"rows": R, "us_per_step": step_s * 1e6, "us_per_step_eager": el_eager / steps * 1e6,
           "us_per_token": step_s * 1e6 / R, "tok_per_s": R / step_s,
           "distinct_experts_mean": float(U.mean()), "bytes_per_step": bytes_step,
           "hbm_gbs": bytes_step / step_s / 1e9, "hbm_frac": bytes_step / step_s / 1e9 / HBM_PEAK_GBS,
           "kernels": {n: {"us": kus[k], "algorithmic_bytes": kbytes[k],
                           "gbs": kbytes[k] / (kus[k] * 1e-6) / 1e9 if kbytes[k] else None}
                       for k, n in enumerate(names)}}
    del layers, xs
    torch.cuda.empty_cache()
    return res


def prefill_workload(torch, synth, steps, warmup, dev, T=2048):
    import numpy as np
    t0 = time.perf_counter()
    layers = [synth.make_layer(l, dev, bias_sigma=0.001, max_rows=T) for l in range(2)]
    xs = [synth.gen_x(2 + i, T, dev) for i in range(2)]
    for lay, x in zip(layers, xs):
        lay.prefill(x)
    torch.cuda.synchronize()
    log(f"[bench] prefill T={T}: ready in {time.perf_counter() - t0:.1f} s")
    el = timed(torch, lambda i: layers[i % 2].prefill(xs[(i // 2) % 2]), steps, warmup)
    step_s = el / steps
    flop = T * 8 * 3 * 2 * 2048 * 6144 + T * 3 * 2 * 2048 * 6144 + T * 2 * 256 * 6144
    bytes_step = 256 * EXPERT_BYTES + SHARED_BYTES + ROUTER_BYTES + 2 * T * H * 2
    counts = np.bincount(layers[0]._pf.sel[:T].cpu().numpy().ravel(), minlength=256)
    res = {"tokens": T, "ms_per_chunk": step_s * 1e3, "tok_per_s": T / step_s, "flop": flop,
           "tflops": flop / step_s / 1e12, "mfma_frac": flop / step_s / 1e12 / MFMA_PEAK_TFLOPS,
           "hbm_frac": bytes_step / step_s / 1e9 / HBM_PEAK_GBS,
           "picks_per_expert": [int(counts.min()), float(counts.mean()), int(counts.max())]}
    del layers, xs
    torch.cuda.empty_cache()
    return res


def partial_workload(torch, synth, steps, warmup, dev, n_layers=4):
    """176 of 256 experts resident (top by Zipf popularity), routed experts only, added into an fp32 partial"""
    import numpy as np
    layers = [synth.make_layer(l, dev, resident=synth.popularity_order(layer=l)[:176], shared=False)
              for l in range(n_layers)]
    out = {}
    for R in (1, 4, 8):
        xs = [synth.gen_x(3000 + 16 * R + i, R, dev) for i in range(32)]
        part = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)

        def step(i):
            lay = layers[i % n_layers]
            lay.route(xs[i % 32])
            lay.experts_decode(R, part, with_shared=False)
        el_eager = timed(torch, step, steps, warmup)
        el = timed_graph(torch, step, steps, warmup)
        U = []
        for i in range(steps):
            lay = layers[i % n_layers]
            sel, _ = lay.route(xs[i % 32])
            U.append(int((sel < 176).sum().item() and len(torch.unique(sel[sel < 176]))))
        U = np.array(U, np.float64)
        step_s = el / steps
        b = float(np.mean(U * EXPERT_BYTES + ROUTER_BYTES + 2 * R * H * 4 + R * H * 2))
        out[f"B{R}"] = {"us_per_step": step_s * 1e6, "us_per_step_eager": el_eager / steps * 1e6,
                        "us_per_token": step_s * 1e6 / R,
                        "resident_experts_mean": float(U.mean()), "hbm_gbs": b / step_s / 1e9,
                        "hbm_frac": b / step_s / 1e9 / HBM_PEAK_GBS}
    del layers
    torch.cuda.empty_cache()
    return out


def tiered_workload(torch, synth, steps, warmup, dev, threads=8):
    """config 3 with the other 80 experts on the host-CPU tier (tier_split.py's split): route on the GPU, hand the
    rows to the pool through the device-mapped mailbox, run the 176 resident experts into the fp32 partial
    meanwhile, then add the pool's partial on the same stream; one layer, 32 seeded inputs per row count"""
    import numpy as np
    from hecate_amd.cpu_tier import CpuTier, decode_split, host_experts
    lay = synth.make_layer(0, dev, resident=synth.popularity_order()[:176], shared=False)
    cpu = CpuTier(threads=threads)
    try:
        with open("/proc/cpuinfo") as f:
            flags = next((ln for ln in f if ln.startswith("flags")), "").split()
    except OSError:
        flags = []
    vnni = "avx512_vnni" in flags and "avx512bw" in flags and os.environ.get("HMOE_CPU_ISA") != "avx2"
    out = {"cpu_threads": threads, "cpu_dot": "avx512-vnni" if vnni else "avx2"}
    try:
        cpu.add_layer(0, 176, host_experts(0, lay.perm[176:], dev))
        for R in (1, 4, 8):
            xs = [synth.gen_x(3500 + 16 * R + i, R, dev) for i in range(32)]
            part = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0,
                                    0.1).view(R, H)
            el = timed(torch, lambda i: decode_split(lay, cpu, 0, xs[i % 32], part), steps, warmup)
            el_gpu = timed(torch, lambda i: (lay.route(xs[i % 32]), lay.experts_decode(R, part, False)), steps, warmup)
            cold = []
            for i in range(32):
                sel, _ = lay.route(xs[i])
                cold.append(len(torch.unique(sel[sel >= 176])))
            out[f"B{R}"] = {"us_per_step": el / steps * 1e6, "us_per_token": el / steps * 1e6 / R,
                            "gpu_tier_alone_us_per_step": el_gpu / steps * 1e6,
                            "cpu_experts_per_step_mean": float(np.mean(cold))}
    finally:
        torch.cuda.synchronize()
        cpu.close()
    del lay
    torch.cuda.empty_cache()
    return out


def graph_workload(torch, synth, steps, warmup, dev, n_layers=16, R=4):
    import numpy as np
    from hecate_amd.stack import DecodeStack
    t0 = time.perf_counter()
    layers = [synth.make_layer(l, dev) for l in range(n_layers)]
    norm_w = [synth.gen_normal(synth.key(synth.SEED, l, synth.KIND["NORM_W"]), H, dev, 1.0, 0.02)
              for l in range(n_layers)]
    st = DecodeStack(layers, norm_w, R)
    st.x.copy_(synth.gen_x(4, R, dev))
    st.capture()
    log(f"[bench] {n_layers}-layer graph R={R}: {sum(l.bank.nbytes for l in layers) / 1e9:.1f} GB ready in "
        f"{time.perf_counter() - t0:.1f} s")
    el = timed(torch, lambda i: st.replay(), steps, warmup)
    U = np.array([len(torch.unique(l.sel[:R])) for l in layers], np.float64)
    step_s = el / steps
    b = float(np.sum(U * EXPERT_BYTES + SHARED_BYTES + ROUTER_BYTES + R * H * 12))
    res = {"layers": n_layers, "rows": R, "us_per_step": step_s * 1e6, "us_per_token": step_s * 1e6 / R,
           "distinct_experts_per_layer": float(U.mean()), "bytes_per_step": b, "hbm_gbs": b / step_s / 1e9,
           "hbm_frac": b / step_s / 1e9 / HBM_PEAK_GBS}
    del st, layers
    torch.cuda.empty_cache()
    return res


def copy_workload(torch, steps, warmup, dev, nbytes=1 << 30):
    """torch's device copy of a known size: the calibration of the FETCH_SIZE / WRITE_SIZE counters (KiB per
    dispatch) and the measured copy bandwidth of the box"""
    src = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(7)
    dst = torch.empty_like(src)
    el = timed(torch, lambda i: dst.copy_(src), steps, warmup)
    res = {"bytes_read": nbytes, "bytes_written": nbytes, "us_per_copy": el / steps * 1e6,
           "gbs_read_plus_write": 2 * nbytes / (el / steps) / 1e9}
    del src, dst
    torch.cuda.empty_cache()
    return res


def cpu_baseline(budget_s=12.0):
    """the CPU expert path (oracle q8_0 mode: runtime/tier/cpuband.cpp restated) on the 16-row Zipf step of layer 0,
    as two 8-row jobs (cpuband caps a job at 8 rows) after the CPU router, timed on this host's cores"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import pyoracle as O
    from hostlayer import HostLayer, x_rows
    from hecate_amd import synth
    threads = max(1, min(16, os.cpu_count() or 1))
    hl = HostLayer(0, bias=synth.zipf_bias(layer=0))
    comp, steps = 0.0, 0
    for i in range(64):
        x = x_rows(i, 16)
        t0 = time.perf_counter()
        sel, rw = O.router(x, hl.wg, hl.bias)
        t1 = time.perf_counter()
        tab = hl.table(sel)                           # host weight generation, not timed
        t2 = time.perf_counter()
        for j in (0, 8):
            O.moe(1, x[j:j + 8], sel[j:j + 8], rw[j:j + 8], tab, 0, 256, hl.shared, threads=threads)
        t3 = time.perf_counter()
        comp += (t1 - t0) + (t3 - t2)
        steps += 1
        if comp >= budget_s:
            break
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
    except Exception:
        pass
    return {"value": 16 * steps / comp, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} steps of the 16-row Zipf decode step of layer 0 (router + 2 x 8-row q8_0 jobs of the "
                      f"restated cpuband path + fp32 shared expert), {comp:.1f} s of compute on {model}, "
                      f"{threads} OpenMP threads"}


def traffic_from_profiles(kernel):
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(kernel)
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None, choices=[None, "decode16", "decode1", "decode8", "prefill", "partial",
                                                     "graph16", "copy", "tiered"])
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the path would shard by "
              f"expert, see the design notes)", file=sys.stderr)
        sys.exit(2)
    import torch
    from hecate_amd import synth
    dev = torch.device("cuda:0")
    K, W = args.steps, args.warmup
    only = args.only
    extra = {}
    head = None
    if only in (None, "decode16"):
        head = decode_workload(torch, synth, 16, K, W, True, dev, tag0=1000)
        log(f"[bench] decode16: {json.dumps(head)}")
    if only in (None, "decode1"):
        extra["decode_b1"] = decode_workload(torch, synth, 1, K, W, False, dev, tag0=0)
        log(f"[bench] decode1: {json.dumps(extra['decode_b1'])}")
    if only in (None, "decode8"):
        extra["decode_b8"] = decode_workload(torch, synth, 8, K, W, False, dev, tag0=500)
        log(f"[bench] decode8: {json.dumps(extra['decode_b8'])}")
    if only in (None, "prefill"):
        extra["prefill_2048"] = prefill_workload(torch, synth, max(10, K // 10), max(2, W // 10), dev)
        log(f"[bench] prefill: {json.dumps(extra['prefill_2048'])}")
    if only in (None, "partial"):
        extra["partial_176"] = partial_workload(torch, synth, K, W, dev)
        log(f"[bench] partial: {json.dumps(extra['partial_176'])}")
    if only in (None, "graph16"):
        extra["graph_16_layers_b4"] = graph_workload(torch, synth, max(20, K // 4), max(3, W // 4), dev)
        log(f"[bench] graph16: {json.dumps(extra['graph_16_layers_b4'])}")
    if only in (None, "tiered"):
        extra["tiered_176_cpu80"] = tiered_workload(torch, synth, max(20, K // 10), max(3, W // 4), dev)
        log(f"[bench] tiered: {json.dumps(extra['tiered_176_cpu80'])}")
    if only == "copy":
        extra["copy_1gib"] = copy_workload(torch, max(10, K // 10), 3, dev)
    if head is None:
        print(json.dumps({"extra": extra}))
        return
    cpu = None if args.no_cpu else cpu_baseline()
    kb = head["kernels"]["B_gate_up"]
    roof = {"bound": "hbm", "kernel": "gu7_kernel (shared gate/up + top-8 selection + routed int4 gate/up + SwiGLU)",
            "achieved": kb["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": kb["gbs"] / HBM_PEAK_GBS,
            "traffic": traffic_from_profiles("gu7_kernel"), "algorithmic_bytes_per_launch": kb["algorithmic_bytes"],
            "launch_us": kb["us"]}
    extra["decode_b16"] = head
    line = {"metric": metric_name(), "value": head["tok_per_s"], "unit": "tok/s", "n_gpus": 1, "steps": K,
            "warmup": W, "ms_per_step": head["us_per_step"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16 (int4 weights, fp32 accumulation)", "data": "synthetic",
            "config": {"workload": "decode_b16_zipf: one routed int4 MoE layer step (router + top-8 of 256 int4 g128 "
                                   "experts + bf16 shared expert + bf16 out), 16 rows, Zipf(1.1) popularity",
                       "rows": 16, "hidden": H, "intermediate": 2048, "experts": 256, "topk": 8,
                       "us_per_token": head["us_per_token"], "hbm_gbs": head["hbm_gbs"]},
            "roofline": roof, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
