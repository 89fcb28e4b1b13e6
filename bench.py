#!/usr/bin/env python3
"""Benchmark of the routed int4 MoE layer on one MI355X (the metric and configurations of BASELINE.json).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only WORKLOAD]

Headline (`value`): BASELINE.json's config 0, the decode step at B = 1: one MoE layer (router + top-8 of 256 int4
g128 experts + bf16 shared expert + bf16 output) per step, in tokens/s, the timed steps captured in one hipGraph and
replayed (eager launches reported beside it). Steps cycle over 6 seeded layers and 64 seeded inputs so consecutive
steps stream different weights (a step's working set is far above the 256 MB last-level cache, as in a real decode
pass through 75+ layers). Extras: decode at 8 rows and at 16 rows with Zipf(1.1) popularity (config 1), the
2048-token prefill chunk (config 2) and an 8192-token chunk on the long-prefill op, the 176-resident partial tier at
1/4/8 rows (config 3), the same split with the other 80 experts on the host-CPU tier, the 16-layer hipGraph step at
4 rows (config 4), and a near-tie audit of the selections. cpu_baseline: the reference's CPU expert path (cpuband.cpp
restated: the pinned host pool of hecate_amd/csrc/cputier.cpp) with the router and the shared expert on the same
cores, per config, on bounded samples.
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


def timed_graph(torch, fn, steps, warmup, events=False):
    """the same steps captured in one hipGraph and replayed, as a decode loop runs its per-row-count step (the
    reference captures its decode step once per row count, rtx_graph.py:6-8); the timed region is one replay, timed
    by the host clock around it or (events) by HIP events recorded on the launch stream"""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    g.replay()                                          # (first replay uploads the graph)
    torch.cuda.synchronize()
    if events:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        el = e0.elapsed_time(e1) * 1e-3
    else:
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
    # per-kernel timing of the same steps: each launch of the step (A router logits, B shared + routed gate/up +
    # SwiGLU (gu7_kernel), C shared + routed down (at one row dn8_kernel, which also adds the parts in order and
    # writes the bf16 out; above, dn6_kernel's part partials), D the ordered reduce + bf16 out of the part form (no
    # launch at one row)) repeated over the timed steps' layers and inputs in one hipGraph, timed with HIP events on
    # the launch stream around its replay: the launch's duration in a decode loop, the step's other launches left out
    # (single launches bracketed by events add the event and launch overhead to each)
    own = R == 1
    kus = [timed_graph(torch, lambda i, ph=ph: layers[i % L].decode(xs[i % P], phases=ph), steps, 2, events=True)
           / steps * 1e6 if not (own and ph == 8) else 0.0 for ph in (1, 2, 4, 8)]
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
    names = ["A_router", "B_gate_up", "C_down_out" if own else "C_down", "D_reduce_out"]
    res = {"rows": R, "us_per_step": step_s * 1e6, "us_per_step_eager": el_eager / steps * 1e6,
           "us_per_token": step_s * 1e6 / R, "tok_per_s": R / step_s,
           "distinct_experts_mean": float(U.mean()), "bytes_per_step": bytes_step,
           "hbm_gbs": bytes_step / step_s / 1e9, "hbm_frac": bytes_step / step_s / 1e9 / HBM_PEAK_GBS,
           "kernels": {n: {"us": kus[k], "algorithmic_bytes": kbytes[k],
                           "gbs": kbytes[k] / (kus[k] * 1e-6) / 1e9 if kbytes[k] else None}
                       for k, n in enumerate(names) if not (own and k == 3)}}
    del layers, xs
    torch.cuda.empty_cache()
    return res


def prefill_workload(torch, synth, steps, warmup, dev, T=2048):
    """per step: one chunk of T tokens through a layer (router, device dispatch plan, grouped GEMMs of the routed
    experts, shared expert, combine, bf16 out), alternating 2 layers and 2 inputs; T > 2048 runs the long-prefill op"""
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
    res = {"tokens": T, "op": "moe4t" if T > 2048 else "moe4p", "ms_per_chunk": step_s * 1e3, "tok_per_s": T / step_s,
           "flop": flop,
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
            # router logits, selection in the gate/up launch, the resident experts added into the partial: the four
            # launches of the decode layer op with y and without the shared expert or the bf16 output
            layers[i % n_layers].decode(xs[i % 32], y=part, out=False, with_shared=False)
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


def tiered_workload(torch, synth, steps, warmup, dev, threads=16):
    """config 3 with the other 80 experts on the host-CPU tier (tier_split.py's split): route on the GPU, hand the
    rows to the pool through the device-mapped mailbox, run the 176 resident experts into the fp32 partial
    meanwhile, then add the pool's partial on the same stream; one layer, 32 seeded inputs per row count"""
    import numpy as np
    from hecate_amd import cn, router
    from hecate_amd.cpu_tier import CpuTier, decode_split, decode_split_norm, host_experts
    lay = synth.make_layer(0, dev, resident=synth.popularity_order()[:176], shared=False)
    # the pool pinned to the CPU baseline's cores (the reference pins its workers, tier_split.py:35-36) and this
    # thread, which waits on the GPU, kept off them
    cores, info = cpu_cores()
    threads = min(threads, len(cores))
    cpu = CpuTier(threads=threads, first_core=cores[0] if info["pinned"] else -1)
    allowed = sorted(os.sched_getaffinity(0))
    spare = [c for c in allowed if c not in set(cores[:threads])]
    if spare:
        os.sched_setaffinity(0, set(spare))
    try:
        with open("/proc/cpuinfo") as f:
            flags = next((ln for ln in f if ln.startswith("flags")), "").split()
    except OSError:
        flags = []
    vnni = "avx512_vnni" in flags and "avx512bw" in flags and os.environ.get("HMOE_CPU_ISA") != "avx2"
    out = {"cpu_threads": threads, "cpu_dot": "avx512-vnni" if vnni else "avx2",
           "first_core": cores[0] if info["pinned"] else None}
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
            # the step with the post-attention norm + router and the combine into the next norm, the hand-off folded
            # into them (norm_route posting the job, combine_norm_cpu adding the pool's partial) against the same step
            # with the hand-off and the collect as launches of their own
            hs = [synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], 100 + 16 * R + i), R * H, dev, 0.0,
                                   0.5).view(R, H) for i in range(4)]
            wp = torch.ones(H, device=dev)
            wn = torch.ones(H, dtype=torch.bfloat16, device=dev)
            r = torch.zeros((R, H), device=dev)
            x2 = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
            xn = torch.empty((R, H), dtype=torch.float16, device=dev)
            nr = torch.zeros((R, H), device=dev)
            cand, ctr = router.norm_route_buffers(R, dev)

            def fused(i):
                r.copy_(hs[(i + 1) % 4])
                decode_split_norm(lay, cpu, 0, hs[i % 4], r, wp, x2, wn, xn, nr, 1e-5, cand, ctr)

            def launches(i):
                r.copy_(hs[(i + 1) % 4])
                router.norm_route(hs[i % 4], r, wp, x2, lay.wg, lay.bias, lay.sel[:R], lay.rw[:R], cand, ctr,
                                  lay.scale, 1e-5)
                cpu.submit(x2, lay.sel[:R], lay.rw[:R], 0)
                lay.experts_decode(R, nr, False, xh=x2)
                cpu.collect(nr)
                cn.combine_norm(None, 0, nr, R, 0, 0, r, wn, xn, 1e-5)
            # (alternating rounds, the median of each: the pool's time varies more between rounds than the launches
            # differ)
            ef, el_ = [], []
            for _ in range(5):
                ef.append(timed(torch, fused, steps, warmup))
                el_.append(timed(torch, launches, steps, warmup))
            el_f, el_l = float(np.median(ef)), float(np.median(el_))
            cpu.check()
            out[f"B{R}"] = {"us_per_step": el / steps * 1e6, "us_per_token": el / steps * 1e6 / R,
                            "gpu_tier_alone_us_per_step": el_gpu / steps * 1e6,
                            "cpu_experts_per_step_mean": float(np.mean(cold)),
                            "with_norms_fused_handoff_us_per_step": el_f / steps * 1e6,
                            "with_norms_handoff_launches_us_per_step": el_l / steps * 1e6}
    finally:
        torch.cuda.synchronize()
        cpu.close()
        os.sched_setaffinity(0, set(allowed))
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
    # (the synthetic codes, uniform in [-8, 7], have mean -0.5 and the group scales are positive, so every weight row
    # has a negative mean: each layer's output carries a common-mode term that the residual accumulates, and from the
    # third layer on the 4 rows' normalised inputs share it and pick mostly the same experts)
    res = {"layers": n_layers, "rows": R, "us_per_step": step_s * 1e6, "us_per_token": step_s * 1e6 / R,
           "distinct_experts_per_layer": float(U.mean()), "distinct_experts_by_layer": [int(u) for u in U],
           "bytes_per_step": b, "hbm_gbs": b / step_s / 1e9, "hbm_frac": b / step_s / 1e9 / HBM_PEAK_GBS}
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


def near_tie_audit(torch, synth, dev):
    """rows whose 8th and 9th selection scores (sigmoid(l) + bias) are closer than a different fp32 summation order of
    the logits could move them: the reference's fused router adds chunk partials in whatever order its atomics land
    (exl3_router.py:66-71), and it notes that its routers can resolve such near-ties differently (exl3_router.py:5-6).
    Bound per expert: 2^-24 sqrt(K) sum_k |x_k w_ek| (the statistical size of the rounding difference between two
    summation orders over K terms) times sigmoid'(l) = a (1 - a); a row is a near-tie when the gap is below the sum of
    its two experts' bounds"""
    import numpy as np
    torch.backends.cuda.matmul.allow_tf32 = False
    K = H
    out = {}
    cases = (("config0_b1", {}, 1, 64, 0), ("config1_b16_zipf", {"bias": synth.zipf_bias()}, 16, 16, 1000),
             ("config2_prefill_2048", {"bias_sigma": 0.001}, 2048, 1, 2))
    for name, kw, R, nx, tag0 in cases:
        wg, b = synth.router_weights(0, dev, **kw)
        rows = near = 0
        worst = float("inf")
        for i in range(nx):
            x = synth.gen_x(tag0 + i, R, dev).float()
            lg = x @ wg.t()
            a = torch.sigmoid(lg)
            sc = a + b
            top = sc.topk(9, dim=1)
            gap = top.values[:, 7] - top.values[:, 8]
            mag = x.abs() @ wg.abs().t()
            bound = 2.0 ** -24 * K ** 0.5 * mag * a * (1 - a)
            bnd = bound.gather(1, top.indices[:, 7:8])[:, 0] + bound.gather(1, top.indices[:, 8:9])[:, 0]
            rows += R
            near += int((gap < bnd).sum().item())
            worst = min(worst, float((gap / bnd).min().item()))
        out[name] = {"rows": rows, "near_ties": near, "min_gap_over_bound": worst}
    return out


def cpu_cores(cap=16):
    """the cores the CPU baseline runs on: the physical cores of the socket of this process's first allowed CPU, minus
    the first 4 (the reference runs 60 workers from core 12 of 72, tier_split.py:35-36, leaving the first cores to
    the serving process), capped at the box's CPU share for one GPU; returns (cores, description)"""
    allowed = sorted(os.sched_getaffinity(0))
    topo = {}
    for c in allowed:
        try:
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id") as f:
                pkg = int(f.read())
            with open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id") as f:
                core = int(f.read())
        except (OSError, ValueError):
            pkg, core = 0, c
        topo[c] = (pkg, core)
    sock = topo[allowed[0]][0]
    seen, phys = set(), []
    for c in allowed:
        if topo[c][0] == sock and topo[c][1] not in seen:
            seen.add(topo[c][1])
            phys.append(c)
    use = phys[4:] if len(phys) > 8 else phys
    use = use[:cap]
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
    except Exception:
        pass
    info = {"nproc": os.cpu_count(), "allowed_cpus": len(allowed), "cpu_model": model,
            "physical_cores_in_socket": len(phys), "threads": len(use), "first_core": use[0],
            "pinned": use == list(range(use[0], use[0] + len(use))),
            "cap_reason": f"all physical cores of the socket minus 4, at most {cap} (the box's CPU share per GPU)"}
    return use, info


def cpu_baseline():
    """the reference's CPU path timed on this host's cores: the routed experts on the pinned pool of
    hecate_amd/csrc/cputier.cpp (cpuband.cpp's jobs of <= 8 rows: q8_0 activations, int4 x int8 dots), the router and
    the shared expert (which the reference keeps on its GPU) through torch's CPU GEMMs (bf16 shared weights, fp32
    accumulation) on the same number of threads after the pool has stopped. Per config, on bounded samples (weights generated on the host
    for the experts the sampled inputs pick, not timed); config 2 has no CPU prefill in the reference (cpuband.cpp:7)
    and is timed as its 8-row jobs, an extension"""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import pyoracle as O
    from hostlayer import HostLayer, x_rows
    from hecate_amd import synth
    from hecate_amd.cpu_tier import CpuTier
    cores, info = cpu_cores()
    threads = len(cores)
    t_setup = time.perf_counter()
    cache = {}

    def expert(layer, e):
        k = (layer, e)
        if k not in cache:
            kk = lambda kind: synth.key(synth.SEED, layer, synth.KIND[kind], e)
            cache[k] = {"gate_q": O.codes(kk("GATE_Q"), 2048, H), "gate_s": O.scales(kk("GATE_S"), 2048, H, synth.SIG_SCALE),
                        "up_q": O.codes(kk("UP_Q"), 2048, H), "up_s": O.scales(kk("UP_S"), 2048, H, synth.SIG_SCALE),
                        "down_q": O.codes(kk("DOWN_Q"), H, 2048), "down_s": O.scales(kk("DOWN_S"), H, 2048, synth.SIG_SCALE)}
        return cache[k]

    # the sampled jobs: (config, pool layer, rows of x, sel, rw) and the host layers they need
    hl0 = HostLayer(0, shared=True)
    hlz = HostLayer(0, bias=synth.zipf_bias(layer=0), shared=False)
    hl2 = HostLayer(0, bias_sigma=0.001, shared=False)
    perm = synth.popularity_order()[:176]
    perm = list(perm) + [e for e in range(256) if e not in set(perm)]
    hl3 = HostLayer(0, perm=perm, n_hot=176, shared=False)
    x0 = [x_rows(i, 1) for i in range(8)]
    jobs = {"config0_b1": [], "config1_b16_zipf": [], "config3_b1": [], "config3_b4": [], "config3_b8": [],
            "config2_prefill_8row_jobs": []}
    r_s = {}                                                 # router + shared time per config (oracle, after the pool)
    for x in x0:
        sel, rw = hl0.route(x)
        jobs["config0_b1"].append((0, x, sel, rw))
    x16 = x_rows(1000, 16)
    sel, rw = hlz.route(x16)
    jobs["config1_b16_zipf"] += [(0, x16[j:j + 8], sel[j:j + 8], rw[j:j + 8]) for j in (0, 8)]
    for B in (1, 4, 8):
        xb = np.concatenate(x0[:B])
        sel, rw = hl3.route(xb)
        jobs[f"config3_b{B}"].append((1, xb, sel, rw))
    x2 = x_rows(2, 8)
    sel, rw = hl2.route(x2)
    jobs["config2_prefill_8row_jobs"].append((0, x2, sel, rw))
    # config 4: the first 4 of the 16 layers of the B = 4 stack (layer l is pool layer 10 + l), the chain computed on
    # the host with the oracle's q8_0 path between them so each layer's job sees its own inputs
    stack = []
    h = O.bf16_to_f32(x_rows(4, 4)).copy()
    y = None
    for l in range(4):
        w = O.normal_f32(synth.key(synth.SEED, l, synth.KIND["NORM_W"]), H, 1.0, 0.02)
        h, xn = O.residual_rmsnorm(h, y, w, 1e-5)
        hl = hl0 if l == 0 else HostLayer(l, shared=True)
        sel, rw = hl.route(xn)
        stack.append((10 + l, xn, sel, rw, hl))
        tab = O.ExpertTable([expert(l, e) if e in set(int(v) for v in sel.ravel()) else None for e in range(256)])
        y = O.moe(1, xn, sel, rw, tab, 0, 256, hl.shared, threads=threads)
    # the pool's layers: every needed expert generated; the window's other slots point at a generated one (never
    # picked by the sampled jobs)
    def pool_layer(layer, ids_needed, ids_of_local):
        ex = {e: expert(layer, e) for e in ids_needed}
        fill = ex[next(iter(ex))]
        return [ex.get(ids_of_local[j], fill) for j in range(len(ids_of_local))]
    need0 = set()
    for cfg in ("config0_b1", "config1_b16_zipf", "config2_prefill_8row_jobs"):
        for _, _, sel, _ in jobs[cfg]:
            need0 |= {int(e) for e in sel.ravel()}
    need3 = set()
    for B in (1, 4, 8):
        for _, _, sel, _ in jobs[f"config3_b{B}"]:
            need3 |= {perm[int(e)] for e in sel.ravel() if int(e) < 176}
    layers = {0: pool_layer(0, need0, list(range(256))), 1: pool_layer(0, need3, perm[:176])}
    for (pl, xn, sel, rw, hl) in stack:
        layers[pl] = pool_layer(pl - 10, {int(e) for e in sel.ravel()}, list(range(256)))
    setup_s = time.perf_counter() - t_setup
    log(f"[bench] cpu baseline: {len(cache)} experts generated in {setup_s:.1f} s, {threads} pool threads on cores "
        f"{cores[0]}..{cores[-1]}")
    # each config's sample is timed in rounds (a round = every sampled job of the config once) until at least MIN_S of
    # work and MIN_ROUNDS rounds; the median round is kept and the spread (10th to 90th percentile over the median)
    # reported, so the figure is stable from run to run
    MIN_S, MIN_ROUNDS = 0.12, 5

    def rounds_of(fn, items):
        fn(*items[0])                                        # untimed: caches, pages, thread wake-up
        out = []
        while len(out) < MIN_ROUNDS or sum(out) < MIN_S:
            out.append(sum(fn(*it) for it in items))
        return out
    tier = CpuTier(threads=threads, first_core=cores[0] if info["pinned"] else -1, mapped=False)
    pool_s = {}
    # the posting thread waits on a core outside the pool's (when there is one), so no pool thread shares its core
    allowed = sorted(os.sched_getaffinity(0))
    spare = [c for c in allowed if c not in set(cores)]
    if spare:
        os.sched_setaffinity(0, {spare[0]})
    try:
        for pl, ex in layers.items():
            tier.add_layer(pl, 0, ex)

        def run(pl, x, sel, rw):
            t0 = time.perf_counter()
            tier.post(x, sel, rw, pl)
            _, err = tier.wait()
            el = time.perf_counter() - t0
            if err:
                raise RuntimeError(f"cpu baseline: job error {err}")
            return el
        for cfg, js in jobs.items():
            pool_s[cfg] = rounds_of(run, js)
        pool_s["config4_stack_b4"] = rounds_of(run, [(pl, xn, sel, rw) for (pl, xn, sel, rw, _) in stack])
    finally:
        tier.close()
        os.sched_setaffinity(0, set(allowed))

    # router (fp32 logits, sigmoid + bias top-8) and shared expert (bf16 weights and activations, fp32 accumulation)
    # through torch's CPU GEMMs on the same number of threads, the pool stopped
    import torch
    import torch.nn.functional as F
    torch.set_num_threads(threads)
    tw = {}

    def cpu_weights(hl):
        if id(hl) not in tw:
            sh = None
            if hl.shared is not None:
                sh = [torch.from_numpy(m.view(np.int16)).view(torch.bfloat16) for m in hl.shared]
            tw[id(hl)] = (torch.from_numpy(hl.wg), torch.from_numpy(hl.bias), sh)
        return tw[id(hl)]

    def router_shared(hl, x, with_shared=True):
        wg, bias, sh = cpu_weights(hl)
        xb = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
        t0 = time.perf_counter()
        with torch.no_grad():
            a = torch.sigmoid(F.linear(xb.float(), wg))
            top = (a + bias).topk(8, dim=1)
            sa = a.gather(1, top.indices)
            rw = (sa * 2.5 / (sa.sum(1, keepdim=True) + 1e-20)).half()
            if with_shared:
                ys = F.linear(F.silu(F.linear(xb, sh[0])) * F.linear(xb, sh[1]), sh[2])
        return time.perf_counter() - t0
    # one untimed call per weight set first: torch's first CPU GEMM creates its thread pool and kernel caches
    for hl in [hl0, hl3] + [s[4] for s in stack]:
        router_shared(hl, x0[0], hl.shared is not None)
    r_s["config0_b1"] = rounds_of(router_shared, [(hl0, x) for x in x0])
    r_s["config1_b16_zipf"] = rounds_of(router_shared, [(hl0, x16)])
    for B in (1, 4, 8):
        r_s[f"config3_b{B}"] = rounds_of(router_shared, [(hl3, np.concatenate(x0[:B]), False)])
    r_s["config2_prefill_8row_jobs"] = rounds_of(router_shared, [(hl0, x2)])
    r_s["config4_stack_b4"] = rounds_of(router_shared, [(hl, xn) for (_, xn, _, _, hl) in stack])
    res = {}
    for cfg in pool_s:
        pr, rr = np.array(pool_s[cfg]), np.array(r_s[cfg])
        p, r = float(np.median(pr)), float(np.median(rr))
        rows = {"config0_b1": 8, "config1_b16_zipf": 16, "config3_b1": 1, "config3_b4": 4, "config3_b8": 8,
                "config2_prefill_8row_jobs": 8, "config4_stack_b4": 4}[cfg]
        n_steps = {"config0_b1": 8}.get(cfg, 1)
        step = (p + r) / n_steps
        if cfg == "config4_stack_b4":
            step = step * 16 / 4                             # 4 of the 16 layers sampled
        spread = lambda a: float((np.percentile(a, 90) - np.percentile(a, 10)) / np.median(a))
        res[cfg] = {"us_per_step": step * 1e6, "tok_per_s": (rows / n_steps) / step,
                    "pool_us": p / n_steps * 1e6, "router_shared_us": r / n_steps * 1e6,
                    "rounds": [len(pr), len(rr)], "timed_s": float(pr.sum() + rr.sum()),
                    "spread_p10_p90": [spread(pr), spread(rr)]}
    res["config2_prefill_8row_jobs"]["ms_per_2048_chunk"] = res["config2_prefill_8row_jobs"]["us_per_step"] * 256 / 1e3
    head = res["config0_b1"]
    info.update({"setup_s": setup_s, "experts_generated": len(cache)})
    return {"value": head["tok_per_s"], "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": (f"config 0 (B = 1): 8 tokens of layer 0 (one 1-row job each of the restated cpuband path on "
                       f"the pinned pool, then router and bf16 shared expert on torch's CPU GEMMs), timed in rounds of "
                       f"the 8 tokens until >= {MIN_S} s and {MIN_ROUNDS} rounds of each part, the median round kept; "
                       f"{info['cpu_model']}, {threads} threads from core {cores[0]}; per-config figures, round counts "
                       f"and spreads in configs"),
            "configs": res, "host": info}


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
    ap.add_argument("--only", default=None, choices=[None, "decode1", "decode16", "decode8", "prefill", "prefill8k",
                                                     "partial", "graph16", "copy", "tiered", "ties", "cpu"])
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
    if only in (None, "decode1"):
        head = decode_workload(torch, synth, 1, K, W, False, dev, tag0=0)
        log(f"[bench] decode1: {json.dumps(head)}")
    if only in (None, "decode8"):
        extra["decode_b8"] = decode_workload(torch, synth, 8, K, W, False, dev, tag0=500)
        log(f"[bench] decode8: {json.dumps(extra['decode_b8'])}")
    if only in (None, "decode16"):
        extra["decode_b16_zipf"] = decode_workload(torch, synth, 16, K, W, True, dev, tag0=1000)
        log(f"[bench] decode16: {json.dumps(extra['decode_b16_zipf'])}")
    if only in (None, "prefill"):
        extra["prefill_2048"] = prefill_workload(torch, synth, max(10, K // 10), max(2, W // 10), dev)
        log(f"[bench] prefill: {json.dumps(extra['prefill_2048'])}")
    if only in (None, "prefill8k"):
        extra["prefill_8192"] = prefill_workload(torch, synth, max(6, K // 30), 2, dev, T=8192)
        log(f"[bench] prefill8k: {json.dumps(extra['prefill_8192'])}")
    if only in (None, "partial"):
        extra["partial_176"] = partial_workload(torch, synth, K, W, dev)
        log(f"[bench] partial: {json.dumps(extra['partial_176'])}")
    if only in (None, "graph16"):
        extra["graph_16_layers_b4"] = graph_workload(torch, synth, max(20, K // 4), max(3, W // 4), dev)
        log(f"[bench] graph16: {json.dumps(extra['graph_16_layers_b4'])}")
    if only in (None, "tiered"):
        extra["tiered_176_cpu80"] = tiered_workload(torch, synth, max(20, K // 10), max(3, W // 4), dev)
        log(f"[bench] tiered: {json.dumps(extra['tiered_176_cpu80'])}")
    if only in (None, "ties"):
        extra["near_tie_audit"] = near_tie_audit(torch, synth, dev)
        log(f"[bench] ties: {json.dumps(extra['near_tie_audit'])}")
    if only == "copy":
        extra["copy_1gib"] = copy_workload(torch, max(10, K // 10), 3, dev)
    cpu = None
    if (only is None and not args.no_cpu) or only == "cpu":
        cpu = cpu_baseline()
        log(f"[bench] cpu: {json.dumps(cpu)}")
    if head is None:
        print(json.dumps({"extra": extra, "cpu_baseline": cpu}))
        return
    kb = head["kernels"]["B_gate_up"]
    roof = {"bound": "hbm", "kernel": "gu7_kernel (shared gate/up + top-8 selection + routed int4 gate/up + SwiGLU)",
            "achieved": kb["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": kb["gbs"] / HBM_PEAK_GBS,
            "traffic": traffic_from_profiles("gu7_kernel"), "algorithmic_bytes_per_launch": kb["algorithmic_bytes"],
            "launch_us": kb["us"], "layer_hbm_frac": head["hbm_frac"]}
    extra["decode_b1"] = head
    line = {"metric": metric_name(), "value": head["tok_per_s"], "unit": "tok/s", "n_gpus": 1, "steps": K,
            "warmup": W, "ms_per_step": head["us_per_step"] / 1e3, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16 (int4 weights, fp32 accumulation)", "data": "synthetic",
            "config": {"workload": "config 0, decode_b1: one routed int4 MoE layer step (router + top-8 of 256 int4 g128 "
                                   "experts + bf16 shared expert + bf16 out), 1 row",
                       "rows": 1, "hidden": H, "intermediate": 2048, "experts": 256, "topk": 8,
                       "us_per_token": head["us_per_token"], "hbm_gbs": head["hbm_gbs"],
                       "bytes_per_token": head["bytes_per_step"]},
            "roofline": roof, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
