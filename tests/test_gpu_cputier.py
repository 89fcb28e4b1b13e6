"""The host-CPU expert tier behind the GPU tier (config 3's tiered split): the 176 resident experts on the GPU, the
other 80 on the host pool, joined on one stream through the device-mapped mailbox. The CPU partial is the oracle's
q8_0 mode (runtime/tier/cpuband.cpp restated) bit for bit, the joined output is the GPU tier's own output plus that
partial, in fp32, bit for bit."""
import numpy as np
import pytest
import torch

import pyoracle as O
from hecate_amd import synth
from hecate_amd.cpu_tier import CpuTier, decode_split, host_experts
from hostref import HostLayer, H

pytestmark = pytest.mark.gpu
N_RES = 176


def log(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def split(dev):
    """the layer's 176 most popular experts resident on the GPU, the other 80 on an 8-thread host pool; the pool is
    stopped and the mailbox freed when the module ends"""
    lay = synth.make_layer(0, dev, resident=synth.popularity_order()[:N_RES], shared=False)
    hl = HostLayer(0, perm=lay.perm, n_hot=256, shared=False)
    cold = host_experts(0, lay.perm[N_RES:], dev)
    cpu = CpuTier(threads=8)
    try:
        cpu.add_layer(0, N_RES, cold)
        yield dict(lay=lay, hl=hl, cold=cold, cpu=cpu)
    finally:
        torch.cuda.synchronize()
        cpu.close()


def test_host_experts_match_the_generator(split):
    s = split
    for j in (0, 41, 79):
        a, b = s["cold"][j], s["hl"].expert(N_RES + j)
        for k in a:
            assert np.array_equal(a[k], b[k]), (j, k)


@pytest.mark.parametrize("R", [1, 4, 8])
def test_tiered_split_decode(dev, split, R):
    log(f"tiered split R={R}")
    s = split
    lay, hl, cpu = s["lay"], s["hl"], s["cpu"]
    x = synth.gen_x(7000 + R, R, dev)
    p0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)
    y = p0.clone()
    jobs0 = cpu.stats()[0]
    sel, rw = decode_split(lay, cpu, 0, x, y)
    torch.cuda.synchronize()
    cpu.check()
    assert cpu.stats()[0] == jobs0 + 1
    sel_h, rw_h = sel.cpu().numpy(), rw.cpu().numpy().view(np.uint16)
    cold = sel_h >= N_RES
    log(f"  cold picks {int(cold.sum())} of {sel_h.size}")
    # the GPU tier alone, on the same routing
    y_gpu = p0.clone()
    lay.experts_decode(R, y_gpu, False)
    torch.cuda.synchronize()
    need = sorted({int(e) - N_RES for e in sel_h[cold]})
    table = O.ExpertTable([hl.expert(N_RES + j) if j in need else None for j in range(256 - N_RES)])
    xn = x.cpu().view(torch.int16).numpy().view(np.uint16)
    cpu_ref = O.moe(1, xn, sel_h, rw_h, table, N_RES, 256 - N_RES, None, threads=16)
    got_cpu = np.ctypeslib.as_array(cpu.mb.out)[:R * H].reshape(R, H)
    assert np.array_equal(got_cpu.view(np.uint32), cpu_ref.view(np.uint32))
    want = y_gpu.cpu().numpy() + cpu_ref
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_tiered_split_replays_in_a_graph(dev, split):
    """the hand-off and collect kernels captured in a hipGraph with the GPU tier: each replay, on a new input, runs
    one CPU job and gives the eager bits; eager steps on other inputs run between the replays"""
    s = split
    lay, cpu = s["lay"], s["cpu"]
    R = 4
    xs = [synth.gen_x(7100 + i, R, dev) for i in range(4)]
    p0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)
    refs = []
    for x in xs:
        y = p0.clone()
        decode_split(lay, cpu, 0, x, y)
        torch.cuda.synchronize()
        cpu.check()
        refs.append(y)
    assert not torch.equal(refs[0], refs[1])
    xg = xs[3].clone()
    yg = torch.empty_like(p0)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        yg.copy_(p0)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            yg.copy_(p0)
            decode_split(lay, cpu, 0, xg, yg)
    torch.cuda.synchronize()
    cpu.check()
    j0 = cpu.stats()[0]
    for i in range(3):
        xg.copy_(xs[i])
        g.replay()
        torch.cuda.synchronize()
        cpu.check()
        assert torch.equal(yg, refs[i]), i
        y2 = p0.clone()
        decode_split(lay, cpu, 0, xs[(i + 1) % 3], y2)
        torch.cuda.synchronize()
        cpu.check()
        assert torch.equal(y2, refs[(i + 1) % 3]), i
    assert cpu.stats()[0] == j0 + 6


def _norm_inputs(R, dev, seed):
    g = torch.Generator().manual_seed(seed)
    h = (torch.randn((R, H), generator=g) * 0.5).to(dev)
    r0 = (torch.randn((R, H), generator=g) * 2.0).to(dev)
    w_post = (1.0 + 0.02 * torch.randn(H, generator=g)).to(dev)
    w_next = (1.0 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    return h, r0, w_post, w_next


def _launch_form(lay, cpu, h, r, w_post, w_next, x2, xn, nr, eps):
    """the same step with the hand-off and the collect as launches of their own: norm_route, cpu submit, the resident
    experts, cpu collect into nr, combine_norm of nr"""
    from hecate_amd import cn, router
    R = h.shape[0]
    cand, ctr = router.norm_route_buffers(R, h.device)
    router.norm_route(h, r, w_post, x2, lay.wg, lay.bias, lay.sel[:R], lay.rw[:R], cand, ctr, lay.scale, eps)
    cpu.submit(x2, lay.sel[:R], lay.rw[:R], 0)
    lay.experts_decode(R, nr, False, xh=x2)
    cpu.collect(nr)
    cn.combine_norm(None, 0, nr, R, 0, 0, r, w_next, xn, eps)


@pytest.mark.parametrize("R", [1, 4, 8])
def test_tiered_fused_handoff_matches_the_launch_form(dev, split, R):
    """norm_route posting the CPU tier's job in its selection launch and combine_norm_cpu adding the pool's partial
    once the job is done (the reference's nr4 hand-off and cn CPU_DONE form) give the bits of the same step with the
    hand-off and the collect as launches of their own: x2, the routing, r and the next layer's xn; one pool job per
    step, the accumulator left zeroed"""
    from hecate_amd.cpu_tier import decode_split_norm
    log(f"fused hand-off R={R}")
    s = split
    lay, cpu = s["lay"], s["cpu"]
    h, r0, w_post, w_next = _norm_inputs(R, dev, 60 + R)
    eps = 1e-5
    outs = []
    for fused in (True, False):
        r = r0.clone()
        x2 = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
        xn = torch.empty((R, H), dtype=torch.float16, device=dev)
        nr = torch.zeros((R, H), dtype=torch.float32, device=dev)
        jobs0 = cpu.stats()[0]
        if fused:
            decode_split_norm(lay, cpu, 0, h, r, w_post, x2, w_next, xn, nr, eps)
        else:
            _launch_form(lay, cpu, h, r, w_post, w_next, x2, xn, nr, eps)
        torch.cuda.synchronize()
        cpu.check()
        assert cpu.stats()[0] == jobs0 + 1
        assert not bool(nr.any())
        outs.append((x2.view(torch.int16).clone(), lay.sel[:R].clone(), lay.rw[:R].view(torch.int16).clone(),
                     r.view(torch.int32).clone(), xn.view(torch.int16).clone()))
    log(f"  cold picks {int((outs[0][1] >= N_RES).sum())} of {outs[0][1].numel()}")
    for name, a, b in zip(("x2", "sel", "rw", "r", "xn"), outs[0], outs[1]):
        assert torch.equal(a, b), name


def test_tiered_fused_handoff_replays_in_a_graph(dev, split):
    """the fused step (norm_route with the hand-off, the resident experts, combine_norm_cpu) captured in a hipGraph:
    each replay, on new inputs, runs one CPU job and gives the eager bits; eager steps run between the replays"""
    from hecate_amd.cpu_tier import decode_split_norm
    s = split
    lay, cpu = s["lay"], s["cpu"]
    R, eps = 4, 1e-5
    ins = [_norm_inputs(R, dev, 80 + i) for i in range(4)]
    w_post, w_next = ins[0][2], ins[0][3]

    def eager(i):
        h, r0 = ins[i][0], ins[i][1]
        r = r0.clone()
        x2 = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
        xn = torch.empty((R, H), dtype=torch.float16, device=dev)
        nr = torch.zeros((R, H), dtype=torch.float32, device=dev)
        decode_split_norm(lay, cpu, 0, h, r, w_post, x2, w_next, xn, nr, eps)
        torch.cuda.synchronize()
        cpu.check()
        return r.clone(), xn.clone()

    refs = [eager(i) for i in range(3)]
    assert not torch.equal(refs[0][1], refs[1][1])
    from hecate_amd import router
    hg, rg, r0g = ins[3][0].clone(), ins[3][1].clone(), ins[3][1].clone()
    x2g = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
    xng = torch.empty((R, H), dtype=torch.float16, device=dev)
    nrg = torch.zeros((R, H), dtype=torch.float32, device=dev)
    cand, ctr = router.norm_route_buffers(R, dev)
    st = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        rg.copy_(r0g)
        decode_split_norm(lay, cpu, 0, hg, rg, w_post, x2g, w_next, xng, nrg, eps, cand, ctr)
        torch.cuda.synchronize()
        cpu.check()
        with torch.cuda.graph(g, stream=st):
            rg.copy_(r0g)
            decode_split_norm(lay, cpu, 0, hg, rg, w_post, x2g, w_next, xng, nrg, eps, cand, ctr)
    torch.cuda.synchronize()
    cpu.check()
    j0 = cpu.stats()[0]
    for i in range(3):
        hg.copy_(ins[i][0])
        r0g.copy_(ins[i][1])
        g.replay()
        torch.cuda.synchronize()
        cpu.check()
        assert torch.equal(rg, refs[i][0]) and torch.equal(xng, refs[i][1]), i
        assert not bool(nrg.any())
        r2, xn2 = eager((i + 1) % 3)
        assert torch.equal(r2, refs[(i + 1) % 3][0]) and torch.equal(xn2, refs[(i + 1) % 3][1]), i
    assert cpu.stats()[0] == j0 + 6
