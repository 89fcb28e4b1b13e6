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
