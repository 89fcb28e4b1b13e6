"""The allocation-free decode entry (hmoe_moe4_forward_noalloc) through the C ABI against hmoe_moe4_forward on the
same inputs: the same kernels on a static workspace, so the same bits; two calls in a row, the second with fewer rows
(the workspace keeps the first call's contents, which must not leak into the second)."""
import ctypes

import numpy as np
import pytest
import torch

from hecate_amd import _lib, synth
from hecate_amd._lib import ptr

pytestmark = pytest.mark.gpu

H = 6144


def test_noalloc_matches_forward(dev):
    L = _lib.lib()
    assert L.hmoe_moe4_noalloc_bytes() == 21_762_048
    lay = synth.make_layer(0, dev)
    gq, uq, dq, gs, us, ds = lay.bank.tables()
    sh = lay.shared
    act, gu32, ctr_a, y32, ctr_b = lay.scr
    st = torch.cuda.current_stream().cuda_stream
    for R in (16, 3):                                           # the second call smaller than the first
        x = synth.gen_x(60 + R, R, dev)
        lay.route(x)
        xh = lay.xh[:R]
        sel, rw = lay.sel[:R], lay.rw[:R]
        p0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)
        y_ref, y_na = p0.clone(), p0.clone()
        print(f"noalloc R={R}", flush=True)
        _lib.check(L.hmoe_moe4_forward(ptr(xh), ptr(sel), ptr(rw), R, lay.n_hot, ptr(gq), ptr(uq), ptr(dq), ptr(gs),
                                       ptr(us), ptr(ds), ptr(act), ptr(gu32), ptr(ctr_a), ptr(y32), ptr(ctr_b),
                                       ptr(y_ref), 0, 0, 0, ptr(sh[0]), ptr(sh[1]), ptr(sh[2]), None, None, None,
                                       _lib.XF_F16, st), "forward")
        _lib.check(L.hmoe_moe4_forward_noalloc(ptr(xh), ptr(sel), ptr(rw), R, lay.n_hot, ptr(gq), ptr(uq), ptr(dq),
                                               ptr(gs), ptr(us), ptr(ds), ptr(y_na), 0, ptr(sh[0]), ptr(sh[1]),
                                               ptr(sh[2]), _lib.XF_F16, st), "forward_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(y_na, y_ref), R
        assert not torch.equal(y_na, p0)
    # beyond the static workspace: refused before any launch
    assert L.hmoe_moe4_forward_noalloc(ptr(xh), ptr(sel), ptr(rw), 17, lay.n_hot, ptr(gq), ptr(uq), ptr(dq), ptr(gs),
                                       ptr(us), ptr(ds), ptr(y_na), 0, None, None, None, _lib.XF_F16, st) == 1
    assert b"static workspace" in L.hmoe_last_error()
    del lay
    torch.cuda.empty_cache()


_CAPTURE_CHILD = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from hecate_amd import _lib, moe4, synth
dev = torch.device("cuda:0")
lay = synth.make_layer(0, dev)
gq, uq, dq, gs, us, ds = lay.bank.tables()
sh = lay.shared
for R in (4, 1):
    x = synth.gen_x(80 + R, R, dev)
    lay.route(x)
    xh, sel, rw = lay.xh[:R], lay.sel[:R], lay.rw[:R]
    y0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * 6144, dev, 0.0, 0.1).view(R, 6144)
    y = y0.clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):                 # R = 4: the process's first call of the entry, inside the capture
        moe4.forward_noalloc(xh, sel, rw, lay.n_hot, gq, uq, dq, gs, us, ds, y, 0, sh[0], sh[1], sh[2])
    y_ref = y0.clone()
    moe4.forward(xh, sel, rw, lay.n_hot, gq, uq, dq, gs, us, ds, *lay.scr, y_ref, 0, 0, 0, sh[0], sh[1], sh[2], 0, 0, 0)
    for rep in range(3):
        y.copy_(y0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), (R, rep)
        junk = torch.randn(1 << 20, device=dev).sum()       # eager work between replays
        torch.cuda.synchronize()
    del g
print("capture ok", flush=True)
"""


def test_noalloc_first_call_under_capture(dev):
    """in a fresh process (the workspace's device address not yet looked up), the first call of the allocation-free
    entry is made under hipGraph capture; three replays (with eager work between) give the bits of
    hmoe_moe4_forward, at R = 4 (down partials + ordered output) and R = 1 (the owning down form)"""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "capture ok" in r.stdout
