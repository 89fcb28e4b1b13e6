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
