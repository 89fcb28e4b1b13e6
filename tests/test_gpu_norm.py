"""GPU parity of the norm operators through the C ABI against the oracle's restatement of the reference's
rms_norm_kernel order (oracle/hmoe_oracle.c orc_rmsnorm_cn, pinned in tests/test_oracle.py): combine_norm
(runtime/tier/cn.cu:189-235) and norm_route (runtime/core/exl3_normroute.py:16-65, nr4_kernel.cuh:122-381). The
residual update and the normed rows are bit-exact (the reference's own criterion for its fused norms,
nr4_kernel.cuh:4-9, cn.cu:1-6), the routing bit-exact."""
import numpy as np
import pytest
import torch

import pyoracle as O
from hecate_amd import cn, router

pytestmark = pytest.mark.gpu
H = 6144


def log(*a):
    print(*a, flush=True)


def bits(t):
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


@pytest.mark.parametrize("rows,wdt,xdt,cbias,cscale,use_f,use_o", [
    (1, torch.float16, torch.float16, 0.0, 1.0, True, False),
    (3, torch.bfloat16, torch.float16, 0.5, 1.0, True, True),
    (8, torch.float32, torch.bfloat16, 0.0, 0.75, False, True),
    (64, torch.float16, torch.bfloat16, -0.25, 1.25, True, True),
])
def test_combine_norm_bit_exact(dev, rows, wdt, xdt, cbias, cscale, use_f, use_o):
    """a = ((f + y) + o) + o2 (f None reads as +0), y zeroed, r = a + r, xn = RMSNorm(r) * (w + cbias) * cscale in the
    rms_norm_kernel order: r, xn bit-exact against the oracle, y zero afterwards; two calls in a row (the second on the
    first's residual) each exact"""
    log(f"combine_norm rows={rows} w={wdt} xn={xdt} cbias={cbias} cscale={cscale} f={use_f} o={use_o}")
    g = torch.Generator().manual_seed(rows * 7 + int(use_f) + 2 * int(use_o))
    w = (1.0 + 0.02 * torch.randn(H, generator=g)).to(wdt)
    r = (torch.randn((rows, H), generator=g) * 3.0).to(dev)
    xn = torch.empty((rows, H), dtype=xdt, device=dev)
    wd = w.to(dev)
    wf = f32(w.float().numpy())
    for call_no in range(2):
        f = (torch.randn((rows, H), generator=g) * 0.5).to(dev) if use_f else None
        y = torch.randn((rows, H), generator=g).to(dev)
        o = (torch.randn((rows, H), generator=g) * 0.1).to(dev) if use_o else None
        o2 = (torch.randn((rows, H), generator=g) * 0.1).to(dev) if use_o else None
        a = f32(f.cpu().numpy()) if use_f else np.zeros((rows, H), np.float32)
        a = f32(a + y.cpu().numpy())
        if use_o:
            a = f32(a + o.cpu().numpy())
            a = f32(a + o2.cpu().numpy())
        r_ref = f32(a + r.cpu().numpy())
        cn.combine_norm(f, ptr_of(o), y, rows, ptr_of(o2), 0, r, wd, xn, 1e-5, cbias, cscale)
        torch.cuda.synchronize()
        assert np.array_equal(bits(r), r_ref.view(np.int32)), call_no
        xn_ref = O.rmsnorm_cn(r_ref, wf, 1e-5, cbias, cscale, bf16=xdt == torch.bfloat16)
        assert np.array_equal(bits(xn), xn_ref), call_no
        assert not bool(y.any())


def ptr_of(t):
    return 0 if t is None else t.data_ptr()


@pytest.mark.parametrize("R,gdt,xdt,wdt,cbias,cscale", [
    (1, torch.float32, torch.bfloat16, torch.float32, 0.0, 1.0),
    (2, torch.float16, torch.float16, torch.float16, 0.0, 1.0),
    (4, torch.float16, torch.float16, torch.bfloat16, 0.125, 1.0),
    (8, torch.float32, torch.float16, torch.float16, 0.0, 0.5),
    (16, torch.float16, torch.bfloat16, torch.float32, 0.0, 1.0),
])
def test_norm_route_bit_exact(dev, R, gdt, xdt, wdt, cbias, cscale):
    """r = y + r and x2 = RMSNorm(r) bit-exact against the oracle, y untouched; the routing (sel, rw) of x2 against the
    gate (the reference's f16 [E, H] or fp32) bit-exact against the oracle's router (fixed-order logits, sigmoid +
    bias keys, ties to the lowest index); with bf16 x2 and an fp32 gate, the same routing as router_fused on x2"""
    log(f"norm_route R={R} gate={gdt} x2={xdt} w={wdt}")
    g = torch.Generator().manual_seed(100 + R)
    y = (torch.randn((R, H), generator=g) * 0.5).to(dev)
    r = (torch.randn((R, H), generator=g) * 2.0).to(dev)
    w = (1.0 + 0.02 * torch.randn(H, generator=g)).to(wdt).to(dev)
    gt = (torch.randn((256, H), generator=g) * 0.02).to(gdt).to(dev)
    bias = (torch.randn(256, generator=g) * 0.01).to(dev)
    x2 = torch.empty((R, H), dtype=xdt, device=dev)
    sel = torch.empty((R, 8), dtype=torch.int64, device=dev)
    rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
    cand, ctr = router.norm_route_buffers(R, dev)
    y0, r0 = y.clone(), r.cpu().numpy()
    router.norm_route(y, r, w, x2, gt, bias, sel, rw, cand, ctr, 2.5, 1e-5, cbias, cscale)
    torch.cuda.synchronize()
    assert torch.equal(bits_t(y), bits_t(y0))
    r_ref = f32(y0.cpu().numpy() + r0)
    assert np.array_equal(bits(r), r_ref.view(np.int32))
    bf = xdt == torch.bfloat16
    x2_ref = O.rmsnorm_cn(r_ref, f32(w.float().cpu().numpy()), 1e-5, cbias, cscale, bf16=bf)
    assert np.array_equal(bits(x2), x2_ref)
    x2f = O.bf16_to_f32(x2_ref) if bf else O.f16_to_f32(x2_ref)
    lg = O.router_logits_f32(x2f, f32(gt.float().cpu().numpy()))
    sel_ref, rw_ref = O.router_select(lg, f32(bias.cpu().numpy()))
    assert np.array_equal(sel.cpu().numpy(), sel_ref)
    assert np.array_equal(bits(rw), rw_ref)
    if bf and gdt == torch.float32:
        logits, c2 = router.buffers(R, dev)
        s2, w2 = torch.empty_like(sel), torch.empty_like(rw)
        router.router_fused(x2, gt, bias, logits, c2, s2, w2, 8, 2.5)
        torch.cuda.synchronize()
        assert torch.equal(s2, sel) and torch.equal(bits_t(w2), bits_t(rw))


def bits_t(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


@pytest.mark.parametrize("R,nparts", [(4, 0), (4, 1), (4, 5), (4, 8), (4, 9), (16, 16), (16, 17), (2, 33)])
def test_decode_combine_norm_part_counts(dev, R, nparts):
    """the decode stack's output launch fused with the next norm (hmoe_decode_combine_norm): the down launch's part
    partials summed in part order from +0 (as many as its count says, across the batch boundaries of 8), r = s + r, xn
    = RMSNorm(r) in the rms_norm_kernel order: r and xn bit-exact against the oracle; parts past the count are never
    added (they hold values that would change the bits)"""
    from hecate_amd._lib import DT_BF16, DT_F32, call, ptr, stream_of
    log(f"decode_combine_norm R={R} parts={nparts}")
    MAX_PARTS, MAXR = 33, 16
    g = torch.Generator().manual_seed(100 * R + nparts)
    y32 = torch.randn((MAX_PARTS, MAXR, H), generator=g)
    r = torch.randn((R, H), generator=g) * 3.0
    w = (1.0 + 0.02 * torch.randn(H, generator=g)).float()
    s = np.zeros((R, H), np.float32)
    yh = y32.numpy()
    for p in range(nparts):
        s = f32(s + yh[p, :R])
    r_ref = f32(s + r.numpy())
    xn_ref = O.rmsnorm_cn(r_ref, f32(w.numpy()), 1e-5, 0.0, 1.0, bf16=True)
    y32d, rd, wd = y32.to(dev), r.to(dev), w.to(dev)
    ctr = torch.tensor([nparts, 0, 0, 0], dtype=torch.int32, device=dev)
    xn = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
    call("hmoe_decode_combine_norm", ptr(y32d), ptr(ctr), R, ptr(rd), ptr(wd), ptr(xn), None, 1e-5, 0.0, 1.0, DT_F32,
         DT_BF16, stream_of(dev))
    torch.cuda.synchronize()
    assert np.array_equal(bits(rd), r_ref.view(np.int32))
    assert np.array_equal(bits(xn), xn_ref)
