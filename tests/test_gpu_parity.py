"""GPU parity of the HIP path against the CPU oracle, through the C ABI (hecate_amd wraps it with ctypes).

Bars: routing (sel, rw), dispatch plans and generated data bit-exact; layer outputs within max |d| <= 2e-2 and
mean |d| / mean |ref| <= 5e-3 of the oracle's exact mode, compared in fp32 before output rounding.
"""
import numpy as np
import pytest
import torch

import pyoracle as O
import torchref
from hecate_amd import moe4, moe4p, moe4t, router, synth, tier
from hecate_amd.stack import DecodeStack
from hecate_amd._lib import call, ptr
from hostref import HostLayer, x_rows, parity, parity_ulp, MAX_ABS, MEAN_REL, H, I, E

pytestmark = pytest.mark.gpu


def u16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def log(*a):
    print(*a, flush=True)


# ---- generators, formats -----------------------------------------------------------------------------------------

@pytest.mark.parametrize("N,K", [(32, 512), (I, H), (H, I)])
def test_gen_i4_matches_host(dev, N, K):
    kq, ks = synth.key(7, 1, 3, 5), synth.key(7, 1, 6, 5)
    q = torch.empty(N * K // 2, dtype=torch.uint8, device=dev)
    s = torch.empty(N * (K // 128), dtype=torch.int16, device=dev)
    call("hmoe_gen_i4", kq, ks, 0.004, N, K, ptr(q), ptr(s), torch.cuda.current_stream().cuda_stream)
    qh = q.cpu().numpy(); sh = s.cpu().numpy().view(np.uint16)
    codes = np.empty((N, K // 2), np.uint8); scales = np.empty((N, K // 128), np.uint16)
    call("hmoe_unpack_i4", qh.ctypes.data, sh.ctypes.data, N, K, codes.ctypes.data, scales.ctypes.data)
    assert np.array_equal(codes, O.codes(kq, N, K))
    assert np.array_equal(scales, O.scales(ks, N, K, 0.004))


def test_gen_dense_and_normal_match_host(dev):
    k = synth.key(3, 0, 9, 0)
    N, K = 64, 256
    t = torch.empty(N * K, dtype=torch.float16, device=dev)
    call("hmoe_gen_dense", k, 0.02, N, K, ptr(t), torch.cuda.current_stream().cuda_stream)
    ref_bf = O.normal_bf16(k, N * K, 0.02).reshape(N, K)
    packed = np.empty(N * K, np.uint16)
    call("hmoe_pack_dense", ref_bf.ctypes.data, N, K, packed.ctypes.data)
    assert np.array_equal(u16(t), packed)
    for dt, fn in ((torch.float32, lambda: O.normal_f32(k, 4099, 0.5, 0.1)), (torch.bfloat16, lambda: O.normal_bf16(k, 4099, 1.0))):
        g = synth.gen_normal(k, 4099, dev, 0.5 if dt == torch.float32 else 0.0, 0.1 if dt == torch.float32 else 1.0, dt)
        got = g.cpu().numpy() if dt == torch.float32 else u16(g)
        assert np.array_equal(got.view(np.uint32 if dt == torch.float32 else np.uint16),
                              fn().view(np.uint32 if dt == torch.float32 else np.uint16))


def test_dequant_exact(dev):
    kq, ks = synth.key(1, 0, 3, 2), synth.key(1, 0, 6, 2)
    N, K = 128, 512
    q = torch.empty(N * K // 2, dtype=torch.uint8, device=dev)
    s = torch.empty(N * (K // 128), dtype=torch.int16, device=dev)
    call("hmoe_gen_i4", kq, ks, 0.004, N, K, ptr(q), ptr(s), torch.cuda.current_stream().cuda_stream)
    got = u16(moe4.dequant(q, s, N, K))
    ref = O.f32_to_f16(O.dequant(O.codes(kq, N, K), O.scales(ks, N, K, 0.004), N, K))
    assert np.array_equal(got, ref)


# ---- router ------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("R,bias_sigma", [(1, 0.01), (4, 0.01), (16, 0.01), (17, 0.001), (300, 0.001)])
def test_router_bit_exact(dev, R, bias_sigma):
    log(f"router R={R}")
    hl = HostLayer(0, bias_sigma=bias_sigma, shared=False)
    x = x_rows(100 + R, R)
    sel_ref, rw_ref = hl.route(x)
    xt = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    wg = torch.from_numpy(hl.wg).to(dev); b = torch.from_numpy(hl.bias).to(dev)
    logits, ctr = router.buffers(R, dev)
    sel = torch.empty((R, 8), dtype=torch.int64, device=dev); rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
    xh = torch.empty((R, H), dtype=torch.float16, device=dev)
    for _ in range(2):                       # repeated calls on the same scratch
        router.router_fused(xt, wg, b, logits, ctr, sel, rw, 8, 2.5, xh)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy(), sel_ref)
    assert np.array_equal(u16(rw), rw_ref)
    assert np.array_equal(u16(xh), O.f32_to_f16(O.bf16_to_f32(x)))


def _adversarial(rng, shape, f32):
    """values across 2^-12 .. 2^12 with exact zeros of both signs and subnormals (bf16 rows when not f32)"""
    v = (rng.standard_normal(shape) * np.exp2(rng.integers(-12, 13, shape))).astype(np.float32)
    m = rng.random(shape)
    v[m < 0.05] = 0.0
    v[(m >= 0.05) & (m < 0.1)] = -0.0
    v[(m >= 0.1) & (m < 0.13)] *= np.float32(2.0 ** -130)               # fp32 / bf16 subnormals
    if f32:
        return v
    return (v.view(np.uint32) >> 16).astype(np.uint16)                    # truncation to bf16 bits


@pytest.mark.parametrize("R,E,adv", [(300, 160, False), (4100, 200, False), (40, 64, True)])
def test_router_large_path_partial_tiles(dev, R, E, adv):
    """the large path's segment GEMM (fp32 MFMA, 128 rows x 64 experts per workgroup) on partial tiles: 300 and 4100
    rows with fewer experts than a whole tile covers, and 40 rows of adversarial operands (magnitudes across 2^+-12,
    signed zeros, subnormals); the folded logits, the selection and the weights bit-exact with the oracle's fixed
    order (each MFMA is a fmaf chain over its 4 k)"""
    log(f"router large path R={R} E={E} adversarial={adv}")
    rng = np.random.default_rng(R + E)
    if adv:
        x, wg = _adversarial(rng, (R, H), False), _adversarial(rng, (E, H), True)
    else:
        x = x_rows(7 + R, R)
        wg = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.001).astype(np.float32)
    lg_ref = O.router_logits(x, wg)
    sel_ref, rw_ref = O.router_select(lg_ref, bias)
    xt = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    logits, ctr = router.buffers(R, dev)
    sel = torch.empty((R, 8), dtype=torch.int64, device=dev); rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
    router.router_fused(xt, torch.from_numpy(wg).to(dev), torch.from_numpy(bias).to(dev), logits, ctr, sel, rw, 8, 2.5)
    torch.cuda.synchronize()
    # the large path leaves the 8 segment planes [8][R][256] in logits: folded in order from +0 they are the logits
    seg = logits[:8 * R * 256].view(8, R, 256).cpu().numpy()[:, :, :E]
    tot = np.zeros((R, E), np.float32)
    for s_ in range(8):
        tot = (tot + seg[s_]).astype(np.float32)
    assert np.array_equal(tot.view(np.uint32), np.asarray(lg_ref, np.float32).view(np.uint32))
    assert np.array_equal(sel.cpu().numpy(), sel_ref)
    assert np.array_equal(u16(rw), rw_ref)


@pytest.mark.parametrize("R", [4, 20])
def test_router_forced_tie_lowest_index(dev, R):
    """the forced tie of the oracle's test at the top-8 boundary through both router paths (R <= 16, R > 16): an
    exact tie of experts 40 and 41 picks 40, a key one or two ulps higher picks its expert; bit-exact with the
    oracle"""
    from test_oracle import forced_tie_router
    for lo, hi, near in ((40, 41, False), (41, 40, False), (40, 41, True), (41, 40, True)):
        x, wg, bias = forced_tie_router(R, lo, hi, near)
        sel_ref, rw_ref = O.router(x, wg, bias)
        xt = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
        logits, ctr = router.buffers(R, dev)
        sel = torch.empty((R, 8), dtype=torch.int64, device=dev)
        rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
        router.router_fused(xt, torch.from_numpy(wg).to(dev), torch.from_numpy(bias).to(dev), logits, ctr, sel, rw,
                            8, 2.5)
        torch.cuda.synchronize()
        assert np.array_equal(sel.cpu().numpy(), sel_ref) and np.array_equal(u16(rw), rw_ref)
        assert all(r[7] == (hi if near else 40) for r in sel_ref)


# ---- decode ------------------------------------------------------------------------------------------------------

_LAYERS = {}
_HOSTS = {}


def host_layer(layer=0, **kw):
    """HostLayer cached across tests (its experts are regenerated on first use only); kw: scalar options"""
    key = (layer, tuple(sorted(kw.items())))
    if key not in _HOSTS:
        _HOSTS[key] = HostLayer(layer, **kw)
    return _HOSTS[key]


def gpu_layer(name, dev, **kw):
    if name not in _LAYERS:
        _LAYERS.clear()
        torch.cuda.empty_cache()
        _LAYERS[name] = synth.make_layer(device=dev, **kw)
    return _LAYERS[name]


def decode_fp32(lay, x, dev, with_shared=True, y0=None):
    R = x.shape[0]
    lay.route(x)
    y = torch.zeros((R, H), dtype=torch.float32, device=dev) if y0 is None else y0.clone()
    lay.experts_decode(R, y, with_shared)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("R", [1, 3, 4, 8, 13, 16])
def test_decode_layer_parity(dev, R):
    log(f"decode R={R}")
    lay = gpu_layer("c0", dev, layer=0)
    hl = host_layer(0)
    x = synth.gen_x(R, R, dev)
    xn = u16(x)
    assert np.array_equal(xn, x_rows(R, R))
    y = decode_fp32(lay, x, dev).cpu().numpy()
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(lay.sel[:R].cpu().numpy(), sel_ref)
    assert np.array_equal(u16(lay.rw[:R]), rw_ref)
    ref = hl.moe(xn, sel_ref, rw_ref)
    ma, mr = parity(y, ref)
    log(f"  max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL
    # bit-reproducible: a second call (same scratch) gives the same bits
    y2 = decode_fp32(lay, x, dev).cpu().numpy()
    assert np.array_equal(y, y2)


def test_decode_zipf_16(dev):
    log("decode zipf R=16")
    bias = synth.zipf_bias()
    lay = gpu_layer("c1", dev, layer=0, bias=bias)
    hl = HostLayer(0, bias=bias)
    x = synth.gen_x(1001, 16, dev)
    xn = u16(x)
    y = decode_fp32(lay, x, dev).cpu().numpy()
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(lay.sel[:16].cpu().numpy(), sel_ref)
    ref = hl.moe(xn, sel_ref, rw_ref)
    ma, mr = parity(y, ref)
    log(f"  U={len(np.unique(sel_ref))} max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL


@pytest.mark.parametrize("R", [1, 4, 8])
def test_partial_resident_176(dev, R):
    log(f"partial R={R}")
    res = synth.popularity_order()[:176]
    lay = gpu_layer("c3", dev, layer=0, resident=res, shared=False)
    hl = HostLayer(0, perm=lay.perm, n_hot=176, shared=False)
    x = synth.gen_x(3000 + R, R, dev)
    xn = u16(x)
    p0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)
    y = decode_fp32(lay, x, dev, with_shared=False, y0=p0).cpu().numpy()
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(lay.sel[:R].cpu().numpy(), sel_ref)
    ref = O.moe(0, xn, sel_ref, rw_ref, hl.table(sel_ref), 0, 176, None, out=p0.cpu().numpy().copy(), accumulate=True,
                threads=16)
    ma, mr = parity(y, ref)
    log(f"  max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL
    # the same partial through the four launches of hmoe_moe_decode_layer (router logits, selection inside the gate/up
    # launch, y accumulated, no shared expert, no bf16 out): the same selection and the same bound
    yf = p0.clone()
    assert lay.decode(x, y=yf, out=False, with_shared=False) is None
    torch.cuda.synchronize()
    assert np.array_equal(lay.sel[:R].cpu().numpy(), sel_ref)
    ma, mr = parity(yf.cpu().numpy(), ref)
    log(f"  fused layer op: max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL
    # picks outside the window change nothing: all-absent selection leaves the partial as it was
    sel_out = torch.full((R, 8), 200, dtype=torch.int64, device=dev)
    lay.sel[:R].copy_(sel_out)
    y0 = p0.clone()
    lay.experts_decode(R, y0, False)
    torch.cuda.synchronize()
    assert torch.equal(y0, p0)


@pytest.mark.parametrize("R", [1, 16])
def test_decode_layer_fused(dev, R):
    """router + experts in the four launches of hmoe_moe_decode_layer; bf16 out = rounded fp32 sum"""
    log(f"fused decode R={R}")
    lay = gpu_layer("c0", dev, layer=0)
    hl = host_layer(0)
    x = synth.gen_x(50 + R, R, dev)
    xn = u16(x)
    y = torch.zeros((R, H), dtype=torch.float32, device=dev)
    out = lay.decode(x, y=y)
    torch.cuda.synchronize()
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(lay.sel[:R].cpu().numpy(), sel_ref)
    assert np.array_equal(u16(lay.rw[:R]), rw_ref)
    yh = y.cpu().numpy()
    ma, mr = parity(yh, hl.moe(xn, sel_ref, rw_ref))
    log(f"  max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL
    assert np.array_equal(u16(out), O.f32_to_bf16(yh))


@pytest.mark.parametrize("lo,n_hot", [(64, 160), (256, 256)])
def test_decode_window_offset(dev, lo, n_hot):
    """the fused layer with its resident window at an offset, [lo, lo + n_hot) with local id = id - lo, and the
    shared expert: picks outside the window are skipped; (256, 256) leaves no routed pick at all (the shared expert
    alone: the kernels' stand-in loads for an empty step)"""
    R = 5
    log(f"decode window [{lo}, {lo + n_hot}) R={R}")
    lay = gpu_layer("c0", dev, layer=0)
    hl = host_layer(0)
    x = synth.gen_x(900 + lo, R, dev)
    xn = u16(x)
    y = torch.zeros((R, H), dtype=torch.float32, device=dev)
    saved = lay.lo, lay.n_hot
    lay.lo, lay.n_hot = lo, n_hot
    try:
        out = lay.decode(x, y=y)
        torch.cuda.synchronize()
    finally:
        lay.lo, lay.n_hot = saved
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(lay.sel[:R].cpu().numpy(), sel_ref)
    inside = ((sel_ref >= lo) & (sel_ref < lo + n_hot)).sum()
    log(f"  picks inside the window: {inside} of {sel_ref.size}")
    ref = O.moe(0, xn, sel_ref, rw_ref, hl.table(sel_ref, lo), lo, n_hot, hl.shared, threads=16)
    yh = y.cpu().numpy()
    ma, mr = parity(yh, ref)
    log(f"  max|d| {ma:.3e} mean-rel {mr:.3e}")
    assert ma <= MAX_ABS and mr <= MEAN_REL
    assert np.array_equal(u16(out), O.f32_to_bf16(yh))


def test_stack_layers_and_graph(dev):
    """two layers with residual + RMSNorm between them: norm bit-exact, routing bit-exact, each layer's output within
    tolerance (checked on the GPU's own layer inputs); the captured hipGraph replays bit-identically"""
    log("stack of 2 layers, R=4")
    _LAYERS.clear()
    torch.cuda.empty_cache()
    R = 4
    layers = [synth.make_layer(l, dev) for l in range(2)]
    ws = [synth.gen_normal(synth.key(synth.SEED, l, synth.KIND["NORM_W"]), H, dev, 1.0, 0.02) for l in range(2)]
    st = DecodeStack(layers, ws, R)
    x = synth.gen_x(4, R, dev)
    st.x.copy_(x)
    tr = []
    h_eager = st.step(trace=tr, fused=False).clone()
    torch.cuda.synchronize()
    h_prev = x.float().cpu().numpy()
    y_prev = None
    for l, (r_after, xn, y, sel, rw) in enumerate(tr):
        hl = host_layer(l)
        r_ref, xn_ref = O.residual_rmsnorm(h_prev, y_prev, ws[l].cpu().numpy(), 1e-5)
        assert np.array_equal(r_after.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
        assert np.array_equal(u16(xn), xn_ref)
        sel_ref, rw_ref = hl.route(xn_ref)
        assert np.array_equal(sel.cpu().numpy(), sel_ref) and np.array_equal(u16(rw), rw_ref)
        ma, mr = parity(y.cpu().numpy(), hl.moe(xn_ref, sel_ref, rw_ref))
        log(f"  layer {l}: max|d| {ma:.3e} mean-rel {mr:.3e}")
        assert ma <= MAX_ABS and mr <= MEAN_REL
        h_prev, y_prev = r_after.cpu().numpy(), y.cpu().numpy()
    assert np.array_equal(h_eager.cpu().numpy(), (tr[-1][0] + tr[-1][2]).cpu().numpy())
    st.capture()
    for rep in range(3):
        st.x.copy_(x)
        st.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.h, h_eager), f"replay {rep} differs from the eager step"
        junk = torch.randn(1 << 20, device=dev).sum()           # eager work between replays
        torch.cuda.synchronize()
    del st, layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("R", [1, 4, 16])
def test_norm_router_bit_identical(dev, R):
    """the fused RMSNorm + router launch against the residual + RMSNorm kernel followed by the router: xn, its f16 copy
    and the logits bit-identical (the reference's own criterion for its fused norm, nr4_kernel.cuh:4-9), xn also
    against the oracle's norm"""
    log(f"norm_router R={R}")
    lay = gpu_layer("c0", dev, layer=0)
    g = torch.Generator().manual_seed(R)
    h = (torch.randn((R, H), generator=g) * 3.0).to(dev)
    w = (1.0 + 0.02 * torch.randn(H, generator=g)).to(dev)
    xn_a = torch.empty((R, H), dtype=torch.bfloat16, device=dev)
    xh_a = torch.empty((R, H), dtype=torch.float16, device=dev)
    call("hmoe_residual_rmsnorm", ptr(h.clone()), None, ptr(w), R, 1e-5, ptr(xn_a), ptr(xh_a),
         torch.cuda.current_stream().cuda_stream)
    lg_a, ctr = router.buffers(R, dev)
    sel = torch.empty((R, 8), dtype=torch.int64, device=dev); rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
    router.router_fused(xn_a, lay.wg, lay.bias, lg_a, ctr, sel, rw, 8, 2.5)
    xn_b = torch.empty_like(xn_a); xh_b = torch.empty_like(xh_a)
    lg_b, _ = router.buffers(R, dev)
    h_before = h.clone()
    for _ in range(2):                                          # repeated calls on the same buffers
        router.norm_router(h, w, 1e-5, lay.wg, lg_b, xn_b, xh_b)
    torch.cuda.synchronize()
    assert torch.equal(h, h_before)
    assert np.array_equal(u16(xn_a), u16(xn_b)) and np.array_equal(u16(xh_a), u16(xh_b))
    E = lay.wg.shape[0]
    la = lg_a[:R * 256].view(R, 256)[:, :E].cpu().numpy().view(np.uint32)
    lb = lg_b[:R * 256].view(R, 256)[:, :E].cpu().numpy().view(np.uint32)
    assert np.array_equal(la, lb)
    _, xn_ref = O.residual_rmsnorm(h_before.cpu().numpy(), None, w.cpu().numpy(), 1e-5)
    assert np.array_equal(u16(xn_b), xn_ref)


@pytest.mark.parametrize("R", [1, 4, 16])
def test_stack_fused_matches_unfused(dev, R):
    """the decode stack with the fused norm + router launch and the layer output added into the residual gives the
    bits of the unfused stack (norm kernel, router inside the decode layer, combine), layer by layer, and its captured
    graph replays them"""
    log(f"fused stack R={R}")
    _LAYERS.clear()
    torch.cuda.empty_cache()
    layers = [synth.make_layer(l, dev) for l in range(2)]
    ws = [synth.gen_normal(synth.key(synth.SEED, l, synth.KIND["NORM_W"]), H, dev, 1.0, 0.02) for l in range(2)]
    st = DecodeStack(layers, ws, R)
    st.x.copy_(synth.gen_x(40 + R, R, dev))
    tu, tf = [], []
    h_u = st.step(trace=tu, fused=False).clone()
    h_f = st.step(trace=tf, fused=True).clone()
    torch.cuda.synchronize()
    for l in range(2):
        assert torch.equal(tu[l][0], tf[l][0]), f"layer {l}: residual"
        assert torch.equal(tu[l][1], tf[l][1]), f"layer {l}: xn"
        assert torch.equal(tu[l][3], tf[l][3]) and torch.equal(tu[l][4], tf[l][4]), f"layer {l}: routing"
    assert torch.equal(h_u, h_f)
    st.capture(fused=True)
    for rep in range(3):
        st.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.h, h_f), f"replay {rep}"
        junk = torch.randn(1 << 20, device=dev).sum()           # eager work between replays
        torch.cuda.synchronize()
    del st, layers
    torch.cuda.empty_cache()


# ---- prefill -----------------------------------------------------------------------------------------------------

def test_dispatch_bit_exact(dev):
    T, n = 2048, 256
    rng = np.random.default_rng(5)
    sel = np.stack([rng.choice(n, 8, replace=False) for _ in range(T)]).astype(np.int64)
    sel[::7, 3] = 300                                   # picks outside the window
    rw = O.f32_to_f16(rng.random((T, 8)).astype(np.float32))
    for bm, bal in ((64, False), (256, True), (16, False)):
        log(f"dispatch bm={bm} balance={bal}")
        pf = tier.PrefillBuffers(T, 8, 0, n, 256, dev, bm=bm)
        pf.run(torch.from_numpy(sel).to(dev), torch.from_numpy(rw.view(np.int16)).to(dev).view(torch.float16), bal)
        torch.cuda.synchronize()
        counts, tok, eid, wt, inv = O.dispatch(sel, rw, 0, n)
        npos = len(tok)
        meta = pf.meta.cpu().numpy()
        assert meta[0] == npos
        assert np.array_equal(pf.counts.cpu().numpy(), counts.astype(np.int32))
        assert np.array_equal(pf.tok[:npos].cpu().numpy(), tok)
        assert np.array_equal(pf.eid[:npos].cpu().numpy(), eid)
        assert np.array_equal(pf.wt[:npos].cpu().numpy().view(np.uint32), wt.view(np.uint32))
        assert np.array_equal(pf.inv.cpu().numpy(), inv)
        rbt_ref = O.pick_groups(counts, bm, bal)
        assert meta[1] == len(rbt_ref) == meta[2]
        assert np.array_equal(pf.rbt[:meta[1]].cpu().numpy(), rbt_ref)
        (_, _, rbt_py), = list(tier.pick_groups(counts, T * 8, bm, bal))
        assert np.array_equal(rbt_py, rbt_ref)


def check_all_rows(lay, hl, x, xn, y, sel_ref, rw_ref, sample=12, seed=0, with_shared=True):
    """every row of y fp32 [T, H] against the torch fp32 reference on the same selection, and that reference pinned to
    the oracle's exact mode on `sample` rows (the first and last among them); returns the bounds"""
    T = x.shape[0]
    sel = torch.from_numpy(sel_ref).to(x.device)
    rw = torch.from_numpy(rw_ref.view(np.int16)).to(x.device).view(torch.float16)
    ref = torchref.moe_rows(lay, x, sel, rw, with_shared).cpu().numpy()
    extra = np.random.default_rng(seed).choice(T, max(min(T, sample) - 2, 0), replace=False)
    rows = np.unique(np.concatenate([[0, T - 1], extra]))
    orc = O.moe(0, xn[rows], sel_ref[rows], rw_ref[rows], hl.table(sel_ref[rows], lay.lo), lay.lo, lay.n_hot,
                hl.shared if with_shared else None, threads=16)
    pa, pr = parity(ref[rows], orc)
    ma, mr = parity(y, ref)
    log(f"  torch reference vs oracle on rows {rows.tolist()}: max|d| {pa:.3e} mean-rel {pr:.3e}")
    log(f"  all {T} rows vs the torch reference: max|d| {ma:.3e} mean-rel {mr:.3e}")
    # the reference shares the f16 weight rounding of the kernels and differs from the oracle by it alone
    assert pa <= MAX_ABS / 2 and pr <= MEAN_REL / 2
    assert ma <= MAX_ABS and mr <= MEAN_REL
    # and per row: no row may hide a large error inside the chunk's mean
    row_rel = np.abs(y - ref).mean(axis=1) / np.maximum(np.abs(ref).mean(axis=1), 1e-30)
    assert row_rel.max() <= 4 * MEAN_REL, int(row_rel.argmax())
    return ma, mr


def test_prefill_parity(dev):
    T = 2048
    log("prefill T=2048")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=T)
    hl = host_layer(0, bias_sigma=0.001)
    x = synth.gen_x(2, T, dev)
    xn = u16(x)
    lay.prefill(x)
    torch.cuda.synchronize()
    pf = lay._pf
    sel = pf.sel[:T].cpu().numpy(); rw = u16(pf.rw[:T])
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(sel, sel_ref) and np.array_equal(rw, rw_ref)
    counts = np.bincount(sel_ref.ravel(), minlength=E)
    log(f"  tokens per expert: min {counts.min()} mean {counts.mean():.1f} max {counts.max()}")
    # the fp32 output before rounding (recompute into a zeroed accumulator), every row
    y = pf.y[:T]
    y.zero_()
    lay.prefill_experts(x, y)
    yh = y.cpu().numpy()
    y.zero_()
    torch.cuda.synchronize()
    check_all_rows(lay, hl, x, xn, yh, sel_ref, rw_ref)
    # the layer's prefill writes its bf16 output from the combine (hmoe_moe4p_forward_bf16): bit-identical to the
    # same sum into a zeroed fp32 partial rounded by finish_bf16, and the partial stays zeroed
    out = lay.prefill(x).clone()
    lay.prefill_experts(x, y)
    out2 = torch.empty_like(out)
    moe4.finish_bf16(y, T, out2)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    assert not bool(y.any())


def test_decode_bits_do_not_depend_on_the_grid(dev):
    """the down kernel's part sums are fixed by (part, row block), not by how the items are spread over workgroups:
    every allowed grid gives the same bits"""
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    for R in (1, 4, 16):
        x = synth.gen_x(40 + R, R, dev)
        outs = [lay.decode(x, blocks=b).clone() for b in (0, 192, 240, 384)]
        torch.cuda.synchronize()
        assert all(torch.equal(outs[0], o) for o in outs[1:]), R


@pytest.mark.parametrize("R", [1])
def test_owning_down_matches_part_sums(dev, R):
    """at one row the down launch owns 24 output rows per workgroup and adds the parts (shared expert, then each slot
    quad) in order itself; the part-sum form (phases bit 16: down partials, then the ordered output launch) gives the
    same bits, for y accumulated into a non-zero start and for the bf16 out, with and without the shared expert"""
    log(f"owning down R={R}")
    lay = gpu_layer("c0", dev, layer=0)
    x = synth.gen_x(60 + R, R, dev)
    y0 = synth.gen_normal(synth.key(synth.SEED, 0, synth.KIND["PARTIAL"], R), R * H, dev, 0.0, 0.1).view(R, H)
    for with_shared in (True, False):
        ya, yb = y0.clone(), y0.clone()
        oa = lay.decode(x, y=ya, with_shared=with_shared).clone()
        ob = lay.decode(x, y=yb, with_shared=with_shared, phases=31).clone()
        torch.cuda.synchronize()
        assert torch.equal(ya.view(torch.int32), yb.view(torch.int32)), with_shared
        assert torch.equal(oa.view(torch.int16), ob.view(torch.int16)), with_shared
        assert not torch.equal(ya, y0)


def test_prefill_empty_and_no_picks(dev):
    """the reference's early returns (moe4p.cu:229 when no pick reaches the tier, tier_split.py:377): an empty chunk
    gives an empty output without an error, and a call with no picks and no shared expert leaves out untouched"""
    log("prefill T=0 and npos=0")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    out = lay.prefill(torch.empty((0, H), dtype=torch.bfloat16, device=dev))
    assert out.shape == (0, H) and out.dtype == torch.bfloat16
    T = 5
    pf = lay._prefill_buffers(T)
    gq, uq, dq, gs, us, ds = lay.bank.tables()
    xe = torch.empty((0, H), dtype=torch.float16, device=dev)
    moe4p.forward(xe, pf.tok, pf.eid, pf.wt, pf.rbt, gq, uq, dq, gs, us, ds, *pf.scr, pf.y[:0], meta=pf.meta, npos=0,
                  nrb=0)
    y = torch.randn(T, H, device=dev)
    y0 = y.clone()
    moe4p.forward(pf.xh[:T], pf.tok, pf.eid, pf.wt, pf.rbt, gq, uq, dq, gs, us, ds, *pf.scr, y, meta=pf.meta, npos=0,
                  nrb=0)
    torch.cuda.synchronize()
    assert torch.equal(y, y0)


def test_host_tensors_are_refused(dev):
    """a host tensor among the arguments raises before any launch (its address would fault the kernel)"""
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    x = synth.gen_x(3, 2, dev)
    with pytest.raises(RuntimeError, match="device"):
        lay.decode(x, y=torch.zeros(2, H))
    with pytest.raises(RuntimeError, match="device"):
        lay.prefill(x.cpu())
    pf = lay._prefill_buffers(2)
    with pytest.raises(RuntimeError, match="device"):
        pf.run(pf.sel[:2].cpu(), pf.rw[:2])
    assert lay.decode(x).shape == (2, H)                       # and the layer still serves device inputs


def test_prefill_replays_in_a_graph(dev):
    """a prefill chunk (router, device dispatch plan, grouped GEMMs, the shared expert's dense GEMMs, combine, bf16
    out) captured once and replayed, with eager work and synchronisations between replays: every replay gives the
    eager chunk's bits"""
    log("prefill graph T=300")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    T = 300
    x = synth.gen_x(77, T, dev)
    ref = lay.prefill(x).clone()                              # eager
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = lay.prefill(x)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), i
        lay.decode(synth.gen_x(5 + i, 4, dev))
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [1, 37, 300])
def test_prefill_ragged(dev, T):
    """prefill chunks that are not a multiple of the 128-row block (the shared expert's last block partial, experts
    with one or two picks): routing bit-exact, the router's f16 copy of x exact, the fp32 output of the f16 input path
    within tolerance on every row, and the bf16 output its rounding"""
    log(f"prefill T={T}")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    hl = host_layer(0, bias_sigma=0.001)
    x = synth.gen_x(700 + T, T, dev)
    xn = u16(x)
    out = lay.prefill(x).clone()
    torch.cuda.synchronize()
    pf = lay._pf
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(pf.sel[:T].cpu().numpy(), sel_ref) and np.array_equal(u16(pf.rw[:T]), rw_ref)
    assert np.array_equal(u16(pf.xh[:T]), O.f32_to_f16(O.bf16_to_f32(xn)))
    assert int(pf.meta[0].item()) == T * 8
    y = pf.y[:T]
    y.zero_()
    lay.prefill_experts(pf.xh[:T], y)
    yh = y.cpu().numpy()
    y.zero_()
    torch.cuda.synchronize()
    assert np.array_equal(u16(out), O.f32_to_bf16(yh))
    check_all_rows(lay, hl, x, xn, yh, sel_ref, rw_ref, seed=T)


def test_prefill_blocks_of_256_picks(dev):
    """moe4p on a dispatch plan with bm = 256 (balanced, as moe4t's pick_groups): blocks of more than 128 picks run as
    two halves in one workgroup; every row within tolerance of the torch reference, and the same routing"""
    T = 2048
    log("prefill T=2048 with 256-pick blocks (moe4p)")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    hl = host_layer(0, bias_sigma=0.001)
    x = synth.gen_x(2, T, dev)
    xn = u16(x)
    pb = tier.PrefillBuffers(T, 8, 0, lay.n_hot, 256, dev, bm=256)
    router.router_fused(x, lay.wg, lay.bias, pb.logits, lay.ctr, pb.sel, pb.rw, 8, 2.5, pb.xh)
    pb.run(pb.sel, pb.rw, balance=True)
    torch.cuda.synchronize()
    rbt = pb.rbt[:int(pb.meta[1].item())].cpu().numpy()
    log(f"  {len(rbt)} row blocks, picks per block: max {rbt[:, 2].max()}, blocks over 128: {(rbt[:, 2] > 128).sum()}")
    gq, uq, dq, gs, us, ds = lay.bank.tables()
    y = torch.zeros((T, H), dtype=torch.float32, device=dev)
    moe4p.forward(pb.xh, pb.tok, pb.eid, pb.wt, pb.rbt, gq, uq, dq, gs, us, ds, *pb.scr, y, inv=pb.inv, meta=pb.meta,
                  topk=8, shared=lay.shared_rows(), npos=pb.F, nrb=pb.nrb_max)
    torch.cuda.synchronize()
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(pb.sel.cpu().numpy(), sel_ref)
    check_all_rows(lay, hl, x, xn, y.cpu().numpy(), sel_ref, rw_ref, seed=256)
    del pb


@pytest.mark.parametrize("T,ordered", [(2049, True), (4096, False), (4096, True), (8192, True)])
def test_long_prefill_moe4t(dev, T, ordered):
    """chunks above 2048 rows on moe4t (tier_split.py:543): 256-pick balanced blocks, the shared expert apart; the
    combine either in the down GEMM's epilogue (fp32 atomics, as the reference) or ordered per token through the
    inverse map (repeat calls bit-identical); routing bit-exact, every row within tolerance"""
    log(f"long prefill T={T} (moe4t, {'ordered' if ordered else 'atomic'} combine)")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    hl = host_layer(0, bias_sigma=0.001)
    x = synth.gen_x(5000 + T, T, dev)
    xn = u16(x)
    lay.deterministic = ordered
    try:
        out = lay.prefill(x).clone()
        if ordered:
            assert torch.equal(lay.prefill(x), out)
    finally:
        lay.deterministic = True
    torch.cuda.synchronize()
    pf = lay._pf
    assert pf.long and pf.bm == 256
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(pf.sel[:T].cpu().numpy(), sel_ref) and np.array_equal(u16(pf.rw[:T]), rw_ref)
    counts = np.bincount(sel_ref.ravel(), minlength=E)
    rbt = pf.rbt[:int(pf.meta[1].item())].cpu().numpy()
    assert np.array_equal(rbt, O.pick_groups(counts, 256, True))
    log(f"  picks per expert {counts.min()}..{counts.max()}, {len(rbt)} blocks of up to {rbt[:, 2].max()} picks")
    y = pf.y[:T]
    y.zero_()
    lay.deterministic = ordered
    try:
        lay.prefill_experts(pf.xh[:T], y)
    finally:
        lay.deterministic = True
    yh = y.cpu().numpy()
    y.zero_()
    torch.cuda.synchronize()
    if ordered:
        # the layer's output comes from the combine itself (hmoe_moe4t_forward_bf16, the shared expert added into the
        # partial first): bit-identical to the two-op form's fp32 sum rounded by finish_bf16, and the partial re-zeroed
        y2 = torch.from_numpy(yh).to(dev)
        o2 = torch.empty_like(out)
        moe4.finish_bf16(y2, T, o2)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), o2.view(torch.int16))
        assert not bool(pf.y[:T].any())
    # (the atomic adds make the last bits of a run order-dependent: bf16 out within one ulp of this run's rounding)
    ob = O.bf16_to_f32(u16(out))
    assert np.abs(ob - O.bf16_to_f32(O.f32_to_bf16(yh))).max() <= 2 ** -7 * max(np.abs(yh).max(), 1.0)
    check_all_rows(lay, hl, x, xn, yh, sel_ref, rw_ref, seed=T)
    lay._pf = None
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [2048, 4096])
def test_prefill_zipf_skew(dev, T):
    """prefill under the Zipf-calibrated selection bias of the decode configs (config 1's skew): the hot experts take
    hundreds of picks, so they run as many row blocks (128 picks on moe4p, 256 on moe4t) next to experts with a
    handful; routing bit-exact, the bf16 output the rounding of the fp32 sum, every row within tolerance"""
    log(f"prefill T={T} under the Zipf bias")
    bias = synth.zipf_bias()
    lay = gpu_layer("c2z", dev, layer=0, bias=bias, max_rows=2048)
    hl = HostLayer(0, bias=bias)
    x = synth.gen_x(7000 + T, T, dev)
    xn = u16(x)
    out = lay.prefill(x).clone()
    torch.cuda.synchronize()
    pf = lay._pf
    sel_ref, rw_ref = hl.route(xn)
    assert np.array_equal(pf.sel[:T].cpu().numpy(), sel_ref) and np.array_equal(u16(pf.rw[:T]), rw_ref)
    counts = np.bincount(sel_ref.ravel(), minlength=E)
    rbt = pf.rbt[:int(pf.meta[1].item())].cpu().numpy()
    log(f"  picks per expert {counts.min()}..{counts.max()}, {len(rbt)} row blocks")
    assert counts.max() > 2 * pf.bm                       # the skew puts several row blocks on one expert
    y = pf.y[:T]
    y.zero_()
    lay.prefill_experts(pf.xh[:T], y)
    yh = y.cpu().numpy()
    y.zero_()
    torch.cuda.synchronize()
    if T <= 2048:
        assert np.array_equal(u16(out), O.f32_to_bf16(yh))
    else:
        # (moe4t adds the shared expert into the partial first: the same fp32 sum, see test_long_prefill_moe4t)
        y2 = torch.from_numpy(yh).to(dev)
        o2 = torch.empty_like(out)
        moe4.finish_bf16(y2, T, o2)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), o2.view(torch.int16))
    check_all_rows(lay, hl, x, xn, yh, sel_ref, rw_ref, seed=T + 1)
    lay._pf = None
    torch.cuda.empty_cache()


def test_moe4t_gemm_entry(dev):
    """moe4t.gemm (moe4t.cu:476-488): one grouped GEMM over given pick inputs, gate/up shape (both sums) and down
    shape, against torch fp32 GEMMs on the dequantised weights of each block's expert"""
    import torch.nn.functional as F
    log("moe4t.gemm")
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    g = torch.Generator().manual_seed(3)
    counts = np.array([200, 0, 17, 256, 1, 130], np.int64)          # blocks of 200, 17, 256, 1, 65 + 65 picks
    rbt = O.pick_groups(counts, 256, True)
    npos = int(counts.sum())
    xs = torch.randn((npos, H), generator=g).half().to(dev)
    act = (torch.randn((npos, I), generator=g) * 0.1).half().to(dev)
    gq, uq, dq, gs, us, ds = lay.bank.tables()
    rb = torch.from_numpy(rbt).to(dev)
    o_gu = moe4t.gemm(xs, rb, gq, uq, torch.zeros((2, npos, I), device=dev), 0, gs, us)
    o_d = moe4t.gemm(act, rb, dq, None, torch.zeros((1, npos, H), device=dev), 1, ds)
    torch.cuda.synchronize()
    starts = np.concatenate([[0], np.cumsum(counts)])
    for e in np.nonzero(counts)[0]:
        p0, p1 = int(starts[e]), int(starts[e + 1])
        wg = moe4.dequant(lay.bank.view("gate_q", e), lay.bank.view("gate_s", e), I, H).float()
        wu = moe4.dequant(lay.bank.view("up_q", e), lay.bank.view("up_s", e), I, H).float()
        wd = moe4.dequant(lay.bank.view("down_q", e), lay.bank.view("down_s", e), H, I).float()
        for got, ref in ((o_gu[0, p0:p1], F.linear(xs[p0:p1].float(), wg)), (o_gu[1, p0:p1], F.linear(xs[p0:p1].float(), wu)),
                         (o_d[0, p0:p1], F.linear(act[p0:p1].float(), wd))):
            d = (got - ref).abs()
            assert d.max().item() <= 2e-3 * max(ref.abs().max().item(), 1.0), (e, d.max().item())


def test_combine_with_partials(dev):
    """moe4.combine with both partials (moe4.cu:700-717): f = ((f + y) + o) + o2 in fp32, bit for bit, and y zeroed;
    with one partial NULL the order is (f + y) + o"""
    log("combine with o / o2")
    g = torch.Generator().manual_seed(11)
    R = 5
    f, y, o, o2 = [(torch.randn((R, H), generator=g) * s).to(dev) for s in (1.0, 0.5, 0.3, 0.2)]
    f0 = f.clone(); y0 = y.clone()
    moe4.combine(f, o, y, R, o2)
    torch.cuda.synchronize()
    fh, yh, oh, o2h = (t.cpu().numpy() for t in (f0, y0, o, o2))
    ref = ((fh + yh) + oh) + o2h
    assert np.array_equal(f.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert not y.any()
    f = f0.clone(); y = y0.clone()
    moe4.combine(f, o, y, R)
    torch.cuda.synchronize()
    assert np.array_equal(f.cpu().numpy().view(np.uint32), ((fh + yh) + oh).view(np.uint32)) and not y.any()
    with pytest.raises(RuntimeError, match="DONE"):
        moe4.combine(f, o, y, R, o2, 1234)


def test_router_with_the_reference_logits_buffer(dev):
    """router_fused with the reference's logits scratch fp32 [8, 256] (exl3_router.py:180) for 2..8 rows"""
    hl = host_layer(0)
    wg = torch.from_numpy(hl.wg).to(dev); b = torch.from_numpy(hl.bias).to(dev)
    logits = torch.zeros((8, 256), dtype=torch.float32, device=dev)
    ctr = torch.zeros(1, dtype=torch.int32, device=dev)
    for R in (2, 8):
        x = x_rows(300 + R, R)
        xt = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
        sel = torch.empty((R, 8), dtype=torch.int64, device=dev); rw = torch.empty((R, 8), dtype=torch.float16, device=dev)
        router.router_fused(xt, wg, b, logits, ctr, sel, rw, 8, 2.5)
        torch.cuda.synchronize()
        sel_ref, rw_ref = hl.route(x)
        assert np.array_equal(sel.cpu().numpy(), sel_ref) and np.array_equal(u16(rw), rw_ref)


def test_decode_fp16_input_as_the_reference_passes_it(dev):
    """moe4.forward with fp16 x and xf=0 (the reference's call, tier_split.py:563-567) reads fp16: the result equals
    the router's f16 copy passed the same way, and the bf16 x path gives the same bits (f16(bf16 x) is exact)"""
    R = 3
    lay = gpu_layer("c2", dev, layer=0, bias_sigma=0.001, max_rows=2048)
    x = synth.gen_x(31, R, dev)
    lay.route(x)
    gq, uq, dq, gs, us, ds = lay.bank.tables()
    outs = []
    for xin in (lay.xh[:R], x):
        y = torch.zeros((R, H), dtype=torch.float32, device=dev)
        moe4.forward(xin, lay.sel[:R], lay.rw[:R], lay.n_hot, gq, uq, dq, gs, us, ds, *lay.scr, y, 0, 0, 0, xf=0)
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    with pytest.raises(RuntimeError, match="fragment"):
        moe4.forward(x, lay.sel[:R], lay.rw[:R], lay.n_hot, gq, uq, dq, gs, us, ds, *lay.scr, outs[0], 0, 0, 0, xf=1)


def test_stack_16_layers_b4(dev):
    """config 4 at its stated size: 16 layers (about 80 GB of int4 experts), B = 4, residual + RMSNorm between them.
    Eager (unfused) step: the norm bit-exact and routing bit-exact on every layer against the oracle (on the GPU's own
    layer inputs), layer outputs within tolerance on layers 0, 7 and 15; the fused step gives the same bits; its
    captured hipGraph replays them three times with eager work between. The synthetic layers' codes (uniform in
    [-8, 7], mean -0.5) and positive group scales give every weight row a negative mean, so each layer's output carries
    a common-mode term that the residual accumulates: from layer 2 on the outputs are O(100-1000), where 2e-2 is finer
    than bf16 itself, so the max-abs bound reads "<= 2e-2 or <= 1 bf16 ulp of the reference" (elementwise)"""
    log("stack of 16 layers, R=4")
    _LAYERS.clear()
    torch.cuda.empty_cache()
    R, L = 4, 16
    layers = [synth.make_layer(l, dev) for l in range(L)]
    ws = [synth.gen_normal(synth.key(synth.SEED, l, synth.KIND["NORM_W"]), H, dev, 1.0, 0.02) for l in range(L)]
    st = DecodeStack(layers, ws, R)
    x = synth.gen_x(4, R, dev)
    st.x.copy_(x)
    tr = []
    h_eager = st.step(trace=tr, fused=False).clone()
    torch.cuda.synchronize()
    h_prev = x.float().cpu().numpy()
    y_prev = None
    U = []
    for l, (r_after, xn, y, sel, rw) in enumerate(tr):
        r_ref, xn_ref = O.residual_rmsnorm(h_prev, y_prev, ws[l].cpu().numpy(), 1e-5)
        assert np.array_equal(r_after.cpu().numpy().view(np.uint32), r_ref.view(np.uint32)), l
        assert np.array_equal(u16(xn), xn_ref), l
        hl = HostLayer(l, shared=l in (0, 7, 15))
        sel_ref, rw_ref = hl.route(xn_ref)
        assert np.array_equal(sel.cpu().numpy(), sel_ref) and np.array_equal(u16(rw), rw_ref), l
        U.append(len(np.unique(sel_ref)))
        if l in (0, 7, 15):
            ref = hl.moe(xn_ref, sel_ref, rw_ref)
            ma, mr = parity(y.cpu().numpy(), ref)
            mu, _ = parity_ulp(y.cpu().numpy(), ref)
            log(f"  layer {l}: max|ref| {np.abs(ref).max():.3e} max|d| {ma:.3e} (bound units {mu:.3f}) mean-rel {mr:.3e}")
            assert mu <= 1.0 and mr <= MEAN_REL
        h_prev, y_prev = r_after.cpu().numpy(), y.cpu().numpy()
    log(f"  distinct experts per layer: {U}")
    assert np.array_equal(h_eager.cpu().numpy(), (tr[-1][0] + tr[-1][2]).cpu().numpy())
    h_f = st.step(fused=True).clone()
    torch.cuda.synchronize()
    assert torch.equal(h_f, h_eager)
    st.capture(fused=True)
    for rep in range(3):
        st.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.h, h_eager), f"replay {rep}"
        junk = torch.randn(1 << 20, device=dev).sum()           # eager work between replays
        torch.cuda.synchronize()
    del st, layers
    torch.cuda.empty_cache()


# ---- reference-format ingest: a layer from the placement file and the reference's int4 files ----------------------

def test_layer_from_reference_files(dev, tmp_path):
    """tier_split_load (tier_split.py:171-269) restated: a placement (hot 4 of a random permutation) and the
    reference's int4 files (fragment-order codes, fp32 row scales) give a GPU layer whose decode (R = 4) and prefill
    (T = 64) partials match the oracle's exact mode on the files' codes with the row scale in every group; routing
    (router rows and bias permuted to the placement order) bit-exact. The bias lifts the four hot experts into every
    row's top-8."""
    from test_placement import write_reference_files
    L, HOT = 6, 4
    perm = [int(e) for e in np.random.default_rng(17).permutation(E)]
    place = tier.load_placement({str(L): {"perm": perm, "hot": HOT, "far": 0, "first": HOT}})
    canon = write_reference_files(tmp_path, L, perm[:HOT], 41)
    bias = np.zeros(E, np.float32)
    bias[perm[:HOT]] = 2.0
    wg, b = synth.router_weights(L, dev, bias=bias)
    lay = tier.layer_from_reference((L, place[L]), str(tmp_path), wg, b, dev, max_rows=64)
    hl = HostLayer(L, bias=bias, perm=perm, n_hot=HOT, shared=False)
    table = O.ExpertTable([canon[perm[j]] for j in range(HOT)])
    for T in (4, 64):
        log(f"reference-file layer, {T} rows")
        x = synth.gen_x(900 + T, T, dev)
        xn = u16(x)
        if T <= 16:
            y = decode_fp32(lay, x, dev, with_shared=False)
            sel, rw = lay.sel[:T].cpu().numpy(), u16(lay.rw[:T])
        else:
            lay.prefill(x, with_shared=False)
            pf = lay._pf
            y = pf.y[:T]
            y.zero_()
            lay.prefill_experts(pf.xh[:T], y, with_shared=False)
            torch.cuda.synchronize()
            sel, rw = pf.sel[:T].cpu().numpy(), u16(pf.rw[:T])
            y = y.clone()
            pf.y[:T].zero_()
        sel_ref, rw_ref = hl.route(xn)
        assert np.array_equal(sel, sel_ref) and np.array_equal(rw, rw_ref)
        assert all(np.isin(np.arange(HOT), sel_ref[r]).all() for r in range(T))
        # (the oracle takes up to 16 rows a call)
        ref = np.concatenate([O.moe(0, xn[r:r + 16], sel_ref[r:r + 16], rw_ref[r:r + 16], table, 0, HOT, None,
                                    threads=16) for r in range(0, T, 16)])
        ma, mr = parity(y.cpu().numpy(), ref)
        log(f"  max|d| {ma:.3e} mean-rel {mr:.3e}")
        assert ma <= MAX_ABS and mr <= MEAN_REL
