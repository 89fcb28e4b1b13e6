"""Pins the CPU oracle (oracle/hmoe_oracle.c) with checks that do not restate its code:

  conversions      torch / numpy RNE conversions, exhaustive over f16
  generator        series functions vs numpy within ulps; normal moments / quantiles; code layout vs a pure-Python
                   restatement of the counter hash; code histogram
  router logits    fp64 matmul error bound; the fixed chain / segment order emulated exactly with Fractions
  router select    numpy lexsort top-k on (-key, index); bias = 0 reduces to top-k of the logits; forced ties
  dispatch         numpy stable argsort + bincount (tier_split.py:405-412 itself); inverse map
  pick_groups      brute-force block enumeration; hecate_amd.tier.pick_groups; invariants
  expert layer     numpy fp64 GEMVs on dequantised weights (tiny shapes); q8_0 mode: a many-pick job equals the sum
                   of its one-pick jobs bit for bit (tools/dev/test_grace_picks.py:63-80) and stays near the exact mode;
                   its quantisation, nibble order and integer dot in closed form; its fp32 lane steps against ARM's
                   published FMLA / FADDP semantics (a closed-form fold case and a fused-vs-unfused random case)
  rmsnorm          fp64 within one bf16 / f16 ulp (cbias, cscale); the reference's rms_norm_kernel tree restated with
                   numpy arrays and exact fmaf, bit for bit, and shown to differ from other orders
Nothing is unpinned: every oracle function used by the GPU parity tests has at least one of these checks.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

import pyoracle as O
from hecate_amd import synth, tier


# ---- conversions --------------------------------------------------------------------------------------------------

def test_f16_exhaustive_and_rne():
    h = np.arange(65536, dtype=np.uint16)
    f = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(f[~nan].view(np.uint32), ref[~nan].view(np.uint32)) and np.isnan(f[nan]).all()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-3, 1.0, 3e4)])
    # exact ties and the subnormal / overflow edges
    x = np.concatenate([x, (np.arange(-2048, 2048) + 0.5).astype(np.float32) * np.float32(2 ** -24),
                        np.array([65504, 65519.99, 65520, 1e6, -1e6, 2 ** -25, 2 ** -24, 6.1e-5], np.float32)])
    assert np.array_equal(O.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(300000).astype(np.float32) * s for s in (1e-30, 1e-3, 1.0, 1e30)])
    x = np.concatenate([x, (np.arange(1, 4000, dtype=np.uint32) * 0x8000 + 0x3f800000).view(np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)


# ---- generator ----------------------------------------------------------------------------------------------------

def test_exp_series_within_ulps():
    xs = np.linspace(-80, 80, 20001, dtype=np.float32)
    got = np.array([O.expf(v) for v in xs[::7]], np.float64)
    ref = np.exp(xs[::7].astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 4e-7


def test_normals_moments_and_quantiles():
    from scipy.stats import norm
    z = O.normal_f32(synth.key(1, 2, 3), 2_000_000)
    assert abs(z.mean()) < 3e-3 and abs(z.std() - 1) < 3e-3
    q = np.quantile(z, [0.001, 0.01, 0.1, 0.5, 0.9, 0.99, 0.999])
    assert np.allclose(q, norm.ppf([0.001, 0.01, 0.1, 0.5, 0.9, 0.99, 0.999]), atol=0.02)
    b = O.normal_bf16(synth.key(1, 2, 3), 1000, 0.02)
    assert np.array_equal(b, O.f32_to_bf16((0.02 * z[:1000]).astype(np.float32)))


def test_codes_layout_and_histogram():
    N, K = 32, 256
    k = synth.key(9, 1, synth.KIND["GATE_Q"], 7)
    c = O.codes(k, N, K)
    for n, kk in [(0, 0), (0, 1), (0, 15), (0, 16), (3, 77), (31, 255), (17, 128)]:
        flat = n * K + kk
        code = (synth.bits(k, flat >> 4) >> (4 * (flat & 15))) & 15
        byte = c[n, kk // 2]
        assert code == ((byte >> 4) if kk & 1 else (byte & 15))
    big = O.codes(k, 2048, 6144)
    hist = np.bincount(np.concatenate([big.ravel() & 15, big.ravel() >> 4]), minlength=16)
    assert np.all(np.abs(hist / hist.mean() - 1) < 0.01)


def test_scales_are_abs_normal_bf16():
    s = O.scales(synth.key(2, 0, 6, 1), 2048, 6144, 0.004)
    f = O.bf16_to_f32(s)
    assert (f >= 0).all() and abs(f.mean() - 0.004 * np.sqrt(2 / np.pi)) < 1e-4


# ---- router -------------------------------------------------------------------------------------------------------

def _fma32(a, b, c):
    """exact single-rounding fmaf through Fractions: the exact value rounded to fp32 once (a value that the rounding
    to fp64 puts on an fp32 midpoint is resolved against the exact value, so no double rounding)"""
    ex = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    d = float(ex)
    f = np.float32(d)
    if Fraction(float(f)) != ex and f != 0 and np.isfinite(f):
        lo, hi = sorted((f, np.nextafter(f, np.float32(np.inf) if Fraction(float(f)) < ex else np.float32(-np.inf))))
        mid = (Fraction(float(lo)) + Fraction(float(hi))) / 2
        if ex != mid:
            f = lo if ex < mid else hi
    return np.float32(f)


def test_router_logits_bound_and_exact_order():
    rng = np.random.default_rng(3)
    R, E, K = 3, 256, 6144
    x = O.f32_to_bf16(rng.standard_normal((R, K)).astype(np.float32))
    w = (rng.standard_normal((E, K)) * 0.02).astype(np.float32)
    lg = O.router_logits(x, w)
    xf = O.bf16_to_f32(x).astype(np.float64)
    ref = xf @ w.astype(np.float64).T
    bound = 1.2e-7 * 2 * K * (np.abs(xf) @ np.abs(w.astype(np.float64)).T) ** 1.0 / np.sqrt(K)
    assert np.all(np.abs(lg - ref) <= bound + 1e-6)
    # the exact fp32 order on a small case: K = 512 (8 segments of 64 = 2 chunks of 32)
    Ks = 512
    xs = O.f32_to_bf16(rng.standard_normal((1, Ks)).astype(np.float32))
    ws = (rng.standard_normal((2, Ks)) * 0.02).astype(np.float32)
    got = O.router_logits(xs, ws)
    xv = O.bf16_to_f32(xs)[0]
    for e in range(2):
        t = np.float32(0)
        for s0 in range(0, Ks, Ks // 8):
            seg = np.float32(0)
            for c in range(s0, s0 + Ks // 8, 32):
                acc = np.float32(0)
                for k in range(c, c + 32):
                    acc = _fma32(xv[k], ws[e, k], acc)
                seg = np.float32(seg + acc)
            t = np.float32(t + seg)
        assert np.float32(got[0, e]).view(np.uint32) == t.view(np.uint32)


def _select_numpy(lg, bias, topk=8, scale=2.5):
    a = np.array([[O.expf(-v) for v in row] for row in lg], np.float32)
    a = (np.float32(1) / (np.float32(1) + a)).astype(np.float32)
    key = (a + (bias if bias is not None else np.float32(0))).astype(np.float32)
    sel, rw = [], []
    for r in range(lg.shape[0]):
        order = np.lexsort((np.arange(lg.shape[1]), -key[r].astype(np.float64)))[:topk]
        s = np.float32(0)
        for e in order:
            s = np.float32(s + a[r, e])
        sel.append(order)
        rw.append([np.float32(np.float32(a[r, e] * np.float32(scale)) / np.float32(s + np.float32(1e-20))) for e in order])
    return np.array(sel, np.int64), np.array(rw, np.float32).astype(np.float16).view(np.uint16)


def test_router_select_matches_lexsort_topk():
    rng = np.random.default_rng(4)
    lg = (rng.standard_normal((40, 256)) * 1.57).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.01).astype(np.float32)
    sel, rw = O.router_select(lg, bias)
    s2, r2 = _select_numpy(lg, bias)
    assert np.array_equal(sel, s2) and np.array_equal(rw, r2)
    w = O.f16_to_f32(rw).astype(np.float64).sum(1)
    assert np.all(np.abs(w - 2.5) < 8 * 2.5 * 2 ** -11)
    assert all(len(set(r)) == 8 for r in sel)


def test_router_select_bias_zero_is_topk_of_logits_and_ties_lowest_index():
    rng = np.random.default_rng(5)
    lg = (rng.standard_normal((20, 256)) * 1.57).astype(np.float32)
    sel, _ = O.router_select(lg, None)
    ref = np.argsort(-lg.astype(np.float64), axis=1, kind="stable")[:, :8]
    assert np.array_equal(sel, ref)
    tie = np.zeros((1, 256), np.float32)
    tie[0, [200, 5, 77, 3]] = 4.0
    sel, _ = O.router_select(tie, None)
    assert list(sel[0]) == [3, 5, 77, 200, 0, 1, 2, 4]


def forced_tie_router(R, lo, hi, near):
    """a router whose experts lo and hi have identical rows and sit at the top-8 boundary: seven experts (100..106)
    far ahead by bias, lo and hi next with bias 3 (selection keys in [3, 4), where the fp32 step is 2^-22), everything
    else behind. near: hi's bias two steps up, so hi's key is one or two ulps above lo's (one step alone can round to
    the same key when act + 3 falls halfway between two)."""
    rng = np.random.default_rng(23)
    wg = (rng.standard_normal((256, 6144)) * 0.0013).astype(np.float32)
    wg[hi] = wg[lo]
    bias = np.zeros(256, np.float32)
    bias[100:107] = 5.0
    bias[lo] = 3.0
    bias[hi] = np.float32(3.0 + 2.0 ** -21) if near else 3.0
    x = O.f32_to_bf16(rng.standard_normal((R, 6144)).astype(np.float32))
    return x, wg, bias


@pytest.mark.parametrize("lo,hi", [(40, 41), (41, 40)])
def test_router_forced_tie_takes_the_lowest_index(lo, hi):
    """exl3_router.py:106-121 / nr4_kernel.cuh:307-366: keys descending, then the lowest expert index. An exact tie
    at the 8th place goes to min(lo, hi); a key one ulp higher wins whatever its index"""
    x, wg, bias = forced_tie_router(6, lo, hi, near=False)
    sel, _ = O.router(x, wg, bias)
    assert all(sorted(r[:7]) == list(range(100, 107)) and r[7] == min(lo, hi) for r in sel)
    x, wg, bias = forced_tie_router(6, lo, hi, near=True)
    sel, _ = O.router(x, wg, bias)
    assert all(r[7] == hi for r in sel)


# ---- dispatch -----------------------------------------------------------------------------------------------------

def test_dispatch_is_stable_argsort_bincount():
    rng = np.random.default_rng(6)
    T, n, lo = 500, 64, 16
    sel = np.stack([rng.choice(n + 40, 8, replace=False) for _ in range(T)]).astype(np.int64)
    rw = O.f32_to_f16(rng.random((T, 8)).astype(np.float32))
    counts, tok, eid, wt, inv = O.dispatch(sel, rw, lo, n)
    fs = sel.ravel() - lo
    keep = (fs >= 0) & (fs < n)
    order = np.argsort(np.where(keep, fs, n + 1), kind="stable")[: keep.sum()]
    assert np.array_equal(counts, np.bincount(fs[keep], minlength=n))
    assert np.array_equal(tok, order // 8) and np.array_equal(eid, fs[order])
    assert np.array_equal(wt, O.f16_to_f32(rw.ravel()[order]))
    assert np.array_equal(inv[order], np.arange(len(order))) and np.all(inv[~keep] == -1)


def _pick_groups_brute(counts, bm, balance):
    rows, pos = [], 0
    for e, c in enumerate(counts):
        if c:
            nb = -(-c // bm)
            sizes = [c // nb + (1 if k < c % nb else 0) for k in range(nb)] if balance else \
                [min(bm, c - bm * k) for k in range(nb)]
            first = pos
            for s in sizes:
                rows.append((e, first, s, 0))
                first += s
        pos += c
    return np.array(rows, np.int32).reshape(-1, 4)


@pytest.mark.parametrize("bm,balance", [(64, False), (256, True), (16, False), (7, True)])
def test_pick_groups_brute_force(bm, balance):
    rng = np.random.default_rng(bm)
    counts = rng.multinomial(3000, np.ones(100) / 100)
    counts[[3, 50]] = 0
    ref = _pick_groups_brute(counts, bm, balance)
    assert np.array_equal(O.pick_groups(counts, bm, balance), ref)
    (p0, p1, rbt), = list(tier.pick_groups(counts, counts.sum(), bm, balance))
    assert (p0, p1) == (0, counts.sum()) and np.array_equal(rbt, ref)
    assert np.all(ref[:, 2] <= bm) and np.array_equal(np.bincount(ref[:, 0], ref[:, 2], 100).astype(np.int64), counts)


def test_pick_groups_splits_at_npos():
    counts = np.array([30, 0, 50, 20, 64, 1], np.int64)
    groups = list(tier.pick_groups(counts, 100, 16))
    assert [(g[0], g[1]) for g in groups] == [(0, 100), (100, 165)]
    assert groups[1][2][0, 0] == 4 and groups[1][2][0, 1] == 0
    with pytest.raises(ValueError):
        list(tier.pick_groups(counts, 40, 16))


# ---- expert layer -------------------------------------------------------------------------------------------------

def _tiny_layer(rng, H=256, I=128, E=6):
    ex = []
    for e in range(E):
        d = {}
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            d[m + "_q"] = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
            d[m + "_s"] = O.f32_to_bf16(np.abs(rng.standard_normal((N, K // 128)) * 0.01).astype(np.float32))
        ex.append(d)
    sh = (O.f32_to_bf16((rng.standard_normal((I, H)) * 0.05).astype(np.float32)),
          O.f32_to_bf16((rng.standard_normal((I, H)) * 0.05).astype(np.float32)),
          O.f32_to_bf16((rng.standard_normal((H, I)) * 0.05).astype(np.float32)))
    return ex, sh


def _moe_numpy(x, sel, rw, ex, sh, H, I, lo=0):
    xf = O.bf16_to_f32(x).astype(np.float64)
    silu = lambda g: g / (1 + np.exp(-g))
    deq = lambda d, m, N, K: O.dequant(d[m + "_q"], d[m + "_s"], N, K).astype(np.float64)
    out = np.zeros((x.shape[0], H))
    for r in range(x.shape[0]):
        for k in range(sel.shape[1]):
            e = int(sel[r, k]) - lo
            if 0 <= e < len(ex):
                w = float(O.f16_to_f32(rw[r, k:k + 1])[0])
                d = ex[e]
                a = silu(deq(d, "gate", I, H) @ xf[r]) * (deq(d, "up", I, H) @ xf[r]) * w
                out[r] += deq(d, "down", H, I) @ a
        if sh is not None:
            g = O.bf16_to_f32(sh[0]).astype(np.float64) @ xf[r]
            u = O.bf16_to_f32(sh[1]).astype(np.float64) @ xf[r]
            out[r] += O.bf16_to_f32(sh[2]).astype(np.float64) @ (silu(g) * u)
    return out


def test_dequant_closed_form():
    rng = np.random.default_rng(7)
    q = rng.integers(0, 256, (16, 128), dtype=np.uint8)
    s = O.f32_to_bf16(rng.random((16, 2)).astype(np.float32))
    d = O.dequant(q, s, 16, 256)
    codes = np.stack([q & 15, q >> 4], -1).reshape(16, 256).astype(np.int32) - 8
    assert np.array_equal(d, (codes * np.repeat(O.bf16_to_f32(s), 128, 1)).astype(np.float32))


def test_moe_exact_matches_numpy_fp64():
    rng = np.random.default_rng(8)
    H, I = 256, 128
    ex, sh = _tiny_layer(rng, H, I)
    x = O.f32_to_bf16(rng.standard_normal((5, H)).astype(np.float32))
    sel = np.array([[1, 3, 9, 0, 5, 2, 4, 7]] * 5, np.int64) + 10
    sel[2] = [15, 11, 10, 13, 12, 14, 30, 40]
    rw = O.f32_to_f16(rng.random((5, 8)).astype(np.float32))
    tab = O.ExpertTable(ex)
    got = O.moe(0, x, sel, rw, tab, 10, len(ex), sh, H=H, I=I, threads=4)
    ref = _moe_numpy(x, sel, rw, ex, sh, H, I, lo=10)
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref))
    part = rng.standard_normal((5, H)).astype(np.float32)
    got2 = O.moe(0, x, sel, rw, tab, 10, len(ex), None, out=part.copy(), accumulate=True, H=H, I=I, threads=4)
    ref2 = _moe_numpy(x, sel, rw, ex, None, H, I, lo=10) + part
    assert np.max(np.abs(got2 - ref2)) <= 1e-6 * np.max(np.abs(ref2))


def test_picks_first_appearance_order():
    sel = np.array([[5, 2, 9, 1], [2, 7, 5, 3]], np.int64)
    rw = O.f32_to_f16(np.array([[0.5, 0.25, 1, 2], [0.125, 1, 4, 1]], np.float32))
    pick, wgt = O.picks(sel, rw, 1, 8)
    assert list(pick) == [4, 1, 0, 6, 2]
    assert np.allclose(wgt[0], [0.5, 4]) and np.allclose(wgt[1], [0.25, 0.125]) and np.allclose(wgt[3], [0, 1])


def test_q8_many_picks_equal_sum_of_one_pick_jobs():
    """tools/dev/test_grace_picks.py:63-80: a job's partial is each row's fp32 sum, from 0, of its picks' outputs in
    pick order; a one-pick job's partial is exactly that pick's output"""
    rng = np.random.default_rng(9)
    H, I = 256, 128
    ex, _ = _tiny_layer(rng, H, I, E=6)
    tab = O.ExpertTable(ex)
    for trial in range(6):
        R = int(rng.integers(1, 9))
        sel = np.stack([rng.choice(40, 8, replace=False) for _ in range(R)]).astype(np.int64)
        rw = O.f32_to_f16((rng.random((R, 8)) * 0.4 + 0.01).astype(np.float32))
        x = O.f32_to_bf16((rng.standard_normal((R, H)) * rng.choice([0.3, 1.0, 4.0])).astype(np.float32))
        got = O.moe(1, x, sel, rw, tab, 0, 6, None, H=H, I=I, threads=2)
        pick, _ = O.picks(sel, rw, 0, 6)
        ref = np.zeros((R, H), np.float32)
        for e in pick:
            s1 = np.full_like(sel, 39); r1 = np.zeros_like(rw)
            for r in range(R):
                hit = np.where(sel[r] == e)[0]
                if len(hit):
                    s1[r, 0] = e; r1[r, 0] = rw[r, hit[0]]
            ref = (ref + O.moe(1, x, s1, r1, tab, 0, 6, None, H=H, I=I, threads=2)).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        ex_ = O.moe(0, x, sel, rw, tab, 0, 6, None, H=H, I=I, threads=2)
        assert np.abs(got - ex_).mean() / np.abs(ex_).mean() < 0.03


# ---- rmsnorm ------------------------------------------------------------------------------------------------------

def _rms_tree_numpy(v):
    """the reference's rms_norm_kernel order restated with numpy arrays (a structure of its own, not the oracle's loops):
    chains [1024] over float4 columns t, t + 1024, ...; the xor butterfly of each 32-lane group as whole-array steps;
    the 32 group sums by the same steps"""
    C = v.size // 4
    cols = v.reshape(C, 4)
    chains = []
    for t in range(1024):
        p = np.float32(0)
        for c in range(t, C, 1024):
            for e in range(4):
                p = _fma32(cols[c, e], cols[c, e], p)
        chains.append(p)
    s = np.array(chains, np.float32).reshape(32, 32)
    idx = np.arange(32)
    for o in (16, 8, 4, 2, 1):
        s = (s + s[:, idx ^ o]).astype(np.float32)
    g = s[:, 0].copy()
    for o in (16, 8, 4, 2, 1):
        g = (g + g[idx ^ o]).astype(np.float32)
    assert np.all(g == g[0]) and np.all(s == s[:, :1])          # every lane holds its butterfly's sum
    return g[0]


def test_rmsnorm_fp64_and_exact_order():
    """residual + RMSNorm in the reference's order (cn.cu:21-31,80-103): fp64 within one bf16 ulp; the reduction tree
    of rms_norm_kernel restated with numpy arrays, bit for bit; r = a + r"""
    rng = np.random.default_rng(10)
    H = 6144
    r = rng.standard_normal((2, H)).astype(np.float32) * 3
    a = rng.standard_normal((2, H)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    r2, xn = O.residual_rmsnorm(r, a, w, 1e-5)
    assert np.array_equal(r2, (a + r).astype(np.float32))
    v = (r + a).astype(np.float64)
    ref = v / np.sqrt((v ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.all(np.abs(O.bf16_to_f32(xn) - ref) <= np.abs(ref) * 2 ** -8 + 1e-7)
    vf = (a + r).astype(np.float32)[0]
    tot = _rms_tree_numpy(vf)
    assert O.rms_sum(vf).view(np.uint32) == tot.view(np.uint32)
    rmf = np.float32(np.float32(1) / np.sqrt(np.float32(tot / np.float32(H)) + np.float32(1e-5), dtype=np.float32))
    exp = O.f32_to_bf16(((vf * w).astype(np.float32) * rmf).astype(np.float32))
    assert np.array_equal(xn[0], exp)


def test_rmsnorm_cn_options_and_order_sensitivity():
    """cbias / cscale / f16 out against fp64 (cn.cu:89,95-96: w + cbias only when cbias != 0, rmf scaled by cscale);
    a sequential sum and a 256-chain fold give other bits on some rows, the tree's numpy restatement the oracle's on
    every row (so the order is pinned, not only the value); a short row (H = 512: threads past H / 4 hold empty
    chains) in the same order"""
    rng = np.random.default_rng(11)
    H = 6144
    v = (rng.standard_normal((6, H)) * np.array([[1], [10], [0.01], [300], [1], [2]])).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    for cbias, cscale, bf in ((0.0, 1.0, True), (0.25, 1.0, False), (0.0, 0.5, False), (-0.5, 2.0, True)):
        xn = O.rmsnorm_cn(v, w, 1e-6, cbias, cscale, bf)
        got = O.bf16_to_f32(xn) if bf else O.f16_to_f32(xn)
        vd = v.astype(np.float64)
        ref = vd / np.sqrt((vd ** 2).mean(1, keepdims=True) + 1e-6) * (w.astype(np.float64) + cbias) * cscale
        tol = np.abs(ref) * (2 ** -8 if bf else 2 ** -11) + 1e-6
        assert np.all(np.abs(got - ref) <= tol), (cbias, cscale, bf)
    differ_seq = differ_256 = 0
    for row in v:
        tot = _rms_tree_numpy(row)
        assert O.rms_sum(row).view(np.uint32) == tot.view(np.uint32)
        seq = np.float32(0)
        for x in row:
            seq = _fma32(x, x, seq)
        part = [np.float32(0)] * 256
        for k in range(H):
            part[k % 256] = _fma32(row[k], row[k], part[k % 256])
        off = 128
        while off:
            for t in range(off):
                part[t] = np.float32(part[t] + part[t + off])
            off >>= 1
        differ_seq += seq != tot
        differ_256 += part[0] != tot
    assert differ_seq > 0 and differ_256 > 0
    short = rng.standard_normal(512).astype(np.float32)
    assert O.rms_sum(short).view(np.uint32) == _rms_tree_numpy(short).view(np.uint32)


def test_bf16_ulp_is_the_spacing_of_bf16():
    """the ulp used by the tolerance's "<= 1 bf16 ulp" reading equals the distance to the next bf16 number"""
    from hostlayer import bf16_ulp
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(2000) * np.exp2(rng.integers(-20, 20, 2000))).astype(np.float32)
    b = O.f32_to_bf16(v)
    up = (b & 0x8000) | ((b & 0x7fff) + 1)                     # next magnitude (sign kept)
    spacing = np.abs(O.bf16_to_f32(up).astype(np.float64) - O.bf16_to_f32(b).astype(np.float64))
    assert np.array_equal(bf16_ulp(O.bf16_to_f32(b)), spacing)


def test_q8_quantisation_and_integer_dot_in_closed_form():
    """cpuband.cpp:106-111 and :80-104 on values where every step is exact: each 32-block's absmax is 127 * 2^e, so
    its scale absmax / 127 is a power of two and v / s lands on chosen integers and half-integers; the weights' group
    scales are powers of two and the integer sums stay below 2^24, so the fp32 result equals the closed form
    s_w * sum over blocks of s_x * sum q * (code - 8) exactly. The half-integer cases tell round-half-to-even
    (lrintf in the default mode: 64.5 -> 64, 63.5 -> 64, -64.5 -> -64, 0.5 -> 0, 2.5 -> 2) from truncation and
    from rounding half away from zero, and the codes differ between neighbouring k, so the nibble order (even k in
    the low nibble) and the scale's divisor (127, not 128) are pinned as well"""
    rng = np.random.default_rng(41)
    N, K, nr = 5, 256, 2
    exps = rng.integers(-6, 2, size=(nr, K // 32))
    qx = rng.integers(-126, 127, size=(nr, K)).astype(np.float64)          # v / s before the ties are planted
    ties = np.array([64.5, 63.5, -64.5, 0.5, 1.5, 2.5, -2.5, -0.5])
    for r in range(nr):
        for b in range(K // 32):
            blk = qx[r, 32 * b: 32 * b + 32]
            blk[0] = 127.0 if (r + b) % 2 == 0 else -127.0                  # the absmax
            blk[1:1 + len(ties)] = ties
    x = (qx * np.exp2(np.repeat(exps, 32, axis=1))).astype(np.float32)     # exact in fp32
    codes = rng.integers(0, 16, size=(N, K)).astype(np.uint8)
    codes[:, 1::2] = (codes[:, 0::2] + 1 + rng.integers(0, 14, size=(N, K // 2))) % 16   # neighbours differ
    packed = np.ascontiguousarray(codes[:, 0::2] | (codes[:, 1::2] << 4))
    sexp = rng.integers(-9, -5, size=(N, K // 128))
    scales = O.f32_to_bf16(np.exp2(sexp).astype(np.float32))
    y, xq, xg = O.q8_gemv(packed, scales, x)
    q_exp = np.where(np.abs(qx - np.trunc(qx)) == 0.5, 2.0 * np.round(qx / 2.0), np.round(qx)).astype(np.int64)
    assert np.array_equal(q_exp[:, 1:9], np.array([[64, 64, -64, 0, 2, 2, -2, 0]] * nr))
    assert np.array_equal(xq.astype(np.int64), q_exp)
    assert np.array_equal(xg, np.exp2(exps).astype(np.float32))
    w = codes.astype(np.int64) - 8
    ref = np.zeros((nr, N))
    for r in range(nr):
        for n in range(N):
            for g in range(K // 128):
                acc = 0.0
                for b in range(4 * g, 4 * g + 4):
                    acc += float(np.exp2(exps[r, b])) * float(np.dot(q_exp[r, 32 * b: 32 * b + 32], w[n, 32 * b: 32 * b + 32]))
                ref[r, n] += float(np.exp2(sexp[n, g])) * acc
    assert np.array_equal(y.astype(np.float64), ref)
    # the case has the power to see a swapped nibble order or a /128 scale
    swapped = codes.copy(); swapped[:, 0::2], swapped[:, 1::2] = codes[:, 1::2], codes[:, 0::2]
    y_sw, _, _ = O.q8_gemv(np.ascontiguousarray(swapped[:, 0::2] | (swapped[:, 1::2] << 4)), scales, x)
    assert not np.array_equal(y_sw, y)
    assert not np.array_equal(np.round(qx * 127.0 / 128.0).astype(np.int64), q_exp)


def _q8_model(packed, scales, xq, xg, fused=True, fold="pairwise"):
    """cpuband.cpp:80-104 (with group-128 scales) from ARM's published semantics of its two float intrinsics:
    vfmaq_n_f32 is FMLA, a fused multiply-add rounded once per lane and step; vaddvq_f32 over 4 lanes is FADDP twice,
    (a0 + a1) + (a2 + a3). The int32 lane sums (vdotq_s32: lane i of a 32-block = k 4i..4i+3 and 16+4i..16+4i+3) by
    numpy int64. fused=False (multiply, round, add, round) and the other folds are the alternatives the pins must tell
    apart."""
    N, K = packed.shape[0], packed.shape[1] * 2
    nr = xq.shape[0]
    codes = np.empty((N, K), np.int64)
    codes[:, 0::2] = packed & 15
    codes[:, 1::2] = packed >> 4
    z = codes - 8
    xr = xq.astype(np.int64)
    nb = K // 32
    # lane sums d[r][n][b][i]
    zb = z.reshape(N, nb, 2, 4, 4)                 # [n][b][half][lane][j]
    xb = xr.reshape(nr, nb, 2, 4, 4)
    d = np.einsum("nbhij,rbhij->rnbi", zb, xb)
    sc = O.bf16_to_f32(scales).astype(np.float32)
    y = np.zeros((nr, N), np.float32)
    for r in range(nr):
        for n in range(N):
            yr = np.float32(0)
            for g in range(K // 128):
                a = [np.float32(0)] * 4
                for b in range(4 * g, 4 * g + 4):
                    for i in range(4):
                        dv, xv = np.float32(d[r, n, b, i]), xg[r, b]
                        a[i] = _fma32(dv, xv, a[i]) if fused else np.float32(np.float32(dv * xv) + a[i])
                if fold == "pairwise":
                    f = np.float32(np.float32(a[0] + a[1]) + np.float32(a[2] + a[3]))
                elif fold == "sequential":
                    f = np.float32(np.float32(np.float32(a[0] + a[1]) + a[2]) + a[3])
                elif fold == "02_13":
                    f = np.float32(np.float32(a[0] + a[2]) + np.float32(a[1] + a[3]))
                else:
                    f = np.float32(np.float32(a[0] + a[3]) + np.float32(a[1] + a[2]))
                yr = _fma32(sc[n, g], f, yr)
            y[r, n] = yr
    return y


def test_q8_lane_fold_and_fused_steps_pinned():
    """the q8_0 mode's fp32 steps, pinned to the published semantics of the reference's NEON intrinsics
    (cpuband.cpp:96-101): a closed-form group whose four lanes hold (2^24, 1, 1, -2^24) and (2^24, 1, -2^24, 1)
    exactly gives 1 under FADDP's (a0 + a1) + (a2 + a3) and 0 or 2 under the sequential, (a0 + a2) + (a1 + a3) and
    (a0 + a3) + (a1 + a2) folds; on random data the oracle equals the fused per-lane model bit for bit and differs from
    the multiply-then-add one"""
    # closed form: K = 128 (one group of 4 blocks), 2 weight rows, 1 row of x
    K = 128
    xq_t = np.zeros(K, np.int64)
    xe = np.zeros(4, np.int64)                   # block exponents: xg = 2^e when the absmax is 127 * 2^e
    codes = np.full((2, K), 8, np.int64)         # code 8: z = 0
    # block 0 (xg = 2^12): lane 0 of row 0 sums 8 x (-8)(-64) = 4096 -> 2^24; lane 3 of row 0 and lane 2 of row 1
    # -4096 -> -2^24; row 1's lane 0 as row 0's
    xe[0] = 12
    for k in list(range(0, 4)) + list(range(16, 20)):
        xq_t[k] = -64; codes[0, k] = 0; codes[1, k] = 0
    for k in list(range(12, 16)) + list(range(28, 32)):
        xq_t[k] = 64; codes[0, k] = 0
    for k in list(range(8, 12)) + list(range(24, 28)):
        xq_t[k] = 64; codes[1, k] = 0
    xq_t[4] = 127                                # the block's absmax, at a z = 0 position (both rows)
    # block 1 (xg = 2^-7): row 0 lanes 1, 2 and row 1 lanes 1, 3 sum (-8)(-16) = 128 -> 1
    xe[1] = -7
    for k, rows in ((32 + 4, (0, 1)), (32 + 8, (0,)), (32 + 12, (1,))):
        xq_t[k] = -16
        for n in rows:
            codes[n, k] = 0
    xq_t[32 + 17] = -127                         # the absmax
    x = (xq_t.astype(np.float64) * np.exp2(np.repeat(np.concatenate([xe[:2], [0, 0]]), 32))).astype(np.float32)
    x[64:] = 0.0                                 # blocks 2, 3 empty (scale 1, all codes contribute 0)
    x = x[None, :]
    packed = np.ascontiguousarray((codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8))
    scales = O.f32_to_bf16(np.ones((2, 1), np.float32))
    y, xq, xg = O.q8_gemv(packed, scales, x)
    assert np.array_equal(xq[0].astype(np.int64), xq_t) and np.array_equal(xg[0], np.array([4096, 2 ** -7, 1, 1],
                                                                                       np.float32))
    assert np.array_equal(y, np.array([[1.0, 1.0]], np.float32))
    for fold, exp in (("sequential", [0.0, 1.0]), ("02_13", [1.0, 2.0]), ("03_12", [2.0, 1.0])):
        assert np.array_equal(_q8_model(packed, scales, xq, xg, fold=fold), np.array([exp], np.float32)), fold
    # random data: the fused per-lane steps bit for bit, and the case has the power to see an unfused one
    rng = np.random.default_rng(77)
    N, K, nr = 12, 512, 3
    x = (rng.standard_normal((nr, K)) * np.exp2(rng.integers(-3, 3, (nr, K)))).astype(np.float32)
    packed = rng.integers(0, 256, (N, K // 2)).astype(np.uint8)
    scales = O.f32_to_bf16(np.abs(rng.standard_normal((N, K // 128)) * 0.01).astype(np.float32))
    y, xq, xg = O.q8_gemv(packed, scales, x)
    assert np.array_equal(y.view(np.uint32), _q8_model(packed, scales, xq, xg).view(np.uint32))
    assert not np.array_equal(y, _q8_model(packed, scales, xq, xg, fused=False))
