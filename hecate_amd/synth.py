"""Seeded synthetic MoE layers of the benchmark configurations, generated on the device with the counter-based
generator of include/hmoe_rng.h (the same values any host can regenerate), plus the key derivation in Python.

Shapes: H 6144, I 2048, 256 experts, top-8, routed scale 2.5. Router W_g fp32 ~N(0, 0.02); selection bias fp32
~N(0, 0.01) (decode), ~N(0, 0.001) (prefill) or Zipf(1.1)-shaped (the 16-row decode step); experts int4 symmetric
(codes uniform in [-8, 7]) with bf16 group-128 scales |N(0, 0.004)|; shared expert bf16 ~N(0, 0.02) (held as F16T);
x bf16 ~N(0, 1).
"""
import math

import numpy as np
import torch

from ._lib import call, ptr, stream_of
from .tier import ExpertBank, MoELayer, H, I

SEED = 0x4ECA7E
E = 256
SIG_ROUTER, SIG_SCALE, SIG_SHARED = 0.02, 0.004, 0.02
KIND = dict(X=0, ROUTER=1, BIAS=2, GATE_Q=3, UP_Q=4, DOWN_Q=5, GATE_S=6, UP_S=7, DOWN_S=8, SH_GATE=9, SH_UP=10,
            SH_DOWN=11, PARTIAL=12, NORM_W=13, PERM=14)
# Zipf(1.1) popularity: bias_e = tau * (log p_rank(e) - mean), tau such that the pick frequency of ranks 4..128 has
# log-log slope -1.1 under the router's logit distribution (calibrate_zipf_tau reproduces it)
ZIPF_S = 1.1
ZIPF_TAU = 0.0585
M64 = (1 << 64) - 1


def mix64(z):
    z = ((z ^ (z >> 30)) * 0xbf58476d1ce4e5b9) & M64
    z = ((z ^ (z >> 27)) * 0x94d049bb133111eb) & M64
    return z ^ (z >> 31)


def key(seed, layer, kind, expert=0):
    """include/hmoe_rng.h hmoe_key"""
    k = mix64((seed ^ 0x6a09e667f3bcc909) & M64)
    k = mix64(k ^ ((layer * 0x9e3779b97f4a7c15) & M64))
    k = mix64(k ^ ((kind * 0xc2b2ae3d27d4eb4f) & M64))
    return mix64(k ^ ((expert * 0x165667b19e3779f9) & M64))


def bits(k, idx):
    return mix64((k + (idx + 1) * 0x9e3779b97f4a7c15) & M64)


def gen_normal(k, n, device, mean=0.0, sigma=1.0, dtype=torch.float32):
    out = torch.empty(n, dtype=dtype, device=device)
    call("hmoe_gen_normal", k, n, float(mean), float(sigma), 0 if dtype == torch.float32 else 1, ptr(out),
         stream_of(out.device))
    return out


def gen_x(tag, R, device, seed=SEED, layer=0):
    """MoE input rows bf16 [R, H] ~N(0, 1)"""
    return gen_normal(key(seed, layer, KIND["X"], tag), R * H, device, dtype=torch.bfloat16).view(R, H)


def popularity_order(seed=SEED, layer=0):
    """seeded permutation: expert ids from most to least popular"""
    k = key(seed, layer, KIND["PERM"], 1)
    return sorted(range(E), key=lambda e: (bits(k, e), e))


def zipf_bias(tau=ZIPF_TAU, seed=SEED, layer=0, s=ZIPF_S):
    order = popularity_order(seed, layer)
    z = np.arange(1, E + 1, dtype=np.float64) ** -s
    z /= z.sum()
    lz = np.log(z)
    b = np.empty(E, np.float32)
    b[np.array(order)] = (tau * (lz - lz.mean())).astype(np.float32)
    return b


def calibrate_zipf_tau(s=ZIPF_S, rows=20000, seed=0):
    """the tau of ZIPF_TAU: bisection on the log-log slope of rank frequency (ranks 4..128) of top-8 picks, logits
    iid N(0, (0.02 sqrt(H))^2) (the router's logit law for x ~ N(0, 1))"""
    rng = np.random.default_rng(seed)
    L = rng.standard_normal((rows, E)) * SIG_ROUTER * math.sqrt(H)
    A = 1.0 / (1.0 + np.exp(-L))
    z = np.arange(1, E + 1, dtype=np.float64) ** -s
    z /= z.sum()
    lz = np.log(z) - np.log(z).mean()
    r = np.arange(1, E + 1)

    def slope(tau):
        top = np.argpartition(-(A + tau * lz), 8, axis=1)[:, :8]
        f = np.bincount(top.ravel(), minlength=E) / top.size
        m = (r >= 4) & (r <= 128) & (f > 0)
        return np.polyfit(np.log(r[m]), np.log(f[m]), 1)[0]

    lo, hi = 0.03, 0.1
    for _ in range(30):
        mid = 0.5 * (lo + hi)
        if slope(mid) > -s:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def gen_bank(layer, experts, device, seed=SEED):
    """ExpertBank holding the listed original expert ids (local id = list index)"""
    bank = ExpertBank(len(experts), device)
    st = stream_of(bank.device)
    for i, e in enumerate(experts):
        for q, s, kq, ks, N, K in (("gate_q", "gate_s", "GATE_Q", "GATE_S", I, H), ("up_q", "up_s", "UP_Q", "UP_S", I, H),
                                   ("down_q", "down_s", "DOWN_Q", "DOWN_S", H, I)):
            call("hmoe_gen_i4", key(seed, layer, KIND[kq], e), key(seed, layer, KIND[ks], e), SIG_SCALE, N, K,
                 bank.addr(q, i), bank.addr(s, i), st)
    return bank


def gen_shared(layer, device, seed=SEED):
    out = []
    for kind, N, K in (("SH_GATE", I, H), ("SH_UP", I, H), ("SH_DOWN", H, I)):
        t = torch.empty(N * K, dtype=torch.float16, device=device)
        call("hmoe_gen_dense", key(seed, layer, KIND[kind]), SIG_SHARED, N, K, ptr(t), stream_of(t.device))
        out.append(t)
    return tuple(out)


def router_weights(layer, device, seed=SEED, bias_sigma=0.01, bias=None):
    wg = gen_normal(key(seed, layer, KIND["ROUTER"]), E * H, device, 0.0, SIG_ROUTER).view(E, H)
    if bias is None:
        b = gen_normal(key(seed, layer, KIND["BIAS"]), E, device, 0.0, bias_sigma)
    else:
        b = torch.as_tensor(np.asarray(bias, np.float32)).to(device)
    return wg, b


def make_layer(layer, device, seed=SEED, bias_sigma=0.01, bias=None, resident=None, shared=True, max_rows=16):
    """the synthetic layer; resident: original expert ids held on the GPU (default all 256, identity order). With a
    subset the expert ids are permuted so the resident ones are [0, n) (router rows and bias permuted alike, as
    rtx_split.py:3-5,116 / tier_split.py:18), and picks of the others contribute nothing."""
    wg, b = router_weights(layer, device, seed, bias_sigma, bias)
    if resident is None:
        perm = list(range(E))
        n = E
    else:
        res = list(resident)
        perm = res + [e for e in range(E) if e not in set(res)]
        n = len(res)
        idx = torch.tensor(perm, dtype=torch.int64, device=wg.device)
        wg = wg.index_select(0, idx).contiguous()
        b = b.index_select(0, idx).contiguous()
    bank = gen_bank(layer, perm[:n], device, seed)
    sh = gen_shared(layer, device, seed) if shared else None
    lay = MoELayer(wg, b, bank, sh, lo=0, n_hot=n, max_rows=max_rows)
    lay.perm = perm
    return lay
