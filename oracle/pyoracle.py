"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product package. Arrays are numpy; bf16 and f16 values travel as uint16 bit patterns.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        i32, i64, u32, u64, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
        sig = {
            "orc_key": (u64, [u64, u32, u32, u32]),
            "orc_gen_normal_f32": (None, [u64, i64, f32, f32, P]),
            "orc_gen_normal_bf16": (None, [u64, i64, f32, P]),
            "orc_gen_codes": (None, [u64, i32, i32, P]),
            "orc_gen_scales": (None, [u64, i32, i32, f32, P]),
            "orc_f32_to_bf16": (None, [P, i64, P]),
            "orc_f32_to_f16": (None, [P, i64, P]),
            "orc_f16_to_f32": (None, [P, i64, P]),
            "orc_expf": (f32, [f32]),
            "orc_router_logits": (None, [P, P, i32, i32, i32, P]),
            "orc_router_logits_f32": (None, [P, P, i32, i32, i32, P]),
            "orc_router_select": (None, [P, P, i32, i32, i32, f32, P, P]),
            "orc_dispatch": (i32, [P, P, i32, i32, i32, i32, P, P, P, P, P]),
            "orc_pick_groups": (i32, [P, i32, i32, i32, P, i32]),
            "orc_picks": (i32, [P, P, i32, i32, i32, i32, P, P]),
            "orc_moe": (i32, [i32, i32, i32, i32, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, i32, P, i32]),
            "orc_q8_gemv": (i32, [P, P, i32, i32, P, i32, P, P, P]),
            "orc_dequant": (None, [P, P, i32, i32, P]),
            "orc_residual_rmsnorm": (None, [P, P, P, i32, i32, f32, P]),
            "orc_rms_sum": (f32, [P, i32]),
            "orc_rmsnorm_cn": (None, [P, P, i32, i32, f32, f32, f32, i32, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- synthetic data ----------------------------------------------------------------------------------------------

def key(seed, layer, kind, expert=0):
    return int(lib().orc_key(seed, layer, kind, expert))


def normal_f32(k, n, mean=0.0, sigma=1.0):
    out = np.empty(n, np.float32)
    lib().orc_gen_normal_f32(k, n, mean, sigma, _p(out))
    return out


def normal_bf16(k, n, sigma=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_gen_normal_bf16(k, n, sigma, _p(out))
    return out


def codes(k, N, K):
    out = np.empty((N, K // 2), np.uint8)
    lib().orc_gen_codes(k, N, K, _p(out))
    return out


def scales(k, N, K, sigma):
    out = np.empty((N, K // 128), np.uint16)
    lib().orc_gen_scales(k, N, K, sigma, _p(out))
    return out


# ---- conversions -------------------------------------------------------------------------------------------------

def bf16_to_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_bf16(_p(f), f.size, _p(out))
    return out


def f32_to_f16(f):
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_f32_to_f16(_p(f), f.size, _p(out))
    return out


def f16_to_f32(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32(_p(h), h.size, _p(out))
    return out


def expf(x):
    return float(lib().orc_expf(float(x)))


# ---- router / dispatch -------------------------------------------------------------------------------------------

def router_logits(x_bf16, w):
    x_bf16 = _c(x_bf16, np.uint16); w = _c(w, np.float32)
    R, K = x_bf16.shape; E = w.shape[0]
    out = np.empty((R, E), np.float32)
    lib().orc_router_logits(_p(x_bf16), _p(w), R, K, E, _p(out))
    return out


def router_logits_f32(x, w):
    """router logits of fp32 rows (exact widenings of bf16 or f16) in the router's fixed order"""
    x = _c(x, np.float32); w = _c(w, np.float32)
    R, K = x.shape
    E = w.shape[0]
    out = np.empty((R, E), np.float32)
    lib().orc_router_logits_f32(_p(x), _p(w), R, K, E, _p(out))
    return out


def router_select(logits, bias, topk=8, scale=2.5):
    logits = _c(logits, np.float32)
    R, E = logits.shape
    b = None if bias is None else _c(bias, np.float32)
    sel = np.empty((R, topk), np.int64); rw = np.empty((R, topk), np.uint16)
    lib().orc_router_select(_p(logits), _p(b), R, E, topk, scale, _p(sel), _p(rw))
    return sel, rw


def router(x_bf16, w, bias, topk=8, scale=2.5):
    return router_select(router_logits(x_bf16, w), bias, topk, scale)


def dispatch(sel, rw, lo, n):
    sel = _c(sel, np.int64); rw = _c(rw, np.uint16)
    T, topk = sel.shape
    F = T * topk
    counts = np.empty(n, np.int64); tok = np.empty(F, np.int32); eid = np.empty(F, np.int32)
    wt = np.empty(F, np.float32); inv = np.empty(F, np.int32)
    npos = lib().orc_dispatch(_p(sel), _p(rw), T, topk, lo, n, _p(counts), _p(tok), _p(eid), _p(wt), _p(inv))
    return counts, tok[:npos], eid[:npos], wt[:npos], inv


def pick_groups(counts, bm, balance):
    counts = _c(counts, np.int64)
    cap = int(np.sum((counts + bm - 1) // bm)) + 1
    rbt = np.empty((cap, 4), np.int32)
    nrb = lib().orc_pick_groups(_p(counts), counts.size, bm, int(bool(balance)), _p(rbt), cap)
    return rbt[:nrb]


def picks(sel, rw, lo, n_hot):
    sel = _c(sel, np.int64); rw = _c(rw, np.uint16)
    R, topk = sel.shape
    pick = np.empty(R * topk, np.int32); wgt = np.empty((R * topk, R), np.float32)
    P = lib().orc_picks(_p(sel), _p(rw), R, topk, lo, n_hot, _p(pick), _p(wgt))
    return pick[:P], wgt[:P]


# ---- expert layer ------------------------------------------------------------------------------------------------

class ExpertTable:
    """host addresses of each local expert's canonical int4 codes and bf16 g128 scales (kept alive here)"""

    def __init__(self, experts):
        # experts: list of dicts {gate_q, gate_s, up_q, up_s, down_q, down_s} (numpy), local id = list index
        self.keep = experts
        n = len(experts)
        self.tabs = {}
        for name in ("gate_q", "gate_s", "up_q", "up_s", "down_q", "down_s"):
            t = np.zeros(max(n, 1), np.uint64)
            for i, ex in enumerate(experts):
                if ex is not None:
                    t[i] = ex[name].ctypes.data
            self.tabs[name] = t


def q8_gemv(q, s, x):
    """orc_q8_gemv: x fp32 [nr][K] quantised per 32 (q8_0), times packed codes q [N][K/2] with bf16 group scales
    s [N][K/128]; returns (y [nr][N], xq int8 [nr][K], xg [nr][K/32])"""
    q = _c(q, np.uint8); s = _c(s, np.uint16); x = _c(x, np.float32)
    N = q.shape[0]; nr, K = x.shape
    xq = np.empty((nr, K), np.int8); xg = np.empty((nr, K // 32), np.float32); y = np.empty((nr, N), np.float32)
    assert lib().orc_q8_gemv(_p(q), _p(s), N, K, _p(x), nr, _p(xq), _p(xg), _p(y)) == 0
    return y, xq, xg


def moe(mode, x_bf16, sel, rw, table, lo, n_hot, shared=None, out=None, accumulate=False, threads=8, H=6144, I=2048):
    """mode 0 = exact (fp32 activations, fp64 accumulation), 1 = q8_0 (cpuband-faithful)"""
    x_bf16 = _c(x_bf16, np.uint16); sel = _c(sel, np.int64); rw = _c(rw, np.uint16)
    R, topk = sel.shape
    if out is None:
        out = np.zeros((R, H), np.float32)
    t = table.tabs
    sg = su = sd = None
    if shared is not None:
        sg, su, sd = (_c(shared[0], np.uint16), _c(shared[1], np.uint16), _c(shared[2], np.uint16))
    rc = lib().orc_moe(mode, R, H, I, _p(x_bf16), _p(sel), _p(rw), topk, lo, n_hot,
                       _p(t["gate_q"]), _p(t["gate_s"]), _p(t["up_q"]), _p(t["up_s"]), _p(t["down_q"]), _p(t["down_s"]),
                       _p(sg), _p(su), _p(sd), int(bool(accumulate)), _p(out), threads)
    if rc != 0:
        raise RuntimeError(f"orc_moe failed ({rc})")
    return out


def dequant(q, s, N, K):
    q = _c(q, np.uint8); s = _c(s, np.uint16)
    out = np.empty((N, K), np.float32)
    lib().orc_dequant(_p(q), _p(s), N, K, _p(out))
    return out


def residual_rmsnorm(r, a, w, eps):
    r = _c(r, np.float32).copy(); w = _c(w, np.float32)
    R, H = r.shape
    aa = None if a is None else _c(a, np.float32)
    xn = np.empty((R, H), np.uint16)
    lib().orc_residual_rmsnorm(_p(r), _p(aa), _p(w), R, H, eps, _p(xn))
    return r, xn


def rms_sum(v):
    """the fp32 sum of squares of one row in the reference's rms_norm_kernel order"""
    v = _c(v, np.float32)
    return np.float32(lib().orc_rms_sum(_p(v), v.size))


def rmsnorm_cn(v, w, eps, cbias=0.0, cscale=1.0, bf16=True):
    """xn of residual rows v [R, H] (after the add) in the reference's rms_norm_kernel order: uint16 bf16 or f16 bits"""
    v = _c(v, np.float32); w = _c(w, np.float32)
    R, H = v.shape
    xn = np.empty((R, H), np.uint16)
    lib().orc_rmsnorm_cn(_p(v), _p(w), R, H, eps, cbias, cscale, int(bool(bf16)), _p(xn))
    return xn
