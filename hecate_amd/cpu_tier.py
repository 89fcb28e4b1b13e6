"""The host-CPU expert tier: runtime/tier/cpuband.cpp (the Grace band) on x86, driven like tier_split.py:65-82
(start the pool), :228-243 (add a layer's cold experts in row-major int4) and :520-644 (submit a decode job after
routing, add the CPU partial in tier_combine).

CpuTier(threads) starts the pool on a mailbox. With mapped=True (the default) the mailbox is pinned, device-mapped
host memory and the GPU drives the hand-off itself, one kernel each (so a hipGraph can hold them): submit() copies
x / sel / rw into the mailbox and posts the next generation, collect() waits (bounded) for the pool to finish it and
adds the partial into y; check() reports a job's error once the stream has passed the collect. post() / wait() drive
the same mailbox from the host (mapped=False needs no GPU), as tools/dev/test_grace_picks.py drives cpuband's ISSUE /
CPU_DONE generations.
"""
import ctypes
import time

import numpy as np
import torch

from ._lib import call, on_device, ptr, stream_of

H, I, TOPK, MAXR = 6144, 2048, 8, 8


class Mailbox(ctypes.Structure):
    """hmoe_cpu_mailbox (include/hecate_moe.h)"""
    _fields_ = [("issue", ctypes.c_uint32), ("pad0", ctypes.c_uint32 * 31),
                ("done", ctypes.c_uint32), ("pad1", ctypes.c_uint32 * 31),
                ("rows", ctypes.c_int32), ("layer", ctypes.c_int32), ("err", ctypes.c_int32),
                ("gpu_err", ctypes.c_int32), ("pad2", ctypes.c_int32 * 28),
                ("sel", ctypes.c_int64 * (MAXR * TOPK)), ("rw", ctypes.c_uint16 * (MAXR * TOPK)),
                ("x", ctypes.c_uint16 * (MAXR * H)), ("out", ctypes.c_float * (MAXR * H))]


class CpuTier:
    def __init__(self, threads=8, first_core=-1, mapped=True):
        self.mapped = mapped
        if mapped:
            p = ctypes.c_void_p()
            call("hmoe_cpu_mailbox_alloc", ctypes.byref(p))
            self.addr = p.value
            self._host = None
        else:
            self._host = Mailbox()
            self.addr = ctypes.addressof(self._host)
        self.mb = Mailbox.from_address(self.addr)
        self._keep = []
        call("hmoe_cpu_start", self.addr, int(threads), int(first_core))
        self.running = True

    def add_layer(self, layer, lo, experts):
        """cold experts of a layer, ids lo .. lo + len(experts) - 1: each a dict of canonical row-major host arrays
        gate_q [I, H/2] u8, gate_s [I, H/128] bf16 bits (u16), up_q / up_s alike, down_q [H, I/2], down_s [H, I/128]"""
        n = len(experts)
        q = (ctypes.c_void_p * (3 * n))()
        s = (ctypes.c_void_p * (3 * n))()
        for e, ex in enumerate(experts):
            for k, m in enumerate(("gate", "up", "down")):
                qa = np.ascontiguousarray(ex[m + "_q"], np.uint8)
                sa = np.ascontiguousarray(ex[m + "_s"], np.uint16)
                N, K = (I, H) if m != "down" else (H, I)
                if qa.size != N * K // 2 or sa.size != N * K // 128:
                    raise RuntimeError(f"cpu tier: expert {e} {m} has the wrong size")
                self._keep += [qa, sa]
                q[3 * e + k], s[3 * e + k] = qa.ctypes.data, sa.ctypes.data
        call("hmoe_cpu_add_layer", int(layer), int(lo), n, q, s)

    # ---- host-driven jobs ----
    def post(self, x_bf16, sel, rw_f16, layer):
        """x bf16 bits u16 [R, H], sel int64 [R, 8], rw f16 bits u16 [R, 8]: fill the mailbox, then post the next
        generation (issue + 1); returns it"""
        x_bf16 = np.ascontiguousarray(x_bf16, np.uint16)
        R = x_bf16.shape[0]
        if not 1 <= R <= MAXR or x_bf16.shape[1] != H:
            raise RuntimeError(f"cpu tier: {R} rows")
        if self.mb.done != self.mb.issue:
            raise RuntimeError("cpu tier: a job is in flight")
        ctypes.memmove(self.mb.x, x_bf16.ctypes.data, x_bf16.nbytes)
        ctypes.memmove(self.mb.sel, np.ascontiguousarray(sel, np.int64).ctypes.data, R * TOPK * 8)
        ctypes.memmove(self.mb.rw, np.ascontiguousarray(rw_f16, np.uint16).ctypes.data, R * TOPK * 2)
        self.mb.rows, self.mb.layer, self.mb.err = R, int(layer), 0
        return self.raise_issue(R)

    def raise_issue(self, rows):
        """post the next generation over whatever job the mailbox holds (x86 stores are seen in order: the job before
        the generation); returns it"""
        g = (int(self.mb.issue) + 1) & 0xFFFFFFFF or 1            # (0 is skipped on wrap-around)
        self.mb.issue = g
        self._rows, self._gen = rows, g
        return g

    def wait(self, timeout=60.0, gen=None):
        """wait until the pool has finished generation gen (default: the last one posted here); the partial fp32
        [R, H] (a copy) and the job's err. Any other value of done (an older job, a stale number) does not end it"""
        t0 = time.perf_counter()
        want = self._gen if gen is None else gen
        while self.mb.done != want:
            if time.perf_counter() - t0 > timeout:
                raise RuntimeError("cpu tier: the job did not finish")
        out = np.ctypeslib.as_array(self.mb.out)[:self._rows * H].reshape(self._rows, H).copy()
        return out, int(self.mb.err)

    # ---- GPU hand-off ----
    def handoff(self, layer):
        """the hand-off words of router.norm_route for a job of `layer` on this pool: (mailbox, layer)"""
        if not self.mapped:
            raise RuntimeError("cpu tier: the hand-off needs the mapped mailbox")
        return (self.addr, int(layer))

    def submit(self, x, sel, rw, layer, stream=None):
        """queue on the stream: x bf16 [R, H], sel int64 [R, 8], rw f16 [R, 8] (device) into the mailbox, flag up"""
        if not self.mapped:
            raise RuntimeError("cpu tier: submit needs the mapped mailbox")
        R = x.shape[0]
        on_device("cpu tier submit", x, sel, rw)
        if not (x.dtype == torch.bfloat16 and x.shape == (R, H) and sel.dtype == torch.int64 and sel.shape == (R, 8)
                and rw.dtype == torch.float16 and rw.shape == (R, 8)
                and x.is_contiguous() and sel.is_contiguous() and rw.is_contiguous()):
            raise RuntimeError("cpu tier submit: x bf16 [R, H], sel int64 [R, 8], rw f16 [R, 8], contiguous")
        call("hmoe_cpu_submit", self.addr, ptr(x), ptr(sel), ptr(rw), int(R), int(layer),
             stream if stream is not None else stream_of(x.device))
        self._rows = R

    def collect(self, y, stream=None):
        """queue on the stream: wait for the pool, then y fp32 [R, H] += the CPU partial"""
        R = y.shape[0]
        on_device("cpu tier collect", y)
        if not (y.dtype == torch.float32 and y.dim() == 2 and y.shape[1] == H and y.is_contiguous()):
            raise RuntimeError("cpu tier collect: y fp32 [R, H], contiguous")
        call("hmoe_cpu_collect", self.addr, ptr(y), int(R), stream if stream is not None else stream_of(y.device))

    def check(self):
        """after the stream has reached the collect: raise on the last job's error or a GPU-side one (clearing it)"""
        g, e = int(self.mb.gpu_err), int(self.mb.err)
        if g:
            self.mb.gpu_err = 0
            raise RuntimeError("cpu tier: " + {1: "the collect's wait for the pool ran out (partial not added)",
                                               2: "the hand-off found the pool busy (job not posted)"}.get(g, str(g)))
        if e:
            raise RuntimeError("cpu tier: " + {1: "bad row count", 2: "the pool holds no such layer"}.get(e, str(e)))

    def stats(self):
        j, p = ctypes.c_longlong(), ctypes.c_longlong()
        call("hmoe_cpu_stats", ctypes.byref(j), ctypes.byref(p))
        return j.value, p.value

    def close(self):
        if self.running:
            call("hmoe_cpu_stop")
            self.running = False
            if self.mapped:
                call("hmoe_cpu_mailbox_free", self.addr)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def host_experts(layer, experts, device, seed=None):
    """canonical row-major host copies (CpuTier.add_layer's format) of the synthetic experts with the given original
    ids: generated on the device by the seeded generator, unpacked on the host"""
    import torch
    from . import synth
    seed = synth.SEED if seed is None else seed
    st = stream_of(device)
    out = []
    for e in experts:
        ex = {}
        for m, kq, ks, N, K in (("gate", "GATE_Q", "GATE_S", I, H), ("up", "UP_Q", "UP_S", I, H),
                                ("down", "DOWN_Q", "DOWN_S", H, I)):
            q = torch.empty(N * K // 2, dtype=torch.uint8, device=device)
            s = torch.empty(N * (K // 128), dtype=torch.int16, device=device)
            call("hmoe_gen_i4", synth.key(seed, layer, synth.KIND[kq], e), synth.key(seed, layer, synth.KIND[ks], e),
                 synth.SIG_SCALE, N, K, ptr(q), ptr(s), st)
            qh = q.cpu().numpy()
            sh = s.cpu().numpy().view(np.uint16)
            codes = np.empty((N, K // 2), np.uint8)
            scales = np.empty((N, K // 128), np.uint16)
            call("hmoe_unpack_i4", qh.ctypes.data, sh.ctypes.data, N, K, codes.ctypes.data, scales.ctypes.data)
            ex[m + "_q"], ex[m + "_s"] = codes, scales
        out.append(ex)
    return out


def decode_split(lay, cpu, layer, x, y, with_shared=False):
    """one decode step of a partly resident layer split as tier_split.py:520-644 splits it: route x bf16 [R, H] on
    the GPU, hand the rows and picks to the CPU tier, run the resident experts into y fp32 [R, H] meanwhile, then
    (on the same stream) wait for the pool and add its partial; the pool's window holds the absent experts"""
    R = x.shape[0]
    sel, rw = lay.route(x)
    cpu.submit(x, sel, rw, layer)
    lay.experts_decode(R, y, with_shared)
    cpu.collect(y)
    return sel, rw


def decode_split_norm(lay, cpu, layer, h, r, w_post, x2, w_next, xn, nr, eps, cand=None, ctr=None):
    """one decode step of a partly resident layer in the reference's fused tier form (tier_split.py:520-644 with
    EXL3_NORM_ROUTE_HANDOFF and the combine into the next norm): norm_route adds h (fp32 [R, H], the attention output)
    into the residual r, normalises it into x2 (bf16) with w_post, routes it into the layer's sel / rw and posts the CPU
    tier's job in its selection launch; the resident experts run into the layer's accumulator nr (fp32 [R, H], zero on
    entry); combine_norm_cpu then waits for the pool and adds nr + the CPU partial into r (nr zeroed), and normalises
    it into xn with w_next (the next layer's input norm). Five launches in all, none of them for the hand-off."""
    from . import cn, router
    R = h.shape[0]
    if cand is None:
        cand, ctr = router.norm_route_buffers(R, h.device)
    sel, rw = lay.sel[:R], lay.rw[:R]
    router.norm_route(h, r, w_post, x2, lay.wg, lay.bias, sel, rw, cand, ctr, lay.scale, eps, ho=cpu.handoff(layer))
    lay.experts_decode(R, nr, False, xh=x2)
    cn.combine_norm_cpu(None, None, nr, R, cpu, r, w_next, xn, eps)
    return sel, rw
