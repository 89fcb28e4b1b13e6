"""The GPU tier's MoE layer on one MI355X: what runtime/tier/tier_split.py does around the moe4 / moe4p ops
(tier_split_load:171-269 resident expert tables, tier_submit:520-574 decode vs prefill, tier_combine:577-644) and the
row-block planner of runtime/tier/rtx_split.py:236-255 (pick_groups), restated for this build's formats.

Decode (<= 16 rows): router_fused (writes the f16 copy of x) -> moe4.forward (routed + shared expert into the
fp32 accumulator) -> bf16 output (accumulator zeroed). Prefill: router -> device dispatch plan (no host sync) ->
moe4p.forward (routed + shared) -> bf16 output. Every launch is static-shaped and allocation-free, so a whole step can
be captured in a hipGraph.
"""
import numpy as np
import torch

from . import moe4, moe4p, moe4t, router
from ._lib import call, lib, on_device, ptr, stream_of

H, I, TOPK = 6144, 2048, 8
LONG_ROWS = 2048        # EXL3_PREFILL_GB300_ROWS: longer chunks run on moe4t with 256-pick blocks (tier_split.py:543)
I4_Q_GU, I4_S_GU = I * H // 2, I * (H // 128) * 2          # bytes of one gate / up matrix (codes, scales)
I4_Q_D, I4_S_D = H * I // 2, H * (I // 128) * 2            # bytes of one down matrix


def pick_groups(counts, npos, bm=64, balance=False):
    """rtx_split.py:236-255: picks sorted by expert, counts per expert; yields groups of whole experts holding at most
    npos picks as (first pick, end pick, row blocks int32 [n, 4] {expert, first pick relative to the group, picks
    <= bm, 0}). balance: an expert's blocks get near-equal sizes (base = c // nb, the first c % nb get one more)."""
    c = np.asarray(counts, dtype=np.int64).reshape(-1)
    n = c.size
    end = np.cumsum(c)
    start = end - c
    e0 = 0
    while e0 < n:
        p0 = int(start[e0])
        e1 = int(np.searchsorted(end, p0 + npos, side="right"))
        if e1 <= e0:
            raise ValueError(f"pick_groups: expert {e0} has {int(c[e0])} picks, more than npos {npos}")
        rows_l = []
        for e in range(e0, e1):
            ce = int(c[e])
            nb = (ce + bm - 1) // bm
            for k in range(nb):
                if balance:
                    base, extra = divmod(ce, nb)
                    rows, first = base + (1 if k < extra else 0), k * base + min(k, extra)
                else:
                    rows, first = min(bm, ce - bm * k), bm * k
                rows_l.append((e, int(start[e]) - p0 + first, rows, 0))
        rbt = np.array(rows_l, dtype=np.int32).reshape(-1, 4)
        yield p0, int(end[e1 - 1]), rbt
        e0 = e1


class ExpertBank:
    """int4 experts resident in HBM in the I4G128 layout: one buffer per matrix kind and int64 device tables of each
    expert's addresses (the tables tier_split.py:206-214,246 builds), local ids 0..n-1"""

    def __init__(self, n, device):
        self.n = n
        self.device = torch.device(device)
        mk = lambda nb: torch.empty(max(n, 1) * nb, dtype=torch.uint8, device=self.device)
        self.buf = {"gate_q": mk(I4_Q_GU), "gate_s": mk(I4_S_GU), "up_q": mk(I4_Q_GU), "up_s": mk(I4_S_GU),
                    "down_q": mk(I4_Q_D), "down_s": mk(I4_S_D)}
        self.size = {"gate_q": I4_Q_GU, "gate_s": I4_S_GU, "up_q": I4_Q_GU, "up_s": I4_S_GU, "down_q": I4_Q_D,
                     "down_s": I4_S_D}
        self.tab = {k: torch.tensor([self.addr(k, e) for e in range(max(n, 1))], dtype=torch.int64, device=self.device)
                    for k in self.buf}

    def addr(self, kind, e):
        return self.buf[kind].data_ptr() + e * self.size[kind]

    def view(self, kind, e):
        return self.buf[kind][e * self.size[kind]:(e + 1) * self.size[kind]]

    def tables(self):
        t = self.tab
        return t["gate_q"], t["up_q"], t["down_q"], t["gate_s"], t["up_s"], t["down_s"]

    @property
    def nbytes(self):
        return sum(b.numel() for b in self.buf.values())


def load_reference_int4(u4dir, layer, experts, device):
    """The reference's on-disk int4 experts of one layer into an ExpertBank (local id j = experts[j], e.g. a
    placement's hot prefix): the files u4dir/layer{L}.safetensors and u4dir/layer{L}.r*.safetensors with keys
    {e}.{gate,up,down}.{q,s} (tier_split.py:207-214; written by tools/quant/gptq_int4.py:205-212): uint8 codes in the
    moe4 fragment order and fp32 row scales. Each matrix is repacked on the host to I4G128 (hmoe_repack_moe4: the same
    codes, every group scale = bf16(row scale), a relative change of at most 2^-9)."""
    import glob
    import os
    from safetensors import safe_open
    files = sorted(glob.glob(os.path.join(u4dir, f"layer{layer}.safetensors")) +
                   glob.glob(os.path.join(u4dir, f"layer{layer}.r*.safetensors")))
    if not files:
        raise RuntimeError(f"load_reference_int4: no layer{layer} files in {u4dir}")
    handles = [safe_open(f, "np") for f in files]
    where = {k: h for h in handles for k in h.keys()}
    bank = ExpertBank(len(experts), device)
    for j, e in enumerate(experts):
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            kq, ks = f"{e}.{m}.q", f"{e}.{m}.s"
            if kq not in where or ks not in where:
                raise RuntimeError(f"load_reference_int4: {kq} / {ks} missing in the layer{layer} files")
            frag = np.ascontiguousarray(where[kq].get_tensor(kq)).view(np.uint8).reshape(-1)
            rs = np.ascontiguousarray(where[ks].get_tensor(ks), dtype=np.float32).reshape(-1)
            if frag.size != N * K // 2 or rs.size != N:
                raise RuntimeError(f"load_reference_int4: {kq} has {frag.size} bytes and {ks} {rs.size} scales "
                                   f"(expected {N * K // 2} and {N})")
            q = np.empty(N * K // 2, np.uint8)
            sc = np.empty(N * (K // 128), np.uint16)
            call("hmoe_repack_moe4", frag.ctypes.data, rs.ctypes.data, N, K, q.ctypes.data, sc.ctypes.data)
            bank.view(f"{m}_q", j).copy_(torch.from_numpy(q))
            bank.view(f"{m}_s", j).copy_(torch.from_numpy(sc.view(np.uint8)))
    return bank


def reference_canonical(u4dir, layer, experts):
    """the same files as load_reference_int4, as the host-CPU tier takes them (CpuTier.add_layer): per expert a dict
    of canonical row-major codes {gate,up,down}_q u8 [N, K/2] (low nibble = even k) and bf16 group scales
    {m}_s u16 [N, K/128], every group = bf16(row scale) (tier_split.py:246-250 makes its Grace copies row-major)"""
    bank = load_reference_int4(u4dir, layer, experts, "cpu")
    out = []
    for j in range(len(experts)):
        ex = {}
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            q = bank.view(f"{m}_q", j).numpy()
            s = bank.view(f"{m}_s", j).numpy()
            c = np.empty((N, K // 2), np.uint8)
            sc = np.empty((N, K // 128), np.uint16)
            call("hmoe_unpack_i4", q.ctypes.data, s.ctypes.data, N, K, c.ctypes.data, sc.ctypes.data)
            ex[m + "_q"], ex[m + "_s"] = c, sc
        out.append(ex)
    return out


class Placement:
    """one layer of the reference's placement file (tier_split.py:18, written by tools/placement/tier_placement.py:
    15-18): local expert j is original expert perm[j]; [0, hot) int4 on the accelerator, [hot, hot + far) int4 on
    the host CPU, [first, E) the reference's third band (3-bit trellis on a second GPU, not built here)"""

    def __init__(self, perm, hot, far, first):
        self.perm, self.hot, self.far, self.first = list(perm), int(hot), int(far), int(first)

    def __repr__(self):
        return f"Placement(hot={self.hot}, far={self.far}, first={self.first}, E={len(self.perm)})"


def load_placement(src):
    """the placement file {layer: {"perm": [E ids], "hot": n, "far": m, "first": n + m}} (a path, JSON text or the
    parsed dict) -> {layer (int): Placement}, checked as the reference loads it: "hot" and "far" default to 0
    (tier_split.py:174 p.get), perm is a permutation of 0 .. E - 1, hot + far <= first <= E, and a layer whose
    first reaches E (no third band, the MTP layer) keeps the identity order (tier_split.py:177)"""
    import json
    import os
    if isinstance(src, dict):
        raw = src
    elif isinstance(src, str) and os.path.exists(src):
        with open(src) as f:
            raw = json.load(f)
    else:
        raw = json.loads(src)
    out = {}
    for key, p in raw.items():
        try:
            L = int(key)
        except (TypeError, ValueError):
            raise ValueError(f"placement: layer key {key!r} is not an integer") from None
        if not isinstance(p, dict) or "perm" not in p or "first" not in p:
            raise ValueError(f"placement: layer {L} needs 'perm' and 'first'")
        perm = [int(e) for e in p["perm"]]
        E = len(perm)
        if sorted(perm) != list(range(E)):
            raise ValueError(f"placement: layer {L} perm is not a permutation of 0..{E - 1}")
        hot, far, first = int(p.get("hot", 0)), int(p.get("far", 0)), int(p["first"])
        if hot < 0 or far < 0 or hot + far > min(first, E):
            raise ValueError(f"placement: layer {L} hot {hot} far {far} first {first} (E {E})")
        if first >= E and perm != list(range(E)):
            raise ValueError(f"placement: layer {L} has no third band but a permuted order (tier_split.py:177)")
        out[L] = Placement(perm, hot, far, first)
    return out


def layer_from_reference(place, u4dir, wg, bias, device, shared=None, cpu=None, max_rows=16):
    """one layer as tier_split_load builds it (tier_split.py:171-269) from a Placement and the reference's int4 files
    (u4dir/layer{L}*.safetensors): router rows and bias permuted to the placement order (rtx_split.py:5,116: local id
    j = original expert perm[j]; wg fp32 [E, H] and bias [E] in the original order), experts perm[0:hot] resident on
    the GPU (load_reference_int4), perm[hot:hot + far] added to the host-CPU tier `cpu` (a CpuTier, if given) as
    layer `place.layer`. Picks of local ids >= hot contribute nothing on the GPU (the partial of the tier split).
    place: a Placement with a .layer attribute, or (layer, Placement)."""
    if isinstance(place, tuple):
        layer, place = place
    else:
        layer = place.layer
    if place.hot < 1 or place.first != place.hot + place.far:
        raise ValueError(f"layer {layer}: the int4 tiers need hot > 0 and first == hot + far "
                         f"(tier_split.py:189), got {place}")
    dev = torch.device(device)
    if wg.shape[0] != len(place.perm) or bias.numel() != len(place.perm):
        raise ValueError(f"layer {layer}: router of {wg.shape[0]} experts for a placement of {len(place.perm)}")
    idx = torch.tensor(place.perm, dtype=torch.int64, device=wg.device)
    wg_p = wg.index_select(0, idx).contiguous().to(dev)
    b_p = bias.reshape(-1).index_select(0, idx).contiguous().to(dev)
    bank = load_reference_int4(u4dir, layer, place.perm[:place.hot], dev)
    lay = MoELayer(wg_p, b_p, bank, shared, lo=0, n_hot=place.hot, max_rows=max_rows)
    lay.perm, lay.place, lay.layer = place.perm, place, layer
    if place.far and cpu is not None:
        cpu.add_layer(layer, place.hot, reference_canonical(u4dir, layer, place.perm[place.hot:place.first]))
    return lay


def f16t_rows(t, N, K):
    """an F16T matrix (1 KB tiles of 16 rows x 32 k, include/hecate_moe.h) as row-major f16 [N, K]: tile (nb, ks),
    lane l = 16 j + r holds row 16 nb + r at k = 32 ks + 8 j .. + 8"""
    return t.view(torch.float16).view(N // 16, K // 32, 4, 16, 8).permute(0, 3, 1, 2, 4).reshape(N, K).contiguous()


class PrefillBuffers:
    """device buffers of a prefill chunk of up to T rows: selection, dispatch plan (hmoe_dispatch), GEMM scratch"""

    def __init__(self, T, topk, lo, n, E, device, bm=128, long=False):
        dev = torch.device(device)
        L = lib()
        self.T, self.topk, self.lo, self.n, self.bm, self.long = T, topk, lo, n, bm, long
        self.F = F = T * topk
        self.nrb_max = int(L.hmoe_dispatch_nrb_max(F, n, bm))
        z = lambda *shape, dt=torch.int32: torch.zeros(shape, dtype=dt, device=dev)
        self.counts, self.tok, self.eid, self.inv = z(n), z(F), z(F), z(F)
        self.wt = z(F, dt=torch.float32)
        self.rbt, self.meta = z(self.nrb_max, 4), z(4)
        self.work = z(int(L.hmoe_dispatch_work_bytes(T, topk, n)) // 4 + 1)
        if long:
            # moe4t's ar and d (its gu is unused: not allocated; d as the f16 rows the kernels write, half the
            # reference's fp32 buffer) and the shared expert's work
            self.scr = [None, torch.empty((F, I), dtype=torch.float16, device=dev),
                        torch.empty((F, H), dtype=torch.float16, device=dev)]
            self.shw = torch.empty(int(L.hmoe_shared_work_bytes(T)) // 4 + 64, dtype=torch.float32, device=dev)
        else:
            self.scr = moe4p.scratch(dev, F, T)
        self.y = z(T, H, dt=torch.float32)
        self.out = z(T, H, dt=torch.bfloat16)
        self.xh = z(T, H, dt=torch.float16)                        # the router's f16 copy of x (the GEMM input)
        self.sel, self.rw = z(T, topk, dt=torch.int64), z(T, topk, dt=torch.float16)
        self.logits = z(int(L.hmoe_router_scratch_bytes(T, E)) // 4, dt=torch.float32)

    def run(self, sel, rw, balance=True):
        """device dispatch plan of a selection (tier_split.py:404-417 + pick_groups in one group), no host sync:
        counts, tok / eid / wt sorted by (expert, flat index), inv, rbt rows, meta = {npos, nrb, nrb wanted, 0}"""
        T = sel.shape[0]
        on_device("dispatch", sel, rw, self.counts)
        if T > self.T:
            raise RuntimeError(f"dispatch: {T} rows > {self.T}")
        call("hmoe_dispatch", ptr(sel), ptr(rw), T, self.topk, self.lo, self.n, self.bm, int(bool(balance)),
             ptr(self.counts), ptr(self.tok), ptr(self.eid), ptr(self.wt), ptr(self.inv), ptr(self.rbt),
             self.nrb_max, ptr(self.meta), ptr(self.work), stream_of(sel.device))
        return self


class MoELayer:
    """one routed int4 MoE layer: router (fp32 W_g [E, H], selection bias), resident experts for ids [lo, lo + n_hot)
    (ExpertBank, local id = id - lo), optional F16T shared expert; max_rows bounds the prefill chunk"""

    def __init__(self, wg, bias, bank, shared=None, lo=0, n_hot=None, topk=TOPK, scale=2.5, max_rows=16):
        self.wg, self.bias, self.bank, self.shared = wg, bias, bank, shared
        self.device = wg.device
        self.E = wg.shape[0]
        self.lo, self.n_hot = lo, bank.n if n_hot is None else n_hot
        self.topk, self.scale = topk, scale
        self.deterministic = True      # long prefill: ordered per-token combine (False: moe4t's atomic epilogue)
        self.max_rows = max(max_rows, 16)
        dev = self.device
        self.logits, self.ctr = router.buffers(self.max_rows, dev, self.E)
        self.sel = torch.zeros((self.max_rows, topk), dtype=torch.int64, device=dev)
        self.rw = torch.zeros((self.max_rows, topk), dtype=torch.float16, device=dev)
        self.xh = torch.zeros((self.max_rows, H), dtype=torch.float16, device=dev)
        self.y = torch.zeros((self.max_rows, H), dtype=torch.float32, device=dev)     # fp32 accumulator, kept zeroed
        self.out = torch.zeros((self.max_rows, H), dtype=torch.bfloat16, device=dev)
        self.scr = moe4.scratch(dev)
        self._pf = None
        self._shared_rows = None                                   # row-major copies of the shared expert (prefill)

    # ---- routing ---------------------------------------------------------------------------------------------
    def route(self, x, write_xh=True):
        R = x.shape[0]
        router.router_fused(x, self.wg, self.bias, self.logits, self.ctr, self.sel[:R], self.rw[:R], self.topk,
                            self.scale, self.xh[:R] if write_xh else None)
        return self.sel[:R], self.rw[:R]

    # ---- decode ----------------------------------------------------------------------------------------------
    def experts_decode(self, R, y, with_shared=True, blocks=0, xh=None, events=None):
        """moe4.forward on the routed selection (and the shared expert) of xh (default self.xh)[:R], added into y;
        events: three torch.cuda.Events recorded before gate/up, between the phases and after down"""
        gq, uq, dq, gs, us, ds = self.bank.tables()
        sh = self.shared if (with_shared and self.shared is not None) else (0, 0, 0)
        xh = self.xh if xh is None else xh
        if events is None:
            moe4.forward(xh[:R], self.sel[:R], self.rw[:R], self.n_hot, gq, uq, dq, gs, us, ds, *self.scr, y, blocks,
                         0, self.lo, sh[0], sh[1], sh[2], 0, 0, 0)
            return
        act, gu32, ctr_a, y32, ctr_b = self.scr
        events[0].record()
        moe4.gate_up(xh[:R], self.sel[:R], self.rw[:R], self.n_hot, gq, uq, gs, us, act, gu32, ctr_a, blocks, self.lo,
                     sh[0], sh[1])
        events[1].record()
        moe4.down(self.sel[:R], self.rw[:R], self.n_hot, dq, ds, act, y32, ctr_b, y, blocks, self.lo, sh[2])
        events[2].record()

    def decode(self, x, y=None, out=True, with_shared=True, phases=15, blocks=0):
        """the decode layer in four launches (hmoe_moe_decode_layer): router + routed + shared experts of x bf16
        [R, H]; returns the bf16 [R, H] output (out=True) and / or adds into the fp32 y. phases: bit mask of the
        launches (1 router, 2 shared + routed gate/up, 4 shared + routed down, 8 output) for callers that time them
        apart"""
        R = x.shape[0]
        on_device("decode", x, self.wg, y)
        if not (1 <= R <= 16 and x.dtype == torch.bfloat16 and x.is_contiguous() and x.shape[1] == H):
            raise RuntimeError("decode: x must be contiguous bf16 [R <= 16, 6144]")
        gq, uq, dq, gs, us, ds = self.bank.tables()
        sh = self.shared if (with_shared and self.shared is not None) else (None, None, None)
        act, gu32, ctr_a, y32, _ = self.scr
        o = self.out[:R] if out else None
        call("hmoe_moe_decode_layer", ptr(x), ptr(self.wg), ptr(self.bias), self.E, self.topk, float(self.scale),
             ptr(self.logits), ptr(self.sel), ptr(self.rw), R, self.n_hot, self.lo, ptr(gq), ptr(uq), ptr(dq), ptr(gs),
             ptr(us), ptr(ds), ptr(sh[0]), ptr(sh[1]), ptr(sh[2]), ptr(act), ptr(gu32), ptr(ctr_a), ptr(y32),
             ptr(y), ptr(o), int(blocks), int(phases), stream_of(x.device))
        return o

    # ---- prefill ----------------------------------------------------------------------------------------------
    def _prefill_buffers(self, T):
        long = T > LONG_ROWS
        if self._pf is not None and self._pf.T >= T and self._pf.long == long:
            return self._pf
        self._pf = None
        self._pf = PrefillBuffers(T, self.topk, self.lo, self.n_hot, self.E, self.device, bm=256 if long else 128,
                                  long=long)
        return self._pf

    def prefill_experts(self, x, y, with_shared=True, out_bf16=None):
        """routed (+ shared) experts of x's routed selection (in the prefill buffers) added into y fp32 [T, H].
        With out_bf16 (bf16 [T, H]) the layer output bf16(experts) is written there instead, and y must hold zeros on
        entry (as MoELayer keeps it) and holds zeros on return: the moe4p form never reads y, the moe4t form (ordered
        combine) adds the shared expert into y first and its combine rounds y + picks and re-zeroes y. Returns whether
        out_bf16 was written (the atomic moe4t form adds into y instead)."""
        T = x.shape[0]
        pf = self._pf
        gq, uq, dq, gs, us, ds = self.bank.tables()
        if pf.long:
            # tier_split.py:427-462: every routed expert on moe4t (256-pick balanced blocks, the down GEMM adding into
            # y), the shared expert apart. With out_bf16 and the ordered combine, the shared expert goes into y first
            # and the combine rounds y + picks to out_bf16 (y + s equals s + y bit for bit) and re-zeroes y
            fused = out_bf16 is not None and self.deterministic
            if fused and with_shared and self.shared is not None:
                moe4t.shared(x, *self.shared_rows(), pf.shw, y)
            moe4t.forward(x, pf.tok, pf.eid, pf.wt, pf.rbt, gq, uq, dq, gs, us, ds, *pf.scr, y, meta=pf.meta,
                          npos=pf.F, nrb=pf.nrb_max, inv=pf.inv[:T * self.topk] if self.deterministic else None,
                          topk=self.topk, out_bf16=out_bf16 if fused else None)
            if not fused and with_shared and self.shared is not None:
                moe4t.shared(x, *self.shared_rows(), pf.shw, y)
            return fused
        sh = self.shared_rows() if (with_shared and self.shared is not None) else None
        moe4p.forward(x, pf.tok, pf.eid, pf.wt, pf.rbt, gq, uq, dq, gs, us, ds, *pf.scr,
                      y if out_bf16 is None else None, inv=pf.inv[:T * self.topk], meta=pf.meta, topk=self.topk,
                      shared=sh, npos=pf.F, nrb=pf.nrb_max, out_bf16=out_bf16)
        return out_bf16 is not None

    def shared_rows(self):
        """the shared expert as row-major f16 (gate [I, H], up [I, H], down [H, I]) for the prefill's dense GEMMs,
        made from the F16T copies on first use"""
        if self._shared_rows is None:
            g, u, d = self.shared
            gu = torch.cat([f16t_rows(g, I, H), f16t_rows(u, I, H)])
            self._shared_rows = (gu[:I], gu[I:], f16t_rows(d, H, I))
        return self._shared_rows

    def prefill(self, x, with_shared=True):
        """the prefill layer: bf16 [T, H] out (router, device dispatch plan, grouped GEMMs, per-token combine); an
        empty chunk gives an empty output (tier_split.py:377 returns out when no pick reaches the tier). Chunks of more
        than LONG_ROWS rows run the routed experts on moe4t (256-pick blocks), as the reference does, with the ordered
        per-token combine through the inverse map (deterministic; MoELayer.deterministic = False takes the reference's
        atomic down epilogue)"""
        T = x.shape[0]
        on_device("prefill", x, self.wg)
        if T == 0:
            return torch.empty((0, H), dtype=torch.bfloat16, device=x.device)
        pf = self._prefill_buffers(T)
        sel, rw = pf.sel[:T], pf.rw[:T]
        router.router_fused(x, self.wg, self.bias, pf.logits, self.ctr, sel, rw, self.topk, self.scale, pf.xh[:T])
        pf.run(sel, rw, balance=True)
        y = pf.y[:T]
        # (y is kept zeroed, so the moe4p path writes the bf16 output from its combine directly)
        if self.prefill_experts(pf.xh[:T], y, with_shared, out_bf16=pf.out[:T]):
            return pf.out[:T]
        return moe4.finish_bf16(y, T, pf.out[:T])

    def forward(self, x):
        return self.decode(x) if x.shape[0] <= 16 else self.prefill(x)
