"""Prefill MoE operator: the drop-in for the reference's `moe4p` extension (runtime/tier/moe4/moe4p.cu:209-251).

forward(x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out) keeps the reference's names and order; the
trailing keywords (inv, meta, topk, shared) are this build's additions: a deterministic per-token combine, sizes read
from a device-side dispatch plan (no host sync), and the shared expert in the same call.
"""
import torch

from ._lib import XF_BF16, call, lib, on_device, ptr, stream_of, xf_of

H, I = 6144, 2048


def scratch(dev, npos, T=0):
    """moe4p.cu:209-215: [gu, ar, d] for up to npos picks (+ T rows for the shared expert); gu holds the f16 copy of
    x when forward gets bf16 x"""
    dev = torch.device(dev)
    L = lib()
    return [torch.zeros(int(L.hmoe_moe4p_scratch_bytes(0, npos, T)) // 4, dtype=torch.float32, device=dev),
            torch.empty((npos + T, I), dtype=torch.float16, device=dev),
            torch.empty((npos + T, H), dtype=torch.float32, device=dev)]


def forward(x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out, inv=None, meta=None, topk=8, shared=None,
            npos=None, nrb=None, out_bf16=None):
    """moe4p.cu:220-245: out[tok] += routed experts of the sorted picks (+ the shared expert on every token); x bf16, or
    its f16 copy (as router_fused writes it). out_bf16 (bf16 [T, H], with inv; out then None): the layer output
    written directly, as forward into a zero out followed by moe4.finish_bf16 (hmoe_moe4p_forward_bf16)"""
    T = x.shape[0]
    if out_bf16 is not None:
        if out is not None or inv is None or out_bf16.dtype != torch.bfloat16 or not out_bf16.is_contiguous() \
                or tuple(out_bf16.shape) != (T, H):
            raise RuntimeError("moe4p: out_bf16 (bf16 [T, H]) replaces out and needs the inverse map")
        out = out_bf16
    on_device("moe4p", x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out, inv, meta,
              *(shared if shared is not None else ()))
    if shared is not None and not all(w.dtype == torch.float16 and w.is_contiguous() and w.numel() == I * H
                                      for w in shared):
        raise RuntimeError("moe4p: the shared expert is row-major f16 gate [I, H], up [I, H], down [H, I]")
    xf = xf_of(x)
    if not (x.dim() == 2 and x.shape[1] == H and x.dtype in (torch.bfloat16, torch.float16)
            and (out.dtype == torch.float32 or out_bf16 is not None)
            and rbt.dim() == 2 and rbt.shape[1] == 4 and x.is_contiguous() and out.is_contiguous()):
        raise RuntimeError("moe4p: shapes")
    npos = tok.numel() if npos is None else npos
    nrb = rbt.shape[0] if nrb is None else nrb
    ps = ar.shape[0] - (T if shared is not None else 0)
    if npos > ps or d.shape[0] < ar.shape[0]:
        raise RuntimeError(f"moe4p: scratch holds {ps} picks, {npos} given")
    # the scratch at least as large as the library writes it (a short one would be written past its end): gu holds
    # the f16 copy of x when x is bf16
    need = int(lib().hmoe_moe4p_scratch_bytes(0, ps, T)) if xf == XF_BF16 else 0
    if need and (gu is None or gu.numel() * gu.element_size() < need):
        raise RuntimeError(f"moe4p: the gu scratch needs {need} bytes")
    if ar.dim() != 2 or ar.shape[1] != I or d.dim() != 2 or d.shape[1] != H:
        raise RuntimeError("moe4p: ar f16 [rows, I] and d fp32 [rows, H]")
    sh = shared if shared is not None else (None, None, None)
    if out_bf16 is not None:
        call("hmoe_moe4p_forward_bf16", ptr(x), ptr(tok), ptr(eid), ptr(wt), ptr(rbt), int(npos), int(nrb), gw.numel(),
             ptr(gw), ptr(uw), ptr(dw), ptr(gs), ptr(us), ptr(ds), ptr(gu), ptr(ar), ptr(d), int(ps), ptr(meta),
             ptr(inv), int(T), int(topk), ptr(sh[0]), ptr(sh[1]), ptr(sh[2]), xf, ptr(out_bf16), stream_of(x.device))
        return
    call("hmoe_moe4p_forward", ptr(x), ptr(tok), ptr(eid), ptr(wt), ptr(rbt), int(npos), int(nrb), gw.numel(),
         ptr(gw), ptr(uw), ptr(dw), ptr(gs), ptr(us), ptr(ds), ptr(gu), ptr(ar), ptr(d), ptr(out), int(ps),
         ptr(meta), ptr(inv), int(T), int(topk), ptr(sh[0]), ptr(sh[1]), ptr(sh[2]), xf, stream_of(x.device))
