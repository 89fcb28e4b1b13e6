"""Fused sigmoid + bias top-k router: the drop-in for runtime/core/exl3_router.py:134-146 router_fused.

router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale) keeps the reference's arguments (x bf16 here, wt fp32
[E, K]); the trailing xh receives an f16 copy of x (moe4.forward reads fp16 x as the reference does). Any row count (the reference handles 2..8).
"""
import ctypes

import torch

from ._lib import call, dt_of, lib, on_device, ptr, stream_of


def buffers(R, device, E=256):
    """(logits scratch, self-resetting counter) for up to R rows"""
    dev = torch.device(device)
    n = int(lib().hmoe_router_scratch_bytes(R, E)) // 4
    return torch.zeros(n, dtype=torch.float32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev)


def router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale, xh=None):
    on_device("router_fused", x, wt, bias, logits, ctr, sel, rw, xh)
    K = x.shape[-1]
    R = x.numel() // K
    E = wt.shape[0]
    if not (x.dtype == torch.bfloat16 and wt.dtype == torch.float32 and x.is_contiguous() and wt.is_contiguous()
            and sel.dtype == torch.int64 and rw.dtype == torch.float16 and logits.numel() * 4 >= int(
                lib().hmoe_router_scratch_bytes(R, E))):
        raise RuntimeError("router_fused: shape / dtype")
    call("hmoe_router_fused", ptr(x), ptr(wt), ptr(bias), ptr(logits), ptr(ctr), ptr(sel), ptr(rw), int(R), int(K),
         int(E), int(topk), float(scale), ptr(xh), stream_of(x.device))
    return sel, rw


def norm_router(h, norm_w, eps, wt, logits, xn, xh=None):
    """nr4_kernel.cuh:122-381 (RMSNorm + router scores in one launch) for the decode path: xn = bf16 RMSNorm(h) * norm_w
    (bit-identical to hmoe_residual_rmsnorm without a residual add) and the router logits of xn into logits (the
    layout MoELayer.decode reads with phases=14); h fp32 [R, H], R <= 16"""
    on_device("norm_router", h, norm_w, wt, logits, xn, xh)
    R, K = h.shape
    E = wt.shape[0]
    if not (h.dtype == torch.float32 and norm_w.dtype == torch.float32 and wt.dtype == torch.float32
            and xn.dtype == torch.bfloat16 and h.is_contiguous() and xn.is_contiguous() and xn.shape == h.shape
            and 1 <= R <= 16 and logits.numel() * 4 >= int(lib().hmoe_router_scratch_bytes(R, E))):
        raise RuntimeError("norm_router: shape / dtype")
    call("hmoe_norm_router", ptr(h), ptr(norm_w), float(eps), int(R), ptr(wt), int(E), ptr(logits), ptr(xn), ptr(xh),
         stream_of(h.device))
    return xn


def norm_route_buffers(R, device, E=256):
    """(cand, ctr) scratch of norm_route for up to R rows: the logits buffer and the reference's counter argument"""
    dev = torch.device(device)
    n = int(lib().hmoe_norm_route_scratch_bytes(R, E)) // 4
    return torch.zeros(n, dtype=torch.float32, device=dev), torch.zeros(64, dtype=torch.int32, device=dev)


def norm_route(y, r, w, x2, gt, bias, sel, rw, cand, ctr, scale, eps, cbias=0.0, cscale=1.0, ho=None):
    """runtime/core/exl3_normroute.py:16-65 norm_route (nr4_kernel.cuh:122-381): r = y + r, x2 = RMSNorm(r) * (w +
    cbias) * cscale (fp16 as in the reference, or bf16), then the router on x2: gt [E, H] fp16 (the reference's
    transposed gate) or fp32, bias fp32 [E] or None, sel int64 / rw fp16 [R, 8]. cand / ctr: norm_route_buffers. ho:
    the band hand-off words, empty or (mailbox, layer) of this build's CPU tier (CpuTier.handoff(layer)): the
    selection launch then also posts the CPU tier's job (x2 bf16, R <= 8), as the reference's kernel releases its
    Grace band's ISSUE (nr4_kernel.cuh:360-378); the reference's 10 / 11-word form addresses bands not built here."""
    on_device("norm_route", y, r, w, x2, gt, bias, sel, rw, cand, ctr)
    R = y.numel() // y.shape[-1]
    E = gt.shape[0]
    ho = list(ho) if ho else []
    if ho and len(ho) != 2:
        raise RuntimeError("norm_route: ho must be empty or (mailbox, layer)")
    hw = (ctypes.c_int64 * 2)(*[int(v) for v in ho]) if ho else None
    if not (y.dtype == torch.float32 and r.dtype == torch.float32 and y.shape[-1] == 6144 and r.numel() == y.numel()
            and x2.numel() >= y.numel() and y.is_contiguous() and r.is_contiguous() and x2.is_contiguous()
            and gt.is_contiguous() and gt.shape[1] == 6144 and w.numel() == 6144 and sel.dtype == torch.int64
            and rw.dtype == torch.float16 and cand.numel() * 4 >= int(lib().hmoe_norm_route_scratch_bytes(R, E))):
        raise RuntimeError("norm_route: shape / dtype")
    call("hmoe_norm_route", ptr(y), ptr(r), ptr(w), ptr(x2), ptr(gt), ptr(bias), ptr(sel), ptr(rw), ptr(cand),
         ptr(ctr), float(scale), float(eps), float(cbias), float(cscale), ctypes.addressof(hw) if hw else None, len(ho), int(R), int(E), dt_of(w),
         dt_of(x2, ("bfloat16", "float16")), dt_of(gt, ("float32", "float16")), stream_of(y.device))
    return sel, rw
