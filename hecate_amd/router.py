"""Fused sigmoid + bias top-k router: the drop-in for runtime/core/exl3_router.py:134-146 router_fused.

router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale) keeps the reference's arguments (x bf16 here, wt fp32
[E, K]); the trailing xh receives an f16 copy of x (moe4.forward reads fp16 x as the reference does). Any row count (the reference handles 2..8).
"""
import torch

from ._lib import call, lib, on_device, ptr, stream_of


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
