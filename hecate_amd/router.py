"""Fused sigmoid + bias top-k router: the drop-in for runtime/core/exl3_router.py:134-146 router_fused.

router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale) keeps the reference's arguments (x bf16 here, wt fp32
[E, K]); the trailing xh receives an f16 copy of x for moe4.forward(xf=1). Any row count (the reference handles 2..8).
"""
import torch

from ._lib import call, lib, ptr, stream_of


def buffers(R, device, E=256):
    """(logits scratch, self-resetting counter) for up to R rows"""
    dev = torch.device(device)
    n = int(lib().hmoe_router_scratch_bytes(R, E)) // 4
    return torch.zeros(n, dtype=torch.float32, device=dev), torch.zeros(1, dtype=torch.int32, device=dev)


def router_fused(x, wt, bias, logits, ctr, sel, rw, topk, scale, xh=None):
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
