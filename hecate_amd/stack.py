"""A decode step through consecutive MoE layers with the residual + RMSNorm between them, as one hipGraph.

h = x (fp32); per layer l: xn = bf16(RMSNorm(h) w_l), route(xn), h += routed + shared experts of xn.

fused (default): four launches per layer: RMSNorm + router logits (runtime/tier/nr4_kernel.cuh:122-381), then the
decode layer's gate/up, down and output launches, the last adding the layer's output into h (the combine of
runtime/tier/cn.cu:48-103). Unfused: five launches per layer, the combine folded into the next layer's input norm
(cn.cu:48-103: r += y_(l-1), y zeroed, then the norm), the router in the decode layer, and one final combine; both
give the same bits. Static-shaped and allocation-free either way.
"""
import torch

from . import moe4, router
from ._lib import call, ptr, stream_of

H = 6144


class DecodeStack:
    def __init__(self, layers, norm_w, R, eps=1e-5):
        if not 1 <= R <= 16:
            raise RuntimeError(f"DecodeStack: {R} rows")
        dev = layers[0].device
        if len(norm_w) < len(layers) or any(w.device != dev or w.dtype != torch.float32 or w.numel() != H for w in norm_w):
            raise RuntimeError("DecodeStack: one fp32 [H] norm weight per layer, on the layers' device")
        self.layers, self.norm_w, self.R, self.eps = layers, norm_w, R, eps
        self.x = torch.zeros((R, H), dtype=torch.bfloat16, device=dev)      # the step's input (static address)
        self.h = torch.zeros((R, H), dtype=torch.float32, device=dev)       # residual stream
        self.y = torch.zeros((R, H), dtype=torch.float32, device=dev)       # MoE output of the current layer
        self.xn = torch.zeros((R, H), dtype=torch.bfloat16, device=dev)
        self.xh = torch.zeros((R, H), dtype=torch.float16, device=dev)
        self.graph = None

    def step(self, trace=None, fused=True):
        """one step; trace (eager only): a list that receives per layer (residual at the layer's input, xn, y, sel,
        rw); fused: y is added into the residual by the layer's output launch, and its trace entry is None"""
        R = self.R
        self.h.copy_(self.x)
        st = stream_of(self.h.device)
        for l, lay in enumerate(self.layers):
            if fused:
                router.norm_router(self.h, self.norm_w[l], self.eps, lay.wg, lay.logits, self.xn)
            else:
                call("hmoe_residual_rmsnorm", ptr(self.h), ptr(self.y) if l > 0 else None, ptr(self.norm_w[l]), R,
                     float(self.eps), ptr(self.xn), None, st)
            if trace is not None:
                trace.append([self.h.clone(), self.xn.clone()])
            if fused:
                lay.decode(self.xn, y=self.h, out=False, phases=14)
            else:
                lay.decode(self.xn, y=self.y, out=False)
            if trace is not None:
                trace[-1] += [None if fused else self.y.clone(), lay.sel[:R].clone(), lay.rw[:R].clone()]
        if not fused:
            moe4.combine(self.h, 0, self.y, R)
        return self.h

    def capture(self, fused=True):
        """capture step() into a hipGraph (after one eager step to settle every buffer)"""
        self.step(fused=fused)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step(fused=fused)
        torch.cuda.synchronize()
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()
        return self.h
