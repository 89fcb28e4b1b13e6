"""A decode step through consecutive MoE layers with the residual + RMSNorm between them, as one hipGraph.

h = x (fp32); per layer l: xn = bf16(RMSNorm(h) w_l), route(xn), h += routed + shared experts of xn. Every norm uses
the reduction order of the reference's rms_norm_kernel (include/hecate_moe.h).

fused (default), by row count:
  one row   three launches per layer: RMSNorm + router logits (runtime/tier/nr4_kernel.cuh:122-381), then the
            decode layer's gate/up and down launches, the down launch adding the layer's output into h itself;
  more rows four launches per layer: the router logits of xn, gate/up, the down partials, then the layer's output
            combine fused with the next layer's input norm (runtime/tier/cn.cu:48-103, hmoe_decode_combine_norm: the
            parts summed in order, h += them, xn of the next layer); after the last layer the plain output launch.
Unfused: the residual + RMSNorm kernel, the router inside the decode layer, the output into y, and one final combine.
All forms give the same bits. Static-shaped and allocation-free either way.
"""
import torch

from . import moe4, router
from ._lib import DT_BF16, DT_F32, call, ptr, stream_of

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
        rw); in the fused forms the layer output is never materialised and its trace entry is None"""
        R = self.R
        self.h.copy_(self.x)
        st = stream_of(self.h.device)
        L = len(self.layers)
        parts = fused and R > 1
        if parts:
            call("hmoe_residual_rmsnorm", ptr(self.h), None, ptr(self.norm_w[0]), R, float(self.eps), ptr(self.xn),
                 None, st)
        for l, lay in enumerate(self.layers):
            if fused and not parts:
                router.norm_router(self.h, self.norm_w[l], self.eps, lay.wg, lay.logits, self.xn)
            elif not fused:
                call("hmoe_residual_rmsnorm", ptr(self.h), ptr(self.y) if l > 0 else None, ptr(self.norm_w[l]), R,
                     float(self.eps), ptr(self.xn), None, st)
            if trace is not None:
                trace.append([self.h.clone(), self.xn.clone()])
            if parts:
                # router logits, gate/up, down partials; then the parts into h with the next layer's norm (or, after
                # the last layer, the plain output launch adding them into h)
                lay.decode(self.xn, y=self.h, out=False, phases=7)
                if l + 1 < L:
                    act, gu32, ctr_a, y32, _ = lay.scr
                    call("hmoe_decode_combine_norm", ptr(y32), ptr(ctr_a), R, ptr(self.h), ptr(self.norm_w[l + 1]),
                         ptr(self.xn), None, float(self.eps), 0.0, 1.0, DT_F32, DT_BF16, st)
                else:
                    lay.decode(self.xn, y=self.h, out=False, phases=8)
            elif fused:
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
