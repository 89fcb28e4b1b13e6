"""A decode step through consecutive MoE layers with the residual + RMSNorm between them (runtime/tier/cn.cu:48-103:
the combine of layer l folded into the input norm of layer l + 1), as one hipGraph.

h = x (fp32); per layer l: r += y_(l-1) (y zeroed), xn = bf16(RMSNorm(h) w_l) (+ its f16 copy), route(xn),
y_l = routed + shared experts of xn; finally h += y_(L-1). Five launches per layer (norm, then the decode layer's
four) and one combine, all static-shaped and allocation-free.
"""
import torch

from . import moe4
from ._lib import call, ptr, stream_of

H = 6144


class DecodeStack:
    def __init__(self, layers, norm_w, R, eps=1e-5):
        if not 1 <= R <= 16:
            raise RuntimeError(f"DecodeStack: {R} rows")
        dev = layers[0].device
        self.layers, self.norm_w, self.R, self.eps = layers, norm_w, R, eps
        self.x = torch.zeros((R, H), dtype=torch.bfloat16, device=dev)      # the step's input (static address)
        self.h = torch.zeros((R, H), dtype=torch.float32, device=dev)       # residual stream
        self.y = torch.zeros((R, H), dtype=torch.float32, device=dev)       # MoE output of the current layer
        self.xn = torch.zeros((R, H), dtype=torch.bfloat16, device=dev)
        self.xh = torch.zeros((R, H), dtype=torch.float16, device=dev)
        self.graph = None

    def step(self, trace=None):
        """one step; trace (eager only): a list that receives per layer (residual after the add, xn, y, sel, rw)"""
        R = self.R
        self.h.copy_(self.x)
        st = stream_of(self.h.device)
        for l, lay in enumerate(self.layers):
            call("hmoe_residual_rmsnorm", ptr(self.h), ptr(self.y) if l > 0 else None, ptr(self.norm_w[l]), R,
                 float(self.eps), ptr(self.xn), None, st)
            if trace is not None:
                trace.append([self.h.clone(), self.xn.clone()])
            lay.decode(self.xn, y=self.y, out=False)
            if trace is not None:
                trace[-1] += [self.y.clone(), lay.sel[:R].clone(), lay.rw[:R].clone()]
        moe4.combine(self.h, 0, self.y, R)
        return self.h

    def capture(self):
        """capture step() into a hipGraph (after one eager step to settle every buffer)"""
        self.step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        torch.cuda.synchronize()
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()
        return self.h
