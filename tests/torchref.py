"""A GPU fp32 reference of the MoE layer for checking every row of a large chunk: torch fp32 GEMMs (no reduced
precision) on the library's own dequantised weights (moe4.dequant: f16(q * s), the value the prefill GEMMs multiply).
It is itself checked against the CPU oracle's exact mode on sampled rows by the tests that use it, so it pins the
rows the oracle cannot afford to compute. Test infrastructure only."""
import torch
import torch.nn.functional as F

from hecate_amd import moe4, tier

H, I = 6144, 2048


def moe_rows(lay, x, sel, rw, with_shared=True):
    """y fp32 [T, H] = sum over the picks in the layer's window of rw * down(silu(gate x) * up x) (+ the shared expert)
    for x bf16 / fp16 [T, H] and the given selection (sel int64 [T, k], rw f16 [T, k]), all on the device"""
    torch.backends.cuda.matmul.allow_tf32 = False
    T, k = sel.shape
    xf = x.float()
    y = torch.zeros((T, H), dtype=torch.float32, device=x.device)
    flat_e = (sel.reshape(-1) - lay.lo)
    flat_t = torch.arange(T, device=x.device).repeat_interleave(k)
    flat_w = rw.reshape(-1).float()
    inside = (flat_e >= 0) & (flat_e < lay.n_hot)
    bank = lay.bank
    for e in torch.unique(flat_e[inside]).tolist():
        m = flat_e == e
        toks, w = flat_t[m], flat_w[m]
        wg = moe4.dequant(bank.view("gate_q", e), bank.view("gate_s", e), I, H).float()
        wu = moe4.dequant(bank.view("up_q", e), bank.view("up_s", e), I, H).float()
        wd = moe4.dequant(bank.view("down_q", e), bank.view("down_s", e), H, I).float()
        xe = xf[toks]
        a = F.silu(F.linear(xe, wg)) * F.linear(xe, wu) * w[:, None]
        y.index_add_(0, toks, F.linear(a, wd))
        del wg, wu, wd
    if with_shared and lay.shared is not None:
        g, u, d = lay.shared
        wg, wu, wd = (tier.f16t_rows(g, I, H).float(), tier.f16t_rows(u, I, H).float(), tier.f16t_rows(d, H, I).float())
        y += F.linear(F.silu(F.linear(xf, wg)) * F.linear(xf, wu), wd)
    return y
