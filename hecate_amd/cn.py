"""The MoE combine fused into the next input norm: the drop-in for runtime/tier/cn.cu:189-235 combine_norm.

combine_norm(f, o, y, rows, o2, done, r, w, xn, eps, cbias, cscale) keeps the reference's arguments: f, y, r fp32
[rows, H]; o / o2 device addresses of fp32 partials (0 = none); done must be 0 (the RTX band's DONE flag; that band is
not built); w the norm weight (fp16 or bf16 as in the reference, or fp32); xn the normed rows (fp16 as in the
reference, or bf16). a = ((f + y) + o) + o2, y zeroed, r = a + r, xn = RMSNorm(r) in the reduction order of the
reference's rms_norm_kernel (include/hecate_moe.h). f may be None (read as +0, as combine_norm_pdl takes it).

combine_norm_cpu(f, o, y, rows, cpu, r, w, xn, eps, cbias, cscale): the same with the CPU tier's partial in the o2
position, added once the job posted through norm_route's hand-off has finished (combine_norm_pdl's CPU_DONE wait,
cn.cu:108-142); cpu is a CpuTier (or its mailbox address).
"""
from ._lib import call, dt_of, on_device, ptr, stream_of

H = 6144


def combine_norm(f, o, y, rows, o2, done, r, w, xn, eps, cbias=0.0, cscale=1.0):
    on_device("combine_norm", r, f, y, w, xn)
    rows = int(rows)
    for name, t in (("y", y), ("r", r)) + ((("f", f),) if f is not None else ()):
        if t.dtype.itemsize != 4 or str(t.dtype) != "torch.float32" or not t.is_contiguous() or t.numel() < rows * H:
            raise RuntimeError(f"combine_norm: {name} must be contiguous fp32 [>= {rows}, {H}]")
    if w.numel() != H or not w.is_contiguous() or not xn.is_contiguous() or xn.numel() < rows * H:
        raise RuntimeError("combine_norm: w must be [H], xn [rows, H], contiguous")
    call("hmoe_combine_norm", ptr(f), ptr(o), ptr(y), rows, ptr(o2), ptr(done), ptr(r), ptr(w), ptr(xn), float(eps),
         float(cbias), float(cscale), dt_of(w), dt_of(xn, ("bfloat16", "float16")), stream_of(r.device))
    return xn


def combine_norm_cpu(f, o, y, rows, cpu, r, w, xn, eps, cbias=0.0, cscale=1.0):
    on_device("combine_norm_cpu", r, f, y, w, xn)
    rows = int(rows)
    mb = getattr(cpu, "addr", cpu)
    if not mb:
        raise RuntimeError("combine_norm_cpu: no mailbox")
    for name, t in (("y", y), ("r", r)) + ((("f", f),) if f is not None else ()):
        if str(t.dtype) != "torch.float32" or not t.is_contiguous() or t.numel() < rows * H:
            raise RuntimeError(f"combine_norm_cpu: {name} must be contiguous fp32 [>= {rows}, {H}]")
    if w.numel() != H or not w.is_contiguous() or not xn.is_contiguous() or xn.numel() < rows * H:
        raise RuntimeError("combine_norm_cpu: w must be [H], xn [rows, H], contiguous")
    call("hmoe_combine_norm_cpu", ptr(f), ptr(o), ptr(y), rows, mb, ptr(r), ptr(w), ptr(xn), float(eps), float(cbias),
         float(cscale), dt_of(w), dt_of(xn, ("bfloat16", "float16")), stream_of(r.device))
    return xn
