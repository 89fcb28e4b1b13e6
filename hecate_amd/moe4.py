"""Decode MoE operator: the drop-in for the reference's `moe4` extension (runtime/tier/moe4/moe4.cu:897-925).

Same op names and argument order as the reference's pybind module; formats are this build's gfx950 ones
(include/hecate_moe.h): x row-major bf16 or fp16 (the reference's fp16 x with xf=0 works unchanged; its fragment-order
xf=1 is refused), I4G128 experts with bf16 group-128 scales, the shared
expert as F16T. Work runs on the current torch stream; errors raise RuntimeError like TORCH_CHECK.
"""
import torch

from ._lib import call, lib, on_device, ptr, stream_of, xf_of

H, I, TOPK, MAXR = 6144, 2048, 8, 16


def _req(cond, msg):
    if not cond:
        raise RuntimeError(f"moe4: {msg}")


def scratch(device):
    """moe4.cu:897-902: [act, gu32, ctr_a, y32, ctr_b] (workspace: any contents work, gu32 / ctr_b are unused)"""
    dev = torch.device(device)
    L = lib()
    nb = [int(L.hmoe_moe4_scratch_bytes(i)) for i in range(5)]
    return [torch.zeros(nb[0] // 2, dtype=torch.float16, device=dev),
            torch.zeros(nb[1] // 4, dtype=torch.float32, device=dev),
            torch.zeros(nb[2] // 4, dtype=torch.int32, device=dev),
            torch.zeros(nb[3] // 4, dtype=torch.float32, device=dev),
            torch.zeros(nb[4] // 4, dtype=torch.int32, device=dev)]


def _addr(v):
    if v is None or (isinstance(v, int) and v == 0):
        return None
    return ptr(v)


def forward(x, sel, rw, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, act, gu32, ctr_a, y32, ctr_b, y, blocks,
            blocks_a, lo, sh_gw=0, sh_uw=0, sh_dw=0, sh_gs=0, sh_us=0, sh_ds=0, xf=0):
    """moe4.cu:828-895: y[R][H] (fp32) += routed experts of the picks in [lo, lo + n_hot) (+ the shared expert)"""
    R = x.shape[0]
    on_device("moe4", x, sel, rw, gate_w, up_w, down_w, gate_s, up_s, down_s, act, gu32, ctr_a, y32, ctr_b, y)
    _req(1 <= R <= MAXR and x.shape[-1] == H, f"x shape {tuple(x.shape)}")
    fmt = xf_of(x, xf)
    _req(x.is_contiguous() and x.is_cuda, "x layout")
    _req(sel.dtype == torch.int64 and sel.is_contiguous() and sel.shape == (R, TOPK),
         "selection must be contiguous int64 [R, 8]")
    _req(rw.dtype == torch.float16 and rw.is_contiguous() and rw.shape == (R, TOPK), "routing weights f16 [R, 8]")
    _req(y.dtype == torch.float32 and y.is_contiguous() and y.shape[-1] == H and y.numel() >= R * H, "y fp32 [R, H]")
    for t in (gate_w, up_w, down_w, gate_s, up_s, down_s):
        _req(t.dtype == torch.int64 and t.is_cuda and t.numel() >= n_hot, "pointer tables int64 [n_hot]")
    call("hmoe_moe4_forward", ptr(x), ptr(sel), ptr(rw), R, int(n_hot), ptr(gate_w), ptr(up_w), ptr(down_w),
         ptr(gate_s), ptr(up_s), ptr(down_s), ptr(act), ptr(gu32), ptr(ctr_a), ptr(y32), ptr(ctr_b), ptr(y),
         int(blocks), int(blocks_a), int(lo), _addr(sh_gw), _addr(sh_uw), _addr(sh_dw), _addr(sh_gs), _addr(sh_us),
         _addr(sh_ds), fmt, stream_of(x.device))


def gate_up(x, sel, rw, n_hot, gate_w, up_w, gate_s, up_s, act, gu32, ctr_a, blocks, lo, sh_gw=0, sh_uw=0, xf=0):
    """phase 1 of forward: act of the routed experts (and the shared expert)"""
    on_device("moe4.gate_up", x, sel, rw, gate_w, up_w, gate_s, up_s, act, gu32, ctr_a)
    call("hmoe_moe4_gate_up", ptr(x), ptr(sel), ptr(rw), x.shape[0], int(n_hot), ptr(gate_w), ptr(up_w), ptr(gate_s),
         ptr(up_s), ptr(act), ptr(gu32), ptr(ctr_a), int(blocks), int(lo), _addr(sh_gw), _addr(sh_uw), xf_of(x, xf),
         stream_of(x.device))


def down(sel, rw, n_hot, down_w, down_s, act, y32, ctr_b, y, blocks, lo, sh_dw=0):
    """phase 2 of forward: y += down projections of act"""
    on_device("moe4.down", y, sel, rw, down_w, down_s, act, y32, ctr_b)
    call("hmoe_moe4_down", ptr(sel), ptr(rw), sel.shape[0], int(n_hot), ptr(down_w), ptr(down_s), ptr(act), ptr(y32),
         ptr(ctr_b), ptr(y), int(blocks), int(lo), _addr(sh_dw), stream_of(y.device))


def combine(f, o_ptr, y, rows, o2_ptr=0, done_ptr=0):
    """moe4.cu:817-824: f += y (+ o) (+ o2); y = 0"""
    on_device("moe4.combine", f, y)
    _req(f.is_contiguous() and f.shape[-1] == H and f.dtype == torch.float32, "f")
    call("hmoe_moe4_combine", ptr(f), _addr(o_ptr), ptr(y), int(rows), _addr(o2_ptr), _addr(done_ptr),
         stream_of(f.device))


def dequant(q, sc, N, K):
    """moe4.cu:904-911: I4G128 codes + scales -> f16 [N, K]"""
    on_device("moe4.dequant", q, sc)
    out = torch.empty((N, K), dtype=torch.float16, device=q.device)
    call("hmoe_moe4_dequant", ptr(q), ptr(sc), int(N), int(K), ptr(out), stream_of(q.device))
    return out


def finish_bf16(y, rows, out):
    """y fp32 [rows, H] -> bf16 out, y zeroed"""
    on_device("finish_bf16", y, out)
    call("hmoe_finish_bf16", ptr(y), int(rows), ptr(out), stream_of(y.device))
    return out


def forward_noalloc(x, sel, rw, n_hot, gate_w, up_w, down_w, gate_s, up_s, down_s, y, lo=0, sh_gw=0, sh_uw=0, sh_dw=0,
                    xf=0):
    """forward without workspace arguments (hmoe_moe4_forward_noalloc): the library's static per-device workspace, no
    allocation anywhere in the call; calls that overlap on one GPU race"""
    R = x.shape[0]
    on_device("moe4.forward_noalloc", x, sel, rw, gate_w, up_w, down_w, gate_s, up_s, down_s, y)
    fmt = xf_of(x, xf)
    _req(x.is_contiguous() and x.shape[-1] == H, "x layout")
    _req(sel.dtype == torch.int64 and sel.is_contiguous() and sel.shape == (R, TOPK), "selection int64 [R, 8]")
    _req(rw.dtype == torch.float16 and rw.is_contiguous() and rw.shape == (R, TOPK), "routing weights f16 [R, 8]")
    _req(y.dtype == torch.float32 and y.is_contiguous() and y.shape[-1] == H and y.numel() >= R * H, "y fp32 [R, H]")
    call("hmoe_moe4_forward_noalloc", ptr(x), ptr(sel), ptr(rw), R, int(n_hot), ptr(gate_w), ptr(up_w), ptr(down_w),
         ptr(gate_s), ptr(up_s), ptr(down_s), ptr(y), int(lo), _addr(sh_gw), _addr(sh_uw), _addr(sh_dw), fmt,
         stream_of(x.device))
