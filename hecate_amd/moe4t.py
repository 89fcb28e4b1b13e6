"""Long-prefill MoE operator: the drop-in for the reference's `moe4t` extension (runtime/tier/moe4/moe4t.cu:476-531).

forward(x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out) keeps the reference's names and order: row
blocks of up to 256 picks (pick_groups(counts, npos, 256, True), tier_split.py:449,457), and the down GEMM adds its
rows into out[tok] itself (fp32 atomics, no combine launch). The trailing keywords (meta, npos, nrb) take the sizes
from the device dispatch plan so that nothing syncs with the host. gemm(xs, rbt, w0, w1, out, down) is the test entry;
it needs the group scales too (s0, s1), which the reference's per-row format applies later.
"""
import torch

from ._lib import call, lib, on_device, ptr, stream_of, xf_of

H, I = 6144, 2048


def scratch(dev, npos):
    """moe4t.cu:490-496: [gu fp32 [2, npos, I], ar f16 [npos, I], d fp32 [1, npos, H]] (gu is unused; d holds the f16
    copy of x when forward gets bf16 x)"""
    dev = torch.device(dev)
    return [torch.empty((2, npos, I), dtype=torch.float32, device=dev),
            torch.empty((npos, I), dtype=torch.float16, device=dev),
            torch.empty((1, npos, H), dtype=torch.float32, device=dev)]


def forward(x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out, meta=None, npos=None, nrb=None, inv=None,
            topk=8, out_bf16=None):
    """moe4t.cu:498-524: out[tok] += routed experts of the sorted picks; x fp16 (as the reference) or bf16 [T, H].
    inv (the dispatch's inverse map, this build's addition): each token adds its picks in top-k order (deterministic)
    instead of the down GEMM's atomic adds. out_bf16 (bf16 [T, H], with inv): the combine also rounds out to it and
    zeroes out, as forward followed by moe4.finish_bf16 (hmoe_moe4t_forward_bf16)"""
    on_device("moe4t", x, tok, eid, wt, rbt, gw, uw, dw, gs, us, ds, gu, ar, d, out, meta, inv)
    T = x.shape[0]
    if not (x.dim() == 2 and x.shape[1] == H and x.is_contiguous() and out.dtype == torch.float32
            and out.is_contiguous() and out.shape[-1] == H and out.numel() >= T * H and rbt.dim() == 2
            and rbt.shape[1] == 4 and rbt.dtype == torch.int32 and tok.dtype == torch.int32
            and wt.dtype == torch.float32):
        raise RuntimeError("moe4t: shapes")
    npos = tok.numel() if npos is None else int(npos)
    nrb = rbt.shape[0] if nrb is None else int(nrb)
    ps = ar.shape[0]
    # d: the reference's fp32 [1, ps, H] (moe4t.scratch) or an f16 [ps, H] buffer: the kernels write f16 rows into it
    # (the copy of bf16 x, then with inv each pick's down row), ps * H * 2 bytes
    if npos > ps or ar.shape[1] != I or ar.dtype != torch.float16 or d.dtype not in (torch.float32, torch.float16) \
            or d.numel() * d.element_size() < ps * H * 2 or not d.is_contiguous():
        raise RuntimeError(f"moe4t: scratch for {ps} picks, {npos} given")
    if out_bf16 is not None:
        if inv is None or out_bf16.dtype != torch.bfloat16 or not out_bf16.is_contiguous() \
                or tuple(out_bf16.shape) != (T, H):
            raise RuntimeError("moe4t: out_bf16 (bf16 [T, H]) needs the inverse map")
        on_device("moe4t", out_bf16)
        call("hmoe_moe4t_forward_bf16", ptr(x), ptr(tok), ptr(eid), ptr(wt), ptr(rbt), npos, nrb, gw.numel(), ptr(gw),
             ptr(uw), ptr(dw), ptr(gs), ptr(us), ptr(ds), ptr(gu), ptr(ar), ptr(d), ptr(out), ps, ptr(meta), T,
             xf_of(x), ptr(inv), int(topk), ptr(out_bf16), stream_of(x.device))
        return
    call("hmoe_moe4t_forward", ptr(x), ptr(tok), ptr(eid), ptr(wt), ptr(rbt), npos, nrb, gw.numel(), ptr(gw),
         ptr(uw), ptr(dw), ptr(gs), ptr(us), ptr(ds), ptr(gu), ptr(ar), ptr(d), ptr(out), ps, ptr(meta), T, xf_of(x),
         ptr(inv), int(topk), stream_of(x.device))


def gemm(xs, rbt, w0, w1, out, down, s0=None, s1=None):
    """moe4t.cu:476-488: one grouped GEMM over the picks' inputs xs f16 [rows, K]: out [2, ps, I] (gate and up sums,
    down = 0) or [1, ps, H] (down = 1), the group scales included"""
    on_device("moe4t.gemm", xs, rbt, w0, w1, out, s0, s1)
    if s0 is None or (not down and s1 is None):
        raise RuntimeError("moe4t.gemm: the group-128 scale tables are needed (s0, and s1 for gate/up)")
    K, N, mats = (I, H, 1) if down else (H, I, 2)
    if not (xs.dtype == torch.float16 and xs.is_contiguous() and xs.dim() == 2 and xs.shape[1] == K
            and out.dtype == torch.float32 and out.is_contiguous() and out.dim() == 3 and out.shape[0] == mats
            and out.shape[2] == N and out.shape[1] >= xs.shape[0] and rbt.dtype == torch.int32):
        raise RuntimeError("moe4t.gemm: shapes")
    call("hmoe_moe4t_gemm", ptr(xs), xs.shape[0], ptr(rbt), rbt.shape[0], w0.numel(), ptr(w0),
         ptr(w1) if not down else None, ptr(s0), ptr(s1) if not down else None, ptr(out), out.shape[1], int(bool(down)),
         stream_of(xs.device))
    return out


def shared(x, sh_gw, sh_uw, sh_dw, work, out):
    """the shared expert alone over a chunk (hmoe_shared_forward): out fp32 [T, H] += its SwiGLU MLP of x"""
    on_device("shared", x, sh_gw, sh_uw, sh_dw, work, out)
    T = x.shape[0]
    if work.numel() * work.element_size() < int(lib().hmoe_shared_work_bytes(T)):
        raise RuntimeError("shared: work too small")
    if not all(w.dtype == torch.float16 and w.is_contiguous() and w.numel() == I * H for w in (sh_gw, sh_uw, sh_dw)):
        raise RuntimeError("shared: weights are row-major f16 gate [I, H], up [I, H], down [H, I]")
    call("hmoe_shared_forward", ptr(x), T, ptr(sh_gw), ptr(sh_uw), ptr(sh_dw), ptr(work), ptr(out), xf_of(x),
         stream_of(x.device))
