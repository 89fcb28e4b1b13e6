"""ctypes binding of libhecate_moe.so (include/hecate_moe.h). The product path has no fallback: if the library is
missing or a call fails, a RuntimeError names it."""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhecate_moe.so")
_L = None

P, i32, i64, u64, f32, sz = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                             ctypes.c_size_t)

SIGNATURES = {
    "hmoe_last_error": (ctypes.c_char_p, []),
    "hmoe_version": (i32, []),
    "hmoe_pack_i4": (i32, [P, P, i32, i32, P, P]),
    "hmoe_unpack_i4": (i32, [P, P, i32, i32, P, P]),
    "hmoe_pack_dense": (i32, [P, i32, i32, P]),
    "hmoe_repack_moe4": (i32, [P, P, i32, i32, P, P]),
    "hmoe_gen_i4": (i32, [u64, u64, f32, i32, i32, P, P, P]),
    "hmoe_gen_dense": (i32, [u64, f32, i32, i32, P, P]),
    "hmoe_gen_normal": (i32, [u64, i64, f32, f32, i32, P, P]),
    "hmoe_router_scratch_bytes": (sz, [i32, i32]),
    "hmoe_router_fused": (i32, [P, P, P, P, P, P, P, i32, i32, i32, i32, f32, P, P]),
    "hmoe_moe4_scratch_bytes": (sz, [i32]),
    "hmoe_moe4_forward": (i32, [P, P, P, i32, i32, P, P, P, P, P, P, P, P, P, P, P, P, i32, i32, i32,
                                P, P, P, P, P, P, i32, P]),
    "hmoe_moe4_noalloc_bytes": (sz, []),
    "hmoe_moe4_forward_noalloc": (i32, [P, P, P, i32, i32, P, P, P, P, P, P, P, i32, P, P, P, i32, P]),
    "hmoe_moe4_gate_up": (i32, [P, P, P, i32, i32, P, P, P, P, P, P, P, i32, i32, P, P, i32, P]),
    "hmoe_moe4_down": (i32, [P, P, i32, i32, P, P, P, P, P, P, i32, i32, P, P]),
    "hmoe_moe_decode_layer": (i32, [P, P, P, i32, i32, f32, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, P, P,
                                    P, P, P, P, i32, i32, P]),
    "hmoe_moe4_combine": (i32, [P, P, P, i32, P, P, P]),
    "hmoe_moe4_dequant": (i32, [P, P, i32, i32, P, P]),
    "hmoe_finish_bf16": (i32, [P, i32, P, P]),
    "hmoe_dispatch_work_bytes": (sz, [i32, i32, i32]),
    "hmoe_dispatch_nrb_max": (i32, [i32, i32, i32]),
    "hmoe_dispatch": (i32, [P, P, i32, i32, i32, i32, i32, i32, P, P, P, P, P, P, i32, P, P, P]),
    "hmoe_moe4p_scratch_bytes": (sz, [i32, i32, i32]),
    "hmoe_moe4p_forward": (i32, [P, P, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, P, i32, P, P, i32, i32,
                                 P, P, P, i32, P]),
    "hmoe_moe4p_forward_bf16": (i32, [P, P, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, i32, P, P, i32, i32,
                                      P, P, P, i32, P, P]),
    "hmoe_shared_work_bytes": (sz, [i32]),
    "hmoe_shared_forward": (i32, [P, i32, P, P, P, P, P, i32, P]),
    "hmoe_moe4t_scratch_bytes": (sz, [i32, i32]),
    "hmoe_moe4t_forward": (i32, [P, P, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, P, i32, P, i32, i32, P, i32,
                                 P]),
    "hmoe_moe4t_forward_bf16": (i32, [P, P, P, P, P, i32, i32, i32, P, P, P, P, P, P, P, P, P, P, i32, P, i32, i32, P,
                                      i32, P, P]),
    "hmoe_moe4t_gemm": (i32, [P, i32, P, i32, i32, P, P, P, P, P, i32, i32, P]),
    "hmoe_residual_rmsnorm": (i32, [P, P, P, i32, f32, P, P, P]),
    "hmoe_combine_norm": (i32, [P, P, P, i32, P, P, P, P, P, f32, f32, f32, i32, i32, P]),
    "hmoe_norm_route_scratch_bytes": (sz, [i32, i32]),
    "hmoe_norm_route": (i32, [P, P, P, P, P, P, P, P, P, P, f32, f32, f32, f32, P, i32, i32, i32, i32, i32, i32, P]),
    "hmoe_decode_combine_norm": (i32, [P, P, i32, P, P, P, P, f32, f32, f32, i32, i32, P]),
    "hmoe_norm_router": (i32, [P, P, f32, i32, P, i32, P, P, P, P]),
    "hmoe_cpu_start": (i32, [P, i32, i32]),
    "hmoe_cpu_add_layer": (i32, [i32, i32, i32, P, P]),
    "hmoe_cpu_stats": (i32, [P, P]),
    "hmoe_cpu_stop": (i32, []),
    "hmoe_cpu_submit": (i32, [P, P, P, P, i32, i32, P]),
    "hmoe_cpu_collect": (i32, [P, P, i32, P]),
    "hmoe_combine_norm_cpu": (i32, [P, P, P, i32, P, P, P, P, f32, f32, f32, i32, i32, P]),
    "hmoe_cpu_mailbox_alloc": (i32, [P]),
    "hmoe_cpu_mailbox_free": (i32, [P]),
}


def lib():
    """the loaded library (raises if it has not been built: python -m hecate_amd.build_lib)"""
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"hecate_amd: {LIB_PATH} is missing; build it with python -m hecate_amd.build_lib")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _L = L
    return _L


def check(rc, what=""):
    if rc != 0:
        msg = lib().hmoe_last_error().decode(errors="replace")
        raise RuntimeError(f"hecate_amd {what}: {msg} (status {rc})")


def call(name, *args):
    check(getattr(lib(), name)(*args), name)


def ptr(t):
    """device (or host) address of a torch tensor / numpy array / int, None for 0"""
    if t is None:
        return None
    if isinstance(t, int):
        return t or None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def on_device(what, x, *ts):
    """raise unless x is a CUDA tensor and every other tensor given (None skipped) is on x's device: a host pointer
    handed to a kernel faults the GPU instead of raising"""
    dev = getattr(x, "device", None)
    if dev is None or dev.type != "cuda":
        raise RuntimeError(f"{what}: x must be a device tensor")
    for t in ts:
        if t is not None and not isinstance(t, int) and getattr(t, "device", None) != dev:
            raise RuntimeError(f"{what}: every tensor must be on the device {dev}")


XF_BF16, XF_FRAG, XF_F16 = 0, 1, 2      # the x format flags of include/hecate_moe.h


def xf_of(x, xf=0):
    """the C ABI's x format flag for a torch tensor passed with the reference's xf: xf = 0 means row-major x, read as
    bf16 or fp16 by its dtype; xf = 1 (the reference's fragment-order x) is refused as the C ABI refuses it"""
    import torch
    if xf == XF_FRAG:
        raise RuntimeError("xf=1 (the reference's B-fragment-order x) is not supported: pass row-major x")
    if x.dtype == torch.bfloat16:
        return XF_BF16
    if x.dtype == torch.float16:
        return XF_F16
    raise RuntimeError(f"x must be bf16 or fp16, not {x.dtype}")


def stream_of(device=None):
    import torch
    return torch.cuda.current_stream(device).cuda_stream


DT_F32, DT_BF16, DT_F16 = 0, 1, 2       # the dtype codes of include/hecate_moe.h (HMOE_DT_*)


def dt_of(t, allowed=("float32", "bfloat16", "float16")):
    """the C ABI's dtype code of a torch tensor (RuntimeError for a dtype the entry does not take)"""
    name = str(t.dtype).replace("torch.", "")
    if name not in allowed:
        raise RuntimeError(f"dtype {t.dtype} not supported here ({', '.join(allowed)})")
    return {"float32": DT_F32, "bfloat16": DT_BF16, "float16": DT_F16}[name]
