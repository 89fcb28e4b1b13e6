"""CPU tests of the product's host side: the C ABI loads and exports every declared symbol (no GPU call), the host
packers of the gfx950 layouts, the ingest of the reference's moe4 weights, the key derivation and the Zipf bias."""
import ctypes
import os
import re

import numpy as np
import pytest

import pyoracle as O
from hecate_amd import _lib, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "hecate_moe.h")).read()
    return sorted(set(re.findall(r"^(?:int|size_t|const char\*)\s+(hmoe_\w+)\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert set(syms) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"
    assert _lib.lib().hmoe_version() == 1


def test_error_path_sets_message():
    L = _lib.lib()
    rc = L.hmoe_pack_i4(None, None, 16, 128, None, None)
    assert rc == 1 and b"null" in L.hmoe_last_error()
    with pytest.raises(RuntimeError, match="shape"):
        buf = np.zeros(64, np.uint8)
        _lib.call("hmoe_pack_i4", buf.ctypes.data, buf.ctypes.data, 15, 128, buf.ctypes.data, buf.ctypes.data)


def test_host_tensors_are_refused():
    """the Python operators refuse host tensors before any call into the library"""
    import torch
    from hecate_amd import moe4, router
    x = torch.zeros(1, 6144, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="device"):
        router.router_fused(x, torch.zeros(256, 6144), torch.zeros(256), torch.zeros(1), torch.zeros(1),
                            torch.zeros(1, 8, dtype=torch.int64), torch.zeros(1, 8, dtype=torch.float16), 8, 2.5)
    with pytest.raises(RuntimeError, match="device"):
        moe4.finish_bf16(torch.zeros(1, 6144), 1, x)


def test_empty_prefill_chunk_is_a_no_op():
    """no tokens and no picks: the prefill entry returns before any check of its buffers and before any GPU call
    (moe4p.cu:229 returns when no pick reaches the tier); tokens without buffers are still refused"""
    L = _lib.lib()
    args = [None] * 5 + [0, 0, 0] + [None] * 10 + [0, None, None, 0, 8, None, None, None, 0, None]
    assert L.hmoe_moe4p_forward(*args) == 0
    args[21] = 3
    assert L.hmoe_moe4p_forward(*args) != 0 and b"null" in L.hmoe_last_error()


def test_prefill_bf16_output_entry_checks():
    """hmoe_moe4p_forward_bf16 (the combine writing the bf16 output): an empty chunk is a no-op, and it refuses a
    chunk without the inverse map (the per-token combine it needs) before any GPU call (the buffer addresses below
    are never dereferenced)"""
    L = _lib.lib()
    args = [None] * 5 + [0, 0, 0] + [None] * 9 + [0, None, None, 0, 8, None, None, None, 0, None, None]
    assert L.hmoe_moe4p_forward_bf16(*args) == 0
    args[20] = 3
    assert L.hmoe_moe4p_forward_bf16(*args) != 0 and b"null" in L.hmoe_last_error()
    fake = 1 << 20
    for i in (0, 1, 3, 4, 15, 16, 26):                      # x, tok, wt, rbt, ar, d, out_bf16
        args[i] = fake
    assert L.hmoe_moe4p_forward_bf16(*args) != 0 and b"inverse map" in L.hmoe_last_error()
    # the long-prefill form: the inverse map and the partial are required (checked before any GPU call)
    targs = [None] * 5 + [0, 0, 0] + [None] * 10 + [0, None, 3, 0, None, 8, None, None]
    assert L.hmoe_moe4t_forward_bf16(*targs) != 0 and b"inverse map" in L.hmoe_last_error()


@pytest.mark.parametrize("N,K", [(16, 512), (64, 1536), (2048, 6144)])
def test_pack_unpack_round_trip_and_layout(N, K):
    rng = np.random.default_rng(N)
    codes = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    scales = rng.integers(0, 65536, (N, K // 128), dtype=np.uint16)
    q = np.empty(N * K // 2, np.uint8); s = np.empty(N * K // 128, np.uint16)
    _lib.call("hmoe_pack_i4", codes.ctypes.data, scales.ctypes.data, N, K, q.ctypes.data, s.ctypes.data)
    c2 = np.empty_like(codes); s2 = np.empty_like(scales)
    _lib.call("hmoe_unpack_i4", q.ctypes.data, s.ctypes.data, N, K, c2.ctypes.data, s2.ctypes.data)
    assert np.array_equal(c2, codes) and np.array_equal(s2, scales)
    # layout: lane l of tile (nb, kg), dword j, element e holds (row nb*16 + l%16, k = kg*128 + 32j + 8(l/16) + e)
    # at bit 4(e/2) + 16(e%2); scales in 128-byte blocks of 16 rows x 4 groups (row-major inside a block)
    w = q.view(np.uint32).reshape(N // 16, K // 128, 64, 4)
    full = np.stack([codes & 15, codes >> 4], -1).reshape(N, K)
    for nb, kg, l, j, e in [(0, 0, 0, 0, 0), (0, 0, 17, 2, 5), (N // 16 - 1, K // 128 - 1, 63, 3, 7), (0, 0, 35, 1, 1)]:
        row, k = nb * 16 + l % 16, kg * 128 + 32 * j + 8 * (l // 16) + e
        assert (w[nb, kg, l, j] >> (4 * (e // 2) + 16 * (e % 2))) & 15 == full[row, k]
    KG = K // 128
    blocks = s.reshape(N // 16, KG // 4, 16, 4)
    assert np.array_equal(blocks.transpose(0, 2, 1, 3).reshape(N, KG), scales)
    for n, g in [(0, 0), (5, 3), (N - 1, KG - 1), (min(17, N - 1), KG // 2)]:
        assert s[((n // 16) * (KG // 4) + g // 4) * 64 + (n % 16) * 4 + g % 4] == scales[n, g]


def test_pack_dense_is_f16_tiles():
    rng = np.random.default_rng(2)
    N, K = 32, 64
    w = O.f32_to_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    out = np.empty(N * K, np.uint16)
    _lib.call("hmoe_pack_dense", w.ctypes.data, N, K, out.ctypes.data)
    t = out.reshape(N // 16, K // 32, 64, 8)
    f16 = O.bf16_to_f32(w).astype(np.float16).view(np.uint16)
    for nb, ks, l, e in [(0, 0, 0, 0), (1, 1, 63, 7), (0, 1, 20, 3)]:
        assert t[nb, ks, l, e] == f16[nb * 16 + l % 16, ks * 32 + 8 * (l // 16) + e]


def test_f16t_rows_inverts_pack_dense():
    """tier.f16t_rows (the prefill's row-major copy of an F16T matrix) undoes hmoe_pack_dense element for element:
    the result is the bf16 matrix's exact f16 values in row-major order"""
    import torch
    from hecate_amd import tier
    rng = np.random.default_rng(5)
    N, K = 48, 96
    w = O.f32_to_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    out = np.empty(N * K, np.uint16)
    _lib.call("hmoe_pack_dense", w.ctypes.data, N, K, out.ctypes.data)
    rows = tier.f16t_rows(torch.from_numpy(out.view(np.int16)), N, K)
    assert rows.shape == (N, K) and rows.dtype == torch.float16 and rows.is_contiguous()
    f16 = O.bf16_to_f32(w).astype(np.float16).view(np.uint16)
    assert np.array_equal(rows.view(torch.int16).numpy().view(np.uint16), f16)


def test_repack_reference_moe4_weights():
    """tools/quant/gptq_int4.py:74-77 pack_u4 (the reference's fragment order, restated as a permutation of the
    code tensor) + fp32 row scales -> this build's I4G128: same codes, scale = bf16(row scale) in every group"""
    rng = np.random.default_rng(3)
    N, K = 128, 512
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    frag = _pack_u4_reference_order(codes)
    rs = (rng.random(N) * 0.01).astype(np.float32)
    q = np.empty(N * K // 2, np.uint8); s = np.empty(N * K // 128, np.uint16)
    _lib.call("hmoe_repack_moe4", frag.ctypes.data, rs.ctypes.data, N, K, q.ctypes.data, s.ctypes.data)
    c2 = np.empty((N, K // 2), np.uint8); s2 = np.empty((N, K // 128), np.uint16)
    _lib.call("hmoe_unpack_i4", q.ctypes.data, s.ctypes.data, N, K, c2.ctypes.data, s2.ctypes.data)
    assert np.array_equal(np.stack([c2 & 15, c2 >> 4], -1).reshape(N, K), codes)
    assert np.array_equal(s2, np.repeat(O.f32_to_bf16(rs)[:, None], K // 128, 1))


def test_key_derivation_matches_the_shared_header():
    for args in [(0, 0, 0, 0), (synth.SEED, 3, 5, 255), (2 ** 63 + 5, 15, 14, 1)]:
        assert synth.key(*args) == O.key(*args)


def test_zipf_tau_is_the_calibrated_one():
    assert abs(synth.calibrate_zipf_tau(rows=8000) - synth.ZIPF_TAU) < 0.003
    b = synth.zipf_bias()
    order = synth.popularity_order()
    assert np.all(np.diff(b[np.array(order)]) < 0) and sorted(order) == list(range(256))


def _pack_u4_reference_order(codes):
    """tools/quant/gptq_int4.py:74-77 pack_u4, restated as a permutation of the code tensor [N, K] (N % 64 == 0,
    K % 64 == 0): the bytes the reference writes to its int4 safetensors"""
    N, K = codes.shape
    c = codes.reshape(N // 64, 4, 2, 8, K // 64, 4, 2, 4, 2).transpose(0, 4, 1, 3, 7, 5, 8, 6, 2).reshape(-1, 2)
    return (c[:, 0] | (c[:, 1] << 4)).astype(np.uint8)


def test_load_reference_int4_files(tmp_path):
    """the reference's on-disk layout (hot file + r229 file, keys {e}.{m}.{q,s}, tier_split.py:207-214) read into an
    ExpertBank in placement order: every matrix's codes exact, group scales = bf16(row scale)"""
    from safetensors.numpy import save_file
    from hecate_amd import tier
    rng = np.random.default_rng(11)
    H, I = 6144, 2048
    want = {}
    hot, cold = {}, {}
    for e, dst in ((7, hot), (3, cold)):
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
            rs = (rng.random(N) * 0.01 + 1e-3).astype(np.float32)
            dst[f"{e}.{m}.q"] = _pack_u4_reference_order(codes)
            dst[f"{e}.{m}.s"] = rs
            want[(e, m)] = (codes, rs)
    save_file(hot, str(tmp_path / "layer5.safetensors"))
    save_file(cold, str(tmp_path / "layer5.r229.safetensors"))
    bank = tier.load_reference_int4(str(tmp_path), 5, [3, 7], "cpu")
    for j, e in enumerate([3, 7]):
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            codes, rs = want[(e, m)]
            q = bank.view(f"{m}_q", j).numpy().copy()
            s = bank.view(f"{m}_s", j).numpy().copy().view(np.uint16)
            c2 = np.empty((N, K // 2), np.uint8); s2 = np.empty((N, K // 128), np.uint16)
            _lib.call("hmoe_unpack_i4", q.ctypes.data, s.ctypes.data, N, K, c2.ctypes.data, s2.ctypes.data)
            assert np.array_equal(np.stack([c2 & 15, c2 >> 4], -1).reshape(N, K), codes), (e, m)
            assert np.array_equal(s2, np.repeat(O.f32_to_bf16(rs)[:, None], K // 128, 1)), (e, m)
    with pytest.raises(RuntimeError):
        tier.load_reference_int4(str(tmp_path), 5, [4], "cpu")


# ---- boundary: argument meanings the reference gives and this build cannot honour are refused, not misread ----------

def _fake(n=1 << 16):
    """a host buffer whose address stands in for every pointer argument (never dereferenced: the calls below are
    refused by their argument checks before any launch)"""
    return np.zeros(n, np.uint8)


def test_fragment_order_x_is_refused():
    """xf = 1 means x in B-fragment order in the reference (moe4.cu:826); the C ABI refuses it instead of reading it
    as row-major, and the Python mirror does the same; an fp16 tensor with xf = 0 (the reference's call) is fp16"""
    import torch
    from hecate_amd import moe4
    L = _lib.lib()
    b = _fake()
    p = b.ctypes.data
    common = [p, p, p, 1, 8, p, p, p, p, p, p, p, p, p, p, p, p, 0, 0, 0, None, None, None, None, None, None]
    assert L.hmoe_moe4_forward(*common, _lib.XF_FRAG, None) == 1
    assert b"fragment-order" in L.hmoe_last_error()
    assert L.hmoe_moe4_gate_up(p, p, p, 1, 8, p, p, p, p, p, p, p, 0, 0, None, None, _lib.XF_FRAG, None) == 1
    assert b"fragment-order" in L.hmoe_last_error()
    pf = [p, p, p, p, p, 8, 1, 8] + [p] * 10 + [8, None, None, 1, 8, None, None, None]
    assert L.hmoe_moe4p_forward(*pf, _lib.XF_FRAG, None) == 1 and b"fragment-order" in L.hmoe_last_error()
    assert L.hmoe_moe4t_forward(p, p, p, p, p, 8, 1, 8, *([p] * 10), 8, None, 1, _lib.XF_FRAG, None, 8, None) == 1
    assert L.hmoe_moe4_forward(*common, 3, None) == 1                       # unknown flags too
    x16 = torch.zeros(1, 6144, dtype=torch.float16)
    assert _lib.xf_of(x16, 0) == _lib.XF_F16 and _lib.xf_of(x16.bfloat16(), 0) == _lib.XF_BF16
    with pytest.raises(RuntimeError, match="fragment"):
        _lib.xf_of(x16, 1)
    with pytest.raises(RuntimeError, match="bf16 or fp16"):
        _lib.xf_of(x16.float(), 0)
    with pytest.raises(RuntimeError, match="device"):
        moe4.forward(x16, *([torch.zeros(1, 8, dtype=torch.int64)] * 2), 8, *([torch.zeros(8, dtype=torch.int64)] * 6),
                     *([torch.zeros(1)] * 5), torch.zeros(1, 6144), 0, 0, 0)


def test_router_scratch_is_the_reference_buffer_up_to_8_rows():
    """exl3_router.py:180 allocates logits fp32 [8, 256] for 2..8 rows: that buffer is large enough here too"""
    L = _lib.lib()
    ref_bytes = 8 * 256 * 4
    for R in range(1, 9):
        assert L.hmoe_router_scratch_bytes(R, 256) <= ref_bytes
    assert L.hmoe_router_scratch_bytes(16, 256) == 16 * 256 * 4
    assert L.hmoe_router_scratch_bytes(17, 256) == 8 * 17 * 256 * 4          # the large path's segment planes


def test_dispatch_block_size_is_bounded():
    """row blocks of up to 256 picks (the reference's moe4t bm) are accepted; larger ones are refused, because the
    grouped GEMMs run a block as at most two 128-pick halves"""
    L = _lib.lib()
    b = _fake()
    p = b.ctypes.data
    args = lambda bm: (p, p, 4, 8, 0, 256, bm, 1, p, p, p, p, p, p, 64, p, p, None)
    assert L.hmoe_dispatch(*args(257)) == 1 and b"bm 257" in L.hmoe_last_error()
    assert L.hmoe_dispatch(*args(0)) == 1
    assert L.hmoe_dispatch_nrb_max(8 * 8192, 256, 256) == 256 + 8 * 8192 // 256


def test_moe4t_no_picks_is_a_no_op():
    """moe4t.cu:508 returns when no pick reaches the tier: npos = 0 returns before any check or launch"""
    L = _lib.lib()
    assert L.hmoe_moe4t_forward(*([None] * 5), 0, 0, 0, *([None] * 10), 0, None, 0, 0, None, 8, None) == 0
    assert L.hmoe_moe4t_scratch_bytes(1, 100) == 100 * 2048 * 2
    assert L.hmoe_moe4t_scratch_bytes(2, 100) == 100 * 6144 * 4
    assert L.hmoe_shared_forward(None, 0, None, None, None, None, None, 0, None) == 0


def test_prefill_chunks_past_the_32_bit_offsets_are_refused():
    """the grouped GEMMs address their input rows by 32-bit byte offsets: a chunk whose f16 x (T x 6144) or act rows
    ((ps + T) x 2048) pass 4 GB is refused before any launch, here and through moe4t and the test entry"""
    L = _lib.lib()
    b = _fake()
    p = b.ctypes.data
    big = 400_000                                                           # 400,000 x 6144 x 2 B > 4 GB
    pf = lambda T, ps: [p, p, p, p, p, 8, 1, 8] + [p] * 10 + [ps, None, None, T, 8, None, None, None, _lib.XF_BF16, None]
    assert L.hmoe_moe4p_forward(*pf(big, 8)) == 1 and b"4 GB" in L.hmoe_last_error()
    assert L.hmoe_moe4p_forward(*pf(8, 1_100_000)) == 1 and b"4 GB" in L.hmoe_last_error()
    assert L.hmoe_moe4t_forward(p, p, p, p, p, 8, 1, 8, *([p] * 10), 8, None, big, _lib.XF_BF16, None, 8, None) == 1
    assert b"4 GB" in L.hmoe_last_error()
    assert L.hmoe_moe4t_gemm(p, big, p, 1, 8, p, p, p, p, p, big, 0, None) == 1 and b"4 GB" in L.hmoe_last_error()
    # the shared expert's dense GEMMs (the long prefill runs them before moe4t's own check)
    assert L.hmoe_shared_forward(p, big, p, p, p, p, p, _lib.XF_BF16, None) == 1 and b"4 GB" in L.hmoe_last_error()


def test_norm_entries_refuse_bad_arguments():
    """combine_norm / norm_route / decode_combine_norm check their arguments before any GPU call: the RTX band's DONE
    flag, the band hand-off words, dtype codes, row counts and alignment are refused with a message (a fake device
    address is never dereferenced: every case fails a check first)"""
    L = _lib.lib()
    A = 1 << 20                                             # an aligned stand-in address (never read)
    F32, BF16, F16 = 0, 1, 2
    # combine_norm(f, o, y, rows, o2, done, r, w, xn, eps, cbias, cscale, w_dtype, xn_dtype, stream)
    assert L.hmoe_combine_norm(A, None, A, 2, None, A, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"DONE" in L.hmoe_last_error()
    assert L.hmoe_combine_norm(A, None, None, 2, None, None, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert L.hmoe_combine_norm(A, None, A, 65, None, None, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"rows" in L.hmoe_last_error()
    assert L.hmoe_combine_norm(A, None, A, 2, None, None, A, A, A, 1e-5, 0.0, 1.0, 7, F16, None) != 0
    assert b"dtype" in L.hmoe_last_error()
    assert L.hmoe_combine_norm(A, None, A, 2, None, None, A, A, A, 1e-5, 0.0, 1.0, F16, F32, None) != 0
    assert L.hmoe_combine_norm(A + 4, None, A, 2, None, None, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"alignment" in L.hmoe_last_error()
    # norm_route(y, r, w, x2, gt, bias, sel, rw, cand, ctr, scale, eps, cbias, cscale, ho, n_ho, R, E, wdt, xdt, gdt, st)
    ho = (ctypes.c_int64 * 10)(*range(10))
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, ho, 10, 4, 256, F16, F16, F16,
                             None) != 0
    assert b"hand-off" in L.hmoe_last_error()
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, None, 0, 17, 256, F16, F16, F16,
                             None) != 0
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, None, 0, 4, 257, F16, F16, F16,
                             None) != 0
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, None, 0, 4, 256, F16, F16, BF16,
                             None) != 0
    assert b"gate dtype" in L.hmoe_last_error()
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, None, A, 2.5, 1e-5, 0.0, 1.0, None, 0, 4, 256, F16, F16, F16,
                             None) != 0
    assert L.hmoe_norm_route_scratch_bytes(8, 256) == 8 * 256 * 4
    # the CPU tier's hand-off {mailbox, layer}: bf16 x2, at most 8 rows, a mailbox, 16-byte aligned sel / rw
    ho2 = (ctypes.c_int64 * 2)(A, 3)
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, ho2, 2, 4, 256, F16, F16, F16,
                             None) != 0
    assert b"bf16" in L.hmoe_last_error()
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, ho2, 2, 9, 256, F16, BF16, F16,
                             None) != 0
    assert L.hmoe_norm_route(A, A, A, A, A, None, A + 8, A, A, A, 2.5, 1e-5, 0.0, 1.0, ho2, 2, 4, 256, F16, BF16, F16,
                             None) != 0
    assert b"aligned" in L.hmoe_last_error()
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, (ctypes.c_int64 * 2)(0, 3), 2, 4,
                             256, F16, BF16, F16, None) != 0
    assert b"mailbox" in L.hmoe_last_error()
    assert L.hmoe_norm_route(A, A, A, A, A, None, A, A, A, A, 2.5, 1e-5, 0.0, 1.0, None, 2, 4, 256, F16, BF16, F16,
                             None) != 0
    # combine_norm_cpu(f, o, y, rows, mb, r, w, xn, eps, cbias, cscale, wdt, xdt, st)
    assert L.hmoe_combine_norm_cpu(None, None, A, 9, A, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"rows" in L.hmoe_last_error()
    assert L.hmoe_combine_norm_cpu(None, None, A, 4, None, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"mailbox" in L.hmoe_last_error()
    assert L.hmoe_combine_norm_cpu(None, None, A + 4, 4, A, A, A, A, 1e-5, 0.0, 1.0, F16, F16, None) != 0
    assert b"alignment" in L.hmoe_last_error()
    # decode_combine_norm(y32, ctr, R, r, w, xn, xh, eps, cbias, cscale, wdt, xdt, st)
    assert L.hmoe_decode_combine_norm(None, A, 4, A, A, A, None, 1e-5, 0.0, 1.0, F32, BF16, None) != 0
    assert L.hmoe_decode_combine_norm(A, A, 17, A, A, A, None, 1e-5, 0.0, 1.0, F32, BF16, None) != 0


def test_norm_mirrors_check_before_calling():
    """the Python mirrors refuse host tensors and wrong dtypes before calling the library"""
    import torch
    from hecate_amd import cn, router
    y = torch.zeros(2, 6144)
    with pytest.raises(RuntimeError, match="device"):
        cn.combine_norm(y, 0, y, 2, 0, 0, y, torch.zeros(6144, dtype=torch.float16), torch.zeros(2, 6144,
                        dtype=torch.float16), 1e-5)
    with pytest.raises(RuntimeError, match="device"):
        router.norm_route(y, y, torch.zeros(6144), torch.zeros(2, 6144, dtype=torch.float16), torch.zeros(256, 6144),
                          None, torch.zeros(2, 8, dtype=torch.int64), torch.zeros(2, 8, dtype=torch.float16),
                          torch.zeros(2048), torch.zeros(64, dtype=torch.int32), 2.5, 1e-5)
    with pytest.raises(RuntimeError, match="device"):
        cn.combine_norm_cpu(None, 0, y, 2, 1 << 20, y, torch.zeros(6144, dtype=torch.float16),
                            torch.zeros(2, 6144, dtype=torch.float16), 1e-5)
    with pytest.raises(RuntimeError, match="dtype"):
        _lib.dt_of(torch.zeros(1, dtype=torch.int32))
    assert _lib.dt_of(torch.zeros(1, dtype=torch.float16)) == 2 and _lib.dt_of(torch.zeros(1)) == 0
