"""Reference-format ingest on the host: the placement file (tier_split.py:18,173-189, written by
tools/placement/tier_placement.py:15-18) and a layer built from it and the reference's int4 files as tier_split_load
does (router rows permuted to the placement order, the hot band resident, the far band on the host-CPU tier). The
far band's job is checked bit-exact against the oracle's q8_0 mode on the files' codes and row scales. No GPU."""
import json

import numpy as np
import pytest
import torch

import pyoracle as O
from hecate_amd import tier
from hecate_amd._lib import call
from hecate_amd.cpu_tier import CpuTier
from hostref import x_rows
from test_abi import _pack_u4_reference_order

H, I, E = 6144, 2048, 256


def _perm(seed):
    return [int(e) for e in np.random.default_rng(seed).permutation(E)]


def test_load_placement_forms_and_defaults(tmp_path):
    p3 = _perm(1)
    raw = {"3": {"perm": p3, "hot": 176, "far": 16, "first": 192},
           "7": {"perm": _perm(2), "hot": 200, "first": 200},                     # no "far": 0 (p.get)
           "78": {"perm": list(range(E)), "hot": 256, "first": 256}}              # the MTP layer: no third band
    f = tmp_path / "place.json"
    f.write_text(json.dumps(raw))
    for src in (raw, json.dumps(raw), str(f)):
        pl = tier.load_placement(src)
        assert sorted(pl) == [3, 7, 78]
        assert pl[3].perm == p3 and (pl[3].hot, pl[3].far, pl[3].first) == (176, 16, 192)
        assert (pl[7].hot, pl[7].far, pl[7].first) == (200, 0, 200)
        assert pl[78].first == 256


@pytest.mark.parametrize("bad, match", [
    ({"x": {"perm": list(range(E)), "hot": 1, "first": 1}}, "not an integer"),
    ({"1": {"hot": 1, "first": 1}}, "needs"),
    ({"1": {"perm": [0] * E, "hot": 1, "first": 1}}, "permutation"),
    ({"1": {"perm": list(range(E)), "hot": 200, "far": 60, "first": 256}}, "hot 200 far 60"),
    ({"1": {"perm": list(range(E))[::-1], "hot": 256, "first": 256}}, "third band"),
])
def test_load_placement_rejects(bad, match):
    with pytest.raises(ValueError, match=match):
        tier.load_placement(bad)


def write_reference_files(tmp_path, layer, experts, seed):
    """the reference's int4 files for `experts` (codes 0..15 = q + 8 in the moe4 fragment order, fp32 row scales,
    gptq_int4.py:205-212), split over layer{L}.safetensors and layer{L}.r*.safetensors; returns each expert's
    canonical row-major codes and bf16 group scales, made here from the generated codes (the oracle's input)"""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    files = [{}, {}]
    canon = {}
    for j, e in enumerate(experts):
        ex = {}
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
            rs = (rng.random(N) * 0.004 + 0.002).astype(np.float32)
            files[j % 2][f"{e}.{m}.q"] = _pack_u4_reference_order(codes)
            files[j % 2][f"{e}.{m}.s"] = rs
            ex[m + "_q"] = np.ascontiguousarray(codes[:, 0::2] | (codes[:, 1::2] << 4))
            ex[m + "_s"] = np.ascontiguousarray(np.repeat(O.f32_to_bf16(rs)[:, None], K // 128, 1))
        canon[e] = ex
    save_file(files[0], str(tmp_path / f"layer{layer}.safetensors"))
    if files[1]:
        save_file(files[1], str(tmp_path / f"layer{layer}.r229.safetensors"))
    return canon


def test_layer_from_reference_on_the_host(tmp_path):
    """placement hot 2 / far 1: router rows and bias in placement order, the hot experts' codes in the bank, and a
    job of the far expert on the CPU tier bit-exact against the oracle's q8_0 mode on the files' data"""
    L = 4
    perm = _perm(9)
    pl = tier.load_placement({str(L): {"perm": perm, "hot": 2, "far": 1, "first": 3}})
    canon = write_reference_files(tmp_path, L, perm[:3], 21)
    rng = np.random.default_rng(5)
    wg = torch.from_numpy((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = torch.from_numpy((rng.standard_normal(E) * 0.01).astype(np.float32))
    cpu = CpuTier(threads=2, mapped=False)
    try:
        lay = tier.layer_from_reference((L, pl[L]), str(tmp_path), wg, bias, "cpu", cpu=cpu)
        assert torch.equal(lay.wg, wg[perm]) and torch.equal(lay.bias, bias[perm])
        assert (lay.lo, lay.n_hot) == (0, 2)
        for j in range(2):
            c = np.empty((I, H // 2), np.uint8); s = np.empty((I, H // 128), np.uint16)
            q = lay.bank.view("up_q", j).numpy(); sc = lay.bank.view("up_s", j).numpy()
            call("hmoe_unpack_i4", q.ctypes.data, sc.ctypes.data, I, H, c.ctypes.data, s.ctypes.data)
            assert np.array_equal(c, canon[perm[j]]["up_q"]) and np.array_equal(s, canon[perm[j]]["up_s"])
        # the far band: local id 2 on the CPU tier (layer L, window [2, 3))
        R = 3
        x = x_rows(31, R)
        sel = np.array([[2, 0, 1, 9, 10, 11, 12, 13], [5, 6, 2, 7, 8, 9, 10, 11], [1, 3, 4, 5, 6, 7, 8, 9]], np.int64)
        rw = O.f32_to_f16((rng.random((R, 8)) * 0.5 + 0.05).astype(np.float32))
        cpu.post(x, sel, rw, L)
        out, err = cpu.wait()
        assert err == 0
        ref = O.moe(1, x, sel, rw, O.ExpertTable([canon[perm[2]]]), 2, 1, None, threads=4)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
        assert np.abs(out[2]).max() == 0 and np.abs(out[0]).max() > 0
    finally:
        cpu.close()


def test_layer_from_reference_refuses_other_bands(tmp_path):
    """a layer without an int4 hot band, or with a trellis band on the accelerator (first > hot + far), is not an
    int4 tier layer (tier_split.py:189 asserts first == hot + far)"""
    wg, bias = torch.zeros(E, H), torch.zeros(E)
    for p in ({"perm": list(range(E)), "hot": 0, "first": 40}, {"perm": _perm(3), "hot": 8, "far": 2, "first": 20}):
        pl = tier.load_placement({"2": p})
        with pytest.raises(ValueError, match="hot > 0 and first == hot"):
            tier.layer_from_reference((2, pl[2]), str(tmp_path), wg, bias, "cpu")
