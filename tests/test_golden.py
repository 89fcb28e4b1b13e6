"""The oracle reproduces its committed fixtures (tests/golden/oracle_vectors.npz, written by make_golden.py) bit for
bit: a regression net under the independent checks of test_oracle.py."""
import os
import sys

import numpy as np

import pyoracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402


def test_oracle_reproduces_fixtures():
    ref = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    now = make_golden.vectors()
    assert set(ref.files) == set(now)
    for k in ref.files:
        a, b = ref[k], now[k]
        assert a.dtype == b.dtype and a.shape == b.shape, k
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), k


def test_fixture_layer_against_fp64():
    v = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    H, I = 256, 128
    xf = O.bf16_to_f32(v["m_x"]).astype(np.float64)
    silu = lambda g: g / (1 + np.exp(-g))
    out = np.zeros((3, H))
    for r in range(3):
        for k in range(8):
            e = int(v["m_sel"][r, k])
            if e < 6:
                w = float(O.f16_to_f32(v["m_rw"][r, k:k + 1])[0])
                dq = lambda m, N, K: O.dequant(v[f"m_{e}_{m}_q"], v[f"m_{e}_{m}_s"], N, K).astype(np.float64)
                out[r] += dq("down", H, I) @ (silu(dq("gate", I, H) @ xf[r]) * (dq("up", I, H) @ xf[r]) * w)
        g = O.bf16_to_f32(v["m_sh_g"]).astype(np.float64) @ xf[r]
        u = O.bf16_to_f32(v["m_sh_u"]).astype(np.float64) @ xf[r]
        out[r] += O.bf16_to_f32(v["m_sh_d"]).astype(np.float64) @ (silu(g) * u)
    assert np.max(np.abs(v["m_out_exact"] - out)) < 1e-6 * np.abs(out).max()
    assert np.abs(v["m_out_q8"] - out).mean() / np.abs(out).mean() < 0.03
