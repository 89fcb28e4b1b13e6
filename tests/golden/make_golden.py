"""Writes tests/golden/oracle_vectors.npz: small input / output vectors of the CPU oracle (router, dispatch,
pick_groups, expert layer in both modes, RMSNorm). The reference ships no golden vectors for this path, so these are
regression fixtures of the oracle, each first checked by tests/test_oracle.py's independent checks.

python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as O  # noqa: E402


def vectors():
    rng = np.random.default_rng(2026)
    v = {}
    # router: 4 rows, K 512, 32 experts
    v["r_x"] = O.f32_to_bf16(rng.standard_normal((4, 512)).astype(np.float32))
    v["r_w"] = (rng.standard_normal((32, 512)) * 0.02).astype(np.float32)
    v["r_b"] = (rng.standard_normal(32) * 0.01).astype(np.float32)
    v["r_logits"] = O.router_logits(v["r_x"], v["r_w"])
    v["r_sel"], v["r_rw"] = O.router_select(v["r_logits"], v["r_b"])
    # dispatch + row blocks: 64 tokens over 24 experts, window [4, 20)
    v["d_sel"] = np.stack([rng.choice(24, 8, replace=False) for _ in range(64)]).astype(np.int64)
    v["d_rw"] = O.f32_to_f16(rng.random((64, 8)).astype(np.float32))
    c, tok, eid, wt, inv = O.dispatch(v["d_sel"], v["d_rw"], 4, 16)
    v.update(d_counts=c, d_tok=tok, d_eid=eid, d_wt=wt, d_inv=inv)
    v["d_rbt64"] = O.pick_groups(c, 8, False)
    v["d_rbt_bal"] = O.pick_groups(c, 16, True)
    # expert layer: H 256, I 128, 6 experts, 3 rows, shared expert
    H, I = 256, 128
    for e in range(6):
        for m, (N, K) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            v[f"m_{e}_{m}_q"] = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
            v[f"m_{e}_{m}_s"] = O.f32_to_bf16(np.abs(rng.standard_normal((N, K // 128)) * 0.01).astype(np.float32))
    for m, (N, K) in (("g", (I, H)), ("u", (I, H)), ("d", (H, I))):
        v[f"m_sh_{m}"] = O.f32_to_bf16((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    v["m_x"] = O.f32_to_bf16(rng.standard_normal((3, H)).astype(np.float32))
    v["m_sel"] = np.array([[0, 2, 4, 9, 1, 7, 8, 11], [5, 4, 3, 2, 1, 0, 12, 13], [10, 3, 14, 15, 6, 1, 9, 2]], np.int64)
    v["m_rw"] = O.f32_to_f16(rng.random((3, 8)).astype(np.float32))
    tab, sh = table(v)
    v["m_out_exact"] = O.moe(0, v["m_x"], v["m_sel"], v["m_rw"], tab, 0, 6, sh, H=H, I=I, threads=2)
    v["m_out_q8"] = O.moe(1, v["m_x"], v["m_sel"], v["m_rw"], tab, 0, 6, sh, H=H, I=I, threads=2)
    # rmsnorm
    v["n_r"] = rng.standard_normal((2, 768)).astype(np.float32)
    v["n_a"] = rng.standard_normal((2, 768)).astype(np.float32)
    v["n_w"] = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    v["n_r_out"], v["n_xn"] = O.residual_rmsnorm(v["n_r"], v["n_a"], v["n_w"], 1e-5)
    return v


def table(v):
    ex = [{f"{m}_{t}": v[f"m_{e}_{m}_{t}"] for m in ("gate", "up", "down") for t in ("q", "s")} for e in range(6)]
    return O.ExpertTable(ex), (v["m_sh_g"], v["m_sh_u"], v["m_sh_d"])


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "oracle_vectors.npz"), **vectors())
    print("wrote", os.path.join(HERE, "oracle_vectors.npz"))
