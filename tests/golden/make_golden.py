"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no stored vectors (its tests draw unseeded randn on the
GPU and compare two implementations live), so these fixtures are minted here
from seeded Philox4x32-10 inputs: they pin the oracle against regressions
and give the GPU tests fixed inputs with known outputs.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), os.path.dirname(os.path.dirname(HERE))]

import oracle as O  # noqa: E402
from helpers import moe_inputs, router_inputs  # noqa: E402


def router_case(name, T, E, k, seed):
    g = router_inputs(T, E, seed)
    w, i, ei = O.topk_softmax(g, k)
    np.savez(os.path.join(HERE, name), kind="router", logits=g, k=k, topk_weight=w, topk_indices=i,
             token_expert_indices=ei)


def moe_case(name, T, H, I, E, k, dt, moe_type, act, seed, wstd):
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, seed, moe_type, wstd=wstd)
    kw = dict(E=E, k=k, act=act, moe_type=moe_type, dtype=dt)
    f32acc = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw)
    exact = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw)
    np.savez_compressed(os.path.join(HERE, name), kind="moe", x=x, gate=G, up=U,
             down=D if D is not None else np.zeros((0,), x.dtype), routing_weights=rw, expert_indices=ri, E=E, k=k,
             act=act, moe_type=moe_type, dtype=dt, out_f32acc=f32acc, out_exact=exact)


if __name__ == "__main__":
    # BASELINE config 1 and the reference's own router test shape
    router_case("router_32x8_k2.npz", 32, 8, 2, seed=1001)
    router_case("router_8x4_k2.npz", 8, 4, 2, seed=1002)
    router_case("router_64x128_k8.npz", 64, 128, 8, seed=1003)
    # small MoE layers, reference test style (I = 4H, E = 8)
    moe_case("moe_qwen3_bf16_T32_H64.npz", 32, 64, 256, 8, 2, O.BF16, O.QWEN3, O.SILU, 1004, 0.2)
    moe_case("moe_qwen3_f16_T4_H64_k2.npz", 4, 64, 256, 8, 2, O.F16, O.QWEN3, O.SILU, 1005, 0.2)
    moe_case("moe_nomic_f32_T16_H16.npz", 16, 16, 64, 8, 2, O.F32, O.NOMIC, O.SILU, 1006, 0.5)
    moe_case("moe_nomic_bf16_gelu_T24_H64.npz", 24, 64, 256, 8, 1, O.BF16, O.NOMIC, O.GELU, 1007, 0.2)
    print("fixtures written to", HERE)
