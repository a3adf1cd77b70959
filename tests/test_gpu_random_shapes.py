"""Seeded random shapes through the default paths of fused_moe (f16 / bf16
weights) and candle_moe_fused_moe_fp8 against the oracle, on sampled rows:
hidden and intermediate sizes with tails (multiples of 8, of 16 for fp8),
1 to 128 experts, k up to 8, Zipf-skewed routing, batches from a single
token to 1024, so that the automatic choice lands on every kernel family
(decode kernels, 32-row, 128x128 and 256x256 tiles) at sizes the fixed
cases do not name. Tolerances as tests/test_gpu_moe.py."""
import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, assert_close, moe_inputs
from test_gpu_fp8 import _quantized_case, _run_fp8
from test_gpu_moe import run_moe

pytestmark = pytest.mark.gpu


def _cases(n=36, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for c in range(n):
        fp8 = bool(rng.random() < 0.4)
        mt = O.QWEN3 if rng.random() < 0.6 else O.NOMIC
        dt = O.BF16 if rng.random() < 0.7 else O.F16
        m = 16 if fp8 else 8
        H, I = int(rng.integers(2, 80)) * m, int(rng.integers(2, 80)) * m
        E = int(rng.choice([1, 2, 4, 6, 8, 16, 32, 64, 128]))
        k = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.choice([1, 3, 8, 16, 33, 64, 100, 128, 200, 256, 512, 700, 1024]))
        zipf = 1.1 if (E >= 16 and rng.random() < 0.5) else 0.0
        out.append((c, fp8, mt, dt, T, H, I, E, k, zipf))
    return out


CASES = _cases()


@pytest.mark.parametrize("c,fp8,mt,dt,T,H,I,E,k,zipf", CASES,
                         ids=[f"{'fp8' if c[1] else 'w16'}-mt{c[2]}-dt{c[3]}-T{c[4]}-H{c[5]}-I{c[6]}-E{c[7]}-k{c[8]}"
                              for c in CASES])
def test_random_shape_default_path(c, fp8, mt, dt, T, H, I, E, k, zipf):
    act = O.SILU if mt == O.QWEN3 else O.GELU
    rows = sorted(set(range(0, T, max(1, T // 64))) | {T - 1})
    if fp8:
        x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, zipf, seed=3000 + c)
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
        want = O.fused_moe(O.to_f32(x, dt), deq["g"], deq["u"], deq.get("d"), rw, ri, E=E, k=k, act=act,
                           moe_type=mt, dtype=O.F32, mode=O.MODE_EXACT, rows=rows)
    else:
        x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 3000 + c, mt, zipf_s=zipf)
        got = run_moe(x, G, U, D if mt == O.QWEN3 else None, rw, ri, E, k, act, mt, dt)
        want = O.fused_moe(x, G, U, D if mt == O.QWEN3 else None, rw, ri, E=E, k=k, act=act, moe_type=mt, dtype=dt,
                           mode=O.MODE_F32ACC, rows=rows)
    kernel = candle_moe.fused_moe_kernel(T, H, I, E, k, dt, mt)
    assert_close(got[rows], want, RTOL[dt], f"{'fp8' if fp8 else '16-bit'} default path (16-bit kernel {kernel})")
