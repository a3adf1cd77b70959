"""The decode kernels (tile policy 18, candle-moe_amd/csrc/moe_gemv_dec.hip)
against the CPU oracle: each workgroup groups the pairs itself, counts the
touched experts and takes one (expert, column block, K slice) item, loads the
weights straight into registers (transposing 8 x 8 blocks of [K,N] weights
into MFMA operands) and splits its slice over its waves; finishing launches
sum the slices' f32 partials in slice order (then the activation, or the k
pairs of a token in slot order). Cases: the BASELINE
decode shapes by default selection, and forced onto shapes that exercise K
and column tails, dropped and repeated experts, more rows per expert than one
chunk, the most pairs over the most experts, both weight layouts ([K,N] and
Nomic's [N,K] fc2), f16 and accumulate mode; owned and caller workspaces bit
for bit. Tolerances as tests/test_gpu_moe.py."""
import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, moe_inputs
from test_gpu_moe import check_case, run_moe, run_raw
from helpers import assert_close

pytestmark = pytest.mark.gpu


def forced(fn):
    try:
        candle_moe.set_tile_policy(candle_moe.TILE_DEC_GEMV)
        return fn()
    finally:
        candle_moe.set_tile_policy(candle_moe.TILE_AUTO)


@pytest.mark.parametrize("T,H,I,E,k,mt", [(1, 2048, 768, 128, 8, O.QWEN3), (8, 4096, 1536, 8, 2, O.QWEN3),
                                          (16, 768, 3072, 8, 2, O.NOMIC)])
def test_decode_shapes_take_the_decode_kernels(T, H, I, E, k, mt):
    assert candle_moe.fused_moe_kernel(T, H, I, E, k, O.BF16, mt) == candle_moe.TILE_DEC_GEMV
    act = O.SILU if mt == O.QWEN3 else O.GELU
    check_case(T, H, I, E, k, O.BF16, mt, act=act, seed=700 + T, zipf=1.1 if E == 128 else 0.0)


# T, H, I, E, k, dtype, moe_type, act: K and column tails (H, I not multiples
# of 32 or of a column block), few and many experts, k = 1 and k > 2
FORCED = [
    (5, 96, 72, 4, 2, O.BF16, O.QWEN3, O.SILU),
    (7, 264, 200, 6, 3, O.F16, O.NOMIC, O.GELU),
    (3, 136, 40, 16, 1, O.BF16, O.QWEN3, O.RELU),
    (33, 512, 256, 8, 2, O.F16, O.QWEN3, O.SILU),
    (12, 320, 648, 64, 4, O.BF16, O.NOMIC, O.SILU),
]


@pytest.mark.parametrize("T,H,I,E,k,dt,mt,act", FORCED)
def test_forced_decode_kernels(T, H, I, E, k, dt, mt, act):
    forced(lambda: check_case(T, H, I, E, k, dt, mt, act=act, seed=710 + T))


def test_decode_kernel_limits():
    # the most pairs (1024) over the most experts (4096): about 1000 touched
    # experts, more (expert, column block) items than one round of workgroups;
    # then 1024 pairs over 2 experts (32 row chunks per workgroup)
    for (T, H, I, E, k, seed) in [(128, 128, 64, 4096, 8, 740), (1024, 64, 96, 2, 1, 741)]:
        def case():
            assert candle_moe.fused_moe_kernel(T, H, I, E, k, O.BF16, O.QWEN3) == candle_moe.TILE_DEC_GEMV
            check_case(T, H, I, E, k, O.BF16, O.QWEN3, seed=seed)
        forced(case)


def test_rows_beyond_one_chunk():
    # 100 tokens over 2 experts, k = 1: ~50 rows per expert, two or more row
    # chunks of 32 per workgroup
    forced(lambda: check_case(100, 256, 128, 2, 1, O.BF16, O.QWEN3, seed=720))
    forced(lambda: check_case(40, 128, 96, 1, 1, O.F16, O.NOMIC, act=O.GELU, seed=721))


def test_dropped_and_repeated_experts():
    T, H, I, E, k = 20, 256, 128, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 730, O.QWEN3)
    ri = ri.copy()
    ri[::3, 1] = 99                 # dropped (>= E)
    ri[1::4, 1] = ri[1::4, 0]       # one expert named twice by a token
    ri[2::7, :] = 77                # every slot dropped
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16)
    got = forced(lambda: run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16))
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw), RTOL[O.BF16], "f32acc")
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw), RTOL[O.BF16], "exact")


def test_accumulate_mode_and_determinism():
    # the raw fused_moe symbol adds into the caller's output; repeated calls
    # give the same bits (no atomics: the k rows are summed in slot order)
    T, H, I, E, k = 16, 512, 384, 32, 4
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 740, O.QWEN3)
    init = O.round_to(O.randn((T, H), seed=741), O.BF16).astype(np.float64)
    a = forced(lambda: run_raw(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init))
    b = forced(lambda: run_raw(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init))
    assert np.array_equal(a, b)
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16,
                       mode=O.MODE_EXACT) + init
    assert_close(a, want, RTOL[O.BF16], "accumulate")


def test_decode_kernels_match_the_32_row_kernel():
    # the same inputs through both decode kernel families
    T, H, I, E, k = 16, 1024, 512, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 750, O.QWEN3)
    a = forced(lambda: run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16))
    try:
        candle_moe.set_tile_policy(candle_moe.TILE_ROWS32)
        b = run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
    finally:
        candle_moe.set_tile_policy(candle_moe.TILE_AUTO)
    assert_close(a, b, RTOL[O.BF16], "decode kernels vs 32-row kernel")


# T, H, I, E, k, dtype, moe_type, act: K slices on both GEMMs (few experts,
# long K), k = 8 over 64 experts, Nomic's [N,K] fc2
FINISH = [
    (8, 1024, 512, 8, 2, O.BF16, O.QWEN3, O.SILU),
    (2, 512, 256, 64, 8, O.BF16, O.QWEN3, O.SILU),
    (16, 256, 512, 8, 2, O.F16, O.NOMIC, O.GELU),
]


@pytest.mark.parametrize("T,H,I,E,k,dt,mt,act", FINISH)
def test_owned_and_caller_workspaces_agree(T, H, I, E, k, dt, mt, act):
    # the library-owned workspace against a caller workspace: the same slices
    # summed in the same order, bit for bit, in accumulate mode
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 760 + T, mt)
    init = O.round_to(O.randn((T, H), seed=761), dt).astype(np.float64)
    a = forced(lambda: run_raw(x, G, U, D, rw, ri, E, k, act, mt, dt, out_init=init))
    b = forced(lambda: run_raw(x, G, U, D, rw, ri, E, k, act, mt, dt, out_init=init, workspace=True))
    assert np.array_equal(a, b)
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=act, moe_type=mt, dtype=dt, mode=O.MODE_EXACT) + init
    assert_close(a, want, RTOL[dt], "accumulate")


@pytest.mark.parametrize("workspace", [False, True])
def test_every_pair_dropped(workspace):
    # no expert touched: the forward writes zeros, the raw symbol leaves its
    # output as it was
    T, H, I, E, k = 4, 256, 128, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 770, O.QWEN3)
    ri = np.full_like(ri, 99)
    init = O.round_to(O.randn((T, H), seed=771), O.BF16).astype(np.float64)
    got = forced(lambda: run_raw(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init,
                                 workspace=workspace))
    assert np.array_equal(got, init)
    fwd = forced(lambda: run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16))
    assert not fwd.any()
