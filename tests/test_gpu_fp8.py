"""FP8 expert weights on the GPU (candle_moe_quantize_fp8 / _dequantize_fp8 /
_fused_moe_fp8) against the CPU oracle.

* dequantize: all 256 codes bit-exact against the oracle's decode (itself
  pinned to the OCP e4m3 definition by tests/test_fp8_oracle.py);
* quantize: codes and scales bit-exact against the oracle's quantizer, both
  input layouts, f32/f16/bf16, with planted zero channels, ties and
  saturating values;
* fused_moe_fp8: against the oracle's f64 MoE over the dequantized weights
  (decode(q) * scale in f32), at the tolerance of the activation dtype
  (rtol 1e-2 f16, 2e-2 bf16, atol = rtol * RMS), at the decode shapes of
  Qwen3 (H4096 I1536 E8 k2, T = 8..64), Qwen3-30B-A3B (H2048 I768 E128 k8,
  T = 1, 16) and Nomic (H768 I3072 E8 k2 GELU), and in accumulate mode.
"""
import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, assert_close, from_dev, moe_inputs, to_dev, torch_dtype

pytestmark = pytest.mark.gpu


def _np(t):
    return t.cpu().numpy()


def test_dequantize_all_codes_bit_exact():
    import torch

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(1, 1, 256).cuda()
    ones = torch.ones((1, 1), dtype=torch.float32, device="cuda:0")
    got = _np(candle_moe.dequantize_fp8(codes, ones, torch.float32)).ravel()
    want = O.e4m3_decode(np.arange(256, dtype=np.uint8))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))  # signed zeros included
    # scaled, rounded to the 16-bit dtypes
    sc = np.array([[0.3712]], np.float32)
    prod = (want * sc[0, 0]).astype(np.float32)
    for dt in (O.BF16, O.F16):
        out = candle_moe.dequantize_fp8(codes, torch.from_numpy(sc).cuda(), torch_dtype(dt))
        g = from_dev(out).ravel()
        w = O.round_to(prod, dt)
        assert np.array_equal(np.isnan(g), np.isnan(w))
        assert np.array_equal(g[fin], w[fin])


def _planted_weights(E, K, N, dt, seed):
    w = O.randn((E, K, N), seed=seed, std=0.05)
    w[0, :, 1] = 0.0                                   # zero channel
    w[1, 3, 2] = 7.0                                   # dominant element
    w[E - 1, :, N - 1] = np.float32(2.0 ** -10)        # a channel of one repeated value
    # values at midpoints of the e4m3 grid after scaling by max/448 = 1 (channel max 448)
    w[0, 0, 3] = 448.0
    w[0, 1:9, 3] = np.array([0.5625, 1.0625, 1.1875, 3 * 2.0 ** -11, 2.0 ** -10, 17.0, 232.0, -9.5], np.float32)
    return O.to_dtype(w, dt)


@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("kn", [True, False])
def test_quantize_matches_oracle_bit_exact(dt, kn):
    E, K, N = 3, 200, 72
    ws = _planted_weights(E, K, N, dt, seed=40 + dt)
    if not kn:
        ws = np.ascontiguousarray(np.transpose(ws, (0, 2, 1)))
    q, s = candle_moe.quantize_fp8(to_dev(ws, dt), input_kn=kn)
    qo, so = O.quantize_fp8(ws, dt, kn=kn)
    assert np.array_equal(_np(s), so)
    assert np.array_equal(_np(q), qo)


# the decode shapes: (name, T, H, I, E, k, act, moe_type, dt, zipf)
CASES = [
    ("qwen3_T8", 8, 4096, 1536, 8, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("qwen3_T16", 16, 4096, 1536, 8, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("qwen3_T32", 32, 4096, 1536, 8, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("qwen3_T64", 64, 4096, 1536, 8, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("qwen3_T16_f16", 16, 4096, 1536, 8, 2, O.SILU, O.QWEN3, O.F16, 0.0),
    ("qwen3_30b_T1", 1, 2048, 768, 128, 8, O.SILU, O.QWEN3, O.BF16, 1.1),
    ("qwen3_30b_T16", 16, 2048, 768, 128, 8, O.SILU, O.QWEN3, O.BF16, 1.1),
    ("nomic_T16", 16, 768, 3072, 8, 2, O.GELU, O.NOMIC, O.BF16, 0.0),
    ("nomic_T16_f16", 16, 768, 3072, 8, 2, O.GELU, O.NOMIC, O.F16, 0.0),
    ("qwen3_odd_T5", 5, 272, 208, 4, 2, O.RELU, O.QWEN3, O.BF16, 0.0),  # sizes off the 64-element tiles
]


def _quantized_case(T, H, I, E, k, moe_type, dt, zipf, seed):
    """Inputs, the GPU-quantized weights (checked against the oracle's
    quantizer) and the dequantized f32 weights in the oracle's layouts."""
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, seed, moe_type, zipf_s=zipf)
    dev = {}
    deq = {}
    # Qwen3: gate/up [E,H,I] and down [E,I,H] are [E,K,N]; Nomic: fc1 [E,H,I]
    # is [E,K,N], fc2 [E,H,I] is [E,N,K]
    specs = [("g", G, True), ("u", U, moe_type == O.QWEN3)] + ([("d", D, True)] if moe_type == O.QWEN3 else [])
    for name, w, kn in specs:
        q, s = candle_moe.quantize_fp8(to_dev(w, dt), input_kn=kn)
        qo, so = O.quantize_fp8(w, dt, kn=kn)
        assert np.array_equal(_np(q), qo) and np.array_equal(_np(s), so), f"quantize {name}"
        dev[name] = (q, s)
        d = O.dequantize_fp8(qo, so)  # [E,N,K]
        deq[name] = np.ascontiguousarray(np.transpose(d, (0, 2, 1))) if kn else d
    return x, rw, ri, dev, deq


def _run_fp8(x, rw, ri, dev, E, k, act, moe_type, dt, out_init=None):
    import torch

    T, H = x.shape
    tx = to_dev(x, dt)
    out = torch.zeros((T, H), dtype=tx.dtype, device="cuda:0") if out_init is None else to_dev(out_init, dt)
    g, u = dev["g"], dev["u"]
    if moe_type == O.QWEN3:
        d = dev["d"]
        candle_moe.fused_moe_fp8(tx, g[0], u[0], d[0], g[1], u[1], d[1], to_dev(rw), to_dev(ri), out, E, k, act,
                                 moe_type)
    else:  # fc1 = gate, fc2 = up
        candle_moe.fused_moe_fp8(tx, g[0], u[0], None, g[1], u[1], None, to_dev(rw), to_dev(ri), out, E, k, act,
                                 moe_type)
    torch.cuda.synchronize()
    return from_dev(out).astype(np.float64)


def _oracle(x, rw, ri, deq, E, k, act, moe_type, dt, out_init=None):
    xf = O.to_f32(x, dt)
    oi = None if out_init is None else O.to_f32(out_init, dt).astype(np.float64)
    return O.fused_moe(xf, deq["g"], deq["u"], deq.get("d"), rw, ri, E=E, k=k, act=act, moe_type=moe_type,
                       dtype=O.F32, mode=O.MODE_EXACT, out_init=oi)


@pytest.mark.parametrize("name,T,H,I,E,k,act,mt,dt,zipf", CASES, ids=[c[0] for c in CASES])
def test_fused_moe_fp8_matches_oracle(name, T, H, I, E, k, act, mt, dt, zipf):
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, zipf, seed=50 + T)
    got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt)
    assert_close(got, want, RTOL[dt], f"{name} fp8 vs f64 oracle on the dequantized weights")


# The 32-row LDS-DMA kernel (tile policy 12; by default from 129 pairs up to
# 32 rows per touched expert) forced on decode cases.
ROWS32_CASES = [c for c in CASES if c[0] in ("qwen3_T32", "qwen3_T64", "qwen3_30b_T16", "nomic_T16", "qwen3_odd_T5")]


@pytest.mark.parametrize("name,T,H,I,E,k,act,mt,dt,zipf", ROWS32_CASES, ids=[c[0] for c in ROWS32_CASES])
def test_fused_moe_fp8_32_row_kernel(name, T, H, I, E, k, act, mt, dt, zipf):
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, zipf, seed=350 + T)
    candle_moe.set_tile_policy(candle_moe.TILE_ROWS32)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt)
    assert_close(got, want, RTOL[dt], f"{name} 32-row fp8 kernel vs f64 oracle")


# The register-operand decode kernel (tile policy 17; by default only up to
# 16 pairs) forced on every decode case: K and N tails, tiles
# of more than 16 rows (two row blocks) and more than 32 (several tiles per
# expert), f16, Nomic's fc1 / fc2, and accumulate mode with dropped pairs.
GEMV_CASES = CASES + [
    ("qwen3_rows24_T48", 48, 1024, 512, 4, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("qwen3_skew_T96", 96, 512, 256, 8, 2, O.SILU, O.QWEN3, O.BF16, 2.0),
    # blocks of 48 and 96 columns on the decode kernels, with column tails
    ("qwen3_cols48_T16", 16, 512, 1504, 8, 2, O.SILU, O.QWEN3, O.BF16, 0.0),
    ("nomic_cols96_T16", 16, 256, 3024, 8, 2, O.GELU, O.NOMIC, O.BF16, 0.0),
]


@pytest.mark.parametrize("name,T,H,I,E,k,act,mt,dt,zipf", GEMV_CASES, ids=[c[0] for c in GEMV_CASES])
def test_fused_moe_fp8_register_operand_kernel(name, T, H, I, E, k, act, mt, dt, zipf):
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, zipf, seed=150 + T)
    candle_moe.set_tile_policy(candle_moe.TILE_W8_GEMV)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt)
    assert_close(got, want, RTOL[dt], f"{name} register-operand fp8 kernel vs f64 oracle")


def test_fused_moe_fp8_register_operand_kernel_accumulates_and_drops():
    T, H, I, E, k = 24, 512, 256, 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, O.QWEN3, O.BF16, 0.0, seed=93)
    ri = ri.copy()
    ri[::3, 1] = E + 5
    init = O.to_dtype(O.randn((T, H), seed=94, std=0.5), O.BF16)
    candle_moe.set_tile_policy(candle_moe.TILE_W8_GEMV)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init)
    assert_close(got, want, RTOL[O.BF16], "register-operand fp8 kernel, accumulate mode with dropped pairs")


# The decode kernels (tile policy 18, by default up to 128 pairs: the pairs
# grouped inside the GEMM kernels, two 16-code loads per lane and column as
# four MFMA operands, column scales in the epilogue) forced on the same cases.
@pytest.mark.parametrize("name,T,H,I,E,k,act,mt,dt,zipf", GEMV_CASES, ids=[c[0] for c in GEMV_CASES])
def test_fused_moe_fp8_decode_kernels(name, T, H, I, E, k, act, mt, dt, zipf):
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, zipf, seed=250 + T)
    candle_moe.set_tile_policy(candle_moe.TILE_DEC_GEMV)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt)
    assert_close(got, want, RTOL[dt], f"{name} fp8 decode kernels vs f64 oracle")


def test_fused_moe_fp8_decode_kernels_at_their_limits():
    # 1024 pairs (the most) over 4096 experts (the most): ~1000 touched
    # experts, more items than one round of workgroups
    T, H, I, E, k = 128, 128, 64, 4096, 8
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, O.QWEN3, O.BF16, 0.0, seed=280)
    candle_moe.set_tile_policy(candle_moe.TILE_DEC_GEMV)
    try:
        assert candle_moe.fused_moe_kernel(T, H, I, E, k, O.BF16, O.QWEN3) == candle_moe.TILE_DEC_GEMV
        got = _run_fp8(x, rw, ri, dev, E, k, O.SILU, O.QWEN3, O.BF16)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, O.SILU, O.QWEN3, O.BF16)
    assert_close(got, want, RTOL[O.BF16], "fp8 decode kernels, 1024 pairs over 4096 experts")


def test_fused_moe_fp8_decode_kernels_accumulate_and_drop():
    T, H, I, E, k = 24, 512, 256, 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, O.QWEN3, O.BF16, 0.0, seed=293)
    ri = ri.copy()
    ri[::3, 1] = E + 5
    init = O.to_dtype(O.randn((T, H), seed=294, std=0.5), O.BF16)
    candle_moe.set_tile_policy(candle_moe.TILE_DEC_GEMV)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init)
    assert_close(got, want, RTOL[O.BF16], "fp8 decode kernels, accumulate mode with dropped pairs")


@pytest.mark.parametrize("mt", [O.QWEN3, O.NOMIC])
def test_fused_moe_fp8_accumulates(mt):
    T, H, I, E, k = (16, 4096, 1536, 8, 2) if mt == O.QWEN3 else (16, 768, 3072, 8, 2)
    act = O.SILU if mt == O.QWEN3 else O.GELU
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, O.BF16, 0.0, seed=77)
    init = O.to_dtype(O.randn((T, H), seed=78, std=0.5), O.BF16)
    got = _run_fp8(x, rw, ri, dev, E, k, act, mt, O.BF16, out_init=init)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, O.BF16, out_init=init)
    assert_close(got, want, RTOL[O.BF16], "fp8 accumulate mode")


def test_fused_moe_fp8_drops_out_of_range_experts():
    # expert ids >= E are dropped by the grouping, as on the bf16 path
    T, H, I, E, k = 24, 512, 256, 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, O.QWEN3, O.BF16, 0.0, seed=91)
    ri = ri.copy()
    ri[::3, 1] = E + 5
    ri[5, :] = 1000
    got = _run_fp8(x, rw, ri, dev, E, k, O.SILU, O.QWEN3, O.BF16)
    want = _oracle(x, rw, ri, deq, E, k, O.SILU, O.QWEN3, O.BF16)
    assert not np.any(want[5]) and not np.any(got[5])
    assert_close(got, want, RTOL[O.BF16], "fp8 with dropped pairs")


@pytest.mark.parametrize("policy", [0, candle_moe.TILE_W8])
@pytest.mark.parametrize("mt,T,H,I,act,dt", [
    (O.QWEN3, 600, 256, 192, O.SILU, O.BF16),
    (O.NOMIC, 700, 320, 256, O.GELU, O.F16),
    (O.QWEN3, 333, 208, 272, O.RELU, O.F16),   # sizes off the 64-element tiles
])
def test_fused_moe_fp8_prefill_kernel_all_rows(mt, T, H, I, act, dt, policy):
    # 40-90 pairs per touched expert over small weights: by default the 32-row
    # kernel (its weight stream is small), forced the 8-wave 256x256 kernel
    # (gate/up or fc1, then the pair-row down / fc2 and the row sums)
    E, k = 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, dt, 0.0, seed=95 + T)
    candle_moe.set_tile_policy(policy)
    try:
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt)
    finally:
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt)
    assert_close(got, want, RTOL[dt], f"fp8 (tile policy {policy}) vs f64 oracle on the dequantized weights")


@pytest.mark.parametrize("mt,T,H,I,E,k,act,dt,zero_cols,accumulate", [
    (O.QWEN3, 600, 256, 192, 8, 2, O.SILU, O.BF16, False, False),
    (O.QWEN3, 600, 256, 1536, 8, 2, O.SILU, O.BF16, True, False),    # 48 K tiles: tail K splits across segments
    (O.QWEN3, 1500, 256, 1536, 8, 2, O.SILU, O.F16, False, True),
    (O.QWEN3, 900, 256, 192, 6, 3, O.RELU, O.BF16, True, False),    # three segments per set
    (O.NOMIC, 700, 320, 256, 8, 2, O.GELU, O.F16, True, True),
])
def test_fused_moe_fp8_expert_sets(mt, T, H, I, E, k, act, dt, zero_cols, accumulate):
    # the expert-set down / fc2 GEMM with fp8 weights keeps its accumulators
    # in the current segment's column units (rescaled at each segment start,
    # made absolute after the K loop); all-zero weight columns (scale 0, unit
    # 1) and accumulate mode included
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 120 + T, mt)
    if zero_cols:
        if mt == O.QWEN3:
            D = D.copy()
            D[1, :, 5] = 0
            D[E - 1, :, 7:9] = 0
        else:
            U = U.copy()
            U[2, 3, :] = 0   # Nomic fc2 is [E,H,I]: output column 3 of expert 2
    dev, deq = {}, {}
    specs = [("g", G, True), ("u", U, mt == O.QWEN3)] + ([("d", D, True)] if mt == O.QWEN3 else [])
    for name, w, kn in specs:
        q, sc = candle_moe.quantize_fp8(to_dev(w, dt), input_kn=kn)
        dev[name] = (q, sc)
        d = O.dequantize_fp8(_np(q), _np(sc))
        deq[name] = np.ascontiguousarray(np.transpose(d, (0, 2, 1))) if kn else d
    init = O.to_dtype(O.randn((T, H), seed=121, std=0.5), dt) if accumulate else None
    try:
        # (expert sets run on the 8-wave kernel, which these sizes do not
        # take by default)
        candle_moe.set_tile_policy(candle_moe.TILE_W8)
        candle_moe.set_combine_policy(candle_moe.COMBINE_EXPERT_SETS)
        got = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt, out_init=init)
    finally:
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
        candle_moe.set_tile_policy(0)
    want = _oracle(x, rw, ri, deq, E, k, act, mt, dt, out_init=init)
    assert_close(got, want, RTOL[dt], "fp8 expert sets vs f64 oracle on the dequantized weights")
    # and the pair path on the same inputs
    try:
        candle_moe.set_combine_policy(candle_moe.COMBINE_PAIRS)
        got2 = _run_fp8(x, rw, ri, dev, E, k, act, mt, dt, out_init=init)
    finally:
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
    assert_close(got2, want, RTOL[dt], "fp8 pair path vs f64 oracle")


@pytest.mark.parametrize("mt,T,H,I,act,rows_every", [
    (O.QWEN3, 256, 1024, 512, O.SILU, 1),     # 64 pairs per expert
    (O.NOMIC, 1024, 768, 3072, O.GELU, 7),    # 256 pairs per expert, Nomic's size
])
def test_fused_moe_fp8_32_row_kernel_by_default_beyond_decode(mt, T, H, I, act, rows_every):
    # beyond 32 pairs per touched expert with a small weight stream the
    # default fp8 path stays on the 32-row kernel (its K splits, the grouping
    # launch, f32 accumulation of the k pairs)
    E, k = 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, mt, O.BF16, 0.0, seed=96 + T)
    got = _run_fp8(x, rw, ri, dev, E, k, act, mt, O.BF16)
    rows = sorted(set(range(0, T, rows_every)) | {T - 1})
    xf = O.to_f32(x, O.BF16)
    want = O.fused_moe(xf, deq["g"], deq["u"], deq.get("d"), rw, ri, E=E, k=k, act=act, moe_type=mt,
                       dtype=O.F32, mode=O.MODE_EXACT, rows=rows)
    assert_close(got[rows], want, RTOL[O.BF16], "fp8 default path beyond decode sizes (sampled rows)")


def test_fused_moe_fp8_prefill_batch_sampled_rows():
    # 2048 tokens: the 8-wave 256x256 fp8 kernel with the tail's K splits
    T, H, I, E, k = 2048, 1024, 512, 8, 2
    x, rw, ri, dev, deq = _quantized_case(T, H, I, E, k, O.QWEN3, O.BF16, 0.0, seed=92)
    got = _run_fp8(x, rw, ri, dev, E, k, O.SILU, O.QWEN3, O.BF16)
    rows = sorted(set(range(0, T, 29)) | {T - 1})
    xf = O.to_f32(x, O.BF16)
    want = O.fused_moe(xf, deq["g"], deq["u"], deq["d"], rw, ri, E=E, k=k, act=O.SILU, moe_type=O.QWEN3,
                       dtype=O.F32, mode=O.MODE_EXACT, rows=rows)
    assert_close(got[rows], want, RTOL[O.BF16], "fp8 at T=2048 (sampled rows)")
