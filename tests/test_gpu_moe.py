"""Fused-MoE parity on the GPU: HIP kernels vs the CPU oracle.

Tolerances (north star): rtol 1e-4 (f32), 1e-2 (f16), 2e-2 (bf16) with
atol = rtol * RMS(expected), in the reference's |a-b| <= atol + rtol*max
form (/root/reference/tests/moe_tests.rs:61-91). The GPU result is checked
against both oracle modes: the candle-native per-op rounding and the f64
evaluation of the same dtype-valued inputs.
"""
import ctypes
import zlib

import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, assert_close, assert_close_norm, from_dev, moe_inputs, tile_covering_rows, to_dev

pytestmark = pytest.mark.gpu

ACT = {O.SILU: candle_moe.Activation.Silu, O.GELU: candle_moe.Activation.Gelu, O.RELU: candle_moe.Activation.Relu}


def run_moe(x, G, U, D, rw, ri, E, k, act, moe_type, dt):
    import torch

    moe = candle_moe.FusedMoE.new(E, k, ACT[act])
    out = moe.forward(to_dev(x, dt), to_dev(G, dt), to_dev(U, dt), None if D is None else to_dev(D, dt),
                      to_dev(rw), to_dev(ri), moe_type)
    torch.cuda.synchronize()
    return from_dev(out).astype(np.float64)


def run_raw(x, G, U, D, rw, ri, E, k, act, moe_type, dt, out_init=None, workspace=False):
    """Through the reference's fused_moe symbol (or its workspace variant)."""
    import torch

    T, H = x.shape
    I = G.shape[2]
    tx, tg, tu = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt)
    td = None if D is None else to_dev(D, dt)
    trw, tri = to_dev(rw), to_dev(ri)
    if out_init is None:
        out = torch.zeros((T, H), dtype=tx.dtype, device="cuda:0")
    else:
        out = torch.from_numpy(out_init.astype(np.float32)).to("cuda:0").to(tx.dtype)
    L = candle_moe.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if workspace:
        n = L.candle_moe_fused_moe_workspace_size(T, H, I, E, k, dt)
        ws = torch.empty(n + 256, dtype=torch.uint8, device="cuda:0")
        base = (ws.data_ptr() + 255) // 256 * 256
        rc = L.candle_moe_fused_moe_ws(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k, act,
                                       moe_type, dt, ctypes.c_void_p(base), n, stream)
        candle_moe.check(rc)
    else:
        L.fused_moe(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k, act, moe_type, dt, stream)
        assert candle_moe.last_error() == "", candle_moe.last_error()
    torch.cuda.synchronize()
    return from_dev(out).astype(np.float64)


def covering_rows(T, H, I, E, k, dt, moe_type, ri, extra=()):
    """The first and last rows of every row tile (and tile half) of the GEMMs
    fused_moe dispatches for this routing (the path's groupings, the
    dispatched kernel's tile height), plus extra rows."""
    BM = candle_moe.fused_moe_tile(T, H, I, E, k, dt, moe_type)
    path = candle_moe.fused_moe_path(T, H, I, E, k, dt, moe_type)
    assert BM >= 32 and path in ("expert-set", "pairs", "simt"), (BM, path)
    rows = sorted(set(tile_covering_rows(ri, E, BM, path)) | set(extra))
    print(f"  {len(rows)} rows cover every {BM}-row tile on the {path} path", flush=True)
    return rows


def check_case(T, H, I, E, k, dt, moe_type, act=O.SILU, seed=0, wstd=0.02, rows=None, skew=0.0, zipf=0.0,
               api="host"):
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, seed, moe_type, wstd=wstd, skew_sigma=skew, zipf_s=zipf)
    if isinstance(rows, str) and rows == "tiles":
        rows = covering_rows(T, H, I, E, k, dt, moe_type, ri, extra=SAMPLE if T == 32768 else ())
    if api == "host":
        got = run_moe(x, G, U, D, rw, ri, E, k, act, moe_type, dt)
    else:
        got = run_raw(x, G, U, D, rw, ri, E, k, act, moe_type, dt, workspace=(api == "ws"))
    kw = dict(E=E, k=k, act=act, moe_type=moe_type, dtype=dt, rows=rows)
    f32acc = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw)
    exact = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw)
    cand = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_CANDLE, **kw)
    if rows is not None:
        got = got[np.asarray(rows)]
    name = f"T={T} H={H} I={I} E={E} k={k} dt={dt} type={moe_type} act={act}"
    assert_close(got, f32acc, RTOL[dt], name + " vs f32-accumulation oracle")
    assert_close(got, exact, RTOL[dt], name + " vs f64 oracle")
    assert_close_norm(got, cand, RTOL[dt], name + " vs candle per-op-rounding oracle")
    return got


# ---- the reference's own test cases (/root/reference/tests/moe_tests.rs:279-397):
# E=8, SiLU, I = 4H, weights N(0,1)
REF_CASES = [
    ("nomic_fp32", O.F32, 16, 16, 2, O.NOMIC),
    ("nomic_fp16_gemm", O.F16, 64, 32, 2, O.NOMIC),
    ("nomic_fp16_gemm_topk1", O.F16, 64, 32, 1, O.NOMIC),
    ("qwen3_fp32", O.F32, 64, 32, 2, O.QWEN3),
    ("qwen3_fp16_direct", O.F16, 64, 4, 2, O.QWEN3),
    ("qwen3_fp16_gemm", O.F16, 64, 32, 2, O.QWEN3),
    ("qwen3_fp16_gemm_topk1", O.F16, 64, 32, 1, O.QWEN3),
    ("qwen3_bf16_direct", O.BF16, 64, 4, 2, O.QWEN3),
    ("qwen3_bf16_gemm", O.BF16, 64, 32, 2, O.QWEN3),
    ("qwen3_bf16_gemm_topk1", O.BF16, 64, 32, 1, O.QWEN3),
]


@pytest.mark.parametrize("name,dt,H,T,k,mt", REF_CASES, ids=[c[0] for c in REF_CASES])
def test_reference_cases(name, dt, H, T, k, mt):
    check_case(T, H, 4 * H, 8, k, dt, mt, wstd=1.0, seed=zlib.crc32(name.encode()) % 1000)


# ---- BASELINE config 3 (Nomic, H768 I3072 E8 k2 GELU) at the sizes the oracle finishes quickly
@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("T", [16, 64])
def test_nomic_config(dt, T):
    check_case(T, 768, 3072, 8, 2, dt, O.NOMIC, act=O.GELU, seed=3)


# ---- BASELINE config 4 (Qwen3, H4096 I1536 E8 k2 SiLU)
@pytest.mark.parametrize("dt", [O.F16, O.BF16])
@pytest.mark.parametrize("T", [8, 16, 32, 64])
def test_qwen3_config(dt, T):
    check_case(T, 4096, 1536, 8, 2, dt, O.QWEN3, seed=4)


# ---- BASELINE config 5 (Qwen3-30B-A3B: H2048 I768 E128 k8, Zipf-skewed routing)
@pytest.mark.parametrize("T", [1, 16, 128])
def test_qwen3_30b_config(T):
    check_case(T, 2048, 768, 128, 8, O.BF16, O.QWEN3, seed=5, zipf=1.1)


# ---- the remaining (T, dtype) points of BASELINE configs 3 and 4: every row
# at T=512 and 4096; at T=32768 the first and last rows of every row tile of
# every GEMM launch (each output row depends only on its own token, its
# routing and the weights, and every column of a checked row is compared)
@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
def test_nomic_config_T512_all_rows(dt):
    check_case(512, 768, 3072, 8, 2, dt, O.NOMIC, act=O.GELU, seed=32)


@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
def test_nomic_config_T4096_all_rows(dt):
    check_case(4096, 768, 3072, 8, 2, dt, O.NOMIC, act=O.GELU, seed=33)


@pytest.mark.slow
@pytest.mark.parametrize("dt", [O.F32, O.F16])
def test_nomic_config_T32768_tile_rows(dt):
    check_case(32768, 768, 3072, 8, 2, dt, O.NOMIC, act=O.GELU, seed=34, rows="tiles")


@pytest.mark.slow
def test_qwen3_config_T32768_f16_tile_rows():
    assert candle_moe.fused_moe_path(32768, 4096, 1536, 8, 2, O.F16) == "expert-set"
    check_case(32768, 4096, 1536, 8, 2, O.F16, O.QWEN3, seed=35, rows="tiles")


def test_activations_and_odd_shapes():
    for act in (O.SILU, O.GELU, O.RELU):
        check_case(40, 96, 72, 4, 2, O.BF16, O.QWEN3, act=act, seed=6)
        check_case(40, 96, 72, 4, 2, O.F32, O.NOMIC, act=act, seed=7)
    # shapes that are not multiples of 8 take the SIMT kernels
    check_case(19, 20, 36, 3, 2, O.BF16, O.QWEN3, seed=8)
    check_case(19, 20, 36, 3, 3, O.F16, O.NOMIC, seed=9)


def test_raw_symbol_and_workspace_variant():
    a = check_case(48, 256, 128, 8, 2, O.BF16, O.QWEN3, seed=10, api="raw")
    b = check_case(48, 256, 128, 8, 2, O.BF16, O.QWEN3, seed=10, api="ws")
    assert np.array_equal(a, b)


def test_output_is_accumulated():
    # the reference kernels add into the caller's output (ffi.rs:35 requires zeros)
    T, H, I, E, k = 32, 128, 64, 4, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 11, O.QWEN3)
    init = O.round_to(O.randn((T, H), seed=12), O.BF16).astype(np.float64)
    got = run_raw(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16, out_init=init)
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16,
                       mode=O.MODE_EXACT) + init
    assert_close(got, want, RTOL[O.BF16], "accumulate into output")


def test_empty_and_invalid_indices():
    import torch

    moe = candle_moe.FusedMoE.new(4, 2, candle_moe.Activation.Silu)
    x = torch.zeros((0, 64), dtype=torch.bfloat16, device="cuda:0")
    g = torch.zeros((4, 64, 32), dtype=torch.bfloat16, device="cuda:0")
    d = torch.zeros((4, 32, 64), dtype=torch.bfloat16, device="cuda:0")
    rw = torch.zeros((0, 2), dtype=torch.float32, device="cuda:0")
    ri = torch.zeros((0, 2), dtype=torch.int32, device="cuda:0")
    out = moe.forward(x, g, g, d, rw, ri, 0)
    assert out.shape == (0, 64)
    # expert ids >= E are dropped (/root/reference/kernels/preprocessing.cuh:49-52)
    T, H, I, E, k = 16, 64, 32, 4, 2
    xx, G, U, D, w, i = moe_inputs(T, H, I, E, k, O.BF16, 13, O.QWEN3)
    i = i.copy()
    i[::3, 1] = 99
    got = run_moe(xx, G, U, D, w, i, E, k, O.SILU, O.QWEN3, O.BF16)
    want = O.fused_moe(xx, G, U, D, w, i, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16, mode=O.MODE_EXACT)
    assert_close(got, want, RTOL[O.BF16], "dropped pairs")


def test_owned_workspace_reused_grown_and_trimmed():
    # the library keeps one workspace per (device, stream) between calls:
    # larger, smaller and larger again on one stream, a second stream, a trim
    import torch

    H, I, E, k = 128, 64, 8, 2
    cases = {T: moe_inputs(T, H, I, E, k, O.BF16, 50 + T, O.QWEN3) for T in (48, 3000, 16, 5000)}
    want = {T: O.fused_moe(*c, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16, mode=O.MODE_F32ACC)
            for T, c in cases.items()}
    side = torch.cuda.Stream()
    for T in (48, 3000, 16, 5000, 48):
        assert_close(run_moe(*cases[T], E, k, O.SILU, O.QWEN3, O.BF16), want[T], RTOL[O.BF16], f"default stream T={T}")
        with torch.cuda.stream(side):
            got = run_moe(*cases[T], E, k, O.SILU, O.QWEN3, O.BF16)
        assert_close(got, want[T], RTOL[O.BF16], f"side stream T={T}")
    candle_moe.trim_workspaces()
    assert_close(run_moe(*cases[3000], E, k, O.SILU, O.QWEN3, O.BF16), want[3000], RTOL[O.BF16], "after trim")
    assert_close(run_raw(*cases[16], E, k, O.SILU, O.QWEN3, O.BF16), want[16], RTOL[O.BF16], "raw after trim")


@pytest.mark.parametrize("combine", [1, 2])
def test_tail_balanced_splits(combine):
    # the 8-wave 256x256 kernel splits the tiles of each XCD's last round
    # along K (here every gate/up tile: 2 per XCD, 4 splits of 8 K tiles);
    # the splits meet in the ordered fixup, so the result matches the oracle
    # and repeats bit for bit
    T, H, I, E, k = 512, 2048, 256, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 60 + combine, O.QWEN3)
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16)
    try:
        candle_moe.set_tile_policy(candle_moe.TILE_W8)
        candle_moe.set_combine_policy(combine)
        a = run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
        b = run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
    finally:
        candle_moe.set_tile_policy(0)
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
    assert np.array_equal(a, b)
    assert_close(a, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw), RTOL[O.BF16], "f32acc")
    assert_close(a, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw), RTOL[O.BF16], "exact")


def test_deterministic_k2():
    x, G, U, D, rw, ri = moe_inputs(512, 1024, 512, 8, 2, O.BF16, 14, O.QWEN3)
    a = run_moe(x, G, U, D, rw, ri, 8, 2, O.SILU, O.QWEN3, O.BF16)
    b = run_moe(x, G, U, D, rw, ri, 8, 2, O.SILU, O.QWEN3, O.BF16)
    assert np.array_equal(a, b)


# ---- full BASELINE sizes: the first and last rows of every row tile of
# every GEMM launch, plus a few fixed tokens (each output row depends only on
# its own token, its routing and the weights)
SAMPLE = [0, 1, 2, 777, 4095, 5000, 12345, 20000, 32767]


@pytest.mark.slow
def test_qwen3_full_size_tile_rows():
    check_case(32768, 4096, 1536, 8, 2, O.BF16, O.QWEN3, seed=15, rows="tiles")


@pytest.mark.slow
def test_nomic_full_size_tile_rows():
    check_case(32768, 768, 3072, 8, 2, O.BF16, O.NOMIC, act=O.GELU, seed=16, rows="tiles")


@pytest.mark.slow
def test_qwen3_30b_prefill_all_rows():
    check_case(4096, 2048, 768, 128, 8, O.BF16, O.QWEN3, seed=17, zipf=1.1)


# ---- the two combine paths (expert-set GEMM vs pair GEMM + pair-row sums or f32 atomics) on the same inputs
SET_CASES = [
    # T, H, I, E, k, dtype, moe_type, act
    (4096, 256, 128, 8, 2, O.BF16, O.QWEN3, O.SILU),
    (4096, 256, 192, 8, 2, O.F16, O.NOMIC, O.GELU),
    (2048, 128, 64, 8, 1, O.BF16, O.QWEN3, O.RELU),
    (4096, 128, 128, 8, 3, O.BF16, O.QWEN3, O.SILU),
    (3000, 192, 128, 4, 2, O.BF16, O.NOMIC, O.SILU),
]


@pytest.mark.parametrize("T,H,I,E,k,dt,mt,act", SET_CASES)
def test_expert_set_path_matches_pair_path(T, H, I, E, k, dt, mt, act):
    try:
        candle_moe.set_combine_policy(candle_moe.COMBINE_EXPERT_SETS)
        assert candle_moe.fused_moe_path(T, H, I, E, k, dt) == "expert-set"
        a = check_case(T, H, I, E, k, dt, mt, act=act, seed=20 + k, rows=list(range(0, T, 97)))
        candle_moe.set_combine_policy(candle_moe.COMBINE_PAIRS)
        assert candle_moe.fused_moe_path(T, H, I, E, k, dt) == "pairs"
        b = check_case(T, H, I, E, k, dt, mt, act=act, seed=20 + k, rows=list(range(0, T, 97)))
    finally:
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
    assert_close(a, b, RTOL[dt], "expert-set vs pair path")


def test_expert_set_path_dropped_and_repeated_experts():
    # ids >= E are dropped; the raw ABI also allows a token to name one expert twice
    T, H, I, E, k = 2048, 128, 128, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 30, O.QWEN3)
    ri = ri.copy()
    ri[::5, 1] = 77
    ri[1::7, 1] = ri[1::7, 0]
    ri[2::11, :] = 9
    try:
        candle_moe.set_combine_policy(candle_moe.COMBINE_EXPERT_SETS)
        got = run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
    finally:
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16)
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw), RTOL[O.BF16], "f32acc")
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw), RTOL[O.BF16], "exact")
    assert (got[2::11] == 0).all()


def test_multi_block_grouping_skewed_dropped_repeated():
    # more items than the one-workgroup grouping takes (per-block histograms,
    # the cross-block scan, the block scatter), with a skewed load, dropped
    # ids and repeated experts, every row checked on both combine paths
    T, H, I, E, k = 9000, 64, 64, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 31, O.QWEN3)
    ri = ri.copy()
    ri[::2, 0] = 3
    ri[::13, 1] = 50
    ri[5::17, 1] = ri[5::17, 0]
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16)
    want = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw)
    for combine in (candle_moe.COMBINE_PAIRS, candle_moe.COMBINE_EXPERT_SETS):
        try:
            candle_moe.set_combine_policy(combine)
            got = run_moe(x, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
        finally:
            candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
        assert_close(got, want, RTOL[O.BF16], "combine %d" % combine)


@pytest.mark.parametrize("T,H,I,E,k,mt,dt,skew", [
    (9000, 64, 64, 8, 2, O.QWEN3, O.BF16, True),      # expert sets: pair and token groupings, 9 + 18 blocks
    (3000, 128, 64, 16, 4, O.NOMIC, O.F16, False),   # pair path, 12 blocks
    (700, 64, 64, 128, 8, O.QWEN3, O.BF16, False),   # 128 bins, 6 blocks
])
def test_grouping_launch_modes_agree(T, H, I, E, k, mt, dt, skew):
    # one launch (a wait for every block's counts), two launches, and one
    # launch whose workgroups all recount every item: the grouping is stable,
    # so the three give the same sorted order and bit-identical outputs, also
    # through the raw symbol (library workspace) and a caller workspace (two
    # launches); checked against the oracle once
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 41, mt)
    if skew:
        ri = ri.copy()
        ri[::2, 0] = 3
        ri[::13, 1] = 50
        ri[5::17, 1] = ri[5::17, 0]
    D = D if mt == O.QWEN3 else None
    outs = {}
    try:
        for mode in (candle_moe.GROUPING_AUTO, candle_moe.GROUPING_TWO_LAUNCHES, candle_moe.GROUPING_ONE_LAUNCH_RECOUNT,
                     candle_moe.GROUPING_AUTO):
            candle_moe.set_grouping_mode(mode)
            outs[mode] = (run_moe(x, G, U, D, rw, ri, E, k, O.SILU, mt, dt),
                          run_raw(x, G, U, D, rw, ri, E, k, O.SILU, mt, dt),
                          run_raw(x, G, U, D, rw, ri, E, k, O.SILU, mt, dt, workspace=True))
    finally:
        candle_moe.set_grouping_mode(candle_moe.GROUPING_AUTO)
    ref = outs[candle_moe.GROUPING_TWO_LAUNCHES][0]
    for mode, got in outs.items():
        for g in got:
            assert np.array_equal(g, ref), "grouping mode %d differs" % mode
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=O.SILU, moe_type=mt, dtype=dt, mode=O.MODE_F32ACC)
    assert_close(ref, want, RTOL[dt], "grouping modes")


def test_headline_shape_takes_expert_set_path():
    assert candle_moe.fused_moe_path(32768, 4096, 1536, 8, 2, O.BF16) == "expert-set"
    assert candle_moe.fused_moe_path(4096, 2048, 768, 128, 8, O.BF16) == "pairs"
    assert candle_moe.fused_moe_path(32, 64, 256, 8, 2, O.F32) == "simt"


@pytest.mark.parametrize("tile", [15, 16])
def test_f32_tiles(tile):
    # the f32 vector-FMA kernel at both tile heights: K not a multiple of its
    # 16-deep chunks, N not a multiple of its 128 (64 for gate/up) columns,
    # [N,K] fc2 weights (Nomic), top-1
    try:
        candle_moe.set_tile_policy(tile)
        check_case(300, 100, 196, 8, 2, O.F32, O.QWEN3, seed=70 + tile)
        check_case(200, 132, 76, 6, 2, O.F32, O.NOMIC, act=O.GELU, seed=71 + tile)
        check_case(40, 64, 48, 8, 1, O.F32, O.QWEN3, seed=72 + tile)
    finally:
        candle_moe.set_tile_policy(0)


def test_f32_decode_splits_deterministic():
    # decode: 32-row f32 tiles with K split over several workgroups, ordered fixup
    T, H, I, E, k = 4, 768, 3072, 8, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.F32, 80, O.NOMIC)
    a = run_moe(x, G, U, None, rw, ri, E, k, O.GELU, O.NOMIC, O.F32)
    b = run_moe(x, G, U, None, rw, ri, E, k, O.GELU, O.NOMIC, O.F32)
    assert np.array_equal(a, b)
    want = O.fused_moe(x, G, U, None, rw, ri, E=E, k=k, act=O.GELU, moe_type=O.NOMIC, dtype=O.F32,
                       mode=O.MODE_EXACT)
    assert_close(a, want, RTOL[O.F32], "f32 decode")


def test_f32_unaligned_operands_take_the_scalar_kernel():
    # 16-byte loads need aligned operands; an input 4 bytes off takes moe_simt_gemm
    import torch

    T, H, I, E, k = 64, 128, 96, 4, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.F32, 81, O.QWEN3)
    big = torch.zeros(T * H + 1, dtype=torch.float32, device="cuda:0")
    big[1:] = to_dev(x).reshape(-1)
    tg, tu, td, trw, tri = to_dev(G), to_dev(U), to_dev(D), to_dev(rw), to_dev(ri)
    out = torch.zeros((T, H), dtype=torch.float32, device="cuda:0")
    L = candle_moe.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    xp = ctypes.c_void_p(big.data_ptr() + 4)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.candle_moe_fused_moe_status(xp, p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k, O.SILU,
                                       O.QWEN3, O.F32, stream)
    candle_moe.check(rc)
    torch.cuda.synchronize()
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.F32, mode=O.MODE_EXACT)
    assert_close(from_dev(out).astype(np.float64), want, RTOL[O.F32], "unaligned f32")


@pytest.mark.parametrize("tile", [1, 5, 7, 12, 14])
@pytest.mark.parametrize("combine", [1, 2])
def test_tile_configs(tile, combine):
    # both MFMA block tiles on both combine paths, ragged groups and column tails
    try:
        candle_moe.set_tile_policy(tile)
        candle_moe.set_combine_policy(combine)
        check_case(3000, 320, 200, 8, 2, O.BF16, O.QWEN3, seed=40 + tile, rows=list(range(0, 3000, 37)))
        check_case(2500, 264, 448, 6, 2, O.F16, O.NOMIC, act=O.GELU, seed=41 + tile, rows=list(range(0, 2500, 41)))
        check_case(700, 128, 64, 8, 1, O.BF16, O.QWEN3, seed=42 + tile)
    finally:
        candle_moe.set_tile_policy(0)
        candle_moe.set_combine_policy(0)


@pytest.mark.parametrize("T", [8, 1024])
def test_step_replayed_from_a_cuda_graph(T):
    """topk_softmax + FusedMoE.forward captured once in a torch CUDA graph (a
    HIP graph) and replayed: the library allocates nothing once its per-stream
    workspace exists (the capture stream is warmed eagerly first) and makes no
    host synchronisation, so the step captures; every replay equals the eager
    result bit for bit (k = 2: deterministic), with eager work of the same
    library on another stream between the replays, and the eager result
    itself matches the oracle."""
    import torch

    H, I, E, k, dt = 512, 256, 8, 2, O.BF16
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 5, O.QWEN3)
    logits = torch.from_numpy(O.randn((T, E), seed=6, stream=1)).to("cuda:0")
    tx, tg, tu, td = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt), to_dev(D, dt)
    tw = torch.empty((T, k), dtype=torch.float32, device="cuda:0")
    ti = torch.empty((T, k), dtype=torch.int32, device="cuda:0")
    te = torch.empty((T, k), dtype=torch.int32, device="cuda:0")
    moe = candle_moe.FusedMoE.new(E, k, candle_moe.Activation.Silu)

    def step():
        candle_moe.apply_topk_softmax_inplace(logits, tw, ti, te)
        return moe.forward(tx, tg, tu, td, tw, ti, 0)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ref = step().clone()
        ref_w, ref_i = tw.clone(), ti.clone()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = O.fused_moe(x, G, U, D, from_dev(ref_w), from_dev(ref_i).astype(np.uint32), E=E, k=k, act=O.SILU,
                       moe_type=O.QWEN3, dtype=dt, mode=O.MODE_F32ACC)
    assert_close(from_dev(ref).astype(np.float64), want, RTOL[dt], "eager step")

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out = step()
    other_w = torch.from_numpy(rw).to("cuda:0")
    other_i = torch.from_numpy(ri.astype(np.int32)).to("cuda:0")
    for _ in range(3):
        eager = moe.forward(tx, tg, tu, td, other_w, other_i, 0)  # default stream, its own workspace
        torch.cuda.synchronize()
        out.zero_()
        tw.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert torch.equal(tw, ref_w) and torch.equal(ti, ref_i)
        assert torch.isfinite(eager.float()).all()


@pytest.mark.parametrize("offset", [0, 1, 4])
def test_pair_path_output_alignment(offset):
    """The pair path's finalize reads and writes the caller's output 8
    elements at a time when it is 16-byte aligned, one at a time otherwise
    (an output that starts 2 or 8 bytes into an allocation): same result,
    accumulated into the caller's values."""
    import torch

    T, H, I, E, k, dt = 48, 136, 64, 4, 2, O.BF16
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 21, O.QWEN3)
    init = O.round_to(O.randn((T, H), seed=22), dt)
    buf = torch.zeros(T * H + 8, dtype=torch.bfloat16, device="cuda:0")
    out = buf[offset:offset + T * H].view(T, H)
    out.copy_(torch.from_numpy(init.astype(np.float32)).to("cuda:0").to(torch.bfloat16))
    L = candle_moe.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    tx, tg, tu, td = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt), to_dev(D, dt)
    trw, tri = to_dev(rw), to_dev(ri)
    assert candle_moe.fused_moe_path(T, H, I, E, k, dt) == "pairs"
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    candle_moe.check(L.candle_moe_fused_moe_status(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k,
                                                   O.SILU, O.QWEN3, dt, stream))
    torch.cuda.synchronize()
    want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=dt,
                       mode=O.MODE_EXACT) + init.astype(np.float64)
    assert_close(from_dev(out).astype(np.float64), want, RTOL[dt], f"output offset {offset}")
    # the elements around the output are untouched
    assert float(buf[:offset].abs().sum()) == 0.0 and float(buf[offset + T * H:].abs().sum()) == 0.0


# ---- pair path on the prefill kernels with k = 4: each pair's weighted row is
# stored once and a token's k rows are summed (no atomics)
@pytest.mark.gpu
@pytest.mark.parametrize("dt, mt, act", [(O.BF16, O.QWEN3, O.SILU), (O.F16, O.NOMIC, O.GELU)])
def test_pair_rows_four_experts_per_token(dt, mt, act):
    T, H, I, E, k = 2048, 128, 64, 16, 4
    assert candle_moe.fused_moe_path(T, H, I, E, k, dt) == "pairs"
    assert candle_moe.fused_moe_kernel(T, H, I, E, k, dt) != 12  # not the 32-row decode kernel
    check_case(T, H, I, E, k, dt, mt, act=act, seed=71, rows=list(range(0, T, 61)))


# ---- the drop-in fused_moe symbol adds into the caller's output
# (/root/reference/src/ffi.rs:35, lib.rs:296): accumulate mode on every
# prefill path, checked against the oracle started from the same output
def run_raw_accumulate(x, G, U, D, rw, ri, E, k, act, moe_type, dt, rows, seed, offset=0, workspace=False):
    """fused_moe (or candle_moe_fused_moe_ws) into an output that already
    holds N(0,1) values and starts `offset` elements into its allocation.
    Returns (output rows, their values before the call)."""
    import torch

    T, H = x.shape
    I = G.shape[2]
    tx, tg, tu = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt)
    td = None if D is None else to_dev(D, dt)
    trw, tri = to_dev(rw), to_dev(ri)
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(seed)
    buf = torch.randn(T * H + 8, generator=gen, device="cuda:0").to(tx.dtype)
    out = buf[offset:offset + T * H].view(T, H)
    ridx = torch.tensor(rows, dtype=torch.long, device="cuda:0")
    init = from_dev(out.index_select(0, ridx)).astype(np.float64)
    around = torch.cat([buf[:offset], buf[offset + T * H:]]).clone()
    L = candle_moe.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if workspace:
        n = L.candle_moe_fused_moe_workspace_size(T, H, I, E, k, dt)
        ws = torch.empty(n + 256, dtype=torch.uint8, device="cuda:0")
        base = (ws.data_ptr() + 255) // 256 * 256
        candle_moe.check(L.candle_moe_fused_moe_ws(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E,
                                                   k, act, moe_type, dt, ctypes.c_void_p(base), n, stream))
    else:
        L.fused_moe(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k, act, moe_type, dt, stream)
        assert candle_moe.last_error() == "", candle_moe.last_error()
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([buf[:offset], buf[offset + T * H:]]), around), "elements around the output changed"
    return from_dev(out.index_select(0, ridx)).astype(np.float64), init


ACC_CASES = [
    # id, T, H, I, E, k, dtype, moe_type, act, zipf, expected (path, kernel, pair rows), forced combine
    ("qwen3_sets_w8", 4096, 512, 256, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, ("expert-set", 7, False), 2),
    ("nomic_sets_w8_f16", 4096, 256, 192, 8, 2, O.F16, O.NOMIC, O.GELU, 0.0, ("expert-set", 7, False), 2),
    ("nomic_T4096_pair_rows_w8", 4096, 768, 3072, 8, 2, O.BF16, O.NOMIC, O.GELU, 0.0, ("pairs", 7, True), 0),
    ("q30b_T4096_pair_rows_o2", 4096, 2048, 768, 128, 8, O.BF16, O.QWEN3, O.SILU, 1.1, ("pairs", 14, True), 0),
    ("small_pair_rows_k4", 2048, 128, 64, 16, 4, O.BF16, O.QWEN3, O.SILU, 0.0, ("pairs", 7, True), 0),
    ("small_pair_rows_k4_f16", 2048, 128, 64, 16, 4, O.F16, O.NOMIC, O.GELU, 0.0, ("pairs", 7, True), 0),
    ("nomic_T512_f32_tile128", 512, 768, 3072, 8, 2, O.F32, O.NOMIC, O.GELU, 0.0, ("simt", 16, False), 0),
    ("qwen3_f32_tile128", 1024, 256, 128, 8, 2, O.F32, O.QWEN3, O.SILU, 0.0, ("simt", 16, False), 0),
]


def check_accumulate(T, H, I, E, k, dt, mt, act, zipf, expect, combine, seed, rows, offset=0, workspace=False):
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, seed, mt, zipf_s=zipf)
    if isinstance(rows, str) and rows == "tiles":
        rows = covering_rows(T, H, I, E, k, dt, mt, ri, extra=SAMPLE)
    try:
        candle_moe.set_combine_policy(combine)
        path, kernel, pair_rows = expect
        if offset % 8 == 0:
            assert candle_moe.fused_moe_path(T, H, I, E, k, dt, mt) == path
        assert candle_moe.fused_moe_kernel(T, H, I, E, k, dt, mt) == kernel
        assert candle_moe.fused_moe_pair_rows(T, H, I, E, k, dt, mt) == pair_rows
        got, init = run_raw_accumulate(x, G, U, D, rw, ri, E, k, act, mt, dt, rows, seed + 1000, offset, workspace)
    finally:
        candle_moe.set_combine_policy(candle_moe.COMBINE_AUTO)
    kw = dict(E=E, k=k, act=act, moe_type=mt, dtype=dt, rows=rows, out_init=init)
    name = f"accumulate T={T} H={H} I={I} E={E} k={k} dt={dt} type={mt} offset={offset}"
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw), RTOL[dt], name + " vs f32acc + init")
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw), RTOL[dt], name + " vs exact + init")
    # the caller's values were added, not dropped: without them the result is far off
    without = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **dict(kw, out_init=None))
    assert float(np.abs(got - without).max()) > 0.5


@pytest.mark.parametrize("case", ACC_CASES, ids=[c[0] for c in ACC_CASES])
@pytest.mark.parametrize("api", ["raw", "ws"])
def test_accumulate_mode_prefill_paths(case, api):
    _, T, H, I, E, k, dt, mt, act, zipf, expect, combine = case
    rows = sorted(set(range(0, T, max(1, T // 97))) | {T - 1})
    check_accumulate(T, H, I, E, k, dt, mt, act, zipf, expect, combine, seed=90 + len(case[0]), rows=rows,
                     workspace=(api == "ws"))


@pytest.mark.parametrize("offset", [1, 4])
def test_accumulate_pair_rows_unaligned_output(offset):
    # an output that is not 16-byte aligned: the token-row sum reads and
    # writes it one element at a time (pair_rows_sum_kernel)
    T, H, I, E, k = 2048, 128, 64, 16, 4
    check_accumulate(T, H, I, E, k, O.BF16, O.QWEN3, O.SILU, 0.0, ("pairs", 7, True), 0, seed=97,
                     rows=list(range(0, T, 23)), offset=offset)


@pytest.mark.parametrize("offset", [1, 4])
def test_accumulate_unaligned_output_leaves_expert_sets(offset):
    # the expert-set down GEMM stores straight into the output with 8-byte
    # stores; an output off a 16-byte boundary takes the pair path instead
    T, H, I, E, k = 4096, 512, 256, 8, 2
    check_accumulate(T, H, I, E, k, O.BF16, O.QWEN3, O.SILU, 0.0, ("expert-set", 7, False), 2, seed=98,
                     rows=list(range(0, T, 41)), offset=offset)


@pytest.mark.slow
def test_accumulate_headline_shape_tile_rows():
    # Qwen3 T=32768 bf16 through the drop-in symbol: the expert-set path with
    # the 8-wave 256x256 kernel, adding into the caller's output
    check_accumulate(32768, 4096, 1536, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, ("expert-set", 7, False), 0, seed=99,
                     rows="tiles")


def test_unaligned_16bit_operands_take_the_scalar_kernel():
    # 16-byte loads need aligned operands: an input 2 bytes off takes moe_simt_gemm
    import torch

    T, H, I, E, k, dt = 96, 128, 64, 8, 2, O.BF16
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 84, O.QWEN3)
    big = torch.zeros(T * H + 8, dtype=torch.bfloat16, device="cuda:0")
    big[1:1 + T * H] = to_dev(x, dt).reshape(-1)
    tg, tu, td, trw, tri = to_dev(G, dt), to_dev(U, dt), to_dev(D, dt), to_dev(rw), to_dev(ri)
    out = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda:0")
    L = candle_moe.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.candle_moe_fused_moe_status(ctypes.c_void_p(big.data_ptr() + 2), p(tg), p(tu), p(td), p(trw), p(tri),
                                       p(out), T, H, I, E, k, O.SILU, O.QWEN3, dt, stream)
    candle_moe.check(rc)
    torch.cuda.synchronize()
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=dt)
    got = from_dev(out).astype(np.float64)
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_F32ACC, **kw), RTOL[dt], "unaligned bf16 f32acc")
    assert_close(got, O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw), RTOL[dt], "unaligned bf16 exact")
