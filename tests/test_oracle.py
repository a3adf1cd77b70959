"""Pins the CPU oracle (CPU only, no GPU).

Each oracle function is checked against something independent of its own
formula: published known-answer vectors, numpy float64 evaluations,
closed-form special cases, brute force, invariants, and the committed
golden fixtures (tests/golden/). A planted mistake (dropped term, wrong
index, transposed operand, reciprocal instead of divide) fails at least
one check here.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import moe_inputs, router_inputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------ RNG
def test_philox_known_answers():
    # Random123 kat_vectors for philox4x32_10 (Salmon et al., SC11)
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert list(O.philox4x32_10(ctr, key)) == want


def test_randn_distribution_and_determinism():
    a = O.randn((1 << 20,), seed=123)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    assert np.array_equal(a, O.randn((1 << 20,), seed=123))
    assert not np.array_equal(a[:1000], O.randn((1000,), seed=123, stream=1))
    b = O.randn((1000,), seed=5, mean=2.0, std=0.02)
    assert abs(b.mean() - 2.0) < 5e-3 and abs(b.std() - 0.02) < 2e-3


# ---------------------------------------------------------- conversions
def test_f16_conversion_matches_numpy():
    v = np.concatenate([O.randn((100000,), seed=1) * s for s in (1e-6, 1e-3, 1.0, 1e3, 7e4)]).astype(np.float32)
    v = np.concatenate([v, np.float32([0.0, -0.0, 65504, 65519.99, 65520, 6e-8, 2.98e-8, 3e-8, np.inf, -np.inf])])
    got = O.to_dtype(v, O.F16)
    want = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(O.to_f32(got, O.F16), want.view(np.float16).astype(np.float32))


def test_bf16_conversion_round_to_nearest_even():
    v = np.concatenate([O.randn((100000,), seed=2) * s for s in (1e-30, 1.0, 1e30)]).astype(np.float32)
    u = v.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(O.to_dtype(v, O.BF16), want)
    # ties: 1 + 2^-8 is halfway between two bf16 values and rounds to even (1.0)
    t = np.float32([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8])
    assert list(O.to_f32(O.to_dtype(t, O.BF16), O.BF16)) == [1.0, 1.0 + 2.0 ** -6]


# --------------------------------------------------------------- router
def f64_router(g, k):
    p = np.exp(g.astype(np.float64) - g.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    order = np.argsort(-p, axis=1, kind="stable")[:, :k]
    return np.take_along_axis(p, order, 1), order


@pytest.mark.parametrize("T,E,k", [(32, 8, 2), (4096, 64, 6), (2048, 128, 8), (100, 256, 16), (50, 3, 2)])
def test_router_against_float64(T, E, k):
    g = router_inputs(T, E, seed=E)
    w, i, ei = O.topk_softmax(g, k)
    pw, pi = f64_router(g, k)
    assert np.array_equal(i, pi.astype(np.uint32))
    # f32 ops on the way (x - max, exp, sum, divide) keep it well inside 1e-6
    assert np.max(np.abs(w - pw) / pw) < 1e-6
    assert np.array_equal(ei, (np.arange(k)[None, :] * T + np.arange(T)[:, None]).astype(np.uint32))
    assert (np.diff(w, axis=1) <= 0).all()
    assert (np.sort(i, axis=1)[:, 1:] != np.sort(i, axis=1)[:, :-1]).all()


def test_router_literal_f32_softmax_agrees():
    # candle's CPU softmax as written (expf, sequential f32 sum) selects the same experts
    g = router_inputs(32768, 64, seed=77)
    w, i, _ = O.topk_softmax(g, 6)
    w2, i2, _ = O.topk_softmax(g, 6, literal=True)
    assert np.array_equal(i, i2)
    assert np.max(np.abs(w - w2) / w) < 1e-6


def test_router_special_cases():
    # E = 1: the single expert with probability 1
    w, i, ei = O.topk_softmax(np.float32([[0.3], [-5.0]]), 1)
    assert (w == 1.0).all() and (i == 0).all() and list(ei[:, 0]) == [0, 1]
    # equal logits: p = 1/E, indices 0..k-1 (ties to the lower index)
    w, i, _ = O.topk_softmax(np.full((3, 8), 1.7, np.float32), 3)
    assert (w == np.float32(1 / 8)).all() and (i == np.arange(3)).all()
    # k = E is a full stable argsort
    g = router_inputs(64, 16, seed=3)
    _, i, _ = O.topk_softmax(g, 16)
    assert np.array_equal(i, np.argsort(-g, axis=1, kind="stable").astype(np.uint32))
    # a planted tie between experts 6 and 2 resolves to 2 first
    g = np.zeros((1, 8), np.float32)
    g[0, [6, 2]] = 4.0
    _, i, _ = O.topk_softmax(g, 2)
    assert list(i[0]) == [2, 6]
    with pytest.raises(ValueError):
        O.topk_softmax(g, 9)


def test_router_large_spread_underflow():
    g = np.float32([[0.0, -200.0, -90.0, 10.0]])
    w, i, _ = O.topk_softmax(g, 4)
    assert list(i[0]) == [3, 0, 2, 1]
    assert w[0, 0] == np.float32(1.0 / (1.0 + np.exp(-10.0)))


# ------------------------------------------------------------- grouping
def brute_group(idx, w, E):
    T, k = idx.shape
    rows = [[] for _ in range(E)]
    for p in range(T * k):
        e = int(idx.flat[p])
        if e < E:
            rows[e].append(p)
    off = np.zeros(E + 2, np.int32)
    s = 0
    for e in range(E):
        off[e] = s
        s += len(rows[e])
    off[E] = s
    off[E + 1] = max((len(r) for r in rows), default=0)
    sp = np.array([p for r in rows for p in r], np.int32)
    return off, sp


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (300, 8, 2), (1000, 128, 8), (77, 3, 3)])
def test_grouping_brute_force(T, E, k):
    _, idx, _ = O.topk_softmax(router_inputs(T, E, seed=T), k)
    w = O.randn((T, k), seed=9)
    off, st, sw, sp = O.preprocess(idx, w, E)
    boff, bsp = brute_group(idx, w, E)
    assert np.array_equal(off, boff)
    assert np.array_equal(sp, bsp)
    assert np.array_equal(st, bsp // k)
    assert np.array_equal(sw, w.reshape(-1)[bsp])
    assert (np.diff(off[: E + 1]) >= 0).all() and off[E] == T * k


def test_grouping_drops_out_of_range_experts():
    idx = np.array([[0, 5], [7, 1], [5, 5]], np.uint32)
    off, st, sw, sp = O.preprocess(idx, np.ones((3, 2), np.float32), 6)
    assert off[6] == 5 and off[7] == 3  # pair (1,0) -> expert 7 dropped; expert 5 has 3 pairs
    assert list(sp) == [0, 3, 1, 4, 5]


# ------------------------------------------------------------------ MoE
def np_moe(x, G, U, D, w, idx, act, moe_type):
    """float64 numpy restatement, one (token, slot) at a time."""
    T, H = x.shape
    out = np.zeros((T, H))
    f = {O.SILU: lambda v: v / (1 + np.exp(-v)),
         O.GELU: lambda v: 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3))),
         O.RELU: lambda v: np.maximum(v, 0)}[act]
    for t in range(T):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e >= G.shape[0]:
                continue
            h = f(x[t] @ G[e])
            if moe_type == O.QWEN3:
                y = (h * (x[t] @ U[e])) @ D[e]
            else:
                y = U[e] @ h  # up[e] is [H, I]: y = h . up^T
            out[t] += w[t, j] * y
    return out


@pytest.mark.parametrize("moe_type", [O.QWEN3, O.NOMIC])
@pytest.mark.parametrize("act", [O.SILU, O.GELU, O.RELU])
@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
def test_moe_exact_against_numpy(moe_type, act, dt):
    T, H, I, E, k = 21, 40, 24, 5, 2
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 7, moe_type, wstd=0.2)
    f = lambda a: None if a is None else O.to_f32(a, dt).astype(np.float64)  # noqa: E731
    want = np_moe(f(x), f(G), f(U), f(D), rw.astype(np.float64), ri, act, moe_type)
    kw = dict(E=E, k=k, act=act, moe_type=moe_type, dtype=dt)
    got = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw)
    assert np.max(np.abs(got - want)) < 1e-12 * max(1.0, np.abs(want).max())
    # rounded modes stay within the dtype tolerance of the exact result
    rtol = {O.F32: 1e-4, O.F16: 1e-2, O.BF16: 2e-2}[dt]
    rms = np.sqrt(np.mean(want ** 2))
    for mode in (O.MODE_F32ACC, O.MODE_CANDLE):
        r = O.fused_moe(x, G, U, D, rw, ri, mode=mode, **kw)
        assert np.linalg.norm(r - want) <= rtol * np.linalg.norm(want)
        if mode == O.MODE_F32ACC:
            assert (np.abs(r - want) <= rtol * (rms + np.abs(want))).all()


def test_moe_one_hot_is_dense_mlp():
    # every token routed to expert 2 with weight 1: a plain dense SwiGLU MLP
    T, H, I, E = 9, 32, 16, 4
    x, G, U, D, _, _ = moe_inputs(T, H, I, E, 1, O.F32, 8, O.QWEN3, wstd=0.3)
    idx = np.full((T, 1), 2, np.uint32)
    w = np.ones((T, 1), np.float32)
    got = O.fused_moe(x, G, U, D, w, idx, E=E, k=1, act=O.SILU, moe_type=O.QWEN3, dtype=O.F32, mode=O.MODE_EXACT)
    xd, g2, u2, d2 = (a.astype(np.float64) for a in (x, G[2], U[2], D[2]))
    a = xd @ g2
    want = ((a / (1 + np.exp(-a))) * (xd @ u2)) @ d2
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    # a transposed operand would not match: Nomic uses up^T
    got_n = O.fused_moe(x, G, U, None, w, idx, E=E, k=1, act=O.RELU, moe_type=O.NOMIC, dtype=O.F32,
                        mode=O.MODE_EXACT)
    assert np.allclose(got_n, np.maximum(xd @ g2, 0) @ u2.T, rtol=1e-12, atol=1e-12)


def test_moe_linear_in_routing_weights_and_rows():
    T, H, I, E, k = 30, 48, 32, 6, 3
    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.F32, 9, O.QWEN3, wstd=0.2)
    kw = dict(E=E, k=k, act=O.SILU, moe_type=O.QWEN3, dtype=O.F32, mode=O.MODE_EXACT)
    a = O.fused_moe(x, G, U, D, rw, ri, **kw)
    b = O.fused_moe(x, G, U, D, 2 * rw, ri, **kw)
    assert np.allclose(b, 2 * a, rtol=1e-12, atol=1e-12)
    rows = [0, 7, 29]
    c = O.fused_moe(x, G, U, D, rw, ri, rows=rows, **kw)
    assert np.array_equal(c, a[rows])
    with pytest.raises(ValueError, match="distinct"):   # one output row per token
        O.fused_moe(x, G, U, D, rw, ri, rows=[0, 7, 7], **kw)
    init = O.randn((T, H), seed=4).astype(np.float64)
    d = O.fused_moe(x, G, U, D, rw, ri, out_init=init, **kw)
    assert np.allclose(d, a + init, rtol=1e-12, atol=1e-12)


def test_moe_combine_order_is_expert_ascending():
    # candle's index_add visits experts in ascending order: with bf16 per-op
    # rounding, out = rnd(rnd(y_lo) + rnd(y_hi)); check on one token
    T, H, I, E = 1, 16, 8, 4
    x, G, U, D, _, _ = moe_inputs(T, H, I, E, 2, O.BF16, 10, O.QWEN3, wstd=0.5)
    w = np.float32([[0.6, 0.4]])
    i1 = np.array([[3, 1]], np.uint32)
    i2 = np.array([[1, 3]], np.uint32)
    w2 = np.float32([[0.4, 0.6]])
    kw = dict(E=E, k=2, act=O.SILU, moe_type=O.QWEN3, dtype=O.BF16)
    assert np.array_equal(O.fused_moe(x, G, U, D, w, i1, **kw), O.fused_moe(x, G, U, D, w2, i2, **kw))


# ------------------------------------------------------------- golden
def test_golden_fixtures_reproduce():
    files = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert files, "no golden fixtures"
    for f in files:
        z = np.load(os.path.join(GOLDEN, f), allow_pickle=False)
        kind = str(z["kind"])
        if kind == "router":
            w, i, ei = O.topk_softmax(z["logits"], int(z["k"]))
            assert np.array_equal(w, z["topk_weight"]) and np.array_equal(i, z["topk_indices"])
            assert np.array_equal(ei, z["token_expert_indices"])
        else:
            dt = int(z["dtype"])
            down = z["down"] if z["down"].size else None
            got = O.fused_moe(z["x"], z["gate"], z["up"], down, z["routing_weights"], z["expert_indices"],
                              E=int(z["E"]), k=int(z["k"]), act=int(z["act"]), moe_type=int(z["moe_type"]),
                              dtype=dt, mode=O.MODE_F32ACC)
            assert np.array_equal(got, z["out_f32acc"]), f
            ex = O.fused_moe(z["x"], z["gate"], z["up"], down, z["routing_weights"], z["expert_indices"],
                             E=int(z["E"]), k=int(z["k"]), act=int(z["act"]), moe_type=int(z["moe_type"]),
                             dtype=dt, mode=O.MODE_EXACT)
            assert np.allclose(ex, z["out_exact"], rtol=1e-12, atol=1e-12), f


@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
def test_router_logits_one_hot_and_scaling(dt):
    # a one-hot row h picks column h of every expert's weight row: logits[t, e]
    # = w[e, h_t] (already dtype values), which the transposed product fails;
    # twice the row gives twice the logits (exact in every dtype)
    T, H, E = 24, 40, 6
    rng = np.random.default_rng(5)
    w = O.to_dtype(rng.standard_normal((E, H)).astype(np.float32), dt)
    h = rng.integers(0, H, T)
    x1 = np.zeros((T, H), np.float32)
    x1[np.arange(T), h] = 1.0
    got = O.router_logits(O.to_dtype(x1, dt), w, dt)
    wf = O.to_f32(w, dt)
    assert np.array_equal(got, wf[:, h].T)
    got2 = O.router_logits(O.to_dtype(2 * x1, dt), w, dt)
    assert np.array_equal(got2, 2 * wf[:, h].T)


def test_router_logits_round_once_to_dtype():
    # sums of exactly representable products: the exact sum, rounded once
    x = np.array([[1.0, 1.0 / 512.0, 1.0 / 512.0]], np.float32)
    w = np.array([[1.0, 1.0, 1.0]], np.float32)
    # 1 + 2^-8 is a bf16 tie (ulp 2^-7 at 1): round to even -> 1.0
    got = O.router_logits(O.to_dtype(x, O.BF16), O.to_dtype(w, O.BF16), O.BF16)
    assert got[0, 0] == 1.0
    # f32 keeps it
    got = O.router_logits(x, w, O.F32)
    assert got[0, 0] == np.float32(1.0 + 2.0 ** -8)


def test_tile_covering_rows_brute_force():
    """The tests' restatement of the grouping's row order and tile edges
    (tests/helpers.py) against a hand-built table on a tiny routing."""
    from helpers import _tile_edges, pair_order, set_order, tile_covering_rows

    ri = np.array([[1, 0], [0, 1], [2, 0], [1, 1], [9, 0], [0, 2], [2, 1]], dtype=np.uint32)  # E = 3, 9 dropped
    E = 3
    order, counts = pair_order(ri, E)
    # pair ids by expert, ascending inside an expert
    assert order.tolist() == [1, 2, 5, 9, 10] + [0, 3, 6, 7, 13] + [4, 11, 12]
    assert counts.tolist() == [5, 5, 3]
    # sets (sorted, dropped -> 3), keys base 4: t0 {0,1}=1 t1 {0,1}=1 t2 {0,2}=2 t3 {1,1}=5
    # t4 {0,3}=3 t5 {0,2}=2 t6 {1,2}=6
    torder, kcounts = set_order(ri, E)
    assert torder.tolist() == [0, 1, 2, 5, 4, 3, 6]
    assert kcounts.tolist() == [2, 2, 1, 1, 1]
    # edges: runs of 5 with BM = 4 -> tile [0,4) halves [0,2) [2,4), tile [4,5)
    assert sorted(set(_tile_edges([5], 4))) == [0, 1, 2, 3, 4]
    assert sorted(set(_tile_edges([5, 3], 8))) == [0, 3, 4, 5, 7]
    assert sorted(set(_tile_edges([10], 4))) == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9]
    assert sorted(set(_tile_edges([10], 8))) == [0, 3, 4, 7, 8, 9]
    # BM = 8 over the pairs: edges 0,3,4 of e0 -> pairs 1,9,10; of e1 -> 0,7,13; e2 (3 rows) 0,2 -> 4,12
    assert tile_covering_rows(ri, E, 8, "pairs") == sorted({1 // 2, 9 // 2, 10 // 2, 0, 7 // 2, 13 // 2, 2, 6})
    # the set order adds the first and last token of each set group
    assert set(tile_covering_rows(ri, E, 8, "expert-set")) == \
        set(tile_covering_rows(ri, E, 8, "pairs")) | {0, 1, 2, 5, 4, 3, 6}
