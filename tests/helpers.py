"""Shared test helpers: seeded inputs, host<->device moves, tolerance checks."""
from __future__ import annotations

import numpy as np

import oracle as O

# MoE output tolerances (north star): rtol per dtype, atol = rtol * RMS(expected)
RTOL = {O.F32: 1e-4, O.F16: 1e-2, O.BF16: 2e-2}


def torch_dtype(dt):
    import torch

    return {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}[dt]


def to_dev(a: np.ndarray, dt=None, dev="cuda:0"):
    """numpy storage array (uint16 bits for f16/bf16) -> torch tensor on dev."""
    import torch

    if dt in (O.F16, O.BF16):
        t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16))
        return t.view(torch_dtype(dt)).to(dev)
    if a.dtype == np.uint32:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def from_dev(t) -> np.ndarray:
    import torch

    if t.dtype in (torch.float16, torch.bfloat16):
        return t.float().cpu().numpy()
    return t.cpu().numpy()


def router_inputs(T: int, E: int, seed: int, skew_sigma: float = 0.0, zipf_s: float = 0.0):
    """Router logits f32 [T, E] ~ N(0,1), optionally plus a per-expert bias:
    N(0, skew_sigma) (skewed), or a Zipf(s) rank bias
    log(r^-s / sum r^-s) over a seeded permutation of ranks (config 5)."""
    g = O.randn((T, E), seed=seed)
    if skew_sigma:
        g = g + O.randn((E,), seed=seed, stream=1, std=skew_sigma)[None, :]
    if zipf_s:
        rng_key = O.randn((E,), seed=seed, stream=2)
        ranks = np.argsort(np.argsort(rng_key)) + 1  # seeded permutation of 1..E
        p = ranks.astype(np.float64) ** (-zipf_s)
        g = g + np.log(p / p.sum()).astype(np.float32)[None, :]
    return np.ascontiguousarray(g, dtype=np.float32)


def moe_inputs(T, H, I, E, k, dt, seed, moe_type, wstd=0.02, xstd=1.0, skew_sigma=0.0, zipf_s=0.0):
    """x [T,H], gate/up [E,H,I], down [E,I,H] (Qwen3) in the API layout,
    routing from the oracle router over seeded logits."""
    x = O.to_dtype(O.randn((T, H), seed=seed, stream=10, std=xstd), dt)
    G = O.to_dtype(O.randn((E, H, I), seed=seed, stream=11, std=wstd), dt)
    U = O.to_dtype(O.randn((E, H, I), seed=seed, stream=12, std=wstd), dt)
    D = O.to_dtype(O.randn((E, I, H), seed=seed, stream=13, std=wstd), dt) if moe_type == O.QWEN3 else None
    rw, ri, _ = O.topk_softmax(router_inputs(T, E, seed + 1, skew_sigma, zipf_s), k)
    return x, G, U, D, rw, ri


def assert_close_norm(got: np.ndarray, want: np.ndarray, rtol: float, what: str = ""):
    """Norm-wise check ||got - want||_2 <= rtol * ||want||_2 (used against the
    candle per-op-rounding path, whose own bf16 rounding of every
    intermediate is larger than rtol at points of cancellation)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    num = float(np.linalg.norm(got - want))
    den = float(np.linalg.norm(want))
    assert num <= rtol * den, f"{what}: relative L2 error {num / max(den, 1e-300):.3g} > {rtol}"


def assert_close(got: np.ndarray, want: np.ndarray, rtol: float, what: str = "", atol: float | None = None):
    """|got - want| <= atol + rtol * max(|got|, |want|)  (the reference's
    check, /root/reference/tests/moe_tests.rs:61-91), atol = rtol * RMS(want)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    if atol is None:
        atol = rtol * float(np.sqrt(np.mean(want ** 2))) if want.size else 0.0
    diff = np.abs(got - want)
    tol = atol + rtol * np.maximum(np.abs(got), np.abs(want))
    bad = diff > tol
    if bad.any():
        i = int(np.argmax(np.where(bad, diff - tol, -np.inf)))
        idx = np.unravel_index(i, got.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{got.size} elements out of tolerance (rtol={rtol}, atol={atol:.3g}); "
            f"worst at {idx}: got {got[idx]!r} want {want[idx]!r}")


def _tile_edges(group_sizes, BM: int):
    """Positions, in a list grouped into runs of group_sizes, of the rows at
    the edges of every BM-row tile and of its two BM/2-row halves (the 8-wave
    kernels' two wave rows): first and last row of each, clipped to the run."""
    pos = []
    start = 0
    for n in group_sizes:
        for t0 in range(start, start + n, BM):
            end = min(t0 + BM, start + n)
            for a in (t0, t0 + BM // 2):
                if a < end:
                    pos += [a, min(a + BM // 2, end) - 1]
        start += n
    return pos


def pair_order(ri: np.ndarray, E: int):
    """Pairs p = t*k + j grouped by expert, stable (ids >= E dropped), and
    the per-expert counts: the grouping's order for the pair GEMMs."""
    flat = ri.reshape(-1).astype(np.int64)
    pairs = np.nonzero(flat < E)[0]
    return pairs[np.argsort(flat[pairs], kind="stable")], np.bincount(flat[pairs], minlength=E)


def set_order(ri: np.ndarray, E: int):
    """Tokens grouped by expert set, stable: the key reads a token's ids
    sorted ascending (ids >= E as E) as base-(E+1) digits; returns the token
    order and the sizes of the nonempty groups in key order."""
    T, k = ri.shape
    ex = np.where(ri.astype(np.int64) < E, ri.astype(np.int64), E)
    digits = np.sort(ex, axis=1, kind="stable")
    key = np.zeros(T, dtype=np.int64)
    for j in range(k):
        key = key * (E + 1) + digits[:, j]
    torder = np.argsort(key, kind="stable")
    _, kcounts = np.unique(key[torder], return_counts=True)
    return torder, kcounts


def tile_covering_rows(ri: np.ndarray, E: int, BM: int, path: str) -> list:
    """Tokens whose rows sit at the first and last row of every row tile (and
    tile half) of the grouped GEMMs fused_moe runs on this routing, from the
    grouping's own order (a stable counting sort, as the oracle's
    om_preprocess): pairs p = t*k + j grouped by expert (gate/up / fc1, and
    the pair path's down / fc2); on the expert-set path also tokens grouped by
    their sorted expert set (the down / fc2 GEMM). Every output column of such
    a row is checked, so every (row tile, column tile) of every launch, K-split
    tiles included, is covered by a checked row."""
    k = ri.shape[1]
    order, counts = pair_order(ri, E)
    toks = set((order[_tile_edges(counts, BM)] // k).tolist())
    if path == "expert-set":
        torder, kcounts = set_order(ri, E)
        toks |= set(torder[_tile_edges(kcounts, BM)].tolist())
    return sorted(toks)
