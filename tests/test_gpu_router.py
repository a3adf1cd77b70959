"""Router GEMM fused with topk-softmax (candle_moe_router_topk) on the GPU.

The fused op computes logits = dtype(hidden @ router_weight.T) with f32
accumulation and feeds them to the same softmax / top-k as topk_softmax.

* Exact cases: inputs k/8 and j/64 (small integers over powers of two), so
  every product and every partial sum is exact in f32 and the GPU's
  accumulation order cannot matter: indices and token_expert_indices must be
  bit-exact and weights within 1e-6 relative of the oracle (router_logits,
  then topk_softmax). The discrete values also produce tied logits, which
  exercise the lower-index tie rule.
* Random normal cases: logits within the f32 accumulation error of a dtype
  rounding point may round either way; tokens with such a logit (or with a
  top-k margin inside that error, for f32) are set aside, must be few, and
  every other token must match as above.
"""
import ctypes

import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import from_dev, to_dev

pytestmark = pytest.mark.gpu


def run_fused(x, w, k, dt):
    import torch

    T, E = x.shape[0], w.shape[0]
    xt, wt = to_dev(x, dt), to_dev(w, dt)
    tw = torch.full((T, k), -7.0, dtype=torch.float32, device="cuda:0")
    ti = torch.full((T, k), -1, dtype=torch.int32, device="cuda:0")
    te = torch.full((T, k), -1, dtype=torch.int32, device="cuda:0")
    candle_moe.router_topk(xt, wt, tw, ti, te)
    torch.cuda.synchronize()
    return from_dev(tw), from_dev(ti).astype(np.uint32), from_dev(te).astype(np.uint32)


def quantized(shape, denom, seed):
    rng = np.random.default_rng(seed)
    return (rng.integers(-8, 9, shape) / denom).astype(np.float32)


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
@pytest.mark.parametrize("T,H,E,k", [(1000, 4096, 8, 2), (333, 768, 8, 2), (129, 2048, 128, 8), (77, 1024, 64, 6),
                                     (50, 512, 16, 4), (40, 256, 32, 3), (9, 64, 5, 5),
                                     # 16-bit E > 32 (matrix cores): 32 tokens per workgroup below
                                     # 16384 tokens, 64 from there; H tails inside a K tile of 64
                                     (8200, 512, 128, 8), (8200, 1000, 40, 3), (300, 1000, 96, 4), (1, 2048, 128, 8),
                                     (16400, 256, 128, 8), (16400, 264, 40, 2)])
def test_router_topk_exact(dt, T, H, E, k):
    x = O.to_dtype(quantized((T, H), 8.0, T + H), dt)
    w = O.to_dtype(quantized((E, H), 64.0, E + k), dt)
    gw, gi, ge = run_fused(x, w, k, dt)
    ww, wi, we = O.topk_softmax(O.router_logits(x, w, dt), k)
    assert np.array_equal(gi, wi)
    assert np.array_equal(ge, we)
    np.testing.assert_allclose(gw, ww, rtol=1e-6, atol=0)


@pytest.mark.parametrize("dt", [O.BF16, O.F32])
def test_router_topk_random_normal(dt):
    T, H, E, k = 4096, 2048, 8, 2
    rng = np.random.default_rng(9)
    xf = rng.standard_normal((T, H)).astype(np.float32)
    wf = (0.02 * rng.standard_normal((E, H))).astype(np.float32)
    x, w = O.to_dtype(xf, dt), O.to_dtype(wf, dt)
    gw, gi, ge = run_fused(x, w, k, dt)
    # The GPU's f32 sums may differ from the exact ones by accumulation
    # roundoff; a logit whose exact value lies within that distance of a dtype
    # rounding point may round either way. err: 16 roundoff units of the sum
    # of magnitudes (the worst case of the GPU's 32 + 64 term summation is 96;
    # the kernel is deterministic, so a bound that holds once holds always).
    x64, w64 = O.to_f32(x, dt).astype(np.float64), O.to_f32(w, dt).astype(np.float64)
    exact = x64 @ w64.T
    err = 16 * 2.0 ** -24 * (np.abs(x64) @ np.abs(w64).T)
    near = O.round_to(exact.astype(np.float32), dt)
    lo = O.round_to((exact - err).astype(np.float32), dt)
    hi = O.round_to((exact + err).astype(np.float32), dt)
    n_amb = (lo != hi).sum(axis=1)
    if dt == O.F32:
        # f32 logits are not rounded: instead a near-tie inside the error can
        # reorder the top k
        srt = np.sort(exact, axis=1)[:, ::-1]
        n_amb = n_amb * 0 + 2 * ((srt[:, :k] - srt[:, 1:k + 1]).min(axis=1) < 2 * err.max(axis=1))
    cands = [O.topk_softmax(c, k) for c in (near, lo, hi)]
    checked = 0
    for t in range(T):
        if n_amb[t] >= 2:
            continue
        ok = [np.array_equal(gi[t], c[1][t]) and np.allclose(gw[t], c[0][t], rtol=2e-5 if dt == O.F32 else 1e-6, atol=0)
              for c in (cands if n_amb[t] else cands[:1])]
        assert any(ok), (t, gi[t], cands[0][1][t], gw[t], cands[0][0][t])
        checked += 1
    assert checked > 0.8 * T, checked
    assert np.array_equal(ge, cands[0][2])


def test_router_topk_errors():
    import torch

    L = candle_moe.lib()
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device="cuda:0")
    w = torch.zeros((200, 64), dtype=torch.bfloat16, device="cuda:0")
    out = torch.zeros((4, 2), dtype=torch.float32, device="cuda:0")
    idx = torch.zeros((4, 2), dtype=torch.int32, device="cuda:0")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.candle_moe_router_topk(p(x), p(w), p(out), p(idx), p(idx), 4, 64, 200, 2, O.BF16, s) != 0
    assert "num_experts" in candle_moe.last_error()
    assert L.candle_moe_router_topk(p(x), p(w), p(out), p(idx), p(idx), 4, 60, 8, 2, O.BF16, s) != 0
    assert "multiple of 8" in candle_moe.last_error()
    xo = ctypes.c_void_p(x.data_ptr() + 2)
    assert L.candle_moe_router_topk(xo, p(w), p(out), p(idx), p(idx), 2, 64, 8, 2, O.BF16, s) != 0
    assert "aligned" in candle_moe.last_error()
    assert L.candle_moe_router_topk(p(x), p(w), p(out), p(idx), p(idx), 4, (1 << 22) + 8, 8, 2, O.BF16, s) != 0
    assert "4194304" in candle_moe.last_error()
    assert L.candle_moe_router_topk(p(x), p(w), p(out), p(idx), p(idx), 0, 64, 8, 2, O.BF16, s) == 0


def test_router_partials_leave_the_workspace_counters_alone():
    # the small-batch router writes f32 partials into the same per-stream
    # workspace whose header holds the one-launch grouping's counters (zero
    # between calls): a prefill call with that grouping and a decode call
    # right after it must still match the oracle and their caller-workspace
    # runs bit for bit
    from test_gpu_moe import run_raw

    x = O.to_dtype(quantized((16, 2048), 8.0, 3), O.BF16)
    w = O.to_dtype(quantized((128, 2048), 64.0, 4), O.BF16)
    for _ in range(3):
        gw, gi, ge = run_fused(x, w, 8, O.BF16)
    ww, wi, we = O.topk_softmax(O.router_logits(x, w, O.BF16), 8)
    assert np.array_equal(gi, wi)
    from helpers import RTOL, assert_close, moe_inputs
    for n, (T, H, I, E, k) in enumerate([(3000, 256, 128, 8, 2), (8, 1024, 512, 8, 2)]):
        xs, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, O.BF16, 780 + n, O.QWEN3)
        run_fused(x, w, 8, O.BF16)  # partials just before the call
        a = run_raw(xs, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16)
        b = run_raw(xs, G, U, D, rw, ri, E, k, O.SILU, O.QWEN3, O.BF16, workspace=True)
        assert np.array_equal(a, b), f"case {n}: owned workspace differs from a caller workspace"
        rows = np.arange(0, T, max(1, T // 40))
        want = O.fused_moe(xs[rows], G, U, D, rw[rows], ri[rows], E=E, k=k, act=O.SILU, moe_type=O.QWEN3,
                           dtype=O.BF16, mode=O.MODE_F32ACC)
        assert_close(a[rows], want, RTOL[O.BF16], f"case {n}")


_REFUSED = []  # the graph of the refused capture, kept until the process ends


def test_router_small_batches_replayed_from_cuda_graphs():
    """The small-batch router (K split over workgroups, f32 partials in the
    per-stream library workspace) in torch CUDA graphs captured on a stream
    warmed by eager calls of the same sizes: every replay equals the eager
    result bit for bit, with eager work between replays, also from a second
    graph captured after the first one is destroyed (the workspace stays the
    eager one). A call captured on a stream without a workspace is refused
    before anything is enqueued."""
    import torch

    H, E, k, dt = 2048, 128, 8, O.BF16
    w = O.to_dtype(quantized((E, H), 64.0, 11), dt)
    xn = [O.to_dtype(quantized((T, H), 8.0, 20 + T), dt) for T in (1, 16, 128)]
    wt = to_dev(w, dt)
    xs = [to_dev(x, dt) for x in xn]
    outs = [tuple(torch.full((x.shape[0], k), -1, dtype=d, device="cuda:0")
                  for d in (torch.float32, torch.int32, torch.int32)) for x in xs]

    def calls():
        for x, (tw, ti, te) in zip(xs, outs):
            candle_moe.router_topk(x, wt, tw, ti, te)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.synchronize()
    ref = [tuple(t.clone() for t in o) for o in outs]
    for x, (rw, ri, re) in zip(xn, ref):
        ww, wi, we = O.topk_softmax(O.router_logits(x, w, dt), k)
        assert np.array_equal(from_dev(ri).astype(np.uint32), wi)
        assert np.array_equal(from_dev(re).astype(np.uint32), we)
        np.testing.assert_allclose(from_dev(rw), ww, rtol=1e-6, atol=0)
    for _ in range(2):  # the second graph is captured after the first is destroyed
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            calls()
        for _ in range(3):
            for o in outs:
                for t in o:
                    t.fill_(-1)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for o, r in zip(outs, ref):
                assert all(torch.equal(a, b) for a, b in zip(o, r))
        del graph
    # the FusedMoE forward (fused_moe's workspace) is refused the same way
    from helpers import moe_inputs

    xm, G, U, D, rwm, rim = moe_inputs(8, 256, 128, 8, 2, dt, 5, O.QWEN3)
    moe_args = [to_dev(a, dt) for a in (xm, G, U, D)] + [to_dev(rwm), to_dev(rim)]
    moe = candle_moe.FusedMoE.new(8, 2, candle_moe.Activation.Silu)
    fresh = torch.cuda.Stream()
    pad = torch.zeros(4, device="cuda:0")
    refused = torch.cuda.CUDAGraph()
    with torch.cuda.graph(refused, stream=fresh):
        pad.add_(1.0)
        with pytest.raises(candle_moe.CandleMoeError, match="being captured") as err:
            candle_moe.router_topk(xs[1], wt, *outs[1])
        assert err.value.code == candle_moe.CANDLE_MOE_ERR_WORKSPACE
        with pytest.raises(candle_moe.CandleMoeError, match="being captured") as err:
            moe.forward(*moe_args, O.QWEN3)
        assert err.value.code == candle_moe.CANDLE_MOE_ERR_WORKSPACE
    _REFUSED.append(refused)
