"""Token->expert grouping on the GPU (candle_moe_group_pairs, the grouping
fused_moe runs; the reference's preprocessing, kernels/preprocessing.cuh:5-313)
against the oracle's counting sort (oracle.preprocess) and the invariants of
the survey's parity plan: offsets monotone, offsets[E] = valid pairs,
offsets[E+1] = largest count, every valid pair exactly once, stable order
(ascending pair id inside an expert), out-of-range expert ids dropped. Sizes
cover the one-workgroup path (up to 2048 pairs) and the three-launch path,
skewed and empty experts, and a single pair."""
import numpy as np
import pytest

import candle_moe
import oracle as O

pytestmark = pytest.mark.gpu


def brute(idx: np.ndarray, E: int):
    valid = idx < E
    counts = np.bincount(idx[valid], minlength=E)[:E]
    offsets = np.concatenate([[0], np.cumsum(counts)[:-1]]) if E > 0 else np.zeros(0)
    order = np.argsort(np.where(valid, idx, E), kind="stable")[: int(valid.sum())]
    return counts, offsets, order


@pytest.mark.parametrize("P,E,drop,skew", [(1, 8, 0.0, 0.0), (100, 8, 0.05, 0.0), (2048, 128, 0.02, 1.1),
                                           (2049, 8, 0.0, 0.0), (65536, 8, 0.01, 0.0), (70001, 128, 0.03, 1.1),
                                           (40000, 4096, 0.0, 0.0), (5000, 3, 0.5, 0.0)])
def test_grouping_matches_counting_sort(P, E, drop, skew):
    import torch

    rng = np.random.default_rng(P + E)
    if skew:
        p = np.arange(1, E + 1, dtype=np.float64) ** -skew
        idx = rng.choice(E, size=P, p=p / p.sum()).astype(np.uint32)
    else:
        idx = rng.integers(0, E, size=P).astype(np.uint32)
    bad = rng.random(P) < drop
    idx[bad] = E + rng.integers(0, 7, size=int(bad.sum())).astype(np.uint32)  # out-of-range ids
    t = torch.from_numpy(idx.view(np.int32)).to("cuda:0")
    off, srt = candle_moe.group_pairs(t, E)
    torch.cuda.synchronize()
    off = off.cpu().numpy().astype(np.int64)
    srt = srt.cpu().numpy().astype(np.int64)
    counts, offsets, order = brute(idx, E)
    nvalid = int(counts.sum())
    assert np.array_equal(off[:E], offsets)
    assert off[E] == nvalid and off[E + 1] == int(counts.max())
    assert np.all(np.diff(off[: E + 1]) >= 0)
    assert np.array_equal(srt[:nvalid], order), "grouped pairs differ from a stable counting sort"
    # the oracle's restatement of the reference preprocessing (a stable
    # counting sort; the reference's own order inside an expert is unspecified)
    # agrees, pairs read as [T, k] with k = 2 where P is even
    k = 2 if P % 2 == 0 else 1
    w = rng.random(P).astype(np.float32)
    o_off, o_tok, o_w, o_pair = O.preprocess(idx.reshape(P // k, k), w.reshape(P // k, k), E)
    assert np.array_equal(o_off, off[: E + 2])
    assert np.array_equal(o_pair, srt[:nvalid])
    assert np.array_equal(o_tok, srt[:nvalid] // k) and np.array_equal(o_w, w[srt[:nvalid]])


def test_grouping_rejections():
    import ctypes
    import torch

    L = candle_moe.lib()
    t = torch.zeros(16, dtype=torch.int32, device="cuda:0")
    o = torch.zeros(10, dtype=torch.int32, device="cuda:0")
    p = lambda x: ctypes.c_void_p(x.data_ptr())  # noqa: E731
    n = L.candle_moe_grouping_workspace_size(16, 8)
    ws = torch.zeros(n + 256, dtype=torch.uint8, device="cuda:0")
    base = ctypes.c_void_p((ws.data_ptr() + 255) // 256 * 256)
    assert L.candle_moe_group_pairs(p(t), 16, 8, p(o), p(t), base, n - 1, None) == candle_moe.CANDLE_MOE_ERR_WORKSPACE
    assert L.candle_moe_group_pairs(p(t), 16, 0, p(o), p(t), base, n, None) == candle_moe.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_group_pairs(p(t), 0, 8, p(o), p(t), base, n, None) == candle_moe.CANDLE_MOE_OK
    torch.cuda.synchronize()
    assert o[8].item() == 0 and o[9].item() == 0
