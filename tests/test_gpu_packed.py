"""Pre-packed 16-bit expert weights (candle_moe_pack_weights,
candle_moe_fused_moe_packed): every weight matrix K-contiguous, [E][N][K].

* pack_weights is the exact transpose (bit for bit, tile tails included);
* fused_moe_packed gives the bits of fused_moe on the API layout: the GEMMs
  feed the matrix cores the same operands in the same K order, only read
  differently (ds_read_b128 of K-contiguous rows instead of transposed LDS
  reads; whole operands loaded straight from memory at decode sizes), on the
  decode kernels, the 32-row, 128x128, 128x256 and 256x256 kernels, the pair
  and expert-set paths, with the output added into;
* and it matches the CPU oracle (tolerances as tests/test_gpu_moe.py).
"""
import ctypes

import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, assert_close, from_dev, moe_inputs, to_dev

pytestmark = pytest.mark.gpu


def run_both(T, H, I, E, k, dt, mt, act, seed, zipf=0.0, tile=0, combine=0):
    import torch

    x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, seed, mt, zipf_s=zipf)
    tx, tg, tu = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt)
    td = None if D is None else to_dev(D, dt)
    trw, tri = to_dev(rw), to_dev(ri)
    init = O.round_to(O.randn((T, H), seed=seed + 1), dt).astype(np.float64)
    outs = []
    try:
        candle_moe.set_tile_policy(tile)
        candle_moe.set_combine_policy(combine)
        for packed in (False, True):
            out = torch.from_numpy(init.astype(np.float32)).to("cuda:0").to(tx.dtype)
            if packed:
                gp = candle_moe.pack_weights(tg)
                up = candle_moe.pack_weights(tu) if mt == O.QWEN3 else tu  # Nomic fc2 is [E,H,I] already
                dp = candle_moe.pack_weights(td) if mt == O.QWEN3 else None
                candle_moe.fused_moe_packed(tx, gp, up, dp, trw, tri, out, E, k, act, mt)
            else:
                L = candle_moe.lib()
                p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
                stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                candle_moe.check(L.candle_moe_fused_moe_status(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out),
                                                               T, H, I, E, k, act, mt, dt, stream))
            torch.cuda.synchronize()
            outs.append(from_dev(out).astype(np.float64))
    finally:
        candle_moe.set_tile_policy(0)
        candle_moe.set_combine_policy(0)
    return (x, G, U, D, rw, ri, init), outs


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("E,K,N", [(3, 4096, 1536), (2, 72, 200), (1, 64, 64), (5, 130, 66)])
def test_pack_is_the_exact_transpose(dt, E, K, N):
    import torch

    w = to_dev(O.to_dtype(O.randn((E, K, N), seed=K + N), dt), dt)
    got = candle_moe.pack_weights(w)
    assert got.shape == (E, N, K)
    assert torch.equal(got, w.transpose(1, 2).contiguous())


CASES = [
    # T, H, I, E, k, dtype, moe_type, act, zipf, tile, combine
    (8, 4096, 1536, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 0, 0),       # decode kernels
    (1, 2048, 768, 128, 8, O.BF16, O.QWEN3, O.SILU, 1.1, 0, 0),
    (16, 768, 3072, 8, 2, O.F16, O.NOMIC, O.GELU, 0.0, 0, 0),
    (16, 512, 1504, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 0, 0),       # 48-column blocks, column tail
    (16, 256, 3024, 8, 2, O.BF16, O.NOMIC, O.GELU, 0.0, 0, 0),       # 96-column blocks, column tail
    (64, 1024, 512, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 12, 0),      # 32-row kernel
    (64, 768, 3072, 8, 2, O.BF16, O.NOMIC, O.GELU, 0.0, 12, 0),
    (512, 1024, 512, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 5, 0),      # 128x128
    (1024, 2048, 768, 64, 4, O.BF16, O.QWEN3, O.SILU, 0.0, 14, 0),   # 128x256, two per CU
    (2048, 1024, 768, 8, 2, O.F16, O.QWEN3, O.SILU, 0.0, 7, 1),      # 256x256, pair rows
    (4096, 512, 256, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 7, 2),      # 256x256, expert sets
    (4096, 256, 192, 8, 2, O.F16, O.NOMIC, O.GELU, 0.0, 7, 2),
    (3000, 320, 200, 8, 2, O.BF16, O.QWEN3, O.SILU, 0.0, 0, 0),      # ragged tails
    (128, 128, 64, 4096, 8, O.BF16, O.QWEN3, O.SILU, 0.0, 18, 0),   # decode kernels: 1024 pairs, 4096 experts
]


@pytest.mark.parametrize("T,H,I,E,k,dt,mt,act,zipf,tile,combine", CASES)
def test_packed_equals_api_layout_and_oracle(T, H, I, E, k, dt, mt, act, zipf, tile, combine):
    (x, G, U, D, rw, ri, init), (api, packed) = run_both(T, H, I, E, k, dt, mt, act, 800 + T, zipf, tile, combine)
    assert np.array_equal(api, packed), "packed weights changed the result"
    rows = None if T <= 1024 else sorted(set(range(0, T, 29)) | {T - 1})
    kw = dict(E=E, k=k, act=act, moe_type=mt, dtype=dt, rows=rows,
              out_init=init if rows is None else init[np.asarray(rows)])
    want = O.fused_moe(x, G, U, D, rw, ri, mode=O.MODE_EXACT, **kw)
    got = packed if rows is None else packed[np.asarray(rows)]
    assert_close(got, want, RTOL[dt], f"packed T={T} H={H} I={I} E={E} k={k} vs f64 oracle")


@pytest.mark.slow
def test_packed_headline_shape():
    T, H, I, E, k = 32768, 4096, 1536, 8, 2
    (x, G, U, D, rw, ri, init), (api, packed) = run_both(T, H, I, E, k, O.BF16, O.QWEN3, O.SILU, 830)
    assert np.array_equal(api, packed)


def test_packed_rejects_f32():
    import torch

    T, H, I, E, k = 4, 64, 32, 4, 2
    x = torch.zeros(T, H, device="cuda:0")
    with pytest.raises(candle_moe.CandleMoeError) as e:
        candle_moe.fused_moe_packed(x, torch.zeros(E, I, H, device="cuda:0"), torch.zeros(E, I, H, device="cuda:0"),
                                    torch.zeros(E, H, I, device="cuda:0"), torch.zeros(T, k, device="cuda:0"),
                                    torch.zeros(T, k, dtype=torch.int32, device="cuda:0"), torch.zeros_like(x), E, k)
    assert e.value.code == candle_moe.CANDLE_MOE_ERR_UNSUPPORTED
