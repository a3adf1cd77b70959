"""candle_moe_fused_moe_noalloc: fused_moe whose workspace is the library's
fixed device array (no allocation). Its output must equal that of
candle_moe_fused_moe_status on the same inputs, call after call, also when a
call follows a larger one that left its own data in the shared array."""
import ctypes

import numpy as np
import pytest

import candle_moe
import oracle as O
from helpers import RTOL, assert_close, from_dev, moe_inputs, to_dev

pytestmark = pytest.mark.gpu


def _call(fn, x, G, U, D, rw, ri, E, k, act, mt, dt, init):
    import torch

    T, H = x.shape
    I = G.shape[2]
    tx, tg, tu = to_dev(x, dt), to_dev(G, dt), to_dev(U, dt)
    td = None if D is None else to_dev(D, dt)
    trw, tri = to_dev(rw), to_dev(ri)
    out = torch.from_numpy(init.astype(np.float32)).to("cuda:0").to(tx.dtype)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    candle_moe.check(fn(p(tx), p(tg), p(tu), p(td), p(trw), p(tri), p(out), T, H, I, E, k, act, mt, dt, stream))
    torch.cuda.synchronize()
    return out


# (T, H, I, E, k, dtype, moe_type, act): batches of more than 2048 pairs (the
# multi-workgroup grouping, whose launches must not depend on what an earlier
# call left in the shared array), a prefill batch on the pair-row path, then
# decode batches on the decode kernels (their f32 partials and slice counts
# live in the shared array) and the f32 kernels, each smaller than the last
SEQUENCE = [
    (1100, 512, 256, 128, 2, O.BF16, O.QWEN3, O.SILU),
    (1536, 256, 128, 64, 2, O.F16, O.NOMIC, O.GELU),
    (512, 1024, 512, 8, 2, O.BF16, O.QWEN3, O.SILU),
    (64, 4096, 1536, 8, 2, O.BF16, O.QWEN3, O.SILU),
    (8, 4096, 1536, 8, 2, O.BF16, O.QWEN3, O.SILU),
    (16, 768, 3072, 8, 2, O.F16, O.NOMIC, O.GELU),
    (4, 768, 3072, 8, 2, O.F32, O.NOMIC, O.GELU),
]


def test_noalloc_matches_status_entry_point_call_after_call():
    L = candle_moe.lib()
    assert L.candle_moe_fused_moe_noalloc_scratch_bytes() == 32 << 20
    for n, (T, H, I, E, k, dt, mt, act) in enumerate(SEQUENCE):
        print(f"noalloc call {n}: T={T} H={H} I={I} E={E} k={k} dt={dt} moe_type={mt}", flush=True)
        need = L.candle_moe_fused_moe_workspace_size(T, H, I, E, k, dt)
        assert 0 < need <= 32 << 20, f"call {n} needs {need} bytes of scratch"
        x, G, U, D, rw, ri = moe_inputs(T, H, I, E, k, dt, 200 + n, mt)
        init = O.round_to(O.randn((T, H), seed=300 + n), dt).astype(np.float64)
        got = _call(L.candle_moe_fused_moe_noalloc, x, G, U, D, rw, ri, E, k, act, mt, dt, init)
        ref = _call(L.candle_moe_fused_moe_status, x, G, U, D, rw, ri, E, k, act, mt, dt, init)
        # same kernels on the same inputs, k = 2 (deterministic combine): bit for bit
        assert np.array_equal(from_dev(got), from_dev(ref)), f"call {n}: noalloc differs from the status entry point"
        want = O.fused_moe(x, G, U, D, rw, ri, E=E, k=k, act=act, moe_type=mt, dtype=dt, mode=O.MODE_F32ACC,
                           out_init=init)
        assert_close(from_dev(got).astype(np.float64), want, RTOL[dt], f"call {n} vs oracle")


def test_noalloc_rejects_calls_beyond_its_scratch():
    import torch

    L = candle_moe.lib()
    T, H, I, E, k = 8192, 4096, 1536, 8, 2
    buf = torch.zeros(256, dtype=torch.uint8, device="cuda:0")
    p = ctypes.c_void_p(buf.data_ptr())
    rc = L.candle_moe_fused_moe_noalloc(p, p, p, p, p, p, p, T, H, I, E, k, O.SILU, O.QWEN3, O.BF16, None)
    assert rc == candle_moe.CANDLE_MOE_ERR_WORKSPACE
    assert "holds 33554432" in candle_moe.last_error()
    torch.cuda.synchronize()
    assert int(buf.sum()) == 0  # nothing ran
