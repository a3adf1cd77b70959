"""CPU oracle for the candle-moe hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package. It is the checker, never the thing measured or
shipped: the product (``candle_moe`` + ``libcandle_moe_hip.so``) does not
import it and has no CPU fallback.

ctypes bindings over ``liboracle.so`` (built from oracle.c by oracle/Makefile).
Each function restates the reference's candle-native semantics; oracle.h
lists the reference file:line each one follows and the check that pins it.
Parity unpinned: the per-op f16/bf16 rounding sequence of candle's CPU ops
and its matmul accumulation order (no reference vector exists for them).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F16, BF16, F32 = 0, 1, 2
SILU, GELU, RELU = 0, 1, 2
QWEN3, NOMIC = 0, 1
MODE_CANDLE, MODE_EXACT, MODE_F32ACC = 0, 1, 2


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i32, u64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_float
        L.om_philox4x32_10.argtypes = [vp, vp, vp]
        L.om_fill_normal.argtypes = [vp, ctypes.c_size_t, u64, u64, f32, f32]
        L.om_f32_to_dtype.argtypes = [vp, vp, ctypes.c_size_t, i32]
        L.om_dtype_to_f32.argtypes = [vp, vp, ctypes.c_size_t, i32]
        for fn in (L.om_topk_softmax, L.om_topk_softmax_f32lit):
            fn.argtypes = [vp, i32, i32, i32, vp, vp, vp]
            fn.restype = i32
        L.om_preprocess.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp]
        L.om_fused_moe.argtypes = [vp] * 8 + [i32] * 9 + [vp, i32, i32]
        L.om_fused_moe.restype = i32
        L.om_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.om_e4m3_decode.restype = f32
        L.om_e4m3_encode.argtypes = [f32]
        L.om_e4m3_encode.restype = ctypes.c_uint8
        L.om_quantize_fp8.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp]
        L.om_dequantize_fp8.argtypes = [vp, vp, ctypes.c_size_t, i32, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().om_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def randn(shape, seed: int, stream: int = 0, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Seeded f32 normals (Philox4x32-10 + Box-Muller)."""
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    lib().om_fill_normal(_p(out), n, seed, stream, mean, std)
    return out.reshape(shape)


_NP16 = {F16: np.uint16, BF16: np.uint16}


def to_dtype(a: np.ndarray, dtype: int) -> np.ndarray:
    """f32 -> storage of dtype (f16/bf16 as raw uint16 bits; f32 copy)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype == F32:
        return a.copy()
    out = np.empty(a.shape, dtype=np.uint16)
    lib().om_f32_to_dtype(_p(a), _p(out), a.size, dtype)
    return out


def to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if dtype == F32:
        return a.astype(np.float32)
    out = np.empty(a.shape, dtype=np.float32)
    lib().om_dtype_to_f32(_p(a), _p(out), a.size, dtype)
    return out


def round_to(a: np.ndarray, dtype: int) -> np.ndarray:
    """Round f32 values to dtype precision and return them as f32."""
    return to_f32(to_dtype(a, dtype), dtype)


def topk_softmax(logits: np.ndarray, k: int, literal: bool = False):
    """Router oracle. Returns (topk_weight f32 [T,k], topk_indices u32 [T,k],
    token_expert_indices u32 [T,k])."""
    g = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = g.shape
    w = np.zeros((T, k), np.float32)
    i = np.zeros((T, k), np.uint32)
    ei = np.zeros((T, k), np.uint32)
    fn = lib().om_topk_softmax_f32lit if literal else lib().om_topk_softmax
    rc = fn(_p(g), T, E, k, _p(w), _p(i), _p(ei))
    if rc != 0:
        raise ValueError(f"invalid router sizes T={T} E={E} k={k}")
    return w, i, ei


def router_logits(x: np.ndarray, w: np.ndarray, dtype: int) -> np.ndarray:
    """Router logits as candle's Linear in `dtype` produces them for the
    callers of topk_softmax (/root/reference/README.md:61-71 usage: logits
    from a separate matmul, then apply_topk_softmax_inplace): x [T,H] and
    w [E,H] (Linear layout) as dtype storage; the products summed exactly (f64
    here; f32 accumulation on the GPU agrees wherever the f32 sum is exact),
    rounded once to dtype, returned as f32 [T,E]. Pinned in
    tests/test_oracle.py by one-hot rows (logit = the weight column, which a
    transposed operand fails) and scaling."""
    xf = to_f32(x, dtype).astype(np.float64)
    wf = to_f32(w, dtype).astype(np.float64)
    return round_to((xf @ wf.T).astype(np.float32), dtype)


def preprocess(idx: np.ndarray, w: np.ndarray, E: int):
    """Grouping oracle: (offsets[E+2], sorted_tok, sorted_w, sorted_pair)."""
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    T, k = idx.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    off = np.zeros(E + 2, np.int32)
    n = T * k
    st = np.full(n, -1, np.int32)
    sw = np.zeros(n, np.float32)
    sp = np.full(n, -1, np.int32)
    lib().om_preprocess(_p(idx), _p(w), T, k, E, _p(off), _p(st), _p(sw), _p(sp))
    valid = int(off[E])
    return off, st[:valid], sw[:valid], sp[:valid]


def fused_moe(x, gate, up, down, w, idx, *, E: int, k: int, act: int, moe_type: int,
              dtype: int, mode: int = MODE_CANDLE, rows=None, out_init=None,
              nthreads: int = 0) -> np.ndarray:
    """MoE oracle. x/gate/up/down are storage arrays of `dtype` (uint16 bits
    for f16/bf16, float32 for f32). Returns float64 [T or len(rows), H]."""
    x = np.ascontiguousarray(x)
    T, H = x.shape
    I = gate.shape[2]
    gate = np.ascontiguousarray(gate)
    up = np.ascontiguousarray(up)
    down = None if down is None else np.ascontiguousarray(down)
    w = np.ascontiguousarray(w, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    if r is not None and len(np.unique(r)) != len(r):
        raise ValueError("fused_moe: rows must be distinct (the C oracle fills one output row per token)")
    nr = T if r is None else len(r)
    out = np.zeros((nr, H), np.float64)
    oi = None if out_init is None else np.ascontiguousarray(out_init, dtype=np.float64)
    rc = lib().om_fused_moe(_p(x), _p(gate), _p(up), _p(down), _p(w), _p(idx), _p(oi), _p(out),
                            T, H, I, E, k, act, moe_type, dtype, mode, _p(r), nr, nthreads)
    if rc != 0:
        raise ValueError(f"om_fused_moe rejected its arguments (code {rc})")
    return out


def e4m3_decode(codes) -> np.ndarray:
    """Exact f32 values of e4m3 codes (NaN for 0x7F / 0xFF)."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    return np.array([lib().om_e4m3_decode(int(v)) for v in c.ravel()], np.float32).reshape(c.shape)


def e4m3_encode(x) -> np.ndarray:
    """Nearest e4m3 codes of f32 values (ties to even, saturating at 448)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    return np.array([lib().om_e4m3_encode(float(v)) for v in a.ravel()], np.uint8).reshape(a.shape)


def quantize_fp8(w: np.ndarray, dtype: int, kn: bool = True):
    """FP8 weight format: w [E,K,N] (kn) or [E,N,K] storage of dtype ->
    (codes [E,N,K] u8, scales [E,N] f32)."""
    w = np.ascontiguousarray(w)
    E = w.shape[0]
    K, N = (w.shape[1], w.shape[2]) if kn else (w.shape[2], w.shape[1])
    q = np.empty((E, N, K), np.uint8)
    s = np.empty((E, N), np.float32)
    lib().om_quantize_fp8(_p(w), dtype, E, K, N, 1 if kn else 0, _p(q), _p(s))
    return q, s


def dequantize_fp8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """decode(q) * s as f32 [E,N,K]."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    out = np.empty(q.shape, np.float32)
    lib().om_dequantize_fp8(_p(q), _p(s), s.size, q.shape[-1], _p(out))
    return out
