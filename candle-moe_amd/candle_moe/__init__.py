"""candle-moe for MI355X: Python mirror of the reference's Rust API.

The reference crate exposes (``/root/reference/src/lib.rs``)::

    apply_topk_softmax_inplace(gating_output, topk_weight, topk_indices, token_expert_indices)
    enum Activation { Silu, Gelu, Relu }
    FusedMoE::new(num_experts, num_selected_experts, activation)
    FusedMoE::forward(input, gate, up, down: Option, routing_weights, expert_indices, moe_type)

This module offers the same names, argument meaning and error behaviour over
torch tensors that live on the GPU (PyTorch is only the device-memory and
stream plumbing). Every call goes through the C ABI of
``libcandle_moe_hip.so`` (``include/candle_moe.h``); there is no CPU
fallback: without the built library every entry point raises.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Optional, Sequence

_HERE = os.path.dirname(os.path.abspath(__file__))
# CANDLE_MOE_LIB selects another build of the library (e.g. one compiled for
# profiling); by default the in-tree libcandle_moe_hip.so is loaded.
LIB_PATH = os.environ.get("CANDLE_MOE_LIB") or os.path.join(os.path.dirname(_HERE), "libcandle_moe_hip.so")

CANDLE_MOE_OK = 0
CANDLE_MOE_ERR_INVALID = 1
CANDLE_MOE_ERR_UNSUPPORTED = 2
CANDLE_MOE_ERR_HIP = 3
CANDLE_MOE_ERR_WORKSPACE = 4

# descriptor dtype codes (include/candle_moe.h CM_DT_*)
DT_F16, DT_BF16, DT_F32, DT_U32, DT_I64, DT_F64, DT_U8 = range(7)
MAX_RANK = 4


class CandleMoeError(RuntimeError):
    """A call was rejected or failed; ``code`` is the CANDLE_MOE_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class Activation(enum.IntEnum):
    """Activation codes of the reference (``/root/reference/src/lib.rs:157-172``)."""

    Silu = 0
    Gelu = 1
    Relu = 2

    def to_int(self) -> int:
        return int(self)


class CmTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MAX_RANK),
        ("strides", ctypes.c_int64 * MAX_RANK),
        ("device", ctypes.c_int32),
    ]


class CmFusedMoE(ctypes.Structure):
    _fields_ = [
        ("num_experts", ctypes.c_int64),
        ("num_selected_experts", ctypes.c_int64),
        ("activation", ctypes.c_int32),
    ]


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"candle_moe: {LIB_PATH} is missing; build it with `make -C candle-moe_amd` "
                "(or __graft_entry__.build()). There is no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, u32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t
        L.topk_softmax.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp]
        L.topk_softmax.restype = None
        L.candle_moe_topk_softmax_status.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp]
        L.candle_moe_topk_softmax_status.restype = i32
        L.candle_moe_topk_softmax_ex.argtypes = [vp, i32, vp, i32, vp, vp, i32, i32, i32, vp]
        L.candle_moe_topk_softmax_ex.restype = i32
        moe_args = [vp] * 7 + [i32] * 6 + [u32, u32]
        L.fused_moe.argtypes = moe_args + [vp]
        L.fused_moe.restype = None
        L.candle_moe_fused_moe_status.argtypes = moe_args + [vp]
        L.candle_moe_fused_moe_status.restype = i32
        L.candle_moe_fused_moe_workspace_size.argtypes = [i32] * 5 + [u32]
        L.candle_moe_fused_moe_workspace_size.restype = sz
        L.candle_moe_fused_moe_ws.argtypes = moe_args + [vp, sz, vp]
        L.candle_moe_fused_moe_ws.restype = i32
        L.candle_moe_fused_moe_noalloc.argtypes = moe_args + [vp]
        L.candle_moe_fused_moe_noalloc.restype = i32
        L.candle_moe_fused_moe_noalloc_scratch_bytes.argtypes = []
        L.candle_moe_fused_moe_noalloc_scratch_bytes.restype = sz
        L.candle_moe_pack_weights.argtypes = [vp, u32, i32, i32, i32, vp, vp]
        L.candle_moe_pack_weights.restype = i32
        L.candle_moe_fused_moe_packed.argtypes = moe_args + [vp]
        L.candle_moe_fused_moe_packed.restype = i32
        L.candle_moe_test_router_exp.argtypes = [u32, u32, vp, vp]
        L.candle_moe_test_router_exp.restype = i32
        L.candle_moe_quantize_fp8.argtypes = [vp, u32, i32, i32, i32, i32, vp, vp, vp]
        L.candle_moe_quantize_fp8.restype = i32
        L.candle_moe_dequantize_fp8.argtypes = [vp, vp, i32, i32, i32, vp, u32, vp]
        L.candle_moe_dequantize_fp8.restype = i32
        L.candle_moe_fused_moe_fp8.argtypes = [vp] * 4 + [vp] * 3 + [vp] * 3 + [i32] * 6 + [u32, u32, vp]
        L.candle_moe_fused_moe_fp8.restype = i32
        L.candle_moe_set_combine_policy.argtypes = [i32]
        L.candle_moe_set_combine_policy.restype = i32
        L.candle_moe_set_tile_policy.argtypes = [i32]
        L.candle_moe_set_tile_policy.restype = i32
        L.candle_moe_fused_moe_path.argtypes = [i32] * 5 + [u32]
        L.candle_moe_fused_moe_path.restype = i32
        L.candle_moe_fused_moe_path_ex.argtypes = [i32] * 5 + [u32, u32]
        L.candle_moe_fused_moe_path_ex.restype = i32
        L.candle_moe_profile_begin.argtypes = []
        L.candle_moe_profile_begin.restype = i32
        L.candle_moe_profile_begin_slots.argtypes = [u32]
        L.candle_moe_profile_begin_slots.restype = i32
        L.candle_moe_profile_end.argtypes = [vp, vp, i32]
        L.candle_moe_profile_end.restype = i32
        L.candle_moe_profile_slot_name.argtypes = [i32]
        L.candle_moe_profile_slot_name.restype = ctypes.c_char_p
        L.candle_moe_router_topk.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, u32, vp]
        L.candle_moe_router_topk.restype = i32
        L.candle_moe_grouping_workspace_size.argtypes = [i32, i32]
        L.candle_moe_grouping_workspace_size.restype = sz
        L.candle_moe_group_pairs.argtypes = [vp, i32, i32, vp, vp, vp, sz, vp]
        L.candle_moe_group_pairs.restype = i32
        L.candle_moe_trim_workspaces.argtypes = []
        L.candle_moe_trim_workspaces.restype = i32
        L.candle_moe_last_error.argtypes = []
        L.candle_moe_last_error.restype = ctypes.c_char_p
        L.candle_moe_version.argtypes = []
        L.candle_moe_version.restype = ctypes.c_char_p
        tp = ctypes.POINTER(CmTensor)
        L.candle_moe_apply_topk_softmax_inplace.argtypes = [tp, tp, tp, tp, vp]
        L.candle_moe_apply_topk_softmax_inplace.restype = i32
        L.candle_moe_validate_topk_softmax.argtypes = [tp, tp, tp, tp]
        L.candle_moe_validate_topk_softmax.restype = i32
        mp = ctypes.POINTER(CmFusedMoE)
        L.candle_moe_fused_moe_forward.argtypes = [mp, tp, tp, tp, tp, tp, tp, u32, tp, vp]
        L.candle_moe_fused_moe_forward.restype = i32
        L.candle_moe_validate_fused_moe.argtypes = [mp, tp, tp, tp, tp, tp, tp, u32, tp]
        L.candle_moe_validate_fused_moe.restype = i32
        _lib = L
    return _lib


def last_error() -> str:
    return lib().candle_moe_last_error().decode()


def check(code: int) -> None:
    if code != CANDLE_MOE_OK:
        raise CandleMoeError(code, last_error())


# ------------------------------------------------------------ descriptors
_DTYPE_CODES = None


def _dtype_codes() -> dict:
    global _DTYPE_CODES
    if _DTYPE_CODES is None:
        import torch

        m = {
            torch.float16: DT_F16,
            torch.bfloat16: DT_BF16,
            torch.float32: DT_F32,
            torch.int64: DT_I64,
            torch.float64: DT_F64,
            torch.uint8: DT_U8,
        }
        if hasattr(torch, "uint32"):
            m[torch.uint32] = DT_U32
        # int32 index tensors are taken as u32 bit patterns (torch's uint32
        # support is partial); values must be non-negative.
        m[torch.int32] = DT_U32
        _DTYPE_CODES = m
    return _DTYPE_CODES


def _torch_dtype_code(t) -> int:
    code = _dtype_codes().get(t.dtype)
    if code is None:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, f"dtype {t.dtype} is not supported")
    return code


def describe(t) -> CmTensor:
    """cm_tensor_t for a torch tensor (GPU tensors carry their ordinal).
    (Called for every tensor of every call: kept to a few attribute reads.)"""
    rank = t.dim()
    if rank > MAX_RANK:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, f"rank {rank} exceeds {MAX_RANK}")
    d = CmTensor()
    d.dtype = _torch_dtype_code(t)
    d.data = t.data_ptr() if t.numel() else None
    d.rank = rank
    if rank:
        d.dims[:rank] = t.shape
        d.strides[:rank] = t.stride()
    d.device = t.get_device()  # -1 for CPU tensors
    return d


def spec(shape: Sequence[int], dtype: int, device: int = 0, strides: Optional[Sequence[int]] = None) -> CmTensor:
    """A data-less descriptor, for the validation entry points."""
    d = CmTensor()
    d.data = None
    d.dtype = dtype
    d.rank = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i, (s, st) in enumerate(zip(shape, strides)):
        d.dims[i] = s
        d.strides[i] = st
    d.device = device
    return d


def _stream_for(t) -> Optional[int]:
    import torch

    if not t.is_cuda:
        return None
    return torch.cuda.current_stream(t.device).cuda_stream


# -------------------------------------------------------------- the API
def apply_topk_softmax_inplace(gating_output, topk_weight, topk_indices, token_expert_indices) -> None:
    """Router softmax + top-k written in place (``/root/reference/src/lib.rs:124-155``).

    gating_output [T, E]; topk_weight [T, k] of the same dtype (f32, f16 or
    bf16); topk_indices / token_expert_indices [T, k] u32 (int32 accepted).
    """
    g, w, i, ei = (describe(t) for t in (gating_output, topk_weight, topk_indices, token_expert_indices))
    check(lib().candle_moe_apply_topk_softmax_inplace(
        ctypes.byref(g), ctypes.byref(w), ctypes.byref(i), ctypes.byref(ei), _stream_for(gating_output)))


def group_pairs(expert_indices, num_experts: int):
    """Token->expert grouping as fused_moe runs it (candle_moe_group_pairs):
    expert_indices [T, k] (or flat) u32/i32 on the GPU -> (offsets [E+2] i32,
    sorted_pairs [T*k] i32). offsets is the exclusive scan of the per-expert
    counts with offsets[E] = valid pairs and offsets[E+1] = the largest count;
    the first offsets[E] sorted_pairs are the pair ids t*k+j, grouped by expert,
    ascending inside an expert; ids >= num_experts are dropped."""
    import torch

    idx = expert_indices.contiguous().view(-1)
    P = idx.numel()
    dev = idx.device
    offsets = torch.empty(num_experts + 2, dtype=torch.int32, device=dev)
    sorted_pairs = torch.empty(max(P, 1), dtype=torch.int32, device=dev)
    n = lib().candle_moe_grouping_workspace_size(P, num_experts)
    if n == 0:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "group_pairs: invalid sizes")
    ws = torch.empty(n + 256, dtype=torch.uint8, device=dev)
    base = (ws.data_ptr() + 255) // 256 * 256
    check(lib().candle_moe_group_pairs(ctypes.c_void_p(idx.data_ptr()), P, num_experts,
                                       ctypes.c_void_p(offsets.data_ptr()), ctypes.c_void_p(sorted_pairs.data_ptr()),
                                       ctypes.c_void_p(base), n, _stream_for(idx)))
    return offsets, sorted_pairs[:P]


def router_topk(hidden, router_weight, topk_weight, topk_indices, token_expert_indices) -> None:
    """Router GEMM fused with topk-softmax (an extension: the reference's
    callers compute ``hidden.matmul`` with candle, then call
    apply_topk_softmax_inplace). hidden [T, H] and router_weight [E, H] (Linear
    layout) of one dtype, contiguous; logits = dtype(hidden @ router_weight.T)
    with f32 accumulation; outputs as apply_topk_softmax_inplace with f32
    topk_weight [T, k]."""
    for t in (hidden, router_weight, topk_weight, topk_indices, token_expert_indices):
        if not t.is_contiguous():
            raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "router_topk: tensors must be contiguous")
    if router_weight.dtype != hidden.dtype or topk_weight.dtype.itemsize != 4:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "router_topk: router_weight must have hidden's dtype, "
                             "topk_weight must be f32")
    T, H = hidden.shape
    E, k = router_weight.shape[0], topk_weight.shape[1]
    if router_weight.shape[1] != H or tuple(topk_indices.shape) != (T, k) or \
            tuple(token_expert_indices.shape) != (T, k) or topk_weight.shape[0] != T:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "router_topk: shape mismatch")
    check(lib().candle_moe_router_topk(
        ctypes.c_void_p(hidden.data_ptr()), ctypes.c_void_p(router_weight.data_ptr()),
        ctypes.c_void_p(topk_weight.data_ptr()), ctypes.c_void_p(topk_indices.data_ptr()),
        ctypes.c_void_p(token_expert_indices.data_ptr()), T, H, E, k, _torch_dtype_code(hidden),
        _stream_for(hidden)))


def quantize_fp8(weights, input_kn: bool = True):
    """FP8 e4m3 codes and per-output-channel f32 scales of expert weights
    (candle_moe_quantize_fp8). weights [E, K, N] (input_kn, the reference's
    gate/up/fc1 layout) or [E, N, K] (down/fc2, already [E, H, I]), f32/f16/bf16,
    contiguous, on the GPU -> (codes [E, N, K] uint8, scales [E, N] f32) with
    weights[e, k, n] ~ decode(codes[e, n, k]) * scales[e, n]."""
    import torch

    if not weights.is_contiguous() or weights.dim() != 3:
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "quantize_fp8: weights must be contiguous [E, K, N] or [E, N, K]")
    E = weights.shape[0]
    K, N = (weights.shape[1], weights.shape[2]) if input_kn else (weights.shape[2], weights.shape[1])
    codes = torch.empty((E, N, K), dtype=torch.uint8, device=weights.device)
    scales = torch.empty((E, N), dtype=torch.float32, device=weights.device)
    check(lib().candle_moe_quantize_fp8(ctypes.c_void_p(weights.data_ptr()), _torch_dtype_code(weights), E, K, N,
                                        1 if input_kn else 0, ctypes.c_void_p(codes.data_ptr()),
                                        ctypes.c_void_p(scales.data_ptr()), _stream_for(weights)))
    return codes, scales


def dequantize_fp8(codes, scales, dtype):
    """decode(codes) * scales as [E, N, K] of torch dtype (candle_moe_dequantize_fp8)."""
    import torch

    E, N, K = codes.shape
    if tuple(scales.shape) != (E, N) or scales.dtype != torch.float32 or not codes.is_contiguous() \
            or not scales.is_contiguous():
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "dequantize_fp8: codes [E, N, K] u8 and scales [E, N] f32")
    out = torch.empty((E, N, K), dtype=dtype, device=codes.device)
    check(lib().candle_moe_dequantize_fp8(ctypes.c_void_p(codes.data_ptr()), ctypes.c_void_p(scales.data_ptr()),
                                          E, N, K, ctypes.c_void_p(out.data_ptr()), _torch_dtype_code(out),
                                          _stream_for(codes)))
    return out


def fused_moe_fp8(input, gate_q, up_q, down_q, gate_scale, up_scale, down_scale, routing_weights, expert_indices,
                  output, num_experts: int, top_k: int, activation: int = 0, moe_type: int = 0) -> None:
    """output += MoE of input over fp8 expert weights (candle_moe_fused_moe_fp8).
    Qwen3 (moe_type 0): gate_q/up_q [E, I, H] u8 with scales [E, I], down_q
    [E, H, I] with down_scale [E, H]. Nomic (moe_type 1, fc1 / fc2 in gate /
    up as for fused_moe): gate_q = fc1 [E, I, H] with gate_scale [E, I], up_q =
    fc2 [E, H, I] with up_scale [E, H] (down_q and down_scale None).
    input/output [T, H] f16 or bf16; routing_weights
    [T, k] f32; expert_indices [T, k] u32/i32. Every tensor must be
    contiguous and on input's device; the codes are uint8 and the scales f32
    of the shapes above (the C entry point takes raw pointers and cannot check
    them), else CandleMoeError."""
    import torch

    def bad(msg):
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "fused_moe_fp8: " + msg)

    if input.dim() != 2 or gate_q.dim() != 3:
        bad("input must be [T, H] and gate_q [E, I, H]")
    T, H = input.shape
    E, I = num_experts, gate_q.shape[1]
    qwen3 = moe_type == 0
    codes = {"gate_q": (gate_q, (E, I, H)), "up_q": (up_q, (E, I, H) if qwen3 else (E, H, I))}
    scales = {"gate_scale": (gate_scale, (E, I)), "up_scale": (up_scale, (E, I) if qwen3 else (E, H))}
    if qwen3:
        codes["down_q"] = (down_q, (E, H, I))
        scales["down_scale"] = (down_scale, (E, H))
    elif down_q is not None or down_scale is not None:
        bad("Nomic (moe_type 1) takes no down_q / down_scale")
    rest = {"routing_weights": (routing_weights, (T, top_k)), "expert_indices": (expert_indices, (T, top_k)),
            "output": (output, (T, H))}
    for group, dtypes in ((codes, (torch.uint8,)), (scales, (torch.float32,)),
                          ({"routing_weights": rest["routing_weights"]}, (torch.float32,)),
                          ({"expert_indices": rest["expert_indices"]}, (torch.int32, torch.uint32)),
                          ({"output": rest["output"]}, (input.dtype,))):
        for name, (t, shape) in group.items():
            if t is None:
                bad(f"{name} is missing")
            if tuple(t.shape) != tuple(shape):
                bad(f"{name} must be {list(shape)}, got {list(t.shape)}")
            if t.dtype not in dtypes:
                bad(f"{name} must be {' or '.join(str(d) for d in dtypes)}, got {t.dtype}")
            if not t.is_contiguous():
                bad(f"{name} must be contiguous")
            if t.device != input.device:
                bad(f"{name} must be on {input.device}, got {t.device}")
    if not input.is_contiguous():
        bad("input must be contiguous")
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    check(lib().candle_moe_fused_moe_fp8(
        p(input), p(gate_q), p(up_q), p(down_q), p(gate_scale), p(up_scale), p(down_scale), p(routing_weights),
        p(expert_indices), p(output), T, H, I, num_experts, top_k, activation, moe_type,
        _torch_dtype_code(input), _stream_for(input)))


def pack_weights(weights):
    """Pre-packed (K-contiguous) form of 16-bit expert weights
    (candle_moe_pack_weights): weights [E, K, N] f16/bf16, contiguous, on the
    GPU -> a new [E, N, K] tensor of the same dtype (gate/up/fc1 [E, H, I] ->
    [E, I, H]; down [E, I, H] -> [E, H, I])."""
    import torch

    if weights.dim() != 3 or not weights.is_contiguous() or weights.dtype not in (torch.float16, torch.bfloat16):
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "pack_weights: weights must be contiguous f16/bf16 [E, K, N]")
    E, K, N = weights.shape
    out = torch.empty((E, N, K), dtype=weights.dtype, device=weights.device)
    check(lib().candle_moe_pack_weights(ctypes.c_void_p(weights.data_ptr()), _torch_dtype_code(weights), E, K, N,
                                        ctypes.c_void_p(out.data_ptr()), _stream_for(weights)))
    return out


def fused_moe_packed(input, gate_packed, up_packed, down_packed, routing_weights, expert_indices, output,
                     num_experts: int, top_k: int, activation: int = 0, moe_type: int = 0) -> None:
    """output += MoE of input over pre-packed weights
    (candle_moe_fused_moe_packed). Qwen3 (moe_type 0): gate/up [E, I, H],
    down [E, H, I] (pack_weights of the API layout); Nomic (moe_type 1):
    gate = fc1 [E, I, H] packed, up = fc2 [E, H, I] as fused_moe takes it,
    down None. input / output [T, H] f16 or bf16, routing_weights [T, k] f32,
    expert_indices [T, k] u32/i32; every tensor contiguous, on input's device
    and of these shapes, else CandleMoeError."""
    import torch

    def bad(msg):
        raise CandleMoeError(CANDLE_MOE_ERR_INVALID, "fused_moe_packed: " + msg)

    if input.dim() != 2 or gate_packed.dim() != 3:
        bad("input must be [T, H] and gate_packed [E, I, H]")
    T, H = input.shape
    E, I = num_experts, gate_packed.shape[1]
    want = {"gate_packed": (gate_packed, (E, I, H)), "up_packed": (up_packed, (E, I, H) if moe_type == 0 else (E, H, I)),
            "routing_weights": (routing_weights, (T, top_k)), "expert_indices": (expert_indices, (T, top_k)),
            "output": (output, (T, H))}
    if moe_type == 0:
        want["down_packed"] = (down_packed, (E, H, I))
    elif down_packed is not None:
        bad("Nomic (moe_type 1) takes no down_packed")
    for name, (t, shape) in want.items():
        if t is None:
            bad(f"{name} is missing")
        if tuple(t.shape) != tuple(shape):
            bad(f"{name} must be {list(shape)}, got {list(t.shape)}")
        if not t.is_contiguous():
            bad(f"{name} must be contiguous")
        if t.device != input.device:
            bad(f"{name} must be on {input.device}")
        dts = {"routing_weights": (torch.float32,), "expert_indices": (torch.int32, torch.uint32)}.get(
            name, (input.dtype,))
        if t.dtype not in dts:
            bad(f"{name} must be {' or '.join(str(d) for d in dts)}, got {t.dtype}")
    if not input.is_contiguous():
        bad("input must be contiguous")
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    check(lib().candle_moe_fused_moe_packed(
        p(input), p(gate_packed), p(up_packed), p(down_packed), p(routing_weights), p(expert_indices), p(output),
        T, H, I, num_experts, top_k, int(activation), int(moe_type), _torch_dtype_code(input), _stream_for(input)))


def validate_topk_softmax(g: CmTensor, w: CmTensor, i: CmTensor, ei: CmTensor) -> None:
    check(lib().candle_moe_validate_topk_softmax(ctypes.byref(g), ctypes.byref(w), ctypes.byref(i), ctypes.byref(ei)))


class FusedMoE:
    """``FusedMoE`` of the reference (``/root/reference/src/lib.rs:244-335``)."""

    def __init__(self, num_experts: int, num_selected_experts: int, activation: Activation):
        self.num_experts = int(num_experts)
        self.num_selected_experts = int(num_selected_experts)
        self.activation = Activation(activation)

    @classmethod
    def new(cls, num_experts: int, num_selected_experts: int, activation: Activation) -> "FusedMoE":
        return cls(num_experts, num_selected_experts, activation)

    def _self(self) -> CmFusedMoE:
        return CmFusedMoE(self.num_experts, self.num_selected_experts, int(self.activation))

    def forward(self, input, gate_weights, up_weights, down_weights, routing_weights, expert_indices,
                moe_type: int):
        """Returns a new [num_tokens, hidden_dim] tensor of input's dtype.

        input [T, H]; gate_weights / up_weights [E, H, I]; down_weights
        [E, I, H] (Qwen3, moe_type 0) or None (Nomic, moe_type 1);
        routing_weights [T, k] f32; expert_indices [T, k] u32.
        """
        import torch

        out_shape = tuple(input.shape[:1]) + tuple(input.shape[1:2]) if input.dim() == 2 else (0, 0)
        output = torch.empty(out_shape, dtype=input.dtype, device=input.device)
        m = self._self()
        descs = [describe(t) for t in (input, gate_weights, up_weights)]
        dd = describe(down_weights) if down_weights is not None else None
        rw, ix, od = describe(routing_weights), describe(expert_indices), describe(output)
        check(lib().candle_moe_fused_moe_forward(
            ctypes.byref(m), ctypes.byref(descs[0]), ctypes.byref(descs[1]), ctypes.byref(descs[2]),
            ctypes.byref(dd) if dd is not None else None, ctypes.byref(rw), ctypes.byref(ix), int(moe_type),
            ctypes.byref(od), _stream_for(input)))
        return output

    __call__ = forward

    def validate(self, input: CmTensor, gate: CmTensor, up: CmTensor, down: Optional[CmTensor],
                 routing: CmTensor, indices: CmTensor, moe_type: int, output: CmTensor) -> None:
        m = self._self()
        check(lib().candle_moe_validate_fused_moe(
            ctypes.byref(m), ctypes.byref(input), ctypes.byref(gate), ctypes.byref(up),
            ctypes.byref(down) if down is not None else None, ctypes.byref(routing), ctypes.byref(indices),
            int(moe_type), ctypes.byref(output)))


def trim_workspaces() -> None:
    """Release the library-owned workspaces of fused_moe and router_topk (one
    per device and stream, kept between calls; hipFree, which waits for the
    device); the next call allocates again."""
    check(lib().candle_moe_trim_workspaces())


def version() -> str:
    return lib().candle_moe_version().decode()


COMBINE_AUTO, COMBINE_PAIRS, COMBINE_EXPERT_SETS = 0, 1, 2
PATH_NAMES = {2: "expert-set", 1: "pairs", 0: "simt", -1: "invalid"}


def set_combine_policy(policy: int) -> None:
    """Process-wide fused_moe combine strategy (COMBINE_*; default auto)."""
    check(lib().candle_moe_set_combine_policy(int(policy)))


# grouping launch modes of candle_moe_set_grouping_mode (include/candle_moe.h)
GROUPING_AUTO, GROUPING_TWO_LAUNCHES, GROUPING_ONE_LAUNCH_RECOUNT = 0, 1, 2


def set_grouping_mode(mode: int) -> None:
    """Process-wide grouping launch mode of fused_moe (GROUPING_*; default auto)."""
    check(lib().candle_moe_set_grouping_mode(int(mode)))


# GEMM kernel codes of candle_moe_set_tile_policy (include/candle_moe.h)
TILE_AUTO, TILE_128, TILE_LDS_128, TILE_W8, TILE_ROWS32, TILE_128x256_OCC2, TILE_F32_ROWS32, TILE_F32_128 = \
    0, 1, 5, 7, 12, 14, 15, 16
TILE_CODES = (TILE_AUTO, TILE_128, TILE_LDS_128, TILE_W8, TILE_ROWS32, TILE_128x256_OCC2, TILE_F32_ROWS32, TILE_F32_128)
_TILE_ROWS = {0: 64, 1: 128, 5: 128, 7: 256, 12: 32, 14: 128, 15: 32, 16: 128, 18: 16}
# fp8 weights only (fused_moe_fp8): the register-operand decode kernel
TILE_W8_GEMV = 17
# 16-bit decode kernels (no grouping launch, weights straight into registers;
# up to 1024 pairs): automatic for a few rows per touched expert
TILE_DEC_GEMV = 18


def set_tile_policy(policy: int) -> None:
    """Process-wide MFMA block tile of fused_moe (TILE_*; default auto)."""
    check(lib().candle_moe_set_tile_policy(int(policy)))


def _path_code(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type):
    return lib().candle_moe_fused_moe_path_ex(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k,
                                              dtype_code, moe_type)


def fused_moe_path(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type=0) -> str:
    """Name of the path fused_moe takes for these sizes under the current policy."""
    code = _path_code(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type)
    return PATH_NAMES[code if code < 0 else code & 3]


def fused_moe_kernel(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type=0) -> int:
    """GEMM kernel code (TILE_*) fused_moe uses for these sizes (-1 if invalid)."""
    code = _path_code(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type)
    return -1 if code < 0 else (code >> 2) & 0x3f


def fused_moe_pair_rows(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code,
                        moe_type=0) -> bool:
    """True when the pair path stores each pair's row and sums a token's k rows
    (False: f32 atomics into an accumulator, or not the pair path)."""
    code = _path_code(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type)
    return code >= 0 and bool(code & (1 << 8))


def fused_moe_tile(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type=0) -> int:
    """Block-tile rows of the GEMM kernels fused_moe uses for these sizes (64 for SIMT)."""
    k = fused_moe_kernel(num_tokens, hidden_dim, intermediate_dim, num_experts, top_k, dtype_code, moe_type)
    return 0 if k < 0 else _TILE_ROWS[k]


__all__ = [
    "Activation", "FusedMoE", "apply_topk_softmax_inplace", "CandleMoeError", "lib", "describe", "spec",
    "validate_topk_softmax", "version", "LIB_PATH", "set_combine_policy", "fused_moe_path",
    "set_tile_policy", "fused_moe_tile", "fused_moe_kernel", "quantize_fp8", "dequantize_fp8", "fused_moe_fp8",
]
