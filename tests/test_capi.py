"""C-ABI contract tests that need no GPU.

* libcandle_moe_hip.so loads and exports every function include/candle_moe.h
  declares (the drop-in symbols topk_softmax / fused_moe among them).
* The host API rejects what the reference's Rust layer rejects, with the
  reference's error text (/root/reference/src/lib.rs:47-94, 184-242), before
  any HIP call; the added checks (contiguity, top-k <= E, Qwen3 without down)
  have their own text.
* The raw symbols' status variants reject invalid sizes without launching.
"""
import ctypes
import os
import re

import pytest

import candle_moe as cm
from candle_moe import DT_BF16, DT_F16, DT_F32, DT_I64, DT_U32, spec

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "candle_moe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", src, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert {"topk_softmax", "fused_moe", "candle_moe_fused_moe_status"} <= set(names)
    L = cm.lib()
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/candle_moe.h but not exported"
    assert cm.version().startswith("candle-moe-hip")


def test_header_symbols_match_reference_ffi_signature():
    # argument order of /root/reference/src/ffi.rs:15-24 and :45-62
    src = open(os.path.join(ROOT, "include", "candle_moe.h")).read()
    topk = re.search(r"void topk_softmax\((.*?)\);", src, re.S).group(1)
    assert [a.split()[-1].strip("*") for a in topk.split(",")] == [
        "gating_output", "topk_weight", "topk_indices", "token_expert_indices", "num_experts", "num_tokens",
        "topk", "stream"]
    moe = re.search(r"void fused_moe\((.*?)\);", src, re.S).group(1)
    assert [a.split()[-1].strip("*") for a in moe.split(",")] == [
        "input", "gate_weights", "up_weights", "down_weights", "routing_weights", "expert_indices", "output",
        "num_tokens", "hidden_dim", "intermediate_dim", "num_experts", "num_selected_experts", "activation_type",
        "moe_type", "dtype", "stream"]


# ---------------------------------------------------------------- router
def topk_specs(T=8, E=4, k=2, gdt=DT_F32, wdt=DT_F32, idt=DT_U32, dev=0):
    return spec((T, E), gdt, dev), spec((T, k), wdt, dev), spec((T, k), idt, dev), spec((T, k), idt, dev)


def topk_err(*specs):
    with pytest.raises(cm.CandleMoeError) as e:
        cm.validate_topk_softmax(*specs)
    assert e.value.code == cm.CANDLE_MOE_ERR_INVALID
    return str(e.value)


def test_topk_valid_specs_pass():
    cm.validate_topk_softmax(*topk_specs())
    cm.validate_topk_softmax(*topk_specs(T=32768, E=128, k=8))
    cm.validate_topk_softmax(*topk_specs(gdt=DT_BF16, wdt=DT_BF16))


def test_topk_rejections_mirror_lib_rs():
    g, w, i, ei = topk_specs()
    assert "is only supported for f32, f16 and bf16" in topk_err(g, spec((8, 2), DT_I64), i, ei)
    assert "gating_output must be a cuda tensor" in topk_err(spec((8, 4), DT_F32, -1), w, i, ei)
    assert "expects input tensors of rank 2" in topk_err(spec((8, 4, 1), DT_F32), w, i, ei)
    assert "num_experts should be power of 2 and smaller than 256" in topk_err(*topk_specs(E=6))
    assert "num_experts should be power of 2 and smaller than 256" in topk_err(*topk_specs(E=512))
    assert "shape mismatch topk_indices" in topk_err(g, w, spec((8, 3), DT_U32), ei)
    assert "shape mismatch token_expert_indices" in topk_err(g, w, i, spec((7, 2), DT_U32))
    assert "unexpected dtype for gating_output" in topk_err(spec((8, 4), DT_F16), w, i, ei)
    assert "unexpected dtype for topk_indices" in topk_err(g, w, spec((8, 2), DT_F32), ei)
    # added checks (the reference reads out of bounds / ignores strides here)
    assert "top_k must be in" in topk_err(*topk_specs(E=4, k=5))
    assert "must be contiguous" in topk_err(spec((8, 4), DT_F32, 0, strides=(8, 1)), w, i, ei)
    assert "shape mismatch gating_output" in topk_err(spec((9, 4), DT_F32), w, i, ei)


def test_topk_status_symbol_rejects_without_launch():
    L = cm.lib()
    assert L.candle_moe_topk_softmax_status(None, None, None, None, 8, 16, 9, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "topk must be in" in cm.last_error()
    assert L.candle_moe_topk_softmax_status(None, None, None, None, 0, 16, 1, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_topk_softmax_status(None, None, None, None, 8, 16, 2, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "null tensor pointer" in cm.last_error()
    # zero tokens is a no-op
    assert L.candle_moe_topk_softmax_status(None, None, None, None, 8, 0, 2, None) == cm.CANDLE_MOE_OK


# ------------------------------------------------------------- fused MoE
def moe_specs(T=16, H=64, I=256, E=8, k=2, dt=DT_BF16, qwen3=True, dev=0):
    x = spec((T, H), dt, dev)
    g = spec((E, H, I), dt, dev)
    u = spec((E, H, I), dt, dev)
    d = spec((E, I, H), dt, dev) if qwen3 else None
    rw = spec((T, k), DT_F32, dev)
    ix = spec((T, k), DT_U32, dev)
    out = spec((T, H), dt, dev)
    return x, g, u, d, rw, ix, out


def moe_err(moe, specs, moe_type=0):
    x, g, u, d, rw, ix, out = specs
    with pytest.raises(cm.CandleMoeError) as e:
        moe.validate(x, g, u, d, rw, ix, moe_type, out)
    return str(e.value)


def test_moe_valid_specs_pass():
    moe = cm.FusedMoE.new(8, 2, cm.Activation.Silu)
    x, g, u, d, rw, ix, out = moe_specs()
    moe.validate(x, g, u, d, rw, ix, 0, out)
    x, g, u, d, rw, ix, out = moe_specs(qwen3=False, dt=DT_F32)
    moe.validate(x, g, u, None, rw, ix, 1, out)
    big = cm.FusedMoE.new(128, 8, cm.Activation.Silu)
    x, g, u, d, rw, ix, out = moe_specs(T=4096, H=2048, I=768, E=128, k=8)
    big.validate(x, g, u, d, rw, ix, 0, out)


def test_moe_rejections_mirror_lib_rs():
    moe = cm.FusedMoE.new(8, 2, cm.Activation.Silu)
    s = list(moe_specs())
    assert "Number of experts mismatch" in moe_err(cm.FusedMoE.new(4, 2, cm.Activation.Silu), s)
    t = list(s); t[1] = spec((8, 32, 256), DT_BF16)
    assert "Hidden dimension mismatch for gate/up weights" in moe_err(moe, t)
    t = list(s); t[3] = spec((8, 256, 32), DT_BF16)
    assert "Hidden dimension mismatch for down weights (expected 64, got 32)" in moe_err(moe, t)
    t = list(s); t[2] = spec((8, 64, 128), DT_BF16)
    assert "Intermediate dimension mismatch (gate: 256, up: 128, down: 256)" in moe_err(moe, t)
    t = list(s); t[4] = spec((15, 2), DT_F32)
    assert "Number of tokens mismatch" in moe_err(moe, t)
    t = list(s); t[5] = spec((16, 3), DT_U32)
    assert "Number of selected experts mismatch" in moe_err(moe, t)
    assert "moe_type must be one of 0 or 1" in moe_err(moe, s, moe_type=2)
    t = [spec(tuple(a.dims[: a.rank]), DT_I64) if a is not None else None for a in s]
    t[4], t[5] = s[4], s[5]
    assert "FusedMoE is only supported for f16, bf16 and f32" in moe_err(moe, t)
    t = list(s); t[0] = spec((16, 64), DT_BF16, -1)
    assert "input must be a cuda tensor" in moe_err(moe, t)
    t = list(s); t[4] = spec((16, 2), DT_BF16)
    assert "unexpected dtype for routing_weights, expected: F32" in moe_err(moe, t)
    t = list(s); t[5] = spec((16, 2), DT_I64)
    assert "unexpected dtype for expert_indices, expected: U32" in moe_err(moe, t)
    t = list(s); t[1] = spec((8, 64, 256), DT_F16)
    assert "unexpected dtype for gate_weights" in moe_err(moe, t)
    t = list(s); t[0] = spec((16, 64, 1), DT_BF16)
    assert "unexpected rank, expected: 2" in moe_err(moe, t)


def test_moe_added_checks():
    moe = cm.FusedMoE.new(8, 2, cm.Activation.Silu)
    s = list(moe_specs())
    t = list(s); t[3] = None
    assert "down_weights is required for moe_type 0" in moe_err(moe, t, moe_type=0)
    t = list(s); t[1] = spec((8, 64, 256), DT_BF16, 0, strides=(16384, 1, 64))
    assert "gate_weights must be contiguous" in moe_err(moe, t)
    t = list(s); t[6] = spec((16, 32), DT_BF16)
    assert "shape mismatch output" in moe_err(moe, t)


def test_moe_status_symbol_rejects_without_launch():
    L = cm.lib()
    args = [None] * 7
    assert L.candle_moe_fused_moe_status(*args, 16, 64, 256, 8, 2, 0, 2, 1, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "moe_type must be one of 0 or 1" in cm.last_error()
    assert L.candle_moe_fused_moe_status(*args, 16, 64, 256, 8, 2, 5, 0, 1, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "activation_type" in cm.last_error()
    assert L.candle_moe_fused_moe_status(*args, 16, 64, 256, 8, 2, 0, 0, 3, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_fused_moe_status(*args, 16, 64, 256, 8, 2, 0, 0, 1, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "null tensor pointer" in cm.last_error()
    assert L.candle_moe_fused_moe_status(*args, 0, 64, 256, 8, 2, 0, 0, 1, None) == cm.CANDLE_MOE_OK


@pytest.mark.parametrize("T, H, I, E, k, mt, path, kernel, rows", [
    # Nomic (H 768, moe_type 1): the down GEMM's 3 column tiles never fill the
    # CUs twice on the two-per-CU tile; up to 128 rows per expert the 32-row
    # kernel (the 128x128 tile would give its down GEMM too few tiles), the
    # rest the 256x256 tile; its pair rows (T*k*H 16-bit values) stay below
    # 256 MiB, so the pair path with pair rows on the tiled kernels; decode
    # batches (<= 32 rows per expert) the decode kernels (18, pair rows)
    (16, 768, 3072, 8, 2, 1, "pairs", 18, True),
    (192, 768, 3072, 8, 2, 1, "pairs", 12, False),
    (512, 768, 3072, 8, 2, 1, "pairs", 12, False),
    (1024, 768, 3072, 8, 2, 1, "pairs", 7, True),
    (4096, 768, 3072, 8, 2, 1, "pairs", 7, True),
    (12288, 768, 3072, 8, 2, 1, "pairs", 7, True),
    (32768, 768, 3072, 8, 2, 1, "pairs", 7, True),
    # Qwen3-30B-A3B (H 2048, 128 experts): two-per-CU 128x256 tile below 1024
    # rows per expert; (E+1)^k keys too many for the expert-set path
    (1, 2048, 768, 128, 8, 0, "pairs", 18, True),
    (16, 2048, 768, 128, 8, 0, "pairs", 18, True),
    (32, 2048, 768, 128, 8, 0, "pairs", 18, True),   # 256 pairs: the decode kernels' last size
    (64, 2048, 768, 128, 8, 0, "pairs", 12, False),  # 512 pairs: the 32-row kernel (f32 atomics)
    (128, 2048, 768, 128, 8, 0, "pairs", 12, False),
    (1024, 2048, 768, 128, 8, 0, "pairs", 14, True),
    (4096, 2048, 768, 128, 8, 0, "pairs", 14, True),
    (16384, 2048, 768, 128, 8, 0, "pairs", 7, True),
    # pair rows beyond 2 GiB: f32 atomics into the [T, H] accumulator instead
    (131072, 2048, 768, 128, 8, 0, "pairs", 7, False),
    # Qwen3 (H 4096): expert sets once the pair rows reach 256 MiB (T >= 16384)
    (8, 4096, 1536, 8, 2, 0, "pairs", 18, True),
    (64, 4096, 1536, 8, 2, 0, "pairs", 18, True),
    (128, 4096, 1536, 8, 2, 0, "pairs", 18, True),
    (512, 4096, 1536, 8, 2, 0, "pairs", 5, True),
    (4096, 4096, 1536, 8, 2, 0, "pairs", 7, True),
    (8192, 4096, 1536, 8, 2, 0, "pairs", 7, True),
    (16384, 4096, 1536, 8, 2, 0, "expert-set", 7, False),
    (32768, 4096, 1536, 8, 2, 0, "expert-set", 7, False),
])
def test_default_path_and_kernel(T, H, I, E, k, mt, path, kernel, rows):
    """The host's default combine path and GEMM kernel (no GPU needed)."""
    assert cm.fused_moe_path(T, H, I, E, k, 1, mt) == path
    assert cm.fused_moe_kernel(T, H, I, E, k, 1, mt) == kernel
    assert cm.fused_moe_pair_rows(T, H, I, E, k, 1, mt) == rows
    if mt == 0:  # the original query answers for Qwen3
        code = cm.lib().candle_moe_fused_moe_path(T, H, I, E, k, 1)
        assert code == (cm.lib().candle_moe_fused_moe_path_ex(T, H, I, E, k, 1, 0) & 0xff)


def test_tile_policy_accepts_only_shipped_kernels():
    for code in cm.TILE_CODES + (cm.TILE_W8_GEMV, cm.TILE_DEC_GEMV):
        cm.set_tile_policy(code)
    cm.set_tile_policy(0)
    for code in (2, 3, 4, 6, 8, 9, 10, 11, 13, 19, -1):
        with pytest.raises(cm.CandleMoeError) as e:
            cm.set_tile_policy(code)
        assert e.value.code == cm.CANDLE_MOE_ERR_INVALID
    cm.set_tile_policy(0)


def test_fp8_kernel_policy_leaves_fused_moe_automatic():
    # policy 17 (fp8 register-operand decode kernel) does not change fused_moe's choice
    shapes = [(16, 4096, 1536, 8, 2), (32768, 4096, 1536, 8, 2), (512, 768, 3072, 8, 2)]
    auto = [cm.fused_moe_kernel(*s, 1, 0) for s in shapes]
    cm.set_tile_policy(cm.TILE_W8_GEMV)
    try:
        assert [cm.fused_moe_kernel(*s, 1, 0) for s in shapes] == auto
    finally:
        cm.set_tile_policy(0)


def test_grouping_mode_setter():
    for mode in (cm.GROUPING_TWO_LAUNCHES, cm.GROUPING_ONE_LAUNCH_RECOUNT, cm.GROUPING_AUTO):
        cm.set_grouping_mode(mode)
    for mode in (3, -1):
        with pytest.raises(cm.CandleMoeError) as e:
            cm.set_grouping_mode(mode)
        assert e.value.code == cm.CANDLE_MOE_ERR_INVALID
    cm.set_grouping_mode(cm.GROUPING_AUTO)


def test_workspace_size():
    L = cm.lib()
    small = L.candle_moe_fused_moe_workspace_size(32, 64, 256, 8, 2, 1)
    big = L.candle_moe_fused_moe_workspace_size(32768, 4096, 1536, 8, 2, 1)
    assert 0 < small < big
    # the expert-set path needs the bf16 intermediate [T*k, I] only; the size
    # also covers operands off a 16-byte boundary (scalar kernel, pair path
    # with the f32 accumulator [T, H])
    assert cm.fused_moe_path(32768, 4096, 1536, 8, 2, 1) == "expert-set"
    assert 65536 * 1536 * 2 + 32768 * 4096 * 4 <= big < 65536 * 1536 * 2 + 32768 * 4096 * 4 + (64 << 20)
    # ... the pair path also the f32 accumulator [T, H]
    assert cm.fused_moe_path(4096, 2048, 768, 128, 8, 1) == "pairs"
    q30 = L.candle_moe_fused_moe_workspace_size(4096, 2048, 768, 128, 8, 1)
    assert q30 >= 32768 * 768 * 2 + 4096 * 2048 * 4
    assert L.candle_moe_fused_moe_workspace_size(32, 64, 256, 0, 2, 1) == 0
    # an upper bound for both moe_types (Nomic's fc1 tile may differ from gate/up's)
    nomic = L.candle_moe_fused_moe_workspace_size(512, 768, 3072, 8, 2, 1)
    assert nomic >= 1024 * 3072 * 2 + 1024 * 768 * 2
    # workspace variant: too-small workspace is refused before anything runs
    rc = L.candle_moe_fused_moe_ws(*([ctypes.c_void_p(256)] * 7), 32, 64, 256, 8, 2, 0, 0, 1,
                                   ctypes.c_void_p(256), 16, None)
    assert rc == cm.CANDLE_MOE_ERR_WORKSPACE


def test_cpp_host_api_rejections(tmp_path):
    """include/candle_moe.hpp compiles with the host C++ compiler alone and
    its FusedMoE / apply_topk_softmax_inplace reject invalid calls with the
    reference's messages (tests/cpp/host_api_rejections.cpp; no GPU)."""
    import shutil
    import subprocess

    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    libdir = os.path.join(ROOT, "candle-moe_amd")
    exe = str(tmp_path / "host_api_rejections")
    subprocess.run([cxx, "-std=c++17", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "host_api_rejections.cpp"), "-o", exe, "-L", libdir,
                    "-lcandle_moe_hip", "-Wl,-rpath," + libdir], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_grouping_entry_point_rejects_without_launch():
    L = cm.lib()
    assert L.candle_moe_grouping_workspace_size(0, 0) == 0
    assert L.candle_moe_grouping_workspace_size(100, 8) > 0
    assert L.candle_moe_group_pairs(None, -1, 8, None, None, None, 0, None) == cm.CANDLE_MOE_ERR_INVALID
    assert "num_pairs" in cm.last_error()
    assert L.candle_moe_group_pairs(None, 4, 5000, None, None, None, 0, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_group_pairs(ctypes.c_void_p(256), 4, 8, ctypes.c_void_p(256), ctypes.c_void_p(256),
                                    ctypes.c_void_p(256), 16, None) == cm.CANDLE_MOE_ERR_WORKSPACE


def test_noalloc_rejects_without_launch():
    # candle_moe_fused_moe_noalloc refuses a call whose workspace exceeds the
    # library's fixed scratch before touching the GPU
    L = cm.lib()
    assert L.candle_moe_fused_moe_noalloc_scratch_bytes() == 32 << 20
    p = ctypes.c_void_p(256)
    rc = L.candle_moe_fused_moe_noalloc(p, p, p, p, p, p, p, 8192, 4096, 1536, 8, 2, 0, 0, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_WORKSPACE
    assert "fused_moe_noalloc" in cm.last_error() and "33554432" in cm.last_error()
    assert L.candle_moe_fused_moe_noalloc(None, None, None, None, None, None, None, 16, 64, 256, 8, 2, 0, 0, 1,
                                          None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_fused_moe_noalloc(None, None, None, None, None, None, None, 0, 64, 256, 8, 2, 0, 0, 1,
                                          None) == cm.CANDLE_MOE_OK


def test_fp8_entry_points_reject_without_launch():
    L = cm.lib()
    p = ctypes.c_void_p(256)
    # f32 activations, and hidden/intermediate sizes off the 16-element grid
    rc = L.candle_moe_fused_moe_fp8(p, p, p, p, p, p, p, p, p, p, 16, 64, 256, 8, 2, 0, 0, 2, None)
    assert rc == cm.CANDLE_MOE_ERR_UNSUPPORTED and "fused_moe_fp8" in cm.last_error()
    rc = L.candle_moe_fused_moe_fp8(p, p, p, p, p, p, p, p, p, p, 16, 72, 256, 8, 2, 0, 0, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_UNSUPPORTED
    rc = L.candle_moe_fused_moe_fp8(p, p, p, p, p, p, p, p, p, p, 16, 64, 200, 8, 2, 0, 0, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_UNSUPPORTED
    # missing scales (Qwen3 needs all three, Nomic gate and up)
    rc = L.candle_moe_fused_moe_fp8(p, p, p, p, p, p, None, p, p, p, 16, 64, 256, 8, 2, 0, 0, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_INVALID and "scale" in cm.last_error()
    rc = L.candle_moe_fused_moe_fp8(p, p, p, None, p, None, None, p, p, p, 16, 64, 256, 8, 2, 0, 1, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_INVALID and "scale" in cm.last_error()
    rc = L.candle_moe_fused_moe_fp8(p, p, None, None, p, p, None, p, p, p, 16, 64, 256, 8, 2, 0, 1, 1, None)
    assert rc == cm.CANDLE_MOE_ERR_INVALID and "null tensor pointer" in cm.last_error()
    assert L.candle_moe_fused_moe_fp8(None, None, None, None, None, None, None, None, None, None, 0, 64, 256, 8, 2,
                                      0, 0, 1, None) == cm.CANDLE_MOE_OK
    assert L.candle_moe_quantize_fp8(p, 3, 1, 16, 16, 1, p, p, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_quantize_fp8(None, 1, 1, 16, 16, 1, p, p, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_quantize_fp8(None, 1, 0, 16, 16, 1, None, None, None) == cm.CANDLE_MOE_OK
    assert L.candle_moe_dequantize_fp8(p, None, 1, 16, 16, p, 1, None) == cm.CANDLE_MOE_ERR_INVALID
    assert L.candle_moe_dequantize_fp8(p, p, 1, -1, 16, p, 1, None) == cm.CANDLE_MOE_ERR_INVALID


def test_fused_moe_fp8_wrapper_checks_layouts_before_the_call():
    """fused_moe_fp8 (Python) passes raw pointers; it first checks every
    tensor's shape, dtype, contiguity and device (CPU tensors: nothing is
    launched, the checks raise before the C call)."""
    import torch

    T, H, I, E, k = 4, 64, 32, 8, 2
    x = torch.zeros(T, H, dtype=torch.bfloat16)
    out = torch.zeros(T, H, dtype=torch.bfloat16)
    rw = torch.zeros(T, k, dtype=torch.float32)
    ri = torch.zeros(T, k, dtype=torch.int32)
    gq, uq, dq = (torch.zeros(E, I, H, dtype=torch.uint8), torch.zeros(E, I, H, dtype=torch.uint8),
                  torch.zeros(E, H, I, dtype=torch.uint8))
    gs, us, ds = torch.ones(E, I), torch.ones(E, I), torch.ones(E, H)

    def call(**kw):
        a = dict(input=x, gate_q=gq, up_q=uq, down_q=dq, gate_scale=gs, up_scale=us, down_scale=ds,
                 routing_weights=rw, expert_indices=ri, output=out, num_experts=E, top_k=k)
        a.update(kw)
        with pytest.raises(cm.CandleMoeError) as ei:
            cm.fused_moe_fp8(**a)
        assert ei.value.code == cm.CANDLE_MOE_ERR_INVALID
        return str(ei.value)

    assert "gate_q" in call(gate_q=torch.zeros(E, H, I, dtype=torch.uint8))  # [E,H,I] passed as [E,I,H]
    assert "down_q" in call(down_q=torch.zeros(E, I, H, dtype=torch.uint8))
    assert "up_q" in call(up_q=torch.zeros(E, I, H, dtype=torch.int8))
    assert "down_scale" in call(down_scale=torch.ones(E, H, dtype=torch.float16))
    assert "up_scale" in call(up_scale=torch.ones(E, I + 1))
    assert "contiguous" in call(gate_q=torch.zeros(E, H, I, dtype=torch.uint8).transpose(1, 2))
    assert "expert_indices" in call(expert_indices=torch.zeros(T, k, dtype=torch.int64))
    assert "routing_weights" in call(routing_weights=torch.zeros(T, k + 1))
    assert "output" in call(output=torch.zeros(T, H, dtype=torch.float16))
    assert "down_scale" in call(down_scale=None)
    # Nomic: fc2 codes [E, H, I] in up_q with an [E, H] scale, nothing in down
    assert "down" in call(moe_type=1, up_q=torch.zeros(E, H, I, dtype=torch.uint8), up_scale=torch.ones(E, H))
    assert "up_q" in call(moe_type=1, down_q=None, down_scale=None)
