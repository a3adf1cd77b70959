"""Arithmetic the router kernel (candle-moe_amd/csrc/topk_softmax.hip) relies
on to reproduce the CPU oracle bit for bit, checked on the host:

* its f64 exponential (exp_f32_f64), restated in C with the coefficients
  read from the kernel source, equals the oracle's (float)exp((double)d) for
  every f32 d in [-104, 0] (and +0 below, NaN for NaN);
* p = e / S (IEEE f32 division, the oracle) equals f32(f64(e) * (1 / f64(S)))
  (the kernel's form);
* the sorting networks of sort_keys / sort_keys32 sort every 0/1 input
  (0-1 principle: then every input).
The GPU side of the same claims is tests/test_gpu_topk.py (weights bit-exact
where the summation order matches the oracle's).
"""
import itertools
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "candle-moe_amd", "csrc", "topk_softmax.hip")


def kernel_source():
    return open(SRC).read()


def exp_coefficients():
    m = re.search(r"kExpCoef\[15\]\s*=\s*\{(.*?)\}", kernel_source(), re.S)
    vals = [v.strip() for v in m.group(1).split(",") if v.strip()]
    assert len(vals) == 15
    return [float.fromhex(v) for v in vals]


def test_exp_coefficients_are_what_they_claim():
    c = exp_coefficients()
    assert abs(c[0] - 1 / np.log(2)) < 1e-15
    assert abs((c[1] + c[2]) - np.log(2)) < 1e-30 + 1e-16 * np.log(2)
    # the ln 2 head has at most 40 significant bits (n * head exact for |n| < 2^13)
    m, _ = np.frexp(c[1])
    assert float(m * 2 ** 40).is_integer()
    import math
    assert c[3:] == [1.0 / math.factorial(n) for n in range(12, 0, -1)]


def test_kernel_exp_equals_oracle_exp_for_every_f32(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = str(tmp_path / "router_exp_exhaustive")
    subprocess.run([cc, "-O2", "-fopenmp", "-ffp-contract=off", "-mfma",
                    os.path.join(ROOT, "tests", "cpp", "router_exp_exhaustive.c"), "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe] + [float.hex(c) for c in exp_coefficients()], capture_output=True, text=True,
                       timeout=600, check=True)
    n, bad = map(int, r.stdout.split())
    assert n == 1120927745 and bad == 0, r.stdout


def test_division_by_reciprocal_is_correctly_rounded():
    rng = np.random.default_rng(7)
    n = 4_000_000
    e = rng.random(n, dtype=np.float32)
    S = (rng.random(n, dtype=np.float32) * 255 + 1).astype(np.float32)
    # sums near powers of two and quotients of every magnitude, denormals included
    S[: n // 4] = (np.float32(2.0) ** rng.integers(0, 8, n // 4).astype(np.float32) *
                   (1 + rng.integers(0, 64, n // 4).astype(np.float32) * np.float32(2 ** -23)))
    e[n // 4: n // 2] = (e[n // 4: n // 2] * np.float32(2.0) ** -rng.integers(0, 140, n // 4).astype(np.float32))
    want = (e / S).view(np.uint32)
    got = (e.astype(np.float64) * (1.0 / S.astype(np.float64))).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


def _networks():
    src = kernel_source()
    body = re.search(r"void sort_keys32\(uint32_t \(&k\)\[N\]\) \{(.*?)\n\}", src, re.S).group(1)
    nets = {}
    for n in (2, 4, 8):
        part = re.search(r"N == %d\) \{(.*?)\}" % n, body, re.S).group(1)
        nets[n] = [(int(a), int(b)) for a, b in re.findall(r"key32_cx\(k\[(\d)\], k\[(\d)\]\)", part)]
    # sort_keys (64-bit keys) uses the same networks
    body64 = re.search(r"void sort_keys\(uint64_t \(&k\)\[N\]\) \{(.*?)\n\}", src, re.S).group(1)
    for n in (2, 4, 8):
        part = re.search(r"N == %d\) \{(.*?)\}" % n, body64, re.S).group(1)
        assert [(int(a), int(b)) for a, b in re.findall(r"key_cx\(k\[(\d)\], k\[(\d)\]\)", part)] == nets[n]
    return nets


@pytest.mark.parametrize("n", [2, 4, 8])
def test_sorting_networks_sort_every_01_input(n):
    net = _networks()[n]
    assert len(net) == {2: 1, 4: 5, 8: 19}[n]
    for bits in itertools.product([0, 1], repeat=n):
        v = list(bits)
        for a, b in net:
            if v[b] > v[a]:
                v[a], v[b] = v[b], v[a]
        assert v == sorted(v, reverse=True), (bits, v)
