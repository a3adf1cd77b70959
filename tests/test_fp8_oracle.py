"""The fp8 weight format's oracle (OCP e4m3 decode / encode, per-channel
quantize), pinned without the GPU.

decode: all 256 codes against the OCP OFP8 e4m3 definition evaluated here in
exact rational arithmetic (value = (-1)^s * 2^(e-7) * (1 + m/8), subnormals
m/8 * 2^-6, S.1111.111 NaN) and against torch.float8_e4m3fn, an independent
implementation of the same format.
encode: against torch's round-to-nearest-even conversion on every finite
value, every midpoint between neighbours and the f32 values either side of
each midpoint, plus log-uniform random values; saturation at 448 (where torch,
which does not saturate, gives NaN above 464) by its closed form.
quantize: the per-channel closed forms (the largest magnitude encodes to 448,
scale = max / 448), both input layouts agreeing, zero channels.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle as O


def spec_value(c: int):
    """OCP e4m3 (E4M3FN) value of code c as a Fraction (None for NaN)."""
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return None
    v = Fraction(m, 8) * Fraction(2) ** -6 if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
    return -v if s else v


def _torch_decode(codes: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(codes.astype(np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def _torch_encode(x: np.ndarray) -> np.ndarray:
    import torch

    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_all_codes_against_spec_and_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_decode(codes)
    tor = _torch_decode(codes)
    for c in range(256):
        want = spec_value(c)
        if want is None:
            assert np.isnan(got[c]) and np.isnan(tor[c]), c
            continue
        assert Fraction(float(got[c])) == want, (c, got[c], want)
        assert Fraction(float(tor[c])) == want, (c, tor[c], want)
        if c & 0x7F == 0:
            assert np.signbit(got[c]) == bool(c & 0x80)
    # the format's landmarks
    assert got[0x7E] == 448.0 and got[0xFE] == -448.0
    assert got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9 and got[0x38] == 1.0
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF])


def test_encode_round_trips_every_finite_code():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    vals = O.e4m3_decode(codes)
    assert np.array_equal(O.e4m3_encode(vals), codes)


def test_encode_matches_torch_on_midpoints_and_neighbours():
    pos = np.array([spec_value(c) for c in range(0x7F)], dtype=object)
    mids = [(pos[i] + pos[i + 1]) / 2 for i in range(len(pos) - 1)]
    mids.append(Fraction(464))  # the midpoint above 448 (torch: ties to even -> 448)
    xs = []
    for m in mids:
        f = np.float32(float(m))
        assert Fraction(float(f)) == m  # every midpoint is an f32
        xs += [f, np.nextafter(f, np.float32(0)), np.nextafter(f, np.float32(np.inf))]
    xs = np.array(xs, np.float32)
    xs = xs[np.abs(xs) <= 464]
    xs = np.concatenate([xs, -xs])
    assert np.array_equal(O.e4m3_encode(xs), _torch_encode(xs))


def test_encode_matches_torch_on_random_and_tiny_values():
    rng = np.random.default_rng(7)
    mag = np.exp2(rng.uniform(-24, np.log2(464), 40000)).astype(np.float32)
    x = np.where(rng.random(mag.size) < 0.5, -mag, mag).astype(np.float32)
    extra = np.array([0.0, -0.0, 2.0 ** -10, 3 * 2.0 ** -11, 2.0 ** -130, 1e-45, 2.0 ** -6 * (1 - 2 ** -5)],
                     np.float32)
    x = np.concatenate([x, extra, -extra])
    assert np.array_equal(O.e4m3_encode(x), _torch_encode(x))


def test_encode_saturates_and_maps_nan():
    x = np.array([448.0, 464.0, 464.5, 1e6, np.inf, -500.0, -np.inf, np.nan], np.float32)
    assert O.e4m3_encode(x).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE, 0x7F]


@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
def test_quantize_closed_forms_and_layouts(dt):
    E, K, N = 3, 40, 24
    w = O.randn((E, K, N), seed=21, std=0.05)
    w[1, :, 5] = 0.0                       # an all-zero channel: scale 1, codes 0
    w[2, 7, 3] = 3.0                       # one dominant element
    ws = O.to_dtype(w, dt)
    wf = O.to_f32(ws, dt)
    q, s = O.quantize_fp8(ws, dt, kn=True)
    assert q.shape == (E, N, K) and s.shape == (E, N)
    amax = np.abs(wf).max(axis=1)          # [E, N]
    want_s = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    assert np.array_equal(s, want_s)
    assert s[1, 5] == 1.0 and not q[1, 5].any()
    # codes: encode(w / scale) with an f32 division, compared with torch's rounding
    ratio = (np.transpose(wf, (0, 2, 1)) / s[:, :, None]).astype(np.float32)
    assert np.abs(ratio).max() <= 448.0 * (1 + 2 ** -23)
    assert np.array_equal(q, _torch_encode(np.minimum(np.maximum(ratio, -448.0), 448.0)))
    # the channel maximum encodes to +-448
    kmax = np.abs(wf).argmax(axis=1)
    for e in range(E):
        for n in range(N):
            if amax[e, n] > 0:
                assert q[e, n, kmax[e, n]] & 0x7F == 0x7E
    # the [E, N, K] input layout gives the same result
    q2, s2 = O.quantize_fp8(np.ascontiguousarray(np.transpose(ws, (0, 2, 1))), dt, kn=False)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # dequantize: one f32 product per element, within half an e4m3 step of w
    d = O.dequantize_fp8(q, s)
    assert np.array_equal(d, (O.e4m3_decode(q) * s[:, :, None]).astype(np.float32))
    err = np.abs(d - np.transpose(wf, (0, 2, 1)))
    assert np.all(err <= np.maximum(np.abs(np.transpose(wf, (0, 2, 1))) * 2.0 ** -4, s[:, :, None] * 2.0 ** -10)
                  * 1.0001)
