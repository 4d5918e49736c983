"""Pin the CPU oracle's Cubic bitstream/metadata/decode/linear restatement.

Each check is independent of the oracle's own text: the reference's known
answers (tests/ops/test_quantization_reference.py), brute-force bit loops,
closed forms of the cubic curve, and an FP64 scalar decoder with an error
bound (tools/quantization/audit_checkpoint.py:32-101 method).
"""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest
import torch

FMT0, FMT1, FMT2 = (
    "float32-scale-float16-ab",
    "int8-scale-int4-ab-global-fp32",
    "e5m9-scale-curve2-tensor-fp16",
)


def _stream(raw_codes, bits):
    stream = sum(code << (i * bits) for i, code in enumerate(raw_codes))
    nbytes = math.ceil(len(raw_codes) * bits / 8)
    return np.frombuffer(stream.to_bytes(nbytes, "little"), np.uint8)[None].copy()


@pytest.mark.parametrize("bits", range(1, 9))
def test_all_codes_cross_byte_and_reserved_zero(oracle, bits):
    # Known answer of tests/ops/test_quantization_reference.py:136-152.
    raw = list(range(1 << bits))
    decoded = oracle.unpack_cubic(_stream(raw, bits), bits, len(raw))[0].tolist()
    expected = []
    for code in raw:
        if bits == 1:
            expected.append(2 * code - 1)
        elif code == 1 << (bits - 1):
            expected.append(0)
        else:
            expected.append(code - (1 << bits) if code >= 1 << (bits - 1) else code)
    assert decoded == expected


@pytest.mark.parametrize("bits", range(1, 9))
def test_unpack_matches_brute_force_bit_loop_and_pack_round_trips(oracle, bits):
    rng = np.random.default_rng(bits)
    k = 77  # odd K: the last code straddles the clamped final byte
    packed = rng.integers(0, 256, size=(5, math.ceil(k * bits / 8)), dtype=np.uint8)
    codes = oracle.unpack_cubic(packed, bits, k)
    for r in range(5):
        bitlist = [(int(packed[r, i // 8]) >> (i % 8)) & 1 for i in range(packed.shape[1] * 8)]
        for i in range(k):
            raw = sum(bitlist[i * bits + j] << j for j in range(bits))
            if bits == 1:
                want = 2 * raw - 1
            else:
                want = raw - (1 << bits) if raw >= 1 << (bits - 1) else raw
                want = 0 if want == -(1 << (bits - 1)) else want
            assert codes[r, i] == want
    # pack is the inverse on the non-reserved domain
    assert np.array_equal(oracle.unpack_cubic(oracle.pack_cubic(codes, bits), bits, k), codes)


def test_compact_partition_coefficients_known_answer(oracle):
    # tests/ops/test_quantization_reference.py:154-171
    payload = {
        "weight_packed": np.array([[0x77], [0x77]], np.uint8),
        "weight_scale": np.array([[2], [3]], np.int8),
        "weight_ab": np.zeros((2, 1), np.uint8),
        "weight_scale_global": np.array([0.5, 2.0], np.float32),
        "weight_a_global": np.array([0.125, 0.25], np.float32),
        "weight_b_global": np.array([0.25, 0.5], np.float32),
    }
    w = oracle.decode_cubic(payload, 4, FMT1, (2, 2), 2, partitions=(1, 1))
    assert np.array_equal(w, np.array([[1.0, 1.0], [6.0, 6.0]], np.float32))


def test_curve2_metadata_uses_high_two_bits_known_answer(oracle):
    # tests/ops/test_quantization_reference.py:173-186
    payload = {
        "weight_packed": np.array([[0x77]] * 4, np.uint8),
        "weight_metadata": np.array([[0x1E00 | (i << 14)] for i in range(4)], np.uint16),
        "weight_curve_a": np.array([[1.0, 0.5, 0.25, 0.0]], np.float16),
        "weight_curve_b": np.zeros((1, 4), np.float16),
    }
    w = oracle.decode_cubic(payload, 4, FMT2, (4, 2), 2, partitions=(4,))
    assert np.array_equal(w, np.ones((4, 2), np.float32))


def test_row_slice_retains_original_partition_globals(oracle):
    # tests/ops/test_quantization_reference.py:86-106: decoding rows 1..5 of a
    # 3-partition matrix equals slicing the full decode.
    payload = {
        "weight_packed": np.full((6, 1), 0x77, np.uint8),
        "weight_scale": np.ones((6, 1), np.int8),
        "weight_ab": np.zeros((6, 1), np.uint8),
        "weight_scale_global": np.array([1.0, 2.0, 4.0], np.float32),
        "weight_a_global": np.ones(3, np.float32),
        "weight_b_global": np.ones(3, np.float32),
    }
    full = oracle.decode_cubic(payload, 4, FMT1, (6, 2), 2, partitions=(2, 2, 2))
    part = {k: v for k, v in payload.items()}
    part["weight_packed"] = payload["weight_packed"][1:5]
    part["weight_scale"] = payload["weight_scale"][1:5]
    part["weight_ab"] = payload["weight_ab"][1:5]
    part["weight_scale_global"] = payload["weight_scale_global"][0:3]
    sliced = oracle.decode_cubic(part, 4, FMT1, (4, 2), 2, partitions=(1, 2, 1))
    assert np.array_equal(sliced, full[1:5])


def _fmt0_payload(codes, bits, s, a, b):
    return {
        "weight_packed": np_pack(codes, bits),
        "weight_scale": np.asarray(s, np.float32),
        "weight_a": np.asarray(a, np.float16),
        "weight_b": np.asarray(b, np.float16),
    }


def np_pack(codes, bits):
    from oracle import oracle as o
    return o.pack_cubic(codes, bits)


@pytest.mark.parametrize("bits", range(2, 9))
def test_curve_special_cases_closed_form(oracle, bits):
    """a=1,b=0 gives f(t)=t; a=0,b=1 gives t*t; a=b=0 gives t*(t*t); f(1)=1.

    Each isolates one polynomial coefficient, so a dropped term, a swapped a/b
    or a wrong nesting fails at least one case.
    """
    d = (1 << (bits - 1)) - 1
    mags = np.arange(-d, d + 1, dtype=np.int8)
    k = len(mags)
    s = np.float32(0.8125)
    for a, b, f in (
        (1.0, 0.0, lambda t: t),
        (0.0, 1.0, lambda t: np.float32(t * t)),
        (0.0, 0.0, lambda t: np.float32(t * np.float32(t * t))),
    ):
        payload = _fmt0_payload(mags[None], bits, [[s]], [[a]], [[b]])
        w = oracle.decode_cubic(payload, bits, FMT0, (1, k), k)[0]
        for q, value in zip(mags.tolist(), w.tolist()):
            t = np.float32(abs(q) / d)  # exactly rounded quotient
            want = np.float32(math.copysign(1.0, q) * np.float32(s * f(t))) if q else 0.0
            assert value == want, (bits, a, b, q)
    # f(1) = 1 exactly for any finite fp16 a, b in a moderate range: |w|max = s
    rng = np.random.default_rng(bits)
    a = rng.uniform(-1, 2, 64).astype(np.float16)
    b = rng.uniform(-1, 1, 64).astype(np.float16)
    codes = np.tile(np.array([[d, -d]], np.int8), (64, 1))
    payload = _fmt0_payload(codes, bits, np.full((64, 1), 3.5, np.float32), a[:, None], b[:, None])
    w = oracle.decode_cubic(payload, bits, FMT0, (64, 2), 2)
    assert np.array_equal(w, np.tile(np.array([[3.5, -3.5]], np.float32), (64, 1)))


def test_bipolar_one_bit_is_code_times_scale(oracle):
    codes = np.array([[1, -1, -1, 1, 1, 1, -1, -1]], np.int8)
    payload = _fmt0_payload(codes, 1, [[0.375]], [[0.5]], [[0.25]])
    w = oracle.decode_cubic(payload, 1, FMT0, (1, 8), 8)
    assert np.array_equal(w[0], codes[0].astype(np.float32) * np.float32(0.375))


@pytest.mark.parametrize("fmt", [FMT0, FMT1, FMT2])
@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_decode_within_fp64_scalar_bound(oracle, fmt, bits):
    """FP64 scalar decode from serialized bytes (audit_checkpoint.py:32-101 method).

    The FP32 decode differs from the exact value only by rounding: <= 8 ulp-level
    relative errors of the magnitude bound |s|(1+|a|+|b|+|1-a-b|).
    """
    rng = np.random.default_rng(100 + bits)
    n, k, gi = 8, 96, 32
    codes = rng.integers(-(1 << (bits - 1)) + 1, 1 << (bits - 1), size=(n, k)).astype(np.int8)
    packed = oracle.pack_cubic(codes, bits)
    groups = (n, k // gi)
    parts = (4, 4)
    if fmt == FMT0:
        payload = {"weight_packed": packed,
                   "weight_scale": rng.uniform(0, 0.1, groups).astype(np.float32),
                   "weight_a": rng.uniform(0, 1.5, groups).astype(np.float16),
                   "weight_b": rng.uniform(-0.5, 0.5, groups).astype(np.float16)}
    elif fmt == FMT1:
        payload = {"weight_packed": packed,
                   "weight_scale": rng.integers(0, 128, groups).astype(np.int8),
                   "weight_ab": rng.integers(0, 256, groups).astype(np.uint8),
                   "weight_scale_global": rng.uniform(1e-4, 1e-3, 2).astype(np.float32),
                   "weight_a_global": rng.uniform(0, 0.1, 2).astype(np.float32),
                   "weight_b_global": rng.uniform(0, 0.1, 2).astype(np.float32)}
    else:
        payload = {"weight_packed": packed,
                   "weight_metadata": rng.integers(0, 1 << 16, groups).astype(np.uint16)
                   & np.uint16(0xDFFF),  # keep scales finite (below the fp16 inf exponent)
                   "weight_curve_a": rng.uniform(0, 1.5, (2, 4)).astype(np.float16),
                   "weight_curve_b": rng.uniform(-0.5, 0.5, (2, 4)).astype(np.float16)}
    w = oracle.decode_cubic(payload, bits, fmt, (n, k), gi, partitions=parts)

    def half(v):
        return struct.unpack("e", struct.pack("e", v))[0]

    def f32(v):
        return struct.unpack("f", struct.pack("f", v))[0]

    for r in range(n):
        part = r // 4
        for c in range(k):
            g = c // gi
            q = int(codes[r, c])
            if fmt == FMT0:
                s = float(payload["weight_scale"][r, g])
                a = float(payload["weight_a"][r, g])
                b = float(payload["weight_b"][r, g])
            elif fmt == FMT1:
                s = int(payload["weight_scale"][r, g]) * float(payload["weight_scale_global"][part])
                ab = int(payload["weight_ab"][r, g])
                lo, hi = ab & 15, ab >> 4
                lo, hi = lo - 16 if lo >= 8 else lo, hi - 16 if hi >= 8 else hi
                a = half(f32(1.0 + f32(lo * float(payload["weight_a_global"][part]))))
                b = half(f32(hi * float(payload["weight_b_global"][part])))
            else:
                m = int(payload["weight_metadata"][r, g])
                s = struct.unpack("e", struct.pack("H", (m & 0x3FFF) << 1))[0]
                a = float(payload["weight_curve_a"][part, m >> 14])
                b = float(payload["weight_curve_b"][part, m >> 14])
            d = (1 << (bits - 1)) - 1
            t = abs(q) / d
            exact = math.copysign(1.0, q) * s * t * (a + t * (b + t * (1 - a - b))) if q else 0.0
            bound = abs(s) * (1 + abs(a) + abs(b) + abs(1 - a - b)) * 8 * 2.0**-24
            assert abs(float(w[r, c]) - exact) <= bound, (r, c, q)


def test_linear_enclosure_accepts_oracle_and_rejects_corruption(oracle):
    rng = np.random.default_rng(7)
    x = oracle.f32_to_bf16_bits(rng.standard_normal((3, 256)).astype(np.float32))
    w = oracle.f32_to_bf16_bits((rng.standard_normal((40, 256)) * 0.02).astype(np.float32))
    y, y32 = oracle.linear_bf16(x, w)
    report = oracle.check_linear_enclosure(x, w, y)
    assert report["max_abs_error"] <= report["max_bound"]
    # FP64 anchor: the ascending FP32 sum is a valid FP32 dot
    anchor = oracle.bf16_bits_to_f32(x).astype(np.float64) @ oracle.bf16_bits_to_f32(w).astype(np.float64).T
    assert np.allclose(y32, anchor, rtol=1e-5, atol=1e-5)
    # A +0.25 corruption of one output is rejected (guardrail test :460-529 method)
    bad = oracle.bf16_bits_to_f32(y).copy()
    bad[1, 7] += 0.25
    with pytest.raises(AssertionError):
        oracle.check_linear_enclosure(x, w, oracle.f32_to_bf16_bits(bad))


def test_bf16_and_half_conversions_match_numpy_and_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-40, 38, 4096),
                        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 6e-8, 3e-8], np.float32)])
    x = x.astype(np.float32)
    got = oracle.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    lib = oracle.lib()
    for v in x[np.isfinite(x)][:2000]:
        assert lib.oracle_float_to_half(float(v)) == np.float16(v).view(np.uint16)
    for h in range(0, 1 << 16, 7):
        f = np.array([h], np.uint16).view(np.float16).astype(np.float32)[0]
        got_f = lib.oracle_half_to_float(h)
        assert (math.isnan(got_f) and math.isnan(f)) or got_f == f


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_torch_restatement_decode_equals_c_oracle(oracle, bits):
    """The CPU baseline's torch decode (oracle/torch_ref.py) is bit-equal to the
    C oracle for every code value, with groups of 64 and a K tail."""
    from oracle import torch_ref

    n, k, gi = 24, 200, 64
    g = torch.Generator().manual_seed(bits)
    row_bytes = (k * bits + 7) // 8
    packed = torch.randint(0, 256, (n, row_bytes), generator=g, dtype=torch.int32).to(torch.uint8)
    groups = (n, (k + gi - 1) // gi)
    payload = {"weight_packed": packed, "weight_scale": torch.rand(groups, generator=g) * 0.05,
               "weight_a": (torch.rand(groups, generator=g) * 1.5 - 0.25).half(),
               "weight_b": (torch.rand(groups, generator=g) - 0.5).half()}
    want = oracle.decode_bf16({key: v.numpy() for key, v in payload.items()}, bits,
                              "float32-scale-float16-ab", (n, k), gi)
    got = torch_ref.decode_fmt0(payload["weight_packed"], payload["weight_scale"], payload["weight_a"],
                                payload["weight_b"], bits, gi, k)
    got = got.view(torch.int16).numpy().view(np.uint16).copy()
    got[got == 0x8000] = 0
    want = want.copy()
    want[want == 0x8000] = 0
    assert np.array_equal(got, want)


def test_torch_restatement_linear_within_one_bf16_step(oracle):
    from oracle import torch_ref

    g = torch.Generator().manual_seed(3)
    x = torch.randn((5, 384), generator=g).to(torch.bfloat16)
    w = (torch.randn((40, 384), generator=g) * 0.02).to(torch.bfloat16)
    xb = x.view(torch.int16).numpy().view(np.uint16)
    wb = w.view(torch.int16).numpy().view(np.uint16)
    _, want = oracle.linear_bf16(xb, wb)
    got = torch_ref.linear_rows(x, w).float().numpy()
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-6)


def test_f16_decode_and_enclosure(oracle):
    """FP16 activations: decoded weights round once to fp16 (numpy's cast equals
    torch's, which the reference uses), and the enclosure takes fp16's unit
    roundoff: an FP32 dot rounded to fp16 passes, an output moved by eight
    fp16 ulps fails."""
    import torch
    rng = np.random.default_rng(7)
    n, k = 48, 256
    groups = n * (k // 128)
    payload = {"weight_packed": rng.integers(0, 256, (n, k * 4 // 8), dtype=np.uint8),
               "weight_scale": rng.uniform(0.001, 0.05, (n, k // 128)).astype(np.float32),
               "weight_a": rng.uniform(0, 1.5, (n, k // 128)).astype(np.float16),
               "weight_b": rng.uniform(-0.5, 0.5, (n, k // 128)).astype(np.float16)}
    assert groups == payload["weight_scale"].size
    w32 = oracle.decode_cubic(payload, 4, "float32-scale-float16-ab", (n, k), 128)
    wh = oracle.decode_f16(payload, 4, "float32-scale-float16-ab", (n, k), 128)
    assert np.array_equal(wh, torch.from_numpy(w32).half().view(torch.int16).numpy().view(np.uint16))
    x = rng.standard_normal((5, k)).astype(np.float16)
    y32 = x.astype(np.float32) @ wh.view(np.float16).astype(np.float32).T
    yh = y32.astype(np.float16)
    report = oracle.check_linear_enclosure(x.view(np.uint16), wh, yh.view(np.uint16), dtype="f16")
    assert report["max_abs_error"] <= report["max_bound"]
    bad = yh.copy()
    i = np.unravel_index(np.argmax(np.abs(bad)), bad.shape)
    bad[i] = np.float16(float(bad[i]) + 8 * float(np.spacing(bad[i])))
    with pytest.raises(AssertionError):
        oracle.check_linear_enclosure(x.view(np.uint16), wh, bad.view(np.uint16), dtype="f16")
