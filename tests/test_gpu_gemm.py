"""GPU parity: the Cubic GEMM against the CPU oracle.

* one-hot identity contraction: the GEMM output is the decoded weight matrix,
  bit for bit equal to bf16(decode_cubic) (tests/ops/test_cubic_marlin.py:285-318
  method, zero signs canonicalised);
* every output inside the FP64 enclosure of guardrail/quantization.py:176-320,
  with max-abs and relative-L2 error reported against the oracle's FP32 GEMM;
* bitwise invariance of a row's output to M and to row permutation;
* grouped (gate/up) launch equal to the separate launches.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, quantization as qz

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
FMTS = (qz.FMT_F32, qz.FMT_I8, qz.FMT_CURVE2)


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_payload(m: qz.QuantizedMatrix) -> dict:
    return {k: v.cpu().numpy() for k, v in m.payload.items()}


def random_matrix(n, k, bits, group_in, fmt, seed, partitions=()):
    """Random payload of every metadata format (reference test style)."""
    g = torch.Generator().manual_seed(seed)
    rows_bytes = math.ceil(k * bits / 8)
    packed = torch.randint(0, 256, (n, rows_bytes), generator=g, dtype=torch.int32).to(torch.uint8)
    groups = (n, math.ceil(k / group_in))
    parts = partitions or (n,)
    if fmt == qz.FMT_F32:
        payload = {"weight_packed": packed,
                   "weight_scale": torch.rand(groups, generator=g) * 0.05,
                   "weight_a": (torch.rand(groups, generator=g) * 1.5 - 0.25).half(),
                   "weight_b": (torch.rand(groups, generator=g) - 0.5).half()}
    elif fmt == qz.FMT_I8:
        payload = {"weight_packed": packed,
                   "weight_scale": torch.randint(0, 128, groups, generator=g, dtype=torch.int32).to(torch.int8),
                   "weight_ab": torch.randint(0, 256, groups, generator=g, dtype=torch.int32).to(torch.uint8),
                   "weight_scale_global": torch.rand(len(parts), generator=g) * 1e-3 + 1e-4,
                   "weight_a_global": torch.rand(len(parts), generator=g) * 0.1,
                   "weight_b_global": torch.rand(len(parts), generator=g) * 0.1}
    else:
        md = torch.randint(0, 1 << 16, groups, generator=g, dtype=torch.int32) & 0xDFFF
        payload = {"weight_packed": packed,
                   "weight_metadata": md.to(torch.uint16),
                   "weight_curve_a": (torch.rand((len(parts), 4), generator=g) * 1.5).half(),
                   "weight_curve_b": (torch.rand((len(parts), 4), generator=g) - 0.5).half()}
    enc = qz.QuantizationScheme(qz.CUBIC_FORMAT, bits, group_in, 1, fmt)
    return qz.QuantizedMatrix(payload, enc, (n, k), tuple(partitions))


def oracle_decode_bits(oracle, m: qz.QuantizedMatrix) -> np.ndarray:
    e = m.encoding
    return oracle.decode_bf16(np_payload(m), e.bits, e.metadata, m.shape, e.group_in,
                              e.group_out, m.partitions)


def canon_zero(bits: np.ndarray) -> np.ndarray:
    out = bits.copy()
    out[out == 0x8000] = 0
    return out


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("fmt", FMTS)
def test_identity_contraction_is_exact_decode(oracle, bits, fmt):
    n, k, gi = 72, 256, 128 if bits % 2 else 64
    print(f"identity bits={bits} fmt={fmt} gi={gi}", flush=True)
    m = random_matrix(n, k, bits, gi, fmt, seed=bits * 10 + FMTS.index(fmt), partitions=(40, 32))
    x = torch.eye(k, dtype=torch.bfloat16, device=DEV)
    y = linear.PackedLinearOperators().linear(x, m.to(DEV))
    torch.cuda.synchronize()
    got = to_bits(y.T.contiguous())        # [n, k] decoded weights
    want = oracle_decode_bits(oracle, m)
    assert np.array_equal(canon_zero(got), canon_zero(want))


@pytest.mark.parametrize("bits", [5, 6, 7])
@pytest.mark.parametrize("gi", [128, 256])
@pytest.mark.parametrize("fmt", FMTS)
def test_identity_level_table_bits_exact(oracle, bits, gi, fmt):
    """5-7 bits with groups of whole k-blocks decode through per-k-block level
    tables in LDS: every code's output equals bf16(decode_cubic), including a
    group that spans two k-blocks and a K tail."""
    n, k = 40, 600  # 4 whole k-blocks and a tail of 88
    m = random_matrix(n, k, bits, gi, fmt, seed=bits * 100 + gi + FMTS.index(fmt), partitions=(24, 16))
    x = torch.eye(k, dtype=torch.bfloat16, device=DEV)
    y = linear.PackedLinearOperators().linear(x, m.to(DEV))
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(oracle_decode_bits(oracle, m)))


@pytest.mark.parametrize("bits", [5, 6, 7, 8])
@pytest.mark.parametrize("gi,fmt", [(128, qz.FMT_F32), (256, FMTS[1]), (128, FMTS[2])])
def test_identity_small_rows_curve_bits_exact(oracle, bits, gi, fmt):
    """Above 4 bits the small-row kernel (M <= 4, K <= 64 k-blocks) evaluates
    every weight from the curve: [4, k] slices of the identity give
    bf16(decode_cubic) for every code, a group spanning two k-blocks and a K
    tail included."""
    n, k = 40, 600
    print(f"small-row identity bits={bits} gi={gi} fmt={fmt}", flush=True)
    m = random_matrix(n, k, bits, gi, fmt, seed=bits * 7 + gi + FMTS.index(fmt), partitions=(24, 16))
    md = m.to(DEV)
    ops = linear.PackedLinearOperators()
    eye = torch.eye(k, dtype=torch.bfloat16, device=DEV)
    y = torch.cat([ops.linear(eye[r:r + 4].contiguous(), md) for r in range(0, k, 4)])
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(oracle_decode_bits(oracle, m)))


@pytest.mark.parametrize("k,gi", [(200, 32), (384, 256), (136, 128)])
def test_identity_partial_groups_and_k_tails(oracle, k, gi):
    m = random_matrix(33, k, 4, gi, qz.FMT_F32, seed=k)
    x = torch.eye(k, dtype=torch.bfloat16, device=DEV)
    y = linear.PackedLinearOperators().linear(x, m.to(DEV))
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(oracle_decode_bits(oracle, m)))


def _check_linear(oracle, m: qz.QuantizedMatrix, x: torch.Tensor, y: torch.Tensor) -> dict:
    w = oracle_decode_bits(oracle, m)
    xb, yb = to_bits(x), to_bits(y)
    report = oracle.check_linear_enclosure(xb, w, yb)
    _, ref32 = oracle.linear_bf16(xb, w)
    yf = oracle.bf16_bits_to_f32(yb).astype(np.float64)
    diff = yf - ref32
    report["vs_oracle_max_abs"] = float(np.abs(diff).max())
    report["vs_oracle_rel_l2"] = float(np.linalg.norm(diff) / max(np.linalg.norm(ref32), 1e-30))
    print(report, flush=True)
    assert report["vs_oracle_rel_l2"] < 1e-2  # bf16 output rounding dominates (2^-9 relative)
    return report


@pytest.mark.parametrize("mrows", [1, 2, 3, 8, 17, 33, 64, 65, 130])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_enclosure_random_activations(oracle, mrows, bits):
    n, k = 200, 1024
    w = torch.randn((n, k), generator=torch.Generator().manual_seed(mrows)) * 0.02
    m = qz.quantize_cubic(w, bits=bits, group_in=128)
    x = torch.randn((mrows, k), generator=torch.Generator().manual_seed(99)).to(torch.bfloat16).to(DEV)
    y = linear.PackedLinearOperators().linear(x, m.to(DEV))
    _check_linear(oracle, m, x, y)


def test_split_k_path_enclosure_and_repeatability(oracle):
    # small N, long K: the plan splits K and merges partials in order
    n, k = 64, 12288
    m = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(5)) * 0.02, 4)
    x = torch.randn((64, k), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    out = torch.empty((64, n), dtype=torch.bfloat16, device=DEV)
    binding = linear.PackedLinearOperators().bind_linear(x, m.to(DEV), out)
    assert binding.scratch, "expected a split-K workspace"
    binding.launch()
    first = out.clone()
    for _ in range(3):
        out.zero_()
        binding.launch()
        assert torch.equal(out, first)
    _check_linear(oracle, m, x, first)


def test_row_is_invariant_to_m_and_permutation():
    # The launch plan's K partition depends on (n, k) only, so each row's
    # summation order is the same for every M of one arithmetic regime: the
    # small-row kernel (M <= 4) and the MFMA-tile kernel (M >= 5), also past
    # one 64-row chunk.
    n, k = 4096, 4096
    m = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(1)) * 0.02, 4)
    md = m.to(DEV)
    ops = linear.PackedLinearOperators()
    base = torch.randn((130, k), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    for regime in ((1, 2, 3, 4), (5, 8, 17, 33, 64, 65, 130)):
        ref = ops.linear(base[:regime[0]].contiguous(), md)[:1]
        for mrows in regime[1:]:
            y = ops.linear(base[:mrows].contiguous(), md)
            assert torch.equal(y[:1], ref), mrows
    for mrows in (64, 65, 130):
        perm = torch.randperm(mrows, generator=torch.Generator().manual_seed(3)).to(DEV)
        y = ops.linear(base[:mrows].contiguous(), md)
        yp = ops.linear(base[:mrows][perm].contiguous(), md)
        assert torch.equal(yp, y[perm]), mrows


def test_grouped_equals_separate_members():
    k = 2048
    gate = qz.quantize_cubic(torch.randn((768, k), generator=torch.Generator().manual_seed(7)) * 0.02, 4)
    up = qz.quantize_cubic(torch.randn((768, k), generator=torch.Generator().manual_seed(8)) * 0.02, 4)
    gate, up = gate.to(DEV), up.to(DEV)
    x = torch.randn((64, k), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(DEV)
    ops = linear.PackedLinearOperators()
    y0 = torch.empty((64, 768), dtype=torch.bfloat16, device=DEV)
    y1 = torch.empty_like(y0)
    ops.bind_linear_group(x, (gate, up), (y0, y1)).launch()
    assert torch.equal(y0, ops.linear(x, gate))
    assert torch.equal(y1, ops.linear(x, up))


def test_lm_head_cfg2_shape_sampled_enclosure(oracle):
    """Qwen3-8B lm_head 151936 x 4096 W4 at M=64: enclosure on sampled row blocks."""
    n, k = 151936, 4096
    g = torch.Generator(device=DEV).manual_seed(0)
    w = torch.randn((n, k), generator=g, device=DEV) * 0.02
    m = qz.quantize_cubic(w, bits=4, group_in=128)
    del w
    x = torch.randn((64, k), generator=torch.Generator(device=DEV).manual_seed(1), device=DEV).to(torch.bfloat16)
    y = linear.PackedLinearOperators().linear(x, m)
    torch.cuda.synchronize()
    for start in (0, 75968, n - 256):
        part = m.rows(start, start + 256).to("cpu")
        _check_linear(oracle, part, x, y[:, start:start + 256])


def test_wide_output_repeatable_and_row_invariant(oracle):
    """A wide output (640 column blocks: more than one round of resident
    workgroups): enclosure on sampled column ranges, repeatability, and a
    row's output independent of M up to 64 rows."""
    n, k = 81920, 1024
    g = torch.Generator(device=DEV).manual_seed(11)
    m = qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
    x = torch.randn((64, k), generator=torch.Generator(device=DEV).manual_seed(12), device=DEV).to(torch.bfloat16)
    out = torch.empty((64, n), dtype=torch.bfloat16, device=DEV)
    ops = linear.PackedLinearOperators()
    binding = ops.bind_linear(x, m, out)
    binding.launch()
    first = out.clone()
    for _ in range(3):
        out.zero_()
        binding.launch()
        assert torch.equal(out, first)
    for start in (0, 512 * 128 - 128, 600 * 128, n - 256):
        part = m.rows(start, start + 256).to("cpu")
        _check_linear(oracle, part, x, first[:, start:start + 256])
    for mrows in (5, 17, 33):
        y = ops.linear(x[:mrows].contiguous(), m)
        assert torch.equal(y, first[:mrows]), mrows
    small = ops.linear(x[:4].contiguous(), m)  # the small-row regime (M <= 4)
    for mrows in (1, 2):
        y = ops.linear(x[:mrows].contiguous(), m)
        assert torch.equal(y, small[:mrows]), mrows


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
def test_llama70b_cfg5_shapes_sampled_enclosure(oracle, bits):
    """Llama-3-70B layer linears (qkv 8192 -> 10240, o
    8192 -> 8192, gate/up 8192 -> 2 x 28672 as one grouped launch, down
    28672 -> 8192), weights N(0, 0.02), at M = 1, 8, 64, 512: every sampled
    output inside the FP64 enclosure (64 columns per linear at a position that
    moves with M; at M = 512 the first and last 64-row chunks), and a row's
    output equal for M = 8 and 64 (MFMA-tile regime)."""
    print(f"cfg5 bits={bits}", flush=True)
    hidden, qkv, inter = 8192, 10240, 28672
    g = torch.Generator(device=DEV).manual_seed(100 + bits)

    def quant(n, k):
        w = torch.randn((n, k), generator=g, device=DEV) * 0.02
        m = qz.quantize_cubic(w, bits=bits, group_in=128)
        del w
        return m

    ops = linear.PackedLinearOperators()
    mats = {"qkv": quant(qkv, hidden), "o": quant(hidden, hidden), "down": quant(hidden, inter)}
    gate, up = quant(inter, hidden), quant(inter, hidden)
    for mi, mrows in enumerate((1, 8, 64, 512)):
        x = torch.randn((mrows, hidden), generator=g, device=DEV).to(torch.bfloat16)
        xd = torch.randn((mrows, inter), generator=g, device=DEV).to(torch.bfloat16)
        row_sets = [slice(0, mrows)] if mrows <= 64 else [slice(0, 64), slice(mrows - 64, mrows)]
        outs = {name: ops.linear(xd if name == "down" else x, m) for name, m in mats.items()}
        yg = torch.empty((mrows, inter), dtype=torch.bfloat16, device=DEV)
        yu = torch.empty((mrows, inter), dtype=torch.bfloat16, device=DEV)
        ops.bind_linear_group(x, (gate, up), (yg, yu)).launch()
        torch.cuda.synchronize()
        checks = [(m, xd if name == "down" else x, outs[name]) for name, m in mats.items()]
        checks += [(gate, x, yg), (up, x, yu)]
        for m, xin, y in checks:
            n = m.shape[0]
            start = (mi * 1237 * 16) % (n - 64)
            part = m.rows(start, start + 64).to("cpu")
            for rows in row_sets:
                _check_linear(oracle, part, xin[rows].contiguous(), y[rows, start:start + 64].contiguous())
        if mrows == 64:
            for name, m in mats.items():
                xin = xd if name == "down" else x
                for sub in (8,):
                    assert torch.equal(ops.linear(xin[:sub].contiguous(), m), outs[name][:sub]), (name, sub)
