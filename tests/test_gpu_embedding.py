"""GPU parity: the packed Cubic embedding lookup against the CPU oracle.

Method of the reference's tests (tests/ops/test_cuda_quantized.py):
* every code of every bit width through the lookup, fp16 and bf16 outputs
  (:341-378, fixture rebuilt here from its description);
* random payloads of the three metadata formats, output groups, partitions,
  ragged K and id shapes: rows bit-equal to the reference decode rounded to
  the output dtype (:655-659 ``embedding_matrix`` equality);
* a bound lookup captured in a HIP graph reads its ids at replay (:699-715);
* the Qwen3-8B embedding shape (151936 x 4096, W4 g128) on sampled tokens.
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


def np_payload(m: qz.QuantizedMatrix) -> dict:
    return {k: v.cpu().numpy() for k, v in m.payload.items()}


def expected_rows(oracle, m: qz.QuantizedMatrix, ids: np.ndarray, dtype) -> np.ndarray:
    """Reference decode of the looked-up rows, rounded once to ``dtype`` (uint16 bits)."""
    e = m.encoding
    w = oracle.decode_cubic(np_payload(m), e.bits, e.metadata, m.shape, e.group_in, e.group_out,
                            m.partitions)
    flat = ids.reshape(-1)
    rows = np.zeros((flat.size, m.shape[1]), np.float32)
    ok = (flat >= 0) & (flat < m.shape[0])
    rows[ok] = w[flat[ok]]
    if dtype == torch.float16:
        bits = rows.astype(np.float16).view(np.uint16)
    else:
        bits = oracle.f32_to_bf16_bits(rows)
    return bits.reshape(*ids.shape, m.shape[1])


def got_bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def random_matrix(n, k, bits, group_in, group_out, fmt, seed, partitions=()):
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (n, math.ceil(k * bits / 8)), generator=g,
                           dtype=torch.int32).to(torch.uint8)
    groups = (n // group_out, math.ceil(k / group_in))
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
    enc = qz.QuantizationScheme(qz.CUBIC_FORMAT, bits, group_in, group_out, fmt)
    return qz.QuantizedMatrix({k: v.to(DEV) for k, v in payload.items()}, enc, (n, k), tuple(partitions))


def all_codes_matrix(bits: int) -> qz.QuantizedMatrix:
    """Every code of ``bits`` (incl. the reserved one) in each of 4 rows, one
    curve per row: scale 2^-7 (e5m9 0x1000), curves a = (0.5, 0.75, 1, 1.25),
    b = (-0.25, 0.125, 0.25, -0.125), group_in 32."""
    k = 256
    codes = np.arange(k) % (1 << bits)
    planes = ((codes[:, None] >> np.arange(bits)) & 1).reshape(-1)
    packed = np.packbits(planes.astype(np.uint8), bitorder="little")
    payload = {
        "weight_packed": torch.from_numpy(np.tile(packed, (4, 1))),
        "weight_metadata": torch.tensor([[0x1000 | (c << 14)] * (k // 32) for c in range(4)],
                                        dtype=torch.int32).to(torch.uint16),
        "weight_curve_a": torch.tensor([[0.5, 0.75, 1.0, 1.25]], dtype=torch.float16),
        "weight_curve_b": torch.tensor([[-0.25, 0.125, 0.25, -0.125]], dtype=torch.float16),
    }
    enc = qz.QuantizationScheme(qz.CUBIC_FORMAT, bits, 32, 1, qz.FMT_CURVE2)
    return qz.QuantizedMatrix({k: v.to(DEV) for k, v in payload.items()}, enc, (4, k))


@pytest.mark.parametrize("bits", range(1, 9))
def test_every_code_every_width(oracle, bits):
    print(f"embedding all-codes bits={bits}", flush=True)
    m = all_codes_matrix(bits)
    ops = linear.PackedLinearOperators()
    for id_dtype in (torch.int64, torch.int32):
        ids = torch.arange(4, device=DEV, dtype=id_dtype)
        for dtype in (torch.float16, torch.bfloat16):
            got = ops.embedding(ids, m, dtype=dtype)
            torch.cuda.synchronize()
            want = expected_rows(oracle, m, ids.cpu().numpy(), dtype)
            assert np.array_equal(got_bits(got), want), (bits, id_dtype, dtype)


CASES = [
    # n, k, bits, group_in, group_out, partitions
    (48, 256, 4, 128, 1, ()),
    (48, 200, 3, 64, 1, (16, 32)),     # partial last group, 3-bit rows not word aligned
    (64, 203, 5, 32, 2, (32, 32)),     # odd K: tail chunk of 3 columns
    (40, 1024, 8, 128, 4, (24, 16)),
    (40, 96, 1, 32, 1, ()),
    (32, 136, 2, 8, 1, ()),            # groups narrower than one 8-column chunk
    (24, 2112, 6, 96, 1, ()),          # two column blocks
    (16, 12, 7, 5, 1, ()),             # group_in not a multiple of anything
    (24, 4160, 4, 64, 1, (8, 16)),     # table path over two column slices, the second partial
    (16, 4096, 2, 16, 1, ()),          # table path with the smallest admitted groups
]


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("case", range(len(CASES)))
def test_random_payloads_bit_exact(oracle, fmt, case):
    n, k, bits, gi, go, parts = CASES[case]
    print(f"embedding random fmt={fmt} case={CASES[case]}", flush=True)
    m = random_matrix(n, k, bits, gi, go, fmt, seed=17 * case + FMTS.index(fmt), partitions=parts)
    ops = linear.PackedLinearOperators()
    g = torch.Generator().manual_seed(case)
    ids = torch.randint(0, n, (2, 5), generator=g)
    ids[0, 0], ids[0, 1], ids[1, 4] = 0, n - 1, ids[1, 3]  # first, last, repeated
    for dtype in (torch.bfloat16, torch.float16):
        got = ops.embedding(ids.to(DEV), m, dtype=dtype)
        torch.cuda.synchronize()
        assert got.shape == (2, 5, k)
        assert np.array_equal(got_bits(got), expected_rows(oracle, m, ids.numpy(), dtype)), dtype


def test_out_of_range_ids_give_zero_rows(oracle):
    m = random_matrix(32, 128, 4, 32, 1, qz.FMT_F32, seed=5)
    ids = torch.tensor([3, -1, 32, 1 << 40, 31], dtype=torch.int64)
    got = linear.PackedLinearOperators().embedding(ids.to(DEV), m, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = expected_rows(oracle, m, ids.numpy(), torch.bfloat16)
    assert np.array_equal(got_bits(got), want)
    assert not got_bits(got)[1:4].any()


def test_bound_lookup_graph_reads_ids_at_replay(oracle):
    m = random_matrix(40, 128, 4, 32, 1, qz.FMT_I8, seed=9, partitions=(24, 16))
    ops = linear.PackedLinearOperators()
    for capacity in (1, 8, 64):
        ids = torch.arange(capacity, device=DEV) % 40
        out = torch.empty((capacity, 128), dtype=torch.bfloat16, device=DEV)
        lookup = ops.bind_embedding(ids, m, out)
        lookup.launch()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            lookup.launch()
        for i in range(3):
            ids.copy_((ids.flip(0) * 7 + i) % 40)
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            want = expected_rows(oracle, m, ids.cpu().numpy(), torch.bfloat16)
            assert np.array_equal(got_bits(out), want), (capacity, i)


def test_bind_validation():
    m = random_matrix(16, 64, 4, 32, 1, qz.FMT_F32, seed=1)
    ops = linear.PackedLinearOperators()
    ids = torch.arange(4, device=DEV)
    ok = torch.empty((4, 64), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.bind_embedding(ids.cpu(), m, ok)
    with pytest.raises(ValueError):
        ops.bind_embedding(ids.float(), m, ok)
    with pytest.raises(ValueError):
        ops.bind_embedding(ids, m, torch.empty((4, 64), dtype=torch.float32, device=DEV))
    with pytest.raises(ValueError):
        ops.bind_embedding(ids, m, torch.empty((4, 63), dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError):
        ops.bind_embedding(ids[:0], m, ok[:0])
    binding = ops.bind_embedding(ids, m, ok)
    ids.resize_(5)
    with pytest.raises(ValueError, match="changed after binding"):
        binding.launch()


def test_qwen3_8b_embedding_shape_sampled(oracle):
    n, k = 151936, 4096
    g = torch.Generator(device=DEV).manual_seed(11)
    groups = (n, k // 128)
    payload = {"weight_packed": torch.randint(0, 256, (n, k // 2), generator=g, device=DEV,
                                              dtype=torch.int32).to(torch.uint8),
               "weight_scale": torch.rand(groups, generator=g, device=DEV) * 0.05,
               "weight_a": (torch.rand(groups, generator=g, device=DEV) * 1.5 - 0.25).half(),
               "weight_b": (torch.rand(groups, generator=g, device=DEV) - 0.5).half()}
    m = qz.QuantizedMatrix(payload, qz.QuantizationScheme(qz.CUBIC_FORMAT, 4, 128), (n, k))
    ids = torch.randint(0, n, (64,), generator=g, device=DEV)
    ids[0], ids[1] = 0, n - 1
    got = linear.PackedLinearOperators().embedding(ids, m, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got_np = got_bits(got)
    for i in (0, 1, 2, 31, 63):
        row = int(ids[i])
        part = m.rows(row, row + 1)
        assert np.array_equal(got_np[i], expected_rows(oracle, part, np.array([0]), torch.bfloat16)[0]), i
