"""GPU parity with FP16 activations (the reference's dispatcher admits FP16 or
BF16 activations with the output in the same dtype,
ops/cuda/linear/quantized.py:348-405; its eager path rounds each decoded weight
to the activation dtype, ops/eager/quantization.py:181-182):

* one-hot identity contraction: the GEMM output is fp16(decode_cubic), bit
  for bit, for every bit width and metadata format, including the small-row
  path (M <= 4) and the level tables of 5-7 bits;
* FP16 outputs inside the FP64 enclosure with fp16's unit roundoff
  (guardrail/quantization.py:256-310), across the M regimes (small rows,
  one 64-row chunk, 128-row chunks) and the split-K plan;
* rows bitwise invariant to M; grouped members equal separate launches;
* a weight prepared for bf16 cannot be bound to fp16 activations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, quantization as qz
from test_gpu_gemm import FMTS, canon_zero, np_payload, random_matrix, to_bits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def decode_f16_bits(oracle, m: qz.QuantizedMatrix) -> np.ndarray:
    e = m.encoding
    return oracle.decode_f16(np_payload(m), e.bits, e.metadata, m.shape, e.group_in, e.group_out,
                             m.partitions)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("rows", [4, 64])
def test_identity_contraction_is_exact_f16_decode(oracle, bits, fmt, rows):
    """rows = 4 runs the small-row kernel on [4, k] slices of the identity
    (groups of 128: bits 1, 3, 5, 7; groups of 64 stay on the MFMA tile
    path); rows = 64 the MFMA tile path."""
    n, k, gi = 72, 256, 128 if bits % 2 else 64
    print(f"f16 identity bits={bits} fmt={fmt} rows={rows}", flush=True)
    m = random_matrix(n, k, bits, gi, fmt, seed=bits * 10 + FMTS.index(fmt), partitions=(40, 32))
    md = m.to(DEV)
    ops = linear.PackedLinearOperators()
    eye = torch.eye(k, dtype=torch.float16, device=DEV)
    y = torch.cat([ops.linear(eye[r:r + rows].contiguous(), md) for r in range(0, k, rows)])
    assert y.dtype is torch.float16
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(decode_f16_bits(oracle, m)))


@pytest.mark.parametrize("bits", [6, 8])
def test_identity_small_rows_curve_bits_f16(oracle, bits):
    """fp16 through the small-row kernel at 6 bits (level tables in LDS) and
    8 bits (curve evaluated per weight): [4, k] identity slices give
    fp16(decode) for every code."""
    n, k, gi = 40, 600, 128
    print(f"f16 small-row identity bits={bits}", flush=True)
    m = random_matrix(n, k, bits, gi, qz.FMT_F32, seed=bits * 31, partitions=(24, 16))
    md = m.to(DEV)
    ops = linear.PackedLinearOperators()
    eye = torch.eye(k, dtype=torch.float16, device=DEV)
    y = torch.cat([ops.linear(eye[r:r + 4].contiguous(), md) for r in range(0, k, 4)])
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(decode_f16_bits(oracle, m)))


@pytest.mark.parametrize("bits,gi", [(5, 128), (6, 256), (7, 128)])
def test_identity_level_tables_f16(oracle, bits, gi):
    n, k = 40, 600
    m = random_matrix(n, k, bits, gi, qz.FMT_F32, seed=bits + gi, partitions=(24, 16))
    y = linear.PackedLinearOperators().linear(torch.eye(k, dtype=torch.float16, device=DEV), m.to(DEV))
    got = to_bits(y.T.contiguous())
    assert np.array_equal(canon_zero(got), canon_zero(decode_f16_bits(oracle, m)))


def _check_f16(oracle, m, x, y):
    w = decode_f16_bits(oracle, m)
    report = oracle.check_linear_enclosure(to_bits(x), w, to_bits(y), dtype="f16")
    ref = x.float().cpu().numpy().astype(np.float64) @ w.view(np.float16).astype(np.float64).T
    diff = y.float().cpu().numpy().astype(np.float64) - ref
    report["vs_fp64_rel_l2"] = float(np.linalg.norm(diff) / max(np.linalg.norm(ref), 1e-30))
    print(report, flush=True)
    assert report["vs_fp64_rel_l2"] < 2e-3  # fp16 output rounding: 2^-12 relative


@pytest.mark.parametrize("mrows", [2, 8, 64, 130])
@pytest.mark.parametrize("bits", [3, 4, 8])
def test_enclosure_f16_activations(oracle, mrows, bits):
    n, k = 200, 1024
    w = torch.randn((n, k), generator=torch.Generator().manual_seed(mrows)) * 0.02
    m = qz.quantize_cubic(w, bits=bits, group_in=128)
    x = torch.randn((mrows, k), generator=torch.Generator().manual_seed(99)).half().to(DEV)
    y = linear.PackedLinearOperators().linear(x, m.to(DEV))
    assert y.dtype is torch.float16
    _check_f16(oracle, m, x, y)


def test_split_k_f16(oracle):
    n, k = 64, 12288
    m = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(5)) * 0.02, 4)
    x = torch.randn((64, k), generator=torch.Generator().manual_seed(6)).half().to(DEV)
    out = torch.empty((64, n), dtype=torch.float16, device=DEV)
    binding = linear.PackedLinearOperators().bind_linear(x, m.to(DEV), out)
    assert binding.scratch, "expected a split-K workspace"
    binding.launch()
    first = out.clone()
    out.zero_()
    binding.launch()
    assert torch.equal(out, first)
    _check_f16(oracle, m, x, first)


def test_f16_rows_invariant_and_grouped_equals_separate():
    n, k = 1024, 4096
    ops = linear.PackedLinearOperators()
    gate = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(1)) * 0.02, 4).to(DEV)
    up = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(2)) * 0.02, 4).to(DEV)
    base = torch.randn((130, k), generator=torch.Generator().manual_seed(3)).half().to(DEV)
    ref = ops.linear(base[:5].contiguous(), gate)[:1]
    for mrows in (8, 64, 65, 130):
        assert torch.equal(ops.linear(base[:mrows].contiguous(), gate)[:1], ref), mrows
    for mrows in (3, 64, 130):
        x = base[:mrows].contiguous()
        yg = torch.empty((mrows, n), dtype=torch.float16, device=DEV)
        yu = torch.empty_like(yg)
        ops.bind_linear_group(x, (gate, up), (yg, yu)).launch()
        assert torch.equal(yg, ops.linear(x, gate)), mrows
        assert torch.equal(yu, ops.linear(x, up)), mrows


def test_prepared_dtype_must_match_activations():
    m = qz.quantize_cubic(torch.randn((64, 256), generator=torch.Generator().manual_seed(4)) * 0.02, 4)
    prepared = linear.prepare_matrix(m.to(DEV), torch.device(DEV))  # bf16 level tables
    x = torch.randn((8, 256), device=DEV).half()
    with pytest.raises(ValueError, match="prepared dtype"):
        linear.bind_prepared(x, prepared, (torch.empty((8, 64), dtype=torch.float16, device=DEV),))
    ph = linear.prepare_matrix(m.to(DEV), torch.device(DEV), torch.float16)
    assert torch.equal(ph.codes, prepared.codes)  # the code stream does not depend on the dtype
    out = torch.empty((8, 64), dtype=torch.float16, device=DEV)
    linear.bind_prepared(x, ph, (out,)).launch()
    assert torch.equal(out, linear.PackedLinearOperators().linear(x, m.to(DEV)))


def test_moe_routed_f16(oracle):
    """Routed experts with FP16 activations: every route row inside its
    expert's fp16 enclosure.  (Routed launches keep K whole; a dense launch of
    the same small expert may split K, so the two need not agree bit for bit.)"""
    from cubic_serve_amd import moe
    experts, tokens, top_k, n, k, block_m = 6, 20, 2, 64, 512, 32
    g = torch.Generator(device=DEV).manual_seed(1)
    gate = tuple(qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
                 for _ in range(experts))
    up = tuple(qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
               for _ in range(experts))
    x = torch.randn((tokens, k), generator=g, device=DEV).half()
    logits = torch.randn((tokens, experts), generator=g, device=DEV)
    logits[:, 0] += 2.0
    ids = torch.argsort(logits, dim=-1, descending=True, stable=True)[:, :top_k]
    rows = moe.route_rows(ids, experts, block_m)
    out = torch.full((tokens * top_k, 2 * n), float("nan"), dtype=torch.float16, device=DEV)
    ops = linear.PackedLinearOperators()
    _, binding = moe.bind_grouped(ops, x, gate, up, out, rows, top_k, moe.CubicMoEParameters(block_m=block_m))
    binding.launch()
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    flat = ids.reshape(-1).cpu().numpy()
    for r in range(tokens * top_k):
        e, t = int(flat[r]), r // top_k
        for c, w in enumerate((gate[e], up[e])):
            wb = decode_f16_bits(oracle, w)
            oracle.check_linear_enclosure(to_bits(x[t:t + 1]), wb, to_bits(out[r:r + 1, c * n:(c + 1) * n]),
                                          dtype="f16")
