"""GPU: the GEMM's K plan is a function of one member's (n, k) only.

Mirrors the reference's Marlin ownership tests (tests/ops/test_cubic_marlin.py
:38-107 and :357-420): grouped members bitwise equal to separate launches,
row 0 bitwise equal for every M (past one 64-row chunk too), a HIP-graph
replay after a row permutation, rows past M untouched (NaN-poisoned), plus
sampled FP64-enclosure checks at the shipped plans of the BASELINE shapes
(cfg2 layer linears at M=64, the cfg3 W3 lm_head at M=256) and grouped ==
separate at the Llama-3-70B gate/up shape.
"""
from __future__ import annotations

import pytest
import torch

from cubic_serve_amd import linear, quantization as qz
from test_gpu_gemm import _check_linear, random_matrix

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits16(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


@pytest.mark.parametrize("bits,group", [(2, 32), (4, 512), (8, 128)])
def test_grouped_three_members_preserve_reduction_and_ownership(bits, group):
    print(f"grouped 3 members bits={bits} group={group}", flush=True)
    n, k = 128, 2048
    weights = tuple(random_matrix(n, k, bits, group, qz.FMT_I8, seed=418 + i, partitions=(64, 64)).to(DEV)
                    for i in range(3))
    corpus = (torch.randn((65, k), generator=torch.Generator().manual_seed(418)) * 0.02).to(torch.bfloat16).to(DEV)
    ops = linear.PackedLinearOperators()
    first = None
    for m in (1, 3, 8, 17, 33, 65):
        if m == 8:
            first = None  # M >= 5 is the MFMA-tile regime: a different (fixed) arithmetic
        x = corpus[:m].clone()
        storage = tuple(torch.full((66, n), float("nan"), dtype=torch.bfloat16, device=DEV) for _ in weights)
        outputs = tuple(t[:m] for t in storage)
        expected = []
        for w, y in zip(weights, outputs):
            ops.bind_linear(x, w, y).launch()
            expected.append(y.clone())
        grouped = ops.bind_linear_group(x, weights, outputs)
        assert len(grouped._launches) == 1  # one launch for the three members
        grouped.launch()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            grouped.launch()
        graph.replay()
        torch.cuda.synchronize()
        for y, want, protected in zip(outputs, expected, storage):
            assert torch.equal(_bits16(y), _bits16(want))
            assert torch.isnan(protected[m:].float()).all()
        if first is not None:
            assert all(torch.equal(_bits16(y[:1]), _bits16(f)) for y, f in zip(outputs, first))
        first = tuple(y[:1].clone() for y in outputs)
        permutation = torch.arange(m - 1, -1, -1, device=DEV)
        x.copy_(corpus[:m][permutation])
        graph.replay()
        torch.cuda.synchronize()
        for y, want, protected in zip(outputs, expected, storage):
            assert torch.equal(_bits16(y), _bits16(want[permutation]))
            assert torch.isnan(protected[m:].float()).all()
        graph.reset()


@pytest.mark.parametrize("n,k", [(4096, 4096), (128, 4352), (6144, 4096)])
def test_row_invariant_across_m_past_one_chunk(n, k):
    """MFMA-tile regime (M >= 5): row 0 and the last row equal across M."""
    print(f"row invariance n={n} k={k}", flush=True)
    w = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(n + k)) * 0.02, 4).to(DEV)
    ops = linear.PackedLinearOperators()
    corpus = torch.randn((130, k), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
    ref = ops.linear(corpus[:5].contiguous(), w)[:1]
    for m in (8, 37, 64, 65, 128, 130):
        y = ops.linear(corpus[:m].contiguous(), w)
        assert torch.equal(_bits16(y[:1]), _bits16(ref)), m
        # the last row too: its own chunk position changes with m
        last = ops.linear(corpus[m - 5:m].contiguous(), w)[4:]
        assert torch.equal(_bits16(y[m - 1:m]), _bits16(last)), m


@pytest.mark.parametrize("bits", [4, 6, 8])
@pytest.mark.parametrize("n,k", [(4096, 4096), (32768, 2048), (48, 4352), (256, 2176), (144, 8320)])
def test_small_rows_regime_invariant_and_enclosed(oracle, n, k, bits):
    """Small-row regime (M <= 4): every row equal across M = 1..4 and to a
    permuted launch, outputs inside the FP64 enclosure (K tails included).
    k = 8320 is 65 k-blocks: 6 bits run the MFMA-tile kernel there, 4 and 8
    bits the small-row kernel."""
    print(f"small rows n={n} k={k} bits={bits}", flush=True)
    w = qz.quantize_cubic(torch.randn((n, k), generator=torch.Generator().manual_seed(n * 3 + k)) * 0.02, bits)
    wd = w.to(DEV)
    ops = linear.PackedLinearOperators()
    x = torch.randn((4, k), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    y4 = ops.linear(x, wd)
    for m in (1, 2, 3):
        assert torch.equal(_bits16(ops.linear(x[:m].contiguous(), wd)), _bits16(y4[:m])), m
    perm = torch.tensor([2, 0, 3, 1], device=DEV)
    assert torch.equal(_bits16(ops.linear(x[perm].contiguous(), wd)), _bits16(y4[perm]))
    cols = min(n, 256)
    for start in sorted({0, (n - cols) // 2 // 16 * 16, n - cols}):
        part = w.rows(start, start + cols)
        _check_linear(oracle, part, x, y4[:, start:start + cols].contiguous())


@pytest.mark.parametrize("m", [1, 8, 64, 130])
def test_grouped_equals_separate_llama70b_gate_up(m):
    """cfg5 gate/up: two 28672 x 8192 members in one launch equal separate launches."""
    print(f"cfg5 gate/up grouped == separate m={m}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(70)
    gate = qz.quantize_cubic(torch.randn((28672, 8192), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
    up = qz.quantize_cubic(torch.randn((28672, 8192), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
    x = torch.randn((m, 8192), generator=g, device=DEV).to(torch.bfloat16)
    ops = linear.PackedLinearOperators()
    yg = torch.empty((m, 28672), dtype=torch.bfloat16, device=DEV)
    yu = torch.empty_like(yg)
    ops.bind_linear_group(x, (gate, up), (yg, yu)).launch()
    assert torch.equal(_bits16(yg), _bits16(ops.linear(x, gate)))
    assert torch.equal(_bits16(yu), _bits16(ops.linear(x, up)))


def test_cfg2_layer_shapes_at_shipped_plans_sampled_enclosure(oracle):
    """Qwen3-8B layer linears at M=64 (qkv, o, grouped gate/up, down): sampled
    64-column slices inside the FP64 enclosure of the oracle's decode."""
    g = torch.Generator(device=DEV).manual_seed(8)
    hidden, inter = 4096, 12288

    def quant(n, k):
        return qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4, group_in=128)

    ops = linear.PackedLinearOperators()
    x = torch.randn((64, hidden), generator=g, device=DEV).to(torch.bfloat16)
    xd = torch.randn((64, inter), generator=g, device=DEV).to(torch.bfloat16)
    qkv, o, down = quant(6144, hidden), quant(hidden, hidden), quant(hidden, inter)
    gate, up = quant(inter, hidden), quant(inter, hidden)
    yg = torch.empty((64, inter), dtype=torch.bfloat16, device=DEV)
    yu = torch.empty_like(yg)
    ops.bind_linear_group(x, (gate, up), (yg, yu)).launch()
    checks = [(qkv, x, ops.linear(x, qkv)), (o, x, ops.linear(x, o)), (down, xd, ops.linear(xd, down)),
              (gate, x, yg), (up, x, yu)]
    torch.cuda.synchronize()
    for w, xin, y in checks:
        n = w.shape[0]
        for start in (0, (n // 2) // 16 * 16, n - 64):
            print(f"cfg2 layer n={n} k={w.shape[1]} cols {start}", flush=True)
            part = w.rows(start, start + 64).to("cpu")
            _check_linear(oracle, part, xin, y[:, start:start + 64].contiguous())


def test_cfg3_w3_lm_head_m256_sampled_enclosure(oracle):
    """cfg3 lm_head 151936 x 4096, Cubic W3 g128, at M=256 (four 64-row chunks)."""
    n, k = 151936, 4096
    g = torch.Generator(device=DEV).manual_seed(3)
    w = qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=3, group_in=128)
    x = torch.randn((256, k), generator=g, device=DEV).to(torch.bfloat16)
    y = linear.PackedLinearOperators().linear(x, w)
    torch.cuda.synchronize()
    for start in (0, 75968, n - 64):
        part = w.rows(start, start + 64).to("cpu")
        for rows in (slice(0, 64), slice(192, 256)):
            print(f"cfg3 lm_head cols {start} rows {rows}", flush=True)
            _check_linear(oracle, part, x[rows].contiguous(), y[rows, start:start + 64].contiguous())


@pytest.mark.parametrize("n,k,gi,bits", [
    (4096, 4096, 128, 4),    # split 4, even partitions
    (48, 4352, 128, 4),      # split 8, odd partitions (a pad block each)
    (6144, 4096, 64, 3),     # per-quarter groups
    (256, 2176, 32, 2),      # K tail, groups of 32
    (24576, 1024, 128, 1),   # split 1
])
@pytest.mark.parametrize("f16", [False, True])
def test_sixteen_rows_equal_mfma_tile_rows(n, k, gi, bits, f16):
    """One m-tile (5..16 rows) and two (17 rows) of the MFMA-tile kernel:
    the first 16 rows of an M = 17 launch equal an M = 16 launch and every
    shorter prefix bit for bit, at even and odd K partitions (pad blocks),
    per-quarter groups, K tails, split 1 and fp16."""
    print(f"16 vs 17 rows n={n} k={k} gi={gi} bits={bits} f16={f16}", flush=True)
    dt = torch.float16 if f16 else torch.bfloat16
    w = random_matrix(n, k, bits, gi, qz.FMT_F32, seed=n + k + bits, partitions=(n // 2, n - n // 2))
    prepared = linear.prepare_matrix(w.to(DEV), DEV, dt)
    x = torch.randn((17, k), generator=torch.Generator().manual_seed(k)).to(dt).to(DEV)
    def run(rows):
        y = torch.empty((rows, n), dtype=dt, device=DEV)
        linear.bind_prepared(x[:rows].contiguous(), prepared, (y,)).launch()
        return y
    y17 = run(17)
    for rows in (16, 11, 5):
        assert torch.equal(_bits16(run(rows)), _bits16(y17[:rows])), rows
