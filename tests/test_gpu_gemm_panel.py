"""GPU: the column-panel GEMM (M <= 64, bits <= 4, whole-k-block groups)
against the MFMA-tile kernel and the FP64 enclosure.

The two kernels compute the same MFMA sequence under the same K plan, so a
row computed at M in 5..64 (column panels) must equal the same row computed
at M = 130 (the single-tile kernel, 128-row chunks) bit for bit.  The shapes
walk the panel kernel's own paths: the 4-deep ring's two-k-block tail (6 and
10 k-blocks per partition), a partition of only the tail, the 2-deep ring
with two tiles per wave, the two-partition exchange (second arrival sums from
registers) and the store-first exchange (3 partitions), ragged N (a partial
last panel), activations with a padded row stride, the m-tile boundaries
(16/17, 32/33 rows), bits 1..4 and fp16 activations.  One sampled block per
shape is also checked against the oracle's enclosure
(guardrail/quantization.py:250-320, bf16).
"""
from __future__ import annotations

import pytest
import torch

from cubic_serve_amd import linear, quantization as qz
from test_gpu_gemm import _check_linear, random_matrix

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (n, k, bits): the plan each takes (split, k-blocks per partition, J, ring)
SHAPES = [
    (200, 768, 4),      # 13 tiles (ragged), split 3 x 2 k-blocks: J=1, 4-deep ring, tail only
    (4096, 768, 3),     # split 3 x 2, J=1, tail only, 3 bits
    (24576, 1280, 4),   # split 1 x 10: J=1, 4-deep ring, two whole rounds + tail
    (12288, 2048, 2),   # split 2 x 8: J=1, two-partition exchange, 2 bits
    (24576, 8192, 4),   # split 2 x 32: J=2, 2-deep ring, two-partition exchange
    (65536, 1024, 1),   # split 1: J=2, 2-deep ring, 1 bit
    (336, 4352, 4),     # split 8 x 5 (odd: a pad block each), J=1, tail
]


def _bits16(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16)


@pytest.mark.parametrize("n,k,bits", SHAPES)
@pytest.mark.parametrize("f16", [False, True])
def test_panel_rows_equal_single_tile_kernel(oracle, n, k, bits, f16):
    print(f"panel vs single-tile n={n} k={k} bits={bits} f16={f16}", flush=True)
    dt = torch.float16 if f16 else torch.bfloat16
    w = random_matrix(n, k, bits, 128, qz.FMT_F32, seed=n + 7 * k + bits)
    prepared = linear.prepare_matrix(w.to(DEV), DEV, dt)
    g = torch.Generator().manual_seed(n ^ k)
    corpus = torch.randn((130, k), generator=g).to(dt).to(DEV)
    # padded row stride for the panel launches: [M, k] views of [M, k + 72]
    padded = torch.zeros((130, k + 72), dtype=dt, device=DEV)
    padded[:, :k] = corpus

    def run(x):
        y = torch.full((x.shape[0], n), float("nan"), dtype=dt, device=DEV)
        linear.bind_prepared(x, prepared, (y,)).launch()
        return y

    ref = run(corpus)  # M = 130: the single-tile kernel
    torch.cuda.synchronize()
    for m in (5, 16, 17, 32, 33, 64):
        y = run(padded[:m, :k])
        assert not torch.isnan(y.float()).any(), m
        assert torch.equal(_bits16(y), _bits16(ref[:m])), m
        # rows past the panel's first m-tile from a shifted window
        if m > 16:
            y2 = run(padded[m - 16:m, :k])
            assert torch.equal(_bits16(y2), _bits16(ref[m - 16:m])), m
    if not f16:  # (fp16 enclosures: test_gpu_gemm_f16.py)
        cols = slice(max(0, n - 48), n)  # the last (possibly partial) panel
        _check_linear(oracle, w.rows(cols.start, cols.stop), corpus[:64].cpu(), ref[:64, cols].contiguous().cpu())


def test_panel_repeat_is_bitwise_stable():
    """The two-partition exchange's order (which partition arrives second)
    varies between launches; the output may not (split 2, one tile per wave)."""
    n, k = 12288, 4096
    w = random_matrix(n, k, 4, 128, qz.FMT_F32, seed=3)
    prepared = linear.prepare_matrix(w.to(DEV), DEV)
    x = torch.randn((64, k), generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(DEV)
    y = torch.empty((64, n), dtype=torch.bfloat16, device=DEV)
    b = linear.bind_prepared(x, prepared, (y,))
    b.launch()
    first = y.clone()
    for _ in range(20):
        y.fill_(0)
        b.launch()
        assert torch.equal(_bits16(y), _bits16(first))
