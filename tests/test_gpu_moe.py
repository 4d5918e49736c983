"""GPU parity: routed-expert Cubic GEMM (MoE) against the CPU oracle.

Every checked route row lies inside the FP64 enclosure of its expert's
decoded weights (guardrail/quantization.py:176-320) applied to its token's
activations; padding slots write nothing.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, moe, quantization as qz

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def experts_of(n, k, count, seed, bits=4):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return tuple(qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=bits, group_in=128)
                 for _ in range(count))


def check_routes(oracle, x, y, groups, ids, top_k, routes_to_check):
    flat = ids.reshape(-1).cpu().numpy()
    for r in routes_to_check:
        e, t = int(flat[r]), r // top_k
        cols = 0
        for g in groups:
            m = g[e]
            payload = {key: v.cpu().numpy() for key, v in m.payload.items()}
            wb = oracle.decode_bf16(payload, m.encoding.bits, m.encoding.metadata, m.shape, m.encoding.group_in)
            n = m.shape[0]
            oracle.check_linear_enclosure(to_bits(x[t:t + 1]), wb, to_bits(y[r:r + 1, cols:cols + n]))
            cols += n


@pytest.mark.parametrize("block_m", [16, 32, 64])
def test_moe_grouped_small(oracle, block_m):
    experts, tokens, top_k, n, k = 6, 20, 2, 64, 512
    gate, up = experts_of(n, k, experts, 1), experts_of(n, k, experts, 2)
    g = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn((tokens, k), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((tokens, experts), generator=g, device=DEV)
    logits[:, 0] += 2.0  # skew: expert 0 takes most tokens (several blocks)
    ids = torch.argsort(logits, dim=-1, descending=True, stable=True)[:, :top_k]
    rows = moe.route_rows(ids, experts, block_m)
    out = torch.full((tokens * top_k, 2 * n), float("nan"), dtype=torch.bfloat16, device=DEV)
    ops = linear.PackedLinearOperators()
    bm, binding = moe.bind_grouped(ops, x, gate, up, out, rows, top_k, moe.CubicMoEParameters(block_m=block_m))
    assert bm == block_m
    binding.launch()
    torch.cuda.synchronize()
    assert not torch.isnan(out).any(), "every route row is written"
    check_routes(oracle, x, out, (gate, up), ids, top_k, range(tokens * top_k))
    # (no bitwise comparison with dense launches of the gathered rows: a
    # routed launch keeps K whole, while a dense launch of one small expert
    # splits K, so their FP32 summation orders differ)


def test_moe_cfg4_shapes(oracle):
    """128 experts, top-8, hidden 2048, intermediate 768,
    W4 g128, 256 tokens (batch 128, k=1), router logits N(0, 1)."""
    experts, tokens, top_k, hidden, inter = 128, 256, 8, 2048, 768
    gate, up = experts_of(inter, hidden, experts, 10), experts_of(inter, hidden, experts, 11)
    down = experts_of(hidden, inter, experts, 12)
    g = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn((tokens, hidden), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((tokens, experts), generator=g, device=DEV)
    ids = torch.argsort(logits, dim=-1, descending=True, stable=True)[:, :top_k]
    rows = moe.route_rows(ids, experts, 32)
    ops = linear.PackedLinearOperators()
    h = torch.empty((tokens * top_k, 2 * inter), dtype=torch.bfloat16, device=DEV)
    _, b1 = moe.bind_grouped(ops, x, gate, up, h, rows, top_k)
    xd = torch.randn((tokens * top_k, inter), generator=g, device=DEV).to(torch.bfloat16)
    yd = torch.empty((tokens * top_k, hidden), dtype=torch.bfloat16, device=DEV)
    _, b2 = moe.bind_routed(ops, xd, down, yd, rows)
    b1.launch()
    b2.launch()
    torch.cuda.synchronize()
    sample = torch.randperm(tokens * top_k, generator=torch.Generator().manual_seed(0))[:24].tolist()
    check_routes(oracle, x, h, (gate, up), ids, top_k, sample)
    check_routes(oracle, xd, yd, (down,), ids, 1, sample[:12])
    first = (h.clone(), yd.clone())
    b1.launch()
    b2.launch()
    assert torch.equal(h, first[0]) and torch.equal(yd, first[1])
