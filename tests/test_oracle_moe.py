"""CPU: the MoE router and route-compaction oracles.

Compaction (ops/cuda/moe/fused.py:174-199) is pinned by the reference's own
known-answer test (tests/ops/test_cuda_quantized_moe.py:25-67): every expert
count / route count pair, spread / concentrated / inactive routes, holes and
out-of-slice experts, reversed physical order, block_m 8/16/32 and poisoned
outputs.  The router (fused.py:44-100) is pinned by a stable argsort and a
float64 softmax (ids exact, weights within one output step), and by the
reference's softmax-midpoint case (tests/unit/test_cuda_moe.py:276-332).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


@pytest.mark.parametrize("experts,size", [(3, 1), (127, 31), (512, 160), (513, 256), (512, 257)])
@pytest.mark.parametrize("mode", ["spread", "concentrated", "inactive"])
def test_compaction_reference_known_answers(oracle, experts, size, mode):
    first = 7
    logical = [first + (j % experts) for j in range(size)]
    if mode == "concentrated":
        logical = [first] * size
    if mode == "inactive":
        logical = [-1] * size
    else:
        logical[::7] = [-1] * len(logical[::7])
        logical[1::11] = [first + experts] * len(logical[1::11])
    for values in (logical, logical[::-1]):
        expected = [j for e in range(first, first + experts) for j, v in enumerate(values) if v == e]
        counts_cpu = [values.count(e) for e in range(first, first + experts)]
        for bm in (8, 16, 32):
            counts, starts, blocks, total, rows = oracle.moe_compact(values, first, experts, bm)
            assert counts.tolist() == counts_cpu
            assert starts.tolist() == [sum(counts_cpu[:e]) for e in range(experts)]
            block_counts = [(n + bm - 1) // bm for n in counts_cpu]
            assert blocks.tolist() == [sum(block_counts[:e]) for e in range(experts)]
            assert total == sum(block_counts)
            assert rows[:len(expected)].tolist() == expected
            assert (rows[len(expected):] == -777).all()


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("experts,top_k", [(128, 8), (16, 8), (64, 1), (512, 10), (8, 8)])
def test_router_against_stable_argsort_and_float64_softmax(oracle, experts, top_k):
    g = torch.Generator().manual_seed(experts + top_k)
    logits = (torch.randn((97, experts), generator=g) * 2).to(torch.bfloat16)
    logits[::5, : experts // 2] = logits[::5, : experts // 2].round()  # ties
    activity = np.ones(97, np.int32)
    activity[3] = 0
    top_logits, top_ids, route_ids, weights = oracle.moe_route(bf16_bits(logits), activity, 90, top_k)
    sel = torch.argsort(logits.float(), dim=-1, descending=True, stable=True)[:, :top_k]
    live = np.arange(97) < 90
    live[3] = False
    assert np.array_equal(top_ids[live], sel.numpy()[live])
    assert np.array_equal(top_logits[live], logits.float().gather(1, sel).numpy()[live])
    ids_sorted, order = torch.sort(sel, dim=-1)
    assert np.array_equal(route_ids[live], ids_sorted.numpy()[live])
    p64 = torch.softmax(logits.double().gather(1, sel), dim=-1).gather(1, order)
    got = (weights.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    step = 2.0 ** (np.floor(np.log2(np.maximum(p64.numpy(), 1e-30))) - 7)  # one bf16 step
    assert (np.abs(got[live] - p64.numpy()[live]) <= step[live]).all()
    assert (top_ids[~live] == -1).all() and (route_ids[~live] == -1).all()
    assert (top_logits[~live] == 0).all() and (weights[~live] == 0).all()


def test_router_softmax_midpoint_case(oracle):
    scores = torch.tensor([-3.484375, -3.640625, -3.703125, -3.984375, -4.0, -4.34375, -4.375, -4.4375])
    experts = torch.tensor([15, 2, 9, 0, 12, 1, 7, 4])
    order = torch.argsort(experts)
    expected_ids = experts[order]
    expected_weights = torch.softmax(scores, dim=0)[order].bfloat16()
    router = torch.full((33, 16), -100.0)
    router[:, experts] = scores
    router[32:] = 73.0
    activity = np.ones(33, np.int32)
    _, _, route_ids, weights = oracle.moe_route(bf16_bits(router), activity, 32, 8)
    assert np.array_equal(route_ids[:32], expected_ids.expand(32, -1).numpy())
    assert np.array_equal(weights[:32], bf16_bits(expected_weights).reshape(1, -1).repeat(32, 0))
    assert (route_ids[32:] == -1).all() and (weights[32:] == 0).all()
