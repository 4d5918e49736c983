"""GPU parity: MoE router (cubic_moe_route) and route compaction
(cubic_moe_compact) against the CPU oracle, bit for bit.

* compaction: the reference's known-answer test
  (tests/ops/test_cuda_quantized_moe.py:25-67) including graph replay and
  poisoned outputs, plus the config-4 and a prefill-sized route count;
* router: random logits (ties, bf16/fp16, inactive rows) against the oracle,
  and the reference's softmax-midpoint case replayed in a graph with the
  logical row count changed between replays (tests/unit/test_cuda_moe.py:276-332);
* router -> compaction -> routed GEMM equals the same GEMM fed from
  independently compacted routes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, moe, quantization as qz

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("experts,size", [(3, 1), (127, 31), (512, 160), (513, 256), (512, 257)])
def test_compaction_reference_known_answers(oracle, experts, size):
    first = 7
    for mode in ("spread", "concentrated", "inactive"):
        logical = [first + (j % experts) for j in range(size)]
        if mode == "concentrated":
            logical = [first] * size
        if mode == "inactive":
            logical = [-1] * size
        else:
            logical[::7] = [-1] * len(logical[::7])
            logical[1::11] = [first + experts] * len(logical[1::11])
        for values in (logical, logical[::-1]):
            ids = torch.tensor(values, device=DEV, dtype=torch.int64)
            for bm in (8, 16, 32):
                storage = torch.full((4 * experts + size + 1,), -777, device=DEV, dtype=torch.int32)
                counts, starts, blocks, spare = storage[:4 * experts].chunk(4)
                total = storage[4 * experts:4 * experts + 1]
                rows = storage[4 * experts + 1:]
                binding = moe.bind_compact_routes(ids, counts, starts, blocks, total, rows,
                                                  first_expert=first, experts=experts, block_m=bm)
                binding.launch()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    binding.launch()
                storage.fill_(-777)
                graph.replay()
                torch.cuda.synchronize()
                w_counts, w_starts, w_blocks, w_total, w_rows = oracle.moe_compact(values, first, experts, bm)
                assert counts.tolist() == w_counts.tolist()
                assert starts.tolist() == w_starts.tolist()
                assert blocks.tolist() == w_blocks.tolist()
                assert total.item() == w_total
                assert rows.tolist() == w_rows.tolist()  # unowned slots stay poisoned
                assert bool((spare == -777).all())


@pytest.mark.parametrize("routes,experts,first", [(2048, 128, 0), (131072, 128, 0), (5000, 1024, 3),
                                                  (64, 1, 0)])
def test_compaction_large_random(oracle, routes, experts, first):
    g = torch.Generator(device=DEV).manual_seed(routes + experts)
    ids = torch.randint(-1, first + experts + 2, (routes,), generator=g, device=DEV)
    ids[: routes // 3] = first + 5 % experts  # skew
    rows = moe.RoutedRows(*(torch.full((n,), -777, dtype=torch.int32, device=DEV)
                            for n in (experts, experts, experts, 1, routes)))
    moe.bind_compact_routes(ids, rows.counts, rows.starts, rows.block_starts, rows.total_blocks,
                            rows.row_map, first_expert=first, experts=experts, block_m=32).launch()
    torch.cuda.synchronize()
    want = oracle.moe_compact(ids.cpu().numpy(), first, experts, 32)
    assert np.array_equal(rows.counts.cpu().numpy(), want[0])
    assert np.array_equal(rows.starts.cpu().numpy(), want[1])
    assert np.array_equal(rows.block_starts.cpu().numpy(), want[2])
    assert int(rows.total_blocks[0]) == want[3]
    assert np.array_equal(rows.row_map.cpu().numpy(), want[4])


def run_router(logits, activity, active, top_k, weights_dtype):
    m = logits.shape[0]
    outs = (torch.full((m, top_k), 5.0, device=DEV), torch.full((m, top_k), 9, dtype=torch.int64, device=DEV),
            torch.full((m, top_k), 9, dtype=torch.int64, device=DEV),
            torch.full((m, top_k), 3.0, dtype=weights_dtype, device=DEV))
    moe.bind_route_selection(logits, activity, torch.tensor([active], dtype=torch.int32, device=DEV),
                             *outs).launch()
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("rows,experts,top_k", [(256, 128, 8), (33, 16, 8), (7, 64, 1), (64, 512, 10),
                                                (5, 1024, 64), (3, 8, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_router_bit_exact(oracle, rows, experts, top_k, dtype):
    print(f"router rows={rows} experts={experts} top_k={top_k} dtype={dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows * experts + top_k)
    logits = (torch.randn((rows, experts), generator=g, device=DEV) * 2).to(dtype)
    logits[::3, : experts // 2] = logits[::3, : experts // 2].round()  # ties
    activity = torch.ones(rows, dtype=torch.int32, device=DEV)
    activity[1::4] = 0
    active = rows - rows // 5
    got = run_router(logits, activity, active, top_k, dtype)
    want = oracle.moe_route(bits16(logits), activity.cpu().numpy(), active, top_k,
                            fp16=dtype == torch.float16, weights_fp16=dtype == torch.float16)
    assert np.array_equal(got[0].cpu().numpy().view(np.uint32), want[0].view(np.uint32))
    assert np.array_equal(got[1].cpu().numpy(), want[1])
    assert np.array_equal(got[2].cpu().numpy(), want[2])
    assert np.array_equal(bits16(got[3]), want[3])


def test_router_softmax_midpoint_in_graph(oracle):
    scores = torch.tensor([-3.484375, -3.640625, -3.703125, -3.984375, -4.0, -4.34375, -4.375, -4.4375],
                          device=DEV)
    experts = torch.tensor([15, 2, 9, 0, 12, 1, 7, 4], device=DEV)
    order = torch.argsort(experts)
    expected_ids = experts[order]
    expected_weights = torch.softmax(scores, dim=0)[order].bfloat16()
    for capacity in (64, 128):
        router = torch.full((capacity, 16), -100.0, device=DEV, dtype=torch.bfloat16)
        router[:, experts] = scores.bfloat16()
        activity = torch.ones(capacity, device=DEV, dtype=torch.int32)
        active_rows = torch.tensor([capacity], device=DEV, dtype=torch.int32)
        routing = moe.MoERouting(router, activity, active_rows, top_k=8, first_expert=5, experts=4)
        routing.launch()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            routing.launch()
        for logical in (8, 32, 33):
            activity.zero_()
            activity[:logical].fill_(1)
            active_rows.fill_(logical)
            router.fill_(-100.0)
            router[:logical, experts] = scores.bfloat16()
            router[logical:].fill_(73.0)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(routing.route_ids[:logical], expected_ids.expand(logical, -1))
            assert torch.equal(routing.route_weights[:logical], expected_weights.expand(logical, -1))
            assert bool((routing.route_ids[logical:] == -1).all())
            assert bool((routing.route_weights[logical:] == 0).all())
            # experts 5..8 of this slice: 7 is the only selected one
            assert routing.rows.counts.tolist() == [0, 0, logical, 0]
            want = oracle.moe_compact(routing.route_ids.cpu().numpy(), 5, 4, 32)
            assert np.array_equal(routing.rows.row_map[:logical].cpu().numpy(), want[4][:logical])


def test_router_feeds_routed_gemm(oracle):
    tokens, experts, top_k, hidden, inter = 64, 16, 4, 256, 128
    g = torch.Generator(device=DEV).manual_seed(4)
    logits = torch.randn((tokens, experts), generator=g, device=DEV).to(torch.bfloat16)
    routing = moe.MoERouting(logits, torch.ones(tokens, dtype=torch.int32, device=DEV),
                             torch.tensor([tokens], dtype=torch.int32, device=DEV), top_k=top_k)
    routing.launch()
    torch.cuda.synchronize()
    ids = routing.route_ids.clone()
    quant = lambda n, k: qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4,
                                           group_in=128)
    gate = tuple(quant(inter, hidden) for _ in range(experts))
    up = tuple(quant(inter, hidden) for _ in range(experts))
    x = torch.randn((tokens, hidden), generator=g, device=DEV).to(torch.bfloat16)
    ops = linear.PackedLinearOperators()
    y_a = torch.empty((tokens * top_k, 2 * inter), dtype=torch.bfloat16, device=DEV)
    y_b = torch.empty_like(y_a)
    moe.bind_grouped(ops, x, gate, up, y_a, routing.rows, top_k)[1].launch()
    independent = moe.route_rows(ids, experts, 32)
    moe.bind_grouped(ops, x, gate, up, y_b, independent, top_k)[1].launch()
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b)
    want = oracle.moe_compact(ids.cpu().numpy(), 0, experts, 32)
    assert np.array_equal(routing.rows.row_map.cpu().numpy(), want[4])
