"""GPU parity, end to end at BASELINE config 4 (128 experts, top-8, hidden
2048, intermediate 768, W4 g128, 256 tokens): router -> compaction ->
route padding -> routed gate/up GEMM -> (SiLU(gate) * up, staged by torch)
-> routed down GEMM, every stage on the device through the C ABI.

* router outputs bit-exact against oracle_moe_route (ops/cuda/moe/fused.py:44-100);
* compaction bit-exact against oracle_moe_compact (fused.py:174-199), fed
  from the device router's own route ids;
* the padded route table and block -> expert map against the layout that
  cubic_moe_pad_routes declares (every owned route once, in compaction order,
  padding slots = `routes`);
* EVERY route row of gate/up and of down inside the FP64 enclosure of its
  expert's decoded weights (guardrail/quantization.py:250-320);
* a second launch of the whole chain is bitwise identical.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, moe, quantization as qz

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def experts_of(n, k, count, seed, bits=4):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return tuple(qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=bits, group_in=128)
                 for _ in range(count))


def decoded(oracle, m: qz.QuantizedMatrix) -> np.ndarray:
    payload = {key: v.cpu().numpy() for key, v in m.payload.items()}
    return oracle.decode_bf16(payload, m.encoding.bits, m.encoding.metadata, m.shape, m.encoding.group_in)


def check_padding(rows: moe.RoutedRows, padded: np.ndarray, block_expert: np.ndarray, padded_total: int,
                  experts: int, routes: int, block_m: int):
    counts, starts = rows.counts.cpu().numpy(), rows.starts.cpu().numpy()
    block_starts, total = rows.block_starts.cpu().numpy(), int(rows.total_blocks[0])
    row_map = rows.row_map.cpu().numpy()
    assert padded_total == total * block_m
    seen = np.zeros(routes, np.int64)
    for e in range(experts):
        nb = -(-int(counts[e]) // block_m)
        assert (block_expert[block_starts[e]:block_starts[e] + nb] == e).all()
        slots = padded[block_starts[e] * block_m:(block_starts[e] + nb) * block_m]
        owned = row_map[starts[e]:starts[e] + counts[e]]
        assert np.array_equal(slots[:counts[e]], owned)
        assert (slots[counts[e]:] == routes).all()
        seen[owned] += 1
    assert (seen == 1).all(), "every route is padded exactly once"


def test_moe_cfg4_router_to_down_every_route(oracle):
    experts, tokens, top_k, hidden, inter, block_m = 128, 256, 8, 2048, 768, 32
    routes = tokens * top_k
    print(f"moe e2e: experts={experts} tokens={tokens} top_k={top_k} hidden={hidden} inter={inter}", flush=True)
    gate, up = experts_of(inter, hidden, experts, 20), experts_of(inter, hidden, experts, 21)
    down = experts_of(hidden, inter, experts, 22)
    g = torch.Generator(device=DEV).manual_seed(23)
    x = torch.randn((tokens, hidden), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.randn((tokens, experts), generator=g, device=DEV).to(torch.bfloat16)
    activity = torch.ones(tokens, dtype=torch.int32, device=DEV)
    active = torch.tensor([tokens], dtype=torch.int32, device=DEV)

    routing = moe.MoERouting(logits, activity, active, top_k=top_k, block_m=block_m)
    ops = linear.PackedLinearOperators()
    h = torch.full((routes, 2 * inter), float("nan"), dtype=torch.bfloat16, device=DEV)
    _, b_up = moe.bind_grouped(ops, x, gate, up, h, routing.rows, top_k)
    act = torch.empty((routes, inter), dtype=torch.bfloat16, device=DEV)
    y = torch.full((routes, hidden), float("nan"), dtype=torch.bfloat16, device=DEV)
    _, b_down = moe.bind_routed(ops, act, down, y, routing.rows)

    def chain():
        routing.launch()
        b_up.launch()
        hf = h.float()
        act.copy_((torch.nn.functional.silu(hf[:, :inter]) * hf[:, inter:]).to(torch.bfloat16))
        b_down.launch()
        torch.cuda.synchronize()

    chain()
    # router, bit for bit
    want = oracle.moe_route(bits16(logits), activity.cpu().numpy(), tokens, top_k)
    assert np.array_equal(routing.top_logits.cpu().numpy().view(np.uint32), want[0].view(np.uint32))
    assert np.array_equal(routing.top_ids.cpu().numpy(), want[1])
    assert np.array_equal(routing.route_ids.cpu().numpy(), want[2])
    assert np.array_equal(bits16(routing.route_weights), want[3])
    # compaction of the device's own routes, bit for bit
    wc = oracle.moe_compact(routing.route_ids.cpu().numpy(), 0, experts, block_m)
    r = routing.rows
    for got, exp in zip((r.counts, r.starts, r.block_starts), wc[:3]):
        assert np.array_equal(got.cpu().numpy(), exp)
    assert int(r.total_blocks[0]) == wc[3]
    assert np.array_equal(r.row_map.cpu().numpy(), wc[4])
    # padded tables of both routed launches
    for binding in (b_up, b_down):
        padded, block_expert = (t.cpu().numpy() for t in binding.scratch)
        launch = binding._launches[0]
        check_padding(r, padded, block_expert, int(launch.padded_total[0]), experts, routes, block_m)
    assert not torch.isnan(h).any() and not torch.isnan(y).any(), "every route row is written"

    # every route of every expert inside the enclosure
    ids = routing.route_ids.reshape(-1).cpu().numpy()
    xb, hb, ab, yb = bits16(x), bits16(h), bits16(act), bits16(y)
    checked = 0
    for e in range(experts):
        rs = np.nonzero(ids == e)[0]
        if rs.size == 0:
            continue
        w_gu = np.concatenate([decoded(oracle, gate[e]), decoded(oracle, up[e])])
        oracle.check_linear_enclosure(xb[rs // top_k], w_gu, hb[rs])
        oracle.check_linear_enclosure(ab[rs], decoded(oracle, down[e]), yb[rs])
        checked += rs.size
    assert checked == routes

    first = (h.clone(), y.clone())
    chain()
    assert torch.equal(h, first[0]) and torch.equal(y, first[1])
