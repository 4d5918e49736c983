"""Host logic of the routed-expert path (no GPU): argument validation of the
router and compaction bindings, which must fail before any launch."""
from __future__ import annotations

import pytest
import torch

from cubic_serve_amd import moe


def test_route_rows_needs_token_by_top_k_ids():
    with pytest.raises(ValueError):
        moe.route_rows(torch.tensor([0, 1]), 4, 16)


def test_router_binding_rejects_cpu_and_bad_abi():
    rows, experts, k = 4, 16, 2
    ops = (torch.zeros((rows, experts), dtype=torch.bfloat16), torch.ones(rows, dtype=torch.int32),
           torch.tensor([rows], dtype=torch.int32), torch.empty((rows, k)),
           torch.empty((rows, k), dtype=torch.int64), torch.empty((rows, k), dtype=torch.int64),
           torch.empty((rows, k), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA"):
        moe.bind_route_selection(*ops)
    with pytest.raises(TypeError):
        moe.bind_route_selection(*ops[:-1], None)


def test_compaction_binding_rejects_cpu():
    ids = torch.zeros(8, dtype=torch.int64)
    e = lambda n: torch.empty(n, dtype=torch.int32)
    with pytest.raises(ValueError, match="CUDA"):
        moe.bind_compact_routes(ids, e(4), e(4), e(4), e(1), e(8), first_expert=0, experts=4, block_m=16)
