"""Host logic of the routed-expert path: route compaction (no GPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import moe


def brute_compaction(ids: np.ndarray, experts: int, block_m: int):
    flat = ids.reshape(-1)
    counts = np.array([(flat == e).sum() for e in range(experts)])
    row_map = [r for e in range(experts) for r in range(flat.size) if flat[r] == e]
    blocks = -(-counts // block_m)
    return counts, np.cumsum(counts) - counts, np.cumsum(blocks) - blocks, blocks.sum(), np.array(row_map)


@pytest.mark.parametrize("tokens,top_k,experts,block_m", [(7, 2, 4, 16), (64, 8, 32, 32), (1, 1, 3, 64)])
def test_route_rows_matches_brute_force(tokens, top_k, experts, block_m):
    g = torch.Generator().manual_seed(tokens * 31 + experts)
    logits = torch.randn((tokens, experts), generator=g)
    ids = torch.argsort(logits, dim=-1, descending=True, stable=True)[:, :top_k]
    rows = moe.route_rows(ids, experts, block_m)
    counts, starts, bstarts, total, row_map = brute_compaction(ids.numpy(), experts, block_m)
    assert np.array_equal(rows.counts.numpy(), counts)
    assert np.array_equal(rows.starts.numpy(), starts)
    assert np.array_equal(rows.block_starts.numpy(), bstarts)
    assert int(rows.total_blocks[0]) == total
    assert np.array_equal(rows.row_map.numpy(), row_map)
    assert rows.row_map.dtype == torch.int32 and rows.routing_top_k == top_k


def test_route_rows_rejects_bad_ids():
    with pytest.raises(ValueError):
        moe.route_rows(torch.tensor([[0, 5]]), 4, 16)
    with pytest.raises(ValueError):
        moe.route_rows(torch.tensor([0, 1]), 4, 16)
