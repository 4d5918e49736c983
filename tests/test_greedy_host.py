"""CPU: host-side validation of the greedy sampler mirror (no kernel launch).

Operands that break the launch ABI (device, dtype, shape, width, parameter
buffers, capacity) are rejected with TensorParallelSamplingError before any
native call, as CapturedGreedySampler does (ops/cuda/sampling/greedy.py:75-180).
"""
from __future__ import annotations

import pytest
import torch

from cubic_serve_amd import greedy
from cubic_serve_amd.greedy import ShardedSamplingParameters, TensorParallelSamplingError


def params(rows, k=20, device="cpu"):
    return ShardedSamplingParameters(
        torch.zeros(rows, device=device), torch.full((rows,), k, dtype=torch.int64, device=device),
        torch.full((rows,), 0.95, device=device), k, torch.ones(rows, dtype=torch.int64, device=device),
        torch.zeros(rows, dtype=torch.int64, device=device))


def test_error_type_is_a_value_error():
    assert issubclass(TensorParallelSamplingError, ValueError)


def test_cpu_operands_are_rejected_before_launch():
    logits = torch.zeros((4, 100), dtype=torch.bfloat16)
    meta = torch.zeros(2, dtype=torch.int32)
    scores = torch.empty((4, 20), dtype=torch.bfloat16)
    ids = torch.empty((4, 20), dtype=torch.int64)
    with pytest.raises(TensorParallelSamplingError, match="CUDA"):
        greedy.greedy_candidates(logits, meta, scores, ids, torch.zeros(16, dtype=torch.uint8))
    with pytest.raises(TensorParallelSamplingError, match="CUDA"):
        greedy.greedy_root(scores[None], ids[None], params(4), meta, torch.empty(4, dtype=torch.int64),
                           torch.empty(4, dtype=torch.bool), vocab_size=100)
    with pytest.raises(TensorParallelSamplingError, match="CUDA"):
        greedy.sampling_final_guard(torch.empty(4, dtype=torch.int64), None, meta, params(4),
                                    torch.empty((), dtype=torch.bool), vocab_size=100)


def test_logits_layout_and_width_are_checked():
    meta = torch.zeros(2, dtype=torch.int32)
    out = (torch.empty((4, 20), dtype=torch.bfloat16), torch.empty((4, 20), dtype=torch.int64))
    for bad in (torch.zeros((4, 100)), torch.zeros((4, 100), dtype=torch.bfloat16).t(),
                torch.zeros(100, dtype=torch.bfloat16)):
        with pytest.raises(TensorParallelSamplingError, match="greedy logits"):
            greedy.greedy_candidates(bad, meta, *out, torch.zeros(16, dtype=torch.uint8))
    logits = torch.zeros((4, 100), dtype=torch.bfloat16)
    for kwargs in ({"width": 101}, {"width": -1}, {"vocab_start": -5}, {"width": 2.0}):
        with pytest.raises(TensorParallelSamplingError, match="width or vocabulary"):
            greedy.greedy_candidates(logits, meta, *out, torch.zeros(16, dtype=torch.uint8), **kwargs)


def test_parameter_buffers_are_checked():
    p = params(4)
    bad_k = ShardedSamplingParameters(p.temperatures, p.top_ks, p.top_ps, 65, p.seeds, p.ordinals)
    no_seed = ShardedSamplingParameters(p.temperatures, p.top_ks, p.top_ps, 20, None, p.ordinals)
    for bad in (bad_k, no_seed):
        with pytest.raises(TensorParallelSamplingError):
            greedy._require_parameters(bad, 4, torch.device("cuda", 0))
    wrong = ShardedSamplingParameters(p.temperatures.double(), p.top_ks, p.top_ps, 20, p.seeds, p.ordinals)
    with pytest.raises(TensorParallelSamplingError, match="temperatures"):
        greedy._require_parameters(wrong, 4, torch.device("cuda", 0))
