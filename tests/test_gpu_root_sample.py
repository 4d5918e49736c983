"""GPU parity: root top-k/top-p sampling (cubic_root_sample) against the CPU oracle.

* the reference's CUDA tests (tests/ops/test_cuda_topk_topp_sampling.py:113-245),
  bf16 and fp16 candidates;
* random candidate sets of every admitted block width (TP x K up to 8 x 20),
  duplicates, NaN/-1 sentinels, malformed pairs, out-of-domain parameters,
  seeds and ordinals above 2^32: tokens and valid flags bit-exact against the
  oracle's Philox path;
* a captured launch replayed with new seeds and scores.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cubic_serve_amd import sampling

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def case(rows: int, dtype, tp: int = 4, k: int = 20):
    scores = torch.randn((tp, rows, k), device=DEV, dtype=dtype)
    ids = (torch.arange(tp * k, device=DEV, dtype=torch.int64).view(tp, 1, k)
           .expand(tp, rows, k).contiguous())
    return [scores, ids,
            torch.full((rows,), 0.8, device=DEV, dtype=torch.float32),
            torch.full((rows,), 0.9, device=DEV, dtype=torch.float32),
            torch.full((rows,), 20, device=DEV, dtype=torch.int64),
            torch.arange(rows, device=DEV, dtype=torch.int64) + 0x123456789,
            torch.zeros(rows, device=DEV, dtype=torch.int64),
            torch.empty(rows, device=DEV, dtype=torch.int64),
            torch.empty(rows, device=DEV, dtype=torch.bool)]


def oracle_of(oracle, ops, constrained=None, allow_underfilled=False):
    scores = ops[0]
    bits = scores.cpu().view(torch.int16).numpy().view(np.uint16)
    host = [t.cpu().numpy() for t in ops[1:7]]
    return oracle.root_sample(bits, *host, fp16=scores.dtype == torch.float16,
                              allow_underfilled=allow_underfilled,
                              constrained_rows=None if constrained is None else constrained.cpu().numpy())


DTYPES = [torch.bfloat16, torch.float16]


@pytest.mark.parametrize("dtype", DTYPES)
def test_greedy_tie_and_invalid_sentinel(dtype):
    ops = case(3, dtype)
    ops[0].fill_(math.nan)
    ops[1].fill_(-1)
    ops[0][0, 0, :2] = torch.tensor([4.0, 4.0], device=DEV)
    ops[1][0, 0, :2] = torch.tensor([19, 3], device=DEV)
    ops[0][0, 1, 0] = 2.0
    ops[1][0, 1, 0] = 7
    ops[1][1, 1, 0] = 8  # mismatched NaN/id sentinel invalidates row 1
    ops[2].zero_()
    ops[4].fill_(20)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    torch.cuda.synchronize()
    assert ops[7].cpu().tolist() == [3, -1, -1]
    assert ops[8].cpu().tolist() == [True, False, False]
    assert not any(isinstance(v, torch.Tensor) for v in vars(prim).values())


@pytest.mark.parametrize("dtype", DTYPES)
def test_seed_and_ordinal_are_deterministic(oracle, dtype):
    ops = case(128, dtype)
    ops[0].zero_()
    ops[4].fill_(2)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    first = ops[7].clone()
    prim.launch(*ops)
    torch.cuda.synchronize()
    assert torch.equal(first, ops[7]) and bool(ops[8].all())
    want, _ = oracle_of(oracle, ops)
    assert np.array_equal(first.cpu().numpy(), want)
    ops[6].add_(1)
    prim.launch(*ops)
    torch.cuda.synchronize()
    assert bool(torch.any(first != ops[7]))
    assert bool(torch.all((ops[7] == 0) | (ops[7] == 1)))


@pytest.mark.parametrize("dtype", DTYPES)
def test_global_top_k_temperature_softmax_and_top_p_support(dtype):
    ops = case(4, dtype)
    ops[0].fill_(math.nan)
    ops[1].fill_(-1)
    ops[0][:, :, :2] = torch.tensor([8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.0, 1.0], device=DEV).view(4, 1, 2)
    ops[1][:, :, :2] = torch.arange(8, device=DEV).view(4, 1, 2)
    ops[2].fill_(1.0)
    ops[3].fill_(0.01)
    ops[4].fill_(4)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    torch.cuda.synchronize()
    assert ops[7].cpu().tolist() == [0, 0, 0, 0] and bool(ops[8].all())


@pytest.mark.parametrize("dtype", DTYPES)
def test_grammar_underfill_is_owned_per_row(dtype):
    ops = case(3, dtype)
    ops[0].fill_(math.nan)
    ops[1].fill_(-1)
    ops[0][0, :, 0] = 2.0
    ops[1][0, :, 0] = torch.tensor([7, 8, 9], device=DEV)
    flags = torch.tensor([True, False, True], device=DEV)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops, allow_underfilled=True, constrained_rows=flags)
    prim.launch(*ops, constrained_rows=flags)
    torch.cuda.synchronize()
    assert ops[7].tolist() == [7, -1, 9] and ops[8].tolist() == [True, False, True]
    flags.copy_(torch.tensor([False, True, True], device=DEV))
    ops[1][1, 2, 0] = 17  # a malformed NaN/id pair remains an error
    prim.launch(*ops, constrained_rows=flags)
    torch.cuda.synchronize()
    assert ops[7].tolist() == [-1, 8, -1] and ops[8].tolist() == [False, True, False]


def test_fixed_abi():
    ops = case(256, torch.bfloat16)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    with pytest.raises(ValueError, match="fixed launch ABI"):
        prim.launch(*(t[:128] if t.ndim == 1 else t for t in ops))
    with pytest.raises(ValueError, match="constrained-row ownership"):
        prim.launch(*ops, constrained_rows=torch.zeros(256, dtype=torch.bool, device=DEV))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tp,k", [(1, 20), (2, 20), (4, 20), (8, 20), (3, 7), (1, 1)])
def test_random_rows_bit_exact(oracle, dtype, tp, k):
    rows = 192
    print(f"root sample random tp={tp} k={k} dtype={dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(tp * 31 + k)
    ops = case(rows, dtype, tp, k)
    ops[0].copy_(torch.randn((tp, rows, k), generator=g, device=DEV) * 3)
    ops[0][:, ::7] = ops[0][:, ::7].round()  # score ties
    ops[1].copy_(torch.randint(0, 151936, (tp, rows, k), generator=g, device=DEV))
    ops[1][0, ::5, 0] = ops[1][min(1, tp - 1), ::5, 0]  # duplicate (score, id) pairs across ranks
    ops[0][0, ::5, 0] = ops[0][min(1, tp - 1), ::5, 0]
    pad = torch.rand((tp, rows, k), generator=g, device=DEV) < 0.15
    ops[0][pad] = math.nan
    ops[1][pad] = -1
    ops[1][:, 11::37, -1] = 5  # NaN with a real id on some rows -> malformed
    ops[0][:, 11::37, -1] = math.nan
    ops[2].copy_(torch.tensor([0.0, 0.3, 0.7, 1.0, 1.5], device=DEV).repeat(rows // 5 + 1)[:rows])
    ops[3].copy_(torch.tensor([1.0, 0.9, 0.5, 0.05], device=DEV).repeat(rows // 4 + 1)[:rows])
    ops[4].copy_(torch.randint(1, k + 1, (rows,), generator=g, device=DEV))
    ops[5].copy_(torch.randint(0, 2**62, (rows,), generator=g, device=DEV))
    ops[6].copy_(torch.randint(0, 2**40, (rows,), generator=g, device=DEV))
    ops[2][3] = math.nan
    ops[3][4] = 0.0
    ops[4][5] = k + 1
    ops[5][6] = -3
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    torch.cuda.synchronize()
    want_t, want_v = oracle_of(oracle, ops)
    assert np.array_equal(ops[7].cpu().numpy(), want_t)
    assert np.array_equal(ops[8].cpu().numpy(), want_v)
    assert want_v.sum() > rows // 3


def test_graph_replay_reads_new_operands(oracle):
    ops = case(64, torch.bfloat16)
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        prim.launch(*ops)
    for i in range(3):
        ops[0].copy_(torch.randn_like(ops[0], dtype=torch.float32).to(torch.bfloat16))
        ops[5].add_(977)
        ops[7].fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_t, want_v = oracle_of(oracle, ops)
        assert np.array_equal(ops[7].cpu().numpy(), want_t), i
        assert np.array_equal(ops[8].cpu().numpy(), want_v), i


def test_sampled_tokens_follow_the_truncated_softmax():
    """20000 rows of the same gathered candidates, distinct (seed, ordinal):
    the Philox-driven draws follow softmax(score / T) restricted to the top-k
    and renormalised over the top-p prefix (exclusive CDF <= top_p), within
    0.015 per token, and never leave that support."""
    rows, tp, k = 20000, 2, 4
    vals = np.array([[2.0, 1.5, 1.0, 0.5], [1.75, 1.25, 0.75, 0.25]], np.float32)  # bf16-exact
    scores = torch.from_numpy(vals).view(tp, 1, k).expand(tp, rows, k).to(torch.bfloat16).contiguous().to(DEV)
    ids = torch.arange(tp * k, device=DEV, dtype=torch.int64).view(tp, 1, k).expand(tp, rows, k).contiguous()
    temp, top_p, top_k = 0.8, 0.85, 4  # top_k <= K, the candidates per rank
    g = torch.Generator().manual_seed(99)
    ops = [scores, ids, torch.full((rows,), temp, device=DEV), torch.full((rows,), top_p, device=DEV),
           torch.full((rows,), top_k, dtype=torch.int64, device=DEV),
           torch.randint(0, 2**40, (rows,), generator=g).to(DEV),
           torch.randint(0, 2**30, (rows,), generator=g).to(DEV),
           torch.empty(rows, dtype=torch.int64, device=DEV), torch.empty(rows, dtype=torch.bool, device=DEV)]
    prim = sampling.RootTopKTopPSamplingPrimitive(*ops)
    prim.launch(*ops)
    torch.cuda.synchronize()
    assert bool(ops[8].all())
    # expected: global order by value, top_k, softmax at T, exclusive-CDF top-p
    flat = [(float(vals[r, c]), r * k + c) for r in range(tp) for c in range(k)]
    flat.sort(key=lambda t: (-t[0], t[1]))
    kept = flat[:top_k]
    w = np.exp((np.array([v for v, _ in kept]) - kept[0][0]) / temp)
    p = w / w.sum()
    excl = np.concatenate([[0.0], np.cumsum(p)[:-1]])
    p = np.where(excl <= top_p, p, 0.0)
    p = p / p.sum()
    expected = np.zeros(tp * k)
    for (v, tok), pr in zip(kept, p):
        expected[tok] = pr
    observed = np.bincount(ops[7].cpu().numpy(), minlength=tp * k) / rows
    assert np.abs(observed - expected).max() < 0.015, (observed, expected)
    assert observed[expected == 0].sum() == 0
