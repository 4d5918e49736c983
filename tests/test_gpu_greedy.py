"""GPU parity: the greedy sampler (cubic_greedy_candidates, cubic_greedy_root,
cubic_sampling_final_guard, cubic_greedy_sample) against the CPU oracle.

* candidate publication bit-exact (scores, ids, every slot) for bf16 and
  fp16 logits over widths from 1 column to the 151936 vocabulary, row
  strides that force the scalar path, active counts below capacity,
  vocabulary offsets, grammar masks (including masks that empty a row) and
  non-finite values in admitted and masked columns; a workspace reused
  across launches of different widths;
* the root over random gathered [TP, C, K] blocks (padding, malformed
  sentinels, ids outside the vocabulary, parameters outside their domain,
  cancelled batches);
* the final guard over random tokens with one predicate flipped at a time,
  with and without root validity;
* the fused single-GPU launch equal to the composition of the three, and the
  reference's captured-sampler test (tests/ops/test_cuda_greedy_sampling.py:
  95-190): every count of each capacity, both row orders, invalid parameters
  rejected, replays of one captured graph interleaved with eager work.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import greedy
from cubic_serve_amd.greedy import (CapturedGreedySampler, ShardedSamplingParameters,
                                    TensorParallelSamplingError)
from cubic_serve_amd.sampling import ShardedSamplingWorkspace

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
DTYPES = [torch.bfloat16, torch.float16]


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def tie_logits(rows, width, dtype, gen, stride=None):
    """Values on a coarse grid (many equal maxima), signed zeros included."""
    stride = width if stride is None else stride
    v = torch.randint(-40, 41, (rows, stride), generator=gen).float() / 4
    v[v == 0] = torch.where(torch.rand(int((v == 0).sum()), generator=gen) < 0.5, -0.0, 0.0)
    return v.to(dtype).to(DEV)


def metadata(active, cancel=False):
    return torch.tensor([active, int(cancel)], dtype=torch.int32, device=DEV)


def params(rows, k=20, t=0.0, p=0.95, seed=1, ordinal=0):
    return ShardedSamplingParameters(
        torch.full((rows,), t, device=DEV), torch.full((rows,), k, dtype=torch.int64, device=DEV),
        torch.full((rows,), p, device=DEV), k, torch.full((rows,), seed, dtype=torch.int64, device=DEV),
        torch.full((rows,), ordinal, dtype=torch.int64, device=DEV))


def host_params(p):
    return [t.cpu().numpy() for t in (p.temperatures, p.top_ps, p.top_ks, p.seeds, p.ordinals)]


def run_candidates(oracle, logits, width, active, k, *, vocab_start=0, mask=None, workspace=None):
    rows = logits.shape[0]
    scores = torch.empty((rows, k), dtype=logits.dtype, device=DEV)
    ids = torch.empty((rows, k), dtype=torch.int64, device=DEV)
    ws = greedy.greedy_workspace(rows, width, DEV) if workspace is None else workspace
    print(f"candidates rows={rows} width={width} stride={logits.stride(0)} active={active} k={k} "
          f"start={vocab_start} mask={mask is not None} dtype={logits.dtype}", flush=True)
    greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width,
                             vocab_start=vocab_start, token_mask=mask)
    torch.cuda.synchronize()
    want_s, want_i = oracle.greedy_candidates(
        bits(logits[:, :width]), active, k, fp16=logits.dtype == torch.float16,
        vocab_start=vocab_start, token_mask=None if mask is None else mask.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(ids.cpu().numpy(), want_i)
    np.testing.assert_array_equal(bits(scores), want_s)
    return want_i


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,width", [(1, 1), (3, 7), (4, 2047), (5, 2048), (8, 4123), (2, 32768),
                                        (3, 151936)])
def test_candidates_match_oracle(oracle, dtype, rows, width):
    gen = torch.Generator().manual_seed(rows * 100003 + width)
    logits = tie_logits(rows, width, dtype, gen)
    ids = run_candidates(oracle, logits, width, rows, 20)
    assert (ids[:, 0] >= 0).all()
    run_candidates(oracle, logits, width, max(1, rows // 2), 3, vocab_start=4096)


@pytest.mark.parametrize("dtype", DTYPES)
def test_candidates_scalar_path_and_strided_rows(oracle, dtype):
    gen = torch.Generator().manual_seed(5)
    for rows, width, stride in ((3, 4123, 4125), (4, 9000, 9001), (2, 33, 40)):
        base = tie_logits(rows, stride, dtype, gen)
        run_candidates(oracle, base, width, rows, 20)
        run_candidates(oracle, base[:, 1:], width - 1, rows, 20)        # 2-byte offset base


@pytest.mark.parametrize("dtype", DTYPES)
def test_candidates_non_finite_and_masks(oracle, dtype):
    gen = torch.Generator().manual_seed(9)
    rows, width, start = 6, 5000, 37
    words = (start + width + 31) // 32 + 2
    logits = tie_logits(rows, width, dtype, gen)
    logits[1, 4999] = float("nan")
    logits[2, 0] = float("inf")
    logits[3, 2500] = float("-inf")
    mask = torch.randint(-2**31, 2**31, (rows, words), generator=gen, dtype=torch.int64).to(torch.int32)
    mask[4] = 0                                   # a row the grammar empties
    mask[3] = 0                                   # non-finite hidden by the mask still rejects
    mask = mask.to(DEV)
    ids = run_candidates(oracle, logits, width, rows, 20, vocab_start=start, mask=mask)
    assert ids[1, 0] == ids[2, 0] == ids[3, 0] == -2 and ids[4, 0] == -1
    run_candidates(oracle, logits, width, rows, 20)


def test_workspace_reuse_across_widths(oracle):
    gen = torch.Generator().manual_seed(3)
    rows = 4
    ws = greedy.greedy_workspace(rows, 151936, DEV)
    for width in (151936, 100, 151936, 70000):
        logits = tie_logits(rows, width, torch.bfloat16, gen)
        run_candidates(oracle, logits, width, rows, 20, workspace=ws)


def random_block(gen, tp, rows, k, vocab, dtype):
    s = torch.randint(-8, 9, (tp, rows, k), generator=gen).float() / 2
    nan = torch.rand((tp, rows, k), generator=gen) < 0.3
    s[nan] = float("nan")
    ids = torch.randint(0, vocab, (tp, rows, k), generator=gen)
    ids[nan] = -1
    bad = torch.rand((tp, rows, k), generator=gen) < 0.01
    ids[bad] = torch.tensor([-2, vocab, -1])[torch.randint(0, 3, (int(bad.sum()),), generator=gen)]
    return s.to(dtype).to(DEV), ids.to(DEV)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("tp,rows,k", [(1, 1, 1), (1, 7, 20), (2, 5, 20), (4, 64, 20), (8, 256, 20),
                                       (3, 9, 64)])
def test_root_matches_oracle(oracle, dtype, tp, rows, k):
    gen = torch.Generator().manual_seed(tp * 1000 + rows * 10 + k)
    vocab = 1000
    s, ids = random_block(gen, tp, rows, k, vocab, dtype)
    p = params(rows, k=k)
    p.temperatures[::7] = 0.5
    p.top_ps[1::11] = 0.0
    p.top_ks[2::13] = k + 1
    p.seeds[3::17] = -1
    p.ordinals[4::19] = -1
    for active, cancel in ((rows, False), (max(0, rows - 3), True), (rows // 2, False)):
        print(f"root tp={tp} rows={rows} k={k} active={active} cancel={cancel} {dtype}", flush=True)
        tokens = torch.empty(rows, dtype=torch.int64, device=DEV)
        valid = torch.empty(rows, dtype=torch.bool, device=DEV)
        greedy.greedy_root(s, ids, p, metadata(active, cancel), tokens, valid, vocab_size=vocab)
        torch.cuda.synchronize()
        want_t, want_v = oracle.greedy_root(bits(s), ids.cpu().numpy(), *host_params(p), active=active,
                                            cancel=cancel, vocab_size=vocab,
                                            fp16=dtype == torch.float16)
        np.testing.assert_array_equal(tokens.cpu().numpy(), want_t)
        np.testing.assert_array_equal(valid.cpu().numpy(), want_v)


def test_final_guard_matches_oracle(oracle):
    gen = torch.Generator().manual_seed(1)
    vocab, k = 500, 20
    for capacity in (1, 5, 256, 1000):
        for trial in range(12):
            active = int(torch.randint(0, capacity + 2, (1,), generator=gen))
            tokens = torch.randint(0, vocab, (capacity,), generator=gen)
            tokens[active:] = -1
            if active < capacity and trial % 3 == 0:
                tokens[active] = -2
            rv = torch.ones(capacity, dtype=torch.bool)
            p = params(capacity, k=k)
            flip = trial % 6
            i = int(torch.randint(0, capacity, (1,), generator=gen))
            if flip == 1:
                tokens[i] = vocab if i < active else 3
            elif flip == 2:
                rv[i] = False
            elif flip == 3:
                p.temperatures[i] = 2.5
            elif flip == 4:
                p.top_ks[i] = 0
            elif flip == 5:
                p.ordinals[i] = -1
            tokens, rv = tokens.to(DEV), rv.to(DEV)
            for root in (rv, None):
                out = torch.empty((), dtype=torch.bool, device=DEV)
                greedy.sampling_final_guard(tokens, root, metadata(active), p, out, vocab_size=vocab)
                want = oracle.final_guard(tokens.cpu().numpy(), None if root is None else rv.cpu().numpy(),
                                          *host_params(p), active=active, k=k, vocab_size=vocab)
                assert bool(out) == want, (capacity, trial, active, root is None)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,width", [(1, 151936), (5, 4123), (64, 151936), (256, 151936)])
def test_fused_sample_equals_composition(oracle, dtype, rows, width):
    gen = torch.Generator().manual_seed(rows + width)
    logits = tie_logits(rows, width, dtype, gen)
    if rows > 1:
        logits[1, width // 2] = float("nan")
    p = params(rows)
    for active, cancel in ((rows, False), (max(1, rows // 3), True)):
        print(f"fused rows={rows} width={width} active={active} cancel={cancel} {dtype}", flush=True)
        meta = metadata(active, cancel)
        outs = []
        for fused in (True, False):
            ws = ShardedSamplingWorkspace(torch.empty((rows, 20), dtype=dtype, device=DEV),
                                          torch.empty((rows, 20), dtype=torch.int64, device=DEV),
                                          None, None)
            tokens = torch.empty(rows, dtype=torch.int64, device=DEV)
            rv = torch.empty(rows, dtype=torch.bool, device=DEV)
            final = torch.empty((), dtype=torch.bool, device=DEV)
            scratch = greedy.greedy_workspace(rows, width, DEV)
            if fused:
                from cubic_serve_amd import _native
                _native.call("cubic_greedy_sample", logits.data_ptr(), int(dtype == torch.float16),
                             logits.stride(0), rows, width, meta.data_ptr(), None, 0, None, 0, 20,
                             *greedy._param_ptrs(p), width, ws.local_scores.data_ptr(),
                             ws.local_token_ids.data_ptr(), tokens.data_ptr(), rv.data_ptr(),
                             final.data_ptr(), scratch.data_ptr(), scratch.numel(),
                             _native.stream_of(DEV))
            else:
                greedy.greedy_candidates(logits, meta, ws.local_scores, ws.local_token_ids, scratch)
                greedy.greedy_root(ws.local_scores[None], ws.local_token_ids[None], p, meta, tokens, rv,
                                   vocab_size=width)
                greedy.sampling_final_guard(tokens, rv, meta, p, final, vocab_size=width)
            torch.cuda.synchronize()
            outs.append((bits(ws.local_scores), ws.local_token_ids.cpu().numpy(), tokens.cpu().numpy(),
                         rv.cpu().numpy(), bool(final)))
        want = oracle.greedy_sample(bits(logits), *host_params(p), active=active, cancel=cancel, k=20,
                                    vocab_size=width, fp16=dtype == torch.float16)
        for got in outs:
            for g, w in zip(got, want):
                np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("dtype", DTYPES)
def test_captured_sampler_reference_corpus(oracle, dtype):
    """tests/ops/test_cuda_greedy_sampling.py:95-190 on one GPU (TP = 1)."""
    width = vocab = 4123
    corpus = ((torch.arange(3 * width).reshape(3, width) * 3) % 29 - 14).to(dtype)
    reference = []
    for row in range(3):
        v = corpus[row].float()
        reference.append(int(torch.nonzero(v == v.max())[0]))
    side = torch.zeros(1, device=DEV)
    for capacity in (1, 2, 4, 16, 64):
        print(f"captured capacity={capacity} {dtype}", flush=True)
        p = params(capacity)
        logits = torch.empty((capacity, width), dtype=dtype, device=DEV)
        ws = ShardedSamplingWorkspace(torch.empty((capacity, 20), dtype=dtype, device=DEV),
                                      torch.empty((capacity, 20), dtype=torch.int64, device=DEV),
                                      None, None)
        plan = CapturedGreedySampler(local_logits=logits, true_vocab_size=vocab,
                                     token_ids=torch.empty(capacity, dtype=torch.int64, device=DEV),
                                     parameters=p, workspace=ws,
                                     root_valid=torch.empty(capacity, dtype=torch.bool, device=DEV))
        try:
            counts = range(1, capacity + 1) if capacity <= 16 else (1, 7, 33, 64)
            for count in counts:
                rows = tuple(r % 3 for r in range(count))
                for perm in (rows, tuple(reversed(rows))):
                    logits.fill_(float("nan"))
                    for dst, src in enumerate(perm):
                        logits[dst].copy_(corpus[src])
                    side.add_(1)                                 # eager work between replays
                    out = plan.replay(count, False)
                    expected = [reference[r] for r in perm] + [-1] * (capacity - count)
                    assert out.cpu().tolist() == expected
                    assert plan.root_valid.cpu().tolist() == [True] * count + [False] * (capacity - count)
            count = min(capacity, 3)
            for buffer, value in ((p.temperatures, 1), (p.top_ps, 0), (p.top_ks, 21), (p.ordinals, -1)):
                saved = buffer.clone()
                buffer[0] = value
                with pytest.raises(TensorParallelSamplingError, match="invalid"):
                    plan.replay(count, False)
                buffer.copy_(saved)
            if count < capacity:
                plan.replay(count, True)                          # cancel: -2 after the last row
                assert plan.token_ids[count].item() == -2
            logits[0, 5] = float("inf")
            with pytest.raises(TensorParallelSamplingError, match="invalid"):
                plan.replay(count, False)
            assert plan.token_ids[0].item() == -1
        finally:
            plan.close()
    assert side.item() > 0


def _expected_masked(logits_bits, mask, start, active, ninf):
    """local_candidates.cu:37-53: row r < active keeps the admitted columns'
    bits and -inf elsewhere; rows >= active are -inf."""
    rows, width = logits_bits.shape
    words = mask.cpu().numpy().view(np.uint32)
    tok = start + np.arange(width)
    admitted = ((words[:, tok >> 5] >> (tok & 31).astype(np.uint32)) & 1).astype(bool)
    out = np.where(admitted, logits_bits, np.uint16(ninf))
    out[active:] = np.uint16(ninf)
    return out


@pytest.mark.parametrize("dtype", DTYPES)
def test_masked_logits_output_and_consumption(oracle, dtype):
    """The grammar-masked logits the reference's candidate preparation writes
    (masked_logits, or the logits themselves with consume_logits): admitted
    columns bit for bit, -inf elsewhere, rows past the active count -inf (left
    as they are when consumed); the published candidates are unchanged."""
    gen = torch.Generator().manual_seed(21)
    rows, width, start, active = 6, 5000, 37, 4
    ninf = 0xFC00 if dtype == torch.float16 else 0xFF80
    words = (start + width + 31) // 32 + 1
    logits = tie_logits(rows, width + 3, dtype, gen)[:, :width]          # strided rows
    mask = torch.randint(-2**31, 2**31, (rows, words), generator=gen, dtype=torch.int64).to(torch.int32)
    mask[2] = 0                                                           # a row the grammar empties
    mask = mask.to(DEV)
    k = 20
    scores = torch.empty((rows, k), dtype=dtype, device=DEV)
    ids = torch.empty((rows, k), dtype=torch.int64, device=DEV)
    ws = greedy.greedy_workspace(rows, width, DEV)
    want = _expected_masked(bits(logits), mask, start, active, ninf)
    want_s, want_i = oracle.greedy_candidates(bits(logits), active, k, fp16=dtype == torch.float16,
                                              vocab_start=start, token_mask=mask.cpu().numpy().view(np.uint32))
    # explicit output
    out = torch.full((rows, width), 1.0, dtype=dtype, device=DEV)
    print(f"masked logits explicit {dtype}", flush=True)
    greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width, vocab_start=start,
                             token_mask=mask, masked_logits=out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out), want)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_i)
    np.testing.assert_array_equal(bits(scores), want_s)
    # consumed in place: active rows masked, the other rows untouched
    before = bits(logits).copy()
    print(f"masked logits consumed {dtype}", flush=True)
    greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width, vocab_start=start,
                             token_mask=mask, consume_logits=True)
    torch.cuda.synchronize()
    after = bits(logits)
    np.testing.assert_array_equal(after[:active], want[:active])
    np.testing.assert_array_equal(after[active:], before[active:])
    np.testing.assert_array_equal(ids.cpu().numpy(), want_i)
    # refused operands, before any launch
    with pytest.raises(TensorParallelSamplingError, match="consumption"):
        greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width, consume_logits=True)
    with pytest.raises(TensorParallelSamplingError, match="masked logits"):
        greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width, vocab_start=start,
                                 token_mask=mask, masked_logits=torch.empty((rows, width - 1), dtype=dtype, device=DEV))
    with pytest.raises(TensorParallelSamplingError, match="masked logits"):
        greedy.greedy_candidates(logits, metadata(active), scores, ids, ws, width=width, vocab_start=start,
                                 token_mask=mask, masked_logits=logits)                # aliases without consuming


def test_captured_sampler_writes_masked_logits(oracle):
    """CapturedGreedySampler(token_mask=, masked_logits=) (greedy.py:49-69):
    every replay rewrites the masked logits for the count it runs."""
    dtype, capacity, width = torch.bfloat16, 4, 3000
    gen = torch.Generator().manual_seed(22)
    logits = tie_logits(capacity, width, dtype, gen)
    mask = torch.randint(-2**31, 2**31, (capacity, (width + 31) // 32), generator=gen,
                         dtype=torch.int64).to(torch.int32).to(DEV)
    out = torch.empty((capacity, width), dtype=dtype, device=DEV)
    ws = ShardedSamplingWorkspace(torch.empty((capacity, 20), dtype=dtype, device=DEV),
                                  torch.empty((capacity, 20), dtype=torch.int64, device=DEV), None, None)
    plan = CapturedGreedySampler(local_logits=logits, true_vocab_size=width,
                                 token_ids=torch.empty(capacity, dtype=torch.int64, device=DEV),
                                 parameters=params(capacity), workspace=ws,
                                 root_valid=torch.empty(capacity, dtype=torch.bool, device=DEV),
                                 token_mask=mask, masked_logits=out)
    try:
        for count in (3, 1, 4):
            print(f"captured masked logits count={count}", flush=True)
            out.fill_(1.0)
            plan.replay(count, False)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits(out), _expected_masked(bits(logits), mask, 0, count, 0xFF80))
    finally:
        plan.close()
