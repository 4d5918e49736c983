"""GPU: cubic_accept_noalloc (static device scratch) against cubic_accept.

Both entry points are called through the C ABI on the same inputs; every
output (published candidates, per-depth decisions, merged prefix, emitted
tokens) must be bit-identical.  Two calls in a row, the second one smaller,
so the second sees the scratch the first left behind.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import _native, sampling

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(c, depth, width, k, temperature, seed):
    g = torch.Generator().manual_seed(seed)
    rows = c * (depth + 1)
    logits = (torch.randn((rows, width), generator=g) * 3).to(torch.bfloat16)
    q_scores = (torch.randn((depth, c, k), generator=g) * 3).to(torch.bfloat16)
    q_ids = torch.stack([torch.randperm(width, generator=g)[:k] for _ in range(depth * c)]).view(depth, c, k)
    # drafts: the target argmax for about two thirds of the rows, a random id otherwise
    target_max = logits.float().argmax(dim=1).view(c, depth + 1)[:, :depth].t()
    random_ids = torch.randint(0, width, (depth, c), generator=g)
    hit = torch.rand((depth, c), generator=g) < 0.67
    drafts = torch.where(hit, target_max, random_ids).to(torch.int64)
    q_ids[:, :, 0] = drafts
    params = dict(
        draft_tokens=drafts, temperatures=torch.full((depth, c), temperature),
        top_ps=torch.full((depth, c), 0.9), top_ks=torch.full((depth, c), k, dtype=torch.int64),
        seeds=torch.randint(0, 1 << 40, (depth, c), generator=g),
        ordinals=torch.randint(0, 1 << 20, (depth, c), generator=g),
        uniforms=torch.rand((depth, c, 2), generator=g))
    return logits, q_scores, q_ids, params


def _run_both(c, depth, width, k, temperature, seed):
    logits, q_scores, q_ids, params = _case(c, depth, width, k, temperature, seed)
    dev = {key: v.to(DEV) for key, v in params.items()}
    plan = sampling.MTPVerifyPlan(logits=logits.to(DEV), q_scores=q_scores.to(DEV),
                                  q_token_ids=q_ids.to(DEV), **dev)
    plan.launch()
    rows = c * (depth + 1)
    out = dict(scores=torch.empty((rows, k), dtype=torch.bfloat16, device=DEV),
               ids=torch.empty((rows, k), dtype=torch.int64, device=DEV),
               decisions=torch.empty((depth, c, 2), dtype=torch.int64, device=DEV),
               merged=torch.empty((c, 2), dtype=torch.int64, device=DEV),
               emitted=torch.empty((c, depth + 1), dtype=torch.int64, device=DEV))
    for t in out.values():
        t.fill_(-7)
    with torch.cuda.device(DEV):
        _native.call("cubic_accept_noalloc", plan.logits.data_ptr(), plan.logits.stride(0),
                     plan.width, c, depth, c, None, plan.row_temperatures.data_ptr(),
                     plan.q_scores.data_ptr(), plan.q_token_ids.data_ptr(), k,
                     dev["draft_tokens"].data_ptr(), dev["temperatures"].data_ptr(),
                     dev["top_ps"].data_ptr(), dev["top_ks"].data_ptr(), dev["seeds"].data_ptr(),
                     dev["ordinals"].data_ptr(), dev["uniforms"].data_ptr(),
                     out["scores"].data_ptr(), out["ids"].data_ptr(), out["decisions"].data_ptr(),
                     out["merged"].data_ptr(), out["emitted"].data_ptr(), _native.stream_of(DEV))
    torch.cuda.synchronize()
    pairs = ((plan.candidate_scores.view(torch.int16), out["scores"].view(torch.int16)),
             (plan.candidate_ids, out["ids"]), (plan.decisions, out["decisions"]),
             (plan.merged, out["merged"]), (plan.emitted, out["emitted"]))
    for want, got in pairs:
        assert torch.equal(want.cpu(), got.cpu())
    return plan.merged.cpu()


def test_noalloc_matches_workspace_entry_two_calls():
    print("noalloc: c=64 depth=3 V=151936 stochastic, then c=4 depth=1 V=32768 greedy", flush=True)
    first = _run_both(64, 3, 151936, 20, 0.7, seed=11)
    second = _run_both(4, 1, 32768, 8, 0.0, seed=12)
    # greedy rows whose draft is the target argmax accept it
    assert (second[:, 0] >= 0).any()
    assert first.shape == (64, 2)


def test_noalloc_rejects_plans_beyond_the_static_scratch():
    lib = _native.lib()
    c, depth, width = 4096, 8, 400003
    need = lib.cubic_accept_workspace_bytes(c, depth, width)
    assert need > (4 << 20)
    rc = lib.cubic_accept_noalloc(*([0] * 2), width, c, depth, c, *([0] * 4), 20, *([0] * 13))
    assert rc == -4
    assert b"static scratch" in lib.cubic_last_error()
