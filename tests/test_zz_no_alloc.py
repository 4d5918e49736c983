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


def _capture_first_main():
    """Run in a fresh process: the first cubic_accept_noalloc call on the device
    is made under HIP graph capture; every replay must match cubic_accept."""
    c, depth, width, k = 16, 3, 32768, 20
    logits, q_scores, q_ids, params = _case(c, depth, width, k, 0.7, seed=21)
    dev = {key: v.to(DEV) for key, v in params.items()}
    plan = sampling.MTPVerifyPlan(logits=logits.to(DEV), q_scores=q_scores.to(DEV),
                                  q_token_ids=q_ids.to(DEV), **dev)
    plan.launch()
    torch.cuda.synchronize()
    want = [plan.candidate_scores.view(torch.int16).clone(), plan.candidate_ids.clone(),
            plan.decisions.clone(), plan.merged.clone(), plan.emitted.clone()]
    rows = c * (depth + 1)
    out = [torch.empty((rows, k), dtype=torch.int16, device=DEV),
           torch.empty((rows, k), dtype=torch.int64, device=DEV),
           torch.empty((depth, c, 2), dtype=torch.int64, device=DEV),
           torch.empty((c, 2), dtype=torch.int64, device=DEV),
           torch.empty((c, depth + 1), dtype=torch.int64, device=DEV)]
    for t in out:
        t.fill_(-7)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = _native.lib().cubic_accept_noalloc(
            plan.logits.data_ptr(), plan.logits.stride(0), plan.width, c, depth, c, None,
            plan.row_temperatures.data_ptr(), plan.q_scores.data_ptr(), plan.q_token_ids.data_ptr(), k,
            dev["draft_tokens"].data_ptr(), dev["temperatures"].data_ptr(), dev["top_ps"].data_ptr(),
            dev["top_ks"].data_ptr(), dev["seeds"].data_ptr(), dev["ordinals"].data_ptr(),
            dev["uniforms"].data_ptr(), out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
            out[3].data_ptr(), out[4].data_ptr(), _native.stream_of(DEV))
        assert rc == 0, _native.lib().cubic_last_error()
    torch.cuda.synchronize()
    # capture ran nothing
    assert all(bool((t == -7).all()) for t in out)
    for replay in range(3):
        for t in out:
            t.fill_(-7)
        plan.launch()  # the workspace entry point, eagerly, between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for w, g in zip(want, out):
            assert torch.equal(w.cpu(), g.cpu()), f"replay {replay}"
    print("capture-first OK", flush=True)


def test_noalloc_first_call_under_graph_capture():
    import subprocess
    import sys
    from pathlib import Path

    print("noalloc: first call under capture, c=16 depth=3 V=32768, 3 replays (fresh process)", flush=True)
    here = Path(__file__).resolve().parent
    res = subprocess.run([sys.executable, "-c", "import test_zz_no_alloc as t; t._capture_first_main()"],
                         cwd=here, env={**__import__("os").environ, "PYTHONPATH": str(here.parent)},
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=110)
    out = res.stdout.decode(errors="replace")
    assert res.returncode == 0 and "capture-first OK" in out, out[-3000:]
