"""GPU: the verify step end to end (Cubic GEMM -> fused acceptance).

* BASELINE configuration 1 (the reference's CPU-runnable case): a W4 g128
  lm_head 32768 x 2048 from N(0, 0.02), bf16 activations at M = 2 (one
  sequence: one MTP draft + the bonus position), greedy acceptance of a
  seeded draft.  Logits inside the GEMM enclosure; accepted length and
  emitted tokens bit-exact against the CPU oracle on the same logits.
* The step captured in a HIP graph: every replay (with eager work and
  synchronisations in between) equals the eager result.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import linear, quantization as qz, sampling

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def to_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def greedy_plan(logits: torch.Tensor, drafts: torch.Tensor, c: int, depth: int) -> sampling.MTPVerifyPlan:
    q_s = torch.full((depth, c, 20), float("nan"), dtype=torch.bfloat16, device=DEV)
    q_s[:, :, 0] = 1.0
    q_i = torch.full((depth, c, 20), -1, dtype=torch.int64, device=DEV)
    q_i[:, :, 0] = drafts
    z = torch.zeros((depth, c), device=DEV)
    return sampling.MTPVerifyPlan(
        logits=logits, q_scores=q_s, q_token_ids=q_i, draft_tokens=drafts.contiguous(),
        temperatures=z, top_ps=torch.ones_like(z),
        top_ks=torch.full((depth, c), 20, dtype=torch.int64, device=DEV),
        seeds=torch.zeros((depth, c), dtype=torch.int64, device=DEV),
        ordinals=torch.zeros((depth, c), dtype=torch.int64, device=DEV))


def oracle_decisions(oracle, plan: sampling.MTPVerifyPlan, logits: torch.Tensor, drafts: np.ndarray, c: int):
    depth = drafts.shape[0]
    z = np.zeros((depth, c))
    return oracle.verify_from_logits(
        to_bits(logits), to_bits(plan.q_scores), plan.q_token_ids.cpu().numpy(), drafts, z,
        np.ones_like(z), np.full(z.shape, 20), z.astype(np.int64), z.astype(np.int64), c)


@pytest.mark.parametrize("hit", [True, False])
def test_cfg1_lm_head_greedy_verify(oracle, hit):
    n, k = 32768, 2048
    g = torch.Generator().manual_seed(0)
    w = torch.randn((n, k), generator=g) * 0.02
    m = qz.quantize_cubic(w.to(DEV), bits=4, group_in=128)
    del w
    x = torch.randn((2, k), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    logits = linear.PackedLinearOperators().linear(x, m)
    torch.cuda.synchronize()
    # logits within the enclosure on sampled row blocks
    for start in (0, n // 2, n - 128):
        part = m.rows(start, start + 128).to("cpu")
        payload = {key: v.numpy() for key, v in part.payload.items()}
        wb = oracle.decode_bf16(payload, 4, qz.FMT_F32, (128, k), 128)
        oracle.check_linear_enclosure(to_bits(x), wb, to_bits(logits[:, start:start + 128]))
    f = oracle.bf16_bits_to_f32(to_bits(logits))
    top0 = int(np.lexsort((np.arange(n), -f[0]))[0])
    draft = top0 if hit else (top0 + 12345) % n
    drafts = torch.tensor([[draft]], dtype=torch.int64, device=DEV)
    plan = greedy_plan(logits, drafts, c=1, depth=1)
    plan.launch()
    torch.cuda.synchronize()
    want = oracle_decisions(oracle, plan, logits, drafts.cpu().numpy(), 1)
    got_merged = plan.merged.cpu().numpy()
    assert np.array_equal(got_merged, want[3])
    top1 = int(np.lexsort((np.arange(n), -f[1]))[0])
    # accepted length and emitted tokens (reference semantics, draft_graph.py:146-157)
    if hit:
        assert got_merged.tolist() == [[1, top1]]
        assert plan.emitted.cpu().numpy().tolist() == [[draft, top1]]
    else:
        assert got_merged.tolist() == [[0, top0]]
        assert plan.emitted.cpu().numpy().tolist() == [[top0, -1]]


def test_step_graph_replays_equal_eager():
    n, k, c, depth = 16384, 1024, 4, 1
    g = torch.Generator(device=DEV).manual_seed(3)
    m = qz.quantize_cubic(torch.randn((n, k), generator=g, device=DEV) * 0.02, bits=4, group_in=128)
    x = torch.randn((c * (depth + 1), k), generator=g, device=DEV).to(torch.bfloat16)
    logits = torch.empty((c * (depth + 1), n), dtype=torch.bfloat16, device=DEV)
    binding = linear.PackedLinearOperators().bind_linear(x, m, logits)
    binding.launch()
    torch.cuda.synchronize()
    top = logits.float().argmax(-1)
    drafts = torch.stack([top[0], top[2] + 1, top[4], top[6] + 3]).reshape(depth, c) % n
    plan = greedy_plan(logits, drafts, c, depth)
    plan.launch()
    torch.cuda.synchronize()
    eager = (logits.clone(), plan.merged.clone(), plan.emitted.clone())

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        binding.launch()
        plan.launch()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        binding.launch()
        plan.launch()
    for i in range(4):
        logits.zero_()
        plan.merged.fill_(-7)
        plan.emitted.fill_(-7)
        _ = (x.float() * 2).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, eager[0]), i
        assert torch.equal(plan.merged, eager[1]), i
        assert torch.equal(plan.emitted, eager[2]), i
