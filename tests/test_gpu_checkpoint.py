"""GPU: checkpoints feed the kernels.

A Cubic checkpoint written to disk, admitted and materialized on the GPU
(whole, TP row shard, TP column shard, stacked expert) goes through the
gfx950 GEMM and the packed embedding: the outputs are bit-equal to the same
kernels fed from the in-memory matrix, and the one-hot GEMM recovers the
oracle's decode bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cubic_serve_amd import checkpoint as ck, linear, quantization as qz

from test_checkpoint import FMTS, decoded, random_matrix

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("bits", [2, 4, 5])
def test_loaded_matrix_through_gemm_and_embedding(oracle, tmp_path, fmt, bits):
    print(f"checkpoint fmt={fmt} bits={bits}", flush=True)
    m = random_matrix(48, 256, bits, 32, 2, fmt, seed=bits, partitions=(32, 16))
    ck.save_cubic_checkpoint(tmp_path, {"model.layers.0.mlp.gate_up_proj": m, "model.embed_tokens": m})
    logical = [ck.LogicalWeight("model.layers.0.mlp.gate_up_proj.weight", (48, 256), output_partitions=(32, 16)),
               ck.LogicalWeight("model.embed_tokens.weight", (48, 256), operation="embedding",
                                output_partitions=(32, 16))]
    plan = ck.CubicCheckpoint.admit(tmp_path, logical)
    ops = linear.PackedLinearOperators()
    x = torch.randn((8, 256), device=DEV).to(torch.bfloat16)
    eye = torch.eye(256, device=DEV, dtype=torch.bfloat16)
    w = plan.weight("model.layers.0.mlp.gate_up_proj.weight")
    for spans, axis, rows, cols in (((ck.AxisSpan(0, 48),), 0, slice(0, 48), slice(0, 256)),
                                    ((ck.AxisSpan(16, 48),), 0, slice(16, 48), slice(0, 256)),
                                    ((ck.AxisSpan(128, 256),), 1, slice(0, 48), slice(128, 256))):
        loaded = plan.materialize(w, device=DEV, axis=axis, spans=spans)
        assert loaded.device == DEV
        if axis == 0:
            y = ops.linear(x, loaded)
            direct = ops.linear(x, m.rows(rows.start, rows.stop).to(DEV))
            torch.cuda.synchronize()
            assert torch.equal(y, direct), spans
        ident = ops.linear(eye[cols.start:cols.stop, cols.start:cols.stop].contiguous(), loaded)
        torch.cuda.synchronize()
        want = oracle.f32_to_bf16_bits(decoded(oracle, m)[rows, cols].T.copy())
        got = bits16(ident)
        got[got == 0x8000] = 0
        want[want == 0x8000] = 0
        assert np.array_equal(got, want), spans
    table = plan.materialize(plan.weight("model.embed_tokens.weight"), device=DEV)
    ids = torch.tensor([0, 47, 16, 31], device=DEV)
    got = ops.embedding(ids, table, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    want = oracle.f32_to_bf16_bits(decoded(oracle, m)[ids.cpu().numpy()])
    assert np.array_equal(bits16(got), want)
