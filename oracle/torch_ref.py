"""Torch-on-CPU restatement of the reference's eager WNA16 path (CPU baseline).

TEST INFRASTRUCTURE ONLY: ``bench.py``'s ``cpu_baseline`` leg times it on the
host cores and ``tests/`` pin it against the C oracle; product code never
imports it.

Reference paths are relative to ``src/cubic_serve/`` of QuantTrio/cubic-serve.

Function        restates                                                  pinned by
--------------  --------------------------------------------------------  -------------------------------------------
decode_fmt0     quantization/extensions/cubic/reference.py:31-47, 98-121  bit-equal to oracle.decode_bf16 (every code,
                (float32-scale-float16-ab metadata), bf16-rounded as       bits 1..8; tests/test_oracle_decode.py)
                ops/eager/quantization.py:181-182 does
linear_rows     ops/eager/linear.py:43-56: one FP32 matmul per input row   within 1 bf16 ulp of oracle.linear_bf16
                (torch.matmul, the reference's own backend call)           (FP32 sums differ only in order)
"""
from __future__ import annotations

import torch


def _codes(packed: torch.Tensor, bits: int, k: int) -> torch.Tensor:
    """Signed Cubic codes [n, k] from the little-endian bitstream."""
    bytes32 = packed.to(torch.int32)
    pos = torch.arange(k, dtype=torch.int64) * bits
    lo_idx, shift = pos // 8, (pos % 8).to(torch.int32)
    hi_idx = torch.clamp(lo_idx + 1, max=packed.shape[1] - 1)
    raw = (bytes32[:, lo_idx] >> shift) | (bytes32[:, hi_idx] << (8 - shift))
    raw = raw & ((1 << bits) - 1)
    if bits == 1:
        return raw * 2 - 1
    half = 1 << (bits - 1)
    signed = torch.where(raw >= half, raw - (1 << bits), raw)
    return torch.where(signed == -half, torch.zeros_like(signed), signed)  # reserved code -> 0


def decode_fmt0(packed: torch.Tensor, scale: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
                bits: int, group_in: int, k: int) -> torch.Tensor:
    """bf16 weights [n, k] of an fmt0 Cubic payload (group_out = 1)."""
    q = _codes(packed, bits, k)
    grp = torch.arange(k) // group_in
    s = scale.float()[:, grp]
    if bits == 1:
        return (q.float() * s).to(torch.bfloat16)
    af, bf = a.float()[:, grp], b.float()[:, grp]
    # t = m / D in binary64, rounded once to binary32; then unfused binary32
    t = (q.abs().double() / ((1 << (bits - 1)) - 1)).float()
    cubic = t * (af + t * (bf + t * ((1.0 - af) - bf)))
    return (q.sign().float() * (s * cubic)).to(torch.bfloat16)


def linear_rows(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """y[m, n] = bf16(x_row . w^T) with FP32 operands, one matmul per row."""
    wt = w.float().t()
    rows = [torch.matmul(r.float().unsqueeze(0), wt) for r in x]
    return torch.cat(rows).to(torch.bfloat16)
