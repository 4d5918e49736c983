"""Routed-expert (MoE) Cubic GEMM behind the Cubic extension's MoE hooks.

Mirrors quantization/extensions/cubic/marlin.py:84-253 (``bind_grouped`` for
gate/up, ``bind_routed`` for down, both returning ``(block_m, binding)`` or
None when not admitted) over ``RoutedRows`` (quantization/api.py:123-134).
Semantics (Marlin-MoE, as the reference's kernel): route ordinal r = token *
top_k + j; output row r = x[r // top_k] . decode(W[expert(r)])^T; grouped
gate/up write gate columns first, then up, to one output row.

Each launch first expands the compact routes into padded blocks of block_m
route slots (cubic_moe_pad_routes, repack.py:253-277 semantics), then runs
the routed GEMM (cubic_moe_gemm): one grid chunk per padded block, the
block's expert's prepared weights, rows gathered through the route table.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from .linear import PackedLinearOperators, PackedOperatorBinding, prepare_matrix
from .quantization import QuantizedMatrix


@dataclass(frozen=True, slots=True)
class RoutedRows:
    """Rank-local routes compacted by expert (quantization/api.py:123-134).

    counts[e] routes of expert e sit in row_map[starts[e] : starts[e] +
    counts[e]] (route ordinals, ascending); block_starts[e] counts blocks of
    block_m; total_blocks is the sum of ceil(counts / block_m).  int32 device
    tensors (total_blocks: one element).
    """

    counts: Tensor
    starts: Tensor
    block_starts: Tensor
    total_blocks: Tensor
    row_map: Tensor
    mean_rows_per_expert: float | None = None
    routing_top_k: int | None = None


@dataclass(frozen=True, slots=True)
class CubicMoEParameters:
    """``native_enabled`` False declines (None), like ``marlin_enabled``."""

    native_enabled: bool = True
    grouped_projections: bool = True
    block_m: int = 32


def route_rows(topk_ids: Tensor, experts: int, block_m: int) -> RoutedRows:
    """Compact top-k routes by expert, stable in route ordinal.

    Tensor restatement of the compaction of ops/cuda/moe/fused.py:175-199
    (histogram, exclusive prefix of counts and of blocks, route order by
    (expert, ordinal)); used to feed the routed GEMM.
    """
    if topk_ids.ndim != 2:
        raise ValueError("routes need [tokens, top_k] expert ids")
    ids = topk_ids.reshape(-1).to(torch.int64)
    if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= experts):
        raise ValueError("expert id out of range")
    routes = ids.numel()
    order = torch.argsort(ids * max(routes, 1) + torch.arange(routes, device=ids.device))
    counts = torch.bincount(ids, minlength=experts)
    blocks = (counts + block_m - 1) // block_m
    i32 = lambda t: t.to(torch.int32).contiguous()
    return RoutedRows(i32(counts), i32(torch.cumsum(counts, 0) - counts),
                      i32(torch.cumsum(blocks, 0) - blocks), i32(blocks.sum().reshape(1)), i32(order),
                      mean_rows_per_expert=routes / experts, routing_top_k=topk_ids.shape[1])


@dataclass(frozen=True, slots=True)
class PreparedExperts:
    codes: Tensor  # [experts, code words] int32
    meta: Tensor   # [experts, meta words] int32
    n: int
    k: int
    bits: int
    group_in: int

    @property
    def experts(self) -> int:
        return self.codes.shape[0]


def prepare_experts(groups: Sequence[Sequence[QuantizedMatrix]], device: torch.device) -> PreparedExperts:
    """Per expert, the group members (gate, up) prepared as one [sum n, k]
    matrix, experts stacked with a fixed stride (load time, allocates)."""
    experts = len(groups[0])
    if any(len(g) != experts for g in groups):
        raise ValueError("every group needs one matrix per expert")
    codes, meta, first = [], [], None
    for e in range(experts):
        parts = [prepare_matrix(g[e], device) for g in groups]
        first = first or parts[0]
        codes.append(torch.cat([p.codes for p in parts]))
        meta.append(torch.cat([p.meta for p in parts]))
    n = sum(g[0].shape[0] for g in groups)
    return PreparedExperts(torch.stack(codes), torch.stack(meta), n, first.k, first.bits, first.group_in)


class _MoELaunch:
    def __init__(self, x: Tensor, prepared: PreparedExperts, output: Tensor, rows: RoutedRows,
                 top_k: int, block_m: int, routes: int):
        dev = x.device
        self.x, self.prepared, self.output, self.rows = x, prepared, output, rows
        self.top_k, self.block_m, self.routes = top_k, block_m, routes
        self.max_blocks = int(_native.lib().cubic_moe_max_blocks(routes, prepared.experts, block_m))
        self.padded = torch.empty(self.max_blocks * block_m, dtype=torch.int32, device=dev)
        self.block_expert = torch.empty(self.max_blocks, dtype=torch.int32, device=dev)
        self.padded_total = torch.zeros(1, dtype=torch.int32, device=dev)
        self.identity = self._identity()

    def _identity(self):
        return tuple((t.data_ptr(), tuple(t.shape), t.dtype) for t in
                     (self.x, self.output, self.rows.counts, self.rows.starts, self.rows.block_starts,
                      self.rows.total_blocks, self.rows.row_map))

    def validate(self) -> None:
        if self._identity() != self.identity:
            raise ValueError("packed launch operands changed after binding")

    def __call__(self, stream: int) -> None:
        r, pr = self.rows, self.prepared
        _native.call("cubic_moe_pad_routes", r.counts.data_ptr(), r.starts.data_ptr(),
                     r.block_starts.data_ptr(), r.total_blocks.data_ptr(), r.row_map.data_ptr(),
                     pr.experts, self.routes, self.block_m, self.padded.data_ptr(),
                     self.block_expert.data_ptr(), self.padded_total.data_ptr(), stream)
        _native.call("cubic_moe_gemm", self.x.data_ptr(), self.x.stride(0), pr.codes.data_ptr(),
                     pr.meta.data_ptr(), pr.codes.shape[1], pr.meta.shape[1], self.padded.data_ptr(),
                     self.block_expert.data_ptr(), self.padded_total.data_ptr(), self.max_blocks,
                     self.block_m, self.routes, self.top_k, pr.n, pr.k, pr.bits, pr.group_in,
                     self.output.data_ptr(), self.output.stride(0), stream)


def _admitted(groups, x: Tensor, output: Tensor, params: CubicMoEParameters) -> bool:
    base = groups[0][0]
    enc = base.encoding
    return (params.native_enabled and params.block_m in (16, 32, 64) and enc.group_out == 1
            and 1 <= enc.bits <= 8 and enc.group_in % 32 == 0 and base.shape[1] % 8 == 0
            and x.dtype == torch.bfloat16 and output.dtype == torch.bfloat16
            and all(w.encoding == enc and w.shape[1] == base.shape[1] and w.shape[0] % 16 == 0
                    for g in groups for w in g))


def _bind(operators: PackedLinearOperators, x: Tensor, groups, output: Tensor, rows: RoutedRows,
          top_k: int, params: CubicMoEParameters):
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("routed Cubic experts must be bound before graph capture")
    if not _admitted(groups, x, output, params):
        return None
    key = ("cubic.mi355x.moe.v1", tuple(tuple(id(w) for w in g) for g in groups), str(x.device))
    cached = operators.prepared_weights.get(key)
    if cached is None:
        cached = operators.prepared_weights[key] = (groups, prepare_experts(groups, x.device))
    prepared = cached[1]
    routes = x.shape[0] * top_k
    if output.shape != (routes, prepared.n) or x.shape[1] != prepared.k:
        raise ValueError(f"routed output must be [{routes}, {prepared.n}] for x {tuple(x.shape)}")
    if rows.row_map.numel() != routes:
        raise ValueError("row_map must hold every route")
    launch = _MoELaunch(x, prepared, output, rows, top_k, params.block_m, routes)
    return params.block_m, PackedOperatorBinding(output, (launch,),
                                                 scratch=(launch.padded, launch.block_expert))


def bind_grouped(operators: PackedLinearOperators, x: Tensor, gate: tuple[QuantizedMatrix, ...],
                 up: tuple[QuantizedMatrix, ...], output: Tensor, rows: RoutedRows, top_k: int,
                 params: CubicMoEParameters | None = None):
    """Gate and up of every expert in one routed launch (marlin.py:230-242)."""
    params = params or CubicMoEParameters()
    if not params.grouped_projections:
        return None
    return _bind(operators, x, (tuple(gate), tuple(up)), output, rows, top_k, params)


def bind_routed(operators: PackedLinearOperators, x: Tensor, weights: tuple[QuantizedMatrix, ...],
                output: Tensor, rows: RoutedRows, params: CubicMoEParameters | None = None):
    """One projection per route (down; x holds one row per route) (marlin.py:245-253)."""
    params = params or CubicMoEParameters()
    return _bind(operators, x, (tuple(weights),), output, rows, 1, params)
