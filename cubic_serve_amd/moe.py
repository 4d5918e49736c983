"""Routed-expert (MoE) Cubic GEMM behind the Cubic extension's MoE hooks.

Router and compaction: ``bind_route_selection`` (ops/cuda/moe/quantized.py:58-180,
kernels ops/cuda/moe/fused.py:44-156) and ``bind_compact_routes``
(_compact_local_routes, fused.py:174-199), composed by ``MoERouting``.

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
from .linear import DTYPE_IDS, PackedLinearOperators, PackedOperatorBinding, prepare_matrix
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


def _i32(n: int, device) -> Tensor:
    return torch.empty((n,), dtype=torch.int32, device=device)


class _RouteLaunch:
    """cubic_moe_route over fixed operands (identity-checked at launch)."""

    def __init__(self, *operands: Tensor):
        self.operands = operands
        self.identity = self._identity()

    def _identity(self):
        return tuple((t.data_ptr(), tuple(t.shape), t.dtype) for t in self.operands)

    def validate(self) -> None:
        if self._identity() != self.identity:
            raise ValueError("routing operands changed after binding")

    def __call__(self, stream: int) -> None:
        logits, activity, active_rows, top_logits, top_ids, route_ids, route_weights = self.operands
        rows, experts = logits.shape
        _native.call("cubic_moe_route", logits.data_ptr(), int(logits.dtype == torch.float16),
                     activity.data_ptr(), active_rows.data_ptr(), rows, experts, top_ids.shape[1],
                     top_logits.data_ptr(), top_ids.data_ptr(), route_ids.data_ptr(),
                     route_weights.data_ptr(), int(route_weights.dtype == torch.float16), stream)


class _CompactLaunch(_RouteLaunch):
    """cubic_moe_compact over fixed operands."""

    def __init__(self, *operands: Tensor, first_expert: int, experts: int, block_m: int):
        super().__init__(*operands)
        self.first_expert, self.experts, self.block_m = first_expert, experts, block_m

    def __call__(self, stream: int) -> None:
        route_ids, counts, starts, block_starts, total, row_map = self.operands
        _native.call("cubic_moe_compact", route_ids.data_ptr(), route_ids.numel(), self.first_expert,
                     self.experts, self.block_m, counts.data_ptr(), starts.data_ptr(),
                     block_starts.data_ptr(), total.data_ptr(), row_map.data_ptr(), stream)


def bind_route_selection(logits: Tensor, activity: Tensor, active_rows: Tensor, top_logits: Tensor,
                         top_ids: Tensor, route_ids: Tensor, route_weights: Tensor) -> PackedOperatorBinding:
    """Router launch (ops/cuda/moe/quantized.py:58-180, kernels fused.py:44-156).

    Per row: top_k experts by (logit desc, id asc) into top_logits/top_ids;
    softmax over those logits, ordered by ascending expert id, into
    route_ids/route_weights.  Rows at or past ``active_rows[0]`` or with
    ``activity`` 0 publish 0 / -1 / -1 / 0.
    """
    tensors = (logits, activity, active_rows, top_logits, top_ids, route_ids, route_weights)
    if any(not isinstance(t, Tensor) for t in tensors):
        raise TypeError("routing operands must be tensors")
    if any(t.device.type != "cuda" or t.device != logits.device or not t.is_contiguous() for t in tensors):
        raise ValueError("routing operands must be contiguous tensors on one CUDA device")
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("routing must be bound before graph capture")
    if logits.ndim != 2 or top_ids.ndim != 2:
        raise ValueError("router needs [rows,experts] logits and [rows,top_k] outputs")
    rows, experts = logits.shape
    top_k = top_ids.shape[1]
    if (logits.dtype not in (torch.bfloat16, torch.float16)
            or activity.dtype is not torch.int32 or activity.shape != (rows,)
            or active_rows.dtype is not torch.int32 or active_rows.shape != (1,)
            or top_logits.dtype is not torch.float32 or top_logits.shape != (rows, top_k)
            or top_ids.dtype is not torch.int64 or route_ids.dtype is not torch.int64
            or route_ids.shape != (rows, top_k) or route_weights.shape != (rows, top_k)
            or route_weights.dtype not in (torch.bfloat16, torch.float16)):
        raise ValueError("routing operands differ from the BF16/FP16 router ABI")
    if not 0 < top_k <= experts:
        raise ValueError("router needs [rows,experts] logits and a valid top-k")
    return PackedOperatorBinding(route_weights, (_RouteLaunch(*tensors),))


def bind_compact_routes(route_ids: Tensor, counts: Tensor, starts: Tensor, block_starts: Tensor,
                        total_blocks: Tensor, row_map: Tensor, *, first_expert: int, experts: int,
                        block_m: int) -> PackedOperatorBinding:
    """Compaction launch (_compact_local_routes, ops/cuda/moe/fused.py:174-199)."""
    tensors = (route_ids, counts, starts, block_starts, total_blocks, row_map)
    if any(t.device.type != "cuda" or t.device != route_ids.device or not t.is_contiguous()
           for t in tensors):
        raise ValueError("compaction operands must be contiguous tensors on one CUDA device")
    if (route_ids.dtype is not torch.int64 or any(t.dtype is not torch.int32 for t in tensors[1:])
            or any(t.shape != (experts,) for t in (counts, starts, block_starts))
            or total_blocks.shape != (1,) or row_map.shape != (route_ids.numel(),)):
        raise ValueError("compaction operands differ from the route ABI")
    if type(first_expert) is not int or first_expert < 0 or type(block_m) is not int or block_m < 1:
        raise ValueError("compaction needs first_expert >= 0 and block_m >= 1")
    return PackedOperatorBinding(row_map, (_CompactLaunch(*tensors, first_expert=first_expert,
                                                          experts=experts, block_m=block_m),))


def route_rows(topk_ids: Tensor, experts: int, block_m: int, first_expert: int = 0) -> RoutedRows:
    """Compact [tokens, top_k] routes by expert on the device (allocates).

    Routes outside [first_expert, first_expert + experts) are skipped; the
    row map then holds only the owned routes (the rest of it is unspecified).
    """
    if topk_ids.ndim != 2:
        raise ValueError("routes need [tokens, top_k] expert ids")
    ids = topk_ids.to(torch.int64).contiguous()
    dev = ids.device
    rows = RoutedRows(_i32(experts, dev), _i32(experts, dev), _i32(experts, dev), _i32(1, dev),
                      _i32(ids.numel(), dev), mean_rows_per_expert=ids.numel() / experts,
                      routing_top_k=topk_ids.shape[1])
    bind_compact_routes(ids, rows.counts, rows.starts, rows.block_starts, rows.total_blocks,
                        rows.row_map, first_expert=first_expert, experts=experts,
                        block_m=block_m).launch()
    return rows


class MoERouting:
    """Router + compaction for fixed [rows, experts] logits (bound once).

    ``launch()`` enqueues the router then the compaction; afterwards
    ``route_ids``/``route_weights`` hold the routes and ``rows`` the
    expert-grouped RoutedRows that bind_grouped / bind_routed consume.
    """

    def __init__(self, logits: Tensor, activity: Tensor, active_rows: Tensor, *, top_k: int,
                 first_expert: int = 0, experts: int | None = None, block_m: int = 32,
                 weights_dtype: torch.dtype | None = None):
        dev = logits.device
        m, global_experts = logits.shape
        experts = global_experts - first_expert if experts is None else experts
        self.top_logits = torch.empty((m, top_k), dtype=torch.float32, device=dev)
        self.top_ids = torch.empty((m, top_k), dtype=torch.int64, device=dev)
        self.route_ids = torch.empty_like(self.top_ids)
        self.route_weights = torch.empty((m, top_k), dtype=weights_dtype or logits.dtype, device=dev)
        self.rows = RoutedRows(_i32(experts, dev), _i32(experts, dev), _i32(experts, dev), _i32(1, dev),
                               _i32(m * top_k, dev), mean_rows_per_expert=m * top_k / experts,
                               routing_top_k=top_k)
        self.select = bind_route_selection(logits, activity, active_rows, self.top_logits, self.top_ids,
                                           self.route_ids, self.route_weights)
        r = self.rows
        self.compact = bind_compact_routes(self.route_ids, r.counts, r.starts, r.block_starts,
                                           r.total_blocks, r.row_map, first_expert=first_expert,
                                           experts=experts, block_m=block_m)

    def launch(self) -> None:
        self.select.launch()
        self.compact.launch()


@dataclass(frozen=True, slots=True)
class PreparedExperts:
    codes: Tensor  # [experts, code words] int32
    meta: Tensor   # [experts, meta words] int32
    n: int
    k: int
    bits: int
    group_in: int
    dtype: torch.dtype = torch.bfloat16  # activation dtype of the level tables

    @property
    def experts(self) -> int:
        return self.codes.shape[0]


def prepare_experts(groups: Sequence[Sequence[QuantizedMatrix]], device: torch.device,
                    dtype: torch.dtype = torch.bfloat16) -> PreparedExperts:
    """Per expert, the group members (gate, up) prepared as one [sum n, k]
    matrix, experts stacked with a fixed stride (load time, allocates)."""
    experts = len(groups[0])
    if any(len(g) != experts for g in groups):
        raise ValueError("every group needs one matrix per expert")
    codes, meta, first = [], [], None
    for e in range(experts):
        parts = [prepare_matrix(g[e], device, dtype) for g in groups]
        first = first or parts[0]
        codes.append(torch.cat([p.codes for p in parts]))
        meta.append(torch.cat([p.meta for p in parts]))
    n = sum(g[0].shape[0] for g in groups)
    return PreparedExperts(torch.stack(codes), torch.stack(meta), n, first.k, first.bits, first.group_in,
                           dtype)


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
                     DTYPE_IDS[pr.dtype], self.output.data_ptr(), self.output.stride(0), stream)


def _admitted(groups, x: Tensor, output: Tensor, params: CubicMoEParameters) -> bool:
    base = groups[0][0]
    enc = base.encoding
    return (params.native_enabled and params.block_m in (16, 32, 64) and enc.group_out == 1
            and 1 <= enc.bits <= 8 and enc.group_in % 32 == 0 and base.shape[1] % 8 == 0
            and x.dtype in DTYPE_IDS and output.dtype == x.dtype
            and all(w.encoding == enc and w.shape[1] == base.shape[1] and w.shape[0] % 16 == 0
                    for g in groups for w in g))


def _bind(operators: PackedLinearOperators, x: Tensor, groups, output: Tensor, rows: RoutedRows,
          top_k: int, params: CubicMoEParameters):
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError("routed Cubic experts must be bound before graph capture")
    if not _admitted(groups, x, output, params):
        return None
    key = ("cubic.mi355x.moe.v1", tuple(tuple(id(w) for w in g) for g in groups), str(x.device), x.dtype)
    cached = operators.prepared_weights.get(key)
    if cached is None:
        cached = operators.prepared_weights[key] = (groups, prepare_experts(groups, x.device, x.dtype))
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
