"""Packed Cubic linear operators on gfx950.

Host mirror of the reference's operator API (paths under src/cubic_serve/):
  PackedOperatorBinding        quantization/common/binding.py:134-265
  PackedLinearOperators        ops/cuda/linear/quantized.py:248-697
    .bind_linear               :559-697   (validation :348-405)
    .bind_linear_group         :445-507
    .linear                    :531-538
  Cubic ``linear`` hooks       quantization/extensions/cubic/linear.py
    arguments                  :71-120
    bind_native                :123-131
    bind_linear                :134-263
    bind_grouped               :297-305
    bind_embedding             :266-294   (operator side quantized.py:776-846)

Every launch goes through the HIP library (include/cubic_mi355x.h); there is
no eager fallback.  Weights are prepared once per matrix (codes repacked into
MFMA fragment order, metadata expanded), cached on the operators object like
the reference's ``prepared_weights`` (cubic/linear.py:43-68).  Bindings own
their split-K workspace and allocate nothing at launch.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch
from torch import Tensor

from . import _native
from .quantization import METADATA_IDS, QuantizedMatrix, partition_rows


MAX_GROUP_MEMBERS = 8  # kMaxGemmMembers of the C ABI


@dataclass(frozen=True, slots=True)
class CubicLinearParameters:
    """Format parameters (quantization/extensions/cubic/policy.py:18-40 analogue).

    ``native_enabled`` plays the role of ``marlin_enabled``: False makes
    bind_native decline (returns None).
    """

    native_enabled: bool = True


@dataclass(frozen=True, slots=True)
class PreparedCubic:
    """Format-prepared derivative of one QuantizedMatrix (device-resident)."""

    codes: Tensor   # int32 words, MFMA fragment order
    meta: Tensor    # int32 words: level tables (bits <= 4) or (scale, a | b << 16) per (column, group)
    n: int
    k: int
    bits: int
    group_in: int
    dtype: torch.dtype = torch.bfloat16  # activation dtype the level tables are rounded to


DTYPE_IDS = {torch.bfloat16: 0, torch.float16: 1}  # CUBIC_DTYPE_BF16 / CUBIC_DTYPE_F16


def _versions(matrix: QuantizedMatrix) -> tuple:
    versions = []
    for tensor in matrix.payload.values():
        try:
            versions.append(tensor._version)
        except RuntimeError:  # inference-mode tensors
            versions.append(None)
    return tuple(versions)


def prepare_matrix(matrix: QuantizedMatrix, device: torch.device | None = None,
                   dtype: torch.dtype = torch.bfloat16) -> PreparedCubic:
    """Repack a Cubic payload for the gfx950 GEMM with `dtype` activations
    (load time, allocates)."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("Cubic weights require cold preparation before capture")
    if dtype not in DTYPE_IDS:
        raise ValueError("Cubic weights serve BF16 or FP16 activations")
    enc = matrix.encoding
    device = torch.device(device) if device is not None else matrix.device
    matrix = matrix.to(device)
    n, k = matrix.shape
    p = matrix.payload
    fmt = METADATA_IDS[enc.metadata]
    code_words = _native.ctypes.c_int64()
    meta_words = _native.ctypes.c_int64()
    _native.call("cubic_prepared_words", n, k, enc.bits, enc.group_in,
                 _native.ctypes.byref(code_words), _native.ctypes.byref(meta_words))
    codes = torch.empty(code_words.value, dtype=torch.int32, device=device)
    meta = torch.empty(meta_words.value, dtype=torch.int32, device=device)
    scratch_bytes = _native.lib().cubic_prepare_scratch_bytes(n, k, enc.group_in)
    scratch = torch.empty(scratch_bytes, dtype=torch.uint8, device=device)
    parts = partition_rows(matrix)
    if fmt == 0:
        tensors = (p["weight_scale"], p["weight_a"], p["weight_b"], None, None, None)
    elif fmt == 1:
        tensors = (p["weight_scale"], p["weight_ab"], None, p["weight_scale_global"],
                   p["weight_a_global"], p["weight_b_global"])
    else:
        tensors = (p["weight_metadata"], p["weight_curve_a"], p["weight_curve_b"], None, None, None)
    with torch.cuda.device(device):
        _native.call("cubic_prepare_weight", fmt, p["weight_packed"].data_ptr(),
                     *(_native.ptr(t) for t in tensors), parts.data_ptr(), n, k, enc.bits,
                     enc.group_in, enc.group_out, DTYPE_IDS[dtype], scratch.data_ptr(), scratch_bytes,
                     codes.data_ptr(), meta.data_ptr(), _native.stream_of(device))
        torch.cuda.current_stream(device).synchronize()
    return PreparedCubic(codes, meta, n, k, enc.bits, enc.group_in, dtype)


def _storage(t: Tensor) -> int:
    return t.untyped_storage().data_ptr()


def gemm_workspace_bytes(m: int, widths: Sequence[int], k: int, bits: int) -> int:
    """Split-K workspace of one bound launch over members of the given widths."""
    lib = _native.lib()
    widths = tuple(widths)
    if len(widths) == 1:
        return lib.cubic_gemm_workspace_bytes(m, widths[0], k, bits)
    if len(set(widths)) == 1:
        return lib.cubic_gemm_group_workspace_bytes(m, len(widths), widths[0], k, bits)
    if len(widths) == 2:
        return lib.cubic_gemm_grouped_workspace_bytes(m, widths[0], widths[1], k, bits)
    raise ValueError("grouped members of different widths are limited to two")


class _GemmLaunch:
    """One bound cubic_gemm / cubic_gemm_group / cubic_gemm_grouped call."""

    def __init__(self, x: Tensor, prepared: PreparedCubic, outputs: Sequence[Tensor],
                 widths: Sequence[int], workspace: Tensor | None):
        self.x, self.prepared, self.outputs, self.widths = x, prepared, tuple(outputs), tuple(widths)
        self.workspace = workspace
        self.identity = tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype)
                              for t in (x, *self.outputs))
        members = len(self.outputs)
        # host tables of a same-width group, built once and kept alive here
        self._ys = (_native.ctypes.c_void_p * members)(*(y.data_ptr() for y in self.outputs))
        self._ldys = (_native.ctypes.c_int64 * members)(*(y.stride(0) for y in self.outputs))

    def validate(self) -> None:
        now = tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype)
                    for t in (self.x, *self.outputs))
        if now != self.identity:
            raise ValueError("packed launch operands changed after binding")

    def __call__(self, stream: int) -> None:
        x, pr = self.x, self.prepared
        m = x.shape[0]
        dt = DTYPE_IDS[pr.dtype]
        ws = self.workspace
        ws_ptr, ws_bytes = (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)
        if len(self.outputs) == 1:
            y = self.outputs[0]
            _native.call("cubic_gemm", x.data_ptr(), x.stride(0), pr.codes.data_ptr(),
                         pr.meta.data_ptr(), m, pr.n, pr.k, pr.bits, pr.group_in, dt, y.data_ptr(),
                         y.stride(0), ws_ptr, ws_bytes, stream)
        elif len(set(self.widths)) == 1:
            _native.call("cubic_gemm_group", x.data_ptr(), x.stride(0), pr.codes.data_ptr(),
                         pr.meta.data_ptr(), m, len(self.widths), self.widths[0], pr.k, pr.bits,
                         pr.group_in, dt, self._ys, self._ldys, ws_ptr, ws_bytes, stream)
        else:
            y0, y1 = self.outputs
            _native.call("cubic_gemm_grouped", x.data_ptr(), x.stride(0), pr.codes.data_ptr(),
                         pr.meta.data_ptr(), m, self.widths[0], self.widths[1], pr.k, pr.bits,
                         pr.group_in, dt, y0.data_ptr(), y0.stride(0), y1.data_ptr(), y1.stride(0),
                         ws_ptr, ws_bytes, stream)


class PackedOperatorBinding:
    """Startup-bound native launches with owned scratch (binding.py:134-265)."""

    def __init__(self, output: Tensor | tuple[Tensor, ...], launches: tuple, *,
                 scratch: tuple[Tensor, ...] = (), row_tile_count: int | None = None):
        if row_tile_count is not None and (type(row_tile_count) is not int or row_tile_count < 1):
            raise ValueError("row tile count must be a positive integer")
        self.output = output
        self.scratch = scratch
        self.row_tile_count = row_tile_count
        self._launches = launches
        self._ordinal = 0

    def validate_operands(self) -> None:
        for item in self._launches:
            item.validate()

    def launch(self) -> int:
        """Enqueue every launch on the current stream; returns the launch ordinal."""
        self.validate_operands()
        self._ordinal += 1
        first = self.output[0] if isinstance(self.output, tuple) else self.output
        with torch.cuda.device(first.device):
            stream = _native.stream_of(first.device)
            for item in self._launches:
                item(stream)
        return self._ordinal


# --------------------------------------------------------------------------- #
# Cubic extension ``linear`` hooks
# --------------------------------------------------------------------------- #
def arguments(operators: "PackedLinearOperators", matrix: QuantizedMatrix):
    """Payload pointer columns + metadata format id (cubic/linear.py:71-120).

    Returns (tensors, fmt) with the reference's 9-slot layout: packed, scale,
    dummy, a|ab, b, global scale, global a, global b, partition-per-group-row.
    The fmt ids follow the reference (1 = int8 globals, 2 = curve2, 3 = f32).
    """
    p, e = matrix.payload, matrix.encoding
    dummy = next(iter(p.values()))
    key = id(matrix)
    cached = operators._partitions.get(key)
    if cached is None or cached[0] is not matrix:
        # the matrix is kept in the value, so its id cannot be reused while cached
        counts = matrix.partitions or (matrix.shape[0],)
        cached = operators._partitions[key] = (matrix, torch.tensor(
            [i for i, count in enumerate(counts) for _ in range(count // e.group_out)],
            dtype=torch.int32, device=dummy.device))
    parts = cached[1]
    if e.metadata == "int8-scale-int4-ab-global-fp32":
        return (p["weight_packed"], p["weight_scale"], dummy, p["weight_ab"], dummy,
                p["weight_scale_global"], p["weight_a_global"], p["weight_b_global"], parts), 1
    if e.metadata == "e5m9-scale-curve2-tensor-fp16":
        return (p["weight_packed"], p["weight_metadata"], dummy, p["weight_curve_a"],
                p["weight_curve_b"], dummy, dummy, dummy, parts), 2
    return (p["weight_packed"], p["weight_scale"], dummy, p["weight_a"], p["weight_b"], dummy,
            dummy, dummy, parts), 3


def bind_native(operators, x, weight, output, params, fp8_token_scales=None):
    """Format-local admission: a binding, or None when not admitted (:123-131)."""
    if fp8_token_scales is not None:
        raise ValueError("Cubic is a weight-only (WNA16) format")
    if isinstance(params, CubicLinearParameters) and not params.native_enabled:
        return None
    if not admitted(weight, x):
        return None
    return operators._bind_gemm(x, (weight,), (output,))


def admitted(weight: QuantizedMatrix, x: Tensor) -> bool:
    """Kernel geometry admission (cubic/marlin.py:256-336 analogue)."""
    e = weight.encoding
    return (1 <= e.bits <= 8 and e.group_in % 32 == 0 and weight.shape[1] % 8 == 0
            and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0)


def bind_linear(operators, x, weight, output, params=None, fp8_token_scales=None):
    """Cubic linear binding (:134-263): native kernel or an explicit error."""
    binding = bind_native(operators, x, weight, output, params, fp8_token_scales)
    if binding is None:
        raise ValueError("Cubic native linear is not admitted for this geometry and has no fallback")
    return binding


def bind_grouped(operators, x, weights, outputs, params=None):
    """Same-input members in one launch (:297-305); None if not admitted.

    Members must share shape and encoding (cubic/marlin.py:347-360 plans the
    launch on one member, so grouping never changes a member's K partition);
    anything else is declined and bound as separate launches.
    """
    if not 2 <= len(weights) <= MAX_GROUP_MEMBERS or any(not admitted(w, x) for w in weights):
        return None
    base = weights[0]
    if any(w.encoding != base.encoding or w.shape != base.shape for w in weights) or base.shape[0] % 16:
        return None
    return operators._bind_gemm(x, tuple(weights), tuple(outputs))


class _EmbeddingLaunch:
    """One bound cubic_embedding call over a payload as stored."""

    def __init__(self, input_ids: Tensor, weight: QuantizedMatrix, output: Tensor, parts: Tensor):
        self.input_ids, self.weight, self.output, self.parts = input_ids, weight, output, parts
        self.identity = self._identity()

    def _identity(self):
        return tuple((t.data_ptr(), tuple(t.shape), t.dtype) for t in
                     (self.input_ids, self.output, *self.weight.payload.values()))

    def validate(self) -> None:
        if self._identity() != self.identity:
            raise ValueError("packed launch operands changed after binding")

    def __call__(self, stream: int) -> None:
        w, e = self.weight, self.weight.encoding
        p = w.payload
        fmt = METADATA_IDS[e.metadata]
        if fmt == 0:
            meta = (p["weight_scale"], p["weight_a"], p["weight_b"], None, None, None)
        elif fmt == 1:
            meta = (p["weight_scale"], p["weight_ab"], None, p["weight_scale_global"],
                    p["weight_a_global"], p["weight_b_global"])
        else:
            meta = (p["weight_metadata"], p["weight_curve_a"], p["weight_curve_b"], None, None, None)
        n, k = w.shape
        _native.call("cubic_embedding", self.input_ids.data_ptr(), self.input_ids.element_size(),
                     self.input_ids.numel(), fmt, p["weight_packed"].data_ptr(),
                     *(_native.ptr(t) for t in meta), self.parts.data_ptr(), n, k, e.bits,
                     e.group_in, e.group_out, self.output.data_ptr(),
                     1 if self.output.dtype == torch.float16 else 0, stream)


def bind_embedding(operators, input_ids, weight, output, params=None):
    """Cubic embedding hook (:266-294): decode the looked-up rows from the payload."""
    if isinstance(params, CubicLinearParameters) and not params.native_enabled:
        raise ValueError("Cubic native embedding is disabled and has no fallback")
    key = ("cubic.mi355x.parts.v1", id(weight), str(input_ids.device))
    cached = operators.prepared_weights.get(key)
    if cached is None:
        cached = operators.prepared_weights[key] = (weight, partition_rows(weight).to(input_ids.device))
    return PackedOperatorBinding(output, (_EmbeddingLaunch(input_ids, weight, output, cached[1]),))


class PackedLinearOperators:
    """Binds Cubic linears to native launches before capture (quantized.py:248)."""

    def __init__(self, device: torch.device | str | None = None):
        self.device = torch.device(device) if device is not None else None
        self.prepared_weights: dict = {}
        self._partitions: dict = {}

    # -- preparation -------------------------------------------------------
    def prepared(self, weights: tuple[QuantizedMatrix, ...], device: torch.device,
                 dtype: torch.dtype = torch.bfloat16) -> PreparedCubic:
        key = ("cubic.mi355x.v1", tuple(id(w) for w in weights), tuple(_versions(w) for w in weights),
               str(device), dtype)
        cached = self.prepared_weights.get(key)
        if cached is not None:
            return cached[1]
        parts = [prepare_matrix(w, device, dtype) for w in weights]
        if len(parts) == 1:
            prepared = parts[0]
        else:
            # members with N % 16 == 0 concatenate tile-for-tile along N
            meta = torch.cat([p.meta for p in parts])
            codes = torch.cat([p.codes for p in parts])
            prepared = PreparedCubic(codes, meta, sum(p.n for p in parts), parts[0].k,
                                     parts[0].bits, parts[0].group_in, dtype)
        self.prepared_weights[key] = (weights, prepared)
        return prepared

    # -- validation (quantized.py:348-405) ------------------------------------
    @staticmethod
    def _validate(x: Tensor, weight: QuantizedMatrix, output: Tensor) -> None:
        if x.dtype not in (torch.float16, torch.bfloat16) or not x.is_cuda:
            raise ValueError("native linear requires CUDA FP16/BF16 activations")
        if not isinstance(weight, QuantizedMatrix):
            raise TypeError("native Cubic linear requires a packed matrix")
        if weight.device != x.device and weight.device.type != "cpu":
            raise ValueError("linear weights and activations must share one device")
        if x.ndim != 2 or not x.is_contiguous() or min(x.shape) <= 0:
            raise ValueError("bound linear requires contiguous positive [M,K] activations")
        if weight.shape[1] != x.shape[1]:
            raise ValueError("bound linear weight K differs")
        n = weight.shape[0]
        if (output.shape != (x.shape[0], n) or output.dtype != x.dtype
                or output.device != x.device or not output.is_contiguous()):
            raise ValueError("bound linear output has an invalid ABI")
        if any(_storage(output) == _storage(t) for t in (x, *weight.payload.values())):
            raise ValueError("bound linear output must not alias its operands")

    def _bind_gemm(self, x: Tensor, weights: tuple, outputs: tuple) -> PackedOperatorBinding:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("Cubic linears must be bound before graph capture")
        prepared = self.prepared(weights, x.device, x.dtype)
        widths = [w.shape[0] for w in weights]
        ws_bytes = gemm_workspace_bytes(x.shape[0], widths, prepared.k, prepared.bits)
        if ws_bytes < 0:
            raise ValueError("invalid GEMM geometry")
        workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
        launch = _GemmLaunch(x, prepared, outputs, widths, workspace)
        out = outputs[0] if len(outputs) == 1 else tuple(outputs)
        return PackedOperatorBinding(out, (launch,),
                                     scratch=(workspace,) if workspace is not None else ())

    # -- public API ------------------------------------------------------------
    def bind_linear(self, x: Tensor, weight: QuantizedMatrix, output: Tensor,
                    params: CubicLinearParameters | None = None) -> PackedOperatorBinding:
        self._validate(x, weight, output)
        return bind_linear(self, x, weight, output, params)

    def bind_linear_group(self, x: Tensor, weights: Sequence[QuantizedMatrix],
                          outputs: Sequence[Tensor],
                          params: CubicLinearParameters | None = None) -> PackedOperatorBinding:
        weights, outputs = tuple(weights), tuple(outputs)
        if len(weights) != len(outputs) or not weights:
            raise ValueError("grouped linear needs one output per member")
        for w, y in zip(weights, outputs):
            self._validate(x, w, y)
        binding = bind_grouped(self, x, weights, outputs, params)
        if binding is not None:
            return binding
        launches = tuple(l for w, y in zip(weights, outputs)
                         for l in bind_linear(self, x, w, y, params)._launches)
        return PackedOperatorBinding(outputs, launches)

    def embedding(self, input_ids: Tensor, weight: QuantizedMatrix, *, dtype: torch.dtype) -> Tensor:
        """Eager lookup (quantized.py:776-784)."""
        output = torch.empty((*input_ids.shape, weight.shape[1]), dtype=dtype, device=input_ids.device)
        self.bind_embedding(input_ids.contiguous(), weight, output).launch()
        return output

    def bind_embedding(self, input_ids: Tensor, weight: QuantizedMatrix, output: Tensor,
                       params: CubicLinearParameters | None = None) -> PackedOperatorBinding:
        """Bind a lookup; ids are read at launch (validation quantized.py:793-826)."""
        if not isinstance(weight, QuantizedMatrix) or len(weight.shape) != 2:
            raise ValueError("native Cubic embedding requires a packed matrix weight")
        tensors = (input_ids, output, *weight.payload.values())
        k = weight.shape[1]
        if (not input_ids.is_cuda
                or input_ids.dtype not in (torch.int32, torch.int64)
                or input_ids.numel() <= 0
                or output.dtype not in (torch.float16, torch.bfloat16)
                or output.shape != (*input_ids.shape, k)
                or any(t.device != input_ids.device or not t.is_contiguous() for t in tensors)):
            raise ValueError("bound embedding requires contiguous same-device IDs, weight and FP16/BF16 output")
        if any(_storage(output) == _storage(t) for t in (input_ids, *weight.payload.values())):
            raise ValueError("bound embedding output must not alias its operands")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("Cubic embeddings must be bound before graph capture")
        return bind_embedding(self, input_ids, weight, output, params)

    def linear(self, x: Tensor, weight: QuantizedMatrix) -> Tensor:
        """Eager convenience: bind, launch once, return the output."""
        output = torch.empty((x.shape[0], weight.shape[0]), dtype=x.dtype, device=x.device)
        self.bind_linear(x, weight, output).launch()
        return output


def bind_prepared(x: Tensor, prepared: PreparedCubic, outputs: Sequence[Tensor],
                  widths: Sequence[int] | None = None) -> PackedOperatorBinding:
    """Bind an already prepared weight (one output, or two grouped members).

    ``widths`` gives the member column counts of a grouped weight; the
    binding owns its split-K workspace.
    """
    outputs = tuple(outputs)
    widths = tuple(widths) if widths is not None else (prepared.n,)
    if len(widths) != len(outputs) or sum(widths) != prepared.n:
        raise ValueError("grouped widths must cover the prepared columns")
    if x.dtype is not prepared.dtype or x.ndim != 2 or x.shape[1] != prepared.k:
        raise ValueError("bound linear requires [M, K] activations of the prepared dtype")
    for y, w in zip(outputs, widths):
        if y.shape != (x.shape[0], w) or y.dtype is not prepared.dtype or not y.is_contiguous():
            raise ValueError("bound linear output has an invalid ABI")
    ws_bytes = gemm_workspace_bytes(x.shape[0], widths, prepared.k, prepared.bits)
    if ws_bytes < 0:
        raise ValueError("invalid GEMM geometry")
    workspace = torch.zeros(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
    launch = _GemmLaunch(x, prepared, outputs, widths, workspace)
    out = outputs[0] if len(outputs) == 1 else outputs
    return PackedOperatorBinding(out, (launch,), scratch=(workspace,) if workspace is not None else ())


def clone_prepared(prepared: PreparedCubic) -> PreparedCubic:
    """A copy in distinct device memory (same values)."""
    return PreparedCubic(prepared.codes.clone(), prepared.meta.clone(), prepared.n, prepared.k,
                         prepared.bits, prepared.group_in, prepared.dtype)
