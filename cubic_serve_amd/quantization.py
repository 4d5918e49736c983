"""Cubic weight records and the build-owned encoder.

Mirrors the boundary types of the reference (paths under src/cubic_serve/):
  QuantizationScheme   models/quantization.py:32-56
  QuantizedMatrix      models/quantized_checkpoint.py:648-730
  payload_headers      quantization/extensions/cubic/layout.py:22-55
  slice_index          quantization/extensions/cubic/layout.py:58-104 (rows, columns)
  parse_group          quantization/extensions/cubic/checkpoint.py:22-55

The reference only decodes Cubic payloads; ``quantize_cubic`` is this build's
deterministic encoder for synthetic fixtures (nearest-level assignment over a
small grid of curves per group).  Parity never depends on its choices: the
kernels are compared with the reference decode of the same payload.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Mapping

import torch
from torch import Tensor

CUBIC_FORMAT = "cubic-bitstream-v1"
FMT_F32 = "float32-scale-float16-ab"
FMT_I8 = "int8-scale-int4-ab-global-fp32"
FMT_CURVE2 = "e5m9-scale-curve2-tensor-fp16"
METADATA_FORMATS = (FMT_F32, FMT_I8, FMT_CURVE2)
METADATA_IDS = {FMT_F32: 0, FMT_I8: 1, FMT_CURVE2: 2}


class QuantizationError(ValueError):
    """A packed payload or encoding violates the Cubic format contract."""


@dataclass(frozen=True, slots=True)
class QuantizationScheme:
    format: str
    bits: int
    group_in: int
    group_out: int = 1
    metadata: str = FMT_F32
    activation: str = "identity"

    def __post_init__(self) -> None:
        if self.format != CUBIC_FORMAT:
            raise QuantizationError(f"unsupported weight format {self.format!r}")
        if any(type(v) is not int or v <= 0 for v in (self.bits, self.group_in, self.group_out)):
            raise QuantizationError("bit width and quantization groups must be positive integers")
        # checkpoint.py:66-77 validate_scheme
        if self.bits not in range(1, 9):
            raise QuantizationError("unsupported Cubic bit width")
        if self.metadata not in METADATA_FORMATS:
            raise QuantizationError("unsupported Cubic metadata")
        if self.activation != "identity":
            raise QuantizationError("activation encoding is incompatible with weight format")


def positive_int(value: object) -> int:
    """models/quantization.py:183-186: a group size or bit width is a positive int."""
    if type(value) is not int or value <= 0:
        raise QuantizationError("quantization group size must be a positive integer")
    return value


def parse_group(group: Mapping[str, object], weights: Mapping[str, object]) -> QuantizationScheme:
    """``cubic-pack-quantized`` config group -> scheme (checkpoint.py:22-55)."""
    if weights.get("dynamic") is not False or weights.get("symmetric") is not True:
        raise QuantizationError("checkpoint weights require static symmetric encoding")
    if group.get("input_activations") is not None:
        raise QuantizationError("Cubic runtime activation transforms require a separate policy")
    size = weights.get("group_size")
    if isinstance(size, list) and len(size) == 2:
        group_out, group_in = (positive_int(v) for v in size)
    else:
        group_out, group_in = 1, positive_int(size)
    bits = positive_int(weights.get("num_bits"))
    if weights.get("packing") != "little-endian-bitstream":
        raise QuantizationError("Cubic requires little-endian bitstream packing")
    if weights.get("reserved_code") != ("binary" if bits == 1 else "zero"):
        raise QuantizationError("Cubic reserved-code convention differs")
    metadata = weights.get("metadata_format", FMT_F32)
    dtypes = {
        FMT_F32: (("torch.float32", "float32"), ("torch.float16", "float16")),
        FMT_I8: (("torch.int8", "int8"), ("packed_int4",)),
        FMT_CURVE2: (("packed_e5m9",), ("torch.float16", "float16")),
    }
    if (metadata not in dtypes or weights.get("scale_dtype") not in dtypes[metadata][0]
            or weights.get("param_dtype") not in dtypes[metadata][1]):
        raise QuantizationError("Cubic metadata dtype declaration differs from its format")
    if metadata == FMT_CURVE2 and weights.get("curve_count") != 4:
        raise QuantizationError("Cubic curve2 requires four curves")
    return QuantizationScheme(CUBIC_FORMAT, bits, group_in, group_out, str(metadata))


def payload_headers(shape: tuple[int, int], encoding: QuantizationScheme,
                    partitions: tuple[int, ...] = ()) -> tuple[tuple[str, torch.dtype, tuple], ...]:
    """(name, dtype, shape) of every payload tensor (layout.py:22-55)."""
    n, k = shape
    if n % encoding.group_out:
        raise QuantizationError("Cubic logical rows do not close output groups")
    groups = (n // encoding.group_out, math.ceil(k / encoding.group_in))
    parts = partitions or (n,)
    if any(p % encoding.group_out for p in parts):
        raise QuantizationError("Cubic partition cuts an output group")
    packed = ("weight_packed", torch.uint8, (n, math.ceil(k * encoding.bits / 8)))
    if encoding.metadata == FMT_I8:
        return (packed, ("weight_scale", torch.int8, groups), ("weight_ab", torch.uint8, groups),
                *((name, torch.float32, (len(parts),))
                  for name in ("weight_scale_global", "weight_a_global", "weight_b_global")))
    if encoding.metadata == FMT_CURVE2:
        return (packed, ("weight_metadata", torch.uint16, groups),
                ("weight_curve_a", torch.float16, (len(parts), 4)),
                ("weight_curve_b", torch.float16, (len(parts), 4)))
    return (packed, ("weight_scale", torch.float32, groups), ("weight_a", torch.float16, groups),
            ("weight_b", torch.float16, groups))


@dataclass(frozen=True, slots=True)
class QuantizedMatrix:
    """Immutable packed matrix; numerical execution is owned by operators."""

    payload: Mapping[str, Tensor]
    encoding: QuantizationScheme
    shape: tuple[int, int]
    partitions: tuple[int, ...] = field(default=())

    def __post_init__(self) -> None:
        expected = payload_headers(self.shape, self.encoding, self.partitions)
        if set(self.payload) != {key for key, _, _ in expected}:
            raise QuantizationError("packed matrix payload does not close its declared encoding")
        if self.partitions and sum(self.partitions) != self.shape[0]:
            raise QuantizationError("Cubic output partitions must sum to N")
        devices = set()
        for key, dtype, shape in expected:
            value = self.payload[key]
            if (not isinstance(value, Tensor) or value.dtype != dtype
                    or tuple(value.shape) != shape or not value.is_contiguous()):
                raise QuantizationError(f"packed matrix payload {key!r} has an invalid physical ABI")
            devices.add(value.device)
        if len(devices) != 1:
            raise QuantizationError("packed matrix payload must share one device")
        object.__setattr__(self, "payload", MappingProxyType(dict(self.payload)))

    @property
    def device(self) -> torch.device:
        return next(iter(self.payload.values())).device

    def to(self, device) -> "QuantizedMatrix":
        target = torch.device(device)
        if self.device == target:
            return self
        return QuantizedMatrix({k: v.to(target) for k, v in self.payload.items()}, self.encoding,
                               self.shape, self.partitions)

    def columns(self, start: int, end: int) -> "QuantizedMatrix":
        """Input-column slice (layout.py:88-104): a slice inside one original
        group keeps that group's metadata; a multi-group slice must align to
        groups (its end may be K); packed bytes must be whole."""
        k = self.shape[1]
        if not 0 <= start < end <= k:
            raise QuantizationError("quantized slice is out of bounds")
        e = self.encoding
        group = e.group_in
        one_group = start // group == (end - 1) // group
        if not one_group and (start % group or (end % group and end != k)):
            raise QuantizationError("input slice must preserve original scale groups")
        if start * e.bits % 8:
            raise QuantizationError("input slice must preserve original packed bytes")
        payload = {}
        for key, tensor in self.payload.items():
            if key.endswith("_global") or key in ("weight_curve_a", "weight_curve_b"):
                payload[key] = tensor
            elif key == "weight_packed":
                payload[key] = tensor[:, start * e.bits // 8:(end * e.bits + 7) // 8].contiguous()
            else:
                payload[key] = tensor[:, start // group:(end + group - 1) // group].contiguous()
        return QuantizedMatrix(payload, e, (self.shape[0], end - start), self.partitions)

    def rows(self, start: int, end: int) -> "QuantizedMatrix":
        """Output-row slice preserving groups and partition globals (layout.py:58-86)."""
        if not 0 <= start < end <= self.shape[0]:
            raise QuantizationError("quantized slice is out of bounds")
        group = self.encoding.group_out
        if start % group or end % group:
            raise QuantizationError("output slice must preserve original scale groups")
        parts, indices, offset = [], [], 0
        for index, count in enumerate(self.partitions or (self.shape[0],)):
            overlap = min(end, offset + count) - max(start, offset)
            if overlap > 0:
                parts.append(overlap)
                indices.append(index)
            offset += count
        payload = {}
        for key, tensor in self.payload.items():
            if key.endswith("_global") or key in ("weight_curve_a", "weight_curve_b"):
                payload[key] = tensor[indices[0]:indices[-1] + 1].contiguous()
            elif key == "weight_packed":
                payload[key] = tensor[start:end].contiguous()
            else:
                payload[key] = tensor[start // group:end // group].contiguous()
        return QuantizedMatrix(payload, self.encoding, (end - start, self.shape[1]), tuple(parts))


def partition_rows(matrix: QuantizedMatrix) -> Tensor:
    """int32 [N]: partition index of every output row."""
    parts = matrix.partitions or (matrix.shape[0],)
    return torch.repeat_interleave(torch.arange(len(parts), dtype=torch.int32),
                                   torch.tensor(parts)).to(matrix.device)


# --------------------------------------------------------------------------- #
# Build-owned encoder (A0)
# --------------------------------------------------------------------------- #
# Candidate curves (a, b); c = 1 - a - b >= 0 keeps every curve monotone on [0, 1].
CURVES = ((1.0, 0.0), (0.75, 0.125), (0.5, 0.25), (0.5, 0.0), (0.375, 0.25), (0.25, 0.375))


def _pack_bitstream(raw: Tensor, bits: int) -> Tensor:
    """[rows, K] raw codes in 0..2^bits-1 -> little-endian bitstream uint8."""
    rows, k = raw.shape
    nbytes = math.ceil(k * bits / 8)
    shifts = torch.arange(bits, device=raw.device, dtype=torch.int32)
    planes = ((raw.to(torch.int32).unsqueeze(-1) >> shifts) & 1).reshape(rows, k * bits)
    planes = torch.nn.functional.pad(planes, (0, nbytes * 8 - k * bits))
    weights = (1 << torch.arange(8, device=raw.device, dtype=torch.int32))
    return (planes.reshape(rows, nbytes, 8) * weights).sum(-1).to(torch.uint8)


def _levels(scale: Tensor, a: Tensor, b: Tensor, bits: int) -> Tensor:
    """[..., D+1] fp32 magnitude levels with the decoder's operation order."""
    d = (1 << (bits - 1)) - 1
    t = (torch.arange(d + 1, dtype=torch.float64, device=scale.device) / d).float()
    a, b, s = a.float().unsqueeze(-1), b.float().unsqueeze(-1), scale.unsqueeze(-1)
    return s * (t * (a + t * (b + t * ((1.0 - a) - b))))


@torch.no_grad()
def quantize_cubic(weight: Tensor, bits: int = 4, group_in: int = 128,
                   row_chunk: int = 4096) -> QuantizedMatrix:
    """Encode an [N, K] float weight as a Cubic fmt0 matrix (group_out = 1).

    Per group of ``group_in`` inputs: scale = max |w|; curve = the candidate of
    CURVES with the least squared error after nearest-level assignment; codes =
    sign(w) * nearest magnitude (the reserved code is never produced).  Works
    on any device; rows are processed in chunks to bound temporary memory.
    """
    if weight.ndim != 2 or not weight.is_floating_point():
        raise QuantizationError("encoder needs a floating [N, K] weight")
    if not 1 <= bits <= 8:
        raise QuantizationError("unsupported Cubic bit width")
    n, k = weight.shape
    groups = math.ceil(k / group_in)
    dev = weight.device
    packed = torch.empty((n, math.ceil(k * bits / 8)), dtype=torch.uint8, device=dev)
    scale = torch.empty((n, groups), dtype=torch.float32, device=dev)
    a_out = torch.empty((n, groups), dtype=torch.float16, device=dev)
    b_out = torch.empty((n, groups), dtype=torch.float16, device=dev)
    curve_a = torch.tensor([c[0] for c in CURVES], dtype=torch.float16, device=dev)
    curve_b = torch.tensor([c[1] for c in CURVES], dtype=torch.float16, device=dev)
    for r0 in range(0, n, row_chunk):
        w = weight[r0:r0 + row_chunk].float()
        rows = w.shape[0]
        wg = torch.nn.functional.pad(w, (0, groups * group_in - k)).reshape(rows, groups, group_in)
        mag = wg.abs()
        s = mag.amax(-1)
        if bits == 1:
            codes = torch.where(wg < 0, -1, 1).to(torch.int32)
            best_a = torch.ones_like(s, dtype=torch.float16)
            best_b = torch.zeros_like(s, dtype=torch.float16)
        else:
            best_err = torch.full_like(s, float("inf"))
            best_m = torch.zeros(wg.shape, dtype=torch.int64, device=dev)
            best_a = torch.zeros_like(s, dtype=torch.float16)
            best_b = torch.zeros_like(s, dtype=torch.float16)
            for ci in range(len(CURVES)):
                a = curve_a[ci].expand_as(s)
                b = curve_b[ci].expand_as(s)
                lv = _levels(s, a, b, bits)                     # [rows, G, D+1]
                mids = 0.5 * (lv[..., 1:] + lv[..., :-1])
                m = torch.searchsorted(mids.contiguous(), mag.contiguous())
                err = ((torch.gather(lv, -1, m) - mag) ** 2).sum(-1)
                better = err < best_err
                best_err = torch.where(better, err, best_err)
                best_m = torch.where(better.unsqueeze(-1), m, best_m)
                best_a = torch.where(better, a, best_a)
                best_b = torch.where(better, b, best_b)
            codes = torch.where(wg < 0, -best_m, best_m).to(torch.int32)
        codes = codes.reshape(rows, groups * group_in)[:, :k]
        raw = codes & ((1 << bits) - 1) if bits > 1 else (codes + 1) // 2
        packed[r0:r0 + rows] = _pack_bitstream(raw, bits)
        scale[r0:r0 + rows] = s
        a_out[r0:r0 + rows] = best_a
        b_out[r0:r0 + rows] = best_b
    encoding = QuantizationScheme(CUBIC_FORMAT, bits, group_in, 1, FMT_F32)
    return QuantizedMatrix({"weight_packed": packed, "weight_scale": scale, "weight_a": a_out,
                            "weight_b": b_out}, encoding, (n, k))
