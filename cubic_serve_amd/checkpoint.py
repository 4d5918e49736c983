"""Cubic checkpoint loader: quantization rules, payload admission, materialization.

Host mirror of the reference's loading path for Cubic checkpoints (paths
under src/cubic_serve/):
  QuantizationConfig, EncodingRule, resolve  models/quantization.py:59-250
  parse_config / parse_group                 quantization/extensions/cubic/checkpoint.py:22-63
  parse_groups                               quantization/common/checkpoint.py:18-38
  payload headers, slices, stacked names     quantization/extensions/cubic/layout.py:22-109
  LogicalWeight, StackedMatrixSlice          models/quantized_checkpoint.py:99-170
  CheckpointWeights.admit / materialize      models/quantized_checkpoint.py:197-560

A checkpoint is a directory with ``config.json`` (``quantization_config``
with ``quant_method: "cubic"``, ``format: "cubic-pack-quantized"``) and
safetensors shards (``model.safetensors`` or an index).  Tensors are read
with ``safetensors.safe_open`` (no code execution), one slice at a time, and
land as ``QuantizedMatrix`` payloads on the requested device; ``prepare``
then repacks them for the gfx950 GEMM (cubic_prepare_weight).
"""
from __future__ import annotations

import hashlib
import json
import re
import struct
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path
from typing import Iterable, Mapping, Sequence

import torch
from torch import Tensor

from .quantization import (
    QuantizationError,
    QuantizationScheme,
    QuantizedMatrix,
    parse_group,
    payload_headers,
)

CUBIC_METHOD = "cubic"
CUBIC_CONFIG_FORMAT = "cubic-pack-quantized"

# safetensors dtype strings <-> torch
DTYPES = {"U8": torch.uint8, "I8": torch.int8, "U16": torch.uint16, "I16": torch.int16,
          "F16": torch.float16, "BF16": torch.bfloat16, "F32": torch.float32, "I32": torch.int32,
          "I64": torch.int64}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}


# --------------------------------------------------------------------------- #
# Rules (models/quantization.py:59-250, cubic/checkpoint.py:58-63)
# --------------------------------------------------------------------------- #
def _strings(value: object) -> tuple[str, ...]:
    if not isinstance(value, (list, tuple)) or any(not isinstance(v, str) or not v for v in value):
        raise QuantizationError("targets and ignore rules must be non-empty strings")
    for entry in value:
        if entry.startswith("re:"):
            try:
                re.compile(entry[3:])
            except re.error as error:
                raise QuantizationError("invalid quantization target expression") from error
    return tuple(value)


@dataclass(frozen=True, slots=True)
class EncodingRule:
    name: str
    targets: tuple[str, ...]
    encoding: QuantizationScheme


def parse_groups(config: Mapping[str, object], parse) -> tuple[EncodingRule, ...]:
    """``config_groups`` -> rules (quantization/common/checkpoint.py:18-38)."""
    groups = config.get("config_groups")
    if not isinstance(groups, Mapping) or not groups:
        raise QuantizationError("quantized checkpoint requires config_groups")
    rules = []
    for name, group in groups.items():
        if not isinstance(name, str) or not isinstance(group, Mapping):
            raise QuantizationError("invalid quantization group")
        targets = _strings(group.get("targets"))
        if not targets:
            raise QuantizationError("encoding rule requires targets")
        weights = group.get("weights")
        if not isinstance(weights, Mapping):
            raise QuantizationError("encoding rule requires weight semantics")
        if group.get("output_activations") is not None:
            raise QuantizationError("output activation quantization is not implemented")
        rules.append(EncodingRule(name, targets, parse(group, weights)))
    return tuple(rules)


def parse_config(config: Mapping[str, object]) -> tuple[tuple[EncodingRule, ...], tuple[str, ...]]:
    """Cubic's checkpoint method (quantization/extensions/cubic/checkpoint.py:58-63)."""
    if config.get("format") != CUBIC_CONFIG_FORMAT:
        raise QuantizationError("Cubic requires its explicit packed format")
    return parse_groups(config, parse_group), _strings(config.get("ignore", []))


@lru_cache(maxsize=4096)
def _pattern(text: str) -> re.Pattern[str]:
    return re.compile(text)


def _ignored(target: str, name: str) -> bool:
    if target.startswith("re:"):
        p = _pattern(target[3:])
        return p.match(name) is not None or p.match("." + name) is not None
    return target == name


_CLASS_TARGETS = {"linear": ("Linear",), "embedding": ("Embedding",),
                  "routed_moe": ("FusedMoE", "RoutedExperts")}


def _match(target: str, name: str, operation: str) -> tuple[int, int, int, int] | None:
    """Precedence key of one target for one module name: exact name, then a
    full regex match (anchored, fewer wildcards, longer), then a class name."""
    if target == name:
        return (3, 0, 0, len(target))
    if target.startswith("re:"):
        pattern = target[3:]
        compiled = _pattern(pattern)
        if compiled.fullmatch(name) is not None or compiled.fullmatch("." + name) is not None:
            return (2, int(pattern.startswith("^")), -pattern.count(".*"), len(pattern))
    if target in _CLASS_TARGETS[operation]:
        return (1, 0, 0, 0)
    return None


@dataclass(frozen=True, slots=True)
class QuantizationConfig:
    """Exporter rules normalized once (models/quantization.py:66-170)."""

    method: str
    rules: tuple[EncodingRule, ...]
    ignored: tuple[str, ...]
    source_scope: str
    digest: str

    @classmethod
    def from_model_config(cls, raw: Mapping[str, object]) -> "QuantizationConfig | None":
        root = raw.get("quantization_config")
        text = raw.get("text_config", {})
        nested = text.get("quantization_config") if isinstance(text, Mapping) else None
        if root is not None and nested is not None and root != nested:
            raise QuantizationError("conflicting root and text quantization declarations")
        config = root if root is not None else nested
        if config is None:
            return None
        if not isinstance(config, Mapping):
            raise QuantizationError("quantization_config must be an object")
        method = config.get("quant_method")
        if not isinstance(method, str):
            raise QuantizationError("checkpoint quantization method must be a string")
        if config.get("sparsity_config") or config.get("transform_config"):
            raise QuantizationError("checkpoint sparsity and input transforms are not implemented")
        if method != CUBIC_METHOD:
            raise QuantizationError(f"unsupported checkpoint quantization method {method!r}")
        rules, ignored = parse_config(config)
        encoded = json.dumps(config, sort_keys=True, separators=(",", ":"), allow_nan=False)
        return cls(method, rules, ignored, "root" if root is not None else "text_config",
                   "b2s256:" + hashlib.blake2s(encoded.encode()).hexdigest())

    def resolve(self, module: str, *, aliases: tuple[str, ...] = (),
                operation: str = "linear") -> QuantizationScheme | None:
        if operation not in _CLASS_TARGETS:
            raise QuantizationError(f"unknown quantized consumer {operation!r}")
        names = (module, *aliases)
        if self.source_scope == "text_config" and module.startswith("model.language_model."):
            names = tuple(n.replace("model.language_model.", "model.") for n in names)
        if any(_ignored(t, n) for t in self.ignored for n in names):
            return None
        matches = [(score, rule.encoding) for rule in self.rules for t in rule.targets for n in names
                   if (score := _match(t, n, operation)) is not None]
        if not matches:
            return None
        best = max(score for score, _ in matches)
        encodings = {enc for score, enc in matches if score == best}
        if len(encodings) != 1:
            raise QuantizationError(f"conflicting encoding rules for {module!r}")
        return encodings.pop()


# --------------------------------------------------------------------------- #
# Layout (quantization/extensions/cubic/layout.py)
# --------------------------------------------------------------------------- #
def payload_header_names(shape: tuple[int, int], encoding: QuantizationScheme,
                         partitions: tuple[int, ...] = ()) -> tuple[tuple[str, str, tuple], ...]:
    """(suffix, safetensors dtype, shape) of every payload tensor (layout.py:22-55)."""
    return tuple((key, DTYPE_NAMES[dtype], tuple(shp))
                 for key, dtype, shp in payload_headers(shape, encoding, partitions))


def slice_index(shape: tuple[int, ...], partitions: tuple[int, ...], encoding: QuantizationScheme,
                key: str, axis: int, start: int, end: int) -> tuple[tuple[slice, ...], tuple[int, ...]]:
    """Payload index of a logical row (axis 0) or column (axis 1) span and the
    partitions it keeps (layout.py:58-104)."""
    full = slice(None)
    if axis == 0:
        group = encoding.group_out
        if start % group or end % group:
            raise QuantizationError("output slice must preserve original scale groups")
        parts, indices, offset = [], [], 0
        for index, count in enumerate(partitions or (shape[0],)):
            overlap = min(end, offset + count) - max(start, offset)
            if overlap > 0:
                parts.append(overlap)
                indices.append(index)
            offset += count
        selected = tuple(parts)
        if key.endswith("_global") or key in ("weight_curve_a", "weight_curve_b"):
            return (slice(indices[0], indices[-1] + 1),), selected
        if key == "weight_packed":
            return (slice(start, end), full), selected
        return (slice(start // group, end // group), full), selected
    group = encoding.group_in
    one_group = start // group == (end - 1) // group
    if not one_group and (start % group or (end % group and end != shape[1])):
        raise QuantizationError("input slice must preserve original scale groups")
    if key.endswith("_global") or key in ("weight_curve_a", "weight_curve_b"):
        return (full,), partitions
    if key == "weight_packed":
        if start * encoding.bits % 8:
            raise QuantizationError("input slice must preserve original packed bytes")
        return (full, slice(start * encoding.bits // 8, (end * encoding.bits + 7) // 8)), partitions
    return (full, slice(start // group, (end + group - 1) // group)), partitions


def stacked_payload_name(source: str, key: str) -> str:
    """Exporter names for original [expert, projection, ...] payloads (layout.py:107-109)."""
    return source + "_" + key.removeprefix("weight_")


# --------------------------------------------------------------------------- #
# Logical weights (models/quantized_checkpoint.py:99-170)
# --------------------------------------------------------------------------- #
@dataclass(frozen=True, slots=True)
class AxisSpan:
    start: int
    stop: int

    def __post_init__(self) -> None:
        if type(self.start) is not int or type(self.stop) is not int or not 0 <= self.start < self.stop:
            raise QuantizationError("axis span must be a nonempty ordered integer range")

    @property
    def size(self) -> int:
        return self.stop - self.start


@dataclass(frozen=True, slots=True)
class StackedMatrixSlice:
    """Rows ``rows`` of expert ``index`` of a stacked [experts, N, K] source."""

    name: str
    shape: tuple[int, int, int]
    index: int
    rows: AxisSpan
    output_partitions: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        if len(self.shape) != 3 or not 0 <= self.index < self.shape[0] or self.rows.stop > self.shape[1]:
            raise QuantizationError("stacked source slice is out of bounds")


@dataclass(frozen=True, slots=True)
class LogicalWeight:
    name: str
    shape: tuple[int, ...]
    dtype: str = "BF16"
    partition: str = "language"
    operation: str = "linear"
    aliases: tuple[str, ...] = ()
    output_partitions: tuple[int, ...] = ()
    stacked_source: StackedMatrixSlice | None = None

    def __post_init__(self) -> None:
        if not self.name or any(type(n) is not int or n <= 0 for n in self.shape):
            raise QuantizationError("logical weight identity and positive shape are required")
        if self.operation not in ("tensor", "linear", "embedding"):
            raise QuantizationError("unknown logical weight consumer")
        if self.operation != "tensor" and len(self.shape) != 2:
            raise QuantizationError("linear and embedding weights require [N,K]")
        if self.output_partitions and sum(self.output_partitions) != self.shape[0]:
            raise QuantizationError("logical output partitions differ from weight rows")
        if self.stacked_source is not None and self.shape != (
                self.stacked_source.rows.size, self.stacked_source.shape[-1]):
            raise QuantizationError("stacked source differs from logical matrix shape")


@dataclass(frozen=True, slots=True)
class EncodedWeight:
    logical: LogicalWeight
    encoding: QuantizationScheme | None
    payload: tuple[tuple[str, str, str], ...]  # (suffix, checkpoint name, shard file)
    stacked_source: StackedMatrixSlice | None = None


@dataclass(frozen=True, slots=True)
class TensorRecord:
    name: str
    dtype: str
    shape: tuple[int, ...]
    shard: str


def read_safetensors_header(path: Path) -> dict:
    """The JSON header of one safetensors file (8-byte little-endian length + JSON)."""
    with open(path, "rb") as f:
        (length,) = struct.unpack("<Q", f.read(8))
        if length > 100 * 1024 * 1024:
            raise QuantizationError(f"implausible safetensors header in {path.name}")
        header = json.loads(f.read(length))
    header.pop("__metadata__", None)
    return header


def inventory(root: Path) -> dict[str, TensorRecord]:
    """Every tensor of the checkpoint by name (index or lone shard)."""
    index = root / "model.safetensors.index.json"
    if index.exists():
        shards = sorted(set(json.loads(index.read_text())["weight_map"].values()))
    else:
        shards = sorted(p.name for p in root.glob("*.safetensors"))
    if not shards:
        raise QuantizationError("checkpoint has no safetensors shards")
    records: dict[str, TensorRecord] = {}
    for shard in shards:
        for name, entry in read_safetensors_header(root / shard).items():
            if name in records:
                raise QuantizationError(f"tensor {name!r} appears in two shards")
            records[name] = TensorRecord(name, entry["dtype"], tuple(entry["shape"]), shard)
    return records


@dataclass(frozen=True)
class CubicCheckpoint:
    """An admitted checkpoint plan (CheckpointWeights, quantized_checkpoint.py:197-560)."""

    root: Path
    quantization: QuantizationConfig | None
    weights: tuple[EncodedWeight, ...]
    records: Mapping[str, TensorRecord] = field(repr=False)

    @classmethod
    def admit(cls, root: str | Path, logical_weights: Iterable[LogicalWeight], *,
              require_quantization: bool = True) -> "CubicCheckpoint":
        root = Path(root)
        raw = json.loads((root / "config.json").read_text())
        config = QuantizationConfig.from_model_config(raw)
        if config is None and require_quantization:
            raise QuantizationError("quantized admission requires declared quantization")
        logical = tuple(sorted(logical_weights, key=lambda w: w.name))
        if not logical or len({w.name for w in logical}) != len(logical):
            raise QuantizationError("logical weight plan must be nonempty and unique")
        records = inventory(root)
        consumed: set[str] = set()
        stacked_rows: dict[str, list[tuple[int, int]]] = {}
        stacked_totals: dict[str, int] = {}
        bindings = []
        for weight in logical:
            module = weight.name.removesuffix(".weight")
            encoding = None
            if config is not None and weight.operation != "tensor":
                encoding = config.resolve(module, aliases=weight.aliases, operation=weight.operation)
            if encoding is None:
                expected = (("weight", weight.dtype, weight.shape),)
                names = [weight.name]
            else:
                expected = payload_header_names(weight.shape, encoding, weight.output_partitions)
                names = [module + "." + suffix for suffix, _, _ in expected]
            source = None
            if not any(n in records for n in names) and weight.stacked_source is not None:
                source = weight.stacked_source
                if encoding is None:
                    expected = (("weight", weight.dtype, source.shape),)
                    names = [source.name]
                else:
                    full = payload_header_names(source.shape[1:], encoding, source.output_partitions)
                    expected = tuple((key, dt, (source.shape[0], *shp)) for key, dt, shp in full)
                    names = [stacked_payload_name(source.name, key) for key, _, _ in expected]
            bound = []
            for (suffix, dtype, shape), name in zip(expected, names):
                record = records.get(name)
                if record is None:
                    raise QuantizationError(f"missing payload {name!r} for {weight.name!r}")
                plain_float = encoding is None and dtype == "BF16" and record.dtype in ("BF16", "F16", "F32")
                if (record.dtype != dtype and not plain_float) or record.shape != tuple(shape):
                    raise QuantizationError(f"payload {name!r}: expected {dtype}{tuple(shape)}, "
                                            f"got {record.dtype}{record.shape}")
                if name in consumed and (source is None or name not in stacked_rows):
                    raise QuantizationError(f"physical payload {name!r} has multiple logical owners")
                consumed.add(name)
                if source is not None:
                    total = source.shape[0] * source.shape[1]
                    if stacked_totals.setdefault(name, total) != total:
                        raise QuantizationError("inconsistent stacked payload logical geometry")
                    start = source.index * source.shape[1] + source.rows.start
                    stacked_rows.setdefault(name, []).append((start, start + source.rows.size))
                bound.append((suffix, name, record.shard))
            bindings.append(EncodedWeight(weight, encoding, tuple(bound), source))
        for name, intervals in stacked_rows.items():
            cursor = 0
            for start, stop in sorted(intervals):
                if start != cursor:
                    raise QuantizationError(f"stacked payload {name!r} has overlapping or missing owners")
                cursor = stop
            if cursor != stacked_totals[name]:
                raise QuantizationError(f"stacked payload {name!r} has unowned rows")
        unknown = sorted(set(records) - consumed)
        if unknown:
            raise QuantizationError(f"checkpoint has {len(unknown)} unowned tensors: {unknown[:8]}")
        return cls(root, config, tuple(bindings), records)

    def weight(self, name: str) -> EncodedWeight:
        for w in self.weights:
            if w.logical.name == name:
                return w
        raise KeyError(name)

    def _read(self, name: str, shard: str, index: tuple) -> Tensor:
        from safetensors import safe_open

        with safe_open(str(self.root / shard), framework="pt", device="cpu") as f:
            return f.get_slice(name)[index].contiguous()

    def materialize(self, weight: EncodedWeight, *, device: torch.device | str = "cpu",
                    compute_dtype: torch.dtype = torch.bfloat16, axis: int = 0,
                    spans: Sequence[AxisSpan] | None = None) -> Tensor | QuantizedMatrix:
        """Read the logical owner spans of one weight from its payloads
        (quantized_checkpoint.py:425-552): a plain tensor in compute_dtype, or
        a QuantizedMatrix whose payload keeps its serialized dtypes."""
        if weight not in self.weights:
            raise QuantizationError("payload binding belongs to another checkpoint plan")
        logical, encoding = weight.logical, weight.encoding
        if type(axis) is not int or not 0 <= axis < len(logical.shape):
            raise QuantizationError("logical slice axis is out of bounds")
        spans = (AxisSpan(0, logical.shape[axis]),) if spans is None else tuple(spans)
        if not spans or any(s.stop > logical.shape[axis] for s in spans):
            raise QuantizationError("logical owner spans are empty or out of bounds")
        if any(a.stop > b.start for a, b in zip(spans, spans[1:])):
            raise QuantizationError("logical owner spans must retain disjoint checkpoint order")
        source = weight.stacked_source
        if encoding is None:
            (_, name, shard), = weight.payload
            parts = []
            for s in spans:
                index = [slice(None)] * len(logical.shape)
                if source is not None:
                    base = source.rows.start if axis == 0 else 0
                    index[axis] = slice(base + s.start, base + s.stop)
                    parts.append(self._read(name, shard, (source.index, *index)))
                else:
                    index[axis] = slice(s.start, s.stop)
                    parts.append(self._read(name, shard, tuple(index)))
            return torch.cat(parts, dim=axis).to(device=device, dtype=compute_dtype)
        if axis == 1 and len(spans) != 1:
            raise QuantizationError("packed input ownership requires one contiguous span")
        if source is None:
            return self._encoded(weight, logical.shape, logical.output_partitions, axis, spans,
                                 device, None)
        # expert `index` of a stacked [experts, N, K] source; logical rows are
        # source.rows of that expert's N
        if axis == 0:
            shifted = tuple(AxisSpan(source.rows.start + sp.start, source.rows.start + sp.stop)
                            for sp in spans)
            return self._encoded(weight, source.shape[1:], source.output_partitions, 0, shifted,
                                 device, source.index)
        rows = self._encoded(weight, source.shape[1:], source.output_partitions, 0, (source.rows,),
                             "cpu", source.index)
        return rows.columns(spans[0].start, spans[0].stop).to(device)

    def _encoded(self, weight: EncodedWeight, shape, partitions, axis: int,
                 spans: Sequence[AxisSpan], device, expert: int | None) -> QuantizedMatrix:
        encoding = weight.encoding
        payload: dict[str, list[Tensor]] = {}
        kept: list[int] = []
        for sp in spans:
            selected: tuple[int, ...] = ()
            for suffix, name, shard in weight.payload:
                index, selected = slice_index(tuple(shape), tuple(partitions), encoding, suffix, axis,
                                              sp.start, sp.stop)
                if expert is not None:
                    index = (expert, *index)
                payload.setdefault(suffix, []).append(self._read(name, shard, index))
            kept.extend(selected)
        merged = {key: (torch.cat(parts, dim=0) if len(parts) > 1 else parts[0]).to(device)
                  for key, parts in payload.items()}
        if axis == 0:
            out_shape, parts = (sum(sp.size for sp in spans), shape[1]), tuple(kept)
        else:
            out_shape, parts = (shape[0], spans[0].size), tuple(partitions)
        if len(parts) == 1:
            parts = ()
        return QuantizedMatrix(merged, encoding, out_shape, parts)


def save_cubic_checkpoint(root: str | Path, matrices: Mapping[str, QuantizedMatrix], *,
                          rules: Mapping[str, Sequence[str]] | None = None,
                          extra: Mapping[str, Tensor] | None = None) -> None:
    """Write a Cubic checkpoint directory (config.json + model.safetensors).

    ``matrices`` maps module names to packed matrices (their payload keys
    become ``{module}.{key}``); all must share one encoding per rule.  By
    default one rule targets every module by exact name.
    """
    from safetensors.torch import save_file

    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    tensors = {f"{module}.{key}": t.detach().cpu().contiguous().clone()
               for module, m in matrices.items() for key, t in m.payload.items()}
    tensors.update({k: v.detach().cpu().contiguous() for k, v in (extra or {}).items()})
    groups = {}
    by_encoding: dict[QuantizationScheme, list[str]] = {}
    for module, m in matrices.items():
        by_encoding.setdefault(m.encoding, []).append(module)
    for i, (enc, modules) in enumerate(by_encoding.items()):
        weights = {"num_bits": enc.bits, "dynamic": False, "symmetric": True,
                   "group_size": enc.group_in if enc.group_out == 1 else [enc.group_out, enc.group_in],
                   "packing": "little-endian-bitstream",
                   "reserved_code": "binary" if enc.bits == 1 else "zero",
                   "metadata_format": enc.metadata}
        weights.update({
            "float32-scale-float16-ab": {"scale_dtype": "torch.float32", "param_dtype": "torch.float16"},
            "int8-scale-int4-ab-global-fp32": {"scale_dtype": "torch.int8", "param_dtype": "packed_int4"},
            "e5m9-scale-curve2-tensor-fp16": {"scale_dtype": "packed_e5m9", "param_dtype": "torch.float16",
                                              "curve_count": 4},
        }[enc.metadata])
        targets = list((rules or {}).get(f"group_{i}", modules))
        groups[f"group_{i}"] = {"targets": targets, "weights": weights}
    config = {"quantization_config": {"quant_method": CUBIC_METHOD, "format": CUBIC_CONFIG_FORMAT,
                                      "config_groups": groups, "ignore": []}}
    (root / "config.json").write_text(json.dumps(config, indent=1))
    save_file(tensors, str(root / "model.safetensors"))


def prepare(matrix: QuantizedMatrix, device: torch.device | str):
    """Repack a loaded matrix for the gfx950 GEMM (cubic_prepare_weight)."""
    from .linear import prepare_matrix

    return prepare_matrix(matrix, torch.device(device))


__all__ = ["AxisSpan", "CubicCheckpoint", "EncodedWeight", "EncodingRule", "LogicalWeight",
           "QuantizationConfig", "StackedMatrixSlice", "inventory", "parse_config", "parse_groups",
           "payload_header_names", "prepare", "read_safetensors_header", "save_cubic_checkpoint",
           "slice_index", "stacked_payload_name"]
