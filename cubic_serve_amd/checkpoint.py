"""Cubic checkpoint loading: quantization rules, payload admission, materialization.

Host side of loading a Cubic checkpoint for the gfx950 kernels.  The rule and
layout *semantics* are the reference's checkpoint format (paths under
src/cubic_serve/); the code is organised around three tables:

  RuleTable      exact names, target expressions and class targets of every
                 ``config_groups`` rule, each with a fixed precedence
                 (models/quantization.py:59-250; quantization/extensions/
                 cubic/checkpoint.py:22-63; quantization/common/checkpoint.py:18-38)
  Manifest       the payload tensors one logical weight needs: checkpoint
                 name, dtype, shape and the stacked-row interval it owns
                 (quantization/extensions/cubic/layout.py:22-109;
                 models/quantized_checkpoint.py:99-170)
  OwnershipLedger  who owns which rows of which physical tensor; admission
                 fails closed on gaps, overlaps and unowned tensors
                 (models/quantized_checkpoint.py:197-420)

A checkpoint is a directory with ``config.json`` (``quantization_config`` with
``quant_method: "cubic"`` and ``format: "cubic-pack-quantized"``) and
safetensors shards (``model.safetensors`` or an index).  Headers are parsed
directly; tensor data is read through ``safetensors.safe_open`` slices (no code
execution), so a shard owner reads only its rows or byte columns.
``prepare`` repacks a loaded matrix for the GEMM (cubic_prepare_weight).
"""
from __future__ import annotations

import hashlib
import json
import re
import struct
from dataclasses import dataclass, field
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

# consumers a rule may name by class, per operation
CLASS_TARGETS = {"linear": frozenset({"Linear"}), "embedding": frozenset({"Embedding"}),
                 "routed_moe": frozenset({"FusedMoE", "RoutedExperts"})}

# precedence tiers (higher wins): exact module name, full target-expression
# match, class name
_EXACT, _EXPRESSION, _CLASS = 3, 2, 1


# --------------------------------------------------------------------------- #
# Rules
# --------------------------------------------------------------------------- #
def _target_list(value: object) -> tuple[str, ...]:
    """Validated target or ignore strings; expressions ("re:...") must compile."""
    if not isinstance(value, (list, tuple)):
        raise QuantizationError("targets and ignore rules must be non-empty strings")
    out = []
    for item in value:
        if not isinstance(item, str) or not item:
            raise QuantizationError("targets and ignore rules must be non-empty strings")
        if item.startswith("re:"):
            try:
                re.compile(item[3:])
            except re.error as error:
                raise QuantizationError("invalid quantization target expression") from error
        out.append(item)
    return tuple(out)


@dataclass(frozen=True, slots=True)
class EncodingRule:
    """One ``config_groups`` entry: its targets and the scheme they receive."""

    name: str
    targets: tuple[str, ...]
    encoding: QuantizationScheme


def parse_groups(config: Mapping[str, object], parse) -> tuple[EncodingRule, ...]:
    """``config_groups`` -> rules, each weight section parsed by ``parse``."""
    groups = config.get("config_groups")
    if not isinstance(groups, Mapping) or not groups:
        raise QuantizationError("quantized checkpoint requires config_groups")
    rules = []
    for name, group in groups.items():
        if not isinstance(name, str) or not isinstance(group, Mapping):
            raise QuantizationError("invalid quantization group")
        targets = _target_list(group.get("targets"))
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
    """The Cubic method's rules and ignore list (cubic/checkpoint.py:58-63)."""
    if config.get("format") != CUBIC_CONFIG_FORMAT:
        raise QuantizationError("Cubic requires its explicit packed format")
    return parse_groups(config, parse_group), _target_list(config.get("ignore", []))


@dataclass(frozen=True)
class _Expression:
    pattern: re.Pattern
    rank: tuple[int, int, int, int]
    encoding: QuantizationScheme

    def hits(self, name: str) -> bool:
        return self.pattern.fullmatch(name) is not None or self.pattern.fullmatch("." + name) is not None


class RuleTable:
    """Every target of every rule, indexed for lookup.

    Precedence of a target for one module name: an exact name beats any
    expression, an expression beats a class name; among expressions an
    anchored one ("^...") beats an unanchored one, then fewer ".*"
    wildcards, then the longer expression.  Several rules at the winning rank
    must agree on the scheme.  Ignore entries are exact names or expressions
    matched at the start of the name (or of "." + name).
    """

    def __init__(self, rules: Sequence[EncodingRule], ignored: Sequence[str]):
        self.exact: dict[str, set[QuantizationScheme]] = {}
        self.expressions: list[_Expression] = []
        self.classes: dict[str, set[QuantizationScheme]] = {}
        for rule in rules:
            for target in rule.targets:
                if target.startswith("re:"):
                    text = target[3:]
                    rank = (_EXPRESSION, int(text.startswith("^")), -text.count(".*"), len(text))
                    self.expressions.append(_Expression(re.compile(text), rank, rule.encoding))
                else:
                    self.exact.setdefault(target, set()).add(rule.encoding)
                    # a plain target may also be a class name
                    self.classes.setdefault(target, set()).add(rule.encoding)
        self.ignore_names = frozenset(t for t in ignored if not t.startswith("re:"))
        self.ignore_patterns = tuple(re.compile(t[3:]) for t in ignored if t.startswith("re:"))

    def ignored(self, name: str) -> bool:
        if name in self.ignore_names:
            return True
        return any(p.match(name) is not None or p.match("." + name) is not None
                   for p in self.ignore_patterns)

    def candidates(self, name: str, operation: str):
        """(rank, scheme) of every target that applies to ``name``."""
        for scheme in self.exact.get(name, ()):
            yield (_EXACT, 0, 0, len(name)), scheme
        for expr in self.expressions:
            if expr.hits(name):
                yield expr.rank, expr.encoding
        for cls in CLASS_TARGETS[operation]:
            for scheme in self.classes.get(cls, ()):
                yield (_CLASS, 0, 0, 0), scheme


@dataclass(frozen=True)
class QuantizationConfig:
    """Exporter rules of one checkpoint, normalised once."""

    method: str
    rules: tuple[EncodingRule, ...]
    ignored: tuple[str, ...]
    source_scope: str            # "root" or "text_config"
    digest: str                  # identity of the declaration: "b2s256:" + BLAKE2s-256 of its canonical JSON
                                 # (models/quantization.py:117-119)
    table: RuleTable = field(repr=False, compare=False, default=None)

    @classmethod
    def from_model_config(cls, raw: Mapping[str, object]) -> "QuantizationConfig | None":
        """The declaration at the root or under ``text_config`` (None if absent)."""
        root = raw.get("quantization_config")
        text = raw.get("text_config")
        nested = text.get("quantization_config") if isinstance(text, Mapping) else None
        if root is not None and nested is not None and root != nested:
            raise QuantizationError("conflicting root and text quantization declarations")
        declared = root if root is not None else nested
        if declared is None:
            return None
        if not isinstance(declared, Mapping):
            raise QuantizationError("quantization_config must be an object")
        method = declared.get("quant_method")
        if not isinstance(method, str):
            raise QuantizationError("checkpoint quantization method must be a string")
        if declared.get("sparsity_config") or declared.get("transform_config"):
            raise QuantizationError("checkpoint sparsity and input transforms are not implemented")
        if method != CUBIC_METHOD:
            raise QuantizationError(f"unsupported checkpoint quantization method {method!r}")
        rules, ignored = parse_config(declared)
        canonical = json.dumps(declared, sort_keys=True, separators=(",", ":"), allow_nan=False)
        return cls(method, rules, ignored, "root" if root is not None else "text_config",
                   "b2s256:" + hashlib.blake2s(canonical.encode()).hexdigest(),
                   RuleTable(rules, ignored))

    def resolve(self, module: str, *, aliases: tuple[str, ...] = (),
                operation: str = "linear") -> QuantizationScheme | None:
        """Scheme of one consumer module (and its aliases), or None when
        ignored or untargeted."""
        if operation not in CLASS_TARGETS:
            raise QuantizationError(f"unknown quantized consumer {operation!r}")
        names = [module, *aliases]
        if self.source_scope == "text_config" and module.startswith("model.language_model."):
            # a text_config declaration names the language model's modules
            # without the multimodal wrapper prefix: when the consumer itself
            # sits under the wrapper, every name (aliases included) drops it;
            # otherwise no name is rewritten (models/quantization.py:131-136)
            names = [n.replace("model.language_model.", "model.") for n in names]
        if any(self.table.ignored(n) for n in names):
            return None
        best, chosen = None, set()
        for name in names:
            for rank, scheme in self.table.candidates(name, operation):
                if best is None or rank > best:
                    best, chosen = rank, {scheme}
                elif rank == best:
                    chosen.add(scheme)
        if best is None:
            return None
        if len(chosen) != 1:
            raise QuantizationError(f"conflicting encoding rules for {module!r}")
        return next(iter(chosen))


# --------------------------------------------------------------------------- #
# Layout
# --------------------------------------------------------------------------- #
def payload_header_names(shape: tuple[int, int], encoding: QuantizationScheme,
                         partitions: tuple[int, ...] = ()) -> tuple[tuple[str, str, tuple], ...]:
    """(suffix, safetensors dtype, shape) of every payload tensor of one matrix."""
    return tuple((key, DTYPE_NAMES[dtype], tuple(shp))
                 for key, dtype, shp in payload_headers(shape, encoding, partitions))


def _per_partition(key: str) -> bool:
    """Payload tensors indexed by output partition rather than by row group."""
    return key.endswith("_global") or key in ("weight_curve_a", "weight_curve_b")


def slice_index(shape: tuple[int, ...], partitions: tuple[int, ...], encoding: QuantizationScheme,
                key: str, axis: int, start: int, end: int) -> tuple[tuple[slice, ...], tuple[int, ...]]:
    """Index into payload tensor ``key`` for logical rows (axis 0) or input
    columns (axis 1) [start, end), and the output partitions the span keeps.

    Rows must keep whole output groups; per-partition tensors keep the
    partitions the span touches.  Columns must keep whole input groups (a
    span inside one group keeps that group) and whole packed bytes.
    """
    everything = slice(None)
    if axis == 0:
        go = encoding.group_out
        if start % go or end % go:
            raise QuantizationError("output slice must preserve original scale groups")
        bounds, kept, touched = 0, [], []
        for index, rows in enumerate(partitions or (shape[0],)):
            lo, hi = max(start, bounds), min(end, bounds + rows)
            if hi > lo:
                kept.append(hi - lo)
                touched.append(index)
            bounds += rows
        if _per_partition(key):
            return (slice(touched[0], touched[-1] + 1),), tuple(kept)
        rows = slice(start, end) if key == "weight_packed" else slice(start // go, end // go)
        return (rows, everything), tuple(kept)
    gi = encoding.group_in
    first_group, last_group = start // gi, (end - 1) // gi
    if first_group != last_group and (start % gi or (end % gi and end != shape[1])):
        raise QuantizationError("input slice must preserve original scale groups")
    if _per_partition(key):
        return (everything,), partitions
    if key == "weight_packed":
        bit0 = start * encoding.bits
        if bit0 % 8:
            raise QuantizationError("input slice must preserve original packed bytes")
        return (everything, slice(bit0 // 8, -(-end * encoding.bits // 8))), partitions
    return (everything, slice(first_group, last_group + 1)), partitions


def stacked_payload_name(source: str, key: str) -> str:
    """Exporter name of a payload of a stacked [expert, N, K] source."""
    return f"{source}_{key[len('weight_'):] if key.startswith('weight_') else key}"


# --------------------------------------------------------------------------- #
# Logical weights (what the model asks for)
# --------------------------------------------------------------------------- #
@dataclass(frozen=True, slots=True)
class AxisSpan:
    """Half-open [start, stop) range of one axis."""

    start: int
    stop: int

    def __post_init__(self) -> None:
        ok = type(self.start) is int and type(self.stop) is int and 0 <= self.start < self.stop
        if not ok:
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
        inside = len(self.shape) == 3 and 0 <= self.index < self.shape[0] and self.rows.stop <= self.shape[1]
        if not inside:
            raise QuantizationError("stacked source slice is out of bounds")


_OPERATIONS = ("tensor", "linear", "embedding")


@dataclass(frozen=True, slots=True)
class LogicalWeight:
    """One weight the model consumes: name, logical shape and consumer."""

    name: str
    shape: tuple[int, ...]
    dtype: str = "BF16"
    partition: str = "language"
    operation: str = "linear"
    aliases: tuple[str, ...] = ()
    output_partitions: tuple[int, ...] = ()
    stacked_source: StackedMatrixSlice | None = None

    def __post_init__(self) -> None:
        if not self.name or not self.shape or any(type(d) is not int or d <= 0 for d in self.shape):
            raise QuantizationError("logical weight identity and positive shape are required")
        if self.operation not in _OPERATIONS:
            raise QuantizationError("unknown logical weight consumer")
        if self.operation != "tensor" and len(self.shape) != 2:
            raise QuantizationError("linear and embedding weights require [N,K]")
        if self.output_partitions and sum(self.output_partitions) != self.shape[0]:
            raise QuantizationError("logical output partitions differ from weight rows")
        src = self.stacked_source
        if src is not None and tuple(self.shape) != (src.rows.size, src.shape[-1]):
            raise QuantizationError("stacked source differs from logical matrix shape")


@dataclass(frozen=True, slots=True)
class EncodedWeight:
    """A logical weight bound to its payload tensors: (suffix, tensor name, shard)."""

    logical: LogicalWeight
    encoding: QuantizationScheme | None
    payload: tuple[tuple[str, str, str], ...]
    stacked_source: StackedMatrixSlice | None = None


@dataclass(frozen=True, slots=True)
class TensorRecord:
    name: str
    dtype: str
    shape: tuple[int, ...]
    shard: str


def read_safetensors_header(path: Path) -> dict:
    """Tensor table of one safetensors file: an 8-byte little-endian length,
    then that many bytes of JSON (``__metadata__`` dropped)."""
    with open(path, "rb") as handle:
        size = struct.unpack("<Q", handle.read(8))[0]
        if size > 100 << 20:
            raise QuantizationError(f"implausible safetensors header in {path.name}")
        table = json.loads(handle.read(size))
    table.pop("__metadata__", None)
    return table


def inventory(root: Path) -> dict[str, TensorRecord]:
    """Every tensor of the checkpoint by name, across its shards."""
    index_file = root / "model.safetensors.index.json"
    if index_file.exists():
        shards = sorted(set(json.loads(index_file.read_text())["weight_map"].values()))
    else:
        shards = sorted(p.name for p in root.glob("*.safetensors"))
    if not shards:
        raise QuantizationError("checkpoint has no safetensors shards")
    found: dict[str, TensorRecord] = {}
    for shard in shards:
        for name, entry in read_safetensors_header(root / shard).items():
            if name in found:
                raise QuantizationError(f"tensor {name!r} appears in two shards")
            found[name] = TensorRecord(name, entry["dtype"], tuple(entry["shape"]), shard)
    return found


# --------------------------------------------------------------------------- #
# Admission
# --------------------------------------------------------------------------- #
@dataclass(frozen=True)
class _Need:
    """One payload tensor a logical weight needs."""

    suffix: str
    tensor: str
    dtype: str
    shape: tuple[int, ...]
    rows: tuple[int, int] | None  # owned interval of a stacked tensor's flattened rows


def _manifest(weight: LogicalWeight, encoding: QuantizationScheme | None,
              records: Mapping[str, TensorRecord]) -> tuple[list[_Need], StackedMatrixSlice | None]:
    """The tensors a weight binds: its own payload when present, else the
    stacked source it is a slice of."""
    module = weight.name.removesuffix(".weight")
    if encoding is None:
        own = [_Need("weight", weight.name, weight.dtype, tuple(weight.shape), None)]
    else:
        own = [_Need(suffix, f"{module}.{suffix}", dt, shp, None)
               for suffix, dt, shp in payload_header_names(tuple(weight.shape), encoding,
                                                           weight.output_partitions)]
    src = weight.stacked_source
    if src is None or any(n.tensor in records for n in own):
        return own, None
    start = src.index * src.shape[1] + src.rows.start
    owned = (start, start + src.rows.size)
    if encoding is None:
        return [_Need("weight", src.name, weight.dtype, tuple(src.shape), owned)], src
    headers = payload_header_names(tuple(src.shape[1:]), encoding, src.output_partitions)
    return [_Need(suffix, stacked_payload_name(src.name, suffix), dt, (src.shape[0], *shp), owned)
            for suffix, dt, shp in headers], src


class OwnershipLedger:
    """Which logical weight owns which part of every physical tensor."""

    def __init__(self):
        self.whole: set[str] = set()
        self.intervals: dict[str, list[tuple[int, int]]] = {}
        self.extent: dict[str, int] = {}

    def claim(self, need: _Need, src: StackedMatrixSlice | None) -> None:
        if need.rows is None:
            if need.tensor in self.whole or need.tensor in self.intervals:
                raise QuantizationError(f"physical payload {need.tensor!r} has multiple logical owners")
            self.whole.add(need.tensor)
            return
        if need.tensor in self.whole:
            raise QuantizationError(f"physical payload {need.tensor!r} has multiple logical owners")
        extent = src.shape[0] * src.shape[1]
        if self.extent.setdefault(need.tensor, extent) != extent:
            raise QuantizationError("inconsistent stacked payload logical geometry")
        self.intervals.setdefault(need.tensor, []).append(need.rows)

    def verify(self, records: Mapping[str, TensorRecord]) -> None:
        for tensor, spans in self.intervals.items():
            reached = 0
            for lo, hi in sorted(spans):
                if lo != reached:
                    raise QuantizationError(f"stacked payload {tensor!r} has overlapping or missing owners")
                reached = hi
            if reached != self.extent[tensor]:
                raise QuantizationError(f"stacked payload {tensor!r} has unowned rows")
        stray = sorted(set(records) - self.whole - set(self.intervals))
        if stray:
            raise QuantizationError(f"checkpoint has {len(stray)} unowned tensors: {stray[:8]}")


def _compatible(need: _Need, record: TensorRecord, encoded: bool) -> bool:
    same_dtype = record.dtype == need.dtype
    # an unencoded bf16 weight may be stored in any float type
    if not same_dtype and not encoded and need.dtype == "BF16":
        same_dtype = record.dtype in ("BF16", "F16", "F32")
    return same_dtype and tuple(record.shape) == tuple(need.shape)


@dataclass(frozen=True)
class CubicCheckpoint:
    """An admitted checkpoint: every logical weight bound to its payload."""

    root: Path
    quantization: QuantizationConfig | None
    weights: tuple[EncodedWeight, ...]
    records: Mapping[str, TensorRecord] = field(repr=False)

    @classmethod
    def admit(cls, root: str | Path, logical_weights: Iterable[LogicalWeight], *,
              require_quantization: bool = True) -> "CubicCheckpoint":
        """Bind every logical weight to checkpoint tensors, fail closed on any
        missing, mistyped, doubly owned or unowned tensor."""
        root = Path(root)
        config = QuantizationConfig.from_model_config(json.loads((root / "config.json").read_text()))
        if config is None and require_quantization:
            raise QuantizationError("quantized admission requires declared quantization")
        plan = tuple(sorted(logical_weights, key=lambda w: w.name))
        if not plan or len({w.name for w in plan}) != len(plan):
            raise QuantizationError("logical weight plan must be nonempty and unique")
        records = inventory(root)
        ledger = OwnershipLedger()
        bound = []
        for weight in plan:
            encoding = None
            if config is not None and weight.operation != "tensor":
                encoding = config.resolve(weight.name.removesuffix(".weight"), aliases=weight.aliases,
                                          operation=weight.operation)
            needs, src = _manifest(weight, encoding, records)
            payload = []
            for need in needs:
                record = records.get(need.tensor)
                if record is None:
                    raise QuantizationError(f"missing payload {need.tensor!r} for {weight.name!r}")
                if not _compatible(need, record, encoding is not None):
                    raise QuantizationError(f"payload {need.tensor!r}: expected {need.dtype}{need.shape}, "
                                            f"got {record.dtype}{record.shape}")
                ledger.claim(need, src)
                payload.append((need.suffix, need.tensor, record.shard))
            bound.append(EncodedWeight(weight, encoding, tuple(payload), src))
        ledger.verify(records)
        return cls(root, config, tuple(bound), records)

    def weight(self, name: str) -> EncodedWeight:
        found = [w for w in self.weights if w.logical.name == name]
        if not found:
            raise KeyError(name)
        return found[0]

    # -- reading ------------------------------------------------------------
    def _read(self, tensor: str, shard: str, index: tuple) -> Tensor:
        from safetensors import safe_open

        with safe_open(str(self.root / shard), framework="pt", device="cpu") as handle:
            return handle.get_slice(tensor)[index].contiguous()

    def materialize(self, weight: EncodedWeight, *, device: torch.device | str = "cpu",
                    compute_dtype: torch.dtype = torch.bfloat16, axis: int = 0,
                    spans: Sequence[AxisSpan] | None = None) -> Tensor | QuantizedMatrix:
        """The owner spans of one weight: a plain tensor in ``compute_dtype``,
        or a QuantizedMatrix whose payload keeps its stored dtypes.  Row spans
        may be several (in checkpoint order); an input-column span is one."""
        if weight not in self.weights:
            raise QuantizationError("payload binding belongs to another checkpoint plan")
        logical = weight.logical
        if type(axis) is not int or not 0 <= axis < len(logical.shape):
            raise QuantizationError("logical slice axis is out of bounds")
        spans = tuple(spans) if spans is not None else (AxisSpan(0, logical.shape[axis]),)
        if not spans or any(s.stop > logical.shape[axis] for s in spans):
            raise QuantizationError("logical owner spans are empty or out of bounds")
        if any(prev.stop > nxt.start for prev, nxt in zip(spans, spans[1:])):
            raise QuantizationError("logical owner spans must retain disjoint checkpoint order")
        src = weight.stacked_source
        if weight.encoding is None:
            return self._plain(weight, axis, spans).to(device=device, dtype=compute_dtype)
        if axis == 1 and len(spans) != 1:
            raise QuantizationError("packed input ownership requires one contiguous span")
        if src is None:
            return self._packed(weight, tuple(logical.shape), logical.output_partitions, axis, spans,
                                None).to(device)
        if axis == 0:
            # expert rows are offset by the slice's first row of the source
            moved = tuple(AxisSpan(src.rows.start + s.start, src.rows.start + s.stop) for s in spans)
            return self._packed(weight, tuple(src.shape[1:]), src.output_partitions, 0, moved,
                                src.index).to(device)
        rows = self._packed(weight, tuple(src.shape[1:]), src.output_partitions, 0, (src.rows,), src.index)
        return rows.columns(spans[0].start, spans[0].stop).to(device)

    def _plain(self, weight: EncodedWeight, axis: int, spans: Sequence[AxisSpan]) -> Tensor:
        (_, tensor, shard), = weight.payload
        src = weight.stacked_source
        offset = src.rows.start if (src is not None and axis == 0) else 0
        pieces = []
        for s in spans:
            index = [slice(None)] * len(weight.logical.shape)
            index[axis] = slice(offset + s.start, offset + s.stop)
            prefix = (src.index,) if src is not None else ()
            pieces.append(self._read(tensor, shard, (*prefix, *index)))
        return torch.cat(pieces, dim=axis)

    def _packed(self, weight: EncodedWeight, shape: tuple[int, ...], partitions: tuple[int, ...],
                axis: int, spans: Sequence[AxisSpan], expert: int | None) -> QuantizedMatrix:
        encoding = weight.encoding
        pieces: dict[str, list[Tensor]] = {suffix: [] for suffix, _, _ in weight.payload}
        kept: list[int] = []
        for s in spans:
            span_parts: tuple[int, ...] = ()
            for suffix, tensor, shard in weight.payload:
                index, span_parts = slice_index(shape, tuple(partitions), encoding, suffix, axis,
                                                s.start, s.stop)
                if expert is not None:
                    index = (expert, *index)
                pieces[suffix].append(self._read(tensor, shard, index))
            kept.extend(span_parts)
        payload = {suffix: torch.cat(parts) if len(parts) > 1 else parts[0]
                   for suffix, parts in pieces.items()}
        if axis == 0:
            out_shape, out_parts = (sum(s.size for s in spans), shape[1]), tuple(kept)
        else:
            out_shape, out_parts = (shape[0], spans[0].size), tuple(partitions)
        return QuantizedMatrix(payload, encoding, out_shape, out_parts if len(out_parts) > 1 else ())


# --------------------------------------------------------------------------- #
# Writing (fixtures and benchmarks)
# --------------------------------------------------------------------------- #
_METADATA_DECLARATION = {
    "float32-scale-float16-ab": {"scale_dtype": "torch.float32", "param_dtype": "torch.float16"},
    "int8-scale-int4-ab-global-fp32": {"scale_dtype": "torch.int8", "param_dtype": "packed_int4"},
    "e5m9-scale-curve2-tensor-fp16": {"scale_dtype": "packed_e5m9", "param_dtype": "torch.float16",
                                      "curve_count": 4},
}


def save_cubic_checkpoint(root: str | Path, matrices: Mapping[str, QuantizedMatrix], *,
                          rules: Mapping[str, Sequence[str]] | None = None,
                          extra: Mapping[str, Tensor] | None = None) -> None:
    """Write a Cubic checkpoint directory (config.json + model.safetensors).

    ``matrices`` maps module names to packed matrices (payload keys become
    ``{module}.{key}``).  One rule per distinct encoding targets its modules
    by exact name unless ``rules`` gives ``group_<i>`` targets.
    """
    from safetensors.torch import save_file

    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    tensors = {f"{module}.{key}": t.detach().cpu().contiguous().clone()
               for module, m in matrices.items() for key, t in m.payload.items()}
    tensors.update({k: v.detach().cpu().contiguous() for k, v in (extra or {}).items()})
    modules_by_scheme: dict[QuantizationScheme, list[str]] = {}
    for module, m in matrices.items():
        modules_by_scheme.setdefault(m.encoding, []).append(module)
    groups = {}
    for i, (enc, modules) in enumerate(modules_by_scheme.items()):
        group_size = enc.group_in if enc.group_out == 1 else [enc.group_out, enc.group_in]
        weights = {"num_bits": enc.bits, "dynamic": False, "symmetric": True, "group_size": group_size,
                   "packing": "little-endian-bitstream",
                   "reserved_code": "binary" if enc.bits == 1 else "zero",
                   "metadata_format": enc.metadata, **_METADATA_DECLARATION[enc.metadata]}
        groups[f"group_{i}"] = {"targets": list((rules or {}).get(f"group_{i}", modules)), "weights": weights}
    declaration = {"quant_method": CUBIC_METHOD, "format": CUBIC_CONFIG_FORMAT,
                   "config_groups": groups, "ignore": []}
    (root / "config.json").write_text(json.dumps({"quantization_config": declaration}, indent=1))
    save_file(tensors, str(root / "model.safetensors"))


def prepare(matrix: QuantizedMatrix, device: torch.device | str, dtype: torch.dtype = torch.bfloat16):
    """Repack a loaded matrix for the gfx950 GEMM with `dtype` activations
    (cubic_prepare_weight)."""
    from .linear import prepare_matrix

    return prepare_matrix(matrix, torch.device(device), dtype)


__all__ = ["AxisSpan", "CubicCheckpoint", "EncodedWeight", "EncodingRule", "LogicalWeight",
           "OwnershipLedger", "QuantizationConfig", "RuleTable", "StackedMatrixSlice", "inventory",
           "parse_config", "parse_groups", "payload_header_names", "prepare",
           "read_safetensors_header", "save_cubic_checkpoint", "slice_index", "stacked_payload_name"]
