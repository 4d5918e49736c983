"""CPU: the Cubic checkpoint loader (config rules, admission, materialization).

Method of the reference's tests (tests/models/test_quantization.py,
tests/models/test_quantized_checkpoint.py): configs that must parse or fail
closed, rule precedence, save -> admit -> materialize round trips for every
metadata format with output groups and partitions, TP row / column shards
whose decoded values equal the slice of the whole (decode by the CPU
oracle), single-group column sub-shards (:671-678), misaligned slices
(:680-687), stacked expert payloads (:376-420), unowned and missing
payloads.
"""
from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch

from cubic_serve_amd import checkpoint as ck, quantization as qz

FMTS = (qz.FMT_F32, qz.FMT_I8, qz.FMT_CURVE2)


def cubic_group(bits=4, group=128, metadata=qz.FMT_F32, **over):
    weights = {"num_bits": bits, "group_size": group, "dynamic": False, "symmetric": True,
               "packing": "little-endian-bitstream", "reserved_code": "binary" if bits == 1 else "zero",
               "metadata_format": metadata,
               **{qz.FMT_F32: {"scale_dtype": "torch.float32", "param_dtype": "torch.float16"},
                  qz.FMT_I8: {"scale_dtype": "torch.int8", "param_dtype": "packed_int4"},
                  qz.FMT_CURVE2: {"scale_dtype": "packed_e5m9", "param_dtype": "torch.float16",
                                  "curve_count": 4}}[metadata]}
    weights.update(over)
    return weights


def config(groups, ignore=()):
    return {"quantization_config": {"quant_method": "cubic", "format": "cubic-pack-quantized",
                                    "config_groups": groups, "ignore": list(ignore)}}


def test_config_parses_and_fails_closed():
    cfg = ck.QuantizationConfig.from_model_config(
        config({"g": {"targets": ["re:.*proj$"], "weights": cubic_group(3, [2, 64], qz.FMT_CURVE2)}}))
    enc = cfg.rules[0].encoding
    assert (enc.bits, enc.group_in, enc.group_out, enc.metadata) == (3, 64, 2, qz.FMT_CURVE2)
    assert ck.QuantizationConfig.from_model_config({"model_type": "x"}) is None
    bad_weights = [dict(dynamic=True), dict(symmetric=False), dict(packing="big-endian"),
                   dict(reserved_code="binary"), dict(scale_dtype="torch.float16"),
                   dict(group_size=0), dict(group_size=128.0), dict(num_bits="4"),
                   dict(metadata_format="other")]
    for change in bad_weights:
        with pytest.raises(qz.QuantizationError):
            ck.QuantizationConfig.from_model_config(
                config({"g": {"targets": ["lm_head"], "weights": cubic_group(**change)}}))
    with pytest.raises(qz.QuantizationError):
        ck.QuantizationConfig.from_model_config(config({"g": {"targets": ["x"], "weights": {
            **cubic_group(metadata=qz.FMT_CURVE2), "curve_count": 3}}}))
    with pytest.raises(qz.QuantizationError):  # activation transforms
        ck.QuantizationConfig.from_model_config(config({"g": {
            "targets": ["x"], "weights": cubic_group(), "input_activations": {"num_bits": 8}}}))
    raw = config({"g": {"targets": ["x"], "weights": cubic_group()}})
    raw["quantization_config"]["format"] = "pack-quantized"
    with pytest.raises(qz.QuantizationError, match="explicit packed format"):
        ck.QuantizationConfig.from_model_config(raw)
    raw = config({"g": {"targets": ["x"], "weights": cubic_group()}})
    raw["quantization_config"]["quant_method"] = "awq"
    with pytest.raises(qz.QuantizationError, match="unsupported"):
        ck.QuantizationConfig.from_model_config(raw)
    with pytest.raises(qz.QuantizationError, match="conflicting root"):
        ck.QuantizationConfig.from_model_config({**raw, "text_config": {"quantization_config": {}}})
    with pytest.raises(qz.QuantizationError, match="target expression"):
        ck.QuantizationConfig.from_model_config(config({"g": {"targets": ["re:("], "weights": cubic_group()}}))


def test_rule_precedence_ignore_and_scope():
    w4, w3, w2 = cubic_group(4), cubic_group(3), cubic_group(2)
    cfg = ck.QuantizationConfig.from_model_config(config({
        "cls": {"targets": ["Linear"], "weights": w2},
        "wide": {"targets": ["re:.*proj$"], "weights": w3},
        "anchored": {"targets": ["re:^model[.]layers[.]0[.].*proj$"], "weights": w4},
        "exact": {"targets": ["lm_head"], "weights": cubic_group(8)},
    }, ignore=["re:^model[.]visual[.]"]))
    assert cfg.resolve("lm_head").bits == 8
    assert cfg.resolve("model.layers.0.mlp.up_proj").bits == 4   # anchored regex beats unanchored
    assert cfg.resolve("model.layers.5.mlp.up_proj").bits == 3
    assert cfg.resolve("model.layers.5.mlp.router").bits == 2     # class-name rule
    assert cfg.resolve("model.embed_tokens", operation="embedding") is None
    assert cfg.resolve("model.visual.proj") is None               # ignored
    assert cfg.resolve("x", aliases=("lm_head",)).bits == 8       # aliases take part
    with pytest.raises(qz.QuantizationError):
        cfg.resolve("x", operation="conv")
    clash = ck.QuantizationConfig.from_model_config(config({
        "a": {"targets": ["lm_head"], "weights": w4}, "b": {"targets": ["lm_head"], "weights": w3}}))
    with pytest.raises(qz.QuantizationError, match="conflicting encoding rules"):
        clash.resolve("lm_head")
    nested = ck.QuantizationConfig.from_model_config(
        {"text_config": config({"g": {"targets": ["model.embed_tokens"], "weights": w4}})})
    assert nested.source_scope == "text_config"
    assert nested.resolve("model.language_model.embed_tokens", operation="embedding").bits == 4


def random_matrix(n, k, bits, group_in, group_out, fmt, seed, partitions=()):
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (n, math.ceil(k * bits / 8)), generator=g, dtype=torch.int32).to(torch.uint8)
    groups = (n // group_out, math.ceil(k / group_in))
    parts = partitions or (n,)
    if fmt == qz.FMT_F32:
        payload = {"weight_packed": packed, "weight_scale": torch.rand(groups, generator=g) * 0.05,
                   "weight_a": (torch.rand(groups, generator=g) * 1.5 - 0.25).half(),
                   "weight_b": (torch.rand(groups, generator=g) - 0.5).half()}
    elif fmt == qz.FMT_I8:
        payload = {"weight_packed": packed,
                   "weight_scale": torch.randint(1, 100, groups, generator=g, dtype=torch.int32).to(torch.int8),
                   "weight_ab": torch.randint(0, 256, groups, generator=g, dtype=torch.int32).to(torch.uint8),
                   "weight_scale_global": torch.rand(len(parts), generator=g) * 1e-3 + 1e-4,
                   "weight_a_global": torch.rand(len(parts), generator=g) * 0.1,
                   "weight_b_global": torch.rand(len(parts), generator=g) * 0.1}
    else:
        md = (torch.randint(0, 0x3C00, groups, generator=g, dtype=torch.int32)
              | (torch.randint(0, 4, groups, generator=g, dtype=torch.int32) << 14))
        payload = {"weight_packed": packed, "weight_metadata": md.to(torch.uint16),
                   "weight_curve_a": (torch.rand((len(parts), 4), generator=g) * 1.5).half(),
                   "weight_curve_b": (torch.rand((len(parts), 4), generator=g) - 0.5).half()}
    enc = qz.QuantizationScheme(qz.CUBIC_FORMAT, bits, group_in, group_out, fmt)
    return qz.QuantizedMatrix(payload, enc, (n, k), tuple(partitions))


def decoded(oracle, m: qz.QuantizedMatrix) -> np.ndarray:
    e = m.encoding
    return oracle.decode_cubic({k: v.cpu().numpy() for k, v in m.payload.items()}, e.bits, e.metadata,
                               m.shape, e.group_in, e.group_out, m.partitions)


def same_payload(a: qz.QuantizedMatrix, b: qz.QuantizedMatrix) -> bool:
    return set(a.payload) == set(b.payload) and all(
        torch.equal(a.payload[k].view(torch.uint8) if a.payload[k].dtype == torch.uint16 else a.payload[k],
                    b.payload[k].view(torch.uint8) if b.payload[k].dtype == torch.uint16 else b.payload[k])
        for k in a.payload)


MATRICES = [(fmt, bits) for fmt in FMTS for bits in (1, 3, 4, 8)]


@pytest.mark.parametrize("fmt,bits", MATRICES)
def test_round_trip_and_shards_preserve_decoded_values(oracle, tmp_path, fmt, bits):
    m = random_matrix(16, 259, bits, 32, 2, fmt, seed=bits, partitions=(8, 8))
    ck.save_cubic_checkpoint(tmp_path, {"model.layers.0.self_attn.qkv_proj": m})
    logical = [ck.LogicalWeight("model.layers.0.self_attn.qkv_proj.weight", (16, 259),
                                output_partitions=(8, 8))]
    plan = ck.CubicCheckpoint.admit(tmp_path, logical)
    w = plan.weights[0]
    whole = plan.materialize(w)
    assert whole.encoding == m.encoding and whole.partitions == m.partitions and same_payload(whole, m)
    full = decoded(oracle, m)
    assert np.array_equal(decoded(oracle, whole), full)
    # output (TP row) shards, incl. one per partition and two disjoint spans
    for spans in ((ck.AxisSpan(0, 8),), (ck.AxisSpan(8, 16),), (ck.AxisSpan(4, 12),),
                  (ck.AxisSpan(0, 4), ck.AxisSpan(10, 16))):
        part = plan.materialize(w, spans=spans)
        rows = np.concatenate([full[s.start:s.stop] for s in spans])
        assert np.array_equal(decoded(oracle, part), rows), spans
    # input (TP column) shards: group aligned, and single-group sub-shards
    for start, stop in ((0, 128), (128, 259), (0, 16), (8, 24), (40, 56), (256, 259)):
        if start * bits % 8:
            continue
        part = plan.materialize(w, axis=1, spans=(ck.AxisSpan(start, stop),))
        assert np.array_equal(decoded(oracle, part), full[:, start:stop]), (start, stop)
        assert np.array_equal(decoded(oracle, m.columns(start, stop)), full[:, start:stop])
    with pytest.raises(qz.QuantizationError, match="original scale groups"):
        plan.materialize(w, axis=1, spans=(ck.AxisSpan(8, 72),))
    with pytest.raises(qz.QuantizationError, match="original scale groups"):
        m.columns(1, 129)
    with pytest.raises(qz.QuantizationError, match="output slice"):
        plan.materialize(w, spans=(ck.AxisSpan(1, 9),))


@pytest.mark.parametrize("fmt", FMTS)
def test_stacked_expert_payloads(oracle, tmp_path, fmt):
    m = random_matrix(16, 259, 4, 32, 2, fmt, seed=7, partitions=(8, 8))
    other = random_matrix(16, 259, 4, 32, 2, fmt, seed=8, partitions=(8, 8))
    physical = {"experts.gate_up_" + key.removeprefix("weight_"): torch.stack((m.payload[key], other.payload[key]))
                for key in m.payload}
    from safetensors.torch import save_file

    (tmp_path / "config.json").write_text(json.dumps(
        config({"g": {"targets": ["re:^experts[.].*"], "weights": cubic_group(4, [2, 32], fmt)}})))
    save_file(physical, str(tmp_path / "model.safetensors"))
    logical = [ck.LogicalWeight(f"experts.{expert}.{part}.weight", (8, 259),
                                stacked_source=ck.StackedMatrixSlice("experts.gate_up", (2, 16, 259), expert,
                                                                     ck.AxisSpan(start, start + 8), (8, 8)))
               for expert in range(2) for part, start in (("gate", 0), ("up", 8))]
    plan = ck.CubicCheckpoint.admit(tmp_path, logical)
    with pytest.raises(qz.QuantizationError, match="unowned|missing owners"):
        ck.CubicCheckpoint.admit(tmp_path, logical[:-1])
    for w in plan.weights:
        view = w.stacked_source
        source = (m, other)[view.index]
        got = plan.materialize(w)
        assert same_payload(got, source.rows(view.rows.start, view.rows.stop)), w.logical.name
        cols = plan.materialize(w, axis=1, spans=(ck.AxisSpan(128, 259),))
        want = decoded(oracle, source)[view.rows.start:view.rows.stop, 128:259]
        assert np.array_equal(decoded(oracle, cols), want)


def test_admission_errors(tmp_path):
    m = random_matrix(16, 64, 4, 32, 1, qz.FMT_F32, seed=1)
    ck.save_cubic_checkpoint(tmp_path, {"a.proj": m}, extra={"norm.weight": torch.ones(64)})
    w = ck.LogicalWeight("a.proj.weight", (16, 64))
    with pytest.raises(qz.QuantizationError, match="unowned tensors"):
        ck.CubicCheckpoint.admit(tmp_path, [w])
    plan = ck.CubicCheckpoint.admit(tmp_path, [w, ck.LogicalWeight("norm.weight", (64,), "F32",
                                                                   operation="tensor")])
    norm = plan.materialize(plan.weight("norm.weight"), compute_dtype=torch.float16)
    assert norm.dtype == torch.float16 and torch.equal(norm, torch.ones(64, dtype=torch.float16))
    with pytest.raises(qz.QuantizationError, match="expected"):
        ck.CubicCheckpoint.admit(tmp_path, [ck.LogicalWeight("a.proj.weight", (16, 96)),
                                            ck.LogicalWeight("norm.weight", (64,), "F32", operation="tensor")])
    with pytest.raises(qz.QuantizationError, match="missing payload"):
        ck.CubicCheckpoint.admit(tmp_path, [w, ck.LogicalWeight("b.proj.weight", (16, 64)),
                                            ck.LogicalWeight("norm.weight", (64,), "F32", operation="tensor")])
    with pytest.raises(qz.QuantizationError, match="nonempty and unique"):
        ck.CubicCheckpoint.admit(tmp_path, [w, w])
    header = ck.read_safetensors_header(tmp_path / "model.safetensors")
    assert header["a.proj.weight_packed"]["dtype"] == "U8" and header["a.proj.weight_scale"]["dtype"] == "F32"


def test_sharded_index(tmp_path):
    from safetensors.torch import save_file

    a = random_matrix(16, 64, 4, 32, 1, qz.FMT_F32, seed=2)
    b = random_matrix(32, 64, 2, 32, 1, qz.FMT_F32, seed=3)
    (tmp_path / "config.json").write_text(json.dumps(config({
        "w4": {"targets": ["a.proj"], "weights": cubic_group(4, 32)},
        "w2": {"targets": ["b.proj"], "weights": cubic_group(2, 32)}})))
    save_file({f"a.proj.{k}": v for k, v in a.payload.items()}, str(tmp_path / "part-1.safetensors"))
    save_file({f"b.proj.{k}": v for k, v in b.payload.items()}, str(tmp_path / "part-2.safetensors"))
    weight_map = {f"a.proj.{k}": "part-1.safetensors" for k in a.payload}
    weight_map.update({f"b.proj.{k}": "part-2.safetensors" for k in b.payload})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    plan = ck.CubicCheckpoint.admit(tmp_path, [ck.LogicalWeight("a.proj.weight", (16, 64)),
                                               ck.LogicalWeight("b.proj.weight", (32, 64))])
    assert same_payload(plan.materialize(plan.weight("a.proj.weight")), a)
    assert same_payload(plan.materialize(plan.weight("b.proj.weight")), b)
    assert plan.weight("b.proj.weight").encoding.bits == 2


def test_declaration_digest_is_blake2s_of_canonical_json():
    # "b2s256:" + BLAKE2s-256 of the declaration as sorted, compact JSON
    # (models/quantization.py:117-119); the hex below was computed with
    # `openssl dgst -blake2s256` over that JSON text, independently of hashlib
    cfg = ck.QuantizationConfig.from_model_config(config({"g": {"targets": ["lm_head"], "weights": cubic_group(4)}}))
    assert cfg.digest == "b2s256:3789becc33d6ca0037fe3c09566b8a90b4d9c3f49c4155318799376a7ec44ff8"
    # key order in the file does not change the identity
    raw = config({"g": {"targets": ["lm_head"], "weights": cubic_group(4)}})
    shuffled = {"quantization_config": dict(reversed(list(raw["quantization_config"].items())))}
    assert ck.QuantizationConfig.from_model_config(shuffled).digest == cfg.digest


def test_text_config_prefix_rewrite_follows_the_module():
    # models/quantization.py:131-136: a text_config declaration rewrites every
    # name (aliases too) only when the module itself sits under
    # model.language_model.; otherwise no name is rewritten
    nested = ck.QuantizationConfig.from_model_config(
        {"text_config": config({"g": {"targets": ["model.layers.0.mlp.up_proj"], "weights": cubic_group(4)}})})
    assert nested.resolve("model.language_model.layers.0.mlp.up_proj").bits == 4
    # wrapped module, wrapped alias: both rewritten, the alias matches
    assert nested.resolve("model.language_model.layers.0.mlp.gate_up",
                          aliases=("model.language_model.layers.0.mlp.up_proj",)).bits == 4
    # unwrapped module: its wrapped alias keeps the prefix and matches nothing
    assert nested.resolve("model.layers.1.mlp.gate_up",
                          aliases=("model.language_model.layers.0.mlp.up_proj",)) is None
    # a root declaration never rewrites
    root = ck.QuantizationConfig.from_model_config(
        config({"g": {"targets": ["model.layers.0.mlp.up_proj"], "weights": cubic_group(4)}}))
    assert root.resolve("model.language_model.layers.0.mlp.up_proj") is None
