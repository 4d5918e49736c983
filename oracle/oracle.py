"""CPU oracle for the MTP verify step: numpy + the C restatement in cubic_oracle.c.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker (or the timed CPU baseline).  Product code never imports it.

Reference paths are relative to ``src/cubic_serve/`` of QuantTrio/cubic-serve.

Function                  restates                                         pinned by
------------------------  -----------------------------------------------  ------------------------------
unpack_cubic              quantization/extensions/cubic/reference.py:31-47  all-codes KAT (tests/ops/test_quantization_reference.py:136-152), brute-force bit loop
pack_cubic                inverse of the above (fixture helper)             round trip with unpack_cubic
cubic_metadata            reference.py:50-95                                KATs [[1,1],[6,6]] (:154-171) and ones(4,2) (:173-186)
decode_cubic              reference.py:98-121                               closed form at t in {0,1}; fl32(m/D) exactness; KATs above
decode_f16                quantization.py:181-182 with FP16 activations     numpy fp32->fp16 cast equals torch's on every decoded value
linear_bf16               ops/eager/linear.py:43-56 + quantization.py:181  FP64 anchor + enclosure bound
check_linear_enclosure    guardrail/quantization.py:176-320 (bf16, fp16)    closed form; rejects a +0.25 (bf16) / one-ulp-times-8 (fp16) corruption
candidates                ops/cuda/sampling/local_candidates.{py,cu}        brute force argsort on tiny rows (bf16, fp16 and fp32 scores)
verify_k1                 ops/cuda/sampling/speculative.py:46-219           reference KATs :73-131, :230-309; frozen-draw sweep :133-228; double-precision _oracle
root_sample               ops/cuda/sampling/topk_topp.py:22-121             reference oracle KATs tests/ops/test_cuda_topk_topp_sampling.py:65-91 and CUDA-test expectations :127-201; float64 brute force with explicit uniforms
moe_route                 ops/cuda/moe/fused.py:44-100                      stable argsort + float64 softmax (ids exact, weights within one bf16 step); reference softmax-midpoint KAT tests/unit/test_cuda_moe.py:276-332
moe_compact               ops/cuda/moe/fused.py:174-199                     reference KAT tests/ops/test_cuda_quantized_moe.py:25-67 (all sizes, modes, orders, block_m)
merge_prefix              executor/draft_graph.py:146-157                   chain KATs tests/generation/test_tp_sampling.py:120-178
philox_uniform            guardrail/quantized_graph/speculative.py:15-30    Random123 Philox4x32-10 known-answer vectors
expf                      (build-fixed exp for the acceptance transform)    <= 2 ulp against libm expf over a dense sweep
greedy_candidates         ops/cuda/sampling/greedy.cu:14-78                 reference test corpora tests/ops/test_cuda_greedy_sampling.py:95-109 (max + min id) and qualify fixtures greedy.py:640-660; literal column-scan loop on tiny rows (ties, +-0, masks, non-finite)
greedy_root               ops/cuda/sampling/greedy.cu:91-114                literal per-candidate loop (greedy.cu:94-98 order) on tiny [tp, rows, k]; reference invalid-parameter cases test_cuda_greedy_sampling.py:179-190
final_guard               ops/cuda/sampling/greedy.cu:117-139               enumerated per-term cases (each predicate flipped alone)
greedy_sample             greedy.py:255-320 at TP = 1                       composition of the three above
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libcubic_oracle.so"
_lib = None

METADATA_FORMATS = (
    "float32-scale-float16-ab",
    "int8-scale-int4-ab-global-fp32",
    "e5m9-scale-curve2-tensor-fp16",
)


def build() -> Path:
    """Compile the C restatement (gcc, -ffp-contract=off) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _lib.oracle_expf.restype = ctypes.c_float
        _lib.oracle_expf.argtypes = [ctypes.c_float]
        _lib.oracle_philox_uniform.restype = ctypes.c_float
        _lib.oracle_philox_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        _lib.oracle_half_to_float.restype = ctypes.c_float
        _lib.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.oracle_float_to_half.restype = ctypes.c_uint16
        _lib.oracle_float_to_half.argtypes = [ctypes.c_float]
        _lib.oracle_float_to_bf16.restype = ctypes.c_uint16
        _lib.oracle_float_to_bf16.argtypes = [ctypes.c_float]
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


# --------------------------------------------------------------------------- #
# bf16 helpers (numpy has no bfloat16: carry raw uint16 bit patterns)
# --------------------------------------------------------------------------- #
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_round_bf16(_p(x), _p(out), ctypes.c_int64(x.size))
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (_c(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def expf(x: float) -> float:
    return lib().oracle_expf(float(x))


def philox_uniform(seed: int, ordinal: int) -> float:
    return lib().oracle_philox_uniform(seed & (2**64 - 1), ordinal & (2**64 - 1))


def philox4x32_10(counter, key) -> list[int]:
    c = (ctypes.c_uint32 * 4)(*counter)
    k = (ctypes.c_uint32 * 2)(*key)
    out = (ctypes.c_uint32 * 4)()
    lib().oracle_philox4x32_10(c, k, out)
    return list(out)


# --------------------------------------------------------------------------- #
# A1-A3: Cubic bitstream, metadata and decode
# --------------------------------------------------------------------------- #
def unpack_cubic(packed: np.ndarray, bits: int, input_size: int) -> np.ndarray:
    packed = _c(packed, np.uint8)
    rows = packed.shape[0]
    if packed.shape[1] != math.ceil(input_size * bits / 8):
        raise ValueError("Cubic packed row length does not match logical K")
    out = np.empty((rows, input_size), np.int8)
    rc = lib().oracle_unpack_cubic(_p(packed), ctypes.c_int64(rows), ctypes.c_int64(input_size),
                                   ctypes.c_int(bits), _p(out))
    if rc:
        raise ValueError("invalid bit width")
    return out


def pack_cubic(codes: np.ndarray, bits: int) -> np.ndarray:
    codes = _c(codes, np.int8)
    rows, k = codes.shape
    out = np.empty((rows, math.ceil(k * bits / 8)), np.uint8)
    lib().oracle_pack_cubic(_p(codes), ctypes.c_int64(rows), ctypes.c_int64(k), ctypes.c_int(bits),
                            _p(out))
    return out


def _group_partitions(n: int, group_out: int, partitions) -> np.ndarray:
    parts = tuple(partitions) if partitions else (n,)
    if sum(parts) != n or any(p <= 0 or p % group_out for p in parts):
        raise ValueError("Cubic output partitions must preserve output-group boundaries")
    return np.repeat(np.arange(len(parts), dtype=np.int32), [p // group_out for p in parts])


def cubic_metadata(payload: dict, metadata: str, shape, group_in: int, group_out: int = 1,
                   partitions=()):
    """Expanded per-group (scale f32, a f16 bits, b f16 bits); reference.py:50-95."""
    n, k = shape
    grows, gcols = n // group_out, math.ceil(k / group_in)
    if metadata == METADATA_FORMATS[0]:
        return (_c(payload["weight_scale"], np.float32).reshape(grows, gcols),
                _c(payload["weight_a"], np.float16).view(np.uint16).reshape(grows, gcols),
                _c(payload["weight_b"], np.float16).view(np.uint16).reshape(grows, gcols))
    parts = _group_partitions(n, group_out, partitions)
    s = np.empty((grows, gcols), np.float32)
    a = np.empty((grows, gcols), np.uint16)
    b = np.empty((grows, gcols), np.uint16)
    if metadata == METADATA_FORMATS[1]:
        lib().oracle_metadata_fmt1(
            _p(_c(payload["weight_scale"], np.int8)), _p(_c(payload["weight_ab"], np.uint8)),
            _p(_c(payload["weight_scale_global"], np.float32)),
            _p(_c(payload["weight_a_global"], np.float32)),
            _p(_c(payload["weight_b_global"], np.float32)), _p(parts),
            ctypes.c_int64(grows), ctypes.c_int64(gcols), _p(s), _p(a), _p(b))
    elif metadata == METADATA_FORMATS[2]:
        lib().oracle_metadata_fmt2(
            _p(_c(payload["weight_metadata"], np.uint16)),
            _p(_c(payload["weight_curve_a"], np.float16).view(np.uint16)),
            _p(_c(payload["weight_curve_b"], np.float16).view(np.uint16)), _p(parts),
            ctypes.c_int64(grows), ctypes.c_int64(gcols), _p(s), _p(a), _p(b))
    else:
        raise ValueError(f"unsupported Cubic metadata {metadata!r}")
    return s, a, b


def decode_cubic(payload: dict, bits: int, metadata: str, shape, group_in: int,
                 group_out: int = 1, partitions=()) -> np.ndarray:
    """FP32 decoded weights [N, K]; reference.py:98-121."""
    n, k = shape
    codes = unpack_cubic(payload["weight_packed"], bits, k)
    s, a, b = cubic_metadata(payload, metadata, shape, group_in, group_out, partitions)
    if not np.isfinite(s).all() or (s < 0).any():
        raise ValueError("Cubic decoded scale must be finite and nonnegative")
    w = np.empty((n, k), np.float32)
    lib().oracle_decode_cubic(_p(codes), _p(s), _p(a), _p(b), ctypes.c_int64(n), ctypes.c_int64(k),
                              ctypes.c_int(bits), ctypes.c_int64(group_in),
                              ctypes.c_int64(group_out), _p(w))
    return w


def decode_bf16(payload: dict, bits: int, metadata: str, shape, group_in: int,
                group_out: int = 1, partitions=()) -> np.ndarray:
    """Decoded weights rounded once to bf16 (raw uint16 bits), as the WNA16 path
    does before its FP32 dot (ops/eager/quantization.py:181-182)."""
    return f32_to_bf16_bits(decode_cubic(payload, bits, metadata, shape, group_in, group_out,
                                         partitions))


def decode_f16(payload: dict, bits: int, metadata: str, shape, group_in: int,
               group_out: int = 1, partitions=()) -> np.ndarray:
    """Decoded weights rounded once to fp16 (raw uint16 bits): the WNA16 path
    with FP16 activations (ops/eager/quantization.py:181-182 casts the decoded
    weight to inputs.dtype); numpy's float32 -> float16 cast is IEEE RNE."""
    w = decode_cubic(payload, bits, metadata, shape, group_in, group_out, partitions)
    return w.astype(np.float16).view(np.uint16)


# --------------------------------------------------------------------------- #
# A5/A6: reference linear and its FP64 enclosure
# --------------------------------------------------------------------------- #
def linear_bf16(x_bits: np.ndarray, w_bits: np.ndarray):
    """y = bf16(sum_k fp32(x) * fp32(w)), ascending k; returns (y bf16 bits, y fp32)."""
    x_bits, w_bits = _c(x_bits, np.uint16), _c(w_bits, np.uint16)
    m, k = x_bits.shape
    n = w_bits.shape[0]
    y = np.empty((m, n), np.uint16)
    y32 = np.empty((m, n), np.float32)
    lib().oracle_linear_bf16(_p(x_bits), ctypes.c_int64(m), ctypes.c_int64(k), _p(w_bits),
                             ctypes.c_int64(n), _p(y), _p(y32))
    return y, y32


def check_linear_enclosure(x_bits: np.ndarray, w_bits: np.ndarray, y_bits: np.ndarray,
                           dtype: str = "bf16") -> dict:
    """guardrail/quantization.py:250-320 for a bf16 or fp16 boundary.

    |y - x.w|_f64 <= sum|x||w| (g32 + g64)/(1 - g64) (1 + u) + |anchor| u + tiny*u
    with g32 = s 2^-24 / (1 - s 2^-24), s = k + 12, g64 = k 2^-53 / (1 - k 2^-53),
    u = eps(dtype)/2, tiny = the dtype's smallest normal.  Raises
    AssertionError on any excess, like the reference.
    """
    if dtype == "bf16":
        to64 = lambda b: bf16_bits_to_f32(b).astype(np.float64)  # noqa: E731
        eps, tiny = 2.0**-7, 2.0**-126
    elif dtype == "f16":
        to64 = lambda b: _c(b, np.uint16).view(np.float16).astype(np.float64)  # noqa: E731
        eps, tiny = 2.0**-10, 2.0**-14
    else:
        raise ValueError(f"dtype {dtype!r}")
    x, w, y = to64(x_bits), to64(w_bits), to64(y_bits)
    k = x.shape[1]
    if not (np.isfinite(x).all() and np.isfinite(y).all()):
        raise AssertionError("native linear contains nonfinite operands or outputs")
    steps = k + 12
    gamma32 = steps * 2.0**-24 / (1.0 - steps * 2.0**-24)
    gamma64 = k * 2.0**-53 / (1.0 - k * 2.0**-53)
    uout = eps / 2.0              # torch.finfo(dtype).eps / 2
    underflow = tiny * uout       # torch.finfo(dtype).tiny * uout
    anchor = x @ w.T
    bound = (np.abs(x) @ np.abs(w).T) * ((gamma32 + gamma64) / (1.0 - gamma64)) * (1.0 + uout)
    bound += np.abs(anchor) * uout + underflow
    error = np.abs(y - anchor)
    if not np.isfinite(error).all() or (error > bound).any():
        raise AssertionError(
            f"native linear exceeds FP32/format/RNE enclosure: excess={(error - bound).max()}")
    return dict(rows=x.shape[0], outputs=w.shape[0], reduction_length=k,
                max_abs_error=float(error.max()), max_bound=float(bound.max()))


# --------------------------------------------------------------------------- #
# A13-A15: acceptance
# --------------------------------------------------------------------------- #
def candidates(logits_bits: np.ndarray, temperatures: np.ndarray, count: int, capacity: int | None = None,
               owned_rows: int | None = None, all_random: bool = False, fp16: bool = False,
               vocab_start: int = 0):
    """[M, V] bf16 (or fp16) logits -> ([M, capacity] scores of the same type, [M, capacity] int64 ids);
    real ids are vocab_start + column (candidate_publish adds the shard's start)."""
    logits_bits = _c(logits_bits, np.uint16)
    rows, width = logits_bits.shape
    capacity = count if capacity is None else capacity
    owned_rows = rows if owned_rows is None else owned_rows
    temps = _c(temperatures, np.float32)
    scores = np.empty((rows, capacity), np.uint16)
    ids = np.empty((rows, capacity), np.int64)
    rc = lib().oracle_candidates_dtype(_p(logits_bits), ctypes.c_int64(rows), ctypes.c_int64(width),
                                       ctypes.c_int64(width), _p(temps), ctypes.c_int64(owned_rows),
                                       ctypes.c_int(count), ctypes.c_int(capacity),
                                       ctypes.c_int(int(all_random)), ctypes.c_int(int(fp16)),
                                       _p(scores), _p(ids))
    if rc:
        raise ValueError("invalid candidate count")
    ids[ids >= 0] += vocab_start
    return scores, ids


def candidates_f32(logits: np.ndarray, temperatures: np.ndarray, count: int, capacity: int | None = None,
                   owned_rows: int | None = None, all_random: bool = False, vocab_start: int = 0):
    """[M, V] float32 logits (SCORE_TYPE 2, local_candidates.py:41) -> ([M, capacity] float32
    scores, [M, capacity] int64 ids); the rules of `candidates`, compared as float32 values."""
    logits = _c(logits, np.float32)
    rows, width = logits.shape
    capacity = count if capacity is None else capacity
    owned_rows = rows if owned_rows is None else owned_rows
    temps = _c(temperatures, np.float32)
    scores = np.empty((rows, capacity), np.float32)
    ids = np.empty((rows, capacity), np.int64)
    rc = lib().oracle_candidates_f32(_p(logits), ctypes.c_int64(rows), ctypes.c_int64(width),
                                     ctypes.c_int64(width), _p(temps), ctypes.c_int64(owned_rows),
                                     ctypes.c_int(count), ctypes.c_int(capacity),
                                     ctypes.c_int(int(all_random)), _p(scores), _p(ids))
    if rc:
        raise ValueError("invalid candidate count")
    ids[ids >= 0] += vocab_start
    return scores, ids


def verify_k1(q_scores, q_ids, p_scores, p_ids, target_rows, draft_tokens, temperatures, top_ps,
              top_ks, seeds, ordinals, active_rows: int, uniforms=None, allow_underfilled=False,
              constrained_rows=None) -> np.ndarray:
    """Decisions [C, 2] int64 for bf16-bit candidate arrays [TP, rows, K]."""
    q_scores, p_scores = _c(q_scores, np.uint16), _c(p_scores, np.uint16)
    q_ids, p_ids = _c(q_ids, np.int64), _c(p_ids, np.int64)
    tp, q_rows, k = q_scores.shape
    p_rows = p_scores.shape[1]
    dec = np.empty((q_rows, 2), np.int64)
    uni = None if uniforms is None else _c(uniforms, np.float32)
    con = None if constrained_rows is None else _c(constrained_rows, np.uint8)
    rc = lib().oracle_verify_k1(
        _p(q_scores), _p(q_ids), _p(p_scores), _p(p_ids), _p(_c(target_rows, np.int32)),
        _p(_c(draft_tokens, np.int64)), _p(_c(temperatures, np.float32)), _p(_c(top_ps, np.float32)),
        _p(_c(top_ks, np.int64)), _p(_c(seeds, np.int64)), _p(_c(ordinals, np.int64)), _p(uni),
        _p(con), ctypes.c_int(int(allow_underfilled)), ctypes.c_int(tp), ctypes.c_int(q_rows),
        ctypes.c_int(p_rows), ctypes.c_int(k), ctypes.c_int(active_rows), _p(dec))
    if rc:
        raise ValueError("candidate block too wide")
    return dec


def root_sample(scores, ids, temperatures, top_ps, top_ks, seeds, ordinals, *, fp16=False,
                uniforms=None, allow_underfilled=False, constrained_rows=None):
    """(tokens int64 [C], valid bool [C]) for fp16/bf16-bit candidates [TP, C, K]
    (ops/cuda/sampling/topk_topp.py:22-121).  ``uniforms`` [C] replaces the
    Philox draw (test hook, as the reference test oracle does)."""
    scores, ids = _c(scores, np.uint16), _c(ids, np.int64)
    tp, rows, k = scores.shape
    tokens = np.empty(rows, np.int64)
    valid = np.empty(rows, np.uint8)
    uni = None if uniforms is None else _c(uniforms, np.float32)
    con = None if constrained_rows is None else _c(constrained_rows, np.uint8)
    rc = lib().oracle_root_sample(
        _p(scores), ctypes.c_int(int(fp16)), _p(ids), _p(_c(temperatures, np.float32)),
        _p(_c(top_ps, np.float32)), _p(_c(top_ks, np.int64)), _p(_c(seeds, np.int64)),
        _p(_c(ordinals, np.int64)), _p(uni), _p(con), ctypes.c_int(int(allow_underfilled)),
        ctypes.c_int(tp), ctypes.c_int(rows), ctypes.c_int(k), _p(tokens), _p(valid))
    if rc:
        raise ValueError("candidate block too wide")
    return tokens, valid.astype(bool)


def moe_route(logits_bits, activity, active_rows: int, top_k: int, *, fp16=False,
              weights_fp16=False):
    """Router outputs (top_logits f32, top_ids, route_ids int64, route_weights
    uint16 bits), each [rows, top_k] (ops/cuda/moe/fused.py:44-100)."""
    logits_bits = _c(logits_bits, np.uint16)
    rows, experts = logits_bits.shape
    tl_ = np.empty((rows, top_k), np.float32)
    ti = np.empty((rows, top_k), np.int64)
    ri = np.empty((rows, top_k), np.int64)
    rw = np.empty((rows, top_k), np.uint16)
    rc = lib().oracle_moe_route(_p(logits_bits), ctypes.c_int(int(fp16)), _p(_c(activity, np.int32)),
                                ctypes.c_int(active_rows), ctypes.c_int(rows), ctypes.c_int(experts),
                                ctypes.c_int(top_k), _p(tl_), _p(ti), _p(ri), _p(rw),
                                ctypes.c_int(int(weights_fp16)))
    if rc:
        raise ValueError("invalid router geometry")
    return tl_, ti, ri, rw


def moe_compact(route_ids, first_expert: int, experts: int, block_m: int, row_map_fill: int = -777):
    """(counts, starts, block_starts, total_blocks, row_map) of
    ops/cuda/moe/fused.py:174-199; unwritten row_map slots keep ``row_map_fill``."""
    ids = _c(route_ids, np.int64).reshape(-1)
    counts = np.empty(experts, np.int32)
    starts = np.empty(experts, np.int32)
    blocks = np.empty(experts, np.int32)
    total = np.empty(1, np.int32)
    row_map = np.full(ids.size, row_map_fill, np.int32)
    lib().oracle_moe_compact(_p(ids), ctypes.c_int(ids.size), ctypes.c_int(first_expert),
                             ctypes.c_int(experts), ctypes.c_int(block_m), _p(counts), _p(starts),
                             _p(blocks), _p(total), _p(row_map))
    return counts, starts, blocks, int(total[0]), row_map


def merge_prefix(decisions: np.ndarray, live_rows: int) -> np.ndarray:
    decisions = _c(decisions, np.int64)
    depth, c, _ = decisions.shape
    out = np.empty((c, 2), np.int64)
    lib().oracle_merge_prefix(_p(decisions), ctypes.c_int(c), ctypes.c_int(depth),
                              ctypes.c_int(live_rows), _p(out))
    return out


def verify_from_logits(logits_bits, q_scores, q_ids, draft_tokens, temperatures, top_ps, top_ks,
                       seeds, ordinals, live_rows: int, uniforms=None, count: int = 20):
    """Composition A13 -> A14 (per depth) -> A15 for C sequences of depth D.

    logits: [C*(D+1), V] bf16 bits, row c*(D+1)+d.  q_*: [D, C, K].  Per-depth
    parameters: [D, C].  Target-row temperatures repeat each sequence's depth-0
    temperature (executor/draft_graph.py:1049-1054).  Returns (candidate scores,
    candidate ids, per-depth decisions [D, C, 2], merged [C, 2]).
    """
    depth, c, k = np.asarray(q_ids).shape
    temps = _c(temperatures, np.float32)
    row_t = np.repeat(temps[0], depth + 1)
    p_scores, p_ids = candidates(logits_bits, row_t, count, owned_rows=live_rows * (depth + 1))
    rows = np.arange(c, dtype=np.int32) * (depth + 1)
    dec = np.empty((depth, c, 2), np.int64)
    for d in range(depth):
        dec[d] = verify_k1(np.asarray(q_scores)[d][None], np.asarray(q_ids)[d][None], p_scores[None],
                           p_ids[None], rows + d, np.asarray(draft_tokens)[d], temps[d],
                           np.asarray(top_ps)[d], np.asarray(top_ks)[d], np.asarray(seeds)[d],
                           np.asarray(ordinals)[d], live_rows,
                           None if uniforms is None else np.asarray(uniforms)[d])
    return p_scores, p_ids, dec, merge_prefix(dec, live_rows)


# --------------------------------------------------------------------------- #
# Greedy sampler (non-speculative decode)
# --------------------------------------------------------------------------- #
NAN_BITS = {"bf16": 0x7FC0, "f16": 0x7E00}   # NaN payload of published padding (not pinned)


def _score_values(bits: np.ndarray, fp16: bool) -> np.ndarray:
    bits = np.asarray(bits, np.uint16)
    return bits.view(np.float16).astype(np.float64) if fp16 else bf16_bits_to_f32(bits).astype(np.float64)


def greedy_candidates(logits_bits, active: int, candidates: int, *, fp16=False, vocab_start=0,
                      token_mask=None):
    """greedy_partial + greedy_merge (ops/cuda/sampling/greedy.cu:14-78).

    logits_bits [rows, width] uint16 (bf16 or fp16 bits); token_mask
    [rows, words] uint32 or None.  Row r < active: the maximum over admitted
    columns, the lowest column among equal values (float equality, so -0 and
    +0 tie), published as (score, vocab_start + column) in slot 0; any
    non-finite visible value (admitted or not) gives (NaN, -2); no admitted
    column, rows >= active or width 0 give (NaN, -1).  Other slots (NaN, -1).
    """
    bits = np.asarray(logits_bits, np.uint16)
    rows, width = bits.shape
    vals = _score_values(bits, fp16)
    nan = NAN_BITS["f16" if fp16 else "bf16"]
    scores = np.full((rows, candidates), nan, np.uint16)
    ids = np.full((rows, candidates), -1, np.int64)
    for r in range(min(active, rows)):
        if width == 0:
            continue
        if not np.isfinite(vals[r]).all():                      # greedy.cu:24, :70
            ids[r, 0] = -2
            continue
        admitted = np.ones(width, bool)
        if token_mask is not None:                               # greedy.cu:26-27
            tokens = vocab_start + np.arange(width)
            words = np.asarray(token_mask, np.uint32)[r][tokens >> 5]
            admitted = ((words >> (tokens & 31).astype(np.uint32)) & 1).astype(bool)
        if not admitted.any():                                   # greedy.cu:67
            continue
        best = vals[r][admitted].max()
        col = int(np.flatnonzero(admitted & (vals[r] == best))[0])   # first maximum
        scores[r, 0] = bits[r, col]
        ids[r, 0] = vocab_start + col
    return scores, ids


def _greedy_params_ok(t, p, k, seed, ordinal, kmax):
    return (math.isfinite(p) and 0.0 < p <= 1.0 and 1 <= k <= kmax and seed >= 0 and ordinal >= 0,
            t == 0.0)


def greedy_root(scores_bits, ids, temperatures, top_ps, top_ks, seeds, ordinals, *, active: int,
                cancel: bool, vocab_size: int, fp16=False):
    """greedy_root (greedy.cu:91-114) over gathered [tp, rows, k] candidates."""
    bits = np.asarray(scores_bits, np.uint16)
    ids = np.asarray(ids, np.int64)
    tp, rows, k = bits.shape
    vals = _score_values(bits, fp16)
    tokens = np.empty(rows, np.int64)
    valid = np.zeros(rows, bool)
    for r in range(rows):
        if r >= active:
            tokens[r] = -2 if (cancel and r == active) else -1
            continue
        s, i = vals[:, r, :].ravel(), ids[:, r, :].ravel()
        real = np.isfinite(s) & (i >= 0) & (i < vocab_size)
        sentinel = np.isnan(s) & (i == -1)
        good = bool((real | sentinel).all())
        params, greedy = _greedy_params_ok(float(np.float32(temperatures[r])), float(np.float32(top_ps[r])),
                                           int(top_ks[r]), int(seeds[r]), int(ordinals[r]), k)
        ok = good and bool(real.any()) and greedy and params
        if ok:
            best = s[real].max()
            tokens[r] = int(i[real & (s == best)].min())
        else:
            tokens[r] = -1
        valid[r] = ok
    return tokens, valid


def final_guard(tokens, root_valid, temperatures, top_ps, top_ks, seeds, ordinals, *, active: int,
                k: int, vocab_size: int) -> bool:
    """sampling_final_guard (greedy.cu:117-139); root_valid None = non-root rank."""
    capacity = len(tokens)
    good = 0 < active <= capacity
    for i in range(capacity):
        tok = int(tokens[i])
        if i < active:
            t = float(np.float32(temperatures[i]))
            params, _ = _greedy_params_ok(0.0, float(np.float32(top_ps[i])), int(top_ks[i]),
                                          int(seeds[i]), int(ordinals[i]), k)
            good &= (0 <= tok < vocab_size and (root_valid is None or bool(root_valid[i]))
                     and math.isfinite(t) and 0.0 <= t <= 2.0 and params)
        elif i == active:
            good &= tok in (-1, -2)
        else:
            good &= tok == -1
    return bool(good)


def greedy_sample(logits_bits, temperatures, top_ps, top_ks, seeds, ordinals, *, active: int,
                  cancel: bool, k: int, vocab_size: int, fp16=False, token_mask=None):
    """Single-GPU composition: candidates -> root -> final guard (TP = 1)."""
    scores, ids = greedy_candidates(logits_bits, active, k, fp16=fp16, token_mask=token_mask)
    tokens, valid = greedy_root(scores[None], ids[None], temperatures, top_ps, top_ks, seeds, ordinals,
                                active=active, cancel=cancel, vocab_size=vocab_size, fp16=fp16)
    final = final_guard(tokens, valid, temperatures, top_ps, top_ks, seeds, ordinals, active=active,
                        k=k, vocab_size=vocab_size)
    return scores, ids, tokens, valid, final


if os.environ.get("CUBIC_ORACLE_BUILD_ON_IMPORT") == "1":  # pragma: no cover
    build()
