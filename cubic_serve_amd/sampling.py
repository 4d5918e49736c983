"""MTP acceptance operators on gfx950.

Host mirror of the reference's sampling API (paths under src/cubic_serve/):
  verify_one_draft_candidates  ops/cuda/sampling/speculative.py:222-328
  LocalCandidatePlan           ops/cuda/sampling/local_candidates.py:17-226
  ShardedSamplingWorkspace     generation/tp_sampling.py:57-64
  merge_prefix                 executor/draft_graph.py:146-157
  RootTopKTopPSamplingPrimitive ops/cuda/sampling/topk_topp.py:124-278
  MTPVerifyPlan                the finish_review composition,
                               executor/draft_graph.py:1034-1067

Candidate selection orders ties by ascending token id (torch.topk leaves the
order of equal scores at the cutoff unspecified).  All arithmetic runs in the
HIP library; there is no eager fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from . import _native


@dataclass(frozen=True, slots=True)
class ShardedSamplingWorkspace:
    """Caller-owned local and gathered candidate buffers (TP = 1: the same)."""

    local_scores: Tensor
    local_token_ids: Tensor
    gathered_scores: Tensor
    gathered_token_ids: Tensor


def _cuda_contiguous(*tensors: Tensor | None) -> bool:
    live = [t for t in tensors if t is not None]
    return all(t.device.type == "cuda" and t.is_contiguous() for t in live) and \
        len({t.device for t in live}) == 1


def verify_one_draft_candidates(
    *,
    q_scores: Tensor,
    q_token_ids: Tensor,
    p_scores: Tensor,
    p_token_ids: Tensor,
    target_rows: Tensor,
    draft_tokens: Tensor,
    temperatures: Tensor,
    top_ps: Tensor,
    top_ks: Tensor,
    seeds: Tensor,
    ordinals: Tensor,
    decisions: Tensor,
    active_rows: int,
    uniforms: Tensor | None = None,
    allow_underfilled: bool = False,
    constrained_rows: Tensor | None = None,
) -> None:
    """Launch one device-only K1 verification step for active proposal rows."""
    if type(allow_underfilled) is not bool:
        raise TypeError("speculative underfill policy must be boolean")
    if constrained_rows is not None and (
        not allow_underfilled or constrained_rows.dtype != torch.bool
        or constrained_rows.shape != temperatures.shape
        or constrained_rows.device != temperatures.device
        or not constrained_rows.is_contiguous()
    ):
        raise ValueError("invalid constrained-row ownership for speculative verification")
    operands = (q_scores, q_token_ids, p_scores, p_token_ids, target_rows, draft_tokens,
                temperatures, top_ps, top_ks, seeds, ordinals, uniforms, decisions)
    if not _cuda_contiguous(*operands):
        raise ValueError("speculative verification requires contiguous CUDA buffers on one device")
    if (
        q_scores.ndim != 3 or p_scores.ndim != 3
        or q_scores.dtype is not torch.bfloat16 or p_scores.dtype is not torch.bfloat16
        or q_token_ids.shape != q_scores.shape or p_token_ids.shape != p_scores.shape
        or q_token_ids.dtype is not torch.int64 or p_token_ids.dtype is not torch.int64
        or q_scores.shape[0] != p_scores.shape[0] or q_scores.shape[2] != p_scores.shape[2]
        or not 1 <= q_scores.shape[0] <= 8 or not 1 <= q_scores.shape[2] <= 20
    ):
        raise ValueError("speculative candidates require matching BF16/int64 [TP,C,K]")
    q_rows = q_scores.shape[1]
    row = (q_rows,)
    if (
        type(active_rows) is not int or not 1 <= active_rows <= q_rows
        or target_rows.shape != row or target_rows.dtype is not torch.int32
        or draft_tokens.shape != row or draft_tokens.dtype is not torch.int64
        or temperatures.shape != row or temperatures.dtype is not torch.float32
        or top_ps.shape != row or top_ps.dtype is not torch.float32
        or top_ks.shape != row or top_ks.dtype is not torch.int64
        or seeds.shape != row or seeds.dtype is not torch.int64
        or ordinals.shape != row or ordinals.dtype is not torch.int64
        or decisions.shape != (q_rows, 2) or decisions.dtype is not torch.int64
        or (uniforms is not None and (uniforms.shape != (q_rows, 2) or uniforms.dtype is not torch.float32))
    ):
        raise ValueError("speculative row buffers differ from proposal capacity")
    tp, _, k = q_scores.shape
    with torch.cuda.device(q_scores.device):
        _native.call("cubic_verify_candidates", *(_native.ptr(t) for t in (
            q_scores, q_token_ids, p_scores, p_token_ids, target_rows, draft_tokens, temperatures,
            top_ps, top_ks, seeds, ordinals, uniforms, constrained_rows)),
            int(allow_underfilled), tp, q_rows, p_scores.shape[1], k, active_rows,
            decisions.data_ptr(), _native.stream_of(q_scores.device))


# Operands of one root-sampling launch, in argument order: name, accepted
# dtypes, and whether the tensor is a candidate grid [TP, C, K] or a per-row
# vector [C].
_ROOT_OPERANDS = (
    ("scores", (torch.bfloat16, torch.float16), "grid"),
    ("token_ids", (torch.int64,), "grid"),
    ("temperatures", (torch.float32,), "row"),
    ("top_ps", (torch.float32,), "row"),
    ("top_ks", (torch.int64,), "row"),
    ("seeds", (torch.int64,), "row"),
    ("ordinals", (torch.int64,), "row"),
    ("output_tokens", (torch.int64,), "row"),
    ("output_valid", (torch.bool,), "row"),
)
_MAX_TP, _MAX_K = 8, 20


def _fingerprint(t: Tensor | None):
    """What a captured launch depends on besides the data: geometry, dtype
    and device (None for an absent optional operand)."""
    if t is None:
        return None
    if not isinstance(t, Tensor):
        raise TypeError("sampling operands must be tensors")
    return (t.dtype, t.device, tuple(t.shape), t.stride())


@dataclass(frozen=True, slots=True)
class RootTopKTopPSamplingMeta:
    """Launch identity for gathered ``[TP, C, K]`` candidates; ``block`` is
    the candidate count TP*K rounded up to a power of two."""

    device: torch.device
    tp: int
    rows: int
    candidates_per_rank: int
    block: int


class RootTopKTopPSamplingPrimitive:
    """Root-owned top-k/top-p sampling over TP-gathered candidates.

    The launch allocates nothing and keeps no host RNG state: each row draws
    from (seed, ordinal).  The operands given to the constructor fix the
    launch; ``launch`` accepts only tensors of the same geometry.  Interface
    of ops/cuda/sampling/topk_topp.py:141-278; the kernel is
    cubic_root_sample (one wave per row).
    """

    def __init__(self, scores: Tensor, token_ids: Tensor, temperatures: Tensor, top_ps: Tensor,
                 top_ks: Tensor, seeds: Tensor, ordinals: Tensor, output_tokens: Tensor,
                 output_valid: Tensor, *, allow_underfilled: bool = False,
                 constrained_rows: Tensor | None = None) -> None:
        if type(allow_underfilled) is not bool:
            raise TypeError("candidate underfill policy must be boolean")
        operands = (scores, token_ids, temperatures, top_ps, top_ks, seeds, ordinals,
                    output_tokens, output_valid)
        self._check_operands(operands)
        self._fixed_constraint = _fingerprint(constrained_rows)
        if constrained_rows is not None:
            usable = (allow_underfilled and constrained_rows.dtype == torch.bool
                      and constrained_rows.shape == temperatures.shape
                      and constrained_rows.device == temperatures.device
                      and constrained_rows.is_contiguous())
            if not usable:
                raise ValueError("invalid constrained-row ownership for root sampling")
        self.allow_underfilled = allow_underfilled
        self._fixed = tuple(_fingerprint(t) for t in operands)
        tp, rows, k = scores.shape
        self.meta = RootTopKTopPSamplingMeta(scores.device, tp, rows, k, 1 << (tp * k - 1).bit_length())

    @property
    def launch_signature(self) -> str:
        m = self.meta
        return (f"tp={m.tp},rows={m.rows},k={m.candidates_per_rank},block={m.block},"
                f"scores=bf16,prob=fp32,rng=philox,allow_underfilled={int(self.allow_underfilled)}")

    def launch(self, scores: Tensor, token_ids: Tensor, temperatures: Tensor, top_ps: Tensor,
               top_ks: Tensor, seeds: Tensor, ordinals: Tensor, output_tokens: Tensor,
               output_valid: Tensor, *, constrained_rows: Tensor | None = None) -> None:
        """Enqueue one launch on the device's current stream."""
        operands = (scores, token_ids, temperatures, top_ps, top_ks, seeds, ordinals,
                    output_tokens, output_valid)
        if tuple(_fingerprint(t) for t in operands) != self._fixed:
            raise ValueError("sampling operands do not match the fixed launch ABI")
        if _fingerprint(constrained_rows) != self._fixed_constraint:
            raise ValueError("constrained-row ownership differs from the fixed launch ABI")
        m = self.meta
        with torch.cuda.device(m.device):
            _native.call("cubic_root_sample", scores.data_ptr(), int(scores.dtype == torch.float16),
                         token_ids.data_ptr(), temperatures.data_ptr(), top_ps.data_ptr(),
                         top_ks.data_ptr(), seeds.data_ptr(), ordinals.data_ptr(),
                         _native.ptr(constrained_rows), int(self.allow_underfilled), m.tp, m.rows,
                         m.candidates_per_rank, output_tokens.data_ptr(), output_valid.data_ptr(),
                         _native.stream_of(m.device))

    @staticmethod
    def _check_operands(operands: tuple) -> None:
        for t in operands:
            _fingerprint(t)
        if not all(t.device.type == "cuda" and t.is_contiguous() for t in operands):
            raise ValueError("all sampling operands must be contiguous CUDA tensors")
        if len({t.device for t in operands}) > 1:
            raise ValueError("all sampling operands must share one CUDA device")
        grid = operands[0].shape
        if len(grid) != 3 or not 1 <= grid[0] <= _MAX_TP or not 1 <= grid[2] <= _MAX_K:
            raise ValueError("scores must be FP16/BF16 [TP,C,K] with TP<=8 and K<=20")
        expected_shape = {"grid": grid, "row": (grid[1],)}
        conforming = grid[1] > 0 and all(
            t.dtype in dtypes and t.shape == expected_shape[role]
            for t, (_, dtypes, role) in zip(operands, _ROOT_OPERANDS))
        if not conforming:
            raise ValueError("expected FP16/BF16 scores/int64 ids [TP,C,K], FP32 temperature/top_p, "
                             "int64 top_k/seed/ordinal/token, and bool valid [C]")


def merge_prefix(decisions: Tensor, out: Tensor, live: Tensor | int) -> None:
    """Per-depth decisions [depth, C, 2] -> (accepted length, bonus) [C, 2].

    ``live`` is the reference's ``ctx`` (device int32, first element = live
    rows) or a host int.
    """
    if (decisions.ndim != 3 or decisions.shape[2] != 2 or decisions.dtype is not torch.int64
            or out.shape != decisions.shape[1:] or out.dtype is not torch.int64
            or not _cuda_contiguous(decisions, out)):
        raise ValueError("merge_prefix needs int64 [depth, C, 2] decisions and [C, 2] output")
    depth, c, _ = decisions.shape
    live_ptr, live_rows = (None, int(live)) if isinstance(live, int) else (live.data_ptr(), 0)
    if not isinstance(live, int) and (live.dtype is not torch.int32 or live.device != out.device):
        raise ValueError("live row count must be a device int32 tensor")
    with torch.cuda.device(out.device):
        _native.call("cubic_merge_prefix", decisions.data_ptr(), c, depth, live_ptr, live_rows,
                     out.data_ptr(), _native.stream_of(out.device))


# logits dtype -> CUBIC_DTYPE_BF16 / _F16 / _F32 (local_candidates.py:41)
_CANDIDATE_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class LocalCandidatePlan:
    """Vocab logits -> published top-k candidates, bound before capture.

    One pass over ``local_logits[:active_rows, :visible_width]`` replaces
    torch.topk + candidate_partial + candidate_publish over this rank's
    vocabulary shard; published ids are ``vocab_start`` + column.  Logits and the
    published scores are bf16, fp16 or fp32 (local_candidates.py:41).
    """

    def __init__(self, *, local_logits: Tensor, workspace: ShardedSamplingWorkspace,
                 active_rows: int, visible_width: int, local_count: int, vocab_start: int = 0,
                 owned_rows: int | None = None, all_random_rows: bool = False,
                 row_activity: Tensor | None = None, metadata: Tensor | None = None,
                 token_mask: Tensor | None = None, masked_logits: Tensor | None = None,
                 consume_logits: bool = False) -> None:
        # the reference's grammar variant (local_candidates.py:79-110, the
        # HAS_GRAMMAR kernels of local_candidates.cu) is reached from its
        # greedy sampler only; cubic_serve_amd.greedy applies the mask inside
        # the greedy launch.  The candidate plan itself does not admit it.
        if token_mask is not None or masked_logits is not None or consume_logits:
            raise ValueError("grammar-masked candidate preparation is not admitted by this build "
                             "(use cubic_serve_amd.greedy for masked greedy sampling)")
        if (local_logits.dtype not in _CANDIDATE_DTYPES or local_logits.ndim != 2
                or local_logits.stride(1) != 1
                or not 0 < active_rows <= local_logits.shape[0]
                or not 0 < local_count <= visible_width <= local_logits.shape[1]
                or workspace.local_scores.dtype != local_logits.dtype
                or workspace.local_token_ids.dtype != torch.int64
                or workspace.local_scores.shape != workspace.local_token_ids.shape
                or workspace.local_scores.shape[0] < active_rows
                or workspace.local_scores.shape[1] < local_count
                or not workspace.local_scores.is_contiguous()
                or not workspace.local_token_ids.is_contiguous()):
            raise ValueError("local candidate preparation has an invalid tensor ABI")
        if type(vocab_start) is not int or vocab_start < 0:
            raise ValueError("vocabulary start must be a non-negative int")
        self.vocab_start = vocab_start
        if local_count > 20 or workspace.local_scores.shape[1] > 64:
            raise ValueError("candidate count must be <= 20 and capacity <= 64")
        if local_logits.device.type != "cuda":
            raise ValueError("local candidate preparation requires one CUDA device")
        # replay-time ownership (local_candidates.py:55-70): rows below the
        # device count metadata[0] whose activity flag is set
        if row_activity is not None and (row_activity.dtype != torch.bool
                                         or row_activity.shape != (active_rows,)
                                         or row_activity.device != local_logits.device
                                         or not row_activity.is_contiguous()):
            raise ValueError("local candidate row activity has an invalid tensor ABI")
        if metadata is not None and (metadata.dtype != torch.int32 or metadata.ndim != 1
                                     or metadata.numel() < 1
                                     or metadata.device != local_logits.device
                                     or not metadata.is_contiguous()):
            raise ValueError("local candidate metadata has an invalid tensor ABI")
        self.row_activity, self.metadata = row_activity, metadata
        self.logits, self.capacity = local_logits, active_rows
        self.width, self.count = visible_width, local_count
        self.outputs = (workspace.local_scores, workspace.local_token_ids)
        self.owned_rows = active_rows if owned_rows is None else owned_rows
        self.all_random = all_random_rows
        dev = local_logits.device
        self.temperatures = torch.empty(active_rows, device=dev)
        nbytes = _native.lib().cubic_candidates_workspace_bytes(active_rows, visible_width)
        if nbytes < 0:
            raise ValueError("vocabulary width not admitted")
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def launch(self, *, temperatures: Tensor) -> None:
        if (temperatures.dtype != torch.float32 or temperatures.device != self.temperatures.device
                or temperatures.shape != self.temperatures.shape or not temperatures.is_contiguous()):
            raise ValueError("local candidate temperatures differ from the bound ABI")
        self.temperatures.copy_(temperatures)
        scores, ids = self.outputs
        with torch.cuda.device(self.logits.device):
            _native.call("cubic_candidates", self.logits.data_ptr(),
                         _CANDIDATE_DTYPES[self.logits.dtype], self.logits.stride(0),
                         self.capacity, self.width, self.vocab_start, self.temperatures.data_ptr(),
                         self.owned_rows,
                         _native.ptr(self.metadata), _native.ptr(self.row_activity),
                         self.count, scores.shape[1], int(self.all_random), scores.data_ptr(),
                         ids.data_ptr(), self.workspace.data_ptr(), self.workspace.numel(),
                         _native.stream_of(self.logits.device))


class MTPVerifyPlan:
    """Fused verify step: candidates of the C*(k+1) target rows, verification
    of every depth and the accepted-prefix merge, in one launch.

    Equals LocalCandidatePlan.launch -> verify_one_draft_candidates per depth
    -> merge_prefix (executor/draft_graph.py:1049-1067) with TP = 1 and
    target row c*(k+1)+d for depth d.  Outputs: ``candidate_scores/ids``
    [C*(k+1), K], ``decisions`` [k, C, 2], ``merged`` [C, 2] (accepted length,
    bonus token) and ``emitted`` [C, k+1] (accepted drafts, then the bonus).
    """

    def __init__(self, *, logits: Tensor, q_scores: Tensor, q_token_ids: Tensor,
                 draft_tokens: Tensor, temperatures: Tensor, top_ps: Tensor, top_ks: Tensor,
                 seeds: Tensor, ordinals: Tensor, uniforms: Tensor | None = None,
                 row_temperatures: Tensor | None = None, visible_width: int | None = None):
        depth, c, k = q_scores.shape
        rows = c * (depth + 1)
        if (logits.dtype is not torch.bfloat16 or logits.ndim != 2 or logits.shape[0] < rows
                or logits.stride(1) != 1 or logits.device.type != "cuda"):
            raise ValueError("verify logits must be CUDA bf16 [C*(k+1), V]")
        if (q_scores.dtype is not torch.bfloat16 or q_token_ids.shape != q_scores.shape
                or q_token_ids.dtype is not torch.int64 or not 1 <= k <= 20 or not 1 <= depth <= 8):
            raise ValueError("draft candidates must be bf16/int64 [k, C, K] with K <= 20")
        per_depth = (depth, c)
        for t, dt in ((draft_tokens, torch.int64), (temperatures, torch.float32),
                      (top_ps, torch.float32), (top_ks, torch.int64), (seeds, torch.int64),
                      (ordinals, torch.int64)):
            if t.shape != per_depth or t.dtype is not dt:
                raise ValueError("per-depth parameters must be [k, C]")
        if uniforms is not None and (uniforms.shape != (depth, c, 2) or uniforms.dtype is not torch.float32):
            raise ValueError("uniforms must be float32 [k, C, 2]")
        if not _cuda_contiguous(logits[:1], q_scores, q_token_ids, draft_tokens, temperatures,
                                top_ps, top_ks, seeds, ordinals, uniforms):
            raise ValueError("verify operands must be contiguous on one CUDA device")
        dev = logits.device
        self.depth, self.c, self.k = depth, c, k
        self.width = logits.shape[1] if visible_width is None else visible_width
        self.logits, self.q_scores, self.q_token_ids = logits, q_scores, q_token_ids
        self.params = (draft_tokens, temperatures, top_ps, top_ks, seeds, ordinals)
        self.uniforms = uniforms
        if row_temperatures is None:
            row_temperatures = temperatures[0].repeat_interleave(depth + 1).contiguous()
        self.row_temperatures = row_temperatures
        self.candidate_scores = torch.empty((rows, k), dtype=torch.bfloat16, device=dev)
        self.candidate_ids = torch.empty((rows, k), dtype=torch.int64, device=dev)
        self.decisions = torch.empty((depth, c, 2), dtype=torch.int64, device=dev)
        self.merged = torch.empty((c, 2), dtype=torch.int64, device=dev)
        self.emitted = torch.empty((c, depth + 1), dtype=torch.int64, device=dev)
        nbytes = _native.lib().cubic_accept_workspace_bytes(c, depth, self.width)
        if nbytes < 0:
            raise ValueError("vocabulary width not admitted")
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def launch(self, live_rows: int | Tensor | None = None) -> None:
        """``live_rows``: live sequences, a host int or a device int32 tensor
        whose first element is read when the launch runs (the reference's
        ``ctx``; a captured launch then follows later writes to it)."""
        live, live_ptr = self.c, None
        if isinstance(live_rows, Tensor):
            if (live_rows.dtype != torch.int32 or live_rows.device != self.logits.device
                    or live_rows.numel() < 1 or not live_rows.is_contiguous()):
                raise ValueError("live row count must be a device int32 tensor")
            live_ptr = live_rows.data_ptr()
        elif live_rows is not None:
            live = live_rows
        d, t, p, k_, s, o = self.params
        with torch.cuda.device(self.logits.device):
            _native.call("cubic_accept", self.logits.data_ptr(), self.logits.stride(0), self.width,
                         self.c, self.depth, live, live_ptr, self.row_temperatures.data_ptr(),
                         self.q_scores.data_ptr(), self.q_token_ids.data_ptr(), self.k,
                         d.data_ptr(), t.data_ptr(), p.data_ptr(), k_.data_ptr(), s.data_ptr(),
                         o.data_ptr(), _native.ptr(self.uniforms),
                         self.candidate_scores.data_ptr(), self.candidate_ids.data_ptr(),
                         self.decisions.data_ptr(), self.merged.data_ptr(), self.emitted.data_ptr(),
                         self.workspace.data_ptr(), self.workspace.numel(),
                         _native.stream_of(self.logits.device))
