"""Greedy sampling for non-speculative decode on gfx950.

Host mirror of the reference's greedy sampler (paths under src/cubic_serve/):
  ShardedSamplingParameters     generation/tp_sampling.py:46-54
  TensorParallelSamplingError   generation/tp_sampling.py:41-42
  greedy_candidates             greedy_partial + greedy_merge,
                                ops/cuda/sampling/greedy.cu:14-78 (greedy.py:255-283)
  greedy_root                   greedy.cu:91-114 (greedy.py:284-303)
  sampling_final_guard          greedy.cu:117-139 (greedy.py:304-320)
  CapturedGreedySampler         ops/cuda/sampling/greedy.py:41-620 on one GPU
                                (one final rank, which is the root; the
                                candidate all-gather and the token broadcast
                                are identities)

Every launch goes through the HIP library (cubic_greedy_* in
include/cubic_mi355x.h); there is no eager fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from . import _native
from .sampling import ShardedSamplingWorkspace


class TensorParallelSamplingError(ValueError):
    """A sampling boundary was violated (invalid operands, tokens or parameters)."""


@dataclass(frozen=True, slots=True)
class ShardedSamplingParameters:
    """Caller-owned per-row sampling parameters at captured-M capacity."""

    temperatures: Tensor
    top_ks: Tensor
    top_ps: Tensor
    max_top_k: int
    seeds: Tensor | None = None
    ordinals: Tensor | None = None


def _require(t: Tensor | None, shape: tuple, dtype: torch.dtype, device: torch.device, label: str):
    if device.type != "cuda":
        raise TensorParallelSamplingError(f"{label} must live on a CUDA device")
    if (not isinstance(t, Tensor) or tuple(t.shape) != shape or t.dtype != dtype
            or t.device != device or not t.is_contiguous()):
        raise TensorParallelSamplingError(f"{label} must be a contiguous {dtype} {list(shape)} on {device}")


def _require_parameters(p: ShardedSamplingParameters, capacity: int, device: torch.device) -> None:
    if type(p.max_top_k) is not int or not 1 <= p.max_top_k <= 64:
        raise TensorParallelSamplingError("max_top_k must be an int in 1..64")
    if p.seeds is None or p.ordinals is None:
        raise TensorParallelSamplingError("greedy sampling requires seed and ordinal buffers")
    for t, dt, label in ((p.temperatures, torch.float32, "temperatures"),
                         (p.top_ps, torch.float32, "top_ps"), (p.top_ks, torch.int64, "top_ks"),
                         (p.seeds, torch.int64, "seeds"), (p.ordinals, torch.int64, "ordinals")):
        _require(t, (capacity,), dt, device, label)


def _param_ptrs(p: ShardedSamplingParameters):
    return (p.temperatures.data_ptr(), p.top_ps.data_ptr(), p.top_ks.data_ptr(),
            p.seeds.data_ptr(), p.ordinals.data_ptr())


def _mask_words(token_mask: Tensor | None, rows: int, device: torch.device) -> int:
    if token_mask is None:
        return 0
    if (token_mask.dtype != torch.int32 or token_mask.ndim != 2 or token_mask.shape[0] != rows
            or token_mask.device != device or not token_mask.is_contiguous()):
        raise TensorParallelSamplingError("grammar bitmask must be contiguous int32 [rows, words]")
    return token_mask.shape[1]


def _masked_output(logits: Tensor, rows: int, width: int, token_mask: Tensor | None,
                   masked_logits: Tensor | None, consume_logits: bool) -> tuple[Tensor | None, int]:
    """The grammar-masked logits output and its row stride, checked as the
    reference's candidate preparation checks it (local_candidates.py:88-110):
    consuming the logits (masking them in place) needs the mask; an explicit
    output is [rows, width] of the logits' dtype on their device, contiguous
    and in storage of its own unless it is the logits themselves."""
    if type(consume_logits) is not bool or consume_logits and token_mask is None:
        raise TensorParallelSamplingError("logits consumption requires an explicit masked terminal consumer")
    if consume_logits and masked_logits is None:
        masked_logits = logits[:rows, :width]
    if masked_logits is None:
        return None, 0
    if (token_mask is None or masked_logits.shape != (rows, width) or masked_logits.dtype != logits.dtype
            or masked_logits.device != logits.device
            or (not consume_logits and not masked_logits.is_contiguous())
            or (consume_logits and (masked_logits.data_ptr() != logits.data_ptr()
                                    or masked_logits.stride() != logits[:rows, :width].stride()))
            or (not consume_logits and masked_logits.untyped_storage().data_ptr()
                == logits.untyped_storage().data_ptr())):
        raise TensorParallelSamplingError("masked logits differ from the grammar consumer ABI")
    return masked_logits, masked_logits.stride(0)


def greedy_workspace(rows: int, width: int, device: torch.device) -> Tensor:
    """Zero-filled workspace for the candidate pass (every launch returns its
    arrival counters to zero, so one fill serves every later launch)."""
    nbytes = _native.lib().cubic_greedy_workspace_bytes(rows, width)
    if nbytes < 0:
        raise TensorParallelSamplingError("greedy geometry not admitted")
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def greedy_candidates(logits: Tensor, metadata: Tensor, scores: Tensor, token_ids: Tensor,
                      workspace: Tensor, *, width: int | None = None, vocab_start: int = 0,
                      token_mask: Tensor | None = None, masked_logits: Tensor | None = None,
                      consume_logits: bool = False) -> None:
    """Exact argmax candidates of ``logits[:metadata[0], :width]`` into slot 0
    of ``scores``/``token_ids`` [rows, K] (greedy.cu:14-78).  With a grammar
    mask, ``masked_logits`` [rows, width] (or the logits themselves, when
    ``consume_logits``) receives the masked logits (local_candidates.cu:37-53)."""
    if logits.dtype not in (torch.bfloat16, torch.float16) or logits.ndim != 2 or logits.stride(1) != 1:
        raise TensorParallelSamplingError("greedy logits must be bf16/fp16 [rows, V] with unit column stride")
    rows = logits.shape[0]
    width = logits.shape[1] if width is None else width
    if type(width) is not int or not 0 <= width <= logits.shape[1] or type(vocab_start) is not int or vocab_start < 0:
        raise TensorParallelSamplingError("greedy visible width or vocabulary start is invalid")
    dev = logits.device
    _require(metadata, (2,), torch.int32, dev, "sampling metadata")
    k = scores.shape[1] if scores.ndim == 2 else 0
    _require(scores, (rows, k), logits.dtype, dev, "candidate scores")
    _require(token_ids, (rows, k), torch.int64, dev, "candidate ids")
    words = _mask_words(token_mask, rows, dev)
    masked, masked_stride = _masked_output(logits, rows, width, token_mask, masked_logits, consume_logits)
    with torch.cuda.device(dev):
        _native.call("cubic_greedy_candidates", logits.data_ptr(), int(logits.dtype == torch.float16),
                     logits.stride(0), rows, width, vocab_start, metadata.data_ptr(),
                     _native.ptr(token_mask), words, _native.ptr(masked), masked_stride, k,
                     scores.data_ptr(), token_ids.data_ptr(), workspace.data_ptr(), workspace.numel(),
                     _native.stream_of(dev))


def greedy_root(gathered_scores: Tensor, gathered_token_ids: Tensor,
                parameters: ShardedSamplingParameters, metadata: Tensor, tokens: Tensor,
                root_valid: Tensor, *, vocab_size: int) -> None:
    """Root decision over gathered [TP, C, K] candidates (greedy.cu:91-114)."""
    if gathered_scores.dtype not in (torch.bfloat16, torch.float16) or gathered_scores.ndim != 3:
        raise TensorParallelSamplingError("gathered scores must be bf16/fp16 [TP, C, K]")
    tp, rows, k = gathered_scores.shape
    dev = gathered_scores.device
    _require(gathered_scores, (tp, rows, k), gathered_scores.dtype, dev, "gathered scores")
    _require(gathered_token_ids, (tp, rows, k), torch.int64, dev, "gathered ids")
    _require(metadata, (2,), torch.int32, dev, "sampling metadata")
    _require(tokens, (rows,), torch.int64, dev, "token buffer")
    _require(root_valid, (rows,), torch.bool, dev, "root validity")
    _require_parameters(parameters, rows, dev)
    with torch.cuda.device(dev):
        _native.call("cubic_greedy_root", gathered_scores.data_ptr(),
                     int(gathered_scores.dtype == torch.float16), gathered_token_ids.data_ptr(),
                     *_param_ptrs(parameters), metadata.data_ptr(), tp, rows, parameters.max_top_k,
                     vocab_size, tokens.data_ptr(), root_valid.data_ptr(), _native.stream_of(dev))


def sampling_final_guard(tokens: Tensor, root_valid: Tensor | None, metadata: Tensor,
                         parameters: ShardedSamplingParameters, final_valid: Tensor, *,
                         vocab_size: int) -> None:
    """Batch validity of the published tokens (greedy.cu:117-139); ``root_valid``
    None is the reference's non-root rank."""
    dev = tokens.device
    capacity = tokens.numel()
    _require(tokens, (capacity,), torch.int64, dev, "token buffer")
    if root_valid is not None:
        _require(root_valid, (capacity,), torch.bool, dev, "root validity")
    _require(metadata, (2,), torch.int32, dev, "sampling metadata")
    _require(final_valid, (), torch.bool, dev, "final validity")
    _require_parameters(parameters, capacity, dev)
    with torch.cuda.device(dev):
        _native.call("cubic_sampling_final_guard", tokens.data_ptr(), _native.ptr(root_valid),
                     metadata.data_ptr(), *_param_ptrs(parameters), capacity, parameters.max_top_k,
                     vocab_size, final_valid.data_ptr(), _native.stream_of(dev))


class CapturedGreedySampler:
    """Fixed-capacity greedy sampler captured in one HIP graph (one GPU).

    The graph holds one launch of cubic_greedy_sample: candidate publication
    into ``workspace.local_scores/local_token_ids`` (which are also the
    gathered buffers at TP = 1), the root decision into ``token_ids`` and
    ``root_valid``, and the batch validity into ``final_valid``.  ``replay``
    writes the (count, cancel) metadata from a pinned host table, replays,
    and raises TensorParallelSamplingError when the batch is rejected.
    """

    def __init__(self, *, local_logits: Tensor, true_vocab_size: int, token_ids: Tensor,
                 parameters: ShardedSamplingParameters, workspace: ShardedSamplingWorkspace,
                 root_valid: Tensor, capture_stream: torch.cuda.Stream | None = None,
                 token_mask: Tensor | None = None, masked_logits: Tensor | None = None,
                 graph_pool=None, consume_logits: bool = False) -> None:
        dev = token_ids.device
        self.device = dev
        self.capacity = token_ids.numel()
        if (dev.type != "cuda" or token_ids.ndim != 1 or self.capacity < 1
                or type(true_vocab_size) is not int or true_vocab_size < 1):
            raise TensorParallelSamplingError("greedy graph topology or capacity is invalid")
        if (local_logits.dtype not in (torch.bfloat16, torch.float16) or local_logits.ndim != 2
                or local_logits.shape[0] != self.capacity or local_logits.stride(1) != 1
                or local_logits.device != dev):
            raise TensorParallelSamplingError("greedy graph logits ownership is invalid")
        _require(token_ids, (self.capacity,), torch.int64, dev, "greedy token buffer")
        _require(root_valid, (self.capacity,), torch.bool, dev, "greedy root validity")
        _require_parameters(parameters, self.capacity, dev)
        k = parameters.max_top_k
        for t, dt, label in ((workspace.local_scores, local_logits.dtype, "local scores"),
                             (workspace.local_token_ids, torch.int64, "local ids")):
            _require(t, (self.capacity, k), dt, dev, label)
        self.width = max(0, min(local_logits.shape[1], true_vocab_size))
        self.vocab_size = true_vocab_size
        self.logits, self.token_ids, self.root_valid = local_logits, token_ids, root_valid
        self.parameters, self.workspace, self.token_mask = parameters, workspace, token_mask
        self._mask_words = _mask_words(token_mask, self.capacity, dev)
        self.masked_logits, self._masked_stride = _masked_output(
            local_logits, self.capacity, self.width, token_mask, masked_logits, consume_logits)
        self.metadata = torch.zeros(2, dtype=torch.int32, device=dev)
        self._metadata_hosts = torch.empty((self.capacity + 1, 2, 2), dtype=torch.int32, pin_memory=True)
        self._metadata_hosts[:, :, 0] = torch.arange(self.capacity + 1)[:, None]
        self._metadata_hosts[:, :, 1] = torch.tensor([0, 1])[None, :]
        self._metadata_key: tuple[int, bool] | None = None
        self.final_valid = torch.zeros((), dtype=torch.bool, device=dev)
        self._scratch = greedy_workspace(self.capacity, self.width, dev)
        self.stream = capture_stream if capture_stream is not None else torch.cuda.Stream(device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            self._set_metadata(1, False)
            self.launch()                      # warm the launch before capture
            self.stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=self.stream, pool=graph_pool):
                self.launch()
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        self.graph = graph

    def launch(self) -> None:
        """Enqueue the fused launch on the current stream (metadata as it stands)."""
        w, p = self.workspace, self.parameters
        with torch.cuda.device(self.device):
            _native.call("cubic_greedy_sample", self.logits.data_ptr(),
                         int(self.logits.dtype == torch.float16), self.logits.stride(0),
                         self.capacity, self.width, self.metadata.data_ptr(),
                         _native.ptr(self.token_mask), self._mask_words,
                         _native.ptr(self.masked_logits), self._masked_stride, p.max_top_k,
                         *_param_ptrs(p), self.vocab_size, w.local_scores.data_ptr(),
                         w.local_token_ids.data_ptr(), self.token_ids.data_ptr(),
                         self.root_valid.data_ptr(), self.final_valid.data_ptr(),
                         self._scratch.data_ptr(), self._scratch.numel(),
                         _native.stream_of(self.device))

    def _set_metadata(self, count: int, cancel: bool) -> None:
        if type(count) is not int or not 0 < count <= self.capacity or type(cancel) is not bool:
            raise TensorParallelSamplingError("sampling metadata is invalid")
        key = (count, cancel)
        if key != self._metadata_key:
            self.metadata.copy_(self._metadata_hosts[count, int(cancel)], non_blocking=True)
            self._metadata_key = key

    def invalidate_metadata(self) -> None:
        """Require a metadata write after a caller graph wrote the metadata tensor."""
        self._metadata_key = None

    def replay(self, count: int, cancel: bool = False, *, validity_out: Tensor | None = None) -> Tensor:
        if self.graph is None:
            raise TensorParallelSamplingError("greedy graph replay is unavailable")
        if validity_out is not None:
            _require(validity_out, (), torch.bool, self.device, "deferred sampling validity")
        self._set_metadata(count, cancel)
        self.graph.replay()
        if validity_out is not None:
            validity_out.copy_(self.final_valid)
            return self.token_ids
        if not bool(self.final_valid.item()):
            raise TensorParallelSamplingError("TP sampling rejected invalid candidates or tokens")
        return self.token_ids

    def close(self) -> None:
        if self.graph is not None:
            torch.cuda.synchronize(self.device)
            self.graph.reset()
            self.graph = None
