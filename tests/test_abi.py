"""CPU checks of the C ABI library: it loads, exports every declared symbol,
and its host-side planning entry points answer without a GPU."""
from __future__ import annotations

import re
from pathlib import Path

import pytest

from cubic_serve_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "cubic_mi355x.h"


def declared_symbols() -> list[str]:
    return re.findall(r"^CUBIC_API [^(]*?\b(cubic_\w+)\(", HEADER.read_text(), flags=re.M)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.SIGNATURES), "ctypes signatures drift from the header"
    assert lib.cubic_abi_version() == 6


def test_host_planning_entry_points():
    lib = _native.lib()
    cw, mw = _native.ctypes.c_int64(), _native.ctypes.c_int64()
    _native.call("cubic_prepared_words", 151936, 4096, 4, 128, _native.ctypes.byref(cw),
                 _native.ctypes.byref(mw))
    assert cw.value * 4 == 151936 * 4096 * 4 // 8       # 4-bit codes, no padding
    assert mw.value * 4 == 151936 * (4096 // 128) * 16  # prepared 4-bit level table per group
    assert lib.cubic_gemm_workspace_bytes(64, 151936, 4096, 4) == 0   # no K split for the lm_head
    assert lib.cubic_gemm_workspace_bytes(64, 4096, 12288, 4) > 0     # down projection splits K
    assert lib.cubic_gemm_workspace_bytes(1, 4096, 12288, 4) < lib.cubic_gemm_workspace_bytes(64, 4096, 12288, 4)
    assert lib.cubic_accept_workspace_bytes(32, 1, 151936) > 0
    assert lib.cubic_accept_workspace_bytes(32, 9, 151936) == -1      # depth above 8
    # one size for every logits dtype: the fp32 plan ([rows, 4096-column tiles, 20] u64 keys
    # + flags) also covers vocabularies too wide for the 16-bit plan
    assert lib.cubic_candidates_workspace_bytes(64, 151936) >= 64 * 38 * (20 * 8 + 4)
    assert lib.cubic_candidates_workspace_bytes(64, 10**7) >= 64 * 2442 * (20 * 8 + 4)


def test_invalid_arguments_fail_before_any_launch():
    with pytest.raises(ValueError, match="count"):
        _native.call("cubic_candidates", 16, 0, 100, 2, 100, 0, 16, 2, None, None, 21, 21, 0, 16, 16, 16, 1 << 20, None)
    with pytest.raises(ValueError, match="dtype"):
        _native.call("cubic_candidates", 16, 3, 100, 2, 100, 0, 16, 2, None, None, 20, 20, 0, 16, 16, 16, 1 << 20, None)
    with pytest.raises(ValueError, match="too large"):   # 16-bit plan: at most 24 tiles of 32768
        _native.call("cubic_candidates", 16, 0, 10**7, 2, 10**7, 0, 16, 2, None, None, 20, 20, 0, 16, 16, 16, 1 << 30, None)
    with pytest.raises(ValueError, match="workspace"):   # fp32 plan, workspace too small
        _native.call("cubic_candidates", 16, 2, 10**7, 2, 10**7, 0, 16, 2, None, None, 20, 20, 0, 16, 16, 16, 1 << 10, None)
    with pytest.raises(ValueError, match="tp"):
        _native.call("cubic_verify_candidates", *([16] * 13), 0, 9, 4, 8, 20, 4, 16, None)
    with pytest.raises(ValueError, match="group_in"):
        _native.call("cubic_gemm", 16, 4096, 16, 16, 64, 4096, 4096, 4, 100, 0, 16, 4096, None, 0, None)
    with pytest.raises(ValueError, match="dtype"):
        _native.call("cubic_gemm", 16, 4096, 16, 16, 64, 4096, 4096, 4, 128, 2, 16, 4096, None, 0, None)
    # the small-row kernel (M <= 4, no workspace) sizes a tile's codes in 32
    # bits: at 2^31 bytes per tile (8 bits, K = 2^27) the plan takes the
    # split-K MFMA-tile kernel instead, which asks for a workspace
    with pytest.raises(ValueError, match="workspace"):
        _native.call("cubic_gemm", 16, 1 << 27, 16, 16, 1, 4096, 1 << 27, 8, 128, 0, 16, 4096, None, 0, None)
    with pytest.raises(ValueError, match="row stride"):   # small-row kernel, 32-bit activation extent
        _native.call("cubic_gemm", 16, 1 << 28, 16, 16, 4, 4096, 4096, 4, 128, 0, 16, 4096, None, 0, None)
    with pytest.raises(ValueError, match="int32 or int64"):
        _native.call("cubic_embedding", 16, 2, 4, 0, 16, 16, 16, 16, None, None, None, None,
                     64, 128, 4, 32, 1, 16, 0, None)
    with pytest.raises(ValueError, match="bf16 or fp16"):
        _native.call("cubic_embedding", 16, 8, 4, 0, 16, 16, 16, 16, None, None, None, None,
                     64, 128, 4, 32, 1, 16, 2, None)
    with pytest.raises(ValueError, match="part_of_row"):
        _native.call("cubic_embedding", 16, 8, 4, 2, 16, 16, 16, 16, None, None, None, None,
                     64, 128, 4, 32, 1, 16, 0, None)
    with pytest.raises(ValueError, match="group_out"):
        _native.call("cubic_embedding", 16, 8, 4, 0, 16, 16, 16, 16, None, None, None, None,
                     64, 128, 4, 32, 3, 16, 0, None)
    with pytest.raises(ValueError, match="TP<=8"):
        _native.call("cubic_root_sample", 16, 0, 16, 16, 16, 16, 16, 16, None, 0, 9, 4, 20, 16, 16, None)
    with pytest.raises(ValueError, match="constrained-row"):
        _native.call("cubic_root_sample", 16, 0, 16, 16, 16, 16, 16, 16, 16, 0, 4, 4, 20, 16, 16, None)


def test_root_sampler_rejects_cpu_storage():
    import torch

    from cubic_serve_amd import sampling

    scores = torch.empty((4, 1, 20), dtype=torch.bfloat16)
    rows = lambda dtype: torch.empty((1,), dtype=dtype)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        sampling.RootTopKTopPSamplingPrimitive(
            scores, torch.empty_like(scores, dtype=torch.int64), rows(torch.float32),
            rows(torch.float32), rows(torch.int64), rows(torch.int64), rows(torch.int64),
            rows(torch.int64), rows(torch.bool))
    with pytest.raises(TypeError, match="boolean"):
        sampling.RootTopKTopPSamplingPrimitive(
            scores, torch.empty_like(scores, dtype=torch.int64), rows(torch.float32),
            rows(torch.float32), rows(torch.int64), rows(torch.int64), rows(torch.int64),
            rows(torch.int64), rows(torch.bool), allow_underfilled=1)


def test_moe_router_and_compaction_arguments():
    with pytest.raises(ValueError, match="top-k"):
        _native.call("cubic_moe_route", 16, 0, 16, 16, 4, 16, 17, 16, 16, 16, 16, 0, None)
    with pytest.raises(ValueError, match="experts"):
        _native.call("cubic_moe_route", 16, 0, 16, 16, 4, 2000, 8, 16, 16, 16, 16, 0, None)
    with pytest.raises(ValueError, match="block_m"):
        _native.call("cubic_moe_compact", 16, 8, 0, 4, 0, 16, 16, 16, 16, 16, None)
    with pytest.raises(ValueError, match="experts"):
        _native.call("cubic_moe_compact", 16, 8, 0, 1025, 16, 16, 16, 16, 16, 16, None)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message (no GPU touched)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    res = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def test_greedy_sampler_arguments():
    lib = _native.lib()
    # one 2048-column tile per row once rows fill the chip; the workspace grows with rows
    assert 0 < lib.cubic_greedy_workspace_bytes(1, 151936) < lib.cubic_greedy_workspace_bytes(256, 151936)
    assert lib.cubic_greedy_workspace_bytes(0, 100) == -1
    ws = lib.cubic_greedy_workspace_bytes(4, 100)
    with pytest.raises(ValueError, match="candidates"):
        _native.call("cubic_greedy_candidates", 16, 0, 100, 4, 100, 0, 16, None, 0, None, 0, 65, 16, 16, 16, ws, None)
    with pytest.raises(ValueError, match="grammar mask"):
        _native.call("cubic_greedy_candidates", 16, 0, 100, 4, 100, 0, 16, 16, 3, None, 0, 20, 16, 16, 16, ws, None)
    with pytest.raises(ValueError, match="masked logits need a grammar mask"):
        _native.call("cubic_greedy_candidates", 16, 0, 100, 4, 100, 0, 16, None, 0, 32, 100, 20, 16, 16, 16, ws, None)
    with pytest.raises(ValueError, match="masked logits geometry"):   # in place needs the logits' stride
        _native.call("cubic_greedy_candidates", 16, 0, 100, 4, 100, 0, 16, 16, 4, 16, 128, 20, 16, 16, 16, ws, None)
    with pytest.raises(ValueError, match="workspace"):
        _native.call("cubic_greedy_candidates", 16, 0, 100, 4, 100, 0, 16, None, 0, None, 0, 20, 16, 16, 16, ws - 1, None)
    with pytest.raises(ValueError, match="TP<=8"):
        _native.call("cubic_greedy_root", 16, 0, 16, 16, 16, 16, 16, 16, 16, 9, 4, 20, 100, 16, 16, None)
    with pytest.raises(ValueError, match="vocabulary"):
        _native.call("cubic_greedy_root", 16, 0, 16, 16, 16, 16, 16, 16, 16, 1, 4, 20, 0, 16, 16, None)
    with pytest.raises(ValueError, match="null"):
        _native.call("cubic_sampling_final_guard", 16, None, 16, None, 16, 16, 16, 16, 4, 20, 100, 16, None)
    with pytest.raises(ValueError, match="exceeds the vocabulary"):
        _native.call("cubic_greedy_sample", 16, 0, 100, 4, 100, 16, None, 0, None, 0, 20, 16, 16, 16, 16, 16, 99,
                     16, 16, 16, 16, 16, 16, ws, None)


def test_candidate_plan_refuses_grammar_masks():
    """The grammar variant of LocalCandidatePlan (token_mask, masked_logits,
    consume_logits: local_candidates.py:79-110) is refused at bind, before any
    device work, with a message naming the masked greedy path."""
    import torch
    from cubic_serve_amd import sampling
    logits = torch.zeros((2, 64), dtype=torch.bfloat16)
    s = torch.empty((2, 20), dtype=torch.bfloat16)
    i = torch.empty((2, 20), dtype=torch.int64)
    ws = sampling.ShardedSamplingWorkspace(s, i, s, i)
    with pytest.raises(ValueError, match="grammar"):
        sampling.LocalCandidatePlan(local_logits=logits, workspace=ws, active_rows=2, visible_width=64,
                                    local_count=20, token_mask=torch.zeros((2, 2), dtype=torch.int32))
    with pytest.raises(ValueError, match="grammar"):
        sampling.LocalCandidatePlan(local_logits=logits, workspace=ws, active_rows=2, visible_width=64,
                                    local_count=20, consume_logits=True)
