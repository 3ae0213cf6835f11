"""The C-ABI library loads and exports every symbol include/lazyrecall.h declares; argument
checks reject bad calls on the host (no GPU needed, nothing is launched); the torch mirror
modules expose the reference's function names and reject CPU tensors like the reference."""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _C, _host, _legacy_C, _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "lazyrecall.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lr_\w+)\s*\(", text, re.M)))


def test_header_and_loader_agree():
    assert declared_symbols() == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    library = _lib.load()
    for name in declared_symbols():
        assert hasattr(library, name), name
    assert library.lr_abi_version() == 1


def test_invalid_arguments_fail_on_host():
    library = _lib.load()
    status = library.lr_compact(None, None, None, 10, 0, 2, None, 0, None, None, None, None)
    assert status == 1 and "Invalid KV layout" in _lib.last_error()
    status = library.lr_pool(None, 10, None, 1, 4, 2, None, None)
    assert status == 1 and "Invalid pool configuration" in _lib.last_error()
    status = library.lr_temporal_risk(None, None, None, None, 4, 2, 10, 5, 5, 1e-6, None, None)
    assert status == 1 and "Invalid risk interval" in _lib.last_error()
    assert library.lr_score_workspace_bytes(2, 4, 250, 1000) > 0


def test_pool_select_checks_arguments_on_host():
    """The fused pool + selection entry refuses bad shapes before touching the device, with the
    messages of lr_pool and lr_select_refine_sets."""
    library = _lib.load()
    args = lambda total, max_count, width, segments, count: (
        None, total, None, max_count, width, None, None, None, segments, count, None, 0, None,
        None, None, None, None, None, None)
    assert library.lr_pool_select_refine_sets(*args(100, 50, 7, 2, 101)) == 1
    assert "Selection count must lie in [1, total]" in _lib.last_error()
    assert library.lr_pool_select_refine_sets(*args(100, 50, 6, 2, 10)) == 1
    assert "Invalid pool configuration" in _lib.last_error()
    assert library.lr_pool_select_refine_sets(*args(100, 50, 7, 70000, 10)) == 1
    assert "Invalid pool layout" in _lib.last_error()
    assert library.lr_pool_select_refine_sets(*args(100, 50, 7, 2, 10)) == 1
    assert "Expected contiguous CUDA tensor" in _lib.last_error()
    # the workspace it needs grows with the segment count (one LDS-histogram row per segment)
    assert (library.lr_select_workspace_bytes(1000, 64, 10)
            > library.lr_select_workspace_bytes(1000, 2, 10))


def test_noalloc_attention_size_check_needs_no_gpu():
    library = _lib.load()
    assert library.lr_packed_attention_scratch_bytes() == 16 << 20
    status = library.lr_packed_attention_noalloc(None, 0, 0, 0, None, None, 0, None, 1, 1, 1, 1,
                                                 128, _lib.LR_DTYPE_BF16, 1 << 24, 0.1, None, None)
    assert status == 1 and "holds at most 16777216 bytes" in _lib.last_error()


def test_stream_copy_checks_size_and_alignment_on_host():
    library = _lib.load()
    assert library.lr_stream_copy(None, None, 0, None) == 0
    assert library.lr_stream_copy(None, None, 24, None) == 1
    assert "multiple of 16" in _lib.last_error()
    assert library.lr_stream_copy(8, 16, 32, None) == 1
    assert "16-byte aligned" in _lib.last_error()


def test_pre_gradient_layers_width_bound_matches_per_layer_check():
    library = _lib.load()
    status = library.lr_pre_gradient_layers(None, 2, 16, 8200, _lib.LR_DTYPE_BF16, None, 0, None)
    assert status == 1 and "at most 8192" in _lib.last_error()


def test_batch_append_host_bounds_the_descriptor_table():
    """Descriptors in the launch's kernel arguments: at most 64 segments, rejected on the host
    before anything touches the device."""
    library = _lib.load()
    table = np.zeros(65 * 7, dtype=np.int64)
    address = table.ctypes.data
    status = library.lr_batch_append_host(address, 65, 1, 1, 8, 2, 1, 1, 1, 1, None)
    assert status == 1 and "Too many segments" in _lib.last_error()
    status = library.lr_batch_append_host(None, 1, 1, 1, 8, 2, 1, 1, 1, 1, None)
    assert status == 1 and "Request metadata mismatch" in _lib.last_error()


def test_append_layers_host_bounds_the_table():
    """An append table in the launch's kernel arguments: at most 48 layers, rejected on the host."""
    library = _lib.load()
    table = np.zeros(49 * 12, dtype=np.int64)
    status = library.lr_append_layers_host(table.ctypes.data, 49, 8, 1, 128, 2, 10, 1, 1, 1, 1,
                                           1, None)
    assert status == 1 and "Too many layers" in _lib.last_error()


def test_zero_work_calls_succeed_without_launching():
    library = _lib.load()
    assert library.lr_compact(None, None, None, 5, 8, 2, None, 5, None, None, None, None) == 0
    assert library.lr_merge(None, None, None, 0, None, None, 0, None, 0, 8, 2, None, None, None, None) == 0


def test_reference_function_names():
    for name in ("temporal_probabilities", "temporal_risk", "append", "compact", "pool", "merge",
                 "pack", "batch_append"):
        assert callable(getattr(_C, name))
    for name in ("append_flattened_cache", "compact_flattened_kv", "decision_risk_scores"):
        assert callable(getattr(_legacy_C, name))
    assert callable(_host.register_host) and callable(_host.unregister_host)


def test_cpu_tensors_rejected_like_reference():
    keys = torch.zeros(4, 8, dtype=torch.bfloat16)
    positions = torch.zeros(4, 1)
    with pytest.raises(RuntimeError, match="Expected contiguous CUDA tensor"):
        _C.compact(keys, keys, positions, torch.zeros(0, dtype=torch.long))
    with pytest.raises(RuntimeError, match="cache must be CUDA"):
        _legacy_C.append_flattened_cache(keys, keys.view(1, 1, 4, 8), torch.zeros(1, dtype=torch.int32),
                                         torch.zeros(2, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="Contiguous CUDA states required"):
        _C.batch_append([keys], [keys], [positions], keys.view(1, 1, 4, 8)[:, :, :1],
                        keys.view(1, 1, 4, 8)[:, :, :1], [[4]], [4])


def test_register_host_failure_raises():
    with pytest.raises(RuntimeError):
        _host.register_host(0, 0)


def test_host_planner_validates_like_the_reference():
    """The C++ planner (module _plan) is built and rejects bad layers on the host."""
    from code_for_iclr27_amd import scoring

    def layer(**over):
        fields = dict(keys=torch.zeros(8, 64, dtype=torch.bfloat16),
                      values=torch.zeros(8, 64, dtype=torch.bfloat16),
                      positions=torch.arange(8, dtype=torch.float32), head_lens=[4, 4],
                      prompt_lens=None, queries=torch.zeros(4, 3, 64, dtype=torch.bfloat16),
                      gradient=torch.zeros(4, 64))
        fields.update(over)
        return scoring.LayerState(**fields)

    with pytest.raises(RuntimeError, match="Expected contiguous CUDA tensor"):
        scoring.plan_segments([layer()])
    with pytest.raises(RuntimeError, match="No layers to score"):
        scoring.plan_segments([])
    with pytest.raises(RuntimeError, match="Query heads must be a multiple of KV heads"):
        scoring.plan_segments([layer(head_lens=[3, 3, 2])])


def test_step_sync_requires_a_pending_step():
    """The audit step's host wait object refuses a wait with no step posted (no GPU needed)."""
    from code_for_iclr27_amd import scoring

    sync = scoring._planner().StepSync()
    with pytest.raises(RuntimeError, match="no audit step is pending"):
        sync.wait(True)


def test_archive_library_exports_every_declared_symbol():
    from code_for_iclr27_amd import archive

    text = (HEADER.parent / "lazyrecall_archive.h").read_text()
    declared = sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(lra_\w+)\s*\(", text, re.M)))
    assert declared == sorted(archive.SIGNATURES)
    library = archive.load()
    for name in declared:
        assert hasattr(library, name), name
