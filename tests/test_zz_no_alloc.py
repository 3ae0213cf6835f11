"""The allocation-free packed attention (lr_packed_attention_noalloc, its partial states in the
library's fixed per-device scratch array) called through the C ABI gives exactly the output of
lr_packed_attention with a caller-allocated workspace (same kernels, same reduction order), on
two calls in a row, the second smaller than the first (the array then still holds the first
call's partials), and refuses a call that needs more scratch than the array holds."""

import ctypes

import numpy as np
import pytest
import torch

from code_for_iclr27_amd import _lib

pytestmark = pytest.mark.gpu


def make(device, batch, kv_heads, groups, dim, lengths, seed):
    g = torch.Generator().manual_seed(seed)
    lengths = np.asarray(lengths, np.int64)
    total = int(lengths.sum())
    queries = torch.randn((batch, kv_heads * groups, 1, dim), generator=g).to(torch.bfloat16)
    keys = torch.randn((total, dim), generator=g).to(torch.bfloat16)
    values = torch.randn((total, dim), generator=g).to(torch.bfloat16)
    cumulative = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    return (queries.to(device), keys.to(device), values.to(device),
            torch.from_numpy(cumulative).to(device), int(lengths.max()))


def attend(entry, queries, keys, values, cumulative, max_keys, kv_heads, groups, workspace):
    batch, _, length, dim = queries.shape
    out = torch.full((batch, length, kv_heads * groups, dim), float("nan"),
                     dtype=queries.dtype, device=queries.device)
    stream = torch.cuda.current_stream(queries.device).cuda_stream
    args = [queries.data_ptr(), queries.stride(0), queries.stride(1), queries.stride(2),
            keys.data_ptr(), values.data_ptr(), keys.shape[0], cumulative.data_ptr(), batch,
            kv_heads, groups, length, dim, _lib.LR_DTYPE_BF16, max_keys, float(dim ** -0.5),
            out.data_ptr()]
    if entry == "lr_packed_attention":
        args += [None if workspace is None else workspace.data_ptr(),
                 0 if workspace is None else workspace.numel()]
    _lib.call(entry, *args, stream)
    return out


def test_noalloc_attention_matches_workspace_entry_point():
    device = torch.device("cuda:0")
    library = _lib.load()
    limit = library.lr_packed_attention_scratch_bytes()
    assert limit == 16 << 20
    rng = np.random.default_rng(0)
    cases = [
        # cfg2's decode shape: 8 requests x 8 KV heads, 4 groups, d128, 1500-2250 keys
        dict(batch=8, kv_heads=8, groups=4, dim=128, lengths=rng.integers(1500, 2251, 64)),
        # a smaller second call (fewer segments and key blocks; the array keeps older partials)
        dict(batch=2, kv_heads=4, groups=6, dim=256, lengths=rng.integers(200, 700, 8)),
    ]
    for seed, case in enumerate(cases):
        queries, keys, values, cumulative, max_keys = make(
            device, case["batch"], case["kv_heads"], case["groups"], case["dim"],
            case["lengths"], seed)
        needed = library.lr_packed_attention_workspace_bytes(
            case["batch"] * case["kv_heads"], case["groups"], 1, max_keys, case["dim"])
        assert 0 < needed <= limit  # both calls use the scratch array
        workspace = torch.empty(needed, dtype=torch.uint8, device=device)
        expect = attend("lr_packed_attention", queries, keys, values, cumulative, max_keys,
                        case["kv_heads"], case["groups"], workspace)
        got = attend("lr_packed_attention_noalloc", queries, keys, values, cumulative, max_keys,
                     case["kv_heads"], case["groups"], None)
        torch.cuda.synchronize()
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got.view(torch.int16), expect.view(torch.int16)), seed


def test_noalloc_attention_refuses_oversized_calls():
    device = torch.device("cuda:0")
    library = _lib.load()
    queries, keys, values, cumulative, _ = make(device, 1, 1, 1, 128, [64], 0)
    out = torch.zeros((1, 1, 1, 128), dtype=torch.bfloat16, device=device)
    max_keys = 1 << 24  # partial states for 2^24 keys exceed the fixed array
    assert library.lr_packed_attention_workspace_bytes(1, 1, 1, max_keys, 128) > \
        library.lr_packed_attention_scratch_bytes()
    status = library.lr_packed_attention_noalloc(
        queries.data_ptr(), queries.stride(0), queries.stride(1), queries.stride(2),
        keys.data_ptr(), values.data_ptr(), keys.shape[0], cumulative.data_ptr(), 1, 1, 1, 1,
        128, _lib.LR_DTYPE_BF16, max_keys, ctypes.c_float(128 ** -0.5), out.data_ptr(),
        torch.cuda.current_stream(device).cuda_stream)
    assert status == 1
    assert "allocation-free entry point holds at most 16777216 bytes" in _lib.last_error()
    torch.cuda.synchronize()
    assert not out.any()  # nothing was enqueued
