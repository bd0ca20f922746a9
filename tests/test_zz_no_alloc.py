"""fllm_dequantize_noalloc, the entry point that allocates nothing: its results equal
fllm_dequantize's bit for bit (and the oracle's Dequantizer restatement) on two calls in a row, the
second smaller than the first, so whatever the first call left in the shared scratch array cannot
leak into the second; sizes past its stated maximum are rejected with FLLM_E_ARG."""
import ctypes as C

import numpy as np
import pytest

import dotnetfoundryllm_amd._native as N
import oracle_bind as O

pytestmark = pytest.mark.gpu


def _blocks(tensor_type, n_blocks, seed):
    bb, _ = N.BLOCK[tensor_type]
    raw = np.random.default_rng(seed).integers(0, 256, n_blocks * bb, dtype=np.uint8)
    if tensor_type == N.Q6_K:
        raw.reshape(n_blocks, bb)[:, 208:210] = (0x00, 0x1C)  # finite f16 d
    elif tensor_type in (N.Q4_K, N.Q5_K):
        raw.reshape(n_blocks, bb)[:, 0:4] = (0x00, 0x1C, 0x00, 0x1C)  # finite f16 d and dmin
    elif tensor_type == N.Q8_0:
        raw.reshape(n_blocks, bb)[:, 0:2] = (0x00, 0x20)
    return raw


def _call(fn, ctx, tensor_type, raw, n):
    dst = np.full(n, np.nan, dtype=np.float32)
    rc = fn(ctx.h, tensor_type, raw.ctypes.data_as(C.c_void_p), raw.nbytes, dst.ctypes.data_as(N.PF32), n)
    return rc, dst


@pytest.mark.parametrize("first,second", [((N.Q6_K, 8000), (N.Q4_K, 100)), ((N.F32, 500000), (N.Q8_0, 3))])
def test_noalloc_matches_allocating_entry_point(ctx, first, second):
    for (tt, nblk), seed in ((first, 1), (second, 2)):
        raw = _blocks(tt, nblk, seed)
        bb, be = N.BLOCK[tt]
        n = nblk * be
        assert raw.nbytes <= N.NOALLOC_MAX_BYTES and n <= N.NOALLOC_MAX_ELEMS
        rc, got = _call(N.dev.fllm_dequantize_noalloc, ctx, tt, raw, n)
        assert rc == N.OK, N.dev.fllm_last_error()
        rc, want = _call(N.dev.fllm_dequantize, ctx, tt, raw, n)
        assert rc == N.OK
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        rc, orc = O.dequantize(tt, raw, n)
        assert rc == 0 and np.array_equal(got.view(np.uint32), orc.view(np.uint32))


def test_noalloc_size_limits(ctx):
    # one block past either limit is rejected before anything runs
    raw = _blocks(N.Q4_K, N.NOALLOC_MAX_ELEMS // 256 + 1, 3)
    rc, _ = _call(N.dev.fllm_dequantize_noalloc, ctx, N.Q4_K, raw, raw.nbytes // 144 * 256)
    assert rc == N.E_ARG and b"at most" in N.dev.fllm_last_error()
    raw = np.zeros(N.NOALLOC_MAX_BYTES + 4, dtype=np.uint8)
    rc, _ = _call(N.dev.fllm_dequantize_noalloc, ctx, N.F32, raw, raw.nbytes // 4)
    assert rc == N.E_ARG
    # the same contract as fllm_dequantize for bad arguments
    raw = _blocks(N.Q8_0, 2, 4)
    assert _call(N.dev.fllm_dequantize_noalloc, ctx, N.Q8_0, raw[:-1], 64)[0] == N.E_ARG
    assert _call(N.dev.fllm_dequantize_noalloc, ctx, 3, raw, 64)[0] == N.E_NOT_SUPPORTED
    assert _call(N.dev.fllm_dequantize_noalloc, ctx, N.Q8_0, raw, 63)[0] == N.E_ARG
