"""IKvCache through the C ABI (fllm_kv_append / fllm_kv_read / fllm_kv_length / fllm_kv_was_evicted /
fllm_seq_reset), eviction of a full cache inside the device forward pass against the oracle, and
the disposal contract of the weights (fllm_model_destroy).

The first group restates tests/DotNetFoundryLLM.Inference.Tests/KvCacheTests.cs against HipKvCache,
except Append_BeyondCapacity_Throws (:61-72), which contradicts KvCache.cs:82-85 (a full cache
evicts its oldest half instead of throwing); the eviction is tested for what the code does. The
device cache belongs to a model, so its layer count and kv_dim come from a tiny model: the
reference's kvDim 2 and 3 cases use kv_dim 4 (one kv head of head_dim 4, the smallest head the
device path takes), with the same positions, lengths and values.
"""
import ctypes as C

import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import dotnetfoundryllm_amd._native as N
import oracle_bind as O
from fixtures import synthetic, upload

pytestmark = pytest.mark.gpu


def tiny_model(ctx, layers, max_ctx=8, seed=0):
    """Llama model of hidden 8, 2 query heads / 1 kv head of head_dim 4 (kv_dim 4), FFN 8, vocab 16,
    F32 weights."""
    d = N.ModelDesc()
    d.arch, d.n_layers, d.hidden, d.ffn, d.n_heads, d.n_kv_heads = N.ARCH_LLAMA, layers, 8, 8, 2, 1
    d.head_dim, d.vocab, d.max_ctx = 4, 16, max_ctx
    d.rope_base, d.rope_scale, d.rope_scaled = 10000.0, 1.0, 0
    d.norm_eps, d.attn_scale = 1e-5, 0.5
    d.attn_softcap = d.final_softcap = 0.0
    d.sliding_window = 0x7FFFFFFF
    rng = np.random.default_rng(seed)
    m = F.Model(ctx, d)
    shapes = {N.SLOT_TOKEN_EMBD: 16 * 8, N.SLOT_OUTPUT_NORM: 8, N.SLOT_OUTPUT: 16 * 8}
    per_layer = {N.SLOT_ATTN_NORM: 8, N.SLOT_ATTN_Q: 8 * 8, N.SLOT_ATTN_K: 4 * 8, N.SLOT_ATTN_V: 4 * 8,
                 N.SLOT_ATTN_OUTPUT: 8 * 8, N.SLOT_FFN_NORM: 8, N.SLOT_FFN_GATE: 8 * 8, N.SLOT_FFN_UP: 8 * 8,
                 N.SLOT_FFN_DOWN: 8 * 8}
    for slot, n in shapes.items():
        m.upload(slot, 0, N.F32, (rng.standard_normal(n) * 0.3).astype(np.float32))
    for l in range(layers):
        for slot, n in per_layer.items():
            m.upload(slot, l, N.F32, (rng.standard_normal(n) * 0.3).astype(np.float32))
    m.finalize()
    return m


@pytest.fixture
def model2(ctx):
    m = tiny_model(ctx, 2)
    yield m
    m.close()


@pytest.fixture
def model1(ctx):
    m = tiny_model(ctx, 1)
    yield m
    m.close()


def test_constructor_initializes_current_length_to_zero(model2):
    with F.HipKvCache(model2, 8) as cache:
        assert cache.current_length == 0 and cache.max_sequence_length == 8 and not cache.was_evicted


def test_constructor_negative_max_seq_throws(model2):
    # KvCacheTests.Constructor_NegativeMaxSeq_Throws: a capacity of 0 selects the model's
    # context length here (the KV factory's argument), so the rejected value is negative
    with pytest.raises(F.ArgumentOutOfRangeException):
        F.HipKvCache(model2, -1)


def test_append_last_layer_increments_current_length(model2):
    with F.HipKvCache(model2, 8) as cache:
        k = np.array([1, 2, 3, 4], np.float32)
        v = np.array([5, 6, 7, 8], np.float32)
        cache.append(0, k, v)
        assert cache.current_length == 0
        cache.append(1, k, v)
        assert cache.current_length == 1


def test_append_wrong_slice_length_throws(model2):
    with F.HipKvCache(model2, 8) as cache:
        with pytest.raises(F.ArgumentException):
            cache.append(0, np.zeros(3, np.float32), np.zeros(4, np.float32))
        with pytest.raises(F.ArgumentException):
            cache.append(0, np.zeros(4, np.float32), np.zeros(5, np.float32))
        assert cache.current_length == 0


def test_append_layer_range_and_order(model2):
    with F.HipKvCache(model2, 8) as cache:
        s = np.ones(4, np.float32)
        with pytest.raises(F.ArgumentOutOfRangeException):
            cache.append(2, s, s)
        with pytest.raises(F.ArgumentOutOfRangeException):
            cache.append(-1, s, s)
        with pytest.raises(F.InvalidOperationException):
            cache.append(1, s, s)  # layer 0 comes first
        cache.append(0, s, s)
        with pytest.raises(F.InvalidOperationException):
            cache.append(0, s, s)  # layer 1 expected
        # range is checked before order, order before lengths (KvCache.cs:63-80)
        with pytest.raises(F.ArgumentOutOfRangeException):
            cache.append(5, np.ones(3, np.float32), s)
        with pytest.raises(F.InvalidOperationException):
            cache.append(0, np.ones(3, np.float32), s)


def test_get_keys_and_values_return_appended_values(ctx):
    m = tiny_model(ctx, 1, max_ctx=4)
    try:
        with F.HipKvCache(m, 4) as cache:
            cache.append(0, [1, 2, 3, 10], [4, 5, 6, 11])
            keys = cache.get_keys(0)
            assert keys.tolist() == [1, 2, 3, 10]
            cache.clear()
            cache.append(0, [1, 2, 3, 10], [7, 8, 9, 12])
            vals = cache.get_values(0)
            assert vals.size == 4 and vals[0] == 7
    finally:
        m.close()


def test_get_keys_after_two_appends_has_correct_length(model1):
    with F.HipKvCache(model1, 8) as cache:
        s = np.array([1, 2, 3, 4], np.float32)
        cache.append(0, s, s)
        cache.append(0, s, s)
        assert cache.get_keys(0).size == 2 * 4


def test_effective_length_counts_layers_appended_this_position(model2):
    # GetKeys of a layer already appended at the position being filled holds one more row
    # (KvCache.cs:109-115)
    with F.HipKvCache(model2, 8) as cache:
        a = np.arange(4, dtype=np.float32)
        cache.append(0, a, -a)
        cache.append(1, a + 10, -a - 10)
        cache.append(0, a + 20, -a - 20)
        assert cache.current_length == 1
        assert cache.get_keys(0).tolist() == list(a) + list(a + 20)
        assert cache.get_values(0).tolist() == list(-a) + list(-a - 20)
        assert cache.get_keys(1).tolist() == list(a + 10)
        with pytest.raises(F.ArgumentOutOfRangeException):
            cache.get_keys(2)


def test_clear_resets_current_length_and_allows_reuse_after_full(model1):
    with F.HipKvCache(model1, 4) as cache:
        s = np.array([1, 2, 3, 4], np.float32)
        cache.append(0, s, s)
        assert cache.current_length == 1
        cache.clear()
        assert cache.current_length == 0
    with F.HipKvCache(model1, 1) as cache:
        cache.append(0, s, s)
        cache.clear()
        cache.append(0, s, s)
        assert cache.current_length == 1


def test_dispose_prevents_further_use(model2):
    cache = F.HipKvCache(model2, 8)
    cache.dispose()
    with pytest.raises(F.ObjectDisposedException):
        cache.append(0, np.zeros(4, np.float32), np.zeros(4, np.float32))
    with pytest.raises(F.ObjectDisposedException):
        cache.get_keys(0)
    with pytest.raises(F.ObjectDisposedException):
        cache.clear()


def evict_restated(rows, cap):
    """KvCache.EvictOldestHalf (KvCache.cs:152-173) on a list of cap rows: [keep, cap) moves to
    [0, cap - keep), the rest is cleared, the length becomes keep = cap // 2."""
    keep = cap // 2
    moved = rows[keep:] + [np.zeros_like(rows[0])] * keep
    return moved, keep


@pytest.mark.parametrize("cap", [4, 5, 1, 2])
def test_full_cache_evicts_oldest_half(ctx, cap):
    m = tiny_model(ctx, 2, max_ctx=8)
    try:
        with F.HipKvCache(m, cap) as cache:
            rows, length = [], 0
            for p in range(cap + 3):
                k = np.full(4, 100 + p, np.float32) + np.arange(4, dtype=np.float32)
                v = -k
                if length >= cap:
                    rows, length = evict_restated(rows, cap)
                for layer in range(2):
                    cache.append(layer, k + 1000 * layer, v - 1000 * layer)
                    if layer == 0:
                        # layer 0 holds the new row already, layer 1 not yet
                        assert cache.get_keys(0).size == 4 * (length + 1)
                        assert cache.get_keys(1).size == 4 * length
                rows = rows[:length] + [k] + rows[length + 1:]
                length += 1
                assert cache.current_length == length
                assert cache.was_evicted == (p >= cap)
                want = np.concatenate(rows[:length])
                assert np.array_equal(cache.get_keys(0), want)
                assert np.array_equal(cache.get_values(0), -want)
                assert np.array_equal(cache.get_keys(1), want + 1000)
                assert np.array_equal(cache.get_values(1), -want - 1000)
            cache.clear()
            assert cache.current_length == 0 and not cache.was_evicted
    finally:
        m.close()


def test_forward_requires_a_complete_position(model2):
    with F.HipKvCache(model2, 8) as cache:
        fwd = F.HipForwardPass(model2)
        cache.append(0, np.ones(4, np.float32), np.ones(4, np.float32))
        with pytest.raises(F.InvalidOperationException):
            fwd.forward(1, 0, cache)
        with pytest.raises(F.InvalidOperationException):
            fwd.prefill([1, 2, 3], 0, cache)
        with pytest.raises(F.InvalidOperationException):
            fwd.decode_greedy(1, 0, 2, cache)
        cache.append(1, np.ones(4, np.float32), np.ones(4, np.float32))
        fwd.forward(1, 1, cache)
        assert cache.current_length == 2
        with pytest.raises(F.ArgumentException):
            fwd.forward(1, 0, object())


def test_forward_keys_appended_by_host_match_oracle(ctx):
    """A forward pass over positions whose K/V rows were appended from the host (the path of a C#
    forward pass filling HipKvCache) reads them like its own."""
    cfg, desc, tensors = synthetic("test-llama")
    m = F.Model(ctx, desc)
    upload(m, tensors)
    orc = O.OracleModel(desc, tensors, 16)
    try:
        with F.HipKvCache(m, 16) as kv:
            fwd = F.HipForwardPass(m)
            toks = [5, 9, 2, 7]
            for p, t in enumerate(toks):
                assert orc.forward(t, p) == 0
            # copy the oracle's rows into the device cache through Append, then continue on the device
            K = [orc.kv(l, 0).reshape(len(toks), -1) for l in range(desc.n_layers)]
            Vv = [orc.kv(l, 1).reshape(len(toks), -1) for l in range(desc.n_layers)]
            for p in range(len(toks)):
                for l in range(desc.n_layers):
                    kv.append(l, K[l][p], Vv[l][p])
            assert kv.current_length == len(toks)
            for p in range(len(toks), len(toks) + 5):
                assert orc.forward(11 + p, p) == 0
                fwd.forward(11 + p, p, kv)
                assert O.normwise_rel_err(fwd.logits, orc.logits()) <= 1e-3
    finally:
        orc.close()
        m.close()


def test_forward_eviction_matches_oracle(ctx):
    """Forward on a full cache evicts the oldest half first (KvCache.cs:82-85) and then attends over
    the kept positions when `position` is within them; a position past them fails after layer 0's
    append, leaving the cache expecting layer 1, as in the oracle (which restates the reference)."""
    cfg, desc, tensors = synthetic("test-llama")
    cap = 7
    m = F.Model(ctx, desc)
    upload(m, tensors)
    orc = O.OracleModel(desc, tensors, cap)
    try:
        with F.HipKvCache(m, cap) as kv:
            fwd = F.HipForwardPass(m)
            for p in range(cap):
                assert orc.forward(20 + p, p) == 0
                fwd.forward(20 + p, p, kv)
            assert kv.current_length == cap and not kv.was_evicted
            # full: keep = 3 positions, the new row goes to slot 3, attention over positions [0, 2]
            for tok, pos in [(40, 2), (41, 4)]:
                assert orc.forward(tok, pos) == 0
                fwd.forward(tok, pos, kv)
                assert O.normwise_rel_err(fwd.logits, orc.logits()) <= 1e-3
            assert kv.was_evicted and kv.current_length == 5 == O.lib.orc_fwd_length(orc.f)
            for l in range(desc.n_layers):
                assert O.normwise_rel_err(kv.get_keys(l), orc.kv(l, 0)) <= 1e-3
                assert O.normwise_rel_err(kv.get_values(l), orc.kv(l, 1)) <= 1e-3
            # a position past the cached ones: both fail, both are left expecting layer 1
            assert orc.forward(42, 6) == -1
            with pytest.raises(F.ArgumentOutOfRangeException):
                fwd.forward(42, 6, kv)
            assert kv.current_length == 5
            n0 = C.c_int32()
            F._check(N.dev.fllm_kv_length(kv.h, 0, C.byref(n0)))
            assert n0.value == 6 and kv.get_keys(1).size == 5 * m.desc.n_kv_heads * m.desc.head_dim
            assert orc.forward(43, 5) == -3
            with pytest.raises(F.InvalidOperationException):
                fwd.forward(43, 5, kv)
            kv.clear()
            O.lib.orc_fwd_reset(orc.f)
            assert orc.forward(44, 0) == 0
            fwd.forward(44, 0, kv)
            assert O.normwise_rel_err(fwd.logits, orc.logits()) <= 1e-3
    finally:
        orc.close()
        m.close()


def test_failed_forward_clears_layer0_row_after_reset(model2):
    """A Forward at a position past the cache fails after layer 0's append (the cache then expects
    layer 1); the row it leaves at that slot reads as zeros, also when an earlier use of the cache
    had written that slot before a reset."""
    with F.HipKvCache(model2, 8) as cache:
        fwd = F.HipForwardPass(model2)
        for p in range(3):
            fwd.forward(1 + p, p, cache)
        assert np.any(cache.get_keys(0)[:4] != 0) and np.any(cache.get_values(0)[:4] != 0)
        cache.clear()
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.forward(5, 1, cache)
        k, v = cache.get_keys(0), cache.get_values(0)
        assert k.size == 4 and v.size == 4  # one effective row (kv_dim 4) in layer 0
        assert np.all(k == 0) and np.all(v == 0)
        assert cache.get_keys(1).size == 0


@pytest.mark.parametrize("debug", [False, True], ids=["batched", "stepwise"])
def test_prefill_overflow_leaves_cache_unchanged(ctx, debug):
    """fllm_prefill checks the capacity before anything runs on both of its paths (the batched
    prefill, and the per-token Forward calls that debug capture selects): a prompt longer than the
    room left returns ArgumentOutOfRange with the length and the rows unchanged, no eviction."""
    cfg, desc, tensors = synthetic("test-llama")
    m = F.Model(ctx, desc)
    upload(m, tensors)
    try:
        with F.HipKvCache(m, 16) as kv:
            F.set_debug(kv, debug)
            fwd = F.HipForwardPass(m)
            toks = F.synth_tokens(3, 0, desc.vocab, 17)
            fwd.prefill(toks[:10], 0, kv)
            assert kv.current_length == 10
            keys = [kv.get_keys(l).copy() for l in range(desc.n_layers)]
            with pytest.raises(F.ArgumentOutOfRangeException):
                fwd.prefill(toks[10:17], 10, kv)
            assert kv.current_length == 10 and not kv.was_evicted
            for l in range(desc.n_layers):
                assert np.array_equal(kv.get_keys(l), keys[l])
            fwd.prefill(toks[10:16], 10, kv)  # exactly the room left
            assert kv.current_length == 16
    finally:
        m.close()


def test_disposed_weights(ctx):
    """LlamaWeights.Dispose + ThrowIfDisposed (LlamaWeights.cs:93-107, 138-139): after the model is
    destroyed, Forward / prefill / decode on its sequences throw ObjectDisposedException before
    anything runs, the cache itself stays usable, and the weights are released with the last
    sequence (no use after free)."""
    m = tiny_model(ctx, 2)
    raw = m.h
    kv = F.HipKvCache(m, 8)
    kv2 = F.HipKvCache(m, 8)
    fwd = F.HipForwardPass(m)
    fwd.forward(3, 0, kv)
    m.close()  # fllm_model_destroy with two live sequences
    assert N.dev.fllm_model_destroy(raw) == N.OK  # idempotent
    with pytest.raises(F.ObjectDisposedException):
        fwd.forward(4, 1, kv)
    with pytest.raises(F.ObjectDisposedException):
        fwd.prefill([4, 5, 6], 1, kv)
    with pytest.raises(F.ObjectDisposedException):
        fwd.decode_greedy(4, 1, 3, kv)
    assert kv.current_length == 1  # nothing ran
    h = C.c_void_p()
    assert N.dev.fllm_seq_create(raw, 8, C.byref(h)) == N.E_DISPOSED
    assert N.dev.fllm_model_finalize(raw) == N.E_DISPOSED
    kv.append(0, np.ones(4, np.float32), np.ones(4, np.float32))  # the cache is not the weights
    kv.append(1, np.ones(4, np.float32), np.ones(4, np.float32))
    assert kv.current_length == 2 and kv.get_keys(0).size == 8
    kv.close()
    with pytest.raises(F.ObjectDisposedException):
        fwd.forward(4, 0, kv2)
    kv2.close()  # the last sequence releases the weights
    # a new model on the same context works as before
    m2 = tiny_model(ctx, 2, seed=1)
    try:
        with F.HipKvCache(m2, 8) as kv3:
            F.HipForwardPass(m2).forward(3, 0, kv3)
            assert kv3.current_length == 1
    finally:
        m2.close()
