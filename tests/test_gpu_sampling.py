"""GPU parity of the device sampling stages against the oracle.

- Repetition penalty (LlamaLanguageModel.ApplyRepetitionPenalty, LlamaLanguageModel.cs:357-373) on
  the device logits: bit-identical to the oracle's list-order loop.
- Nucleus sampler (SamplerPipeline.Sample with topK off: temperature, softmax, top-p, draw;
  SamplerPipeline.cs:58-89, TopPSampler.cs:60-110, TemperatureSampler.cs:53-70): a top set of the
  softmax whose mass is the smallest reaching top_p, the same nucleus as the oracle's except where
  its mass is within rounding of top_p, the same distribution up to the oracle's f32 normalisation
  (relative 2e-6 after renormalising both), the draw where u falls in the device's running sum,
  and the oracle's token except where u lies within the oracle's f32 summation error of a CDF
  boundary (the device sums exactly; the oracle, like the reference's loops, in f32 order).
- Top-k on the device then top-p over the survivors on the host: bit-exact.
- The greedy token loop with a repetition penalty, against the oracle's loop.
"""
import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import oracle_bind as O
from fixtures import synthetic, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def big_vocab(ctx):
    """One layer of the tiny Llama shape (vocab 32000, not a multiple of the sampler's 1024 threads)."""
    cfg, desc, tensors = synthetic("tiny-llama-q4k", n_layers=1)
    m = F.Model(ctx, desc)
    upload(m, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    fwd.forward(1, 0, kv)
    yield desc, m, kv, fwd
    kv.close()
    m.close()


def _inv_temp(temp):
    """1f / temperature in float32, as SamplerPipeline.cs:69 computes it."""
    return np.float32(1.0) / np.float32(temp) if temp != 1.0 else np.float32(1.0)


def _oracle_probs(lg, temp, top_p):
    a = lg.astype(np.float32).copy()
    if temp != 1.0:
        a = a * _inv_temp(temp)
    a = np.ascontiguousarray(a, dtype=np.float32)
    O.lib.orc_softmax(O.fp(a), a.size)
    return O.apply_top_p(a, top_p)


def test_repetition_penalty_bit_exact(big_vocab):
    desc, m, kv, fwd = big_vocab
    rng = np.random.default_rng(21)
    V = desc.vocab
    for trial, penalty in enumerate((1.3, 0.8, 3.0, 1.1)):
        lg = (rng.standard_normal(V) * 4).astype(np.float32)
        lg[rng.integers(0, V, 50)] = 0.0  # zero takes the multiply branch
        n_ids = (7, 600, 3000, 1)[trial]
        ids = rng.integers(0, 200 if trial == 2 else V, n_ids).astype(np.int32)  # trial 2: many repeats
        ids[::97] = -5  # out of range entries are skipped
        ids[1::101] = V + 3
        for _ in range(2):  # twice: the counters are left zeroed for the next call
            fwd.write_logits(lg)
            fwd.penalize(ids, penalty)
            got = fwd.logits
            want = O.repetition_penalty(lg, ids, penalty)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    fwd.write_logits(lg)
    fwd.penalize(ids, 1.0)
    assert np.array_equal(fwd.logits, lg)
    with pytest.raises(F.ArgumentOutOfRangeException):
        fwd.penalize(ids, 0.0)
    with pytest.raises(F.ArgumentOutOfRangeException):
        fwd.penalize(ids, -1.5)


def _check_draw(p, u, tok):
    """tok is where u falls in the running sum of p (float64), up to 1e-6."""
    assert p[tok] > 0
    cdf = np.cumsum(p.astype(np.float64))
    lo = cdf[tok - 1] if tok > 0 else 0.0
    assert lo <= u + 1e-6 and u < cdf[tok] + 1e-6, (tok, u, lo, cdf[tok])


@pytest.mark.parametrize("temp,top_p", [(1.0, 1.0), (0.8, 1.0), (0.8, 0.9), (1.0, 0.5), (1.5, 0.95), (0.7, 0.05)])
def test_nucleus_matches_oracle(big_vocab, temp, top_p):
    desc, m, kv, fwd = big_vocab
    rng = np.random.default_rng(int(temp * 100 + top_p * 1000))
    r_dev, r_orc = O.Xoshiro(77), O.Xoshiro(77)
    sp = F.SamplerPipeline(temp, 0, top_p, 77)  # the host pipeline draws the same u
    inv = _inv_temp(temp)
    same_nucleus = ambiguous = 0
    try:
        for j in range(30):
            lg = (rng.standard_normal(desc.vocab) * (3.0 if j % 3 else 0.3)).astype(np.float32)
            if j % 5 == 1:
                lg = np.round(lg, 1)  # many equal probabilities, also at the nucleus edge
            sm = _oracle_probs(lg, temp, 1.0)
            want_p = O.apply_top_p(sm, top_p)
            u = r_dev.next_float()
            fwd.write_logits(lg)
            tok = fwd.sample_nucleus(float(inv), top_p, u)
            got_p = fwd.probs()
            if inv != 1.0:  # the scaled logits stay in place, as in the reference
                assert np.array_equal(fwd.logits, lg * inv)
            fwd.write_logits(lg)
            assert sp.sample(kv) == tok
            _check_draw(got_p, u, tok)
            kd, ko = got_p > 0, want_p > 0
            # the device nucleus is a top set of the softmax, minimal for top_p
            if (~kd).any():
                assert sm[kd].min() >= sm[~kd].max()
            # masses of the oracle's softmax renormalised in float64 (its f32 sum is off by ~1e-5)
            sm64 = sm.astype(np.float64) / np.sum(sm, dtype=np.float64)
            if top_p < 1.0:
                mass = float(sm64[kd].sum())
                assert mass >= top_p - 5e-6 and mass - float(sm64[kd].min()) < top_p + 5e-6
            else:
                assert kd.all() or np.all(sm[~kd] == 0)
            ref_tok = O.sampler_pipeline_p(lg, temp, 0, top_p, r_orc)
            if np.array_equal(kd, ko):
                same_nucleus += 1
                # the oracle's sequential f32 sums over 32000 terms drift by up to 32000 * 2^-24 of
                # the total (a common factor; the device's tree sum is within 1e-7); the shapes agree
                # to float32 exp rounding
                g64, w64 = got_p.astype(np.float64), want_p.astype(np.float64)
                assert abs(g64.sum() - 1.0) < 1e-6
                np.testing.assert_allclose(g64 / g64.sum(), w64 / w64.sum(), rtol=2e-6, atol=1e-15)
                if tok != ref_tok:  # only where u sits on a boundary of the oracle's running sum,
                    # within the worst-case drift of its f32 sums (n terms: n * 2^-24 of the total)
                    cdf = np.cumsum(w64)
                    k = min(tok, ref_tok)
                    assert abs(cdf[k] - u) < 2.0 * desc.vocab * 2.0**-24, (j, tok, ref_tok, u)
                    ambiguous += 1
            else:
                # the oracle sums the sorted probabilities in f32 order, the device exactly: the two
                # nuclei are nested, and the oracle's is minimal for top_p within the worst-case drift
                # of its sums (softmax over the vocabulary, then the walk over its kept entries)
                small, big = (kd, ko) if kd.sum() < ko.sum() else (ko, kd)
                assert not (small & ~big).any()
                drift = (desc.vocab + int(ko.sum())) * 2.0**-24
                mo = float(sm64[ko].sum())
                assert mo >= top_p - drift and mo - float(sm64[ko].min()) < top_p + drift
        assert ambiguous <= 12  # flat draws (a third of them) have boundaries ~3e-5 apart
        assert same_nucleus >= 8  # near-flat draws over 32000 entries often end a few entries apart
    finally:
        sp.close()


def test_topk_then_top_p_matches_oracle(big_vocab):
    """Top-k on the device, softmax / top-p / draw over the survivors on the host: bit-exact."""
    desc, m, kv, fwd = big_vocab
    rng = np.random.default_rng(3)
    for temp, k, top_p in ((0.8, 40, 0.9), (1.0, 200, 0.5), (1.2, 5, 0.99)):
        sp = F.SamplerPipeline(temp, k, top_p, 99)
        r = O.Xoshiro(99)
        try:
            for j in range(25):
                lg = np.round(rng.standard_normal(desc.vocab) * 2, 2).astype(np.float32)
                fwd.write_logits(lg)
                assert sp.sample(kv) == O.sampler_pipeline_p(lg, temp, k, top_p, r)
        finally:
            sp.close()


def test_nucleus_edge_cases(big_vocab):
    desc, m, kv, fwd = big_vocab
    V = desc.vocab
    # one dominant token: every top_p keeps only it, every u draws it
    lg = np.zeros(V, dtype=np.float32)
    lg[12345] = 80.0
    for top_p, u in ((0.5, 0.0), (0.999, 0.9999), (1.0, 0.5)):
        fwd.write_logits(lg)
        assert fwd.sample_nucleus(1.0, top_p, u) == 12345
    # uniform logits: all probabilities equal, the nucleus is the first indices in order
    lg = np.full(V, 0.25, dtype=np.float32)
    fwd.write_logits(lg)
    fwd.sample_nucleus(1.0, 0.00101, 0.5)  # 32.3 entries' mass: the edge is unambiguous
    p = fwd.probs()
    want = _oracle_probs(lg, 1.0, 0.00101)
    assert np.array_equal(p > 0, want > 0) and int((p > 0).sum()) == int((want > 0).sum())
    assert np.nonzero(p)[0].max() == int((want > 0).sum()) - 1  # ties taken by ascending index
    # u just below 1 with top_p 1: the last index (the reference's fallback when rounding leaves
    # the running sum below u picks the last nonzero probability)
    fwd.write_logits(lg)
    assert fwd.sample_nucleus(1.0, 1.0, float(np.nextafter(np.float32(1), np.float32(0)))) in (V - 1, V - 2)
    # (inv_temp 0 is an infinite temperature, accepted: test_inverse_temperature_contract)
    for bad in ((1.0, 0.0, 0.5), (1.0, 1.1, 0.5), (1.0, 0.9, 1.0), (1.0, 0.9, -0.1), (-1.0, 0.9, 0.5)):
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.sample_nucleus(*bad)


def _oracle_loop(orc, prompt, n, temp, top_k, top_p, seed, penalty):
    pos = 0
    for t in prompt[:-1]:
        assert orc.forward(int(t), pos) == 0
        pos += 1
    r = O.Xoshiro(seed)
    nxt, out = int(prompt[-1]), []
    for _ in range(n):
        assert orc.forward(nxt, pos) == 0
        pos += 1
        lg = orc.logits().copy()
        if penalty != 1.0:
            lg = O.repetition_penalty(lg, np.array(out, dtype=np.int32), penalty)
        nxt = O.sampler_pipeline_p(lg, temp, top_k, top_p, r)
        out.append(nxt)
    return out


@pytest.mark.parametrize("penalty", [1.3, 0.7])
def test_token_loop_with_repetition_penalty(ctx, penalty):
    """Greedy loop with a repetition penalty (the sampled loops cannot be compared token for token:
    the model's logits agree with the oracle's to 1e-3, not bit for bit)."""
    cfg, desc, tensors = synthetic("test-llama")
    m = F.Model(ctx, desc)
    upload(m, tensors)
    kv = F.HipKvCache(m)
    orc = O.OracleModel(desc, tensors)
    prompt = F.synth_tokens(cfg["seed"], 3, desc.vocab, 20)
    lm = F.LlamaLanguageModel(m, kv)
    sampler = F.SamplerPipeline(0.0, 0, 1.0, 4242)
    try:
        toks, stats = lm.generate(prompt, 24, sampler, stop_at_eos=False, repetition_penalty=penalty)
        assert stats.completion_tokens == 24
        assert list(toks) == _oracle_loop(orc, prompt, 24, 0.0, 0, 1.0, 4242, penalty)
    finally:
        sampler.close()
        orc.close()
        kv.close()
        m.close()


def test_topk_sample_select_and_fallback(big_vocab):
    """Top-k over the 32000 vocabulary: the sample-select path (a threshold from 2048 evenly spaced
    entries, then an exact select among the entries reaching it) and both of its fallbacks to the
    full radix select (too few entries reach the sample's threshold; too many, with all logits
    equal) give the oracle's survivors, ties kept, in index order; k up to 256 returns through the
    sequence's pinned result block, k = 300 through the caller's arrays."""
    desc, m, kv, fwd = big_vocab
    V = desc.vocab
    rng = np.random.default_rng(17)
    sampled = (np.arange(2048, dtype=np.int64) * V) // 2048
    cases = []
    lg = rng.standard_normal(V).astype(np.float32)
    cases.append((lg, 40))
    lg = lg.copy()
    # the sample's top is the array's top: its 18th largest (the threshold for k = 40 over 32000)
    # is reached by 18 entries only, fewer than k
    lg[sampled[:30]] = 100.0 + np.arange(30, dtype=np.float32)
    cases.append((lg, 40))
    cases.append((np.full(V, 0.5, dtype=np.float32), 40))  # every entry ties
    lg = np.round(rng.standard_normal(V) * 2, 1).astype(np.float32)
    cases.append((lg, 256))
    cases.append((lg, 300))  # more candidates than the pinned result block holds
    cases.append((lg, 1))
    for lg, k in cases:
        for inv in (1.0, 1.25):
            fwd.write_logits(lg)
            ids, vals = fwd.sample_topk(inv, k, cap=V)
            scaled = lg * np.float32(inv) if inv != 1.0 else lg.copy()
            ref = scaled.copy()
            O.lib.orc_apply_topk(O.fp(ref), ref.size, k)
            keep = np.nonzero(ref != -np.inf)[0]
            assert np.array_equal(ids, keep)
            assert np.array_equal(vals, scaled[keep])
            assert np.array_equal(fwd.logits, scaled)


def test_nucleus_and_topk_small_vocab(ctx):
    """A vocabulary of 512 (one partly filled 4096-entry segment; top-k takes the one-workgroup
    select): the nucleus is the oracle's where its edge is unambiguous, the draw sits where u falls
    in the device's running sum, and top-k survivors are bit-exact."""
    cfg, desc, tensors = synthetic("test-llama")
    m = F.Model(ctx, desc)
    upload(m, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    fwd.forward(1, 0, kv)
    rng = np.random.default_rng(8)
    r = O.Xoshiro(5)
    try:
        for j in range(40):
            lg = (rng.standard_normal(desc.vocab) * 2).astype(np.float32)
            temp, top_p = (0.8, 0.9) if j % 2 else (1.0, 1.0)
            sm = _oracle_probs(lg, temp, 1.0)
            want = O.apply_top_p(sm, top_p)
            u = r.next_float()
            fwd.write_logits(lg)
            tok = fwd.sample_nucleus(float(_inv_temp(temp)), top_p, u)
            got = fwd.probs()
            _check_draw(got, u, tok)
            drift = 2 * desc.vocab * 2.0**-24
            kd, ko = got > 0, want > 0
            if not np.array_equal(kd, ko):  # only at an edge within the oracle's f32 drift
                sm64 = sm.astype(np.float64) / np.sum(sm, dtype=np.float64)
                assert abs(float(sm64[kd & ko].sum()) - top_p) < drift + float(sm64[kd ^ ko].max())
            else:
                np.testing.assert_allclose(got.astype(np.float64) / got.sum(dtype=np.float64),
                                           want.astype(np.float64) / want.sum(dtype=np.float64), rtol=2e-6, atol=1e-15)
            fwd.write_logits(lg)
            ids, vals = fwd.sample_topk(1.0, 7, cap=desc.vocab)
            ref = lg.copy()
            O.lib.orc_apply_topk(O.fp(ref), ref.size, 7)
            keep = np.nonzero(ref != -np.inf)[0]
            assert np.array_equal(ids, keep) and np.array_equal(vals, lg[keep])
    finally:
        kv.close()
        m.close()


def test_topk_at_qwen2_vocabulary(ctx):
    """Top-k 40 at temperature 0.8 over the Qwen2-7B vocabulary (152064 entries, 38 segments of the
    grid sampler, the last one partly filled): survivors bit-exact with the oracle's ApplyTopK on
    the scaled logits, and SamplerPipeline(0.8, 40, 1.0, seed) draws the oracle pipeline's tokens
    with the same XoshiroRandom stream, on the model's own logits and on synthetic ones."""
    cfg, desc, tensors = synthetic("test-qwen2-v152k")
    assert desc.vocab == 152064
    m = F.Model(ctx, desc)
    upload(m, tensors)
    kv = F.HipKvCache(m)
    fwd = F.HipForwardPass(m)
    rng = np.random.default_rng(152064)
    inv = float(_inv_temp(0.8))
    try:
        cases = []
        for p, t in enumerate((5, 151999, 77)):
            fwd.forward(t, p, kv)
            cases.append(fwd.logits)
        cases.append(rng.standard_normal(desc.vocab).astype(np.float32))
        lg = np.round(rng.standard_normal(desc.vocab) * 3, 1).astype(np.float32)  # many ties at the edge
        cases.append(lg)
        lg = lg.copy()
        lg[-5:] = 50.0  # the top entries in the partly filled last segment
        cases.append(lg)
        for lg in cases:
            fwd.write_logits(lg, kv)
            ids, vals = fwd.sample_topk(inv, 40, cap=desc.vocab)
            scaled = lg * np.float32(inv)
            ref = scaled.copy()
            O.lib.orc_apply_topk(O.fp(ref), ref.size, 40)
            keep = np.nonzero(ref != -np.inf)[0]
            assert np.array_equal(ids, keep) and np.array_equal(vals, scaled[keep])
        sp = F.SamplerPipeline(0.8, 40, 1.0, 0x5EED)
        r = O.Xoshiro(0x5EED)
        try:
            for lg in cases * 4:
                fwd.write_logits(lg, kv)
                assert sp.sample(kv) == O.sampler_pipeline_p(lg, 0.8, 40, 1.0, r)
        finally:
            sp.close()
    finally:
        kv.close()
        m.close()


def test_topk_signed_zero_threshold(big_vocab):
    """TopKSampler compares floats (TopKSampler.cs:55-60, 93-105), so -0 and +0 tie: when the k-th
    largest value is a zero, every zero of either sign survives, as in the oracle."""
    desc, m, kv, fwd = big_vocab
    V = desc.vocab
    rng = np.random.default_rng(40)
    for k, neg_first in ((40, True), (40, False), (7, True)):
        lg = -np.abs(rng.standard_normal(V)).astype(np.float32) - 1.0
        lg[rng.choice(V, k // 2, replace=False)] = 5.0
        zeros = rng.choice(np.nonzero(lg < 0)[0], 300, replace=False)
        lg[zeros] = 0.0
        lg[zeros[::2]] = -0.0
        if neg_first:
            lg[zeros.min()] = -0.0
        else:
            lg[zeros.min()] = 0.0
        fwd.write_logits(lg)
        ids, vals = fwd.sample_topk(1.0, k, cap=V)
        ref = lg.copy()
        O.lib.orc_apply_topk(O.fp(ref), ref.size, k)
        keep = np.nonzero(ref != -np.inf)[0]
        assert keep.size == k // 2 + 300
        assert np.array_equal(ids, keep)
        assert np.array_equal(vals.view(np.uint32), lg[keep].view(np.uint32))


def test_inverse_temperature_contract(big_vocab):
    """inv_temp = 1/Temperature (SamplerPipeline.cs:67-70) must be finite and >= 0 on both device
    samplers; 0 (an infinite temperature) makes every logit zero, so top-k keeps every entry and the
    nucleus is the uniform distribution."""
    desc, m, kv, fwd = big_vocab
    V = desc.vocab
    lg = np.random.default_rng(2).standard_normal(V).astype(np.float32)
    for bad in (float("nan"), -1.0, float("inf")):
        fwd.write_logits(lg)
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.sample_topk(bad, 40, cap=V)
        with pytest.raises(F.ArgumentOutOfRangeException):
            fwd.sample_nucleus(bad, 1.0, 0.5)
    fwd.write_logits(lg)
    ids, vals = fwd.sample_topk(0.0, 40, cap=V)
    assert np.array_equal(ids, np.arange(V)) and np.all(vals == 0.0)
    fwd.write_logits(lg)
    tok = fwd.sample_nucleus(0.0, 1.0, 0.6180339)
    got = fwd.probs()
    assert np.all(got == got[0]) and abs(float(got.sum(dtype=np.float64)) - 1.0) < 1e-5
    assert abs(tok - int(0.6180339 * V)) <= 1
    sp = F.SamplerPipeline(float("inf"), 0, 1.0, 7)
    try:
        fwd.write_logits(lg)
        tok = sp.sample(kv)
        assert 0 <= tok < V
    finally:
        sp.close()
