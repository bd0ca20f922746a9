"""Pins the oracle's tensor operations, sampling and RNG (CPU only).

Reference tests restated: TensorOperationsTests.cs:9-107, GreedySamplerTests.cs,
TopKSamplerTests.cs:45-71, SamplerPipelineTests.cs:24-70, TopPSamplerTests.cs,
RepetitionPenaltySamplerTests.cs. Beyond those: closed forms
(RoPE at position 0 is the identity and preserves pair norms; softcap(x) -> x for |x| << cap;
GELU/SiLU fixed points), float64 brute force for Dot/LinearProjection, numpy's order
statistic for the top-k threshold, and published known answers of SplitMix64 and
xoshiro256** for the RNG.
"""
import math

import numpy as np
import pytest

import oracle_bind as O

fp = O.fp


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def test_dot_and_linear_against_float64():
    assert O.lib.orc_dot(fp(f32([1, 2, 3])), fp(f32([4, 5, 6])), 3) == 32.0  # TensorOperationsTests Dot
    rng = np.random.default_rng(0)
    for n in (1, 7, 8, 9, 64, 1000, 4097):
        a, b = f32(rng.standard_normal(n)), f32(rng.standard_normal(n))
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        got = O.lib.orc_dot(fp(a), fp(b), n)
        bound = n * 2 ** -23 * float(np.dot(np.abs(a), np.abs(b))) + 1e-30
        assert abs(got - exact) <= bound
    W = f32(rng.standard_normal((37, 300)))
    x = f32(rng.standard_normal(300))
    y = O.linear(W, x)
    assert np.allclose(y, W.astype(np.float64) @ x.astype(np.float64), rtol=1e-5, atol=1e-4)


def test_rmsnorm_and_gemma_norm():
    x = f32([1, 2, 3, 4])
    w = f32([1, 1, 1, 1])
    dst = np.zeros(4, dtype=np.float32)
    O.lib.orc_rmsnorm(fp(x), fp(w), fp(dst), 4, 1e-5)
    assert abs(math.sqrt(float(np.mean(dst.astype(np.float64) ** 2))) - 1.0) < 0.01  # TensorOperationsTests
    rng = np.random.default_rng(1)
    x = f32(rng.standard_normal(256) * 3)
    w = f32(rng.standard_normal(256))
    O.lib.orc_rmsnorm(fp(x), fp(w), fp(dst := np.zeros(256, np.float32)), 256, 1e-5)
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    assert np.allclose(dst, ref, rtol=1e-5, atol=1e-6)
    g = np.zeros(256, np.float32)
    O.lib.orc_gemma_rmsnorm(fp(x), fp(w), fp(g), 256)
    refg = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * (1.0 + w)
    assert np.allclose(g, refg, rtol=1e-5, atol=1e-6)
    # Gemma norm applied in place (Gemma2ForwardPass.cs:90 passes the same span twice)
    xi = x.copy()
    O.lib.orc_gemma_rmsnorm(fp(xi), fp(w), fp(xi), 256)
    assert np.array_equal(xi, g)


def test_activations_and_softcap():
    x = f32([100.0])
    O.lib.orc_silu(fp(x), 1)
    assert x[0] > 99.0  # TensorOperationsTests Silu
    z = f32([0.0, -0.0])
    O.lib.orc_silu(fp(z), 2)
    assert np.all(z == 0)
    v = f32(np.linspace(-6, 6, 101))
    s = v.copy()
    O.lib.orc_silu(fp(s), s.size)
    assert np.allclose(s, v / (1 + np.exp(-v.astype(np.float64))), rtol=1e-6, atol=1e-7)
    g = v.copy()
    O.lib.orc_gelu(fp(g), g.size)
    vv = v.astype(np.float64)
    assert np.allclose(g, 0.5 * vv * (1 + np.tanh(0.7978845608 * (vv + 0.044715 * vv ** 3))), rtol=1e-6, atol=1e-7)
    c = f32([1e-3, -2e-3, 1000.0, -1000.0])
    O.lib.orc_softcap(fp(c), 4, 30.0)
    assert abs(c[0] - 1e-3) < 1e-9 and abs(c[1] + 2e-3) < 1e-9 and abs(c[2] - 30) < 1e-5 and abs(c[3] + 30) < 1e-5


def test_softmax():
    x = f32([1, 2, 3, 4])
    O.lib.orc_softmax(fp(x), 4)
    assert abs(float(x.sum()) - 1.0) < 1e-5  # TensorOperationsTests Softmax_SumsToOne
    y = f32([1, 2, 10, 3])
    O.lib.orc_softmax(fp(y), 4)
    assert y[2] == y.max()
    z = f32([-np.inf, 1.0, -np.inf, 1.0])
    O.lib.orc_softmax(fp(z), 4)
    assert list(z) == [0.0, 0.5, 0.0, 0.5]


def test_rope_closed_forms():
    inv = np.zeros(2, dtype=np.float32)
    O.lib.orc_rope_inv_freqs(10000.0, 4, fp(inv))
    assert inv[0] == 1.0 and abs(inv[1] - 0.01) < 1e-9  # 1/10000^(2/4)
    x = f32([1, 0, 1, 0])
    O.lib.orc_apply_rope(fp(x), 1.0, fp(inv), 2)
    assert not np.array_equal(x, f32([1, 0, 1, 0]))  # TensorOperationsTests ApplyRope_ChangesVector
    rng = np.random.default_rng(2)
    hd = 128
    inv = np.zeros(hd // 2, dtype=np.float32)
    O.lib.orc_rope_inv_freqs(500000.0, hd, fp(inv))
    v = f32(rng.standard_normal(hd))
    r0 = v.copy()
    O.lib.orc_apply_rope(fp(r0), 0.0, fp(inv), hd // 2)
    assert np.array_equal(r0, v)  # identity at position 0
    r = v.copy()
    O.lib.orc_apply_rope(fp(r), 37.0, fp(inv), hd // 2)
    pn = np.hypot(v[0::2].astype(np.float64), v[1::2])
    assert np.allclose(np.hypot(r[0::2].astype(np.float64), r[1::2]), pn, rtol=1e-6)
    # interleaved pairs: the first pair rotates by exactly 37 rad
    ang = math.atan2(r[1], r[0]) - math.atan2(v[1], v[0])
    assert abs(math.remainder(ang - 37.0, 2 * math.pi)) < 1e-5


def test_argmax_semantics():
    for logits, want in [([1, 5, 3], 1), ([9, 1, 1], 0), ([1, 1, 9], 2), ([7.0], 0), ([2, 5, 5, 1], 1),
                         ([-0.0, 0.0], 1), ([1, np.nan, 5, np.nan], 1)]:
        a = f32(logits)
        assert O.lib.orc_argmax(fp(a), a.size) == want


def test_topk_threshold_matches_order_statistic():
    a = f32([1, 5, 0.5, 3])
    O.lib.orc_apply_topk(fp(a), 4, 2)  # TopKSamplerTests: keeps indices 1 and 3
    assert a[0] == -np.inf and a[2] == -np.inf and a[1] == 5 and a[3] == 3
    b = f32([1, 2, 3])
    O.lib.orc_apply_topk(fp(b), 3, 10)
    assert list(b) == [1, 2, 3]
    rng = np.random.default_rng(3)
    for n, k in [(100, 1), (1000, 40), (5000, 40), (152064, 40), (64, 64 - 1)]:
        x = f32(np.round(rng.standard_normal(n) * 4, 1))  # many ties
        th = O.lib.orc_topk_threshold(fp(x), n, k)
        assert th == np.sort(x)[::-1][k - 1]


# Published known answers for the two generators XoshiroRandom combines
# (XoshiroRandom.cs:9-44). None of them is computed by code in this repository.
# SplitMix64 from seed 1234567: Rosetta Code, "Pseudo-random numbers/Splitmix64".
SPLITMIX64_1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                      4593380528125082431, 16408922859458223821]
# SplitMix64 from seed 0 (the reference's default seed): the outputs listed with Vigna's
# splitmix64.c and used by Java's SplittableRandom test suites.
SPLITMIX64_0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
# xoshiro256** from the state {1, 2, 3, 4}: the reference vector of the rand_xoshiro crate's
# Xoshiro256StarStar test. The first three follow by hand: rotl(2 * 5, 7) * 9 = 11520; the step
# leaves s1 = 0, so the second is 0; then s1 = 262149 and rotl(262149 * 5, 7) * 9 = 1509978240.
XOSHIRO256SS_1234 = [11520, 0, 1509978240, 1215971899390074240, 1216172134540287360,
                     607988272756665600, 16172922978634559625, 8476171486693032832,
                     10595114339597558777, 2904607092377533576]


def next_float_of(u64):
    """NextFloat's mapping (XoshiroRandom.cs:44) of a known 64-bit output, in exact arithmetic:
    the top 53 bits times 2^-53 is a double without rounding, then one rounding to float."""
    return np.float32(math.ldexp(u64 >> 11, -53))


def test_xoshiro_seeding_is_splitmix64():
    """XoshiroRandom(seed) holds the first four SplitMix64 outputs of the seed as s0..s3."""
    for seed, want in ((1234567, SPLITMIX64_1234567), (0, SPLITMIX64_0)):
        r = O.Xoshiro(seed)
        assert [r.s.s0, r.s.s1, r.s.s2, r.s.s3] == want[:4]


def test_xoshiro256ss_known_answers():
    """The step from an injected state, against the published vector."""
    import ctypes as C
    s = O.OrcXoshiro(1, 2, 3, 4)
    assert [O.lib.orc_xoshiro_next(C.byref(s)) for _ in range(10)] == XOSHIRO256SS_1234
    s = O.OrcXoshiro(1, 2, 3, 4)
    got = [O.lib.orc_xoshiro_next_float(C.byref(s)) for _ in range(10)]
    assert got == [next_float_of(v) for v in XOSHIRO256SS_1234]
    assert got[1] == 0.0 and got[0] == np.float32(5 * 2.0 ** -53)  # 11520 >> 11 = 5


def test_xoshiro_next_float_range_and_rounding():
    """NextFloat lies in [0, 1] (the float rounding of (2^53 - 1) 2^-53 is 1.0f, as in the
    reference), is the float nearest the 53-bit fraction, and the extreme outputs map as the
    closed form says."""
    assert next_float_of(0) == 0.0
    assert next_float_of((1 << 64) - 1) == np.float32(1.0)
    assert next_float_of(1 << 11) == np.float32(2.0 ** -53)
    r = O.Xoshiro(7)
    for _ in range(2000):
        f = r.next_float()
        assert 0.0 <= f <= 1.0


def test_sampler_pipeline_reference_cases():
    rng = O.Xoshiro(5)
    assert O.sampler_pipeline(f32([0.1, 5.0, 3.0]), 0.0, 0, rng) == 1  # temperature 0 -> argmax
    for _ in range(20):
        assert O.sampler_pipeline(f32([1, 10, 0.5, 3]), 1.0, 1, rng) == 1  # top-k 1 -> argmax
    a, b = O.Xoshiro(123), O.Xoshiro(123)
    logits = [0.5, 0.3, 0.9, 0.1]
    assert [O.sampler_pipeline(f32(logits), 1.0, 0, a) for _ in range(50)] == \
           [O.sampler_pipeline(f32(logits), 1.0, 0, b) for _ in range(50)]
    # the draw frequencies follow softmax(logits / T) restricted to the top k
    r = O.Xoshiro(9)
    lg = f32([2.0, 1.0, 0.5, 3.0, -1.0])
    counts = np.zeros(5)
    for _ in range(20000):
        counts[O.sampler_pipeline(lg, 0.8, 3, r)] += 1
    p = np.exp(lg.astype(np.float64) / 0.8)
    p[[2, 4]] = 0
    p /= p.sum()
    assert np.allclose(counts / counts.sum(), p, atol=0.015)


def test_top_p_reference_cases():
    # TopPSamplerTests.cs: ApplyTopP_SmallP_ZeroesOutLowProbTokens
    q = O.apply_top_p(f32([0.02, 0.90, 0.05, 0.03]), 0.91)
    assert q[0] == 0 and q[3] == 0 and q[1] > 0 and q[2] > 0
    # ApplyTopP_RenormalizesRemainingProbabilities
    q = O.apply_top_p(f32([0.1, 0.6, 0.2, 0.1]), 0.8)
    assert abs(float(q.sum()) - 1.0) < 1e-5
    assert q[0] == 0 and q[3] == 0  # 0.6f + 0.2f rounds to 0.8f, which reaches p (>=, not >)
    assert q[1] > 0 and q[2] > 0
    # ApplyTopP_P1_LeavesDistributionUnchanged
    a = f32([0.1, 0.6, 0.2, 0.1])
    assert np.array_equal(O.apply_top_p(a, 1.0), a)


@pytest.mark.parametrize("seed", range(6))
def test_top_p_nucleus_invariants(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(2, 400))
    e = np.exp(rng.normal(0, 1.5, n)).astype(np.float32)
    probs = (e / e.sum()).astype(np.float32)
    for p in (0.05, 0.3, 0.7, 0.9, 0.99):
        q = O.apply_top_p(probs, p)
        kept = q > 0
        assert kept.any()
        # every kept probability is at least every dropped one
        if (~kept).any():
            assert probs[kept].min() >= probs[~kept].max()
        # minimal prefix: the kept mass reaches p, the kept mass without its smallest entry does not
        mass = float(np.sum(probs[kept], dtype=np.float64))
        assert mass >= p - 1e-5
        assert mass - float(probs[kept].min()) < p + 1e-5
        # renormalised over the nucleus, in proportion to the input
        assert abs(float(q.sum(dtype=np.float64)) - 1.0) < 1e-5
        np.testing.assert_allclose(q[kept], probs[kept] / mass, rtol=2e-6)


def test_repetition_penalty_reference_cases():
    # RepetitionPenaltySamplerTests.cs (the model loop applies the same rule, LlamaLanguageModel.cs:357-373)
    lg = O.repetition_penalty(f32([0.1, 5.0, 4.0]), [1], 1.5)
    assert lg[1] == np.float32(5.0) / np.float32(1.5) and O.lib.orc_argmax(fp(lg), 3) == 2
    lg = O.repetition_penalty(f32([-2.0, 0.0, 1.0]), [0], 2.0)
    assert lg[0] == -4.0 and O.lib.orc_argmax(fp(lg), 3) == 2
    lg = O.repetition_penalty(f32([5.0, 5.0, 0.5]), [0, 1], 10.0)
    assert lg[0] == lg[1] == 0.5
    # repeats apply again, zero takes the multiply branch, ids out of range are skipped
    lg = O.repetition_penalty(f32([8.0, 0.0, -1.0]), [0, 0, 0, 1, 2, 2, 3, -1], 2.0)
    assert lg.tolist() == [1.0, 0.0, -4.0]


def test_activation_digit_bytes_match_the_digit_recurrence():
    """The matrix-core GEMV's activation table stores each quantized value X = rint(v * 127 / amax *
    65536) (so |X| <= 127 * 65536) as signed base-256 digits X = 65536 b2 + 256 b1 + b0, each in
    [-128, 127]. The device packs them as byte 0 of X, byte 1 of X + 128 and byte 2 of X + 32896
    (csrc/actab.hpp digits3_pack4); over every X of the range those bytes equal the digits of the
    recurrence b0 = int8(X), b1 = int8((X - b0) / 256), b2 = ((X - b0) / 256 - b1) / 256, and the
    digits rebuild X."""
    lim = 127 * 65536
    X = np.arange(-lim, lim + 1, dtype=np.int32)
    b0 = ((X & 0xFF) ^ 0x80) - 0x80
    x1 = (X - b0) >> 8
    b1 = ((x1 & 0xFF) ^ 0x80) - 0x80
    b2 = (x1 - b1) >> 8
    assert np.array_equal(65536 * b2 + 256 * b1 + b0, X)
    assert b2.min() >= -128 and b2.max() <= 127 and int(b2.max()) == 127
    assert np.array_equal(X & 0xFF, b0 & 0xFF)
    assert np.array_equal(((X + 128) >> 8) & 0xFF, b1 & 0xFF)
    assert np.array_equal(((X + 32896) >> 16) & 0xFF, b2 & 0xFF)
