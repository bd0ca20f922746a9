"""Pins the oracle's dequantizers (CPU only).

Checks, in order of strength:
  - the reference's own known-answer tests (tests/DotNetFoundryLLM.Quantization.Tests/DequantizerTests.cs),
  - exhaustive 16-bit conversion tables against numpy's IEEE binary16,
  - ggml's published get_scale_min_k4 layout (which the reference's DecodeKScaleMin follows) and
    its inverse, brute-forced over every 6-bit value,
  - one-hot probes that pin each format's element order to the layout the reference documents
    (Dequantizer.cs:284-291 Q4_K, :351-365 Q5_K, :404-415 Q6_K), so a transposed index fails,
  - two-rounding (no fused multiply-add) arithmetic order.
"""
import struct

import numpy as np
import pytest

import oracle_bind as O

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 15, 30


def h16(v):
    return struct.pack("<H", v)


# ---- DequantizerTests.cs known answers -------------------------------------------------
def test_half_and_bf16_known_values():
    assert O.lib.orc_half_to_float(0x0000) == 0.0
    assert O.lib.orc_half_to_float(0x3C00) == 1.0
    assert O.lib.orc_half_to_float(0xBC00) == -1.0
    assert O.lib.orc_bf16_to_float(0x0000) == 0.0
    assert O.lib.orc_bf16_to_float(0x3F80) == 1.0
    assert O.lib.orc_bf16_to_float(0x4000) == 2.0


def test_f32_round_trip_and_wrong_length():
    orig = np.array([1.5, -2.25, 0.0, 3.14], dtype=np.float32)
    rc, out = O.dequantize(F32, orig.tobytes())
    assert rc == 0 and np.array_equal(out, orig)
    rc, _ = O.dequantize(F32, bytes(5), n=1)
    assert rc == -2


def test_f16_bf16_known_values():
    rc, out = O.dequantize(F16, h16(0x3C00) + h16(0xBC00))
    assert rc == 0 and list(out) == [1.0, -1.0]
    rc, out = O.dequantize(BF16, h16(0x3F80) + h16(0x4000))
    assert rc == 0 and list(out) == [1.0, 2.0]


def test_q4_0_known_blocks():
    rc, out = O.dequantize(Q4_0, h16(0) + bytes([0x88] * 16))
    assert rc == 0 and np.all(out == 0)
    rc, out = O.dequantize(Q4_0, h16(0x3C00) + bytes([0x79] + [0x88] * 15))
    assert rc == 0 and out[0] == 1.0 and out[16] == -1.0 and out[1] == 0.0
    rc, _ = O.dequantize(Q4_0, bytes(17), n=32)
    assert rc == -2


def test_q8_0_known_block():
    blk = bytearray(34)
    blk[0:2] = h16(0x3C00)
    blk[2] = 0xFF
    blk[3] = 0
    blk[4] = 1
    rc, out = O.dequantize(Q8_0, bytes(blk))
    assert rc == 0 and list(out[:3]) == [-1.0, 0.0, 1.0]
    rc, _ = O.dequantize(Q8_0, bytes(33), n=32)
    assert rc == -2


def test_unknown_type_and_element_counts():
    rc, _ = O.dequantize(99, bytes(4), n=1)
    assert rc == -4
    for t, nb, want in [(F32, 16, 4), (Q4_0, 18, 32), (Q8_0, 34, 32), (Q4_K, 144, 256), (Q5_K, 176, 256)]:
        c = O.I64()
        assert O.lib.orc_element_count(t, nb, O.C.byref(c)) == 0 and c.value == want


def test_k_quant_zero_blocks_and_wrong_lengths():
    for t, nb in [(Q4_K, 144), (Q5_K, 176)]:
        blk = bytearray(nb)
        blk[0:2] = h16(0x3C00)
        rc, out = O.dequantize(t, bytes(blk))
        assert rc == 0 and np.all(out == 0)
        rc, _ = O.dequantize(t, bytes(nb - 1), n=256)
        assert rc == -2


# ---- exhaustive conversions -------------------------------------------------------------
def test_half_exhaustive_against_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    raw = bits.tobytes()
    rc, out = O.dequantize(F16, raw)
    assert rc == 0
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    rc, out = O.dequantize(BF16, bits.tobytes())
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), bits.astype(np.uint32) << 16)


# ---- K-quant 6-bit scale/min layout (ggml get_scale_min_k4) -----------------------------
def ggml_get_scale_min_k4(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def ggml_pack(sc, mn):
    q = [0] * 12
    for j in range(8):
        if j < 4:
            q[j] = sc[j]
            q[j + 4] = mn[j]
        else:
            q[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            q[j - 4] |= (sc[j] >> 4) << 6
            q[j] |= (mn[j] >> 4) << 6
    return bytes(q)


def test_kscale_min_matches_ggml_on_every_byte_value():
    for pos in range(12):
        for v in range(256):
            q = bytearray(12)
            q[pos] = v
            for g in range(8):
                s, m = O.C.c_int(), O.C.c_int()
                O.lib.orc_decode_kscale_min(bytes(q), g, O.C.byref(s), O.C.byref(m))
                assert (s.value, m.value) == ggml_get_scale_min_k4(g, q)


def test_kscale_min_round_trip_every_value():
    rng = np.random.default_rng(0)
    for trial in range(400):
        sc = list(rng.integers(0, 64, 8))
        mn = list(rng.integers(0, 64, 8))
        if trial < 64:
            sc = [trial] * 8
            mn = [63 - trial] * 8
        q = ggml_pack(sc, mn)
        for g in range(8):
            s, m = O.C.c_int(), O.C.c_int()
            O.lib.orc_decode_kscale_min(q, g, O.C.byref(s), O.C.byref(m))
            assert (s.value, m.value) == (sc[g], mn[g])


# ---- element-order probes ----------------------------------------------------------------
def q4k_block(qs, d=0x3C00, dmin=0, sc=(1,) * 8, mn=(0,) * 8):
    return h16(d) + h16(dmin) + ggml_pack(list(sc), list(mn)) + bytes(qs)


def test_q4_k_element_order_probe():
    for j in (0, 1, 15, 16, 37, 127):
        qs = bytearray(128)
        qs[j] = 0x21
        rc, out = O.dequantize(Q4_K, q4k_block(qs))
        assert rc == 0
        g, i = j // 16, 2 * (j % 16)
        want = np.zeros(256, dtype=np.float32)
        want[g * 32 + i] = 1.0
        want[g * 32 + i + 1] = 2.0
        assert np.array_equal(out, want), j


def test_q4_k_scale_and_min_per_group():
    qs = bytes([0x11] * 128)  # every q = 1
    sc = [1, 2, 3, 4, 5, 6, 7, 63]
    mn = [0, 1, 2, 3, 4, 5, 6, 63]
    rc, out = O.dequantize(Q4_K, q4k_block(qs, d=0x3C00, dmin=0x3800, sc=sc, mn=mn))  # dmin = 0.5
    assert rc == 0
    for g in range(8):
        assert np.all(out[g * 32:(g + 1) * 32] == np.float32(sc[g] * 1 - 0.5 * mn[g]))


def test_q5_k_high_bit_probe():
    for k, b in [(0, 0), (0, 7), (3, 5), (31, 7)]:
        qh = bytearray(32)
        qh[k] |= 1 << b
        blk = h16(0x3C00) + h16(0) + ggml_pack([1] * 8, [0] * 8) + bytes(qh) + bytes(128)
        rc, out = O.dequantize(Q5_K, blk)
        assert rc == 0
        want = np.zeros(256, dtype=np.float32)
        want[8 * k + b] = 16.0
        assert np.array_equal(out, want)


def test_q6_k_layout_probe():
    ql = bytearray(128)
    qh = bytearray(64)
    scales = bytearray([1] * 16)
    ql[5] = 0x21                     # elements 10, 11 -> low nibbles 1, 2
    qh[7] = 0b11100100               # elements 28..31 -> high fields 0,1,2,3
    scales[15] = 2                   # elements 240..255 doubled
    blk = bytes(ql) + bytes(qh) + bytes(scales) + h16(0x3C00)
    rc, out = O.dequantize(Q6_K, blk)
    assert rc == 0
    want = np.full(256, -32.0, dtype=np.float32)
    want[10], want[11] = -31.0, -30.0
    want[28:32] = [-32.0, -16.0, 0.0, 16.0]
    want[240:] = -64.0
    assert np.array_equal(out, want)


def test_q8_k_values():
    blk = struct.pack("<f", 0.5) + bytes((i - 128) & 0xFF for i in range(256)) + bytes(32)
    rc, out = O.dequantize(Q8_K, blk)
    assert rc == 0
    assert np.array_equal(out, (np.arange(256) - 128).astype(np.float32) * np.float32(0.5))


# ---- arithmetic order ---------------------------------------------------------------------
# d (11 significant bits) * scale (6 bits) * q (4-6 bits) is exact in float32, so the only
# rounding in a K-quant element is the final subtraction of mg: fused and unfused forms agree.
def test_q4_k_two_rounding_order():
    rng = np.random.default_rng(1)
    for _ in range(200):
        d = np.float16(rng.uniform(1e-3, 4e-3))
        dmin = np.float16(rng.uniform(1e-3, 4e-3))
        sc = list(rng.integers(0, 64, 8))
        mn = list(rng.integers(0, 64, 8))
        qs = rng.integers(0, 256, 128, dtype=np.uint8)
        blk = h16(int(d.view(np.uint16))) + h16(int(dmin.view(np.uint16))) + ggml_pack(sc, mn) + qs.tobytes()
        rc, out = O.dequantize(Q4_K, blk)
        assert rc == 0
        for g in range(8):
            dg = np.float32(d) * np.float32(sc[g])
            mg = np.float32(dmin) * np.float32(mn[g])
            for i in range(0, 32, 7):
                b = qs[g * 16 + i // 2]
                q = np.float32(b & 15 if i % 2 == 0 else b >> 4)
                two = np.float32(np.float32(dg * q) - mg)
                fused = np.float32(np.float64(dg) * np.float64(q) - np.float64(mg))
                assert two == fused
                assert out[g * 32 + i] == two
