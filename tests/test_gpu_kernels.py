"""GPU parity of the dequantization and fused dequant-GEMV kernels against the oracle.

Dequantization is bit-exact (every type, random blocks, the reference's known-answer blocks,
all 65536 F16/BF16 bit patterns). GEMV results are compared with the oracle's dequantized F32
weights times x in float64, normwise: max|y - y_ref| / max|y_ref| <= 1e-3 (the bar for
float32-accumulated results); the kernels' own accuracy is float32-level, so a second bound of
1e-5 is asserted to catch any layout or indexing mistake that a loose bar would let through.
"""
import numpy as np
import pytest

import dotnetfoundryllm_amd as F
import dotnetfoundryllm_amd._native as N
import oracle_bind as O

pytestmark = pytest.mark.gpu

ALL_TYPES = [N.F32, N.F16, N.BF16, N.Q4_0, N.Q8_0, N.Q4_K, N.Q5_K, N.Q6_K, N.Q8_K]
RANGES = {N.Q8_0: (1e-3, 1e-2), N.F32: (0.0, 1.0), N.F16: (0.0, 1.0), N.BF16: (0.0, 1.0)}


def synth(t, n, seed=1, tid=0):
    p0, p1 = RANGES.get(t, (1e-3, 4e-3))
    return F.synth_tensor(t, seed, tid, n, 0, p0, p1)


@pytest.mark.parametrize("t", ALL_TYPES)
def test_dequantize_bit_exact_random_blocks(ctx, t):
    for nblocks in (1, 3, 257):
        n = nblocks * N.BLOCK[t][1] * (256 if N.BLOCK[t][1] == 1 else 1)
        raw = synth(t, n, seed=nblocks, tid=t)
        got = F.Dequantizer.dequantize(ctx, t, raw)
        rc, want = O.dequantize(t, raw)
        assert rc == 0
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_exhaustive_16bit(ctx):
    bits = np.arange(65536, dtype=np.uint16)
    for t in (N.F16, N.BF16):
        got = F.Dequantizer.dequantize(ctx, t, bits.tobytes())
        rc, want = O.dequantize(t, bits.tobytes())
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_reference_known_answers(ctx):
    h = lambda v: int(v).to_bytes(2, "little")  # noqa: E731
    out = F.Dequantizer.dequantize(ctx, N.Q4_0, h(0x3C00) + bytes([0x79] + [0x88] * 15))
    assert out[0] == 1.0 and out[16] == -1.0 and out[1] == 0.0
    blk = bytearray(34)
    blk[0:2] = h(0x3C00)
    blk[2], blk[4] = 0xFF, 1
    assert list(F.Dequantizer.dequantize(ctx, N.Q8_0, bytes(blk))[:3]) == [-1.0, 0.0, 1.0]
    for t, nb in ((N.Q4_K, 144), (N.Q5_K, 176)):
        z = bytearray(nb)
        z[0:2] = h(0x3C00)
        assert np.all(F.Dequantizer.dequantize(ctx, t, bytes(z)) == 0)
    assert list(F.Dequantizer.dequantize(ctx, N.F16, h(0x3C00) + h(0xBC00))) == [1.0, -1.0]


def test_dequantize_error_contract(ctx):
    with pytest.raises(F.NotSupportedException):
        F.Dequantizer.dequantize(ctx, 99, bytes(4), 1)
    with pytest.raises(F.ArgumentException):
        F.Dequantizer.dequantize(ctx, N.Q4_K, bytes(143), 256)
    with pytest.raises(F.ArgumentException):
        F.Dequantizer.dequantize(ctx, N.Q8_0, bytes(68), 32)  # destination too small
    assert F.Dequantizer.element_count(N.Q6_K, 210) == 256


def run_gemv(ctx, t, rows, cols, seed=3, x=None):
    raw = synth(t, rows * cols, seed=seed, tid=rows)
    if x is None:
        x = np.random.default_rng(seed).standard_normal(cols).astype(np.float32)
    wb, xb, yb = F.DeviceBuffer(ctx, raw.nbytes), F.DeviceBuffer(ctx, x.nbytes), F.DeviceBuffer(ctx, rows * 4)
    try:
        wb.write(raw)
        xb.write(x)
        F.gemv(ctx, t, wb, rows, cols, xb, yb)
        ctx.sync()
        y = yb.read(rows * 4)
    finally:
        for b in (wb, xb, yb):
            b.close()
    rc, wf = O.dequantize(t, raw, rows * cols)
    assert rc == 0
    ref = wf.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    return y, ref


# the microbenchmark shapes (rows x cols) and their types
GEMV_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("t", [N.Q4_K, N.Q8_0, N.Q6_K])
@pytest.mark.parametrize("shape", GEMV_SHAPES)
def test_gemv_microbenchmark_shapes(ctx, t, shape):
    y, ref = run_gemv(ctx, t, *shape)
    err = O.normwise_rel_err(y, ref)
    print(f"type {t} {shape}: normwise rel err {err:.2e}")
    assert err <= 1e-3
    assert err <= 1e-5


@pytest.mark.parametrize("t", [N.Q4_K, N.Q8_0, N.Q6_K, N.Q5_K])
@pytest.mark.parametrize("shape", GEMV_SHAPES + [(64, 18944), (16, 256), (48, 3584), (32, 2560)])
def test_gemv_tiles_layout(ctx, t, shape):
    """fllm_gemv_pack + fllm_gemv_ex(FLLM_LAYOUT_TILES) against the oracle's F32 dot (18944
    columns: 74 chunks, 8 per wave over 10 waves; 3584 and 2560 columns: 14 and 10 chunks, 4 per
    wave with the last wave partly past the row)."""
    rows, cols = shape
    raw = synth(t, rows * cols, seed=5, tid=rows + 1)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    wb, tb = F.DeviceBuffer(ctx, raw.nbytes), F.DeviceBuffer(ctx, raw.nbytes)
    xb, yb = F.DeviceBuffer(ctx, x.nbytes), F.DeviceBuffer(ctx, rows * 4)
    try:
        wb.write(raw)
        xb.write(x)
        F.gemv_pack(ctx, t, wb, rows, cols, tb)
        F.gemv(ctx, t, tb, rows, cols, xb, yb, layout=F.LAYOUT_TILES)
        ctx.sync()
        y = yb.read(rows * 4)
    finally:
        for b in (wb, tb, xb, yb):
            b.close()
    rc, wf = O.dequantize(t, raw, rows * cols)
    assert rc == 0
    ref = wf.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    err = O.normwise_rel_err(y, ref)
    print(f"type {t} {shape} tiles: normwise rel err {err:.2e}")
    assert err <= 1e-5


def test_gemv_tiles_contract(ctx):
    raw = synth(N.Q4_K, 32 * 512, seed=6, tid=1)
    wb, tb = F.DeviceBuffer(ctx, raw.nbytes), F.DeviceBuffer(ctx, raw.nbytes)
    xb, yb = F.DeviceBuffer(ctx, 512 * 4), F.DeviceBuffer(ctx, 32 * 4)
    try:
        wb.write(raw)
        with pytest.raises(F.NotSupportedException):
            F.gemv_pack(ctx, N.Q4_0, wb, 32, 512, tb)             # no tile layout for Q4_0
        with pytest.raises(F.NotSupportedException):
            F.gemv_pack(ctx, N.Q4_K, wb, 24, 512, tb)             # rows not a multiple of 16
        with pytest.raises(F.ArgumentException):
            F.gemv_pack(ctx, N.Q4_K, wb, 32, 512, wb)             # not in place
        with pytest.raises(F.ArgumentOutOfRangeException):
            F.gemv(ctx, N.Q4_K, wb, 32, 512, xb, yb, layout=7)    # unknown layout
    finally:
        for b in (wb, tb, xb, yb):
            b.close()


@pytest.mark.parametrize("t,rows,cols", [
    (N.Q4_K, 512, 1408),     # rows straddle Q4_K blocks (5.5 blocks per row)
    (N.Q6_K, 300, 3584),     # rows only 4-byte aligned (2940 bytes)
    (N.Q6_K, 77, 18944),     # wide row, K split over 10 waves
    (N.Q5_K, 300, 3584), (N.Q5_K, 64, 18944),
    (N.Q8_0, 333, 96), (N.Q8_0, 130, 3584),
    (N.Q4_0, 257, 512), (N.Q4_K, 1, 256), (N.Q4_K, 13, 2048 + 256),
    (N.F32, 100, 260), (N.F32, 50, 99), (N.F16, 200, 520), (N.BF16, 200, 3584), (N.F16, 9, 36),
    (N.Q8_K, 40, 512),
])
def test_gemv_types_and_shapes(ctx, t, rows, cols):
    y, ref = run_gemv(ctx, t, rows, cols)
    err = O.normwise_rel_err(y, ref)
    print(f"type {t} {rows}x{cols}: normwise rel err {err:.2e}")
    assert err <= 1e-3
    assert err <= 1e-5


def test_gemv_special_activations(ctx):
    # zero groups, a single spike, large dynamic range inside a group
    x = np.zeros(4096, dtype=np.float32)
    x[5] = 1e4
    x[100:132] = np.linspace(-1e-6, 1e3, 32)
    x[4000] = -3.0
    for t in (N.Q4_K, N.Q6_K, N.Q8_0):
        y, ref = run_gemv(ctx, t, 512, 4096, x=x)
        assert O.normwise_rel_err(y, ref) <= 1e-5


def test_gemv_argument_checks(ctx):
    wb = F.DeviceBuffer(ctx, 144 * 16)
    xb, yb = F.DeviceBuffer(ctx, 4096 * 4), F.DeviceBuffer(ctx, 16 * 4)
    try:
        with pytest.raises(F.ArgumentException):
            F.gemv(ctx, N.Q4_K, wb, 16, 4096, xb, yb)          # weight buffer too small
        with pytest.raises(F.ArgumentException):
            F.gemv(ctx, N.Q4_K, wb, 1, 256, xb, yb, w_offset=8)  # misaligned offset
        with pytest.raises(F.ArgumentException):
            F.gemv(ctx, N.Q4_K, wb, 1, 100, xb, yb)            # not whole blocks
        with pytest.raises(F.NotSupportedException):
            F.gemv(ctx, 3, wb, 1, 32, xb, yb)
    finally:
        for b in (wb, xb, yb):
            b.close()
