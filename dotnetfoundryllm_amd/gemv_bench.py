"""Isolated decode-GEMV microbenchmark: fllm_gemv_ex (LinearProjection, LlamaForwardPass.cs:237-260)
for 4096x4096, 14336x4096 and 4096x14336 in Q4_K, Q8_0 and Q6_K, with an F32 input x ~ N(0, 1), on
GGUF rows as uploaded and on the same matrices regrouped by fllm_gemv_pack (the layout the model
path reads).

Weights are seeded random blocks as for the synthetic models (K-quants: nibbles and 6-bit
scales/mins uniform, f16 d/dmin in [1e-3, 4e-3]; Q8_0: int8 uniform, f16 d in [1e-3, 1e-2]).
Each matrix is replicated so that the launches, which go round-robin over the copies, read at
least 1 GiB of distinct weights between two reads of the same copy (the 256 MiB last-level
cache cannot serve them). The time per launch is the mean over launches back to back between one
HIP event pair (fllm_gemv_time_ex: the launch gaps count); bytes are the stored weight bytes
(algorithmic, per launch).

    python -m dotnetfoundryllm_amd.gemv_bench [--iters N] [--copies-bytes B]
"""
import argparse

import numpy as np

from . import LAYOUT_GGUF, LAYOUT_TILES, Context, DeviceBuffer, gemv_pack, gemv_time, synth_tensor
from ._native import Q4_K, Q6_K, Q8_0, type_bytes
from .configs import KQ_RANGE, Q8_RANGE

SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]
TYPES = [(Q4_K, "Q4_K"), (Q8_0, "Q8_0"), (Q6_K, "Q6_K")]
HBM_PEAK_GBS = 8000.0


def weight_range(t):
    """Range of the blocks' f16 scales: Q8_0 d in [1e-3, 1e-2], K-quant d / dmin in [1e-3, 4e-3]."""
    return Q8_RANGE if t == Q8_0 else KQ_RANGE


def run(iters=200, copies_bytes=1 << 30, seed=0x5EED01, out=print):
    """[(type name, rows, cols, layout name, bytes, copies, us per launch, GB/s)]; progress to out."""
    ctx = Context(0)
    rng = np.random.default_rng(seed)
    rows_out = []
    try:
        for t, tname in TYPES:
            p0, p1 = weight_range(t)
            for rows, cols in SHAPES:
                nb = type_bytes(t, rows * cols)
                n_copies = max(2, -(-copies_bytes // nb))
                x = rng.standard_normal(cols).astype(np.float32)
                xb, yb = DeviceBuffer(ctx, x.nbytes), DeviceBuffer(ctx, rows * 4)
                xb.write(x)
                bufs, tiles = [], []
                try:
                    for c in range(n_copies):
                        raw = synth_tensor(t, seed, 1000 * rows + c, rows * cols, 0, p0, p1)
                        b = DeviceBuffer(ctx, raw.nbytes)
                        b.write(raw)
                        bufs.append(b)
                        tb = DeviceBuffer(ctx, raw.nbytes)
                        gemv_pack(ctx, t, b, rows, cols, tb)
                        tiles.append(tb)
                    for layout, name, ws in ((LAYOUT_GGUF, "GGUF rows", bufs), (LAYOUT_TILES, "tiles", tiles)):
                        gemv_time(ctx, t, ws, rows, cols, xb, yb, 20, layout)  # warm-up
                        us = gemv_time(ctx, t, ws, rows, cols, xb, yb, iters, layout)
                        gbs = nb / (us * 1e-6) / 1e9
                        rows_out.append((tname, rows, cols, name, nb, n_copies, us, gbs))
                        out(f"{tname} {rows}x{cols} {name}: {nb / 1e6:.2f} MB x {n_copies} copies, {us:.2f} us, "
                            f"{gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)")
                finally:
                    for b in bufs + tiles + [xb, yb]:
                        b.close()
    finally:
        ctx.close()
    return rows_out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--copies-bytes", type=int, default=1 << 30)
    a = ap.parse_args()
    res = run(a.iters, a.copies_bytes)
    print("\n| type | rows x cols | layout | MB | copies | us per launch | GB/s | % of 8 TB/s |")
    print("|---|---|---|---|---|---|---|---|")
    for tname, rows, cols, name, nb, n, us, gbs in res:
        print(f"| {tname} | {rows} x {cols} | {name} | {nb / 1e6:.2f} | {n} | {us:.2f} | {gbs:.0f} | "
              f"{100 * gbs / HBM_PEAK_GBS:.1f}% |")


if __name__ == "__main__":
    main()
