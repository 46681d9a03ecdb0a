"""Writes the golden fixtures under tests/golden/ from the reference's own numpy weight code.

Run once, in the build container, where the reference checkout exists:
    python tests/golden/make_fixtures.py /root/reference

It imports the reference's `python/trpack/blocks.py` (q4k_rows, q8_0_rows, q5_1_rows,
rows_to_groups) and
`python/trpack/codec.py` (pack_tq) — both numpy-only — and records their outputs on small,
seeded inputs.  These are the only pins for the Q4_K scale/min bit layout, the (q, d, m) forms of
the Q8_0 / Q5_1 conversions and the TQ byte layout that do not depend on this repository's own
reading of them.  The fixtures are data only
(inputs and expected outputs); the tests never import the reference.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref_root: str) -> None:
    sys.path.insert(0, os.path.join(ref_root, "python"))
    from trpack import blocks, codec  # noqa: E402  (reference code, read-only)

    rng = np.random.default_rng(20261201)
    out = {}

    # --- Q4_K rows: random superblocks plus hand-made edge cases -----------------------------
    rows, K = 6, 512
    raw = rng.integers(0, 256, size=(rows, K // 256 * 144), dtype=np.uint8)
    # fp16 d / dmin in a realistic range for rows 0..3
    for r in range(rows):
        for sb in range(K // 256):
            o = sb * 144
            d = np.float16(rng.uniform(1e-4, 2e-3))
            dm = np.float16(rng.uniform(1e-4, 2e-3))
            raw[r, o:o + 2] = np.frombuffer(d.tobytes(), np.uint8)
            raw[r, o + 2:o + 4] = np.frombuffer(dm.tobytes(), np.uint8)
    # row 4: all scale bytes 0xff (every 6-bit scale/min = 63), row 5: scale bytes 0
    raw[4, 4:16] = 0xFF
    raw[4, 144 + 4:144 + 16] = 0xFF
    raw[5, 4:16] = 0
    raw[5, 144 + 4:144 + 16] = 0
    q, dd, mm = blocks.q4k_rows(raw, K)
    q16, dd16, mm16 = blocks.rows_to_groups(q, dd, mm, 16)
    out["q4k_raw"] = raw
    out["q4k_q"] = q.astype(np.uint8)
    out["q4k_dd"] = dd.view(np.uint16)
    out["q4k_mm"] = mm.view(np.uint16)
    out["q4k_dd16"] = dd16.view(np.uint16)
    out["q4k_mm16"] = mm16.view(np.uint16)
    out["q4k_tq4_32"] = codec.pack_tq(q.astype(np.uint8), dd, mm, 4, 32)
    out["q4k_tq4_16"] = codec.pack_tq(q16.astype(np.uint8), dd16, mm16, 4, 16)

    # --- TQ byte layout for every codec (the shapes of python/tests/test_codec.py) ------------
    for bits, kb, r_, k_ in [(4, 32, 32, 64), (5, 32, 16, 96), (8, 32, 40, 64), (5, 16, 48, 80), (8, 16, 16, 32),
                             (4, 16, 16, 48), (4, 32, 5, 64)]:
        qq = rng.integers(0, 1 << bits, size=(r_, k_), dtype=np.uint8)
        d = rng.uniform(0.001, 0.1, size=(r_, k_ // kb)).astype(np.float16)
        m = rng.uniform(-1, 1, size=(r_, k_ // kb)).astype(np.float16)
        tag = f"tq{bits}_{kb}_{r_}x{k_}"
        out[tag + "_q"] = qq
        out[tag + "_d"] = d.view(np.uint16)
        out[tag + "_m"] = m.view(np.uint16)
        out[tag + "_bytes"] = codec.pack_tq(qq, d, m, bits, kb)
        out[tag + "_deq"] = codec.unpack_tq(out[tag + "_bytes"], r_, k_, bits, kb)

    # --- numpy's f32 -> f16 cast on awkward values (ties, subnormals, overflow) --------------
    f = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(1e-3),
        np.array([65504, 65519.99, 65520, 1e-7, 5.96e-8, 2.98e-8, 2.9802322e-8, 6.1e-5, 6.103515625e-05,
                  1.0009765625, 1.00048828125, 1.00146484375, -0.0], np.float32),
        (rng.uniform(-20, 20, 4000)).astype(np.float32),
        np.ldexp(rng.uniform(1, 2, 2000), rng.integers(-30, -10, 2000)).astype(np.float32),
    ])
    out["f16_in"] = f
    out["f16_out"] = f.astype(np.float16).view(np.uint16)

    # --- Q8_0 / Q5_1 rows (the real model's down formats): random blocks plus edge cases -------
    rows, K = 5, 256
    nb = K // 32
    raw8 = rng.integers(0, 256, size=(rows, nb * 34), dtype=np.uint8)
    raw5 = rng.integers(0, 256, size=(rows, nb * 24), dtype=np.uint8)
    for r in range(rows):
        for b in range(nb):
            d = np.float16(rng.uniform(1e-4, 2e-3))
            m = np.float16(-rng.uniform(1e-3, 3e-2))
            raw8[r, 34 * b:34 * b + 2] = np.frombuffer(d.tobytes(), np.uint8)
            raw5[r, 24 * b:24 * b + 2] = np.frombuffer(d.tobytes(), np.uint8)
            raw5[r, 24 * b + 2:24 * b + 4] = np.frombuffer(m.tobytes(), np.uint8)
    # row 3: d near the f16 limit (-128 d overflows f16 to -inf), a subnormal d, d = 0, d = -0;
    # row 4: int8 extremes -128 / 127 / 0 / -1
    for b, dv in enumerate([65504.0, 600.0, 512.0, 6e-8, 0.0, -0.0, -3.0, 1.0]):
        raw8[3, 34 * b:34 * b + 2] = np.frombuffer(np.float16(dv).tobytes(), np.uint8)
        raw5[3, 24 * b:24 * b + 2] = np.frombuffer(np.float16(dv).tobytes(), np.uint8)
    raw8[4, 2:34] = 0x80
    raw8[4, 36:68] = 0x7F
    raw8[4, 70:102] = 0x00
    raw8[4, 104:136] = 0xFF
    # Q5_1 qh: all ones, all zeros, alternating, one bit per half
    raw5[4, 4:8] = 0xFF
    raw5[4, 24 + 4:24 + 8] = 0x00
    raw5[4, 48 + 4:48 + 8] = 0xAA
    raw5[4, 72 + 4:72 + 8] = [0x01, 0x00, 0x01, 0x00]
    q8, d8, m8 = blocks.q8_0_rows(raw8, K)
    q5, d5, m5 = blocks.q5_1_rows(raw5, K)
    out["q80_raw"], out["q80_q"], out["q80_d"], out["q80_m"] = raw8, q8, d8.view(np.uint16), m8.view(np.uint16)
    out["q51_raw"], out["q51_q"], out["q51_d"], out["q51_m"] = raw5, q5, d5.view(np.uint16), m5.view(np.uint16)


    path = os.path.join(HERE, "blocks_codec.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, sum(v.nbytes for v in out.values()), "bytes raw")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
