"""Writes the golden decode fixtures ``tests/golden/decode_<fmt>.npz``.

The reference stores no golden vectors for this path, so the fixtures are built
from first principles: random *integer parameters* (scales, mins, quants, fp16
super-scales) are packed into wire blocks by an element-by-element ENCODER written
here from the published GGUF / MLX layouts, and the expected weight of every
element is computed from the parameters themselves in float64 (exact) and
rounded once to float32.  The decoder under test never takes part in producing
the fixture, so a decoder that swaps nibbles, scale indices or bit positions
fails against it.

Run:  python tests/golden/make_golden.py   (deterministic; seed 1234)
"""

from __future__ import annotations

import pathlib

import numpy as np

OUT = pathlib.Path(__file__).resolve().parent


def f16_bytes(v: float) -> bytes:
    return np.array([v], dtype=np.float16).tobytes()


def rnd_f16(rng, scale):
    # fp16-representable value, including subnormals and negatives for min scales
    return float(np.float16(rng.standard_normal() * scale))


def enc_q8_0(rng, nblocks):
    blob, expect = bytearray(), []
    for _ in range(nblocks):
        d = rnd_f16(rng, 0.02)
        q = [int(v) for v in rng.integers(-128, 128, 32)]
        blob += f16_bytes(d)
        blob += bytes((v & 0xFF) for v in q)
        expect += [d * v for v in q]
    return blob, expect


def enc_q5_0(rng, nblocks):
    blob, expect = bytearray(), []
    for _ in range(nblocks):
        d = rnd_f16(rng, 0.02)
        q = [int(v) for v in rng.integers(0, 32, 32)]          # 5-bit unsigned, w = (q-16)*d
        qh = 0
        for e in range(32):
            qh |= ((q[e] >> 4) & 1) << e
        qs = [(q[l] & 15) | ((q[l + 16] & 15) << 4) for l in range(16)]
        blob += f16_bytes(d) + int(qh).to_bytes(4, "little") + bytes(qs)
        expect += [(v - 16) * d for v in q]
    return blob, expect


def enc_q4_k(rng, nblocks):
    blob, expect = bytearray(), []
    for _ in range(nblocks):
        d, dmin = rnd_f16(rng, 0.01), rnd_f16(rng, 0.01)
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        mn = [int(v) for v in rng.integers(0, 64, 8)]
        q = [int(v) for v in rng.integers(0, 16, 256)]
        s = [0] * 12
        for j in range(8):              # ggml packing of 6-bit scales / mins
            if j < 4:
                s[j] |= sc[j] & 63
                s[j + 4] |= mn[j] & 63
            else:
                s[j + 4] |= (sc[j] & 15) | ((mn[j] & 15) << 4)
                s[j - 4] |= (sc[j] >> 4) << 6
                s[j] |= (mn[j] >> 4) << 6
        qs = bytearray(128)
        for g in range(8):
            for l in range(32):
                byte = (g // 2) * 32 + l
                qs[byte] |= (q[32 * g + l] & 15) << (4 * (g % 2))
        blob += f16_bytes(d) + f16_bytes(dmin) + bytes(s) + bytes(qs)
        expect += [d * sc[e // 32] * q[e] - dmin * mn[e // 32] for e in range(256)]
    return blob, expect


def enc_q6_k(rng, nblocks):
    blob, expect = bytearray(), []
    for _ in range(nblocks):
        d = rnd_f16(rng, 0.005)
        sc = [int(v) for v in rng.integers(-128, 128, 16)]
        q = [int(v) for v in rng.integers(0, 64, 256)]          # 6-bit unsigned, w = d*sc*(q-32)
        ql, qh = bytearray(128), bytearray(64)
        for e in range(256):
            h, rem = divmod(e, 128)
            s, l = divmod(rem, 32)
            ql[64 * h + 32 * (s & 1) + l] |= (q[e] & 15) << (4 * (s >> 1))
            qh[32 * h + l] |= ((q[e] >> 4) & 3) << (2 * s)
        blob += bytes(ql) + bytes(qh) + bytes((v & 0xFF) for v in sc) + f16_bytes(d)
        for e in range(256):
            h, rem = divmod(e, 128)
            s, l = divmod(rem, 32)
            expect.append(d * sc[8 * h + 2 * s + l // 16] * (q[e] - 32))
    return blob, expect


def enc_mlx(rng, N, K, gs):
    q = rng.integers(0, 16, (N, K))
    qweight = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    scales = (rng.standard_normal((N, K // gs)) * 0.02).astype(np.float16)
    biases = (rng.standard_normal((N, K // gs)) * 0.02).astype(np.float16)
    s = np.repeat(scales.astype(np.float64), gs, axis=1)
    b = np.repeat(biases.astype(np.float64), gs, axis=1)
    return qweight, scales, biases, (s * q + b).astype(np.float32)


def main() -> None:
    rng = np.random.default_rng(1234)
    specs = {"q8_0": (enc_q8_0, 32), "q5_0": (enc_q5_0, 32), "q4_k": (enc_q4_k, 256), "q6_k": (enc_q6_k, 256)}
    for fmt, (enc, qk) in specs.items():
        N, K = 3, 4 * qk if qk == 32 else 512
        nb = K // qk
        blob, expect = enc(rng, N * nb)
        blob = np.frombuffer(bytes(blob), np.uint8).reshape(N, -1)
        # float64 products of fp16 and small ints are exact; one rounding to fp32
        w = np.array(expect, np.float64).astype(np.float32).reshape(N, K)
        np.savez(OUT / f"decode_{fmt}.npz", blob=blob, K=np.int64(K), w=w)
    qweight, scales, biases, w = enc_mlx(rng, 3, 256, 64)
    np.savez(OUT / "decode_mlx_q4.npz", qweight=qweight, scales=scales, biases=biases, K=np.int64(256),
             group_size=np.int64(64), w=w)


if __name__ == "__main__":
    main()
