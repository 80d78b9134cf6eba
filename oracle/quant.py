"""NumPy restatement of the reference's block decoders and dense reference matmul.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

All decoders return float32 arrays whose values are *exact*: every product
``d*sc*q`` / ``dmin*m`` / ``s*q`` fits in 24 significand bits, so Q8_0, Q5_0 and
Q6_K are exact in fp32 and Q4_K (``d*sc*q - dmin*m``) and MLX (``s*q + b``) are
rounded exactly once.  NumPy float32 arithmetic is used step by step (NumPy never
contracts to FMA), which yields exactly ``RN32(exact value)``.

Layouts (all little endian), cited from the reference:

* Q8_0, 34 B / 32 weights: fp16 d | int8 qs[32]; w = d*q.
  ``packages/alloy-server/src/alloy_server/gguf/quant.py:497-521`` (split_q8_0_weight),
  ``packages/alloy-metal/src/alloy/std/quant.py:811-832`` (embedding_q8_0).
* Q5_0, 22 B / 32 weights: fp16 d | u32 qh | u8 qs[16]; element l<16 is
  ``(qs[l]&15) | bit_l(qh)<<4``, element l+16 is ``(qs[l]>>4) | bit_{l+16}(qh)<<4``;
  w = (q-16)*d.  ``.../gguf/quant.py:414-494`` (split_q5_0_weight, docstring 421-428).
* Q4_K, 144 B / 256 weights: fp16 d | fp16 dmin | 12 B packed 6-bit scales/mins |
  128 B nibbles; sub-block g uses get_scale_min_k4(g); element l of sub-block g is
  byte ``qs[(g//2)*32+l]``, low nibble for even g; w = d*sc*q - dmin*m.
  ``tests/kernels/test_quant_q4k_native.py:45-70``,
  ``packages/alloy-metal/src/alloy/std/quant.py:835-884`` (embedding_q4_k).
* Q6_K, 210 B / 256 weights: ql[128] | qh[64] | int8 scales[16] | fp16 d; element
  e = 128h + 32s + l: ql byte 64h+32(s&1)+l, nibble shift 4(s>>1); qh byte 32h+l,
  shift 2s; q = (nib | qh2<<4) - 32; scale 8h+2s+l//16; w = d*sc*q.
  ``packages/alloy-metal/src/alloy/std/quant.py:1200-1270`` (embedding_q6_k).
* MLX 4-bit affine: qweight u8[N,K/2] (byte k//2, low nibble for even k), fp16
  scales/biases [N,K/GS]; w = s*q + b.
  ``packages/alloy-server/src/alloy_server/mlx/quant.py:1-24``,
  ``packages/alloy-metal/src/alloy/std/quant.py:2486-2488, 2804-2830``.
"""

from __future__ import annotations

import numpy as np

QK = {"q8_0": 32, "q5_0": 32, "q4_k": 256, "q6_k": 256}
BLOCK_BYTES = {"q8_0": 34, "q5_0": 22, "q4_k": 144, "q6_k": 210}


def _f16_at(blocks: np.ndarray, off: int) -> np.ndarray:
    """fp16 stored at byte offset ``off`` of every block -> float32 (exact)."""
    raw = np.ascontiguousarray(blocks[..., off:off + 2])
    return raw.view(np.float16)[..., 0].astype(np.float32)


def _blocks(w: np.ndarray, fmt: str, K: int) -> np.ndarray:
    w = np.asarray(w)
    if w.dtype != np.uint8:
        raise TypeError(f"{fmt} blob must be uint8, got {w.dtype}")
    qk, bb = QK[fmt], BLOCK_BYTES[fmt]
    if K % qk:
        raise ValueError(f"{fmt}: K={K} not divisible by {qk}")
    N = w.shape[0]
    nb = K // qk
    if w.shape != (N, nb * bb):
        raise ValueError(f"{fmt}: blob shape {w.shape} != {(N, nb * bb)}")
    return w.reshape(N, nb, bb)


def dequant_q8_0(w: np.ndarray, K: int) -> np.ndarray:
    b = _blocks(w, "q8_0", K)
    d = _f16_at(b, 0)
    q = np.ascontiguousarray(b[..., 2:34]).view(np.int8).astype(np.float32)
    return (d[..., None] * q).reshape(b.shape[0], K)


def dequant_q5_0(w: np.ndarray, K: int) -> np.ndarray:
    b = _blocks(w, "q5_0", K)
    d = _f16_at(b, 0)
    qh = np.ascontiguousarray(b[..., 2:6]).view("<u4")[..., 0].astype(np.uint32)
    qs = b[..., 6:22].astype(np.uint32)
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=-1)                 # elements 0..31
    hb = (qh[..., None] >> np.arange(32, dtype=np.uint32)) & 1
    q = (nib | (hb << 4)).astype(np.int32) - 16
    return (d[..., None] * q.astype(np.float32)).reshape(b.shape[0], K)


def q4_k_scale_min(sc12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """get_scale_min_k4 for all 8 sub-blocks: (..., 12) bytes -> (..., 8) sc, m.

    ``tests/kernels/test_quant_q4k_native.py:45-49``."""
    s = sc12.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    m = np.empty_like(sc)
    sc[..., 0:4] = s[..., 0:4] & 63
    m[..., 0:4] = s[..., 4:8] & 63
    sc[..., 4:8] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:8] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def dequant_q4_k(w: np.ndarray, K: int) -> np.ndarray:
    b = _blocks(w, "q4_k", K)
    N, nb = b.shape[:2]
    d = _f16_at(b, 0)
    dmin = _f16_at(b, 2)
    sc, m = q4_k_scale_min(b[..., 4:16])
    qs = b[..., 16:144].reshape(N, nb, 4, 32)
    q = np.stack([qs & 0xF, qs >> 4], axis=3).reshape(N, nb, 8, 32).astype(np.float32)
    dsc = d[..., None] * sc.astype(np.float32)                         # exact
    dm = dmin[..., None] * m.astype(np.float32)                        # exact
    wv = dsc[..., None] * q - dm[..., None]                            # one rounding
    return wv.reshape(N, K)


def dequant_q6_k(w: np.ndarray, K: int) -> np.ndarray:
    b = _blocks(w, "q6_k", K)
    N, nb = b.shape[:2]
    ql = b[..., 0:128].astype(np.int32)
    qh = b[..., 128:192].astype(np.int32)
    sc = np.ascontiguousarray(b[..., 192:208]).view(np.int8).astype(np.float32)
    d = _f16_at(b, 208)
    out = np.empty((N, nb, 256), np.float32)
    l = np.arange(32)
    for h in range(2):
        for s in range(4):
            nib = (ql[..., 64 * h + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 0xF
            hi = (qh[..., 32 * h + l] >> (2 * s)) & 3
            q = ((nib | (hi << 4)) - 32).astype(np.float32)
            scale = sc[..., 8 * h + 2 * s + l // 16]
            out[..., 128 * h + 32 * s + l] = (d[..., None] * scale) * q
    return out.reshape(N, K)


def dequant_mlx_q4(qweight: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                   group_size: int | None = None) -> np.ndarray:
    qweight = np.asarray(qweight)
    if qweight.dtype != np.uint8:
        raise TypeError("MLX qweight must be uint8")
    N, half = qweight.shape
    K = 2 * half
    gs = group_size if group_size is not None else K // scales.shape[1]
    if K % gs or scales.shape != (N, K // gs) or biases.shape != scales.shape:
        raise ValueError("MLX buffer shapes inconsistent")
    q = np.stack([qweight & 0xF, qweight >> 4], axis=-1).reshape(N, K).astype(np.float32)
    s = np.repeat(np.asarray(scales, np.float16).astype(np.float32), gs, axis=1)
    bb = np.repeat(np.asarray(biases, np.float16).astype(np.float32), gs, axis=1)
    return s * q + bb


def dequant(fmt: str, w: np.ndarray, K: int, scales=None, biases=None, group_size=None) -> np.ndarray:
    if fmt == "q8_0":
        return dequant_q8_0(w, K)
    if fmt == "q5_0":
        return dequant_q5_0(w, K)
    if fmt == "q4_k":
        return dequant_q4_k(w, K)
    if fmt == "q6_k":
        return dequant_q6_k(w, K)
    if fmt == "mlx_q4":
        return dequant_mlx_q4(w, scales, biases, group_size)
    raise NotImplementedError(fmt)


# --- the reference's split layouts (repacks done by its GGUF loader) ---------------

def split_q8_0(w: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Wire Q8_0 -> (qweight int8[N,K], scales f16[N,K/32]).

    ``packages/alloy-server/src/alloy_server/gguf/quant.py:497-521``."""
    b = _blocks(w, "q8_0", K)
    N, nb = b.shape[:2]
    scales = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(N, nb).copy()
    qweight = np.ascontiguousarray(b[..., 2:34]).view(np.int8).reshape(N, K).copy()
    return qweight, scales


def split_q5_0(w: np.ndarray, K: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Wire Q5_0 -> (qweight u8[N,K/2], qhigh u8[N,K/2], scales f16[N,K/32]).

    K-sequential nibbles; qhigh byte k/2 holds element k's 5th bit in bit 0 and
    element k+1's in bit 4.  ``.../gguf/quant.py:414-494``."""
    b = _blocks(w, "q5_0", K)
    N, nb = b.shape[:2]
    scales = np.ascontiguousarray(b[..., 0:2]).view(np.float16).reshape(N, nb).copy()
    qh = np.ascontiguousarray(b[..., 2:6]).view("<u4")[..., 0].astype(np.uint32)
    bits = ((qh[..., None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)
    qhigh = (bits[..., 0::2] | (bits[..., 1::2] << 4)).reshape(N, K // 2)
    qs = b[..., 6:22]
    seq = np.concatenate([qs & 0xF, qs >> 4], axis=-1)
    qweight = (seq[..., 0::2] | (seq[..., 1::2] << 4)).astype(np.uint8).reshape(N, K // 2)
    return qweight, qhigh, scales


def dequant_q8_0_split(qweight: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Decode of the split layout, as ``embedding_q8_0`` reads it
    (``packages/alloy-metal/src/alloy/std/quant.py:811-832``)."""
    N, K = qweight.shape
    s = np.repeat(np.asarray(scales, np.float16).astype(np.float32), 32, axis=1)
    return s * qweight.astype(np.float32)


def dequant_q5_0_split(qweight: np.ndarray, qhigh: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Decode of the split layout, as ``embedding_q5_0`` / ``dot_q5_0_v2`` read it
    (``packages/alloy-metal/src/alloy/std/quant.py:1025-1034, 1165-1197``)."""
    N, half = qweight.shape
    K = 2 * half
    nib = np.stack([qweight & 0xF, qweight >> 4], axis=-1).reshape(N, K).astype(np.int32)
    hb = np.stack([qhigh & 1, (qhigh >> 4) & 1], axis=-1).reshape(N, K).astype(np.int32)
    q = ((nib | (hb << 4)) - 16).astype(np.float32)
    s = np.repeat(np.asarray(scales, np.float16).astype(np.float32), 32, axis=1)
    return s * q


def join_q8_0(qweight: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Inverse of ``split_q8_0``: split layout -> wire blocks."""
    N, K = qweight.shape
    nb = K // 32
    out = np.empty((N, nb, 34), np.uint8)
    out[..., 0:2] = np.ascontiguousarray(scales, np.float16).view(np.uint8).reshape(N, nb, 2)
    out[..., 2:34] = np.ascontiguousarray(qweight).view(np.uint8).reshape(N, nb, 32)
    return out.reshape(N, nb * 34)


def join_q5_0(qweight: np.ndarray, qhigh: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Inverse of ``split_q5_0``: split layout -> wire blocks."""
    N, half = qweight.shape
    K = 2 * half
    nb = K // 32
    nib = np.stack([qweight & 0xF, qweight >> 4], axis=-1).reshape(N, nb, 32)
    hb = np.stack([qhigh & 1, (qhigh >> 4) & 1], axis=-1).reshape(N, nb, 32).astype(np.uint32)
    qh = (hb << np.arange(32, dtype=np.uint32)).sum(axis=-1, dtype=np.uint64).astype("<u4")
    out = np.empty((N, nb, 22), np.uint8)
    out[..., 0:2] = np.ascontiguousarray(scales, np.float16).view(np.uint8).reshape(N, nb, 2)
    out[..., 2:6] = qh.view(np.uint8).reshape(N, nb, 4)
    out[..., 6:22] = (nib[..., 0:16] | (nib[..., 16:32] << 4)).astype(np.uint8)
    return out.reshape(N, nb * 22)


# --- dense reference ------------------------------------------------------------------

def ref_matmul(x: np.ndarray, w_deq: np.ndarray) -> np.ndarray:
    """fp64 reference ``y = x @ W^T`` (x given as fp16/fp32 values, W exact fp32)."""
    return np.asarray(x, np.float64) @ np.asarray(w_deq, np.float64).T


def parity_errors(y: np.ndarray, ref: np.ndarray, x: np.ndarray, w_deq: np.ndarray):
    """The north-star metrics: relative Frobenius error, and the worst ratio of the
    per-element error to ``||x_m|| * max|w_n|`` (bar: <= 1e-3 and <= 2e-3)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    err = y - ref
    rel_fro = float(np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-300))
    xn = np.linalg.norm(np.asarray(x, np.float64), axis=1)                     # (M,)
    wmax = np.abs(np.asarray(w_deq, np.float64)).max(axis=1)                    # (N,)
    bound = xn[:, None] * wmax[None, :]
    ratio = float(np.max(np.abs(err) / np.maximum(bound, 1e-300)))
    return rel_fro, ratio
