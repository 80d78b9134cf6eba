"""Seeded synthetic weights/activations with the distributions of the benchmark configs.

Distributions (one per format, as the benchmark configurations state them):
  Q8_0   d = fp16(|N(0,1)|*0.01), q ~ U{-127..127} int8
  Q4_K   d, dmin = fp16(|N(0,1)|*0.005), 12 scale bytes + 128 quant bytes ~ U{0..255}
  Q6_K   ql, qh ~ U{0..255}, scales ~ U{-64..63} int8, d = fp16(|N(0,1)|*0.002)
  Q5_0   d = fp16(|N(0,1)|*0.01) (unspecified upstream; chosen as Q8_0), qh, qs ~ U{0..255}
  MLX4   qweight ~ U{0..255}, scales = fp16(|N(0,1)|*0.01), biases = fp16(N(0, 0.01))
  x      fp16 N(0,1)

``numpy_*`` generators are seeded ``np.random.Generator`` streams (used for parity
tests); ``torch_*`` generators build the same distributions directly on a device
with a seeded ``torch.Generator`` (used for the large benchmark shapes).
"""

from __future__ import annotations

import numpy as np
import torch

from .formats import BLOCK

D_SCALE = {"q8_0": 0.01, "q5_0": 0.01, "q4_k": 0.005, "q6_k": 0.002}


def _put_f16(blk: np.ndarray, off: int, vals: np.ndarray) -> None:
    blk[..., off:off + 2] = vals.astype(np.float16).view(np.uint8).reshape(vals.shape + (2,))


def numpy_blocks(fmt: str, N: int, K: int, rng: np.random.Generator) -> np.ndarray:
    """GGUF wire blob uint8[N, K/QK*BB] for fmt in q8_0, q5_0, q4_k, q6_k."""
    qk, bb = BLOCK[fmt]
    nb = K // qk
    blk = rng.integers(0, 256, size=(N, nb, bb), dtype=np.uint8)
    d = np.abs(rng.standard_normal((N, nb))) * D_SCALE[fmt]
    if fmt == "q8_0":
        _put_f16(blk, 0, d)
        blk[..., 2:] = rng.integers(-127, 128, size=(N, nb, 32), dtype=np.int8).view(np.uint8)
    elif fmt == "q5_0":
        _put_f16(blk, 0, d)
    elif fmt == "q4_k":
        _put_f16(blk, 0, d)
        _put_f16(blk, 2, np.abs(rng.standard_normal((N, nb))) * D_SCALE[fmt])
    elif fmt == "q6_k":
        blk[..., 192:208] = rng.integers(-64, 64, size=(N, nb, 16), dtype=np.int8).view(np.uint8)
        _put_f16(blk, 208, d)
    else:
        raise KeyError(fmt)
    return blk.reshape(N, nb * bb)


def numpy_mlx(N: int, K: int, group_size: int, rng: np.random.Generator):
    """(qweight uint8[N,K/2], scales f16[N,K/gs], biases f16[N,K/gs])."""
    qweight = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    g = K // group_size
    scales = (np.abs(rng.standard_normal((N, g))) * 0.01).astype(np.float16)
    biases = (rng.standard_normal((N, g)) * 0.01).astype(np.float16)
    return qweight, scales, biases


def numpy_x(M: int, K: int, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal((M, K)).astype(np.float16)


# ------------------------------------------------------------------ on-device

def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _abs_normal_f16(shape, scale, g, device) -> torch.Tensor:
    return (torch.randn(shape, generator=g, device=device).abs_() * scale).to(torch.float16)


def torch_blocks(fmt: str, N: int, K: int, seed: int, device) -> torch.Tensor:
    """Same distribution as numpy_blocks, generated on `device`."""
    qk, bb = BLOCK[fmt]
    nb = K // qk
    g = _gen(seed, device)
    blk = torch.randint(0, 256, (N, nb, bb), generator=g, device=device, dtype=torch.uint8)
    d = _abs_normal_f16((N, nb), D_SCALE[fmt], g, device)
    if fmt == "q8_0":
        blk[..., 0:2] = d.view(torch.uint8).view(N, nb, 2)
        q = torch.randint(-127, 128, (N, nb, 32), generator=g, device=device, dtype=torch.int8)
        blk[..., 2:] = q.view(torch.uint8)
    elif fmt == "q5_0":
        blk[..., 0:2] = d.view(torch.uint8).view(N, nb, 2)
    elif fmt == "q4_k":
        blk[..., 0:2] = d.view(torch.uint8).view(N, nb, 2)
        dm = _abs_normal_f16((N, nb), D_SCALE[fmt], g, device)
        blk[..., 2:4] = dm.view(torch.uint8).view(N, nb, 2)
    elif fmt == "q6_k":
        sc = torch.randint(-64, 64, (N, nb, 16), generator=g, device=device, dtype=torch.int8)
        blk[..., 192:208] = sc.view(torch.uint8)
        blk[..., 208:210] = d.view(torch.uint8).view(N, nb, 2)
    else:
        raise KeyError(fmt)
    return blk.view(N, nb * bb)


def torch_q8_0_split(N: int, K: int, seed: int, device):
    """Q8_0 in the reference operator's split layout (int8 quants [N, K], fp16 scales
    [N, K/32]) with the wire blocks' distribution: quants uniform in [-127, 127], scales
    |N(0,1)| * 0.01 — the same 34 bytes per 32 weights."""
    g = _gen(seed, device)
    qweight = torch.randint(-127, 128, (N, K), generator=g, device=device, dtype=torch.int8)
    scales = _abs_normal_f16((N, K // 32), D_SCALE["q8_0"], g, device)
    return qweight, scales


def torch_mlx(N: int, K: int, group_size: int, seed: int, device):
    g = _gen(seed, device)
    qweight = torch.randint(0, 256, (N, K // 2), generator=g, device=device, dtype=torch.uint8)
    gcount = K // group_size
    scales = _abs_normal_f16((N, gcount), 0.01, g, device)
    biases = (torch.randn((N, gcount), generator=g, device=device) * 0.01).to(torch.float16)
    return qweight, scales, biases


def torch_x(M: int, K: int, seed: int, device) -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn((M, K), generator=g, device=device).to(torch.float16)
