"""Quantization formats: buffer tables and validation, mirroring the reference.

``QUANT_FORMATS`` follows the reference's table of GGUF formats
(``packages/alloy-server/src/alloy_server/gguf/quant.py:38-78``): the buffers a
quantized Linear holds, their dtypes, and column counts as a function of the
contraction dim.  ``validate_quant_buffers`` / ``validate_mlx_buffers`` raise the
same exception types for the same conditions as the reference
(``gguf/quant.py:81-105``; ``packages/alloy-server/src/alloy_server/mlx/quant.py:88-109``).

Wire-block sizes (bytes per block, weights per block) of the GGUF formats are in
``BLOCK``; ``row_bytes`` gives the bytes of one weight row.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass

import torch

# GGUF wire blocks: name -> (weights per block, bytes per block)
BLOCK = {"q8_0": (32, 34), "q5_0": (32, 22), "q4_k": (256, 144), "q6_k": (256, 210)}


def row_bytes(fmt: str, K: int) -> int:
    qk, bb = BLOCK[fmt]
    if K % qk:
        raise ValueError(f"{fmt}: K={K} not divisible by {qk}")
    return (K // qk) * bb


def bits_per_weight(fmt: str, group_size: int = 64) -> float:
    if fmt in BLOCK:
        qk, bb = BLOCK[fmt]
        return 8.0 * bb / qk
    if fmt == "mlx_q4":
        return 4.0 + 32.0 / group_size
    raise KeyError(fmt)


@dataclass(frozen=True)
class QuantBuffer:
    name: str
    dtype: torch.dtype
    cols: Callable[[int], int]


@dataclass(frozen=True)
class QuantFormat:
    name: str
    align: int
    buffers: tuple[QuantBuffer, ...]

    @property
    def buffer_names(self) -> tuple[str, ...]:
        return tuple(b.name for b in self.buffers)


QUANT_FORMATS: dict[str, QuantFormat] = {
    "q8_0": QuantFormat("q8_0", 32, (
        QuantBuffer("qweight", torch.int8, lambda k: k),
        QuantBuffer("scales", torch.float16, lambda k: k // 32),
    )),
    "q5_0": QuantFormat("q5_0", 32, (
        QuantBuffer("qweight", torch.uint8, lambda k: k // 2),
        QuantBuffer("qhigh", torch.uint8, lambda k: k // 2),
        QuantBuffer("scales", torch.float16, lambda k: k // 32),
    )),
    "q4_k": QuantFormat("q4_k", 256, (
        QuantBuffer("blocks", torch.uint8, lambda k: (k // 256) * 144),
    )),
    "q6_k": QuantFormat("q6_k", 256, (
        QuantBuffer("qweight", torch.uint8, lambda k: (k // 256) * 210),
    )),
}


def validate_quant_buffers(fmt: QuantFormat, buffers: dict[str, torch.Tensor], *, rows: int, dim: int,
                           kind: str) -> None:
    if set(buffers) != set(fmt.buffer_names):
        raise ValueError(f"{fmt.name} {kind} expects buffers {fmt.buffer_names}, got {tuple(buffers)}")
    if dim % fmt.align != 0:
        raise ValueError(f"{fmt.name} {kind} dim {dim} not divisible by {fmt.align}")
    for b in fmt.buffers:
        t = buffers[b.name]
        if t.dtype is not b.dtype:
            raise TypeError(f"{fmt.name} {kind} buffer {b.name!r} requires {b.dtype}, got {t.dtype}")
        if t.ndim != 2:
            raise ValueError(f"{fmt.name} {kind} buffer {b.name!r} must be rank-2, got {tuple(t.shape)}")
        expected = (rows, b.cols(dim))
        if tuple(t.shape) != expected:
            raise ValueError(
                f"{fmt.name} {kind} buffer {b.name!r} shape {tuple(t.shape)} != {expected} (rows={rows} dim={dim})"
            )


def validate_mlx_buffers(qweight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, rows: int,
                         dim: int, kind: str) -> None:
    if qweight.dtype is not torch.uint8:
        raise TypeError(f"MLX {kind} qweight must be uint8, got {qweight.dtype}")
    if scales.dtype is not torch.float16 or biases.dtype is not torch.float16:
        raise TypeError(f"MLX {kind} scales/biases must be float16")
    if tuple(qweight.shape) != (rows, dim // 2) or scales.shape != biases.shape or scales.shape[0] != rows:
        raise ValueError(
            f"MLX {kind} buffer shapes inconsistent: qweight {tuple(qweight.shape)}, "
            f"scales {tuple(scales.shape)} (rows={rows} dim={dim})"
        )
    groups = scales.shape[1]
    if groups == 0 or dim % groups != 0 or (dim // groups) % 8 != 0:
        raise ValueError(f"MLX {kind} group size {dim}/{groups} unsupported (must divide dim, multiple of 8)")


def mlx_group_size(qweight: torch.Tensor, scales: torch.Tensor) -> int:
    """group_size from the qweight/scales column counts
    (``packages/alloy-torch/src/alloy_torch/ops/linalg.py:509-511``)."""
    return (qweight.shape[1] * 2) // scales.shape[1]


def mlx_qweight_to_uint8(weight: torch.Tensor) -> torch.Tensor:
    """MLX packed uint32 weight [N, K/8] -> uint8 [N, K/2], a little-endian
    reinterpret (``packages/alloy-server/src/alloy_server/mlx/quant.py:20-24``)."""
    return weight.contiguous().view(torch.uint8)
