"""Weight formats of the quantized-linear path: GGUF wire-block geometry, the buffers
each drop-in module holds, and their validation.

The buffer sets are the reference modules' interface (names, dtypes and column counts
of ``packages/alloy-server/src/alloy_server/gguf/quant.py:36-78`` and
``packages/alloy-server/src/alloy_server/mlx/quant.py:27-59``): Q8_0 and Q5_0 in the
reference's split layout, Q4_K and Q6_K as raw GGUF rows, MLX 4-bit as uint8 nibbles
plus fp16 group scales and biases.  The checks keep the reference's exception contract
(``ValueError`` for a wrong buffer set, shape or divisibility, ``TypeError`` for a
dtype; ``gguf/quant.py:81-105``, ``mlx/quant.py:88-109``).
"""

from __future__ import annotations

import torch

# GGUF wire blocks: name -> (weights per block, bytes per block)
BLOCK = {"q8_0": (32, 34), "q5_0": (32, 22), "q4_k": (256, 144), "q6_k": (256, 210)}


def row_bytes(fmt: str, K: int) -> int:
    """Bytes of one weight row of K elements in GGUF wire blocks."""
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


def module_buffers(fmt: str, rows: int, K: int) -> dict[str, tuple[torch.dtype, tuple[int, int]]]:
    """The buffers (name -> (dtype, shape)) a quantized weight of ``rows`` x ``K`` is held
    in, in the order the reference op takes them.  K must be a multiple of the block."""
    if fmt == "q8_0":
        return {"qweight": (torch.int8, (rows, K)), "scales": (torch.float16, (rows, K // 32))}
    if fmt == "q5_0":
        half = (rows, K // 2)
        return {"qweight": (torch.uint8, half), "qhigh": (torch.uint8, half),
                "scales": (torch.float16, (rows, K // 32))}
    if fmt == "q4_k":
        return {"blocks": (torch.uint8, (rows, row_bytes(fmt, K)))}
    if fmt == "q6_k":
        return {"qweight": (torch.uint8, (rows, row_bytes(fmt, K)))}
    raise KeyError(fmt)


def check_module_buffers(fmt: str, buffers: dict[str, torch.Tensor], *, rows: int, K: int, what: str) -> None:
    """Raise unless ``buffers`` are exactly the ``module_buffers(fmt, rows, K)`` set."""
    qk = BLOCK[fmt][0]
    if K % qk:
        raise ValueError(f"{what}: {fmt} rows of {K} elements are not divisible into blocks of {qk}")
    want = module_buffers(fmt, rows, K)
    if set(buffers) != set(want):
        raise ValueError(f"{what}: a {fmt} weight is held in buffers ({', '.join(want)}), "
                         f"given ({', '.join(buffers) or 'nothing'})")
    for name, (dtype, shape) in want.items():
        t = buffers[name]
        if t.dtype != dtype:
            raise TypeError(f"{what}: {fmt} buffer {name} holds {dtype}, given {t.dtype}")
        if tuple(t.shape) != shape:
            raise ValueError(f"{what}: {fmt} buffer {name} for {rows} rows of {K} elements is {shape}, "
                             f"given {tuple(t.shape)}")


def check_mlx_buffers(qweight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, rows: int, K: int,
                      what: str) -> int:
    """Raise unless (qweight, scales, biases) hold ``rows`` x ``K`` MLX 4-bit weights;
    returns the group size."""
    if qweight.dtype != torch.uint8:
        raise TypeError(f"{what}: MLX qweight holds uint8 nibble pairs, given {qweight.dtype}")
    for name, t in (("scales", scales), ("biases", biases)):
        if t.dtype != torch.float16:
            raise TypeError(f"{what}: MLX {name} are float16, given {t.dtype}")
    if K % 2 or tuple(qweight.shape) != (rows, K // 2):
        raise ValueError(f"{what}: MLX qweight for {rows} rows of {K} elements is ({rows}, {K // 2}), "
                         f"given {tuple(qweight.shape)}")
    if scales.ndim != 2 or scales.shape[0] != rows or tuple(biases.shape) != tuple(scales.shape):
        raise ValueError(f"{what}: MLX scales {tuple(scales.shape)} and biases {tuple(biases.shape)} "
                         f"must both be ({rows}, groups)")
    groups = scales.shape[1]
    gs = K // groups if groups else 0
    if groups == 0 or gs * groups != K or gs % 8:
        raise ValueError(f"{what}: {K} elements in {groups} MLX groups is not a whole group size "
                         f"that is a multiple of 8")
    return gs


def mlx_group_size(qweight: torch.Tensor, scales: torch.Tensor) -> int:
    """group_size from the qweight/scales column counts
    (``packages/alloy-torch/src/alloy_torch/ops/linalg.py:509-511``)."""
    return (qweight.shape[1] * 2) // scales.shape[1]


def mlx_qweight_to_uint8(weight: torch.Tensor) -> torch.Tensor:
    """MLX packed uint32 weight [N, K/8] -> uint8 [N, K/2]: the little-endian bytes of
    each word, low nibble first (``packages/alloy-server/src/alloy_server/mlx/quant.py:20-24``)."""
    return weight.contiguous().view(torch.uint8)
