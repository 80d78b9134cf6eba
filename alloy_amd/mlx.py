"""MLX 4-bit safetensors checkpoints to the buffers of ``MLXQ4Linear`` / ``MLXQ4Embedding``.

Follows the reference's tensor scan (``packages/alloy-server/src/alloy_server/mlx/
loader.py:58-110``): a tensor ``<base>.weight`` is quantized when ``<base>.scales``
exists; its packed uint32 ``[N, K/8]`` weight is reinterpreted as uint8 ``[N, K/2]``
(``mlx_qweight_to_uint8``), and ``.scales`` / ``.biases`` are converted to float16.
Every other tensor is dense (floating tensors converted to ``dense_dtype``).  Only
4-bit checkpoints are accepted (``loader.py:60-63``).
"""

from __future__ import annotations

from contextlib import ExitStack
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .formats import mlx_group_size, mlx_qweight_to_uint8, validate_mlx_buffers

WEIGHT_SUFFIX = ".weight"


def mlx_quantization(config: dict) -> dict | None:
    """The ``quantization`` (or ``quantization_config``) block of an MLX config.json."""
    q = config.get("quantization") or config.get("quantization_config")
    return dict(q) if q else None


@dataclass
class MLXCheckpoint:
    quantized: dict[str, dict[str, torch.Tensor]] = field(default_factory=dict)   # base -> buffers
    dense: dict[str, torch.Tensor] = field(default_factory=dict)
    group_size: int | None = None

    def linear(self, base: str, bias: torch.Tensor | None = None):
        from .modules import MLXQ4Linear
        b = self.quantized[base]
        n, k = b["qweight"].shape[0], b["qweight"].shape[1] * 2
        bias = torch.nn.Parameter(bias, requires_grad=False) if bias is not None else None
        return MLXQ4Linear(in_features=k, out_features=n, bias=bias, **b)

    def embedding(self, base: str):
        from .modules import MLXQ4Embedding
        b = self.quantized[base]
        return MLXQ4Embedding(num_embeddings=b["qweight"].shape[0], embedding_dim=b["qweight"].shape[1] * 2, **b)


def read_mlx_checkpoint(shards: list[str | Path], config: dict | None = None, *,
                        dense_dtype: torch.dtype = torch.float32) -> MLXCheckpoint:
    """Read MLX safetensors shards.  ``config`` (the model's config.json) is checked to be
    a 4-bit quantization when given."""
    from safetensors import safe_open

    if config is not None:
        quant = mlx_quantization(config)
        if quant is None:
            raise ValueError("not an MLX-quantized model")
        if int(quant.get("bits", 0)) != 4:
            raise NotImplementedError(f"only MLX 4-bit is supported, got {quant}")
    out = MLXCheckpoint()
    with ExitStack() as stack:
        index = {}
        for shard in shards:
            h = stack.enter_context(safe_open(str(shard), framework="pt"))
            for key in h.keys():
                index[key] = h
        bases = {k[:-len(WEIGHT_SUFFIX)] for k in index
                 if k.endswith(WEIGHT_SUFFIX) and k[:-len(WEIGHT_SUFFIX)] + ".scales" in index}
        for key, h in index.items():
            if key.endswith((".scales", ".biases")):
                continue
            base = key[:-len(WEIGHT_SUFFIX)] if key.endswith(WEIGHT_SUFFIX) else None
            if base is not None and base in bases:
                q = mlx_qweight_to_uint8(h.get_tensor(key))
                s = index[base + ".scales"].get_tensor(base + ".scales").to(torch.float16)
                b = index[base + ".biases"].get_tensor(base + ".biases").to(torch.float16)
                validate_mlx_buffers(q, s, b, rows=q.shape[0], dim=q.shape[1] * 2, kind=base)
                gs = mlx_group_size(q, s)
                if out.group_size is None:
                    out.group_size = gs
                out.quantized[base] = {"qweight": q, "scales": s, "biases": b}
            else:
                t = h.get_tensor(key)
                out.dense[key] = t.to(dense_dtype) if t.is_floating_point() else t
    return out
