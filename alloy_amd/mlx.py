"""MLX 4-bit safetensors checkpoints to the buffers of ``MLXQ4Linear`` / ``MLXQ4Embedding``.

The checkpoint convention (the one ``packages/alloy-server/src/alloy_server/mlx/
loader.py:58-110`` reads): a quantized weight is stored as ``<base>.weight`` (packed
uint32 ``[N, K/8]``, eight nibbles per word, low first) with ``<base>.scales`` and
``<base>.biases`` beside it; every other tensor is dense.  Here the packed words are
viewed as uint8 ``[N, K/2]`` (``mlx_qweight_to_uint8``), scales and biases become
float16, dense floating tensors ``dense_dtype``; only 4-bit checkpoints are accepted.
"""

from __future__ import annotations

from contextlib import ExitStack
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .formats import check_mlx_buffers, mlx_group_size, mlx_qweight_to_uint8

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
    """Read MLX safetensors shards.  ``config`` (the model's config.json), when given,
    must declare a 4-bit quantization (``NotImplementedError`` for other widths,
    ``ValueError`` for none)."""
    from safetensors import safe_open

    if config is not None:
        quant = mlx_quantization(config)
        if quant is None:
            raise ValueError("config.json declares no MLX quantization")
        if int(quant.get("bits", 0)) != 4:
            raise NotImplementedError(f"MLX checkpoints of {quant.get('bits')} bits are not supported (4 only)")
    ckpt = MLXCheckpoint()
    with ExitStack() as stack:
        handles = [stack.enter_context(safe_open(str(p), framework="pt")) for p in shards]
        where = {key: h for h in handles for key in h.keys()}      # tensor name -> its shard

        def load(key: str) -> torch.Tensor:
            return where[key].get_tensor(key)

        # a quantized weight is the triple <base>.weight / .scales / .biases
        triples = {key[: -len(".scales")] for key in where if key.endswith(".scales")}
        triples = {b for b in triples if b + WEIGHT_SUFFIX in where}
        for base in sorted(triples):
            if base + ".biases" not in where:
                raise ValueError(f"MLX tensor {base} has scales but no biases")
            qweight = mlx_qweight_to_uint8(load(base + WEIGHT_SUFFIX))
            scales, biases = load(base + ".scales").half(), load(base + ".biases").half()
            check_mlx_buffers(qweight, scales, biases, rows=qweight.shape[0], K=2 * qweight.shape[1], what=base)
            ckpt.group_size = ckpt.group_size or mlx_group_size(qweight, scales)
            ckpt.quantized[base] = {"qweight": qweight, "scales": scales, "biases": biases}
        owned = {base + sfx for base in triples for sfx in (WEIGHT_SUFFIX, ".scales", ".biases")}
        for key in where.keys() - owned:
            t = load(key)
            ckpt.dense[key] = t.to(dense_dtype) if t.is_floating_point() else t
    return ckpt
