"""Drop-in quantized modules with the reference's buffer tables and forward.

``GGUFQ{8_0,5_0,4_K,6_K}Linear`` mirror ``packages/alloy-server/src/alloy_server/gguf/quant.py:108-193``
(same constructor keywords, buffer names/dtypes/shapes, validation errors and
forward: flatten leading dims, call ``torch.ops.alloy.gguf_*_mm``, add the bias).
``MLXQ4Linear`` mirrors ``packages/alloy-server/src/alloy_server/mlx/quant.py:27-59``.
``MLXMoeExperts`` holds stacked MLX-4 experts with fused gate_up rows
(``[0:I]`` gate, ``[I:2I]`` up, as ``models/qwen3_5.py:232-297`` fuses GGUF
experts) and routes through ``torch.ops.alloy.mlx_moe_routed``.
"""

from __future__ import annotations

import torch

from . import ops as _ops  # noqa: F401  (registers torch.ops.alloy.*)
from .formats import QUANT_FORMATS, QuantFormat, validate_mlx_buffers, validate_quant_buffers

_MM = {
    "q8_0": lambda: torch.ops.alloy.gguf_q8_0_mm.default,
    "q5_0": lambda: torch.ops.alloy.gguf_q5_0_mm.default,
    "q4_k": lambda: torch.ops.alloy.gguf_q4_k_mm.default,
    "q6_k": lambda: torch.ops.alloy.gguf_q6_k_mm.default,
}


_EMBED = {
    "q8_0": lambda: torch.ops.alloy.gguf_q8_0_embedding.default,
    "q5_0": lambda: torch.ops.alloy.gguf_q5_0_embedding.default,
    "q4_k": lambda: torch.ops.alloy.gguf_q4_k_embedding.default,
    "q6_k": lambda: torch.ops.alloy.gguf_q6_k_embedding.default,
}


class GGUFQuantLinear(torch.nn.Module):
    FORMAT: QuantFormat

    def __init__(self, *, in_features: int, out_features: int, bias: torch.nn.Parameter | None = None,
                 **buffers: torch.Tensor) -> None:
        super().__init__()
        validate_quant_buffers(self.FORMAT, buffers, rows=out_features, dim=in_features, kind="linear")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        for b in self.FORMAT.buffers:
            self.register_buffer(b.name, buffers[b.name].contiguous())
        if bias is not None:
            self.bias = bias
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x_shape = x.shape
        flat = x.reshape(-1, self.in_features).contiguous()
        out = _MM[self.FORMAT.name]()(flat, *(self._buffers[b.name] for b in self.FORMAT.buffers))
        if self.bias is not None:
            out = out + self.bias
        return out.reshape(*x_shape[:-1], self.out_features)


class GGUFQ8_0Linear(GGUFQuantLinear):
    """Linear over the reference's split Q8_0 layout (int8 qweight + fp16 scales)."""
    FORMAT = QUANT_FORMATS["q8_0"]


class GGUFQ5_0Linear(GGUFQuantLinear):
    """Linear over the reference's split Q5_0 layout (qweight, qhigh, scales)."""
    FORMAT = QUANT_FORMATS["q5_0"]


class GGUFQ4_KLinear(GGUFQuantLinear):
    """Linear over GGUF-native Q4_K 144-byte superblocks."""
    FORMAT = QUANT_FORMATS["q4_k"]


class GGUFQ6_KLinear(GGUFQuantLinear):
    """Linear over GGUF Q6_K 210-byte blocks."""
    FORMAT = QUANT_FORMATS["q6_k"]


class GGUFQuantEmbedding(torch.nn.Module):
    """Embedding over GGUF packed weights (``S/gguf/quant.py:144-197``): ``forward(ids)``
    returns the exact fp32 rows ``(*ids.shape, embedding_dim)`` times ``embed_scale``."""

    FORMAT: QuantFormat

    def __init__(self, *, num_embeddings: int, embedding_dim: int, embed_scale: float = 1.0,
                 **buffers: torch.Tensor) -> None:
        super().__init__()
        validate_quant_buffers(self.FORMAT, buffers, rows=num_embeddings, dim=embedding_dim, kind="embedding")
        self.num_embeddings = int(num_embeddings)
        self.embedding_dim = int(embedding_dim)
        self.embed_scale = float(embed_scale)
        for b in self.FORMAT.buffers:
            self.register_buffer(b.name, buffers[b.name].contiguous())

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        out = _EMBED[self.FORMAT.name]()(input_ids, *(self._buffers[b.name] for b in self.FORMAT.buffers))
        if self.embed_scale != 1.0:
            out = out * self.embed_scale
        return out


class GGUFQ8_0Embedding(GGUFQuantEmbedding):
    FORMAT = QUANT_FORMATS["q8_0"]


class GGUFQ5_0Embedding(GGUFQuantEmbedding):
    FORMAT = QUANT_FORMATS["q5_0"]


class GGUFQ4_KEmbedding(GGUFQuantEmbedding):
    FORMAT = QUANT_FORMATS["q4_k"]


class GGUFQ6_KEmbedding(GGUFQuantEmbedding):
    FORMAT = QUANT_FORMATS["q6_k"]


_TIED = {GGUFQ8_0Embedding: GGUFQ8_0Linear, GGUFQ5_0Embedding: GGUFQ5_0Linear,
         GGUFQ4_KEmbedding: GGUFQ4_KLinear, GGUFQ6_KEmbedding: GGUFQ6_KLinear}


def tied_output_head(embedding: torch.nn.Module, output: torch.nn.Module | None = None) -> torch.nn.Module:
    """The quantized lm_head that shares a quantized input embedding's buffers
    (``S/gguf/quant.py:553-623``): a Linear output head without bias becomes the
    matching GGUF Linear over the same rows; anything else raises as the reference does.
    An ``MLXQ4Embedding`` becomes an ``MLXQ4Linear`` over its buffers
    (``packages/alloy-server/src/alloy_server/mlx/quant.py:148-168``)."""
    if isinstance(embedding, MLXQ4Embedding):
        if output is not None and not isinstance(output, torch.nn.Linear):
            raise TypeError(f"Tied MLX embeddings require a Linear output head, got {type(output).__name__}")
        return MLXQ4Linear(in_features=embedding.embedding_dim, out_features=embedding.num_embeddings,
                           qweight=embedding.qweight, scales=embedding.scales, biases=embedding.biases)
    cls = _TIED.get(type(embedding))
    if cls is None:
        raise TypeError(f"no tied output head for {type(embedding).__name__}")
    name = embedding.FORMAT.name.upper()
    if output is not None and not isinstance(output, torch.nn.Linear):
        raise TypeError(f"Tied {name} GGUF embeddings require a Linear output head, got {type(output).__name__}")
    if output is not None and output.bias is not None:
        raise NotImplementedError(f"Tied {name} GGUF output head bias is not supported")
    bufs = {b.name: embedding._buffers[b.name] for b in embedding.FORMAT.buffers}
    return cls(in_features=embedding.embedding_dim, out_features=embedding.num_embeddings, **bufs)


class MLXQ4Embedding(torch.nn.Module):
    """Embedding over MLX 4-bit affine weights: exact fp32 rows of ``mlx_q4_embedding``."""

    def __init__(self, *, num_embeddings: int, embedding_dim: int, qweight: torch.Tensor, scales: torch.Tensor,
                 biases: torch.Tensor) -> None:
        super().__init__()
        validate_mlx_buffers(qweight, scales, biases, rows=num_embeddings, dim=embedding_dim, kind="embedding")
        self.num_embeddings, self.embedding_dim = int(num_embeddings), int(embedding_dim)
        for name, t in (("qweight", qweight), ("scales", scales), ("biases", biases)):
            self.register_buffer(name, t.contiguous())

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return torch.ops.alloy.mlx_q4_embedding.default(input_ids, self.qweight, self.scales, self.biases)


class MLXQ4Linear(torch.nn.Module):
    """Linear over MLX affine int4 groups: qweight (out, in//2) uint8, fp16 scales/biases."""

    def __init__(self, *, in_features: int, out_features: int, qweight: torch.Tensor, scales: torch.Tensor,
                 biases: torch.Tensor, bias: torch.nn.Parameter | None = None) -> None:
        super().__init__()
        validate_mlx_buffers(qweight, scales, biases, rows=out_features, dim=in_features, kind="linear")
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.register_buffer("qweight", qweight.contiguous())
        self.register_buffer("scales", scales.contiguous())
        self.register_buffer("biases", biases.contiguous())
        if bias is not None:
            self.bias = bias
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x_shape = x.shape
        flat = x.reshape(-1, self.in_features).contiguous()
        out = torch.ops.alloy.mlx_q4_mm.default(flat, self.qweight, self.scales, self.biases)
        if self.bias is not None:
            out = out + self.bias
        return out.reshape(*x_shape[:-1], self.out_features)


class MLXMoeExperts(torch.nn.Module):
    """Stacked MLX-4 routed experts: gate_up (E, 2I, H/2) + down (E, H, I/2).

    ``forward(hidden (T,H) f16, router_logits (T,E) f32) -> (T,H) f32`` — top-k
    routing, softmax over the k winners, ``sum_s w_s * down_e(silu(gate_e x) * up_e x)``.
    """

    def __init__(self, *, num_experts: int, top_k: int, hidden_size: int, moe_intermediate: int,
                 gate_up_qweight, gate_up_scales, gate_up_biases, down_qweight, down_scales, down_biases):
        super().__init__()
        self.num_experts, self.top_k = int(num_experts), int(top_k)
        self.hidden_size, self.moe_intermediate = int(hidden_size), int(moe_intermediate)
        E, I, H = self.num_experts, self.moe_intermediate, self.hidden_size
        validate_mlx_buffers(gate_up_qweight.reshape(E * 2 * I, -1), gate_up_scales.reshape(E * 2 * I, -1),
                             gate_up_biases.reshape(E * 2 * I, -1), rows=E * 2 * I, dim=H, kind="moe gate_up")
        validate_mlx_buffers(down_qweight.reshape(E * H, -1), down_scales.reshape(E * H, -1),
                             down_biases.reshape(E * H, -1), rows=E * H, dim=I, kind="moe down")
        for name, t in (("gate_up_qweight", gate_up_qweight), ("gate_up_scales", gate_up_scales),
                        ("gate_up_biases", gate_up_biases), ("down_qweight", down_qweight),
                        ("down_scales", down_scales), ("down_biases", down_biases)):
            self.register_buffer(name, t.contiguous())

    def forward(self, hidden: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        shape = hidden.shape
        flat = hidden.reshape(-1, self.hidden_size).contiguous()
        logits = router_logits.reshape(-1, self.num_experts).to(torch.float32).contiguous()
        y = torch.ops.alloy.mlx_moe_routed.default(
            flat, logits, self.gate_up_qweight, self.gate_up_scales, self.gate_up_biases, self.down_qweight,
            self.down_scales, self.down_biases, self.num_experts, self.top_k, self.moe_intermediate)
        return y.reshape(*shape[:-1], self.hidden_size)


class GGUFQwen35MoeExperts(torch.nn.Module):
    """Stacked GGUF routed experts (``S/models/qwen3_5.py:232-301``): ``gate_up_blocks``
    (E, 2I, (H/256)*144) native Q4_K with rows ``[0:I]`` gate and ``[I:2I]`` up, and
    ``down_qweight`` (E, H, (I/256)*210) Q6_K.  A weight holder: the compute runs in
    ``gguf_moe_routed``, driven by :class:`GGUFQwen35MoeBlock`; ``forward`` raises."""

    def __init__(self, *, gate_up_blocks: torch.Tensor, down_qweight: torch.Tensor, num_experts: int,
                 hidden_size: int, moe_intermediate_size: int) -> None:
        super().__init__()
        if hidden_size % 256 != 0 or moe_intermediate_size % 256 != 0:
            raise ValueError("Qwen3.5-MoE expert dims must be divisible by 256: "
                             f"hidden={hidden_size} moe_intermediate={moe_intermediate_size}")
        expected = {"gate_up_blocks": (num_experts, 2 * moe_intermediate_size, hidden_size // 256 * 144),
                    "down_qweight": (num_experts, hidden_size, moe_intermediate_size // 256 * 210)}
        actual = {"gate_up_blocks": tuple(gate_up_blocks.shape), "down_qweight": tuple(down_qweight.shape)}
        if actual != expected:
            raise ValueError(f"Qwen3.5-MoE expert weight shapes do not match config: got {actual} expected {expected}")
        if gate_up_blocks.dtype is not torch.uint8 or down_qweight.dtype is not torch.uint8:
            raise TypeError("Qwen3.5-MoE expert weights must be uint8 packed blocks")
        self.num_experts = int(num_experts)
        self.hidden_size = int(hidden_size)
        self.moe_intermediate_size = int(moe_intermediate_size)
        self.register_buffer("gate_up_blocks", gate_up_blocks.contiguous())
        self.register_buffer("down_qweight", down_qweight.contiguous())

    def forward(self, *args, **kwargs):
        raise RuntimeError("GGUFQwen35MoeExperts is a weight holder; compute is driven by GGUFQwen35MoeBlock "
                           "via the gguf_moe_routed op, not this forward.")


class GGUFQwen35MoeBlock(torch.nn.Module):
    """Sparse MoE block (``S/models/qwen3_5.py:304-343``):
    ``out = gguf_moe_routed(x, x @ Wr^T, experts...) + sigmoid(Wg x) * shared(x)``.

    ``orig_block`` provides ``gate`` (router linear), ``experts``
    (:class:`GGUFQwen35MoeExperts`), ``shared_expert`` and ``shared_expert_gate``."""

    def __init__(self, orig_block: torch.nn.Module, *, num_experts: int, top_k: int, moe_intermediate: int) -> None:
        super().__init__()
        self.gate = orig_block.gate
        self.experts = orig_block.experts
        self.shared_expert = orig_block.shared_expert
        self.shared_expert_gate = orig_block.shared_expert_gate
        self.num_experts = int(num_experts)
        self.top_k = int(top_k)
        self.moe_intermediate = int(moe_intermediate)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        in_shape = hidden_states.shape
        x = hidden_states.reshape(-1, in_shape[-1])
        router_logits = torch.nn.functional.linear(x, self.gate.weight)
        routed = torch.ops.alloy.gguf_moe_routed(x, router_logits, self.experts.gate_up_blocks,
                                                 self.experts.down_qweight, self.num_experts, self.top_k,
                                                 self.moe_intermediate)
        shared = self.shared_expert(x)
        shared = torch.sigmoid(self.shared_expert_gate(x)) * shared
        return (routed + shared).reshape(in_shape)
