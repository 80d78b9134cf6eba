"""Drop-in quantized modules over ``torch.ops.alloy``.

Constructor keywords, buffer names and forward semantics are the reference modules'
interface, so a model built for the reference binds to these unchanged:

* ``GGUFQ{8_0,5_0,4_K,6_K}Linear(in_features=, out_features=, bias=, <buffers>)`` —
  ``packages/alloy-server/src/alloy_server/gguf/quant.py:108-143``: ``forward`` flattens
  the leading dimensions, calls ``gguf_<fmt>_mm`` and adds the bias;
* ``GGUFQ*Embedding(num_embeddings=, embedding_dim=, embed_scale=, <buffers>)`` —
  ``gguf/quant.py:144-197``, and ``tied_output_head`` (``gguf/quant.py:553-623``);
* ``MLXQ4Linear`` / ``MLXQ4Embedding`` — ``packages/alloy-server/src/alloy_server/mlx/quant.py:27-85, 148-168``;
* ``GGUFQwen35MoeExperts`` / ``GGUFQwen35MoeBlock`` —
  ``packages/alloy-server/src/alloy_server/models/qwen3_5.py:232-343``;
* ``MLXMoeExperts``: stacked MLX 4-bit experts (fused gate/up rows) for ``mlx_moe_routed``.

Buffer checks raise ``ValueError`` (shape, divisibility, buffer set) or ``TypeError``
(dtype), as the reference's do.
"""

from __future__ import annotations

import torch

from . import ops as _ops  # noqa: F401  (registers torch.ops.alloy.*)
from .formats import check_mlx_buffers, check_module_buffers, module_buffers


def _op(name: str):
    return getattr(torch.ops.alloy, name).default


def _hold(module: torch.nn.Module, buffers: dict[str, torch.Tensor]) -> None:
    for name, t in buffers.items():
        module.register_buffer(name, t.contiguous())


def _flat_apply(x: torch.Tensor, k: int, n: int, fn, bias) -> torch.Tensor:
    """fn over x viewed as (rows, k), the result viewed back as (..., n), plus bias."""
    lead = x.shape[:-1]
    y = fn(x.reshape(-1, k).contiguous())
    if bias is not None:
        y = y + bias
    return y.reshape(*lead, n)


class _GGUFLinear(torch.nn.Module):
    fmt = ""

    def __init__(self, *, in_features: int, out_features: int, bias: torch.nn.Parameter | None = None,
                 **buffers: torch.Tensor) -> None:
        super().__init__()
        what = f"{type(self).__name__}({in_features} -> {out_features})"
        check_module_buffers(self.fmt, buffers, rows=out_features, K=in_features, what=what)
        self.in_features, self.out_features = int(in_features), int(out_features)
        # buffers in the op's argument order
        _hold(self, {name: buffers[name] for name in module_buffers(self.fmt, 0, in_features)})
        self.register_parameter("bias", bias)

    def _weights(self) -> list[torch.Tensor]:
        return [self._buffers[name] for name in module_buffers(self.fmt, 0, self.in_features)]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        op, w = _op(f"gguf_{self.fmt}_mm"), self._weights()
        return _flat_apply(x, self.in_features, self.out_features, lambda a: op(a, *w), self.bias)


class GGUFQ8_0Linear(_GGUFLinear):
    """Q8_0 in the reference's split layout: ``qweight`` int8 [N, K], ``scales`` fp16 [N, K/32]."""
    fmt = "q8_0"


class GGUFQ5_0Linear(_GGUFLinear):
    """Q5_0 in the reference's split layout: ``qweight``, ``qhigh`` uint8 [N, K/2], ``scales`` fp16 [N, K/32]."""
    fmt = "q5_0"


class GGUFQ4_KLinear(_GGUFLinear):
    """Q4_K as GGUF rows: ``blocks`` uint8 [N, K/256*144]."""
    fmt = "q4_k"


class GGUFQ6_KLinear(_GGUFLinear):
    """Q6_K as GGUF rows: ``qweight`` uint8 [N, K/256*210]."""
    fmt = "q6_k"


GGUFQuantLinear = _GGUFLinear


class _GGUFEmbedding(torch.nn.Module):
    fmt = ""
    linear: type[_GGUFLinear]

    def __init__(self, *, num_embeddings: int, embedding_dim: int, embed_scale: float = 1.0,
                 **buffers: torch.Tensor) -> None:
        super().__init__()
        what = f"{type(self).__name__}({num_embeddings} x {embedding_dim})"
        check_module_buffers(self.fmt, buffers, rows=num_embeddings, K=embedding_dim, what=what)
        self.num_embeddings, self.embedding_dim = int(num_embeddings), int(embedding_dim)
        self.embed_scale = float(embed_scale)
        _hold(self, {name: buffers[name] for name in module_buffers(self.fmt, 0, embedding_dim)})

    def weights(self) -> dict[str, torch.Tensor]:
        return {name: self._buffers[name] for name in module_buffers(self.fmt, 0, self.embedding_dim)}

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        rows = _op(f"gguf_{self.fmt}_embedding")(input_ids, *self.weights().values())
        return rows if self.embed_scale == 1.0 else rows * self.embed_scale


class GGUFQ8_0Embedding(_GGUFEmbedding):
    fmt, linear = "q8_0", GGUFQ8_0Linear


class GGUFQ5_0Embedding(_GGUFEmbedding):
    fmt, linear = "q5_0", GGUFQ5_0Linear


class GGUFQ4_KEmbedding(_GGUFEmbedding):
    fmt, linear = "q4_k", GGUFQ4_KLinear


class GGUFQ6_KEmbedding(_GGUFEmbedding):
    fmt, linear = "q6_k", GGUFQ6_KLinear


GGUFQuantEmbedding = _GGUFEmbedding


class MLXQ4Linear(torch.nn.Module):
    """MLX affine 4-bit linear: ``qweight`` uint8 [N, K/2], ``scales`` / ``biases`` fp16 [N, K/gs]."""

    def __init__(self, *, in_features: int, out_features: int, qweight: torch.Tensor, scales: torch.Tensor,
                 biases: torch.Tensor, bias: torch.nn.Parameter | None = None) -> None:
        super().__init__()
        self.group_size = check_mlx_buffers(qweight, scales, biases, rows=out_features, K=in_features,
                                            what=f"MLXQ4Linear({in_features} -> {out_features})")
        self.in_features, self.out_features = int(in_features), int(out_features)
        _hold(self, {"qweight": qweight, "scales": scales, "biases": biases})
        self.register_parameter("bias", bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        op, w = _op("mlx_q4_mm"), (self.qweight, self.scales, self.biases)
        return _flat_apply(x, self.in_features, self.out_features, lambda a: op(a, *w), self.bias)


class MLXQ4Embedding(torch.nn.Module):
    """MLX 4-bit embedding: exact fp32 rows of ``mlx_q4_embedding``."""

    def __init__(self, *, num_embeddings: int, embedding_dim: int, qweight: torch.Tensor, scales: torch.Tensor,
                 biases: torch.Tensor) -> None:
        super().__init__()
        self.group_size = check_mlx_buffers(qweight, scales, biases, rows=num_embeddings, K=embedding_dim,
                                            what=f"MLXQ4Embedding({num_embeddings} x {embedding_dim})")
        self.num_embeddings, self.embedding_dim = int(num_embeddings), int(embedding_dim)
        _hold(self, {"qweight": qweight, "scales": scales, "biases": biases})

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return _op("mlx_q4_embedding")(input_ids, self.qweight, self.scales, self.biases)


def tied_output_head(embedding: torch.nn.Module, output: torch.nn.Module | None = None) -> torch.nn.Module:
    """The quantized output head over a quantized input embedding's own buffers (no
    copy): the matching Linear of its format, ``num_embeddings`` outputs.  ``output``,
    the model's unquantized head if any, must be a bias-free ``nn.Linear``
    (``TypeError`` / ``NotImplementedError`` otherwise, as ``gguf/quant.py:553-623`` and
    ``mlx/quant.py:148-168``)."""
    if not isinstance(embedding, (_GGUFEmbedding, MLXQ4Embedding)):
        raise TypeError(f"tied_output_head needs a quantized embedding, given {type(embedding).__name__}")
    if output is not None:
        if not isinstance(output, torch.nn.Linear):
            raise TypeError(f"a tied quantized head replaces an nn.Linear, given {type(output).__name__}")
        if output.bias is not None:
            raise NotImplementedError("a tied quantized head has no bias; the given head has one")
    n, k = embedding.num_embeddings, embedding.embedding_dim
    if isinstance(embedding, MLXQ4Embedding):
        return MLXQ4Linear(in_features=k, out_features=n, qweight=embedding.qweight, scales=embedding.scales,
                           biases=embedding.biases)
    return embedding.linear(in_features=k, out_features=n, **embedding.weights())


class MLXMoeExperts(torch.nn.Module):
    """Stacked MLX-4 routed experts: gate_up (E, 2I, H/2) with rows ``[0:I]`` gate and
    ``[I:2I]`` up (the fusion ``models/qwen3_5.py:383-385`` applies to GGUF experts),
    down (E, H, I/2), fp16 scales / biases per group.

    ``forward(hidden (..., H) f16, router_logits (..., E)) -> (..., H) f32``: top-k
    routing, softmax over the k winners, ``sum_s w_s * down_e(silu(gate_e x) * up_e x)``.
    """

    def __init__(self, *, num_experts: int, top_k: int, hidden_size: int, moe_intermediate: int,
                 gate_up_qweight, gate_up_scales, gate_up_biases, down_qweight, down_scales, down_biases):
        super().__init__()
        E, H, I = int(num_experts), int(hidden_size), int(moe_intermediate)
        self.num_experts, self.top_k, self.hidden_size, self.moe_intermediate = E, int(top_k), H, I
        for part, (q, s, b), rows, k in (("gate_up", (gate_up_qweight, gate_up_scales, gate_up_biases), 2 * I, H),
                                         ("down", (down_qweight, down_scales, down_biases), H, I)):
            if q.ndim != 3 or q.shape[0] != E or s.ndim != 3 or s.shape[0] != E:
                raise ValueError(f"MLXMoeExperts {part}: buffers must be stacked over {E} experts, "
                                 f"given {tuple(q.shape)} and {tuple(s.shape)}")
            check_mlx_buffers(q.reshape(E * rows, -1), s.reshape(E * rows, -1), b.reshape(E * rows, -1),
                              rows=E * rows, K=k, what=f"MLXMoeExperts {part}")
        _hold(self, {"gate_up_qweight": gate_up_qweight, "gate_up_scales": gate_up_scales,
                     "gate_up_biases": gate_up_biases, "down_qweight": down_qweight, "down_scales": down_scales,
                     "down_biases": down_biases})

    def forward(self, hidden: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        lead = hidden.shape[:-1]
        x = hidden.reshape(-1, self.hidden_size).contiguous()
        logits = router_logits.reshape(-1, self.num_experts).float().contiguous()
        y = _op("mlx_moe_routed")(x, logits, self.gate_up_qweight, self.gate_up_scales, self.gate_up_biases,
                                  self.down_qweight, self.down_scales, self.down_biases, self.num_experts,
                                  self.top_k, self.moe_intermediate)
        return y.reshape(*lead, self.hidden_size)


class GGUFQwen35MoeExperts(torch.nn.Module):
    """Stacked GGUF routed experts: ``gate_up_blocks`` uint8 (E, 2I, H/256*144), native
    Q4_K with rows ``[0:I]`` gate and ``[I:2I]`` up, and ``down_qweight`` uint8
    (E, H, I/256*210), Q6_K.  It only holds the weights (as the reference's container
    does): :class:`GGUFQwen35MoeBlock` runs them through ``gguf_moe_routed`` and
    ``forward`` raises ``RuntimeError``."""

    def __init__(self, *, gate_up_blocks: torch.Tensor, down_qweight: torch.Tensor, num_experts: int,
                 hidden_size: int, moe_intermediate_size: int) -> None:
        super().__init__()
        E, H, I = int(num_experts), int(hidden_size), int(moe_intermediate_size)
        if H % 256 or I % 256:
            raise ValueError(f"GGUF MoE experts are Q4_K / Q6_K rows: hidden {H} and intermediate {I} "
                             f"must be multiples of 256")
        want = {"gate_up_blocks": (E, 2 * I, H // 256 * 144), "down_qweight": (E, H, I // 256 * 210)}
        for name, t in (("gate_up_blocks", gate_up_blocks), ("down_qweight", down_qweight)):
            if tuple(t.shape) != want[name]:
                raise ValueError(f"GGUF MoE {name} for E={E}, H={H}, I={I} is {want[name]}, "
                                 f"given {tuple(t.shape)}")
            if t.dtype != torch.uint8:
                raise TypeError(f"GGUF MoE {name} holds uint8 blocks, given {t.dtype}")
        self.num_experts, self.hidden_size, self.moe_intermediate_size = E, H, I
        _hold(self, {"gate_up_blocks": gate_up_blocks, "down_qweight": down_qweight})

    def forward(self, *args, **kwargs):
        raise RuntimeError("GGUFQwen35MoeExperts only holds the expert weights; GGUFQwen35MoeBlock runs them "
                           "(torch.ops.alloy.gguf_moe_routed)")


class GGUFQwen35MoeBlock(torch.nn.Module):
    """Sparse MoE block: ``gguf_moe_routed(x, x Wr^T, experts) + sigmoid(x Wg^T) * shared(x)``.

    ``orig_block`` supplies ``gate`` (the router linear), ``experts``
    (:class:`GGUFQwen35MoeExperts`), ``shared_expert`` and ``shared_expert_gate``
    (``models/qwen3_5.py:304-343``)."""

    def __init__(self, orig_block: torch.nn.Module, *, num_experts: int, top_k: int, moe_intermediate: int) -> None:
        super().__init__()
        for name in ("gate", "experts", "shared_expert", "shared_expert_gate"):
            setattr(self, name, getattr(orig_block, name))
        self.num_experts, self.top_k, self.moe_intermediate = int(num_experts), int(top_k), int(moe_intermediate)

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1])
        routed = torch.ops.alloy.gguf_moe_routed(x, torch.nn.functional.linear(x, self.gate.weight),
                                                 self.experts.gate_up_blocks, self.experts.down_qweight,
                                                 self.num_experts, self.top_k, self.moe_intermediate)
        gated_shared = torch.sigmoid(self.shared_expert_gate(x)) * self.shared_expert(x)
        return (routed + gated_shared).reshape(shape)
