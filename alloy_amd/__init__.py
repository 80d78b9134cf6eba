"""alloy_amd — MI355X-native (gfx950) quantized-weight matmul.

Drop-in for Alloy's quantized-linear path: GGUF Q8_0 / Q5_0 / Q4_K / Q6_K and
MLX 4-bit affine weights, decode GEMV, prefill GEMM and routed-expert MoE, as
hand-written HIP kernels behind a C ABI (``include/alloy_amd.h``) bound with
ctypes.  Importing the package registers the ``torch.ops.alloy.*`` ops.
"""

from . import formats, gguf, mlx, synth
from ._lib import LIB_PATH, LibraryMissing, lib
from .modules import (GGUFQ4_KEmbedding, GGUFQ4_KLinear, GGUFQ5_0Embedding, GGUFQ5_0Linear, GGUFQ6_KEmbedding,
                      GGUFQ6_KLinear, GGUFQ8_0Embedding, GGUFQ8_0Linear, GGUFQuantEmbedding, GGUFQuantLinear,
                      GGUFQwen35MoeBlock, GGUFQwen35MoeExperts, MLXMoeExperts, MLXQ4Embedding, MLXQ4Linear,
                      tied_output_head)
from .ops import dequant, gguf_moe_routed, mlx_moe_routed, moe_workspace_bytes, qmm, qmm_glu, router_topk

__all__ = [
    "LIB_PATH", "LibraryMissing", "lib", "formats", "gguf", "mlx", "synth",
    "GGUFQuantLinear", "GGUFQ8_0Linear", "GGUFQ5_0Linear", "GGUFQ4_KLinear", "GGUFQ6_KLinear",
    "MLXQ4Linear", "MLXMoeExperts", "GGUFQwen35MoeExperts", "GGUFQwen35MoeBlock",
    "GGUFQuantEmbedding", "GGUFQ8_0Embedding", "GGUFQ5_0Embedding", "GGUFQ4_KEmbedding", "GGUFQ6_KEmbedding",
    "MLXQ4Embedding", "tied_output_head",
    "qmm", "qmm_glu", "dequant", "router_topk", "mlx_moe_routed", "gguf_moe_routed", "moe_workspace_bytes",
]
