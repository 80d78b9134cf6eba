"""The reference's quantized-linear operator surface, backed by the HIP library.

Registers the ``alloy::*`` ops with the reference's schemas
(``packages/alloy-torch/src/alloy_torch/custom_ops.py:47-106``) for the CUDA
dispatch key (HIP on PyTorch-ROCm) and the Meta key (shapes only).  There is no
CPU kernel: a call on CPU tensors raises, and a call without the built library
raises ``LibraryMissing`` — nothing falls back to another implementation.

Semantics follow the reference handlers (``ops/linalg.py:346-739``): activations
are ``(M, K)`` with K taken from ``activations.shape[1]``; the output is
``(M, N)`` in ``activations.dtype`` (float16 or float32).  The MoE op returns
float32 ``(T, H)`` like ``gguf_moe_routed`` (``custom_ops.py:729-742``).

Besides the ops, plain functions ``qmm`` (any format / path) and ``dequant``
(the bit-exactness probe) expose the whole C ABI to Python.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .formats import BLOCK, mlx_group_size

_vp = ctypes.c_void_p


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return _vp(0 if t is None else t.data_ptr())


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return _vp(torch.cuda.current_stream(dev).cuda_stream)


def _dt(dtype: torch.dtype, what: str) -> int:
    if dtype == torch.float16:
        return _lib.DT_F16
    if dtype == torch.float32:
        return _lib.DT_F32
    raise TypeError(f"{what} must be float16 or float32, got {dtype}")


def _check_act(a: torch.Tensor) -> tuple[int, int]:
    if a.ndim != 2:
        raise ValueError(f"activations must be rank-2 (M, K), got {tuple(a.shape)}")
    _dt(a.dtype, "activations")
    return a.shape[0], a.shape[1]


def _need(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{name} requires {dtype}, got {t.dtype}")
    if t.ndim != 2:
        raise ValueError(f"{name} must be rank-2, got {tuple(t.shape)}")


def _same_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    if dev.type != "cuda":
        raise RuntimeError(f"alloy_amd ops run on the GPU only (got a {dev.type} tensor)")
    return dev


# ------------------------------------------------------------------ shape checks (shared by Meta + HIP)

def shape_gguf_blocks(fmt: str, activations: torch.Tensor, blocks: torch.Tensor) -> tuple[int, int, int]:
    M, K = _check_act(activations)
    qk, bb = BLOCK[fmt]
    _need(blocks, torch.uint8, f"{fmt} blocks")
    if K % qk:
        raise ValueError(f"{fmt}: K={K} not divisible by {qk}")
    if blocks.shape[1] != (K // qk) * bb:
        raise ValueError(f"{fmt}: blocks row bytes {blocks.shape[1]} != {(K // qk) * bb} for K={K}")
    return M, blocks.shape[0], K


def shape_q8_0(activations, qweight, scales) -> tuple[int, int, int]:
    M, K = _check_act(activations)
    _need(qweight, torch.int8, "q8_0 qweight")
    _need(scales, torch.float16, "q8_0 scales")
    N = qweight.shape[0]
    if K % 32 or tuple(qweight.shape) != (N, K) or tuple(scales.shape) != (N, K // 32):
        raise ValueError(f"q8_0 buffers {tuple(qweight.shape)}, {tuple(scales.shape)} inconsistent with K={K}")
    return M, N, K


def shape_q5_0(activations, qweight, qhigh, scales) -> tuple[int, int, int]:
    M, K = _check_act(activations)
    _need(qweight, torch.uint8, "q5_0 qweight")
    _need(qhigh, torch.uint8, "q5_0 qhigh")
    _need(scales, torch.float16, "q5_0 scales")
    N = scales.shape[0]
    if K % 32 or tuple(qweight.shape) != (N, K // 2) or tuple(qhigh.shape) != (N, K // 2) \
            or tuple(scales.shape) != (N, K // 32):
        raise ValueError(f"q5_0 buffers inconsistent with K={K}")
    return M, N, K


def shape_mlx(activations, qweight, scales, biases) -> tuple[int, int, int, int]:
    M, K = _check_act(activations)
    _need(qweight, torch.uint8, "mlx qweight")
    _need(scales, torch.float16, "mlx scales")
    _need(biases, torch.float16, "mlx biases")
    N = qweight.shape[0]
    if qweight.shape[1] * 2 != K or scales.shape != biases.shape or scales.shape[0] != N or scales.shape[1] == 0:
        raise ValueError(f"mlx buffers {tuple(qweight.shape)}, {tuple(scales.shape)} inconsistent with K={K}")
    gs = mlx_group_size(qweight, scales)
    if gs * scales.shape[1] != K:
        raise ValueError(f"mlx group size does not divide K={K}")
    return M, N, K, gs


# ------------------------------------------------------------------ general entry points

def qmm(fmt: str, x: torch.Tensor, w: torch.Tensor, *, scales=None, biases=None, aux=None,
        group_size: int = 0, N: int | None = None, out_dtype: torch.dtype | None = None,
        path: str = "auto", opts: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """y[M,N] = x[M,K] @ dequant(w)^T through ``alloy_qmm`` (any format, any path)."""
    M, K = _check_act(x)
    if N is None:
        N = w.shape[0]
    dev = _same_device(x, w)
    out_dtype = out_dtype or x.dtype
    x = x.contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=dev)
    with torch.cuda.device(dev):
        ws = gemm_workspace(fmt, M, N, K, dev, opts) if path in ("auto", "gemm", "gemv_mfma") else None
        _lib.call("alloy_qmm_ws", _lib.FMT[fmt], _p(w), _p(aux), _p(scales), _p(biases), group_size,
                  _p(x), _dt(x.dtype, "activations"), _p(out), _dt(out.dtype, "output"), M, N, K,
                  _lib.PATH[path], opts, _p(ws), 0 if ws is None else ws.numel(), _stream(dev))
    return out


def gemm_workspace(fmt: str, M: int, N: int, K: int, dev, opts: int = 0) -> torch.Tensor | None:
    """The split-K workspace the plan wants for this shape (None: no split): the prefill
    GEMM's (M > 16) or the M <= 16 kernels'; with a split count forced in ``opts`` (bits
    40-43; for the GEMM with a forced tile, bits 36-39), that split's."""
    need = int(_lib.lib().alloy_gemm_workspace_bytes(_lib.FMT[fmt], M, N, K)) if M > 1 else 0
    forced = (opts >> 40) & 0xF
    if forced > 1 and (M <= 16 or (opts >> 36) & 0xF >= 4):
        need = max(need, forced * M * N * 4)
    return torch.empty(need, dtype=torch.uint8, device=dev) if need > 0 else None


def dequant(fmt: str, w: torch.Tensor, K: int, *, scales=None, biases=None, aux=None, group_size: int = 0,
            rows: tuple[int, int] | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decode weight rows [r0, r1) to (r1-r0, K) fp32 (exact) or fp16 (RN of exact)."""
    N = w.shape[0] if fmt != "q5_0_split" else w.shape[0]
    r0, r1 = rows if rows is not None else (0, N)
    dev = _same_device(w)
    out = torch.empty((r1 - r0, K), dtype=out_dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("alloy_dequant", _lib.FMT[fmt], _p(w), _p(aux), _p(scales), _p(biases), group_size,
                  _p(out), _dt(out_dtype, "output"), r0, r1 - r0, N, K, _stream(dev))
    return out


def router_topk(logits: torch.Tensor, top_k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(T,E) f32 logits -> (idx i32 (T,k), weights f32 (T,k))."""
    if logits.dtype != torch.float32 or logits.ndim != 2:
        raise TypeError("router logits must be float32 (T, E)")
    T, E = logits.shape
    dev = _same_device(logits)
    logits = logits.contiguous()
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("alloy_moe_router_topk", _p(logits), _p(idx), _p(w), T, E, top_k, _stream(dev))
    return idx, w


def moe_workspace_bytes(T: int, E: int, top_k: int, H: int, I: int) -> int:
    return int(_lib.lib().alloy_moe_workspace_bytes(T, E, top_k, H, I))


def mlx_moe_routed(hidden, router_logits, gate_up_qweight, gate_up_scales, gate_up_biases, down_qweight,
                   down_scales, down_biases, num_experts: int, top_k: int, moe_intermediate: int,
                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    T, H, I, E, gs = shape_moe(hidden, router_logits, gate_up_qweight, gate_up_scales, gate_up_biases,
                               down_qweight, down_scales, down_biases, num_experts, top_k, moe_intermediate)
    dev = _same_device(hidden, router_logits, gate_up_qweight, down_qweight)
    hidden = hidden.contiguous()
    router_logits = router_logits.contiguous()
    need = moe_workspace_bytes(T, E, top_k, H, I)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("alloy_mlx_moe_routed", _p(hidden), _p(router_logits), _p(gate_up_qweight),
                  _p(gate_up_scales), _p(gate_up_biases), _p(down_qweight), _p(down_scales), _p(down_biases),
                  gs, E, top_k, T, H, I, _p(workspace), workspace.numel(), _p(y), _stream(dev))
    return y


def _glu_workspace(fmt: str, x: torch.Tensor, M: int, N: int, K: int, gs: int, dev) -> tuple:
    need = int(_lib.lib().alloy_glu_workspace_bytes(_lib.FMT[fmt], M, N, K, gs, _dt(x.dtype, "activations")))
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    return ws, need


def qmm_glu(fmt: str, act: str, x: torch.Tensor, gate: dict, up: dict, *, group_size: int = 0,
            N: int | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y = act(x @ dequant(gate)^T) * (x @ dequant(up)^T) through ``alloy_qmm_glu``;
    ``gate`` / ``up``: dicts with ``w`` and optional ``aux``, ``scales``, ``biases``."""
    M, K = _check_act(x)
    N = gate["w"].shape[0] if N is None else N
    dev = _same_device(x, gate["w"], up["w"])
    x = x.contiguous()
    y = torch.empty((M, N), dtype=out_dtype or x.dtype, device=dev)
    ws, need = _glu_workspace(fmt, x, M, N, K, group_size, dev)
    g = [_p(gate.get(k)) for k in ("w", "aux", "scales", "biases")]
    u = [_p(up.get(k)) for k in ("w", "aux", "scales", "biases")]
    with torch.cuda.device(dev):
        _lib.call("alloy_qmm_glu", _lib.FMT[fmt], _lib.ACT[act], *g, *u, group_size, _p(x), _dt(x.dtype, "activations"),
                  _p(y), _dt(y.dtype, "output"), M, N, K, _p(ws), need, _stream(dev))
    return y


def _same_shape(a: torch.Tensor, b: torch.Tensor, what: str) -> None:
    if tuple(a.shape) != tuple(b.shape) or a.dtype != b.dtype:
        raise ValueError(f"{what}: gate and up buffers differ ({tuple(a.shape)} vs {tuple(b.shape)})")


def _run_glu(name: str, fmt: str, activations, gate_bufs, up_bufs, M, N, K, gs=0, gs_arg=False):
    dev = _same_device(activations, *gate_bufs, *up_bufs)
    x = activations.contiguous()
    y = _empty_out(x, N)
    if M and N:
        ws, need = _glu_workspace(fmt, x, M, N, K, gs, dev)
        extra = (gs,) if gs_arg else ()
        with torch.cuda.device(dev):
            _lib.call(name, _p(x), _dt(x.dtype, "activations"), *[_p(b.contiguous()) for b in gate_bufs],
                      *[_p(b.contiguous()) for b in up_bufs], *extra, _p(y), _dt(y.dtype, "output"), M, N, K,
                      _p(ws), need, _stream(dev))
    return y


def shape_glu_q4_k(activations, gate_blocks, up_blocks):
    _same_shape(gate_blocks, up_blocks, "gguf_q4_k glu")
    return shape_gguf_blocks("q4_k", activations, gate_blocks)


def shape_glu_mlx(activations, gq, gsc, gb, uq, usc, ub):
    for a, b in ((gq, uq), (gsc, usc), (gb, ub)):
        _same_shape(a, b, "mlx_q4_silu")
    return shape_mlx(activations, gq, gsc, gb)


def shape_glu_q8_0(activations, gq, gsc, uq, usc):
    for a, b in ((gq, uq), (gsc, usc)):
        _same_shape(a, b, "gguf_q8_0_silu")
    return shape_q8_0(activations, gq, gsc)


def _q4_k_silu(activations, gate_blocks, up_blocks):
    M, N, K = shape_glu_q4_k(activations, gate_blocks, up_blocks)
    return _run_glu("alloy_gguf_q4_k_silu", "q4_k", activations, [gate_blocks], [up_blocks], M, N, K)


def _q4_k_gelu(activations, gate_blocks, up_blocks):
    M, N, K = shape_glu_q4_k(activations, gate_blocks, up_blocks)
    return _run_glu("alloy_gguf_q4_k_gelu", "q4_k", activations, [gate_blocks], [up_blocks], M, N, K)


def _mlx_silu(activations, gq, gsc, gb, uq, usc, ub):
    M, N, K, gs = shape_glu_mlx(activations, gq, gsc, gb, uq, usc, ub)
    return _run_glu("alloy_mlx_q4_silu", "mlx_q4", activations, [gq, gsc, gb], [uq, usc, ub], M, N, K, gs, True)


def _q8_0_silu(activations, gq, gsc, uq, usc):
    M, N, K = shape_glu_q8_0(activations, gq, gsc, uq, usc)
    return _run_glu("alloy_gguf_q8_0_silu", "q8_0_split", activations, [gq, gsc], [uq, usc], M, N, K)


def _embedding(fmt: str, input_ids: torch.Tensor, bufs: dict, N: int, K: int, gs: int = 0) -> torch.Tensor:
    if input_ids.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"input_ids must be int32 or int64, got {input_ids.dtype}")
    dev = _same_device(input_ids, *[b for b in bufs.values() if b is not None])
    ids = input_ids.contiguous()
    out = torch.empty(tuple(ids.shape) + (K,), dtype=torch.float32, device=dev)
    if ids.numel():
        with torch.cuda.device(dev):
            _lib.call("alloy_embedding", _lib.FMT[fmt], _p(bufs.get("w")), _p(bufs.get("aux")),
                      _p(bufs.get("scales")), _p(bufs.get("biases")), gs, _p(ids),
                      int(ids.dtype == torch.int64), ids.numel(), N, K, _p(out), _stream(dev))
    return out


def _emb_rows(t: torch.Tensor, what: str) -> int:
    if t.ndim != 2:
        raise ValueError(f"{what} must be 2-D, got shape {tuple(t.shape)}")
    return t.shape[0]


def _q4_k_embedding(input_ids, blocks):
    if blocks.dtype != torch.uint8 or blocks.ndim != 2 or blocks.shape[1] % 144:
        raise ValueError(f"gguf_q4_k_embedding: blocks must be uint8 (N, k*144), got {tuple(blocks.shape)}")
    return _embedding("q4_k", input_ids, dict(w=blocks.contiguous()), blocks.shape[0], blocks.shape[1] // 144 * 256)


def _q6_k_embedding(input_ids, packed_weights):
    if packed_weights.dtype != torch.uint8 or packed_weights.ndim != 2 or packed_weights.shape[1] % 210:
        raise ValueError(f"gguf_q6_k_embedding: packed_weights must be uint8 (N, k*210), got {tuple(packed_weights.shape)}")
    return _embedding("q6_k", input_ids, dict(w=packed_weights.contiguous()), packed_weights.shape[0],
                      packed_weights.shape[1] // 210 * 256)


def _q8_0_embedding(input_ids, qweight, scales):
    N, K = _emb_rows(qweight, "qweight"), qweight.shape[1]
    if qweight.dtype != torch.int8 or scales.dtype != torch.float16 or tuple(scales.shape) != (N, K // 32) or K % 32:
        raise ValueError("gguf_q8_0_embedding: qweight int8 (N, K) and scales float16 (N, K/32) expected")
    return _embedding("q8_0_split", input_ids, dict(w=qweight.contiguous(), scales=scales.contiguous()), N, K)


def _q5_0_embedding(input_ids, qweight, qhigh, scales):
    N, K = _emb_rows(qweight, "qweight"), qweight.shape[1] * 2
    if (qweight.dtype != torch.uint8 or qhigh.dtype != torch.uint8 or tuple(qhigh.shape) != tuple(qweight.shape)
            or scales.dtype != torch.float16 or tuple(scales.shape) != (N, K // 32) or K % 32):
        raise ValueError("gguf_q5_0_embedding: qweight/qhigh uint8 (N, K/2) and scales float16 (N, K/32) expected")
    return _embedding("q5_0_split", input_ids,
                      dict(w=qweight.contiguous(), aux=qhigh.contiguous(), scales=scales.contiguous()), N, K)


def _mlx_embedding(input_ids, qweight, scales, biases):
    N = _emb_rows(qweight, "qweight")
    K = qweight.shape[1] * 2
    if scales.ndim != 2 or scales.shape[0] != N or tuple(biases.shape) != tuple(scales.shape):
        raise ValueError("mlx_q4_embedding: scales/biases must be (N, K/group)")
    gs = K // scales.shape[1] if scales.shape[1] else 0
    if gs <= 0 or gs * scales.shape[1] != K:
        raise ValueError(f"mlx_q4_embedding: group size does not divide K={K}")
    return _embedding("mlx_q4", input_ids, dict(w=qweight.contiguous(), scales=scales.contiguous(),
                                                  biases=biases.contiguous()), N, K, gs)


def gguf_moe_routed(hidden, router_logits, gate_up_blocks, down_qweight, num_experts: int, top_k: int,
                    moe_intermediate: int, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Routed GGUF experts (Q4_K fused gate/up, Q6_K down) -> float32 (T, H), like the
    reference's ``gguf_moe_routed`` (``custom_ops.py:59-66``, ``ops/moe.py:110-249``)."""
    T, H, I, E = shape_gguf_moe(hidden, router_logits, gate_up_blocks, down_qweight, num_experts, top_k,
                                moe_intermediate)
    dev = _same_device(hidden, router_logits, gate_up_blocks, down_qweight)
    hidden = hidden.contiguous()
    logits = router_logits.to(torch.float32).contiguous()
    need = moe_workspace_bytes(T, E, top_k, H, I)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    y = torch.empty((T, H), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("alloy_gguf_moe_routed", _p(hidden), _p(logits), _p(gate_up_blocks.contiguous()),
                  _p(down_qweight.contiguous()), E, top_k, T, H, I, _p(workspace), workspace.numel(), _p(y),
                  _stream(dev))
    return y


def shape_gguf_moe(hidden, router_logits, gate_up_blocks, down_qweight, num_experts, top_k, moe_intermediate):
    if hidden.ndim != 2 or hidden.dtype != torch.float16:
        raise TypeError("hidden must be float16 (T, H)")
    T, H = hidden.shape
    E, I = int(num_experts), int(moe_intermediate)
    if H % 256 or I % 256:
        raise ValueError(f"expert dims must be divisible by 256: hidden={H} moe_intermediate={I}")
    if not router_logits.dtype.is_floating_point or tuple(router_logits.shape) != (T, E):
        raise ValueError(f"router_logits must be floating point {(T, E)}")
    expected = {"gate_up_blocks": (E, 2 * I, H // 256 * 144), "down_qweight": (E, H, I // 256 * 210)}
    actual = {"gate_up_blocks": tuple(gate_up_blocks.shape), "down_qweight": tuple(down_qweight.shape)}
    if actual != expected:
        raise ValueError(f"expert weight shapes do not match: got {actual} expected {expected}")
    if gate_up_blocks.dtype != torch.uint8 or down_qweight.dtype != torch.uint8:
        raise TypeError("expert weights must be uint8 packed blocks")
    if not (0 < top_k <= E):
        raise ValueError(f"top_k={top_k} invalid for {E} experts")
    return T, H, I, E


def shape_moe(hidden, router_logits, gu_q, gu_s, gu_b, dn_q, dn_s, dn_b, num_experts, top_k, moe_intermediate):
    if hidden.ndim != 2 or hidden.dtype != torch.float16:
        raise TypeError("hidden must be float16 (T, H)")
    T, H = hidden.shape
    E, I = int(num_experts), int(moe_intermediate)
    if router_logits.dtype != torch.float32 or tuple(router_logits.shape) != (T, E):
        raise ValueError(f"router_logits must be float32 {(T, E)}")
    if gu_q.dtype != torch.uint8 or tuple(gu_q.shape) != (E, 2 * I, H // 2):
        raise ValueError(f"gate_up qweight must be uint8 {(E, 2 * I, H // 2)}, got {tuple(gu_q.shape)}")
    if dn_q.dtype != torch.uint8 or tuple(dn_q.shape) != (E, H, I // 2):
        raise ValueError(f"down qweight must be uint8 {(E, H, I // 2)}, got {tuple(dn_q.shape)}")
    for t, nm in ((gu_s, "gate_up scales"), (gu_b, "gate_up biases"), (dn_s, "down scales"), (dn_b, "down biases")):
        if t.dtype != torch.float16:
            raise TypeError(f"{nm} must be float16")
    if gu_s.shape != gu_b.shape or dn_s.shape != dn_b.shape or gu_s.ndim != 3 or dn_s.ndim != 3:
        raise ValueError("scales/biases shapes inconsistent")
    gs = H // gu_s.shape[2]
    if gu_s.shape[:2] != (E, 2 * I) or gs * gu_s.shape[2] != H or tuple(dn_s.shape) != (E, H, I // gs):
        raise ValueError("scales/biases shapes inconsistent with one group size")
    if not (0 < top_k <= E):
        raise ValueError(f"top_k={top_k} invalid for {E} experts")
    return T, H, I, E, gs


# ------------------------------------------------------------------ torch.library ops

_LIB = torch.library.Library("alloy", "DEF")
_LIB.define("gguf_q4_k_mm(Tensor activations, Tensor blocks) -> Tensor")
_LIB.define("gguf_q6_k_mm(Tensor activations, Tensor packed_weights) -> Tensor")
_LIB.define("gguf_q8_0_mm(Tensor activations, Tensor qweight, Tensor scales) -> Tensor")
_LIB.define("gguf_q5_0_mm(Tensor activations, Tensor qweight, Tensor qhigh, Tensor scales) -> Tensor")
_LIB.define("mlx_q4_mm(Tensor activations, Tensor qweight, Tensor scales, Tensor biases) -> Tensor")
_LIB.define("batched_gguf_q4_k_mm(Tensor activations, Tensor[] blocks) -> Tensor[]")
_LIB.define("batched_gguf_q6_k_mm(Tensor activations, Tensor[] packed_weights) -> Tensor[]")
_LIB.define("batched_gguf_q8_0_mm(Tensor activations, Tensor[] qweights, Tensor[] scales) -> Tensor[]")
_LIB.define("batched_gguf_q5_0_mm(Tensor activations, Tensor[] qweights, Tensor[] qhighs, Tensor[] scales) -> Tensor[]")
_LIB.define("batched_mlx_q4_mm(Tensor activations, Tensor[] qweights, Tensor[] scales, Tensor[] biases) -> Tensor[]")
# wire-block Q8_0 / Q5_0 (the raw GGUF blob; the reference only has the split ops)
_LIB.define("gguf_q8_0_blocks_mm(Tensor activations, Tensor blocks) -> Tensor")
_LIB.define("gguf_q5_0_blocks_mm(Tensor activations, Tensor blocks) -> Tensor")
# quantized embeddings (reference custom_ops.py:67-69, 83-85, 89-91, 97-99, 103)
_LIB.define("gguf_q4_k_embedding(Tensor input_ids, Tensor blocks) -> Tensor")
_LIB.define("gguf_q6_k_embedding(Tensor input_ids, Tensor packed_weights) -> Tensor")
_LIB.define("gguf_q8_0_embedding(Tensor input_ids, Tensor qweight, Tensor scales) -> Tensor")
_LIB.define("gguf_q5_0_embedding(Tensor input_ids, Tensor qweight, Tensor qhigh, Tensor scales) -> Tensor")
_LIB.define("mlx_q4_embedding(Tensor input_ids, Tensor qweight, Tensor scales, Tensor biases) -> Tensor")
# fused gated pairs (reference custom_ops.py:53-58, 79-82, 108-111)
_LIB.define("gguf_q4_k_silu(Tensor activations, Tensor gate_blocks, Tensor up_blocks) -> Tensor")
_LIB.define("gguf_q4_k_gelu(Tensor activations, Tensor gate_blocks, Tensor up_blocks) -> Tensor")
_LIB.define(
    "mlx_q4_silu(Tensor activations, Tensor gate_qweight, Tensor gate_scales, "
    "Tensor gate_biases, Tensor up_qweight, Tensor up_scales, Tensor up_biases) -> Tensor"
)
_LIB.define(
    "gguf_q8_0_silu(Tensor activations, Tensor gate_qweight, Tensor gate_scales, "
    "Tensor up_qweight, Tensor up_scales) -> Tensor"
)
# GGUF routed experts (reference custom_ops.py:59-66)
_LIB.define(
    "gguf_moe_routed(Tensor hidden, Tensor router_logits, Tensor gate_up_blocks, "
    "Tensor down_qweight, int num_experts, int top_k, int moe_intermediate) -> Tensor"
)
# MLX-4 routed experts (the MLX counterpart of the reference's gguf_moe_routed)
_LIB.define(
    "mlx_moe_routed(Tensor hidden, Tensor router_logits, Tensor gate_up_qweight, Tensor gate_up_scales, "
    "Tensor gate_up_biases, Tensor down_qweight, Tensor down_scales, Tensor down_biases, "
    "int num_experts, int top_k, int moe_intermediate) -> Tensor"
)


def _empty_out(activations, N):
    return torch.empty((activations.shape[0], N), dtype=activations.dtype, device=activations.device)


def _run_named(name: str, activations: torch.Tensor, bufs: list[torch.Tensor], M: int, N: int, K: int,
               extra_after_bufs: tuple = ()) -> torch.Tensor:
    dev = _same_device(activations, *bufs)
    x = activations.contiguous()
    bufs = [b.contiguous() for b in bufs]
    y = _empty_out(x, N)
    if M and N:
        with torch.cuda.device(dev):
            _lib.call(name, _p(x), _dt(x.dtype, "activations"), *[_p(b) for b in bufs], *extra_after_bufs,
                      _p(y), _dt(y.dtype, "output"), M, N, K, _stream(dev))
    return y


def _q4_k(activations, blocks):
    M, N, K = shape_gguf_blocks("q4_k", activations, blocks)
    if M > 16:            # prefill: the GEMM may split K into a workspace
        _same_device(activations, blocks)
        return qmm("q4_k", activations, blocks.contiguous(), N=N)
    return _run_named("alloy_gguf_q4_k_mm", activations, [blocks], M, N, K)


def _q6_k(activations, packed_weights):
    M, N, K = shape_gguf_blocks("q6_k", activations, packed_weights)
    return _run_named("alloy_gguf_q6_k_mm", activations, [packed_weights], M, N, K)


def _q8_0(activations, qweight, scales):
    M, N, K = shape_q8_0(activations, qweight, scales)
    return _run_named("alloy_gguf_q8_0_mm", activations, [qweight, scales], M, N, K)


def _q5_0(activations, qweight, qhigh, scales):
    M, N, K = shape_q5_0(activations, qweight, qhigh, scales)
    return _run_named("alloy_gguf_q5_0_mm", activations, [qweight, qhigh, scales], M, N, K)


def _mlx(activations, qweight, scales, biases):
    M, N, K, gs = shape_mlx(activations, qweight, scales, biases)
    return _run_named("alloy_mlx_q4_mm", activations, [qweight, scales, biases], M, N, K, (gs,))


def _q8_0_blocks(activations, blocks):
    M, N, K = shape_gguf_blocks("q8_0", activations, blocks)
    return _run_named("alloy_gguf_q8_0_blocks_mm", activations, [blocks], M, N, K)


def _q5_0_blocks(activations, blocks):
    M, N, K = shape_gguf_blocks("q5_0", activations, blocks)
    return _run_named("alloy_gguf_q5_0_blocks_mm", activations, [blocks], M, N, K)


_SINGLE = {
    "gguf_q4_k_mm": _q4_k,
    "gguf_q6_k_mm": _q6_k,
    "gguf_q8_0_mm": _q8_0,
    "gguf_q5_0_mm": _q5_0,
    "mlx_q4_mm": _mlx,
    "gguf_q8_0_blocks_mm": _q8_0_blocks,
    "gguf_q5_0_blocks_mm": _q5_0_blocks,
}

_SHAPE = {
    "gguf_q4_k_mm": lambda a, b: shape_gguf_blocks("q4_k", a, b)[1],
    "gguf_q6_k_mm": lambda a, b: shape_gguf_blocks("q6_k", a, b)[1],
    "gguf_q8_0_mm": lambda a, q, s: shape_q8_0(a, q, s)[1],
    "gguf_q5_0_mm": lambda a, q, h, s: shape_q5_0(a, q, h, s)[1],
    "mlx_q4_mm": lambda a, q, s, b: shape_mlx(a, q, s, b)[1],
    "gguf_q8_0_blocks_mm": lambda a, b: shape_gguf_blocks("q8_0", a, b)[1],
    "gguf_q5_0_blocks_mm": lambda a, b: shape_gguf_blocks("q5_0", a, b)[1],
}

for _name, _fn in _SINGLE.items():
    torch.library.impl(_LIB, _name, "CUDA")(_fn)

    def _meta(*args, _n=_name):
        return _empty_out(args[0], _SHAPE[_n](*args))

    torch.library.impl(_LIB, _name, "Meta")(_meta)


def _ptr_array(tensors):
    arr = (ctypes.c_void_p * len(tensors))(*[t.data_ptr() if t is not None else None for t in tensors])
    return arr, ctypes.cast(arr, ctypes.c_void_p)


def _batched(name: str, single: str, fmt: str, slots: tuple):
    """Native batched op: every matrix against the same activations in as few launches
    as the library can (one per 8 matrices at M = 1), outputs separate (M, N_i)."""
    def run(activations, *lists):
        mats = list(zip(*lists))
        if not mats:
            return []
        M, K = _check_act(activations)
        Ns = [_SHAPE[single](activations, *bufs) for bufs in mats]
        gs = shape_mlx(activations, *mats[0])[3] if fmt == "mlx_q4" else 0
        if fmt == "mlx_q4" and any(shape_mlx(activations, *b)[3] != gs for b in mats):
            raise ValueError(f"{name}: all matrices must share one group size")
        dev = _same_device(activations, *[b for bufs in mats for b in bufs])
        x = activations.contiguous()
        outs = [torch.empty((M, N), dtype=x.dtype, device=dev) for N in Ns]
        if M == 0:
            return outs
        cols = {k: [None] * len(mats) for k in ("w", "aux", "scales", "biases")}
        for i, bufs in enumerate(mats):
            for slot, b in zip(slots, bufs):
                cols[slot][i] = b.contiguous()
        keep = [_ptr_array(cols[k]) if any(t is not None for t in cols[k]) else (None, None)
                for k in ("w", "aux", "scales", "biases")]
        y_arr = _ptr_array(outs)
        n_arr = (ctypes.c_int64 * len(Ns))(*Ns)
        with torch.cuda.device(dev):
            _lib.call("alloy_qmm_batched", _lib.FMT[fmt], len(mats), *[p for _, p in keep],
                      ctypes.cast(n_arr, ctypes.c_void_p), gs, _p(x), _dt(x.dtype, "activations"), y_arr[1],
                      _dt(x.dtype, "output"), M, K, _stream(dev))
        del cols, keep, y_arr, n_arr
        return outs
    return run


_BATCHED = {
    "batched_gguf_q4_k_mm": ("gguf_q4_k_mm", "q4_k", ("w",)),
    "batched_gguf_q6_k_mm": ("gguf_q6_k_mm", "q6_k", ("w",)),
    "batched_gguf_q8_0_mm": ("gguf_q8_0_mm", "q8_0_split", ("w", "scales")),
    "batched_gguf_q5_0_mm": ("gguf_q5_0_mm", "q5_0_split", ("w", "aux", "scales")),
    "batched_mlx_q4_mm": ("mlx_q4_mm", "mlx_q4", ("w", "scales", "biases")),
}

for _name, (_single, _fmt, _slots) in _BATCHED.items():
    torch.library.impl(_LIB, _name, "CUDA")(_batched(_name, _single, _fmt, _slots))

    def _bmeta(activations, *lists, _s=_single):
        return [_empty_out(activations, _SHAPE[_s](activations, *bufs)) for bufs in zip(*lists)]

    torch.library.impl(_LIB, _name, "Meta")(_bmeta)


torch.library.impl(_LIB, "mlx_moe_routed", "CUDA")(mlx_moe_routed)
torch.library.impl(_LIB, "gguf_moe_routed", "CUDA")(gguf_moe_routed)

_EMB = {
    "gguf_q4_k_embedding": (_q4_k_embedding, lambda ids, b: b.shape[1] // 144 * 256),
    "gguf_q6_k_embedding": (_q6_k_embedding, lambda ids, b: b.shape[1] // 210 * 256),
    "gguf_q8_0_embedding": (_q8_0_embedding, lambda ids, q, s: q.shape[1]),
    "gguf_q5_0_embedding": (_q5_0_embedding, lambda ids, q, h, s: q.shape[1] * 2),
    "mlx_q4_embedding": (_mlx_embedding, lambda ids, q, s, b: q.shape[1] * 2),
}
for _name, (_fn, _width) in _EMB.items():
    torch.library.impl(_LIB, _name, "CUDA")(_fn)

    def _emb_meta(input_ids, *bufs, _w=_width):
        return torch.empty(tuple(input_ids.shape) + (_w(input_ids, *bufs),), dtype=torch.float32,
                           device=input_ids.device)

    torch.library.impl(_LIB, _name, "Meta")(_emb_meta)

_GLU = {
    "gguf_q4_k_silu": (_q4_k_silu, shape_glu_q4_k),
    "gguf_q4_k_gelu": (_q4_k_gelu, shape_glu_q4_k),
    "mlx_q4_silu": (_mlx_silu, shape_glu_mlx),
    "gguf_q8_0_silu": (_q8_0_silu, shape_glu_q8_0),
}
for _name, (_fn, _shape) in _GLU.items():
    torch.library.impl(_LIB, _name, "CUDA")(_fn)

    def _glu_meta(*args, _s=_shape):
        return _empty_out(args[0], _s(*args)[1])

    torch.library.impl(_LIB, _name, "Meta")(_glu_meta)


@torch.library.impl(_LIB, "gguf_moe_routed", "Meta")
def _gguf_moe_meta(hidden, router_logits, gate_up_blocks, down_qweight, num_experts, top_k, moe_intermediate):
    shape_gguf_moe(hidden, router_logits, gate_up_blocks, down_qweight, num_experts, top_k, moe_intermediate)
    return torch.empty((hidden.shape[0], hidden.shape[1]), dtype=torch.float32, device=hidden.device)


@torch.library.impl(_LIB, "mlx_moe_routed", "Meta")
def _moe_meta(hidden, router_logits, gu_q, gu_s, gu_b, dn_q, dn_s, dn_b, num_experts, top_k, moe_intermediate):
    shape_moe(hidden, router_logits, gu_q, gu_s, gu_b, dn_q, dn_s, dn_b, num_experts, top_k, moe_intermediate)
    return torch.empty((hidden.shape[0], hidden.shape[1]), dtype=torch.float32, device=hidden.device)
