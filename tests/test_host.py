"""CPU tests of the host side: the C-ABI library loads and exports every declared
symbol, its argument validation maps to the reference's exception types without
touching a GPU, and the torch ops' Meta kernels / drop-in modules validate like
the reference."""

import ctypes
import pathlib
import re

import pytest
import torch

import alloy_amd
from alloy_amd import _lib, formats
from alloy_amd.modules import GGUFQ4_KLinear, GGUFQ8_0Linear, GGUFQwen35MoeExperts, MLXQ4Linear

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "alloy_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(alloy_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = alloy_amd.lib()
    names = declared_functions()
    assert "alloy_qmm" in names and len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"
    assert lib.alloy_version().startswith(b"alloy_amd")


def _qmm_status(fmt, K, M=1, N=4, w=16, x=16, y=16, gs=0, path=0, opts=0, xdt=1, scales=16, biases=16, aux=16):
    lib = alloy_amd.lib()
    vp = ctypes.c_void_p
    return lib.alloy_qmm(_lib.FMT[fmt], vp(w), vp(aux), vp(scales), vp(biases), gs, vp(x), xdt, vp(y), 0,
                         M, N, K, path, opts, None)


def test_capi_validation_without_gpu():
    # every case fails validation before any HIP call (fake, aligned pointers)
    assert _qmm_status("q4_k", K=300) == _lib.E_SHAPE
    assert _qmm_status("q4_k", K=256, w=8) == _lib.E_ALIGN
    assert _qmm_status("q4_k", K=256, xdt=7) == _lib.E_DTYPE
    assert _qmm_status("mlx_q4", K=256, gs=48) == _lib.E_SHAPE
    assert _qmm_status("mlx_q4", K=256, gs=16) == _lib.E_UNSUPPORTED
    assert _qmm_status("q4_k", K=256, path=9) == _lib.E_ARG
    assert _qmm_status("q4_k", K=256, opts=3) == _lib.E_ARG
    assert _qmm_status("q4_k", K=256, w=0) == _lib.E_ARG
    assert _qmm_status("q4_k", K=256, M=0) == _lib.OK           # empty: nothing launched
    with pytest.raises(ValueError, match="not divisible"):
        _lib.check(_qmm_status("q6_k", K=100))
    with pytest.raises(NotImplementedError):
        _lib.check(_qmm_status("mlx_q4", K=256, gs=16))


def test_moe_workspace_layout():
    lib = alloy_amd.lib()
    small = lib.alloy_moe_workspace_bytes(1, 128, 8, 2048, 768)
    big = lib.alloy_moe_workspace_bytes(256, 128, 8, 2048, 768)
    R = 256 * 8
    assert big >= R * (2048 * 4 + 768 * 2) and big > small > 0
    assert lib.alloy_moe_workspace_bytes(0, 0, 8, 2048, 768) == 0


def test_split_workspace_plan():
    """The K-split workspace the M <= 16 plan asks for: four fp32 partial slices with
    <= 64 row tiles, two with <= 128, none beyond, for M < 8, K < 4096 or Q4_K past
    K = 8192; M = 1 never splits."""
    lib = alloy_amd.lib()
    F = _lib.FMT
    assert lib.alloy_gemm_workspace_bytes(F["q6_k"], 8, 1024, 4096) == 4 * 8 * 1024 * 4
    assert lib.alloy_gemm_workspace_bytes(F["q5_0"], 16, 2048, 14336) == 2 * 16 * 2048 * 4
    assert lib.alloy_gemm_workspace_bytes(F["mlx_q4"], 8, 1000, 4096) == 4 * 8 * 1000 * 4
    assert lib.alloy_gemm_workspace_bytes(F["q8_0"], 8, 4096, 4096) == 0
    assert lib.alloy_gemm_workspace_bytes(F["q6_k"], 4, 1024, 4096) == 0
    assert lib.alloy_gemm_workspace_bytes(F["q6_k"], 8, 1024, 3072) == 0
    assert lib.alloy_gemm_workspace_bytes(F["q4_k"], 16, 1024, 11008) == 0
    assert lib.alloy_gemm_workspace_bytes(F["q4_k"], 1, 1024, 4096) == 0
    # few rows and tokens: the v_dot2 wave-row kernel, no split
    assert lib.alloy_gemm_workspace_bytes(F["q4_k"], 8, 512, 4096) == 0
    assert lib.alloy_gemm_workspace_bytes(F["q6_k"], 8, 512, 4096) == 4 * 8 * 512 * 4


def test_glu_workspace_plan():
    """The gated pair runs as one fused launch (no workspace) at N <= 8192 and M <= 16
    for Q4_K at M >= 4 or M >= 2 with M * N > 6144 and for MLX at any such M; every
    other case takes two fp32 product buffers."""
    lib = alloy_amd.lib()
    F = _lib.FMT
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 4, 1024, 4096, 0, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["mlx_q4"], 16, 4096, 2048, 64, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 1, 1024, 4096, 0, _lib.DT_F16) == 2 * 1024 * 4
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 2, 4096, 4096, 0, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 2, 768, 2048, 0, _lib.DT_F16) == 2 * 2 * 768 * 4
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 4, 8192, 3072, 0, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 4, 14336, 4096, 0, _lib.DT_F16) == 2 * 4 * 14336 * 4
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 1, 8192, 3072, 0, _lib.DT_F16) == 2 * 8192 * 4
    assert lib.alloy_glu_workspace_bytes(F["q4_k"], 17, 1024, 4096, 0, _lib.DT_F16) == 2 * 17 * 1024 * 4
    assert lib.alloy_glu_workspace_bytes(F["q6_k"], 8, 1024, 4096, 0, _lib.DT_F16) == 2 * 8 * 1024 * 4
    assert lib.alloy_glu_workspace_bytes(F["mlx_q4"], 1, 8192, 3072, 64, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["mlx_q4"], 4, 8192, 3072, 64, _lib.DT_F16) == 0
    assert lib.alloy_glu_workspace_bytes(F["mlx_q4"], 1, 14336, 4096, 64, _lib.DT_F16) == 2 * 14336 * 4


def meta(shape, dtype):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_meta_shapes():
    a = meta((5, 512), torch.float16)
    assert torch.ops.alloy.gguf_q4_k_mm(a, meta((300, 288), torch.uint8)).shape == (5, 300)
    assert torch.ops.alloy.gguf_q6_k_mm(a, meta((7, 420), torch.uint8)).shape == (5, 7)
    assert torch.ops.alloy.gguf_q8_0_mm(a, meta((9, 512), torch.int8), meta((9, 16), torch.float16)).shape == (5, 9)
    assert torch.ops.alloy.gguf_q5_0_mm(a, meta((9, 256), torch.uint8), meta((9, 256), torch.uint8),
                                        meta((9, 16), torch.float16)).shape == (5, 9)
    out = torch.ops.alloy.mlx_q4_mm(a, meta((11, 256), torch.uint8), meta((11, 8), torch.float16),
                                    meta((11, 8), torch.float16))
    assert out.shape == (5, 11) and out.dtype == torch.float16
    assert torch.ops.alloy.gguf_q8_0_blocks_mm(a, meta((3, 16 * 34), torch.uint8)).shape == (5, 3)
    outs = torch.ops.alloy.batched_gguf_q4_k_mm(a, [meta((4, 288), torch.uint8), meta((6, 288), torch.uint8)])
    assert [o.shape for o in outs] == [(5, 4), (5, 6)]
    E, H, I = 4, 256, 64
    y = torch.ops.alloy.mlx_moe_routed(meta((3, H), torch.float16), meta((3, E), torch.float32),
                                       meta((E, 2 * I, H // 2), torch.uint8), meta((E, 2 * I, H // 64), torch.float16),
                                       meta((E, 2 * I, H // 64), torch.float16), meta((E, H, I // 2), torch.uint8),
                                       meta((E, H, I // 64), torch.float16), meta((E, H, I // 64), torch.float16),
                                       E, 2, I)
    assert y.shape == (3, H) and y.dtype == torch.float32


def test_meta_validation_errors():
    a = meta((5, 512), torch.float16)
    with pytest.raises(ValueError):
        torch.ops.alloy.gguf_q4_k_mm(a, meta((3, 144), torch.uint8))         # wrong row bytes
    with pytest.raises(TypeError):
        torch.ops.alloy.gguf_q4_k_mm(a, meta((3, 288), torch.int8))          # wrong dtype
    with pytest.raises(TypeError):
        torch.ops.alloy.gguf_q4_k_mm(meta((5, 512), torch.bfloat16), meta((3, 288), torch.uint8))


def test_ops_refuse_cpu_tensors():
    a = torch.zeros((1, 256), dtype=torch.float16)
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.alloy.gguf_q4_k_mm(a, torch.zeros((2, 144), dtype=torch.uint8))


def test_module_validation_matches_reference():
    with pytest.raises(ValueError, match="not divisible into blocks"):
        GGUFQ4_KLinear(in_features=100, out_features=2, blocks=torch.zeros((2, 144), dtype=torch.uint8))
    with pytest.raises(TypeError):
        GGUFQ8_0Linear(in_features=64, out_features=2, qweight=torch.zeros((2, 64), dtype=torch.uint8),
                       scales=torch.zeros((2, 2), dtype=torch.float16))
    with pytest.raises(ValueError, match="is held in buffers"):
        GGUFQ8_0Linear(in_features=64, out_features=2, qweight=torch.zeros((2, 64), dtype=torch.int8))
    with pytest.raises(ValueError, match="not a whole group size"):
        MLXQ4Linear(in_features=64, out_features=2, qweight=torch.zeros((2, 32), dtype=torch.uint8),
                    scales=torch.zeros((2, 3), dtype=torch.float16), biases=torch.zeros((2, 3), dtype=torch.float16))
    m = GGUFQ4_KLinear(in_features=512, out_features=3, blocks=torch.zeros((3, 288), dtype=torch.uint8))
    assert m.blocks.shape == (3, 288)
    assert formats.row_bytes("q6_k", 4096) == 3360


def test_gguf_moe_meta_and_validation():
    E, H, I, T = 4, 512, 256, 3
    gu, dn = meta((E, 2 * I, H // 256 * 144), torch.uint8), meta((E, H, I // 256 * 210), torch.uint8)
    y = torch.ops.alloy.gguf_moe_routed(meta((T, H), torch.float16), meta((T, E), torch.float16), gu, dn, E, 2, I)
    assert y.shape == (T, H) and y.dtype == torch.float32
    with pytest.raises(ValueError, match="divisible by 256"):
        torch.ops.alloy.gguf_moe_routed(meta((T, 320), torch.float16), meta((T, E), torch.float32),
                                        meta((E, 2 * I, 180), torch.uint8), dn, E, 2, I)
    with pytest.raises(ValueError, match="do not match"):
        torch.ops.alloy.gguf_moe_routed(meta((T, H), torch.float16), meta((T, E), torch.float32),
                                        meta((E, I, H // 256 * 144), torch.uint8), dn, E, 2, I)
    with pytest.raises(TypeError):
        torch.ops.alloy.gguf_moe_routed(meta((T, H), torch.float16), meta((T, E), torch.float32),
                                        meta((E, 2 * I, H // 256 * 144), torch.int8), dn, E, 2, I)
    # the C ABI: shape and size checks fail before any HIP call
    lib = alloy_amd.lib()
    st = lib.alloy_gguf_moe_routed(16, 16, 256, 256, E, 2, T, 320, I, 256, 1 << 20, 16, None)
    assert st == _lib.E_SHAPE
    st = lib.alloy_gguf_moe_routed(16, 16, 256, 256, E, 2, T, 8192, I, 256, 1 << 30, 16, None)
    assert st == _lib.E_UNSUPPORTED


def test_gguf_moe_modules_validate_like_reference():
    E, H, I = 2, 512, 256
    ok = GGUFQwen35MoeExperts(gate_up_blocks=torch.zeros((E, 2 * I, 288), dtype=torch.uint8),
                              down_qweight=torch.zeros((E, H, 210), dtype=torch.uint8), num_experts=E,
                              hidden_size=H, moe_intermediate_size=I)
    assert ok.gate_up_blocks.shape == (E, 2 * I, 288)
    with pytest.raises(RuntimeError, match="only holds the expert weights"):
        ok()
    with pytest.raises(ValueError, match="multiples of 256"):
        GGUFQwen35MoeExperts(gate_up_blocks=torch.zeros((E, 2 * 100, 288), dtype=torch.uint8),
                             down_qweight=torch.zeros((E, H, 210), dtype=torch.uint8), num_experts=E,
                             hidden_size=H, moe_intermediate_size=100)
    with pytest.raises(ValueError, match="gate_up_blocks for E=2"):
        GGUFQwen35MoeExperts(gate_up_blocks=torch.zeros((E, I, 288), dtype=torch.uint8),
                             down_qweight=torch.zeros((E, H, 210), dtype=torch.uint8), num_experts=E,
                             hidden_size=H, moe_intermediate_size=I)
    with pytest.raises(TypeError):
        GGUFQwen35MoeExperts(gate_up_blocks=torch.zeros((E, 2 * I, 288), dtype=torch.int8),
                             down_qweight=torch.zeros((E, H, 210), dtype=torch.uint8), num_experts=E,
                             hidden_size=H, moe_intermediate_size=I)


def test_embedding_meta_and_modules():
    ids = meta((2, 3), torch.int64)
    assert torch.ops.alloy.gguf_q6_k_embedding(ids, meta((10, 420), torch.uint8)).shape == (2, 3, 512)
    assert torch.ops.alloy.gguf_q8_0_embedding(ids, meta((10, 64), torch.int8), meta((10, 2), torch.float16)).shape == (2, 3, 64)
    assert torch.ops.alloy.gguf_q5_0_embedding(ids, meta((10, 32), torch.uint8), meta((10, 32), torch.uint8),
                                               meta((10, 2), torch.float16)).shape == (2, 3, 64)
    from alloy_amd.modules import GGUFQ6_KEmbedding, tied_output_head
    e = GGUFQ6_KEmbedding(num_embeddings=4, embedding_dim=256, qweight=torch.zeros((4, 210), dtype=torch.uint8))
    head = tied_output_head(e)
    assert head.out_features == 4 and head.in_features == 256 and head.qweight.data_ptr() == e.qweight.data_ptr()
    with pytest.raises(TypeError):
        tied_output_head(e, torch.nn.Embedding(4, 256))
    with pytest.raises(ValueError):
        GGUFQ6_KEmbedding(num_embeddings=4, embedding_dim=100, qweight=torch.zeros((4, 210), dtype=torch.uint8))
