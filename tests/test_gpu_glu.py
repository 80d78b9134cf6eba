"""GPU parity of the fused gated pair y = act(x G^T) * (x U^T) (the reference's
gguf_q4_k_silu / gguf_q4_k_gelu / mlx_q4_silu / gguf_q8_0_silu ops) against the
NumPy oracle, through the C ABI: the one-launch x-stationary path (Q4_K / MLX at
M <= 16 where it is the faster one) and the two-product + combine path (the rest)."""

import numpy as np
import pytest
import torch

import alloy_amd
from alloy_amd import synth
from oracle import glu as og
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def make(fmt, N, K, rng, dev, gs=64):
    """Device buffers (dict for qmm_glu) and the oracle's fp32 weights."""
    if fmt == "mlx_q4":
        qw, sc, bi = synth.numpy_mlx(N, K, gs, rng)
        bufs = dict(w=torch.from_numpy(qw).to(dev), scales=torch.from_numpy(sc).to(dev),
                    biases=torch.from_numpy(bi).to(dev))
        return bufs, oq.dequant_mlx_q4(qw, sc, bi, gs)
    base = fmt.replace("_split", "")
    blob = synth.numpy_blocks(base, N, K, rng)
    W = oq.dequant(base, blob, K)
    if fmt == "q8_0_split":
        qw, sc = oq.split_q8_0(blob, K)
        return dict(w=torch.from_numpy(qw).to(dev), scales=torch.from_numpy(sc).to(dev)), W
    return dict(w=torch.from_numpy(blob).to(dev)), W


def check_glu(y, x, G, U, act, what):
    """Relative Frobenius error <= 1e-3 and, per element, the north-star bound on each of
    the two products carried through act(g)*u (oracle.glu.glu_error_bound)."""
    ref = og.glu(x, G, U, act)
    err = np.asarray(y, np.float64) - ref
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    worst = float(np.max(np.abs(err) / og.glu_error_bound(x, G, U, act)))
    assert rel <= 1e-3 and worst <= 1.0, f"{what}: rel_fro={rel:.3e} max err/bound={worst:.3f}"


@pytest.mark.parametrize("fmt", ["q4_k", "mlx_q4", "q8_0_split", "q6_k"])
@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("M", [1, 3, 4, 16, 40])
def test_glu_matches_oracle(dev, fmt, act, M):
    rng = np.random.default_rng(M * 7 + len(fmt))
    N, K = 200, 2048
    gate, G = make(fmt, N, K, rng, dev)
    up, U = make(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    gs = 64 if fmt == "mlx_q4" else 0
    y32 = alloy_amd.qmm_glu(fmt, act, xt, gate, up, group_size=gs, out_dtype=torch.float32)
    check_glu(y32.cpu().numpy(), x, G, U, act, f"{fmt} {act} M={M}")
    # fp16 output: the same fp32 values, rounded once
    y16 = alloy_amd.qmm_glu(fmt, act, xt, gate, up, group_size=gs, out_dtype=torch.float16)
    assert torch.equal(y16, y32.half()), f"{fmt} {act} M={M}: fp16 output is not RN16 of the fp32 one"


@pytest.mark.parametrize("M", [1, 8, 33])
def test_named_glu_ops(dev, M):
    rng = np.random.default_rng(11 + M)
    N, K = 96, 1024
    x = torch.from_numpy(synth.numpy_x(M, K, rng)).to(dev)
    g, _ = make("q4_k", N, K, rng, dev)
    u, _ = make("q4_k", N, K, rng, dev)
    for name, act in (("gguf_q4_k_silu", "silu"), ("gguf_q4_k_gelu", "gelu")):
        y = getattr(torch.ops.alloy, name)(x, g["w"], u["w"])
        assert y.dtype == torch.float16 and y.shape == (M, N)
        assert torch.equal(y, alloy_amd.qmm_glu("q4_k", act, x, g, u))
    gm, _ = make("mlx_q4", N, K, rng, dev)
    um, _ = make("mlx_q4", N, K, rng, dev)
    y = torch.ops.alloy.mlx_q4_silu(x, gm["w"], gm["scales"], gm["biases"], um["w"], um["scales"], um["biases"])
    assert torch.equal(y, alloy_amd.qmm_glu("mlx_q4", "silu", x, gm, um, group_size=64))
    g8, _ = make("q8_0_split", N, K, rng, dev)
    u8, _ = make("q8_0_split", N, K, rng, dev)
    y = torch.ops.alloy.gguf_q8_0_silu(x, g8["w"], g8["scales"], u8["w"], u8["scales"])
    assert torch.equal(y, alloy_amd.qmm_glu("q8_0_split", "silu", x, g8, u8))


@pytest.mark.parametrize("fmt,N,K,Ms", [("q4_k", 8192, 3072, (1, 4)), ("q4_k", 4096, 4096, (2, 4, 9, 16)),
                                         ("mlx_q4", 8192, 3072, (1, 2, 16)), ("q4_k", 8320, 2048, (3, 16))])
def test_glu_decode_shapes(dev, fmt, N, K, Ms):
    # Llama-3.2-3B gate/up at decode (K = 3072, N = 8192: two products + combine for
    # Q4_K at M = 1, one fused launch otherwise), a 4096 x 4096 pair at M = 2..16
    # (fused) and N = 8320 (past the fused limit: two products + combine)
    rng = np.random.default_rng(5)
    gs = 64 if fmt == "mlx_q4" else 0
    gate, G = make(fmt, N, K, rng, dev)
    up, U = make(fmt, N, K, rng, dev)
    for M in Ms:
        x = synth.numpy_x(M, K, rng)
        y = alloy_amd.qmm_glu(fmt, "silu", torch.from_numpy(x).to(dev), gate, up, group_size=gs,
                              out_dtype=torch.float32)
        rows = rng.choice(N, 64, replace=False)
        check_glu(y.cpu().numpy()[:, rows], x, G[rows], U[rows], "silu", f"{fmt} gate/up {N}x{K} M={M}")
