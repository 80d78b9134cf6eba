"""GPU parity of the routed-expert MoE (router, sort, grouped GEMVs, combine) over
MLX-4 and GGUF (Q4_K gate/up, Q6_K down) experts against the oracle composition,
through the C ABI."""

import numpy as np
import pytest
import torch

import alloy_amd
from alloy_amd import synth
from oracle import moe as om
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def make_experts(E, H, I, gs, rng):
    gu = synth.numpy_mlx(E * 2 * I, H, gs, rng)
    dn = synth.numpy_mlx(E * H, I, gs, rng)
    return gu, dn


def to_dev(arrs, shape_q, shape_s, dev):
    q, s, b = arrs
    return (torch.from_numpy(q).reshape(shape_q).to(dev), torch.from_numpy(s).reshape(shape_s).to(dev),
            torch.from_numpy(b).reshape(shape_s).to(dev))


def run_case(dev, T, E, k, H, I, gs, seed, tokens=None, x_scale=1.0):
    rng = np.random.default_rng(seed)
    gu, dn = make_experts(E, H, I, gs, rng)
    x = (synth.numpy_x(T, H, rng).astype(np.float32) * x_scale).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    guq, gus, gub = to_dev(gu, (E, 2 * I, H // 2), (E, 2 * I, H // gs), dev)
    dnq, dns, dnb = to_dev(dn, (E, H, I // 2), (E, H, I // gs), dev)
    y = torch.ops.alloy.mlx_moe_routed(torch.from_numpy(x).to(dev), torch.from_numpy(logits).to(dev),
                                       guq, gus, gub, dnq, dns, dnb, E, k, I).cpu().numpy()
    sel = np.arange(T) if tokens is None else np.asarray(tokens)
    cache = {}

    def gu_e(e):
        if ("g", e) not in cache:
            r = slice(e * 2 * I, (e + 1) * 2 * I)
            cache[("g", e)] = oq.dequant_mlx_q4(gu[0][r], gu[1][r], gu[2][r], gs)
        return cache[("g", e)]

    def dn_e(e):
        if ("d", e) not in cache:
            r = slice(e * H, (e + 1) * H)
            cache[("d", e)] = oq.dequant_mlx_q4(dn[0][r], dn[1][r], dn[2][r], gs)
        return cache[("d", e)]

    idx, w = om.router_topk(logits[sel], k)
    ref, bound = om.routed_reference(x[sel], idx, w, gu_e, dn_e, I)
    check_routed(y[sel], ref, bound, f"MoE T={T}")
    return y


def check_routed(y, ref, bound, what):
    """Both north-star bars on routed outputs: relative Frobenius error <= 1e-3 and,
    per element, |err| <= 2e-3 * sum_s w_s * ||h_s|| * max|D_e row| (the dense bound
    on each slot's down product, weighted like the output)."""
    err = np.asarray(y, np.float64) - ref
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    worst = float(np.max(np.abs(err) / bound))
    assert rel <= 1e-3 and worst <= 1.0, f"{what}: rel_fro={rel:.3e} max err/bound={worst:.3f}"


@pytest.mark.parametrize("T", [1, 2, 4, 5, 40])
def test_moe_small(dev, T):
    run_case(dev, T, E=8, k=2, H=256, I=128, gs=64, seed=T)


@pytest.mark.parametrize("E,k,T,x_scale", [(8, 4, 3, 1.0), (200, 4, 3, 1.0), (300, 6, 5, 1.0), (16, 2, 9, 40.0),
                                             (16, 2, 7, 1e-3)])
def test_moe_routed_small_t(dev, E, k, T, x_scale):
    # few tokens with I a multiple of 256: per-route GEMVs, the router fused into gate/up
    # (E <= 256) or a launch of its own (E = 300); experts shared by several tokens;
    # large and tiny activations exercise the per-route power-of-two scaling of
    # silu(g)*u before its fp16 rounding
    run_case(dev, T, E=E, k=k, H=512, I=256, gs=64, seed=E + T, x_scale=x_scale)


@pytest.mark.parametrize("E,k,T,x_scale", [(4, 2, 16, 1.0), (8, 2, 12, 1.0), (16, 4, 8, 1.0), (16, 2, 12, 1e-3),
                                             (128, 8, 16, 30.0)])
def test_moe_many_routes_per_expert(dev, E, k, T, x_scale):
    # 8 <= T <= 16 on the per-route path: four experts at top-2 over 16 tokens put
    # about 8 routes on each expert (one expert read by many workgroups at once);
    # tiny and large activations exercise the per-route scaling of silu(g)*u
    run_case(dev, T, E=E, k=k, H=512, I=256, gs=64, seed=3 * E + T, x_scale=x_scale)


@pytest.mark.parametrize("T", [8, 12])
def test_moe_config5_mid_t(dev, T):
    run_case(dev, T, E=128, k=8, H=2048, I=768, gs=64, seed=300 + T)


@pytest.mark.parametrize("gs", [32, 64, 128, 256])
def test_moe_group_sizes(dev, gs):
    # K of gate/up 512 and of down 256: the x-stationary expert kernels with 2 and 1
    # waves; 21 tokens x top-2 over 8 experts gives full and partial column tiles
    run_case(dev, 21, E=8, k=2, H=512, I=256, gs=gs, seed=gs)


@pytest.mark.parametrize("T", [1, 16, 256])
def test_moe_config5(dev, T):
    # 128 experts, top-8, H=2048, I=768, gs=64; at T = 256 every 4th token (64 tokens)
    # against the oracle
    tokens = None if T <= 16 else list(range(0, T, 4))
    run_case(dev, T, E=128, k=8, H=2048, I=768, gs=64, seed=100 + T, tokens=tokens)


def test_router_topk(dev):
    rng = np.random.default_rng(5)
    T, E, k = 300, 128, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, [5, 9, 100]] = 7.5          # tie at the top
    logits[1, :] = 0.0                     # all tied
    idx, w = alloy_amd.router_topk(torch.from_numpy(logits).to(dev), k)
    ridx, rw = om.router_topk(logits, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.allclose(w.cpu().numpy(), rw, atol=1e-6, rtol=1e-5)


def test_moe_deterministic(dev):
    rng = np.random.default_rng(1)
    E, H, I, gs, k, T = 16, 512, 256, 64, 4, 64
    gu, dn = make_experts(E, H, I, gs, rng)
    guq, gus, gub = to_dev(gu, (E, 2 * I, H // 2), (E, 2 * I, H // gs), dev)
    dnq, dns, dnb = to_dev(dn, (E, H, I // 2), (E, H, I // gs), dev)
    x = torch.from_numpy(synth.numpy_x(T, H, rng)).to(dev)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    a = torch.ops.alloy.mlx_moe_routed(x, lg, guq, gus, gub, dnq, dns, dnb, E, k, I)
    b = torch.ops.alloy.mlx_moe_routed(x, lg, guq, gus, gub, dnq, dns, dnb, E, k, I)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ GGUF experts
def run_gguf_case(dev, T, E, k, H, I, seed, tokens=None, logits_dtype=torch.float32):
    """gguf_moe_routed (Q4_K fused gate/up, Q6_K down) against the oracle composition
    (reference role: tests/kernels/test_moe.py:123-145 with the oracle decoders)."""
    rng = np.random.default_rng(seed)
    gu = synth.numpy_blocks("q4_k", E * 2 * I, H, rng)
    dn = synth.numpy_blocks("q6_k", E * H, I, rng)
    x = synth.numpy_x(T, H, rng)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    lg = torch.from_numpy(logits).to(dev).to(logits_dtype)
    if logits_dtype != torch.float32:
        logits = lg.float().cpu().numpy()
    y = torch.ops.alloy.gguf_moe_routed(torch.from_numpy(x).to(dev), lg,
                                        torch.from_numpy(gu).reshape(E, 2 * I, -1).to(dev),
                                        torch.from_numpy(dn).reshape(E, H, -1).to(dev), E, k, I).cpu().numpy()
    sel = np.arange(T) if tokens is None else np.asarray(tokens)
    idx, w = om.router_topk(logits[sel], k)
    cache = {}

    def deq(kind, e):
        if (kind, e) not in cache:
            if kind == "g":
                cache[(kind, e)] = oq.dequant_q4_k(gu[e * 2 * I:(e + 1) * 2 * I], H)
            else:
                cache[(kind, e)] = oq.dequant_q6_k(dn[e * H:(e + 1) * H], I)
        return cache[(kind, e)]

    ref, bound = om.routed_reference(x[sel], idx, w, lambda e: deq("g", e), lambda e: deq("d", e), I)
    check_routed(y[sel], ref, bound, f"GGUF MoE T={T}")
    return y


@pytest.mark.parametrize("T", [1, 2, 4, 5, 21])
def test_gguf_moe_small(dev, T):
    # gate/up K = 512 (2 waves), down K = 256 (1 wave); full and partial tiles
    run_gguf_case(dev, T, E=8, k=2, H=512, I=256, seed=50 + T)


@pytest.mark.parametrize("E,k,T", [(4, 2, 16), (16, 4, 8), (8, 2, 11)])
def test_gguf_moe_many_routes_per_expert(dev, E, k, T):
    # per-route few-token path (Q4_K gate/up, Q6_K down) with many routes per expert
    run_gguf_case(dev, T, E=E, k=k, H=512, I=256, seed=70 + E + T)


@pytest.mark.parametrize("T", [1, 8, 16, 256])
def test_gguf_moe_qwen3_shape(dev, T):
    # Qwen3-MoE-like: 128 experts, top-8, H = 2048, I = 768; at T = 256 every 4th token
    # (64 tokens) checked
    tokens = None if T <= 16 else list(range(0, T, 4))
    run_gguf_case(dev, T, E=128, k=8, H=2048, I=768, seed=200 + T, tokens=tokens)


def test_gguf_moe_fp16_logits_and_deterministic(dev):
    y1 = run_gguf_case(dev, 4, E=16, k=4, H=1024, I=512, seed=9, logits_dtype=torch.float16)
    y2 = run_gguf_case(dev, 4, E=16, k=4, H=1024, I=512, seed=9, logits_dtype=torch.float16)
    assert np.array_equal(y1, y2)


def test_gguf_moe_block_module(dev):
    # the block adds sigmoid(Wg x) * shared(x) to the routed output (qwen3_5.py:304-343)
    E, k, H, I, T = 8, 2, 512, 256, 3
    rng = np.random.default_rng(3)
    gu = torch.from_numpy(synth.numpy_blocks("q4_k", E * 2 * I, H, rng)).reshape(E, 2 * I, -1).to(dev)
    dn = torch.from_numpy(synth.numpy_blocks("q6_k", E * H, I, rng)).reshape(E, H, -1).to(dev)
    experts = alloy_amd.GGUFQwen35MoeExperts(gate_up_blocks=gu, down_qweight=dn, num_experts=E, hidden_size=H,
                                             moe_intermediate_size=I)

    class Orig(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate = torch.nn.Linear(H, E, bias=False, dtype=torch.float16, device=dev)
            self.experts = experts
            self.shared_expert = torch.nn.Linear(H, H, bias=False, dtype=torch.float16, device=dev)
            self.shared_expert_gate = torch.nn.Linear(H, 1, bias=False, dtype=torch.float16, device=dev)

    orig = Orig()
    blk = alloy_amd.GGUFQwen35MoeBlock(orig, num_experts=E, top_k=k, moe_intermediate=I)
    x = torch.from_numpy(synth.numpy_x(T, H, rng)).to(dev)
    out = blk(x)
    logits = torch.nn.functional.linear(x, orig.gate.weight)
    routed = torch.ops.alloy.gguf_moe_routed(x, logits, gu, dn, E, k, I)
    shared = torch.sigmoid(orig.shared_expert_gate(x)) * orig.shared_expert(x)
    assert out.shape == (T, H)
    assert torch.equal(out, routed + shared)
