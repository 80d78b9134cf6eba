"""GPU parity of the MLX-4 routed-expert MoE (router, sort, grouped GEMVs, combine)
against the oracle composition, through the C ABI."""

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


def run_case(dev, T, E, k, H, I, gs, seed, tokens=None):
    rng = np.random.default_rng(seed)
    gu, dn = make_experts(E, H, I, gs, rng)
    x = synth.numpy_x(T, H, rng)
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
    ref = np.zeros((len(sel), H))
    for ti, t in enumerate(sel):
        xt = x[t].astype(np.float64)
        for s in range(k):
            e = int(idx[ti, s])
            a = gu_e(e).astype(np.float64) @ xt
            h = om.silu(a[:I]) * a[I:]
            ref[ti] += w[ti, s] * (dn_e(e).astype(np.float64) @ h)
    err = y[sel] - ref
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    assert rel <= 1e-3, f"MoE T={T}: rel_fro={rel:.3e}"
    return y


@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_small(dev, T):
    run_case(dev, T, E=8, k=2, H=256, I=128, gs=64, seed=T)


@pytest.mark.parametrize("gs", [32, 64, 128, 256])
def test_moe_group_sizes(dev, gs):
    # K of gate/up 512 and of down 256: the x-stationary expert kernels with 2 and 1
    # waves; 21 tokens x top-2 over 8 experts gives full and partial column tiles
    run_case(dev, 21, E=8, k=2, H=512, I=256, gs=gs, seed=gs)


@pytest.mark.parametrize("T", [1, 16, 256])
def test_moe_config5(dev, T):
    # 128 experts, top-8, H=2048, I=768, gs=64; check up to 12 tokens against the oracle
    tokens = None if T <= 16 else list(range(0, T, 23))
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
