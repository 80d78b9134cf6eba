"""CPU tests pinning the NumPy oracle (no GPU needed).

* golden fixtures from an independent encoder (tests/golden/make_golden.py)
* hand-computed known-answer blocks (values written out below)
* split-layout decode == wire decode (two restatements of Q8_0 / Q5_0)
* fp64 matmul vs brute-force loops, router vs HF formula and tie rule,
  MoE composition vs a brute-force loop.
"""

import pathlib

import numpy as np
import pytest

from oracle import glu as og
from oracle import moe as om
from oracle import quant as oq

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("fmt", ["q8_0", "q5_0", "q4_k", "q6_k"])
def test_golden_fixture(fmt):
    z = np.load(GOLD / f"decode_{fmt}.npz")
    w = oq.dequant(fmt, z["blob"], int(z["K"]))
    assert np.array_equal(bits(w), bits(z["w"]))


def test_golden_fixture_mlx():
    z = np.load(GOLD / "decode_mlx_q4.npz")
    w = oq.dequant_mlx_q4(z["qweight"], z["scales"], z["biases"], int(z["group_size"]))
    assert np.array_equal(bits(w), bits(z["w"]))


def _f16(v):
    return list(np.array([v], np.float16).view(np.uint8))


def test_kat_q8_0():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = _f16(0.5)
    q = np.zeros(32, np.int8)
    q[:5] = [-128, -1, 0, 1, 127]
    blk[2:] = q.view(np.uint8)
    w = oq.dequant_q8_0(blk[None], 32)[0]
    assert list(w[:5]) == [-64.0, -0.5, 0.0, 0.5, 63.5] and not w[5:].any()


def test_kat_q5_0():
    blk = np.zeros(22, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[2:6] = [0x01, 0, 0, 0]        # only element 0 has its 5th bit set
    blk[6] = 0xF1                      # element 0 nibble 1, element 16 nibble 15
    w = oq.dequant_q5_0(blk[None], 32)[0]
    assert w[0] == 1.0 and w[16] == -1.0
    assert all(w[i] == -16.0 for i in range(32) if i not in (0, 16))


def test_kat_q4_k():
    blk = np.zeros(144, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[2:4] = _f16(0.5)
    s = blk[4:16]
    s[0] = 2          # sc0 = 2
    s[4] = 3          # m0 = 3
    s[1] = 0xC0       # sc1 = 0, top bits of sc5 = 3
    s[5] = 0x40       # m1 = 0, top bits of m5 = 1
    s[9] = 0x21       # sc5 low = 1, m5 low = 2   -> sc5 = 49, m5 = 18
    qs = blk[16:]
    qs[0] = 0x7A      # sub-block 0 el 0 = 10, sub-block 1 el 0 = 7
    qs[67] = 0x5C     # sub-block 4 el 3 = 12, sub-block 5 el 3 = 5
    w = oq.dequant_q4_k(blk[None], 256)[0]
    assert w[0] == 1.0 * 2 * 10 - 0.5 * 3            # 18.5
    assert all(w[1:32] == -1.5)                        # q = 0 in sub-block 0
    assert w[32] == 0.0                                # sc1 = m1 = 0
    assert w[128 + 3] == 0.0                           # sub-block 4: sc = m = 0
    assert w[160 + 3] == 1.0 * 49 * 5 - 0.5 * 18      # 236.0
    assert w[160] == -9.0                              # q = 0 in sub-block 5


def test_kat_q6_k():
    blk = np.zeros(210, np.uint8)
    sc = np.zeros(16, np.int8)
    sc[0], sc[13] = -3, 64
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = _f16(0.25)
    blk[84] = 0x90    # ql byte 64+20: high nibble 9  (h=1, s=2, l=20)
    blk[128 + 52] = 0x20   # qh byte 32+20: bits 4-5 = 2
    w = oq.dequant_q6_k(blk[None], 256)[0]
    assert w[128 + 64 + 20] == 0.25 * 64 * 9           # 144.0
    assert all(w[0:16] == 0.25 * -3 * -32)             # 24.0
    assert all(w[16:32] == 0.0)                        # scale index 1 is 0


def test_kat_mlx():
    qweight = np.zeros((1, 32), np.uint8)
    qweight[0, 0] = 0x3C
    w = oq.dequant_mlx_q4(qweight, np.array([[0.5]], np.float16), np.array([[-1.0]], np.float16), 64)[0]
    assert w[0] == 5.0 and w[1] == 0.5 and all(w[2:] == -1.0)


@pytest.mark.parametrize("fmt", ["q8_0", "q5_0"])
def test_split_layout_matches_wire(fmt):
    from alloy_amd import synth
    rng = np.random.default_rng(3)
    N, K = 7, 256
    blob = synth.numpy_blocks(fmt, N, K, rng)
    w = oq.dequant(fmt, blob, K)
    if fmt == "q8_0":
        qw, sc = oq.split_q8_0(blob, K)
        assert np.array_equal(bits(oq.dequant_q8_0_split(qw, sc)), bits(w))
        assert np.array_equal(oq.join_q8_0(qw, sc), blob)
    else:
        qw, qh, sc = oq.split_q5_0(blob, K)
        assert np.array_equal(bits(oq.dequant_q5_0_split(qw, qh, sc)), bits(w))
        assert np.array_equal(oq.join_q5_0(qw, qh, sc), blob)


def test_exactness_lemma_q4_k():
    """Q4_K values are RN32 of the exact rational: recompute in float64 and round once."""
    from alloy_amd import synth
    rng = np.random.default_rng(5)
    blob = synth.numpy_blocks("q4_k", 5, 512, rng)
    w = oq.dequant_q4_k(blob, 512)
    b = blob.reshape(5, 2, 144)
    d = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = b[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    sc, m = oq.q4_k_scale_min(b[..., 4:16])
    qs = b[..., 16:].reshape(5, 2, 4, 32)
    q = np.stack([qs & 15, qs >> 4], 3).reshape(5, 2, 8, 32).astype(np.float64)
    exact = d[..., None, None] * sc[..., None] * q - dmin[..., None, None] * m[..., None]
    assert np.array_equal(bits(exact.astype(np.float32).reshape(5, 512)), bits(w))


def test_ref_matmul_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 5)).astype(np.float16)
    w = rng.standard_normal((4, 5)).astype(np.float32)
    y = oq.ref_matmul(x, w)
    for m in range(3):
        for n in range(4):
            s = 0.0
            for k in range(5):
                s += float(x[m, k]) * float(w[n, k])
            assert abs(y[m, n] - s) < 1e-12


def test_parity_metric_detects_errors():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 64)).astype(np.float16)
    w = rng.standard_normal((8, 64)).astype(np.float32)
    ref = oq.ref_matmul(x, w)
    assert oq.parity_errors(ref, ref, x, w) == (0.0, 0.0)
    bad = ref.copy()
    bad[0, 3] += 1.0
    rel, ratio = oq.parity_errors(bad, ref, x, w)
    assert rel > 1e-3 and ratio > 2e-3


def test_router_matches_hf_and_ties():
    rng = np.random.default_rng(2)
    T, E, k = 6, 128, 8
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, 10] = logits[0, 3] = logits[0, 77] = 9.0     # a three-way tie at the top
    idx, w = om.router_topk(logits, k)
    assert list(idx[0, :3]) == [3, 10, 77]                  # ties -> lowest index first
    # HF: softmax over all, top-k, renormalise
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-logits[t, e], e))[:k]
        assert list(idx[t]) == order
        ref = p[t, order] / p[t, order].sum()
        assert np.allclose(w[t], ref, rtol=1e-12, atol=1e-15)


def test_moe_composition_brute_force():
    rng = np.random.default_rng(4)
    T, E, H, I, k = 3, 5, 16, 8, 2
    x = rng.standard_normal((T, H)).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32)
    dn = rng.standard_normal((E, H, I)).astype(np.float32)
    y = om.moe_routed(x, logits, gu, dn, k)
    idx, w = om.router_topk(logits, k)
    for t in range(T):
        acc = np.zeros(H)
        for s in range(k):
            e = idx[t, s]
            g = [sum(float(gu[e, i, c]) * float(x[t, c]) for c in range(H)) for i in range(2 * I)]
            h = [g[i] / (1 + np.exp(-g[i])) * g[I + i] for i in range(I)]
            for j in range(H):
                acc[j] += w[t, s] * sum(float(dn[e, j, i]) * h[i] for i in range(I))
        assert np.allclose(y[t], acc, rtol=1e-10, atol=1e-10)


def test_glu_activations_pinned():
    import math
    from scipy.special import expit
    from oracle import glu as og
    v = np.linspace(-30.0, 30.0, 601)
    assert np.allclose(og.silu(v), v * expit(v), rtol=1e-12, atol=1e-300)
    # tanh-form GELU vs the exact erf GELU: the approximation is within 5e-4 absolute
    exact = np.array([0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) for t in v])
    assert np.max(np.abs(og.gelu_tanh(v) - exact)) < 5e-4
    assert og.gelu_tanh(np.array([0.0]))[0] == 0.0
    assert abs(og.gelu_tanh(np.array([12.0]))[0] - 12.0) < 1e-6     # the clamp: tanh(10) = 1 - 4e-9
    assert abs(og.gelu_tanh(np.array([-12.0]))[0]) < 1e-7        # 0.5 v (1 - tanh(10))


def test_glu_pair_brute_force():
    from oracle import glu as og
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 6)).astype(np.float16)
    g = rng.standard_normal((3, 6)).astype(np.float32)
    u = rng.standard_normal((3, 6)).astype(np.float32)
    for act in ("silu", "gelu"):
        y = og.glu(x, g, u, act)
        for m in range(2):
            for n in range(3):
                a = sum(float(x[m, k]) * float(g[n, k]) for k in range(6))
                b = sum(float(x[m, k]) * float(u[n, k]) for k in range(6))
                fa = a / (1.0 + np.exp(-a)) if act == "silu" else \
                    0.5 * a * (1.0 + np.tanh(np.clip(0.7978845608028654 * (a + 0.044715 * a ** 3), -10, 10)))
                assert abs(y[m, n] - fa * b) < 1e-12 * max(1.0, abs(fa * b))


def test_glu_error_bound_pinned():
    """glu_error_bound: products perturbed anywhere inside their per-element bounds keep
    act(g)*u inside it (mean value theorem; random and corner perturbations), and a
    planted output error of twice the bound is caught."""
    rng = np.random.default_rng(3)
    M, N, K = 3, 40, 64
    x = rng.standard_normal((M, K))
    G, U = rng.standard_normal((N, K)) * 0.3, rng.standard_normal((N, K)) * 0.3
    for act in ("silu", "gelu"):
        f = og.ACTS[act]
        g, u = x @ G.T, x @ U.T
        xn = np.linalg.norm(x, axis=1)[:, None]
        bg = 2e-3 * xn * np.abs(G).max(axis=1)[None, :]
        bu = 2e-3 * xn * np.abs(U).max(axis=1)[None, :]
        bound = og.glu_error_bound(x, G, U, act)
        for sg, su in [(1, 1), (1, -1), (-1, 1), (-1, -1)]:
            err = f(g + sg * bg) * (u + su * bu) - f(g) * u
            assert np.all(np.abs(err) <= bound * (1 + 1e-12))
        for _ in range(20):
            err = f(g + rng.uniform(-1, 1, g.shape) * bg) * (u + rng.uniform(-1, 1, u.shape) * bu) - f(g) * u
            assert np.all(np.abs(err) <= bound * (1 + 1e-12))
        planted = f(g) * u + 2 * bound * np.sign(rng.standard_normal(g.shape))
        assert np.any(np.abs(planted - f(g) * u) > bound)
    # the activations' slopes stay under ACT_SLOPE on a dense grid
    v = np.linspace(-12, 12, 200001)
    for act in ("silu", "gelu"):
        slope = np.diff(og.ACTS[act](v)) / np.diff(v)
        assert np.abs(slope).max() <= og.ACT_SLOPE


def test_routed_reference_bound_pinned():
    """routed_reference: a hand-computed one-token, two-slot case; outputs recomputed
    with every gate, up and down product perturbed inside its dense bound stay inside
    the bound (to first order: the perturbations are small); a planted error of twice
    the bound is caught."""
    I, H = 2, 3
    Gs = {0: np.array([[1.0, 0, 0], [0, 1.0, 0], [1.0, 1.0, 0], [0, 0, 2.0]]),   # (2I, H): gate rows, up rows
          1: np.array([[0, 0, 1.0], [1.0, 0, 0], [0, 2.0, 0], [1.0, 0, 1.0]])}
    Ds = {0: np.array([[1.0, 2.0], [0, -3.0], [0.5, 0]]), 1: np.array([[-1.0, 0], [2.0, 2.0], [0, 4.0]])}
    x = np.array([[1.0, 2.0, 3.0]])
    idx = np.array([[1, 0]])
    w = np.array([[0.75, 0.25]])
    ref, bound = om.routed_reference(x, idx, w, lambda e: Gs[e], lambda e: Ds[e], I)
    want_ref = np.zeros(H)
    for s, e in enumerate((1, 0)):
        a = Gs[e] @ x[0]
        h = np.array([a[j] / (1 + np.exp(-a[j])) * a[I + j] for j in range(I)])
        want_ref += w[0, s] * (Ds[e] @ h)
    assert np.allclose(ref[0], want_ref, rtol=1e-14)
    # random perturbations of every product inside its bound
    rng = np.random.default_rng(8)
    xn = np.linalg.norm(x[0])
    for _ in range(200):
        y = np.zeros(H)
        for s, e in enumerate((1, 0)):
            a = Gs[e] @ x[0] + rng.uniform(-1, 1, 2 * I) * 2e-3 * xn * np.abs(Gs[e]).max(axis=1)
            h = om.silu(a[:I]) * a[I:]
            d = Ds[e] @ h + rng.uniform(-1, 1, H) * 2e-3 * np.linalg.norm(h) * np.abs(Ds[e]).max(axis=1)
            y += w[0, s] * d
        assert np.all(np.abs(y - ref[0]) <= bound[0] * (1 + 1e-9))
    planted = ref[0] + 2 * bound[0]
    assert np.all(np.abs(planted - ref[0]) > bound[0])
