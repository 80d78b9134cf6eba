"""NumPy restatement of the reference's MoE router and routed-expert composition.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* Router — ``packages/alloy-metal/src/alloy/std/moe.py:31-79`` (moe_router_topk):
  per token, the TOP_K largest logits in descending order, ties to the lowest
  expert index, then a softmax over the K selected logits (equal to HF's
  softmax -> top-k -> renormalise, ``tests/kernels/test_moe.py:166-175``).
* Routed block — ``packages/alloy-metal/src/alloy/std/moe.py:1-24`` and
  ``packages/alloy-torch/src/alloy_torch/ops/moe.py:110-249``: for each token and
  slot, ``h = silu(G_e x) * (U_e x)``, ``y += w * D_e h``, summed in slot order.
  Fused gate_up rows ``[0:I]`` are gate, ``[I:2I]`` up
  (``packages/alloy-server/src/alloy_server/models/qwen3_5.py:383-385``).
* Per-element error bound of the routed output (``routed_reference``): the dense
  north-star bound on each of a slot's three products, carried to the output to first
  order; pinned in ``tests/test_oracle.py`` by a hand-computed case, by perturbing
  every product inside its bound, and by planted errors.
"""

from __future__ import annotations

import numpy as np


def router_topk(logits: np.ndarray, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """(T,E) float32 logits -> idx int32 (T,k), weights float64 (T,k)."""
    logits = np.asarray(logits, np.float32)
    order = np.argsort(-logits, axis=1, kind="stable")[:, :top_k]      # ties: lowest index first
    vals = np.take_along_axis(logits, order, axis=1).astype(np.float64)
    e = np.exp(vals - vals[:, :1])
    return order.astype(np.int32), e / e.sum(axis=1, keepdims=True)


def silu(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def moe_routed(x: np.ndarray, logits: np.ndarray, gate_up_deq: np.ndarray, down_deq: np.ndarray,
               top_k: int) -> np.ndarray:
    """fp64 routed-expert output.

    x (T,H); gate_up_deq (E, 2I, H) exact fp32 weights; down_deq (E, H, I)."""
    x = np.asarray(x, np.float64)
    idx, w = router_topk(logits, top_k)
    T = x.shape[0]
    E, two_i, H = gate_up_deq.shape
    I = two_i // 2
    y = np.zeros((T, H), np.float64)
    used = np.unique(idx)
    gu = {int(e): np.asarray(gate_up_deq[e], np.float64) for e in used}
    dn = {int(e): np.asarray(down_deq[e], np.float64) for e in used}
    for t in range(T):
        for s in range(top_k):
            e = int(idx[t, s])
            a = gu[e] @ x[t]
            h = silu(a[:I]) * a[I:]
            y[t] += w[t, s] * (dn[e] @ h)
    return y


def routed_reference(x: np.ndarray, idx: np.ndarray, w: np.ndarray, gate_up, down, I: int,
                     ratio: float = 2e-3) -> tuple[np.ndarray, np.ndarray]:
    """fp64 routed output and its per-element error bound for the tokens of x (n,H).

    idx/w: (n, top_k) routing; gate_up(e) -> (2I, H) and down(e) -> (H, I) exact fp32
    weights of expert e.  Each of a slot's three products may carry the dense bound
    (|err| <= ratio * ||input|| * max|weight row|); to first order the output then errs
    by at most, per element i,
      sum_s w_s * (ratio * ||h_s|| * max_j |D_e[i,j]|  +  ||D_e[i,:]|| * ||dh_s||)
    where dh_s = 1.13 |u| Bg + |silu(g)| Bu + 1.13 Bg Bu is the bound of
    h = silu(g) * u given Bg, Bu on the gate / up products (as in oracle.glu) and the
    second term is Cauchy-Schwarz over the down product's row."""
    x = np.asarray(x, np.float64)
    n, top_k = idx.shape
    H = x.shape[1]
    ref = np.zeros((n, H))
    bound = np.zeros((n, H))
    for t in range(n):
        xn = np.linalg.norm(x[t])
        for s in range(top_k):
            e = int(idx[t, s])
            gu = np.asarray(gate_up(e), np.float64)
            a = gu @ x[t]
            g, u = a[:I], a[I:]
            h = silu(g) * u
            row_max = np.abs(gu).max(axis=1)
            bg, bu = ratio * xn * row_max[:I], ratio * xn * row_max[I:]
            dh = 1.13 * np.abs(u) * bg + np.abs(silu(g)) * bu + 1.13 * bg * bu
            d = np.asarray(down(e), np.float64)
            ref[t] += w[t, s] * (d @ h)
            bound[t] += w[t, s] * (ratio * np.linalg.norm(h) * np.abs(d).max(axis=1)
                                   + np.linalg.norm(d, axis=1) * np.linalg.norm(dh))
    return ref, bound
