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
