"""NumPy restatement of the reference's fused gated pair (gate . up with an
activation) — TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``y = act(x @ G^T) * (x @ U^T)`` — ``packages/alloy-metal/src/alloy/std/quant.py``
  ``dot_q4_k_silu`` / ``dot_q4_k_gelu_v2`` (``:1456-1940``; store of
  ``gelu_tanh(g) * u`` at ``:1647``), ``dot_mlx_q4_silu`` (``:2833-2887``) and the
  Q8_0 pair (``:356-759``).
* silu(v) = v / (1 + exp(-v)); gelu in the tanh form
  ``0.5 v (1 + tanh(clamp(0.7978845608 (v + 0.044715 v^3), -10, 10)))``
  (``packages/alloy-metal/src/alloy/_compiler/trace/__init__.py:432-450``,
  ``packages/alloy-metal/src/alloy/_runtime/buffer_ops.py:50-62``).

Pinning: silu against ``scipy.special.expit`` (v * sigmoid(v)); gelu against the
exact erf GELU (``0.5 v (1 + erf(v / sqrt 2))``, ``math.erf``) within the tanh
form's known approximation error, and its limits (0 at 0, v for large v, 0 for
very negative v); the pair against a brute-force loop; ``glu_error_bound`` by
perturbing both products within their bounds and by planted errors beyond it
(``tests/test_oracle.py``).
"""

from __future__ import annotations

import numpy as np

from .quant import ref_matmul


def silu(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


def gelu_tanh(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float64)
    u = np.clip(0.7978845608028654 * (v + 0.044715 * v ** 3), -10.0, 10.0)
    return 0.5 * v * (1.0 + np.tanh(u))


ACTS = {"silu": silu, "gelu": gelu_tanh}


def glu(x: np.ndarray, gate_deq: np.ndarray, up_deq: np.ndarray, act: str) -> np.ndarray:
    """fp64 act(x @ G^T) * (x @ U^T) for x (M,K), G and U (N,K) dequantised weights."""
    return ACTS[act](ref_matmul(x, gate_deq)) * ref_matmul(x, up_deq)


# |act'(v)| <= ACT_SLOPE for both activations (silu' lies in [-0.100, 1.100], the tanh
# GELU's in [-0.129, 1.129])
ACT_SLOPE = 1.13


def glu_error_bound(x: np.ndarray, gate_deq: np.ndarray, up_deq: np.ndarray, act: str,
                    ratio: float = 2e-3) -> np.ndarray:
    """Per-element error bound (M,N) of act(g)*u given the north-star bound on each product,
    |g_err| <= ratio*||x_m||*max|G_n| = Bg and likewise Bu: by the mean value theorem
    |act(g+dg)(u+du) - act(g)u| <= ACT_SLOPE*|u|*Bg + |act(g)|*Bu + ACT_SLOPE*Bg*Bu."""
    g, u = ref_matmul(x, gate_deq), ref_matmul(x, up_deq)
    xn = np.linalg.norm(np.asarray(x, np.float64), axis=1)[:, None]
    bg = ratio * xn * np.abs(np.asarray(gate_deq, np.float64)).max(axis=1)[None, :]
    bu = ratio * xn * np.abs(np.asarray(up_deq, np.float64)).max(axis=1)[None, :]
    return ACT_SLOPE * np.abs(u) * bg + np.abs(ACTS[act](g)) * bu + ACT_SLOPE * bg * bu
