"""CPU oracle for the quantized-weight matmul path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain NumPy, what the reference (rayanht/alloy)
computes on its quantized-linear path, so that the HIP kernels can be checked
against it.  It is imported only by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``; the product (``alloy_amd``) never
imports, links or calls it and fails loudly when its HIP library is missing.

Modules
-------
``oracle.quant``  block decoders (Q8_0, Q5_0, Q4_K, Q6_K, MLX 4-bit affine),
                  the reference's split-layout repacks, fp64 reference matmul.
``oracle.moe``    router top-k + softmax, per-expert MoE composition.
``oracle.glu``    fused gated pair act(x G^T) * (x U^T), silu and tanh-form gelu.

Parity pinning (how each function is checked, beyond retyping it):

* every decoder: known-answer blocks whose expected values are written out by
  hand in ``tests/test_oracle.py``, plus an independent element-by-element
  ENCODER (``tests/golden/make_golden.py``) whose round trip
  encode(params) -> decode == d*sc*q - dmin*m is checked on random parameters
  (committed fixtures ``tests/golden/*.npz``), plus the fp32 exactness lemma
  (every product below is exact in fp32, so the decode is unique).
* Q8_0 / Q5_0: decoded two ways — from the wire block and from the reference's
  split layout (``split_q8_0`` / ``split_q5_0``) — which must agree bit for bit.
* matmul: fp64 product cross-checked against brute-force Python loops.
* router: checked against the HF formula softmax -> top-k -> renormalise and the
  lowest-index tie rule on constructed ties.
* MoE: checked against a brute-force per-token loop over experts.
* gated pair: silu against scipy's logistic function, tanh-form gelu against the
  exact erf GELU within its approximation error, the pair against a brute-force loop.

No function here is "parity unpinned".
"""
