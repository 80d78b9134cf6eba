"""The allocation-free GGUF MoE entry point (alloy_gguf_moe_routed_noalloc) against the
workspace entry point (alloy_gguf_moe_routed), through the C ABI: two calls in a row on
one GPU, the second with fewer tokens (a different kernel path: the few-token routed
GEMVs instead of the sorted grouped ones), each bit-identical to the workspace entry
point's output, and the first also checked against the oracle composition."""

import ctypes

import numpy as np
import pytest
import torch

import alloy_amd
from alloy_amd import _lib, synth
from oracle import moe as om
from oracle import quant as oq

pytestmark = pytest.mark.gpu

E, K_TOP, H, I = 128, 8, 2048, 768


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _experts(dev, rng):
    gu = synth.numpy_blocks("q4_k", E * 2 * I, H, rng)
    dn = synth.numpy_blocks("q6_k", E * H, I, rng)
    return gu, dn, torch.from_numpy(gu).reshape(E, 2 * I, -1).to(dev), torch.from_numpy(dn).reshape(E, H, -1).to(dev)


def _both(dev, x, lg, gut, dnt, T):
    lib = alloy_amd.lib()
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    ws_bytes = int(lib.alloy_moe_workspace_bytes(T, E, K_TOP, H, I))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    y_ws = torch.full((T, H), float("nan"), dtype=torch.float32, device=dev)
    y_na = torch.full((T, H), float("nan"), dtype=torch.float32, device=dev)
    rc = lib.alloy_gguf_moe_routed(_p(x), _p(lg), _p(gut), _p(dnt), E, K_TOP, T, H, I, _p(ws), ws_bytes, _p(y_ws), st)
    assert rc == 0, lib.alloy_last_error()
    rc = lib.alloy_gguf_moe_routed_noalloc(_p(x), _p(lg), _p(gut), _p(dnt), E, K_TOP, T, H, I, _p(y_na), st)
    assert rc == 0, lib.alloy_last_error()
    torch.cuda.synchronize()
    return y_ws.cpu().numpy(), y_na.cpu().numpy()


def test_noalloc_matches_workspace_entry(dev):
    rng = np.random.default_rng(1234)
    gu, dn, gut, dnt = _experts(dev, rng)
    for T in (64, 5):                            # second call: fewer tokens, other kernel path
        x = synth.numpy_x(T, H, rng)
        logits = rng.standard_normal((T, E)).astype(np.float32)
        xt, lg = torch.from_numpy(x).to(dev), torch.from_numpy(logits).to(dev)
        y_ws, y_na = _both(dev, xt, lg, gut, dnt, T)
        assert np.array_equal(y_ws.view(np.uint32), y_na.view(np.uint32)), f"T={T}: noalloc != workspace entry"
        assert np.isfinite(y_na).all()
        if T == 64:                              # and the oracle composition on a few tokens
            sel = [0, 17, 63]
            idx, w = om.router_topk(logits[sel], K_TOP)
            for ti, t in enumerate(sel):
                ref = np.zeros(H)
                for s in range(K_TOP):
                    e = int(idx[ti, s])
                    a = oq.dequant_q4_k(gu[e * 2 * I:(e + 1) * 2 * I], H).astype(np.float64) @ x[t].astype(np.float64)
                    h = om.silu(a[:I]) * a[I:]
                    ref += w[ti, s] * (oq.dequant_q6_k(dn[e * H:(e + 1) * H], I).astype(np.float64) @ h)
                rel = np.linalg.norm(y_na[t] - ref) / np.linalg.norm(ref)
                assert rel <= 1e-3, f"token {t}: rel={rel:.3e}"


def test_noalloc_rejects_oversize(dev):
    lib = alloy_amd.lib()
    T = 4096                                     # workspace far beyond the static scratch
    assert lib.alloy_moe_workspace_bytes(T, E, K_TOP, H, I) > (32 << 20)
    rc = lib.alloy_gguf_moe_routed_noalloc(None, None, None, None, E, K_TOP, T, H, I, None, None)
    assert rc == _lib.E_UNSUPPORTED
    assert b"static scratch" in lib.alloy_last_error()
