"""GPU parity of the dense path (dequant probe, v_dot2 GEMV, MFMA GEMV, MFMA GEMM)
against the NumPy oracle, through the C ABI.

Bars (from the north star): dequantised fp32 weights bit-exact; fp16 staging values
equal to RN16 of them; matmul relative Frobenius error <= 1e-3 and per-element
|err| <= 2e-3 * ||x_m|| * max|w_n|.  Full benchmark shapes are checked on sampled
weight rows (the oracle decodes only those rows)."""

import numpy as np
import pytest
import torch

import alloy_amd
from alloy_amd import synth
from oracle import quant as oq

pytestmark = pytest.mark.gpu

FORMATS = ["q8_0", "q5_0", "q4_k", "q6_k", "mlx_q4", "q8_0_split", "q5_0_split"]
REL_FRO, MAX_RATIO = 1e-3, 2e-3


class Weight:
    """A synthetic weight in one format: device buffers + oracle fp32 values."""

    def __init__(self, fmt, N, K, rng, dev, gs=64):
        self.fmt, self.N, self.K, self.gs = fmt, N, K, 0
        self.scales = self.biases = self.aux = None
        base = fmt.replace("_split", "")
        if fmt == "mlx_q4":
            qw, sc, bi = synth.numpy_mlx(N, K, gs, rng)
            self.host = (qw, sc, bi)
            self.w = torch.from_numpy(qw).to(dev)
            self.scales, self.biases = torch.from_numpy(sc).to(dev), torch.from_numpy(bi).to(dev)
            self.gs = gs
            self.W = oq.dequant_mlx_q4(qw, sc, bi, gs)
        else:
            blob = synth.numpy_blocks(base, N, K, rng)
            self.blob = blob
            self.W = oq.dequant(base, blob, K)
            if fmt == "q8_0_split":
                qw, sc = oq.split_q8_0(blob, K)
                self.w, self.scales = torch.from_numpy(qw).to(dev), torch.from_numpy(sc).to(dev)
            elif fmt == "q5_0_split":
                qw, qh, sc = oq.split_q5_0(blob, K)
                self.w, self.aux, self.scales = (torch.from_numpy(a).to(dev) for a in (qw, qh, sc))
            else:
                self.w = torch.from_numpy(blob).to(dev)

    def kw(self):
        return dict(scales=self.scales, biases=self.biases, aux=self.aux, group_size=self.gs)

    def op_args(self):
        """The buffers in the order of the reference op's schema."""
        if self.fmt == "mlx_q4":
            return [self.w, self.scales, self.biases]
        if self.fmt == "q8_0_split":
            return [self.w, self.scales]
        if self.fmt == "q5_0_split":
            return [self.w, self.aux, self.scales]
        return [self.w]

    def qmm(self, x, **kw):
        return alloy_amd.qmm(self.fmt, x, self.w, N=self.N, **self.kw(), **kw)

    def dequant(self, **kw):
        return alloy_amd.dequant(self.fmt, self.w, self.K, **self.kw(), **kw)


def check(y, x, W, what):
    ref = oq.ref_matmul(x, W)
    rel, ratio = oq.parity_errors(y, ref, x, W)
    assert rel <= REL_FRO and ratio <= MAX_RATIO, f"{what}: rel_fro={rel:.3e} max_ratio={ratio:.3e}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequant_bit_exact(dev, fmt):
    rng = np.random.default_rng(11)
    K = 1024 if fmt not in ("q4_k", "q6_k") else 1536
    wt = Weight(fmt, 37, K, rng, dev)
    got = wt.dequant().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), wt.W.view(np.uint32)), f"{fmt} fp32 dequant not bit-exact"
    got16 = wt.dequant(out_dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), wt.W.astype(np.float16).view(np.uint16)), f"{fmt} fp16 staging"
    part = wt.dequant(rows=(5, 9)).cpu().numpy()
    assert np.array_equal(part.view(np.uint32), wt.W[5:9].view(np.uint32))


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("N,K", [(203, 2048), (64, 3072), (130, 768)])
def test_gemv_dot2_m1(dev, fmt, N, K):
    if fmt in ("q4_k", "q6_k") and K % 256:
        pytest.skip("K not a multiple of 256")
    rng = np.random.default_rng(N + K)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(1, K, rng)
    xt = torch.from_numpy(x).to(dev)
    y = wt.qmm(xt, path="gemv", out_dtype=torch.float32).cpu().numpy()
    check(y, x, wt.W, f"{fmt} gemv N={N} K={K}")
    # every lanes-per-row choice and every kernel variant (1 = register ring with an
    # LDS row combine, 3 = wave rows with buffer loads (16/32/64 lanes; shapes needing
    # more than 4 units per lane fall back to the ring))
    for variant in (1, 3):
        for L in ((0, 16, 32, 64) if variant == 3 else (0, 16, 32, 48, 64, 128, 256)):
            yl = wt.qmm(xt, path="gemv", out_dtype=torch.float32, opts=L | (variant << 36)).cpu().numpy()
            check(yl, x, wt.W, f"{fmt} gemv L={L} variant={variant}")


@pytest.mark.parametrize("fmt", ["q6_k", "q5_0", "q8_0", "q4_k"])
@pytest.mark.parametrize("M,N,K", [(1, 1, 512), (3, 37, 512), (1, 1001, 4096), (2, 77, 14336), (8, 4099, 2048),
                                   (5, 9, 1024), (2, 1024, 4096)])
def test_gemv_tile_staged(dev, fmt, M, N, K):
    """The LDS-staged kernel (GEMV variant 4, up to 8 activation rows): partial last
    tiles, one row, the largest tiles; shapes it does not take (tiles over 48 KiB,
    records over the LDS) run the default kernels."""
    rng = np.random.default_rng(N * 7 + K + M)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for od in (torch.float32, torch.float16):
        y = wt.qmm(xt, path="gemv", out_dtype=od, opts=4 << 36).float().cpu().numpy()
        check(y, x, wt.W, f"{fmt} tile-staged gemv M={M} N={N} K={K} {od}")
    # the default route (the tile kernel for Q6_K at M = 1 and for small M on few rows)
    y = wt.qmm(xt, out_dtype=torch.float32).cpu().numpy()
    check(y, x, wt.W, f"{fmt} default route M={M} N={N} K={K}")
    y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=9 << 36).cpu().numpy()
    check(y, x, wt.W, f"{fmt} tile via the MFMA-path variant M={M} N={N} K={K}")


@pytest.mark.parametrize("fmt", ["q6_k", "q5_0", "q8_0"])
@pytest.mark.parametrize("N,K", [(1, 4096), (77, 14336), (1001, 4096), (4099, 14336), (3, 8192), (513, 2048),
                                 (65, 16384)])
def test_gemv_tile_ring_m1(dev, fmt, N, K):
    """M = 1 through the tile ring (depth 2 / 4: 1, 2 or 4 rows per tile by the row's
    unit count, two or four tiles in flight, rows summed across waves), the four-row
    tile kernel (depth 1) and the automatic choice (depth 0: the ring for Q6_K at
    K = 14336 and where the four-row tile would pass 48 KiB, Q8_0 at K = 14336),
    against the oracle; partial last tiles and fewer tiles than workgroups."""
    rng = np.random.default_rng(N * 3 + K)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(1, K, rng)
    xt = torch.from_numpy(x).to(dev)
    ys = {}
    for depth in (0, 1, 2, 4):
        for od in (torch.float32, torch.float16):
            y = wt.qmm(xt, path="gemv", out_dtype=od, opts=(4 << 36) | (depth << 32)).float().cpu().numpy()
            check(y, x, wt.W, f"{fmt} tile ring M=1 N={N} K={K} depth={depth} {od}")
            ys[depth, od] = y
    # four and two tiles in flight: the same arithmetic in the same order
    assert np.array_equal(ys[4, torch.float32], ys[2, torch.float32]), "ring depth changed the result"
    y = wt.qmm(xt, out_dtype=torch.float32).cpu().numpy()
    check(y, x, wt.W, f"{fmt} default route M=1 N={N} K={K}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_gemv_dot2_multi_row_and_f32_x(dev, fmt):
    rng = np.random.default_rng(7)
    N, K = 96, 1024
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(3, K, rng)
    y = wt.qmm(torch.from_numpy(x).to(dev), path="gemv", out_dtype=torch.float32).cpu().numpy()
    check(y, x, wt.W, f"{fmt} gemv M=3")
    x32 = rng.standard_normal((2, K)).astype(np.float32)
    y32 = wt.qmm(torch.from_numpy(x32).to(dev), path="gemv").cpu().numpy()
    check(y32, x32, wt.W, f"{fmt} gemv f32 activations")


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("M", [1, 4, 8, 16, 21])
def test_gemv_mfma(dev, fmt, M):
    rng = np.random.default_rng(M)
    N, K = 150, 2560 if fmt not in ("q4_k", "q6_k") else 2304
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for rg in (1, 2):
        y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=rg << 28).cpu().numpy()
        check(y, x, wt.W, f"{fmt} gemv_mfma M={M} rg={rg}")
    if fmt in ("q4_k", "q6_k", "mlx_q4", "q8_0", "q5_0", "q8_0_split", "q5_0_split") and M <= 16:
        # every kernel explicitly: 1 = 16x16x32 tiles, 5 = 4x4x4 broadcast (Q4_K),
        # 6 = x-stationary 16x16x32 (Q4_K), 7 = generic x-stationary (Q4_K, Q6_K, MLX),
        # 8 = x-stationary with fp16-dequantised weights (Q4_K, Q6_K, MLX, Q8_0, Q5_0)
        variants = {"q4_k": (1, 5, 6, 7, 8), "q8_0": (1, 8), "q5_0": (1, 8), "q8_0_split": (1, 8),
                    "q5_0_split": (1, 8)}.get(fmt, (1, 7, 8))
        for variant in variants:
            y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=variant << 36).cpu().numpy()
            check(y, x, wt.W, f"{fmt} gemv_mfma M={M} variant={variant}")


@pytest.mark.parametrize("fmt", ["q6_k", "q5_0", "q8_0", "q8_0_split", "q5_0_split"])
@pytest.mark.parametrize("M", [3, 8, 16])
@pytest.mark.parametrize("K,N", [(8192, 72), (11008, 33), (14336, 40)])
def test_gemv_xs_multipass(dev, fmt, M, K, N):
    """K beyond 16 waves x 8 slots: the dequantising x-stationary kernel in passes over
    K (2, 3 and 4 passes; the last pass of K = 11008 leaves waves without units, whose
    loads fall past the row or the buffer and must add nothing); forced and default."""
    rng = np.random.default_rng(K + N + M)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for opts in (8 << 36, 0):
        y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=opts).cpu().numpy()
        check(y, x, wt.W, f"{fmt} xs multi-pass M={M} K={K} N={N} opts={opts:#x}")
    y16 = wt.qmm(xt, path="gemv_mfma", opts=8 << 36).float().cpu().numpy()
    check(y16, x, wt.W, f"{fmt} xs multi-pass fp16 out M={M} K={K} N={N}")


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q5_0", "q8_0", "q8_0_split", "q5_0_split", "mlx_q4"])
@pytest.mark.parametrize("M", [3, 8, 16])
@pytest.mark.parametrize("K,N,splits", [(2048, 132, 3), (8192, 72, 2), (8192, 72, 5), (11008, 40, 4),
                                        (1024, 40, 7), (2048, 130, 2)])
def test_gemv_xs_k_split(dev, fmt, M, K, N, splits):
    """M <= 16 with K cut into ranges of whole 256-element units (one grid row each,
    fp32 partials summed in order): even splits, a short last split (8192 / 5 = 7 units
    x 4 + 4, 11008 / 4 = 11 x 3 + 10), more splits than units per wave (1024 / 7 gives
    4 splits of one unit), multi-pass K inside a split (Q6_K / Q5_0 / Q8_0 at 11008 / 4);
    M N not a multiple of 4 (M = 3, N = 130) runs unsplit.  fp32 and fp16 output."""
    if fmt == "q4_k" and K > 8192:
        pytest.skip("Q4_K over K = 8192 takes the Q4_K x-stationary kernel (no K split)")
    rng = np.random.default_rng(K + N + M + splits)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    opts = splits << 40
    y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=opts).cpu().numpy()
    check(y, x, wt.W, f"{fmt} K split M={M} K={K} N={N} S={splits}")
    y16 = wt.qmm(xt, path="gemv_mfma", opts=opts).float().cpu().numpy()
    check(y16, x, wt.W, f"{fmt} K split fp16 out M={M} K={K} N={N} S={splits}")


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("M,N,K", [(33, 130, 1024), (200, 256, 2048), (128, 64, 4096)])
def test_gemm(dev, fmt, M, N, K):
    rng = np.random.default_rng(M * N)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    y = wt.qmm(xt, path="gemm", out_dtype=torch.float32).cpu().numpy()
    check(y, x, wt.W, f"{fmt} gemm M={M} N={N} K={K}")
    if fmt == "q4_k":
        # every kernel: 1 = 128x128 generic, 4/5/6/7/8 = Q4_K tiles of 256x256 / 128x256 /
        # 128x128 / 64x256 / 64x128
        for variant in (1, 4, 5, 6, 7, 8):
            yv = wt.qmm(xt, path="gemm", out_dtype=torch.float32, opts=variant << 36)
            check(yv.cpu().numpy(), x, wt.W, f"{fmt} gemm M={M} N={N} K={K} variant={variant}")
    else:
        # 1 = 128x128 kernel; 4/5/7 = the swizzled kernel's 256x256 / 128x256 / 64x256 tiles
        for variant in (1, 4, 5, 7):
            yv = wt.qmm(xt, path="gemm", out_dtype=torch.float32, opts=variant << 36)
            check(yv.cpu().numpy(), x, wt.W, f"{fmt} gemm M={M} N={N} K={K} variant={variant}")


SWIZZLED_FORMATS = ["q8_0", "q5_0", "q6_k", "mlx_q4", "q8_0_split", "q5_0_split"]


@pytest.mark.parametrize("fmt", SWIZZLED_FORMATS)
@pytest.mark.parametrize("M,N,Ks", [(100, 300, 7), (257, 130, 17), (65, 512, 1), (96, 256, 3)])
def test_gemm_swizzled_other_formats(dev, fmt, M, N, Ks):
    """The swizzled GEMM for the other formats: K in 64-element steps (1, 3, 7 and 17
    steps: prologue only, the unrolled loop's tail and a full unroll plus tail; Q6_K in
    256-element super-blocks), rows and tokens past the tiles, every tile, fp32 and
    fp16 outputs; the blocks of the matrix's last row end at the end of its buffer."""
    K = 64 * Ks if fmt != "q6_k" else 256 * Ks
    rng = np.random.default_rng(M + N + Ks)
    wt = Weight(fmt, N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for variant in (0, 4, 5, 7):
        yv = wt.qmm(xt, path="gemm", out_dtype=torch.float32, opts=variant << 36)
        check(yv.cpu().numpy(), x, wt.W, f"{fmt} swizzled gemm M={M} N={N} K={K} variant={variant}")
    y16 = wt.qmm(xt, path="gemm", opts=5 << 36)
    check(y16.float().cpu().numpy(), x, wt.W, f"{fmt} swizzled gemm fp16 out M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K", [(130, 200, 768), (300, 130, 2816), (65, 257, 256)])
def test_gemm_q4k_odd_superblocks(dev, M, N, K):
    """K with an odd number of super-blocks (3, 11, 1): the kernel's 12-step loop ends
    with a 4- or 8-step tail, or runs the tail alone; every Q4_K tile."""
    rng = np.random.default_rng(M + K)
    wt = Weight("q4_k", N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for variant in (4, 5, 6, 7, 8):
        yv = wt.qmm(xt, path="gemm", out_dtype=torch.float32, opts=variant << 36)
        check(yv.cpu().numpy(), x, wt.W, f"gemm K={K} variant={variant}")
    yd = wt.qmm(xt, path="gemm", out_dtype=torch.float32)
    check(yd.cpu().numpy(), x, wt.W, f"gemm K={K} default plan")


@pytest.mark.parametrize("M,K,N", [(512, 4096, 256), (300, 2048, 130), (512, 14336, 512)])
def test_gemm_split_k(dev, M, K, N):
    """Few output tiles: the Q4_K GEMM plan splits K into a workspace and sums the
    slices in order; checked against the oracle for fp32 and fp16 outputs, against the
    unsplit launch, and for determinism; then every Q4_K tile with forced splits."""
    rng = np.random.default_rng(M + N)
    wt = Weight("q4_k", N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    need = int(alloy_amd.lib().alloy_gemm_workspace_bytes(alloy_amd._lib.FMT["q4_k"], M, N, K))
    assert need > 0, "this shape should take the split-K plan"
    y = wt.qmm(xt, out_dtype=torch.float32, path="gemm")
    check(y.cpu().numpy(), x, wt.W, f"split-K GEMM M={M} K={K} N={N}")
    assert torch.equal(y, wt.qmm(xt, out_dtype=torch.float32, path="gemm"))
    y16 = torch.ops.alloy.gguf_q4_k_mm(xt, wt.w)
    assert y16.dtype == torch.float16
    check(y16.float().cpu().numpy(), x, wt.W, "split-K GEMM fp16 out")
    y1 = torch.empty((M, N), dtype=torch.float32, device=dev)
    alloy_amd.lib().alloy_qmm(alloy_amd._lib.FMT["q4_k"], wt.w.data_ptr(), None, None, None, 0, xt.data_ptr(), 1,
                              y1.data_ptr(), 0, M, N, K, 3, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    check(y1.cpu().numpy(), x, wt.W, "unsplit GEMM (no workspace)")
    # every Q4_K tile with a forced split of 2 and 4
    for variant in (4, 5, 6, 7, 8):
        for S in (2, 4):
            yv = wt.qmm(xt, out_dtype=torch.float32, path="gemm", opts=(variant << 36) | (S << 40))
            check(yv.cpu().numpy(), x, wt.W, f"GEMM variant={variant} splits={S}")


def test_gemm_split_k_odd_slices(dev):
    """K splits whose slices hold an odd number of super-blocks (K = 1536: 3 per slice
    at S = 2, 2 at S = 3): each slice ends in the kernel's 4- or 8-step tail and its
    prefetches stop at the slice's end."""
    rng = np.random.default_rng(77)
    M, N, K = 260, 300, 1536
    wt = Weight("q4_k", N, K, rng, dev)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for variant in (4, 5, 6, 7, 8):
        for S in (2, 3):
            yv = wt.qmm(xt, out_dtype=torch.float32, path="gemm", opts=(variant << 36) | (S << 40))
            check(yv.cpu().numpy(), x, wt.W, f"GEMM K={K} variant={variant} splits={S}")


def test_outputs_deterministic_and_f16(dev):
    rng = np.random.default_rng(9)
    wt = Weight("q4_k", 300, 4096, rng, dev)
    for M, path in ((1, "gemv"), (8, "gemv_mfma"), (64, "gemm")):
        x = torch.from_numpy(synth.numpy_x(M, 4096, rng)).to(dev)
        a = wt.qmm(x, path=path, out_dtype=torch.float32)
        b = wt.qmm(x, path=path, out_dtype=torch.float32)
        assert torch.equal(a, b), f"{path} not deterministic"
        h = wt.qmm(x, path=path)
        assert h.dtype == torch.float16
        assert torch.equal(h, a.to(torch.float16)), f"{path} fp16 output is not RN16 of the fp32 result"


# ------------------------------------------------------------------ full benchmark shapes

def _sampled(fmt, N, K, M, dev, seed, path="auto"):
    """Run the kernel at the full shape; check sampled rows against the oracle."""
    base = fmt.replace("_split", "")
    w = synth.torch_blocks(base, N, K, seed, dev)
    x = synth.torch_x(M, K, seed + 1, dev)
    y = alloy_amd.qmm(base, x, w, out_dtype=torch.float32, path=path).cpu().numpy()
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([rng.integers(0, N, 48), [0, N - 1]]))
    blob = w[torch.from_numpy(rows).to(dev)].cpu().numpy()
    W = oq.dequant(base, blob, K)
    xs = x.cpu().numpy()
    check(y[:, rows], xs, W, f"{fmt} {M}x{K}x{N} {path}")


@pytest.mark.parametrize("fmt,M,K,N", [("q4_k", 9, 2048, 13000), ("q6_k", 5, 1024, 12301), ("q4_k", 16, 8192, 200),
                                        ("q4_k", 13, 1024, 5000)])
def test_gemv_dequant_xs_launches(dev, fmt, M, K, N):
    # the default M <= 16 kernel for Q4_K / Q6_K with fp16-dequantised weights: one
    # workgroup per CU looping over the tiles (N >= 12288, partial last tile), 16-slot
    # waves (K = 8192), two tiles per reduction (Q4_K, M > 8, mid-size N)
    _sampled(fmt, N, K, M, dev, seed=M + K + N)


LLAMA32_3B = [(3072, 3072), (3072, 1024), (3072, 8192), (8192, 3072), (3072, 128256)]   # (K, N)
LLAMA3_8B = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]


@pytest.mark.parametrize("K,N", LLAMA32_3B)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_q4_k_decode_shapes(dev, K, N, M):
    _sampled("q4_k", N, K, M, dev, seed=K + N + M)


@pytest.mark.parametrize("fmt", ["q6_k", "q5_0"])
@pytest.mark.parametrize("K,N", LLAMA3_8B)
@pytest.mark.parametrize("M", [1, 8])
def test_q6_k_q5_0_decode_shapes(dev, fmt, K, N, M):
    _sampled(fmt, N, K, M, dev, seed=K + 3 * N + M)


@pytest.mark.parametrize("fmt,M,K,N,runs", [("q4_k", 4096, 14336, 4096, 40), ("q8_0", 2048, 14336, 4096, 20)])
def test_gemm_repeatable(dev, fmt, M, K, N, runs):
    """Repeated prefill GEMMs on the same inputs give bit-identical outputs: a stage
    barrier that let a wave read an LDS stage before its buffer-to-LDS copy landed
    made 4096 x 14336 x 4096 differ in 15 % of runs."""
    w = synth.torch_blocks(fmt, N, K, 17, dev)
    x = synth.torch_x(M, K, 18, dev)
    ref = alloy_amd.qmm(fmt, x, w, out_dtype=torch.float32, path="gemm")
    y = torch.empty_like(ref)
    diff = 0
    for _ in range(runs):
        alloy_amd.qmm(fmt, x, w, out=y, path="gemm")
        diff += 0 if torch.equal(y, ref) else 1
    assert diff == 0, f"{fmt} {M}x{K}x{N}: {diff} of {runs} repeated GEMMs differ from the first"


def test_q8_0_config1(dev):
    _sampled("q8_0", 4096, 4096, 1, dev, seed=0)


def test_q8_0_split_config1(dev):
    """Config 1 through the reference operator's layout (gguf_q8_0_mm: int8 qweight and
    fp16 scales), as bench.py times it: the same blocks split by the oracle, full shape,
    sampled rows against the oracle's decode of the wire blocks."""
    N = K = 4096
    rng = np.random.default_rng(1)
    blob = synth.numpy_blocks("q8_0", N, K, rng)
    qw, sc = oq.split_q8_0(blob, K)
    x = synth.numpy_x(1, K, rng)
    y = torch.ops.alloy.gguf_q8_0_mm(torch.from_numpy(x).to(dev), torch.from_numpy(qw).to(dev),
                                     torch.from_numpy(sc).to(dev)).float().cpu().numpy()
    rows = np.unique(np.concatenate([rng.integers(0, N, 48), [0, N - 1]]))
    check(y[:, rows], x, oq.dequant("q8_0", blob[rows], K), f"q8_0 split config 1 {N}x{K}")


@pytest.mark.parametrize("M", [512, 2048, 4096])
@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 14336), (14336, 4096)])
def test_q4_k_prefill_shapes(dev, M, K, N):
    _sampled("q4_k", N, K, M, dev, seed=M + K + N, path="gemm")


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 14336), (14336, 4096)])
def test_q4_k_prefill_m4096_op_fp16(dev, K, N):
    """Config 4 at M = 4096 through the reference's op (fp16 output, the default plan
    with its workspace), sampled weight rows against the oracle."""
    M, seed = 4096, 5 * K + N
    w = synth.torch_blocks("q4_k", N, K, seed, dev)
    x = synth.torch_x(M, K, seed + 1, dev)
    y = torch.ops.alloy.gguf_q4_k_mm(x, w)
    assert y.dtype == torch.float16 and y.shape == (M, N)
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([rng.integers(0, N, 48), [0, N - 1]]))
    W = oq.dequant("q4_k", w[torch.from_numpy(rows).to(dev)].cpu().numpy(), K)
    check(y.float().cpu().numpy()[:, rows], x.cpu().numpy(), W, f"gguf_q4_k_mm M={M} K={K} N={N}")


def test_q4_k_prefill_k11008(dev):
    # 43 super-blocks per row (odd), a real prefill width (Llama-2-7B down projection)
    _sampled("q4_k", 1000, 11008, 700, dev, seed=11008, path="gemm")


@pytest.mark.parametrize("gs", [32, 128, 256])
def test_gemv_xs_mlx_group_sizes(dev, gs):
    # x-stationary MLX GEMV with 8, 2 and 1 groups per 256-element unit
    rng = np.random.default_rng(gs)
    N, K, M = 150, 2048, 5
    wt = Weight("mlx_q4", N, K, rng, dev, gs=gs)
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    for variant in (0, 7, 8):
        y = wt.qmm(xt, path="gemv_mfma", out_dtype=torch.float32, opts=variant << 36).cpu().numpy()
        check(y, x, wt.W, f"mlx_q4 gs={gs} gemv_mfma M={M} variant={variant}")


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q8_0_split", "q5_0_split", "mlx_q4"])
@pytest.mark.parametrize("M", [1, 3])
def test_batched_ops(dev, fmt, M):
    # the reference's batched_*_mm: separate outputs per matrix; at M = 1 one launch
    # per 8 matrices (10 matrices here: two launches), an empty matrix in between
    rng = np.random.default_rng(40 + M)
    K = 1024
    Ns = [96, 33, 0, 200, 17, 64, 48, 31, 16, 130]
    ws = [Weight(fmt, N, K, rng, dev) if N else None for N in Ns]
    x = synth.numpy_x(M, K, rng)
    xt = torch.from_numpy(x).to(dev)
    name = {"q4_k": "batched_gguf_q4_k_mm", "q6_k": "batched_gguf_q6_k_mm", "q8_0_split": "batched_gguf_q8_0_mm",
            "q5_0_split": "batched_gguf_q5_0_mm", "mlx_q4": "batched_mlx_q4_mm"}[fmt]
    lists = None
    for N, w in zip(Ns, ws):
        if w is None:
            if fmt == "mlx_q4":
                bufs = [torch.zeros((0, K // 2), dtype=torch.uint8, device=dev),
                        torch.zeros((0, K // 64), dtype=torch.float16, device=dev),
                        torch.zeros((0, K // 64), dtype=torch.float16, device=dev)]
            elif fmt == "q8_0_split":
                bufs = [torch.zeros((0, K), dtype=torch.int8, device=dev),
                        torch.zeros((0, K // 32), dtype=torch.float16, device=dev)]
            elif fmt == "q5_0_split":
                bufs = [torch.zeros((0, K // 2), dtype=torch.uint8, device=dev)] * 2 + \
                       [torch.zeros((0, K // 32), dtype=torch.float16, device=dev)]
            else:
                bufs = [torch.zeros((0, K // 256 * (144 if fmt == "q4_k" else 210)), dtype=torch.uint8, device=dev)]
        else:
            bufs = w.op_args()
        lists = [[b] for b in bufs] if lists is None else [l + [b] for l, b in zip(lists, bufs)]
    outs = getattr(torch.ops.alloy, name)(xt, *lists)
    assert len(outs) == len(Ns)
    for N, w, y in zip(Ns, ws, outs):
        assert y.shape == (M, N) and y.dtype == torch.float16
        if w is not None:
            check(y.float().cpu().numpy(), x, w.W, f"{name} M={M} N={N}")


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k", "q8_0_split", "q5_0_split", "mlx_q4"])
def test_embedding_bit_exact(dev, fmt):
    # the reference's gguf_q*_embedding / mlx_q4_embedding: exact fp32 rows; ids
    # outside the table give zero rows; int32 and int64 ids, any id shape
    rng = np.random.default_rng(23)
    N, K = 300, 1024
    wt = Weight(fmt, N, K, rng, dev)
    name = {"q4_k": "gguf_q4_k_embedding", "q6_k": "gguf_q6_k_embedding", "q8_0_split": "gguf_q8_0_embedding",
            "q5_0_split": "gguf_q5_0_embedding", "mlx_q4": "mlx_q4_embedding"}[fmt]
    ids = rng.integers(0, N, size=(3, 7))
    ids[0, 0], ids[2, 6] = -1, N
    for dt in (torch.int64, torch.int32):
        out = getattr(torch.ops.alloy, name)(torch.from_numpy(ids).to(dev).to(dt), *wt.op_args())
        assert out.shape == (3, 7, K) and out.dtype == torch.float32
        got = out.cpu().numpy()
        want = np.where(((ids >= 0) & (ids < N))[..., None], wt.W[np.clip(ids, 0, N - 1)], 0.0).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name} {dt}"


def test_embedding_modules_and_tied_head(dev):
    rng = np.random.default_rng(4)
    N, K = 64, 512
    wt = Weight("q4_k", N, K, rng, dev)
    emb = alloy_amd.GGUFQ4_KEmbedding(num_embeddings=N, embedding_dim=K, embed_scale=2.0, blocks=wt.w)
    ids = torch.tensor([[1, 5, 63]], device=dev)
    assert np.array_equal(emb(ids).cpu().numpy()[0], 2.0 * wt.W[[1, 5, 63]])
    head = alloy_amd.tied_output_head(emb, torch.nn.Linear(K, N, bias=False))
    x = torch.from_numpy(synth.numpy_x(2, K, rng)).to(dev)
    check(head(x).float().cpu().numpy(), x.cpu().numpy(), wt.W, "tied Q4_K head")
    with pytest.raises(NotImplementedError):
        alloy_amd.tied_output_head(emb, torch.nn.Linear(K, N, bias=True))


@pytest.mark.gpu
def test_modules_loaded_from_gguf_and_mlx_files(dev, tmp_path):
    """GGUF file -> GGUF*Linear / Embedding and MLX safetensors -> MLXQ4Linear on the GPU."""
    from safetensors.torch import save_file

    from alloy_amd import gguf, mlx
    rng = np.random.default_rng(21)
    N, K = 96, 1024
    blobs = {fm: synth.numpy_blocks(fm, N, K, rng) for fm in ("q8_0", "q5_0", "q4_k", "q6_k")}
    p = tmp_path / "w.gguf"
    gguf.write_gguf(p, {"general.architecture": "llama"}, [(f"w.{fm}", fm, (K, N), b) for fm, b in blobs.items()])
    f = gguf.read_gguf(p)
    x = torch.from_numpy(synth.numpy_x(3, K, rng)).to(dev)
    for fm, b in blobs.items():
        W = oq.dequant(fm, b, K)
        check(f.linear(f"w.{fm}").to(dev)(x).float().cpu().numpy(), x.cpu().numpy(), W, f"gguf file {fm}")
        emb = f.embedding(f"w.{fm}").to(dev)
        ids = torch.tensor([0, 7, N - 1], device=dev)
        assert np.array_equal(emb(ids).cpu().numpy(), W[[0, 7, N - 1]]), fm
    q8, s, bb = synth.numpy_mlx(N, K, 64, rng)
    st = tmp_path / "model.safetensors"
    save_file({"proj.weight": torch.from_numpy(q8.view("<u4").copy()).view(torch.int32),
               "proj.scales": torch.from_numpy(s), "proj.biases": torch.from_numpy(bb)}, str(st))
    ck = mlx.read_mlx_checkpoint([st], {"quantization": {"group_size": 64, "bits": 4}})
    W = oq.dequant("mlx_q4", q8, K, scales=s, biases=bb, group_size=64)
    check(ck.linear("proj").to(dev)(x).float().cpu().numpy(), x.cpu().numpy(), W, "mlx file")
