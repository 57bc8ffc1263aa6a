"""GPU parity of the FP8 MFMA GEMM (gpic_fp8_gemm). Exact cases (small-integer operands, power-of-two scales, identity)
are bit-exact; general cases are within the north-star tolerance of the scaled matmul of the same e4m3 operands:
relative Frobenius error <= 1e-2 (asserted tighter where the bf16 output rounding is the only error)."""
import os

import numpy as np
import pytest
import torch

import gpic_fp8 as G
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
E4 = torch.float8_e4m3fn
TOL = 1e-2


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def e4(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).view(E4).to(dev)


def rand_e4(shape, scale, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=dev) * scale).clamp(-448, 448).to(E4)


def ref_fp32(a, sa, b, sb):
    """The scaled matmul of the same operands on the GPU in fp32 (no TF32): the reference's reference() formula."""
    torch.backends.cuda.matmul.allow_tf32 = False
    return (a.float() * sa) @ (b.float() * sb).t()


def rel(x, ref):
    return (torch.linalg.norm(x.float() - ref) / torch.linalg.norm(ref)).item()


def assert_elementwise(c, a, sa, b, sb):
    """Every element within one bf16 rounding of the exact scaled product (2^-8 relative) plus an fp32
    accumulation-order allowance (2^-16 of the sum of |terms|). Catches localised corruption that a Frobenius norm
    over millions of elements would average away."""
    af = a.double() * float(sa)
    bf = b.double() * float(sb)
    exact = af @ bf.t()
    bound = exact.abs() * 2.0 ** -8 + (af.abs() @ bf.abs().t()) * 2.0 ** -16
    err = (c.double() - exact).abs()
    bad = (err > bound).sum().item()
    assert bad == 0, f"{bad} elements out of bounds; worst excess {(err - bound).max().item():.3g}"


def pollute(dev):
    """Run a GEMM over other data first, so every CU's LDS holds something else: a read of LDS before the loads that
    should fill it would then show up as wrong values instead of lucky leftovers."""
    g = torch.Generator(device=dev).manual_seed(99)
    x = (torch.randn(4096, 2048, generator=g, device=dev) * 300).clamp(-448, 448).to(E4)
    y = (torch.randn(2048, 2048, generator=g, device=dev) * 300).clamp(-448, 448).to(E4)
    G.fp8_gemm(x, torch.ones(1, device=dev), y, torch.ones(1, device=dev))


def test_exact_golden(dev, gold):
    a, b = e4(gold["gemm_a"], dev), e4(gold["gemm_b"], dev)
    sa = torch.tensor(gold["gemm_sa"], device=dev)
    sb = torch.tensor(gold["gemm_sb"], device=dev)
    c = G.fp8_gemm(a, sa, b, sb)
    assert np.array_equal(bits(c), gold["gemm_c"])
    bias = torch.from_numpy(gold["gemm_bias"].view(np.int16)).view(torch.bfloat16).to(dev)
    c = G.fp8_gemm(a, sa, b, sb, bias)
    assert np.array_equal(bits(c), gold["gemm_cbias"])


@pytest.mark.parametrize("M,N,K", [(1, 16, 16), (300, 272, 1040), (512, 1024, 4096), (64, 64, 32768)])
def test_exact_integers(dev, M, N, K):
    """Integers in [-4, 4] with power-of-two scales: every partial sum is exact in fp32, so C is bit-exact."""
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    a = torch.randint(-4, 5, (M, K), generator=g, device=dev).float().to(E4)
    b = torch.randint(-4, 5, (N, K), generator=g, device=dev).float().to(E4)
    sa = torch.tensor([0.5], device=dev)
    sb = torch.tensor([0.25], device=dev)
    pollute(dev)
    c = G.fp8_gemm(a, sa, b, sb)
    exact = (a.double() @ b.double().t()) * 0.125
    assert torch.equal(c, exact.float().to(torch.bfloat16))


def test_identity(dev):
    a = rand_e4((200, 256), 30.0, 1, dev)
    eye = torch.eye(256, device=dev).to(E4)
    c = G.fp8_gemm(a, torch.tensor([2.0], device=dev), eye, torch.tensor([0.5], device=dev))
    assert torch.equal(c, a.float().to(torch.bfloat16))


@pytest.mark.parametrize("M,N,K", [(17, 48, 160), (1000, 1024, 1024), (333, 3072, 1024), (2048, 1024, 8192),
                                   (1024, 1024, 32768), (3072, 1024, 32768)])
def test_against_oracle(dev, M, N, K):
    a = rand_e4((M, K), 40.0, 2, dev)
    b = rand_e4((N, K), 40.0, 3, dev)
    sa = torch.tensor([0.013], device=dev)
    sb = torch.tensor([0.021], device=dev)
    pollute(dev)
    c = G.fp8_gemm(a, sa, b, sb)
    assert_elementwise(c, a, 0.013, b, 0.021)
    if M * N * K <= 2 ** 31:
        ref = torch.from_numpy(O.mm64(a.view(torch.uint8).cpu().numpy(), np.float32(0.013),
                                      b.view(torch.uint8).cpu().numpy(), np.float32(0.021))).float().to(dev)
    else:
        ref = ref_fp32(a, sa, b, sb)
    r = rel(c, ref)
    assert r <= TOL and r < 4e-3
    # deterministic, including the split-K shapes, whatever ran before
    pollute(dev)
    assert torch.equal(c, G.fp8_gemm(a, sa, b, sb))


def test_bias_epilogue(dev):
    a = rand_e4((256, 1024), 20.0, 4, dev)
    b = rand_e4((1024, 1024), 20.0, 5, dev)
    sa = torch.tensor([0.01], device=dev)
    sb = torch.tensor([0.02], device=dev)
    bias = torch.randn(1024, device=dev).to(torch.bfloat16)
    c0 = G.fp8_gemm(a, sa, b, sb)
    c1 = G.fp8_gemm(a, sa, b, sb, bias)
    assert torch.equal(c1, (c0.float() + bias.float()).to(torch.bfloat16))   # the two roundings of :188-190


def test_strided_operands(dev):
    wide = rand_e4((128, 1024), 30.0, 6, dev)
    a = wide[:, 256:768]                      # row stride 1024, K = 512
    b = rand_e4((64, 512), 30.0, 7, dev)
    s = torch.tensor([1.0], device=dev)
    c = G.fp8_gemm(a, s, b, s)
    assert torch.equal(c, G.fp8_gemm(a.contiguous(), s, b, s))
    assert rel(c, ref_fp32(a, 1.0, b, 1.0)) < 4e-3


@pytest.mark.parametrize("name,M,N,K", [("qkv", 32768, 3072, 1024), ("proj", 32768, 1024, 1024),
                                        ("w12", 32768, 8192, 1024), ("w3", 32768, 1024, 4096),
                                        ("wgrad_qkv", 3072, 1024, 32768), ("wgrad_w12", 8192, 1024, 32768)])
def test_d12_shapes(dev, name, M, N, K):
    """BASELINE config 3 / 4 shapes: X ~ N(0,1), W ~ N(0, 1/K), per-tensor casts, against the fp32 scaled matmul."""
    g = torch.Generator(device=dev).manual_seed(42)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev) / K ** 0.5).to(torch.bfloat16)
    xq, sx = G.tcast(x)
    wq, sw = G.tcast(w)
    pollute(dev)
    c = G.fp8_gemm(xq, sx, wq, sw)
    assert rel(c, ref_fp32(xq, sx, wq, sw)) < 4e-3
    assert_elementwise(c, xq, sx.item(), wq, sw.item())


@pytest.mark.parametrize("M,N,K,bias,lda_pad", [
    (9000, 4000, 512, False, 0),      # 36 x 16 = 576 work items: 3 rounds per CU, ragged last row / column of tiles
    (4999, 2992, 1040, True, 16),     # partial K tile (K % 128 = 16), bias, padded leading dimension of A
    (700, 528, 9984, False, 0),       # few tiles: split K, the last split shorter; 256 x 128 tiles
    (33, 4112, 2048, True, 0),        # one tile row, many columns, bias
    (6000, 256, 4096, False, 48),     # one tile column, split K may or may not apply
    (257, 257 // 16 * 16 + 16, 160, True, 0),   # tiny K, two splits with a partial tile
    (1024, 1024, 6592, False, 0),     # text-block proj wgrad: K = 128 images x 51.5 tokens, many splits, tail tile
    (6592, 1024, 3072, True, 0),      # text-block qkv dgrad: 208 tiles of 256 x 128 (104 wide ones idle CUs)
])
def test_shape_sweep(dev, M, N, K, bias, lda_pad):
    """Shapes that put several work items on each CU, partial tiles in M, N and K, split-K with a short last split,
    the bias epilogue and a padded leading dimension: every element within the bound of assert_elementwise against
    the float64 product, and the same bytes on a second call."""
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    base = (torch.randn(M, K + lda_pad, generator=g, device=dev) * 20).clamp(-448, 448).to(E4)
    a = base[:, :K]
    b = rand_e4((N, K), 20.0, M + 1, dev)
    sa = torch.tensor([0.011], device=dev)
    sb = torch.tensor([0.017], device=dev)
    bv = (torch.randn(N, generator=g, device=dev) * 0.5).to(torch.bfloat16) if bias else None
    pollute(dev)
    c = G.fp8_gemm(a, sa, b, sb, bv)
    if bias:
        c0 = G.fp8_gemm(a, sa, b, sb)
        assert torch.equal(c, (c0.float() + bv.float()).to(torch.bfloat16))
        c = c0
    assert_elementwise(c, a, 0.011, b, 0.017)
    assert torch.equal(c, G.fp8_gemm(a, sa, b, sb))


@pytest.mark.parametrize("M,N,K,bias,pad", [
    (3072, 1024, 32768, False, 0),   # d12 qkv wgrad: dW [3N, C] from dY [T, 3N] and X [T, C]
    (8192, 1024, 32768, False, 0),   # d12 w12 wgrad
    (1024, 4096, 32768, False, 0),   # d12 w3 wgrad
    (1024, 1024, 6592, False, 0),    # text-block proj wgrad: split K, partial last K tile
    (272, 528, 300, True, 0),        # ragged tiles in M and N, K % 16 != 0 (rows past K read as zeros), bias
    (16, 16, 1, False, 0),           # one K row
    (4112, 2992, 1040, True, 32),    # padded leading dimensions, bias, partial K tile
    (9008, 4000, 512, False, 16),    # several work items per CU
    (6592, 1024, 4096, True, 0),     # text-block w3 fwd shape: 256 x 128 tiles, ragged M, bias
    (704, 528, 9984, False, 0),      # 256 x 128 tiles with 13 K splits, a partial last column of tiles (N = 528)
    (1056, 528, 2000, True, 48),     # 256 x 128 tiles, padded leading dimensions, bias, partial K tile
])
def test_mn_matches_tn(dev, M, N, K, bias, pad):
    """gpic_fp8_gemm_mn (both operands with K as the row index, the untransposed bytes of the wgrad) gives the same
    bits as gpic_fp8_gemm on the transposed operands: the MFMA sees the same values at every position (K padded
    with zeros to a multiple of 16 for the TN call). Both layouts get the same plan (tile width and K split); the
    small shapes here, the text proj wgrad and the last three cases take the 256 x 128 tile, the others 256 x 256.
    Elementwise against the float64 product as well."""
    g = torch.Generator(device=dev).manual_seed(M * 7 + N * 3 + K)
    a = (torch.randn(K, M + pad, generator=g, device=dev) * 20).clamp(-448, 448).to(E4)[:, :M]
    b = (torch.randn(K, N + pad, generator=g, device=dev) * 20).clamp(-448, 448).to(E4)[:, :N]
    sa = torch.tensor([0.013], device=dev)
    sb = torch.tensor([0.007], device=dev)
    bv = (torch.randn(N, generator=g, device=dev) * 0.5).to(torch.bfloat16) if bias else None
    k16 = (K + 15) // 16 * 16
    at = torch.zeros(M, k16, dtype=torch.uint8, device=dev)
    bt = torch.zeros(N, k16, dtype=torch.uint8, device=dev)
    at[:, :K] = a.view(torch.uint8).t()
    bt[:, :K] = b.view(torch.uint8).t()
    want = G.fp8_gemm(at.view(E4), sa, bt.view(E4), sb, bv)
    pollute(dev)
    c = G.fp8_gemm_mn(a, sa, b, sb, bv)
    assert torch.equal(bits_t(c), bits_t(want)), f"{(c != want).sum().item()} elements differ"
    if not bias and M * N <= 1 << 22:
        assert_elementwise(c, a.t(), 0.013, b.t(), 0.007)
    assert torch.equal(c, G.fp8_gemm_mn(a, sa, b, sb, bv))


def bits_t(t):
    return t.view(torch.int16)


def test_mn_past_32bit_offsets_falls_back(dev):
    """K x row stride >= 2^31 is past the MN-major kernel's 32-bit load offsets: the op routes through the K-major
    kernel on the transposed bytes (same bits). Checked on a strided view: a [K, 32] slice of a [K, 65536] tensor,
    K = 32768 (K x 65536 = 2^31)."""
    K = 32768
    g = torch.Generator(device=dev).manual_seed(77)
    base = (torch.randn(K, 65536, generator=g, device=dev) * 8).clamp(-448, 448).to(E4)
    a = base[:, :32]
    b = (torch.randn(K, 48, generator=g, device=dev) * 8).clamp(-448, 448).to(E4)
    s1 = torch.tensor([0.01], device=dev)
    c = G.fp8_gemm_mn(a, s1, b, s1)
    want = G.fp8_gemm_mn(a.contiguous(), s1, b, s1)
    assert torch.equal(c.view(torch.int16), want.view(torch.int16))


def _sweep_shapes():
    """A seeded list of ragged problems (M any size, every other one a multiple of 16; N and K multiples of 16),
    spread over both tile widths, unsplit and split K, with partial last tiles in every dimension."""
    rng = np.random.default_rng(20261201)
    out = []
    for i in range(40):
        m = int(rng.integers(1, 5000)) if i % 4 else int(rng.integers(1, 300))
        if i % 2 == 0:
            m = (m + 15) // 16 * 16      # half the cases also run the MN-major layout
        n = 16 * int(rng.integers(1, 260))
        k = 16 * int(rng.integers(1, 700)) if i % 3 else 16 * int(rng.integers(700, 2200))
        out.append((m, n, k, bool(i % 2), int(rng.integers(0, 3)) * 16))
    return out


@pytest.mark.parametrize("M,N,K,bias,pad", _sweep_shapes())
def test_random_shape_sweep(dev, M, N, K, bias, pad):
    """Seeded ragged shapes through the planner's choices (tile width, K split): the K-major GEMM within the
    elementwise bound of the float64 product and the bias added after the bf16 rounding; where M % 16 == 0, the
    MN-major GEMM on the transposed bytes gives the same bits."""
    g = torch.Generator(device=dev).manual_seed(M * 31 + N * 7 + K)
    a = (torch.randn(M, K + pad, generator=g, device=dev) * 20).clamp(-448, 448).to(E4)[:, :K]
    b = (torch.randn(N, K + pad, generator=g, device=dev) * 20).clamp(-448, 448).to(E4)[:, :K]
    sa = torch.tensor([0.013], device=dev)
    sb = torch.tensor([0.019], device=dev)
    bv = (torch.randn(N, generator=g, device=dev) * 0.5).to(torch.bfloat16) if bias else None
    c0 = G.fp8_gemm(a, sa, b, sb)
    if M * N * K <= 1 << 33:
        assert_elementwise(c0, a, 0.013, b, 0.019)
    else:
        assert rel(c0, ref_fp32(a, sa, b, sb)) < 4e-3
    if bias:
        c = G.fp8_gemm(a, sa, b, sb, bv)
        assert torch.equal(c, (c0.float() + bv.float()).to(torch.bfloat16))
    if M % 16 == 0:
        at = a.t().contiguous()
        bt = b.t().contiguous()
        assert torch.equal(bits_t(G.fp8_gemm_mn(at, sa, bt, sb)), bits_t(c0))
