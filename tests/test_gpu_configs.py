"""Parity of the BASELINE configs at their full sizes (fp8_native.py:114-178,255-266,320-331):

- config 1: X [4096 x 768] . W [768 x 768], seed 0 -- casts bit-exact against the oracle, the linear within the
  elementwise bound of the oracle's float64 scaled product (and 1e-2 relative Frobenius), and reference() close;
- config 4: the d12 backward's dgrads at M = 32768 (qkv, proj, w12, w3: dX = dY . W with dY ~ N(0, 1e-2) cast per
  tensor and W's transposed bytes from tcast_t) and the proj wgrad through the MN-major kernel the step uses, every
  element within the float64 bound;
- config 5: the d18 block (C 1792, H 7168, M 32768, 1% outlier activation channels x50): its casts (flat hybrid,
  two-pass, transposing) and the SwiGLU product and dz casts bit-exact against the oracle, and its 12 GEMMs within
  1e-2 of the fp32 scaled matmul with a row sample of each within the float64 bound;
- the d12 SwiGLU casts of the step at full size ([32768 x 8192]) bit-exact against the oracle.
"""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from oracle import oracle as O
from parity import OUTLIER_SLACK, assert_bf16_bits_equal, assert_elementwise, bits, qb, ref_fp32, rel, sample_rows

pytestmark = pytest.mark.gpu
M = 32768


def bf(shape, std, g, dev):
    return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16)


def act(shape, g, dev, outliers=0.0):
    """X ~ N(0, 1) with round(outliers * cols) columns x50 in fp32, rounded once to bf16 (configs 2 and 5)."""
    x = torch.randn(*shape, generator=g, device=dev)
    cols = torch.randperm(shape[1], generator=g, device=dev)[:round(outliers * shape[1])]
    x[:, cols] *= 50.0
    return x.to(torch.bfloat16)


def assert_cast(x, q, s):
    """q, s (the GPU's tcast of x) equal the oracle's bytes and dequantization scale."""
    oq, od, _ = O.tcast(bits(x))
    assert s.item() == od, (s.item(), od)
    assert np.array_equal(qb(q), oq.reshape(qb(q).shape)), f"{(qb(q) != oq).sum()} bytes differ"


# ------------------------------------------------------------------------------------------------ config 1

def test_config1_linear(dev):
    g = torch.Generator().manual_seed(0)
    X = torch.randn(4096, 768, generator=g).to(torch.bfloat16)
    W = (torch.randn(768, 768, generator=g) / 768 ** 0.5).to(torch.bfloat16)
    x, w = X.to(dev), W.to(dev)
    xq, sx = G.tcast(x)
    wq, sw = G.tcast(w)
    assert_cast(X, xq, sx)
    assert_cast(W, wq, sw)
    y = G.fp8_linear(x, w)
    oxq, osx, _ = O.tcast(bits(X))
    owq, osw, _ = O.tcast(bits(W))
    ref = O.mm64(oxq, osx, owq, osw)
    assert O.rel_fro(y.float().cpu().numpy(), ref) < 4e-3
    assert_elementwise(y, xq, sx.item(), wq, sw.item())
    # phase 3 runs the same forward; reference() (plain torch on the CPU, its eager 448 / a) agrees within 1e-2
    assert torch.equal(G.fp8_linear_f8(x, w), y)
    yr = G.reference(X, W)
    assert rel(y.cpu(), yr) < 1e-2


# ------------------------------------------------------------------------------------------------ config 4

@pytest.mark.parametrize("name,k,n", [("qkv", 1024, 3072), ("proj", 1024, 1024), ("w12", 1024, 8192),
                                      ("w3", 4096, 1024)])
def test_config4_dgrad_full_size(dev, name, k, n):
    """dX [M, k] = dY [M, n] . W [n, k]: dY ~ N(0, 1e-2) cast flat (bit-exact against the oracle), W's bytes
    transposed by tcast_t (the oracle's bytes of W, transposed), every element within the float64 bound."""
    g = torch.Generator(device=dev).manual_seed(400 + n + k)
    w = bf((n, k), k ** -0.5, g, dev)
    dy = bf((M, n), 0.1, g, dev)
    dyq, sdy = G.tcast(dy)
    assert_cast(dy, dyq, sdy)
    _, wqt, sw = G.tcast_t(w, False)
    owq, osw, _ = O.tcast(bits(w))
    assert sw.item() == osw and np.array_equal(qb(wqt)[:, :n], owq.T)
    dx = G.fp8_gemm(dyq, sdy, wqt, sw, None, False)
    assert dx.shape == (M, k)
    assert rel(dx, ref_fp32(dyq, sdy.item(), wqt, sw.item())) < 4e-3
    assert_elementwise(dx, dyq, sdy.item(), wqt, sw.item())


def test_config4_proj_wgrad_mn_major_full_size(dev):
    """dW [1024, 1024] = dY [M, 1024]^T . X [M, 1024] from the untransposed bytes (fp8_gemm_mn, split K over the
    32768 tokens), every element within the float64 bound, and bit-identical to the K-major kernel on the transposed
    bytes."""
    g = torch.Generator(device=dev).manual_seed(44)
    x = act((M, 1024), g, dev)
    dy = bf((M, 1024), 0.1, g, dev)
    xq, sx = G.tcast(x)
    dyq, sdy = G.tcast(dy)
    dw = G.fp8_gemm_mn(dyq, sdy, xq, sx)
    assert_elementwise(dw, dyq.t(), sdy.item(), xq.t(), sx.item())
    tn = G.fp8_gemm(G.tcast_t(dy)[1], sdy, G.tcast_t(x)[1], sx)
    assert torch.equal(dw.view(torch.int16), tn.view(torch.int16))


# ------------------------------------------------------------------------------------------------ config 5 (d18)

C18, H18 = 1792, 7168


@pytest.fixture(scope="module")
def d18(dev):
    g = torch.Generator(device=dev).manual_seed(5)
    t = {"x": act((M, C18), g, dev, 0.01), "xh": act((M, H18), g, dev, 0.01)}
    for name, (k, n) in {"qkv": (C18, 3 * C18), "proj": (C18, C18), "w12": (C18, 2 * H18), "w3": (H18, C18)}.items():
        t["w_" + name] = bf((n, k), k ** -0.5, g, dev)
    return t


def test_config5_activation_casts(dev, d18):
    """The d18 activations with outlier channels: [32768 x 1792] (flat single-pass hybrid) and [32768 x 7168]
    (two-pass) bit-exact against the oracle, flat and transposed."""
    for key in ("x", "xh"):
        x = d18[key]
        q, s = G.tcast(x)
        assert_cast(x, q, s)
        q2, qt, s2 = G.tcast_t(x)
        assert s2.item() == s.item() and torch.equal(q2.view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(qt.view(torch.uint8), q.view(torch.uint8).t())


@pytest.mark.parametrize("name", ["qkv", "proj", "w12", "w3"])
def test_config5_weight_casts(dev, d18, name):
    w = d18["w_" + name]
    q, qt, s = G.tcast_t(w)
    assert_cast(w, q, s)
    r16 = (w.shape[0] + 15) // 16 * 16
    assert qt.shape == (w.shape[1], r16) and torch.equal(qt.view(torch.uint8)[:, :w.shape[0]], q.view(torch.uint8).t())


def test_config5_swiglu_casts(dev, d18):
    """The d18 SwiGLU: the product cast of z = w12(x) [32768 x 14336] and the backward's dz cast (without dz in
    memory, as phase 3 runs it, and through dz) bit-exact against the oracle."""
    xq, sx = G.tcast(d18["x"])
    wq, sw = G.tcast(d18["w_w12"])
    z = G.fp8_gemm(xq, sx, wq, sw)
    g = torch.Generator(device=dev).manual_seed(55)
    da = bf((M, H18), 0.01, g, dev)
    zb, dab = bits(z), bits(da)
    aq, sa = G.swiglu_tcast(z)
    oq, od, _ = O.swiglu_tcast(zb)
    assert sa.item() == od and np.array_equal(qb(aq), oq)
    dzq, sdz = G.swiglu_bwd_q(z, da)
    odz, odq, odd, _ = O.swiglu_bwd(zb, dab)
    assert sdz.item() == odd and np.array_equal(qb(dzq), odq)
    dz, dzq2, sdz2 = G.swiglu_bwd(z, da)
    assert_bf16_bits_equal(bits(dz), odz)
    assert sdz2.item() == odd and torch.equal(dzq2.view(torch.uint8), dzq.view(torch.uint8))


def d18_gemms():
    lin = {"qkv": (C18, 3 * C18), "proj": (C18, C18), "w12": (C18, 2 * H18), "w3": (H18, C18)}
    return [(n, kind, k, nn) for n, (k, nn) in lin.items() for kind in ("fwd", "dgrad", "wgrad")]


@pytest.mark.parametrize("name,kind,k,n", d18_gemms())
def test_config5_gemms(dev, d18, name, kind, k, n):
    """The d18 block's 12 FP8 GEMMs in the layouts the step gives them (forward and dgrad K-major, wgrad MN-major
    from the untransposed bytes): within 4e-3 relative Frobenius of the fp32 scaled matmul, and 512 sampled rows of
    each within the float64 bound (with the MFMA allowance for the activations' outlier channels where they are an
    operand: forward and wgrad)."""
    g = torch.Generator(device=dev).manual_seed(sum(map(ord, name + kind)))
    x = d18["xh"] if k == H18 else d18["x"]
    w = d18["w_" + name]
    xq, sx = G.tcast(x)
    if kind == "fwd":
        wq, sw = G.tcast(w)
        a, sa, b, sb = xq, sx.item(), wq, sw.item()
        c = G.fp8_gemm(xq, sx, wq, sw)
    else:
        dyq, sdy = G.tcast(bf((M, n), 0.1, g, dev))
        if kind == "dgrad":
            _, wqt, sw = G.tcast_t(w, False)
            a, sa, b, sb = dyq, sdy.item(), wqt, sw.item()
            c = G.fp8_gemm(dyq, sdy, wqt, sw, None, False)
        else:
            a, sa, b, sb = dyq.t(), sdy.item(), xq.t(), sx.item()
            c = G.fp8_gemm_mn(dyq, sdy, xq, sx)
    assert c.shape == (a.shape[0], b.shape[0])
    assert rel(c, ref_fp32(a, sa, b, sb)) < 4e-3
    assert_elementwise(c, a, sa, b, sb, rows=sample_rows(c.shape[0], 512, 7).to(dev),
                       slack=OUTLIER_SLACK if kind != "dgrad" else 2.0 ** -16)


# ------------------------------------------------------------------------------------------------ d12 SwiGLU

def test_d12_swiglu_casts_full_size_against_oracle(dev):
    """The d12 SwiGLU casts of the step ([32768 x 8192] z, [32768 x 4096] da) against the oracle, bit for bit: the
    product cast (phase 2/3 forward), dzq without dz (phase 3) and dz with dzq (phase 2), NaN / inf planted."""
    g = torch.Generator(device=dev).manual_seed(1212)
    z = bf((M, 8192), 2.0, g, dev)
    da = bf((M, 4096), 0.01, g, dev)
    z[11, 3] = float("nan")
    da[4000, 17] = float("inf")
    zb, dab = bits(z), bits(da)
    aq, sa = G.swiglu_tcast(z)
    oq, od, _ = O.swiglu_tcast(zb)
    assert sa.item() == od and np.array_equal(qb(aq), oq)
    dzq, sdz = G.swiglu_bwd_q(z, da)
    odz, odq, odd, _ = O.swiglu_bwd(zb, dab)
    assert sdz.item() == odd and np.array_equal(qb(dzq), odq)
    dz, dzq2, _ = G.swiglu_bwd(z, da)
    assert_bf16_bits_equal(bits(dz), odz)         # (the NaN planted in z gives NaN dz: its payload may differ)
    assert np.array_equal(qb(dzq2), odq)
