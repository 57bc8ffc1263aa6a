"""GPU parity of the up projection with its SwiGLU product cast (gpic_fp8_gemm_swiglu_tcast, gemm.hip's SwiGLU
instance): z, the product's e4m3 bytes and its scale must equal, bit for bit, the two ops it replaces -- fp8_gemm
(fp8_native.py:175-178) then swiglu_tcast (fp8_native.py:130-144) -- and the bytes and scale must equal the oracle's
swiglu_tcast of that z."""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from oracle import oracle as O
from parity import bits, qb

pytestmark = pytest.mark.gpu


def operands(M, C, H, seed, dev, k=1.0, outliers=0.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, C, generator=g, device=dev) * k
    if outliers:
        cols = torch.randperm(C, generator=g, device=dev)[:max(1, round(outliers * C))]
        x[:, cols] *= 50.0
    w12 = torch.randn(2 * H, C, generator=g, device=dev) / C ** 0.5
    xq, sx = G.tcast(x.to(torch.bfloat16))
    wq, sw = G.tcast(w12.to(torch.bfloat16))
    return xq, sx, wq, sw


def fused_and_unfused(xq, sx, wq, sw):
    z0 = G.fp8_gemm(xq, sx, wq, sw)
    q0, s0 = G.swiglu_tcast(z0)
    z1, q1, s1 = G.gemm_swiglu_tcast(xq, sx, wq, sw)
    return (z0, q0, s0), (z1, q1, s1)


def assert_same(u, f):
    (z0, q0, s0), (z1, q1, s1) = u, f
    assert torch.equal(z0.view(torch.int16), z1.view(torch.int16)), "z"
    assert s0.item() == s1.item(), (s0.item(), s1.item())
    assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8)), "product bytes"


@pytest.mark.parametrize("M,C,H,k,outliers", [
    (32768, 1024, 4096, 1.0, 0.0),      # d12: one GPU's tokens, width 1024, hidden 4096
    (32768, 1792, 7168, 1.0, 0.01),     # d18 with 1% outlier channels x50
    (1000, 256, 256, 1.0, 0.0),         # M not a multiple of the 256-row tile: zero rows past M in the last tiles
    (300, 1040, 128, 1.0, 0.0),         # K % 128 != 0: the partial-K-tile instance
    (512, 512, 384, 300.0, 0.0),        # |z1| >= 2^8 for many values: sigmoid computed outside the table
    (512, 512, 384, 1e-6, 0.0),         # |z1| < 2^-16: the other side of the table
])
def test_fused_equals_unfused(dev, M, C, H, k, outliers):
    xq, sx, wq, sw = operands(M, C, H, M + C + H, dev, k, outliers)
    assert_same(*fused_and_unfused(xq, sx, wq, sw))


def test_fused_against_oracle(dev):
    """The product's bytes and scale are the oracle's swiglu_tcast of the fused op's own z."""
    xq, sx, wq, sw = operands(640, 384, 256, 5, dev, outliers=0.02)
    z, q, s = G.gemm_swiglu_tcast(xq, sx, wq, sw)
    oq, od, _ = O.swiglu_tcast(bits(z))
    assert s.item() == od
    assert np.array_equal(qb(q), oq)


def test_nan_and_empty(dev):
    """A NaN byte in the e4m3 input (tcast itself never writes one: it saturates NaN to -448) makes its row of z NaN;
    the product ignores it in the amax and casts it to -448, as swiglu_tcast does; an empty M gives the scale of an
    empty tensor."""
    g = torch.Generator(device=dev).manual_seed(6)
    x = torch.randn(300, 256, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(512, 256, generator=g, device=dev) / 16).to(torch.bfloat16)
    xq, sx = G.tcast(x)
    wq, sw = G.tcast(w)
    xq.view(torch.uint8)[17, 3] = 0x7F   # e4m3fn NaN
    u, f = fused_and_unfused(xq, sx, wq, sw)
    (z0, q0, s0), (z1, q1, s1) = u, f
    nan0, nan1 = torch.isnan(z0), torch.isnan(z1)
    assert torch.equal(nan0, nan1) and nan0[17].all()
    assert torch.equal(z0[~nan0].view(torch.int16), z1[~nan1].view(torch.int16))
    assert s0.item() == s1.item() and torch.equal(q0.view(torch.uint8), q1.view(torch.uint8))
    z, q, s = G.gemm_swiglu_tcast(xq[:0], sx, wq, sw)
    assert z.shape == (0, 512) and q.shape == (0, 256)
    assert s.item() == np.float32(1e-12) / np.float32(448.0)


def test_mlp_uses_the_fused_op_with_the_same_bits(dev, monkeypatch):
    """fp8_mlp_f8 (native3) forward and backward give the same bits whether the up projection runs fused or as the
    two ops (the fused op switched off by hiding it behind the two-op path)."""
    from gpic_fp8 import fp8_native as F
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(4, 256, 512, generator=g, device=dev).to(torch.bfloat16)
    w12 = (torch.randn(2048, 512, generator=g, device=dev) / 512 ** 0.5).to(torch.bfloat16)
    w3 = (torch.randn(512, 1024, generator=g, device=dev) / 1024 ** 0.5).to(torch.bfloat16)
    dy = (torch.randn(4, 256, 512, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    calls = []
    real = F.gemm_swiglu_tcast

    def counted(*a):
        calls.append(1)
        return real(*a)

    runs = []
    for fused in (True, False):
        if fused:
            monkeypatch.setattr(F, "gemm_swiglu_tcast", counted)
        else:
            monkeypatch.setattr(F, "_up_swiglu", lambda xq, sx, wq, sw: (lambda z: (z, *F.swiglu_tcast(z)))(
                F.fp8_gemm(xq, sx, wq, sw)))
        leaves = [t.detach().clone().requires_grad_() for t in (x, w12, w3)]
        y = G.fp8_mlp_f8(*leaves)
        y.backward(dy)
        runs.append([y] + [t.grad for t in leaves])
    assert calls, "the fused op was not used"
    for a, b in zip(*runs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
