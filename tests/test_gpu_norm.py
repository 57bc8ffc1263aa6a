"""GPU parity of the norm sites' producer with its e4m3 cast (gpic_fp8_res_mod_rmsnorm, norm.hip) against the oracle,
bit for bit (x_new, rstd, h, h's bytes and scale), and of the functions built on it: the reference's mod_rmsnorm /
res_mod_rmsnorm API (fused_norm.py:293-313) and the fused FP8 consumers, which must equal the same computation done
unfused (the norm writing bf16 h, then the phase-3 linear / MLP casting it) bit for bit, forward and backward."""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O
from parity import assert_bf16_bits_equal, bits, qb

pytestmark = pytest.mark.gpu


def inputs(B, N, C, seed, dev, res=True, k=1.0, outliers=0.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(B, N, C, generator=g, device=dev) * k
    if outliers:
        cols = torch.randperm(C, generator=g, device=dev)[:round(outliers * C)]
        x[..., cols] *= 50.0
    x = x.to(torch.bfloat16)
    a = torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16)
    # gate / shift / scale as the block gets them: [B, 1, C] chunks (strided views) of one adaLN output
    mod = (torch.randn(B, 1, 6 * C, generator=g, device=dev) * 0.2).to(torch.bfloat16)
    shift, scale, gate = mod[..., :C], mod[..., C:2 * C], mod[..., 2 * C:3 * C]
    w = (1 + 0.1 * torch.randn(C, generator=g, device=dev))
    return x, (a if res else x), (gate if res else x), w, shift, scale


def oracle(x, a, gate, w, shift, scale, eps, res):
    B, N, C = x.shape
    u = lambda t, r: bits(t.reshape(r, C))
    return O.mod_rmsnorm_q(u(x, B * N), w.cpu().numpy(), u(shift, B), u(scale, B), N, eps,
                           u(a, B * N) if res else None, u(gate, B) if res else None)


def check(x, a, gate, w, shift, scale, eps, res):
    B, N, C = x.shape
    xn, h, hq, s, rstd = G.res_mod_rmsnorm_q(x, a, gate, w, shift, scale, eps, res, True)
    oxn, oh, orstd, ohq, od = oracle(x, a, gate, w, shift, scale, eps, res)
    if res:
        assert np.array_equal(bits(xn.reshape(-1, C)), oxn)
    assert np.array_equal(rstd.cpu().numpy().view(np.uint32), orstd.view(np.uint32)), "rstd"
    assert_bf16_bits_equal(bits(h.reshape(-1, C)), oh)
    assert s.item() == od, (s.item(), od)
    assert np.array_equal(qb(hq.reshape(-1, C)), ohq)
    # without the bf16 h: the same bytes
    _, h0, hq0, s0, _ = G.res_mod_rmsnorm_q(x, a, gate, w, shift, scale, eps, res, False)
    assert h0.numel() == 0 and s0.item() == s.item() and torch.equal(hq0.view(torch.uint8), hq.view(torch.uint8))
    # the norm alone (no cast, the reference's op): the same h, x_new and rstd
    xn1, h1, hq1, s1, r1 = G.res_mod_rmsnorm_q(x, a, gate, w, shift, scale, eps, res, True, False)
    assert hq1.numel() == 0 and s1.numel() == 0
    assert torch.equal(h1.view(torch.int16), h.view(torch.int16)) and torch.equal(r1.view(torch.int32), rstd.view(torch.int32))
    if res:
        assert torch.equal(xn1.view(torch.int16), xn.view(torch.int16))
    return hq, s


@pytest.fixture
def knob():
    yield
    L.set_single_pass(True, -1)


@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("B,N,C", [
    (128, 256, 1024),    # d12, one GPU's 32768 tokens: the single pass (8 rows per wave, 1024 workgroups)
    (128, 256, 1792),    # d18: more than the single pass holds -> two passes
    (2, 100, 768),       # single pass, a partly filled last workgroup
    (3, 64, 2560),       # wider than the single pass takes (C / 256 = 10) -> two passes
    (8, 512, 256),       # narrow rows (10 per wave)
    (128, 256, 896),     # d11 (the ladder's width 896): the last group of each row half full
    (128, 256, 1152),    # d13 (1152)
    (3, 40, 100),        # one partial group per row (lanes 0-24)
    (2, 33, 2340),       # wider than 2048 and no multiple of 256: the row-at-a-time kernel with a partial group
])
def test_norm_against_oracle(dev, B, N, C, res):
    x, a, gate, w, shift, scale = inputs(B, N, C, B + N + C + res, dev, res, outliers=0.01)
    check(x, a, gate, w, shift, scale, 1e-6, res)


@pytest.mark.parametrize("res", [False, True])
def test_norm_wave_past_the_end(dev, res):
    """24 rows of 8 tokens (3 batches) at C = 1024: one workgroup of 4 waves x 8 rows, the fourth wave wholly past the
    end. Its rows re-read the last row and count in the maximum, so they must take the last batch's modulation, not
    the next batch row's: the row after the modulation slice (inside the same allocation) holds 1000s here, which
    would set the scale."""
    B, N, C = 3, 8, 1024
    x, a, _, w, _, _ = inputs(B, N, C, 31, dev, res)
    g = torch.Generator(device=dev).manual_seed(32)
    mod_full = (torch.randn(B + 1, 1, 6 * C, generator=g, device=dev) * 0.2).to(torch.bfloat16)
    mod_full[B] = 1000.0
    mod = mod_full[:B]
    shift, scale, gate = mod[..., :C], mod[..., C:2 * C], mod[..., 2 * C:3 * C]
    check(x, a if res else x, gate if res else x, w, shift, scale, 1e-6, res)


def test_norm_single_two_pass_and_zero_wait_agree(dev, knob):
    """The d12 site 2 through the single pass, its zero-wait path (partials not yet published computed from the rows)
    and the forced two-pass path: the same bytes, equal to the oracle's."""
    x, a, gate, w, shift, scale = inputs(128, 256, 1024, 11, dev, True)
    outs = []
    for enabled, wait in ((True, -1), (True, 0), (False, -1)):
        L.set_single_pass(enabled, wait)
        outs.append(check(x, a, gate, w, shift, scale, 1e-6, True))
    for hq, s in outs[1:]:
        assert s.item() == outs[0][1].item() and torch.equal(hq.view(torch.uint8), outs[0][0].view(torch.uint8))


def test_norm_nan_row_and_empty(dev):
    """A NaN in x makes its row NaN (as the reference's would), ignored by the amax and cast to -448 (the cast rule);
    an empty input writes only the scale of an empty tensor."""
    x, a, gate, w, shift, scale = inputs(4, 64, 1024, 12, dev, True)
    x[1, 7, 100] = float("nan")
    check(x, a, gate, w, shift, scale, 1e-6, True)
    e = x[:, :0]
    xn, h, hq, s, rstd = G.res_mod_rmsnorm_q(e, e, gate, w, shift, scale, 1e-6, True, True)
    assert hq.numel() == 0 and s.item() == np.float32(1e-12) / np.float32(448.0)


def _eager(x, a, gate, w, shift, scale, eps, res):
    """The reference kernel's formula (x + gate * a in fp32, one rounding of h) in torch fp32 autograd."""
    xs = (x.float() + gate.float() * a.float()) if res else x.float()
    xs = xs.to(torch.bfloat16).float() if res else xs
    r = torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + eps)
    n = (w.float() * (xs * r))
    return xs, n * (1 + scale.float()) + shift.float()


@pytest.mark.parametrize("res", [False, True])
def test_drop_in_api_and_backward(dev, res):
    """mod_rmsnorm / res_mod_rmsnorm (the reference's API): h is the kernel's (the oracle's) and the gradients of x,
    a, gate, w, shift, scale are within 1e-2 of fp32 autograd of the reference kernel's formula."""
    B, N, C, eps = 4, 128, 1024, 1e-6
    x, a, gate, w, shift, scale = inputs(B, N, C, 13 + res, dev, res)
    leaves = [t.detach().clone().requires_grad_() for t in (x, a, gate, w, shift, scale)]
    xl, al, gl, wl, shl, scl = leaves
    if res:
        xn, h = G.res_mod_rmsnorm(xl, al, gl, wl, shl, scl, eps)
    else:
        h = G.mod_rmsnorm(xl, wl, shl, scl, eps)
    _, oh, _, _, _ = oracle(x, a, gate, w, shift, scale, eps, res)
    assert_bf16_bits_equal(bits(h.reshape(-1, C)), oh)
    dh = (torch.randn_like(h) * 0.1).to(torch.bfloat16)
    dxn = (torch.randn_like(h) * 0.1).to(torch.bfloat16) if res else None
    torch.autograd.backward([h, xn] if res else [h], [dh, dxn] if res else [dh])
    ref_leaves = [t.detach().float().clone().requires_grad_() for t in (x, a, gate, w, shift, scale)]
    rxs, rh = _eager(*ref_leaves, eps, res)
    torch.autograd.backward([rh, rxs] if res else [rh], [dh.float(), dxn.float()] if res else [dh.float()])
    names = ("x", "a", "gate", "w", "shift", "scale") if res else ("x", None, None, "w", "shift", "scale")
    for n, got, want in zip(names, leaves, ref_leaves):
        if n is None:
            continue
        r = (torch.linalg.norm(got.grad.float() - want.grad) / torch.linalg.norm(want.grad)).item()
        assert r < 1e-2, (n, r)


@pytest.mark.parametrize("C", [896, 1024])
@pytest.mark.parametrize("res", [False, True])
def test_reference_named_ops(dev, res, C):
    """torch.ops.gpic.res_mod_rmsnorm_fwd / _bwd (the reference's op names and schemas, fused_norm.py:151-245): the
    forward's outputs equal the kernel op's bit for bit, its registered backward gives the same gradients as
    mod_rmsnorm / res_mod_rmsnorm bit for bit, and the backward op equals the kernel's backward op."""
    from gpic_fp8 import norm as NM
    B, N, eps = 4, 128, 1e-6
    x, a, gate, w, shift, scale = inputs(B, N, C, 29 + res + C, dev, res)
    xn, h, rstd = torch.ops.gpic.res_mod_rmsnorm_fwd(x, a, gate, w, shift, scale, eps, res)
    xn1, h1, _, _, r1 = G.res_mod_rmsnorm_q(x, a, gate, w, shift, scale, eps, res, True, False)
    assert torch.equal(h.view(torch.int16), h1.view(torch.int16)) and torch.equal(rstd.view(torch.int32), r1.view(torch.int32))
    assert (xn.numel() == 0) if not res else torch.equal(xn.view(torch.int16), xn1.view(torch.int16))
    dh = (torch.randn_like(h) * 0.1).to(torch.bfloat16)
    dxn = (torch.randn_like(h) * 0.1).to(torch.bfloat16)
    grads = []
    for via_op in (True, False):
        leaves = [t.detach().clone().requires_grad_() for t in (x, a, gate, w, shift, scale)]
        xl, al, gl, wl, shl, scl = leaves
        if via_op:
            on, oh, _ = torch.ops.gpic.res_mod_rmsnorm_fwd(xl, al if res else xl, gl if res else xl, wl, shl, scl, eps,
                                                           res)
        elif res:
            on, oh = G.res_mod_rmsnorm(xl, al, gl, wl, shl, scl, eps)
        else:
            on, oh = None, G.mod_rmsnorm(xl, wl, shl, scl, eps)
        torch.autograd.backward([oh, on] if res else [oh], [dh, dxn] if res else [dh])
        grads.append([t.grad for t in (leaves if res else (xl, wl, shl, scl))])
    for got, want in zip(*grads):
        assert torch.equal(got, want)
    xs = xn if res else x
    out = torch.ops.gpic.res_mod_rmsnorm_bwd(dh, dxn, xs, a, gate, w, scale, rstd, res, res)
    ref = NM.res_mod_rmsnorm_bwd_k(dh, dxn if res else None, xs, a if res else None, gate if res else None, w, scale,
                                   rstd)
    for got, want in zip(out, ref):
        assert torch.equal(got, want)


def test_fused_site1_linear_equals_unfused(dev):
    """fp8_mod_rmsnorm_linear (h cast in the norm, never written in bf16) against mod_rmsnorm then fp8_linear_f8 (h
    written in bf16 and cast by tcast): the same output and gradients bit for bit."""
    B, N, C, eps = 8, 256, 1024, 1e-6
    x, _, _, w, shift, scale = inputs(B, N, C, 21, dev, False, outliers=0.01)
    g = torch.Generator(device=dev).manual_seed(22)
    weight = (torch.randn(3 * C, C, generator=g, device=dev) / C ** 0.5).to(torch.bfloat16)
    dy = (torch.randn(B, N, 3 * C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    runs = []
    for fused in (True, False):
        leaves = [t.detach().clone().requires_grad_() for t in (x, w, shift, scale, weight)]
        xl, wl, shl, scl, Wl = leaves
        y = (G.fp8_mod_rmsnorm_linear(xl, wl, shl, scl, eps, Wl) if fused
             else G.fp8_linear_f8(G.mod_rmsnorm(xl, wl, shl, scl, eps), Wl))
        y.backward(dy)
        runs.append([y] + [t.grad for t in leaves])
    for got, want in zip(*runs):
        assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got,
                           want.view(torch.int16) if want.dtype == torch.bfloat16 else want)


def test_fused_site2_mlp_equals_unfused(dev):
    """fp8_res_mod_rmsnorm_mlp against res_mod_rmsnorm then fp8_mlp_f8: x_new, the MLP output and every gradient
    (x, a, gate, w, shift, scale, w12, w3) bit for bit."""
    B, N, C, H, eps = 8, 256, 1024, 4096, 1e-6
    x, a, gate, w, shift, scale = inputs(B, N, C, 31, dev, True)
    g = torch.Generator(device=dev).manual_seed(32)
    w12 = (torch.randn(2 * H, C, generator=g, device=dev) / C ** 0.5).to(torch.bfloat16)
    w3 = (torch.randn(C, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16)
    dy = (torch.randn(B, N, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    dxn = (torch.randn(B, N, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    runs = []
    for fused in (True, False):
        leaves = [t.detach().clone().requires_grad_() for t in (x, a, gate, w, shift, scale, w12, w3)]
        xl, al, gl, wl, shl, scl, w12l, w3l = leaves
        if fused:
            xn, y = G.fp8_res_mod_rmsnorm_mlp(xl, al, gl, wl, shl, scl, eps, w12l, w3l)
        else:
            xn, h = G.res_mod_rmsnorm(xl, al, gl, wl, shl, scl, eps)
            y = G.fp8_mlp_f8(h, w12l, w3l)
        torch.autograd.backward([xn, y], [dxn, dy])
        runs.append([xn, y] + [t.grad for t in leaves])
    for got, want in zip(*runs):
        assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got,
                           want.view(torch.int16) if want.dtype == torch.bfloat16 else want)


def torch_backward(dh, dxn, xs, a, gate, w, scale, rstd):
    """The reference's analytic backward of the norm site (fused_norm.py:94-147) in torch fp32 ops, the checker of
    the HIP kernel: (dx, da, d_gate, d_w, d_shift, d_scale) with dx, da before their bf16 rounding."""
    B, N, C = xs.shape
    r = rstd.view(B, N, 1)
    t = xs.float() * r
    wf = w.float()
    n = (wf * t).to(torch.bfloat16).float()
    dhf = dh.float()
    dsh, dsc = dhf.sum(1), (dhf * n).sum(1)
    dn = dhf * (1.0 + scale.reshape(B, 1, C).float())
    dw = (dn * t).sum((0, 1))
    dt = dn * wf
    dx = r * (dt - t * ((dt * t).sum(-1, keepdim=True) / C))
    if dxn is not None:
        dx = dx + dxn.float()
    if a is None:
        return dx, None, None, dw, dsh, dsc
    return dx, dx * gate.reshape(B, 1, C).float(), (dx * a.float()).sum(1), dw, dsh, dsc


def _close_bf16(got, want, name):
    """got (bf16) within one bf16 rounding of want (fp32) plus 1e-5 of want's rms: the row sum's order differs from
    torch's, so dt - t * mean may differ in its last fp32 bits where it cancels."""
    g, w = got.float(), want
    tol = w.abs() * 2.0 ** -8 + 1e-5 * w.pow(2).mean().sqrt()
    bad = ((g - w).abs() > tol).sum().item()
    assert bad == 0, f"{name}: {bad} elements out of bounds"


def _close_f32(got, want, name, rel=1e-5):
    err = ((got - want).abs().max() / want.abs().max().clamp_min(1e-30)).item()
    assert err < rel, (name, err)


@pytest.mark.parametrize("res,dxn", [(False, False), (True, True), (True, False)])
@pytest.mark.parametrize("B,N,C", [(128, 256, 1024), (4, 100, 768), (2, 64, 1792), (3, 50, 2048), (64, 128, 896),
                                   (8, 100, 1152), (3, 30, 100)])
def test_backward_kernel(dev, B, N, C, res, dxn):
    """The HIP backward (gpic_fp8_res_mod_rmsnorm_bwd) against the reference's formula in torch fp32, and twice in a
    row bit for bit (fixed summation order)."""
    from gpic_fp8 import norm as NM
    x, a, gate, w, shift, scale = inputs(B, N, C, 40 + B + C + res, dev, res)
    xn, h, _, _, rstd = G.res_mod_rmsnorm_q(x, a, gate, w, shift, scale, 1e-6, res, True, False)
    xs = xn if res else x
    g = torch.Generator(device=dev).manual_seed(41)
    dh = (torch.randn(B, N, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    dx_up = (torch.randn(B, N, C, generator=g, device=dev) * 0.1).to(torch.bfloat16) if (res and dxn) else None
    args = (dh, dx_up, xs, a if res else None, gate if res else None, w, scale, rstd)
    out = NM.res_mod_rmsnorm_bwd_k(*args)
    ref = torch_backward(*args)
    dx, da, dg, dwk, dsh, dsc = out
    _close_bf16(dx, ref[0], "dx")
    _close_f32(dwk, ref[3], "d_w")
    _close_f32(dsh, ref[4], "d_shift")
    _close_f32(dsc, ref[5], "d_scale")
    if res:
        _close_bf16(da, ref[1], "da")
        _close_f32(dg, ref[2], "d_gate")
    again = NM.res_mod_rmsnorm_bwd_k(*args)
    for u, v in zip(out, again):
        assert torch.equal(u.view(torch.int32) if u.dtype == torch.float32 else u.view(torch.int16),
                           v.view(torch.int32) if v.dtype == torch.float32 else v.view(torch.int16))


def test_backward_kernel_empty(dev):
    """No rows: dx and da are empty, every column sum is zero."""
    from gpic_fp8 import norm as NM
    x, a, gate, w, shift, scale = inputs(2, 8, 256, 42, dev, True)
    e = x[:, :0]
    dx, da, dg, dw, dsh, dsc = NM.res_mod_rmsnorm_bwd_k(e, e, e, e, gate, w, scale,
                                                      torch.empty(0, device=dev, dtype=torch.float32))
    assert dx.numel() == 0 and da.numel() == 0 and torch.equal(dw, torch.zeros_like(dw))
    assert not dg.any() and not dsh.any() and not dsc.any() and dg.shape == (2, 256)


def test_wide_rows_refuse_gradients_before_the_forward(dev):
    """Rows wider than the backward kernel takes (C > 2048): the forward runs without gradients, and asking for them
    raises before any work (not in the backward)."""
    x, a, gate, w, shift, scale = inputs(2, 8, 2560, 43, dev, True)
    with torch.no_grad():
        G.res_mod_rmsnorm(x, a, gate, w, shift, scale, 1e-6)
    with pytest.raises(ValueError, match="at most 2048"):
        G.res_mod_rmsnorm(x.requires_grad_(), a, gate, w, shift, scale, 1e-6)


# ---- a converted model takes the fused path: FlattenDiTBlock's lever-K branch (JiT_T2I.py:189-207)

import copy  # noqa: E402

import torch.nn as nn  # noqa: E402


class _RMSNorm(nn.Module):
    """rmsnorm.py's module: weight, variance_epsilon"""
    def __init__(self, d):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.variance_epsilon = 1e-6


class _Attn(nn.Module):
    """Attention's linears (qkv_x without bias, proj with, JiT_T2I.py:130,136); x is used for its shape and qkv_x only,
    as in the reference. The attention itself in fp32."""
    def __init__(self, d, heads):
        super().__init__()
        self.heads = heads
        self.qkv_x = nn.Linear(d, 3 * d, bias=False)
        self.proj = nn.Linear(d, d)

    def forward(self, x, y, pos, mask=None):
        B, N, C = x.shape
        q, k, v = self.qkv_x(x).float().view(B, N, 3, self.heads, C // self.heads).permute(2, 0, 3, 1, 4)
        a = torch.softmax(q @ k.transpose(-1, -2).contiguous() / (C // self.heads) ** 0.5, -1)
        return self.proj((a @ v).transpose(1, 2).reshape(B, N, C).to(torch.bfloat16))


class _MLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.w12 = nn.Linear(d, 2 * h, bias=False)
        self.w3 = nn.Linear(h, d, bias=False)

    def forward(self, x):
        x1, x2 = self.w12(x).chunk(2, dim=-1)
        return self.w3(torch.nn.functional.silu(x1) * x2)


class _LeverKBlock(nn.Module):
    """FlattenDiTBlock's modules; forward = its lever-K branch (JiT_T2I.py:201-207) over the drop-in norm API."""
    def __init__(self, d, heads):
        super().__init__()
        self.norm1 = _RMSNorm(d)
        self.attn = _Attn(d, heads)
        self.norm2 = _RMSNorm(d)
        self.mlp = _MLP(d, 4 * d)
        self.adaLN_modulation = nn.Sequential(nn.Linear(d, 6 * d, bias=True))

    def forward(self, x, y, c, pos, mask=None):
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaLN_modulation(c).chunk(6, dim=-1)
        h = G.mod_rmsnorm(x, self.norm1.weight, shift_msa, scale_msa, self.norm1.variance_epsilon)
        x, h = G.res_mod_rmsnorm(x, self.attn(h, y, pos, mask), gate_msa, self.norm2.weight, shift_mlp, scale_mlp,
                                 self.norm2.variance_epsilon)
        return x + gate_mlp * self.mlp(h)


class _LeverKNet(nn.Module):
    def __init__(self, d, heads, n):
        super().__init__()
        self.blocks = nn.ModuleList(_LeverKBlock(d, heads) for _ in range(n))

    def forward(self, x, c):
        for b in self.blocks:
            x = b(x, None, c, None)
        return x


@pytest.mark.parametrize("C", [896, 1024])
def test_converted_block_takes_the_fused_path(dev, C, monkeypatch):
    """convert_fp8(net, "native3+norm") against "native3" on the same weights (the blocks' lever-K branch over
    mod_rmsnorm / res_mod_rmsnorm and the phase-3 linears): the output and every gradient bit for bit, while the
    converted model never writes a bf16 h (every call of the norm op casts in the producer). C = 896 is the d11
    width (rows of 3.5 groups of 256)."""
    from gpic_fp8 import norm as NM
    torch.manual_seed(5)
    B, N = 4, 256
    net_u = _LeverKNet(C, 8, 2).to(dev).to(torch.bfloat16)
    for b in net_u.blocks:   # non-trivial norm weights and modulation
        with torch.no_grad():
            b.norm1.weight.add_(0.1 * torch.randn_like(b.norm1.weight))
            b.norm2.weight.add_(0.1 * torch.randn_like(b.norm2.weight))
            b.adaLN_modulation[0].weight.mul_(5.0)
    net_f = copy.deepcopy(net_u)
    assert G.convert_fp8(net_u, "native3") == 8 and G.convert_fp8(net_f, "native3+norm") == 8
    assert all(type(b.attn.qkv_x) is G.Fp8NormLinearF8 for b in net_f.blocks)
    x = torch.randn(B, N, C, device=dev).to(torch.bfloat16)
    c = torch.randn(B, 1, C, device=dev).to(torch.bfloat16)
    dy = (torch.randn(B, N, C, device=dev) * 0.1).to(torch.bfloat16)
    calls = []
    real = NM.res_mod_rmsnorm_q

    def spy(*args, **kw):
        calls.append(args[8] if len(args) > 8 else kw.get("want_h"))
        return real(*args, **kw)
    outs = []
    for net in (net_f, net_u):
        monkeypatch.setattr(NM, "res_mod_rmsnorm_q", spy)
        calls.clear()
        xl, cl = x.clone().requires_grad_(), c.clone().requires_grad_()
        y = net(xl, cl)
        y.backward(dy)
        outs.append([y, xl.grad, cl.grad] + [p.grad for p in net.parameters()])
        if net is net_f:
            assert calls == [False] * 4, calls       # two sites x two blocks, all casting in the norm
        else:
            assert calls == [True] * 4, calls        # the reference's ops: bf16 h, then the linears cast it
        monkeypatch.undo()
    for got, want in zip(*outs):
        assert got is not None and want is not None
        assert torch.equal(got.view(torch.int16) if got.dtype == torch.bfloat16 else got,
                           want.view(torch.int16) if want.dtype == torch.bfloat16 else want)
