"""The image blocks' two norm sites with the FP8 cast of their output folded into the producer (the activation amax
taken where h is made): baselines/PixelGen/src/models/layers/fused_norm.py (the reference's MFU lever K) on the HIP
kernels of nano-gpic_amd/csrc/norm.hip.

    site 1 (norm1):  h = RMSNorm(x) * (1 + scale) + shift                                   mod_rmsnorm
    site 2 (norm2):  x_new = x + gate * a;  h = RMSNorm(x_new) * (1 + scale) + shift        res_mod_rmsnorm

The reference computes h in bf16 and its FP8 linear then reads h again for the amax and the cast
(fp8_native.py:3-6 names these separate passes as why FP8 lost end to end). Here one kernel writes h's tensorwise
e4m3 bytes and scale directly, and h itself only when asked. Functions:

- mod_rmsnorm / res_mod_rmsnorm / reference: the reference's API (fused_norm.py:293-313) with bf16 h, on the kernel,
  and its ops under their names and schemas: gpic::res_mod_rmsnorm_fwd (differentiable) and gpic::res_mod_rmsnorm_bwd;
- fp8_mod_rmsnorm_linear(x, w_norm, shift, scale, eps, weight, bias): site 1 feeding a phase-3 FP8 linear (qkv_x);
- fp8_res_mod_rmsnorm_mlp(x, a, gate, w_norm, shift, scale, eps, w12, w3): site 2 feeding the phase-3 FP8 SwiGLU MLP,
  returning (x_new, mlp output);
- convert_fused_norm(net) (convert_native(..., fused_norm=True), recipes "native3+norm", "native3+text+norm"): the
  image blocks' forward routed through the two fused consumers, so a converted model takes the fused path.

The backward of the norm is the reference's analytic one (fused_norm.py:94-147) on a HIP kernel
(res_mod_rmsnorm_bwd_k); the linears' backward is phase 3's (FP8 dgrad and wgrad), the wgrad reading h's e4m3 bytes
kept from the forward.
"""
import types
from typing import Optional

import torch

from . import _lib as L
from .fp8_native import (E4, Fp8LinearF8, fp8_gemm, fp8_gemm_mn, fp8_linear_f8, swiglu_bwd_q, swiglu_tcast, tcast,
                         tcast_t)


# The widest rows the backward kernel takes (its per-column sums live in registers); the forward takes any width.
BWD_MAX_C = 2048


def _check_bwd_width(C, ctx):
    """Raises in an autograd Function's forward, before its work, when a gradient will be asked of a norm wider than
    the backward takes (ctx.needs_input_grad: which inputs the graph wants gradients of)."""
    if C > BWD_MAX_C and any(ctx.needs_input_grad):
        raise ValueError(f"the norm's backward kernel takes rows of at most {BWD_MAX_C} elements, got C = {C}; "
                         "run the forward under torch.no_grad() or with inputs that need no gradient")


def _vec(t, B, C):
    """A [B, 1, C] modulation chunk (a view of the adaLN output) as a [B, C] view with unit column stride, a row
    stride that is a multiple of 4 and an 8-byte aligned start, without a copy where it already is one."""
    t = t.reshape(B, C)
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 8:
        t = L.aligned(t.contiguous())
    return t


@L.custom_op("gpic::fp8_res_mod_rmsnorm")
def res_mod_rmsnorm_q(x: torch.Tensor, a: torch.Tensor, gate: torch.Tensor, w: torch.Tensor, shift: torch.Tensor,
                      scale: torch.Tensor, eps: float, has_res: bool, want_h: bool, want_q: bool = True
                      ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """x [B, N, C] bf16 (C % 4 == 0), a [B, N, C] bf16 (has_res), gate / shift / scale [B, 1, C], w [C] ->
    (x_new [B, N, C] bf16 or an empty tensor, h [B, N, C] bf16 or an empty tensor (want_h), h's e4m3 bytes [B, N, C]
    and their dequantization scale [1] fp32 (empty tensors unless want_q), rstd [B * N] fp32). want_q=False is the
    norm alone (the reference's op)."""
    L.require_gpu(x, a, gate, w, shift, scale)
    if not (want_h or want_q):
        raise ValueError("res_mod_rmsnorm_q needs want_h or want_q")
    if x.dim() != 3 or x.dtype != torch.bfloat16 or x.shape[2] % 4 or x.shape[2] == 0:
        raise ValueError(f"the norm kernel takes bf16 x [B, N, C] with C % 4 == 0, got {x.dtype} {tuple(x.shape)}")
    B, N, C = x.shape
    xc = L.aligned(x.contiguous())
    ac = L.aligned(a.to(torch.bfloat16).contiguous()) if has_res else None
    if has_res and ac.shape != x.shape:
        raise ValueError(f"a must be [B, N, C] like x, got {tuple(a.shape)}")
    g = _vec(gate, B, C) if has_res else None
    sh, sc = _vec(shift, B, C), _vec(scale, B, C)
    wf = L.aligned(w.to(torch.float32).contiguous())
    dev = x.device
    xn = torch.empty_like(xc) if has_res else x.new_empty(0)
    h = torch.empty_like(xc) if want_h else x.new_empty(0)
    hq = torch.empty((B, N, C) if want_q else (0,), dtype=E4, device=dev)
    s = torch.empty(1 if want_q else 0, dtype=torch.float32, device=dev)
    rstd = torch.empty(B * N, dtype=torch.float32, device=dev)
    with L.on_device(dev):
        ws = L.cast_workspace(dev)
        L.check(L.lib().gpic_fp8_res_mod_rmsnorm(
            xc.data_ptr(), L.ptr(ac), L.ptr(g), g.stride(0) if has_res else 0, wf.data_ptr(), sh.data_ptr(),
            sh.stride(0), sc.data_ptr(), sc.stride(0), B * N, max(N, 1), C, float(eps), xn.data_ptr() if has_res else None,
            h.data_ptr() if want_h else None, rstd.data_ptr(), hq.data_ptr() if want_q else None,
            s.data_ptr() if want_q else None, ws.data_ptr(),
            L.stream_ptr(dev)), "gpic_fp8_res_mod_rmsnorm")
    return xn, h, hq, s, rstd


@res_mod_rmsnorm_q.register_fake
def _(x, a, gate, w, shift, scale, eps, has_res, want_h, want_q=True):
    B, N, C = x.shape
    return (torch.empty_like(x) if has_res else x.new_empty(0), torch.empty_like(x) if want_h else x.new_empty(0),
            x.new_empty((B, N, C) if want_q else (0,), dtype=E4), x.new_empty(1 if want_q else 0, dtype=torch.float32),
            x.new_empty(B * N, dtype=torch.float32))


@L.custom_op("gpic::fp8_res_mod_rmsnorm_bwd")
def res_mod_rmsnorm_bwd_k(dh: torch.Tensor, dxn: Optional[torch.Tensor], xs: torch.Tensor, a: Optional[torch.Tensor],
                          gate: Optional[torch.Tensor], w: torch.Tensor, scale: torch.Tensor, rstd: torch.Tensor
                          ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The norm site's backward (fused_norm.py:94-147, op :249-275) on the HIP kernel: dh [B, N, C] (the gradient of
    h), dxn (that of x_new, site 2) or None, xs = x_new (site 2) or x, a and gate (site 2) or None, rstd [B * N].
    Returns dx, da (empty at site 1), d_gate [B, C] (empty at site 1), d_w [C], d_shift [B, C], d_scale [B, C]: fp32
    column sums taken in a fixed order."""
    L.require_gpu(dh, xs, w, scale, rstd)
    B, N, C = xs.shape
    res = a is not None
    dhc = L.aligned(dh.to(torch.bfloat16).contiguous())
    xsc = L.aligned(xs.contiguous())
    dxc = L.aligned(dxn.to(torch.bfloat16).contiguous()) if (res and dxn is not None) else None
    ac = L.aligned(a.to(torch.bfloat16).contiguous()) if res else None
    g = _vec(gate, B, C) if res else None
    sc = _vec(scale, B, C)
    wf = L.aligned(w.to(torch.float32).contiguous())
    dev = xs.device
    dx = torch.empty_like(xsc)
    da = torch.empty_like(xsc) if res else xs.new_empty(0)
    f32 = dict(dtype=torch.float32, device=dev)
    if B * N == 0:   # no rows: every column sum is zero
        z = torch.zeros(B, C, **f32)
        return dx, da, (z.clone() if res else torch.empty(0, **f32)), torch.zeros(C, **f32), z.clone(), z.clone()
    dg = torch.empty(B, C, **f32) if res else torch.empty(0, **f32)
    dw, dsh, dsc = torch.empty(C, **f32), torch.empty(B, C, **f32), torch.empty(B, C, **f32)
    with L.on_device(dev):
        nws = L.lib().gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes(B * N, max(N, 1), C)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=dev)
        L.check(L.lib().gpic_fp8_res_mod_rmsnorm_bwd(
            dhc.data_ptr(), L.ptr(dxc), xsc.data_ptr(), L.ptr(ac), L.ptr(g), g.stride(0) if res else 0, wf.data_ptr(),
            sc.data_ptr(), sc.stride(0), rstd.data_ptr(), B * N, max(N, 1), C, dx.data_ptr(),
            da.data_ptr() if res else None, dsh.data_ptr(), dsc.data_ptr(), dg.data_ptr() if res else None,
            dw.data_ptr(), ws.data_ptr(), nws, L.stream_ptr(dev)), "gpic_fp8_res_mod_rmsnorm_bwd")
    return dx, da, dg, dw, dsh, dsc


@res_mod_rmsnorm_bwd_k.register_fake
def _(dh, dxn, xs, a, gate, w, scale, rstd):
    B, N, C = xs.shape
    res = a is not None
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(xs), torch.empty_like(xs) if res else xs.new_empty(0),
            xs.new_empty((B, C) if res else (0,), **f32), xs.new_empty(C, **f32), xs.new_empty(B, C, **f32),
            xs.new_empty(B, C, **f32))


def _norm_backward(dh, dxn, xs, a, gate, w, scale, rstd):
    """The norm site's backward: (dx, da or None, d_gate or None, d_w, d_shift, d_scale), the column sums fp32."""
    dx, da, dg, dw, dsh, dsc = L.call(res_mod_rmsnorm_bwd_k, dh, dxn if a is not None else None, xs, a, gate, w,
                                      scale, rstd)
    if a is None:
        return dx, None, None, dw, dsh, dsc
    return dx, da, dg, dw, dsh, dsc


def _param_grads(B, C, dg, dw, dsh, dsc, gate, w, shift, scale):
    vec = lambda v, like: None if v is None else v.to(like.dtype).view(B, 1, C).reshape(like.shape)
    return vec(dg, gate) if gate is not None else None, dw.to(w.dtype), vec(dsh, shift), vec(dsc, scale)


# ------------------------------------------------------------------ the reference's op names and schemas

@L.custom_op("gpic::res_mod_rmsnorm_fwd")
def res_mod_rmsnorm_fwd(x: torch.Tensor, a: torch.Tensor, gate: torch.Tensor, w: torch.Tensor, shift: torch.Tensor,
                        scale: torch.Tensor, eps: float, has_res: bool
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The reference's op (fused_norm.py:151-171) on the HIP kernel: (x_new, or an empty tensor without the residual;
    h [B, N, C] bf16; rstd [B * N] fp32). Differentiable (its backward is res_mod_rmsnorm_bwd, as the reference
    registers it, :224-245). mod_rmsnorm / res_mod_rmsnorm below take the autograd Function instead, which refuses a
    gradient at C > 2048 before the forward runs."""
    xn, h, _, _, rstd = L.call(res_mod_rmsnorm_q, x, a, gate, w, shift, scale, eps, has_res, True, False)
    return xn, h, rstd


@res_mod_rmsnorm_fwd.register_fake
def _(x, a, gate, w, shift, scale, eps, has_res):
    B, N, C = x.shape
    return (torch.empty_like(x) if has_res else x.new_empty(0), torch.empty_like(x),
            x.new_empty(B * N, dtype=torch.float32))


@L.custom_op("gpic::res_mod_rmsnorm_bwd")
def res_mod_rmsnorm_bwd(dh: torch.Tensor, dxn: torch.Tensor, xn: torch.Tensor, a: torch.Tensor, gate: torch.Tensor,
                        w: torch.Tensor, scale: torch.Tensor, rstd: torch.Tensor, has_res: bool, has_dxn: bool
                        ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The reference's op (fused_norm.py:180-212) on the HIP kernel, with its argument meaning: xn is x_new (has_res)
    or x; a, gate (and dxn unless has_dxn) are ignored without the residual. Returns dx, da, d_gate [B, C], d_w [C],
    d_shift [B, C], d_scale [B, C] (fp32 column sums; da and d_gate empty without the residual)."""
    dx, da, dg, dw, dsh, dsc = L.call(res_mod_rmsnorm_bwd_k, dh, dxn if (has_res and has_dxn) else None, xn,
                                      a if has_res else None, gate if has_res else None, w, scale, rstd)
    return dx, da, dg, dw, dsh, dsc


@res_mod_rmsnorm_bwd.register_fake
def _(dh, dxn, xn, a, gate, w, scale, rstd, has_res, has_dxn):
    B, N, C = xn.shape
    f32 = dict(dtype=torch.float32)
    return (torch.empty_like(xn), torch.empty_like(xn) if has_res else xn.new_empty(0),
            xn.new_empty((B, C) if has_res else (0,), **f32), xn.new_empty(C, **f32), xn.new_empty(B, C, **f32),
            xn.new_empty(B, C, **f32))


def _fwd_setup(ctx, inputs, output):
    x, a, gate, w, shift, scale, eps, has_res = inputs
    xn, h, rstd = output
    ctx.has_res = has_res
    ctx.save_for_backward(xn if has_res else x, a if has_res else None, gate if has_res else None, w, shift, scale,
                          rstd)


def _fwd_backward(ctx, dxn, dh, drstd):
    xs, a, gate, w, shift, scale, rstd = ctx.saved_tensors
    B, _, C = xs.shape
    if C > BWD_MAX_C:
        raise ValueError(f"the norm's backward kernel takes rows of at most {BWD_MAX_C} elements, got C = {C}")
    has_dxn = ctx.has_res and dxn is not None
    dx, da, dg, dw, dsh, dsc = L.call(res_mod_rmsnorm_bwd, dh, dxn if has_dxn else dh, xs, a if ctx.has_res else xs,
                                      gate if ctx.has_res else w, w, scale, rstd, ctx.has_res, has_dxn)
    dgate, dw, dshift, dscale = _param_grads(B, C, dg if ctx.has_res else None, dw, dsh, dsc, gate, w, shift, scale)
    return (dx, da if ctx.has_res else None, dgate, dw, dshift, dscale, None, None)


res_mod_rmsnorm_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup)


class _ResModRMSNorm(torch.autograd.Function):
    """The reference's res_mod_rmsnorm_fwd with bf16 h (fused_norm.py:150-175, 245-287) on the HIP kernel."""
    @staticmethod
    def forward(ctx, x, a, gate, w, shift, scale, eps, has_res):
        _check_bwd_width(x.shape[-1], ctx)
        xn, h, _, _, rstd = L.call(res_mod_rmsnorm_q, x, a, gate, w, shift, scale, eps, has_res, True, False)
        ctx.has_res = has_res
        ctx.save_for_backward(xn if has_res else x, a if has_res else None, gate if has_res else None, w, shift, scale,
                              rstd)
        return (xn if has_res else x.new_empty(0)), h

    @staticmethod
    def backward(ctx, dxn, dh):
        xs, a, gate, w, shift, scale, rstd = ctx.saved_tensors
        B, _, C = xs.shape
        dx, da, dg, dw, dsh, dsc = _norm_backward(dh, dxn if ctx.has_res else None, xs, a, gate, w, scale, rstd)
        dgate, dw, dshift, dscale = _param_grads(B, C, dg, dw, dsh, dsc, gate, w, shift, scale)
        return dx, da, dgate, dw, dshift, dscale, None, None


def mod_rmsnorm(x, w, shift, scale, eps):
    """h = RMSNorm(x) * (1 + scale) + shift; x [B, N, C], w [C], shift and scale [B, 1, C] (fused_norm.py:293-295)."""
    return _ResModRMSNorm.apply(x, x, x, w, shift, scale, eps, False)[1]


def res_mod_rmsnorm(x, a, gate, w, shift, scale, eps):
    """x_new = x + gate * a; h = RMSNorm(x_new) * (1 + scale) + shift. Returns (x_new, h) (fused_norm.py:298-302)."""
    return _ResModRMSNorm.apply(x, a, gate, w, shift, scale, eps, True)


def reference(x, a, gate, w, shift, scale, eps, has_res):
    """The model's own ops in eager mode (fused_norm.py:305-313), for tests: returns (x_new or x, h)."""
    if has_res:
        x = x + gate * a
    hs = x.to(torch.float32)
    var = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(var + eps)
    n = (w * hs).to(x.dtype)
    return x, n * (1 + scale) + shift


class _Fp8ModRMSNormLinear(torch.autograd.Function):
    """Site 1 feeding a phase-3 FP8 linear: the norm kernel casts h to e4m3 (h is never written in bf16), the GEMM
    reads those bytes; backward: FP8 dgrad (dh) and wgrad (from h's bytes), then the norm's backward."""
    @staticmethod
    def forward(ctx, x, w_norm, shift, scale, eps, weight, bias):
        B, N, C = x.shape
        _check_bwd_width(C, ctx)
        _, _, hq, sh, rstd = L.call(res_mod_rmsnorm_q, x, x, x, w_norm, shift, scale, eps, False, False)
        hq2 = hq.view(B * N, C)
        wq, wqt, sw = L.call(tcast_t, weight)
        y = L.call(fp8_gemm, hq2, sh, wq, sw, None if bias is None else bias.to(torch.bfloat16))
        ctx.save_for_backward(x, w_norm, shift, scale, rstd, hq2, sh, wqt, sw)
        ctx.has_b, ctx.wdt = bias is not None, weight.dtype
        return y.view(B, N, weight.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x, w_norm, shift, scale, rstd, hq2, sh, wqt, sw = ctx.saved_tensors
        B, N, C = x.shape
        dy2 = dy.reshape(B * N, -1).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        dh = L.call(fp8_gemm, dyq, sdy, wqt, sw, None, False).view(B, N, C)
        dweight = L.call(fp8_gemm_mn, dyq, sdy, hq2, sh).to(ctx.wdt)
        db = dy2.sum(0).to(ctx.wdt) if ctx.has_b else None
        dx, _, _, dw, dsh, dsc = _norm_backward(dh, None, x, None, None, w_norm, scale, rstd)
        _, dw, dshift, dscale = _param_grads(B, C, None, dw, dsh, dsc, None, w_norm, shift, scale)
        return dx, dw, dshift, dscale, None, dweight, db


class _Fp8ResModRMSNormMLP(torch.autograd.Function):
    """Site 2 feeding the phase-3 FP8 SwiGLU MLP: x_new = x + gate * a and h's e4m3 bytes from one kernel, then
    w12, the SwiGLU product cast and w3 as _Fp8MLPF8; returns (x_new, y). Backward: the MLP's (FP8 dgrads and
    wgrads, w12's wgrad from h's bytes), then the norm's with the upstream gradient of x_new."""
    @staticmethod
    def forward(ctx, x, a, gate, w_norm, shift, scale, eps, w12, w3):
        B, N, C = x.shape
        _check_bwd_width(C, ctx)
        xn, _, hq, sh, rstd = L.call(res_mod_rmsnorm_q, x, a, gate, w_norm, shift, scale, eps, True, False)
        hq2 = hq.view(B * N, C)
        w12q, w12qt, s12 = L.call(tcast_t, w12)
        z = L.call(fp8_gemm, hq2, sh, w12q, s12)
        aq, sa = L.call(swiglu_tcast, z)
        w3q, w3qt, s3 = L.call(tcast_t, w3)
        y = L.call(fp8_gemm, aq, sa, w3q, s3)
        ctx.save_for_backward(xn, a, gate, w_norm, shift, scale, rstd, hq2, sh, z, aq, sa, w12qt, s12, w3qt, s3)
        ctx.dt = (w12.dtype, w3.dtype)
        return xn, y.view(B, N, w3.shape[0])

    @staticmethod
    def backward(ctx, dxn, dy):
        xn, a, gate, w_norm, shift, scale, rstd, hq2, sh, z, aq, sa, w12qt, s12, w3qt, s3 = ctx.saved_tensors
        B, N, C = xn.shape
        dy2 = dy.reshape(B * N, -1).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        da_ = L.call(fp8_gemm, dyq, sdy, w3qt, s3, None, False)
        dw3 = L.call(fp8_gemm_mn, dyq, sdy, aq, sa)
        dzq, sdz = L.call(swiglu_bwd_q, z, da_)
        dh = L.call(fp8_gemm, dzq, sdz, w12qt, s12, None, False).view(B, N, C)
        dw12 = L.call(fp8_gemm_mn, dzq, sdz, hq2, sh)
        dx, da, dg, dw, dsh, dsc = _norm_backward(dh, dxn, xn, a, gate, w_norm, scale, rstd)
        dgate, dw, dshift, dscale = _param_grads(B, C, dg, dw, dsh, dsc, gate, w_norm, shift, scale)
        return dx, da, dgate, dw, dshift, dscale, None, dw12.to(ctx.dt[0]), dw3.to(ctx.dt[1])


def fp8_mod_rmsnorm_linear(x, w_norm, shift, scale, eps, weight, bias: Optional[torch.Tensor] = None):
    """linear(mod_rmsnorm(x, w_norm, shift, scale, eps)) with every GEMM in FP8 and the cast of h in the norm."""
    with torch.autocast("cuda", enabled=False):
        return _Fp8ModRMSNormLinear.apply(x.to(torch.bfloat16), w_norm, shift, scale, eps, weight, bias)


def fp8_res_mod_rmsnorm_mlp(x, a, gate, w_norm, shift, scale, eps, w12, w3):
    """(x_new, mlp(h)) for x_new, h = res_mod_rmsnorm(x, a, gate, w_norm, shift, scale, eps), the SwiGLU MLP in FP8
    (every GEMM) and the cast of h in the norm."""
    with torch.autocast("cuda", enabled=False):
        return _Fp8ResModRMSNormMLP.apply(x.to(torch.bfloat16), a.to(torch.bfloat16), gate, w_norm, shift, scale, eps,
                                          w12, w3)


# ------------------------------------------------------------------------------------------------ converter

class Fp8NormLinearF8(Fp8LinearF8):
    """The qkv_x of an image block converted with fused_norm: an Fp8LinearF8 (the same parameters and state-dict keys)
    that, when its block's forward has handed it the pending site-1 norm, takes the norm's e4m3 output directly
    (fp8_mod_rmsnorm_linear: h is never written in bf16) instead of a bf16 h. The block passes the attention a
    placeholder on the meta device in place of h; the attention reads only its shape and hands it to qkv_x
    (JiT_T2I.py:138-185), so any other use of it fails loudly. Called without a pending norm it is an Fp8LinearF8."""
    def forward(self, x):
        pend = self.__dict__.pop("_gpic_norm", None)
        if pend is None:
            return fp8_linear_f8(x, self.weight, self.bias)
        marker, xs, w_norm, shift, scale, eps = pend
        if x is not marker:
            raise RuntimeError("qkv_x was handed a pending norm but called on another tensor")
        return fp8_mod_rmsnorm_linear(xs, w_norm, shift, scale, eps, self.weight, self.bias)


def _norm_eps(norm):
    return getattr(norm, "variance_epsilon", getattr(norm, "eps", 1e-6))


def fused_norm_ok(blk):
    """An image block with the structure of FlattenDiTBlock (JiT_T2I.py:189-210) whose norm sites the fused path can
    take: norm1 / norm2 RMSNorms of width C (C % 4 == 0, C <= BWD_MAX_C), adaLN_modulation, attn.qkv_x and the SwiGLU
    MLP's w12 / w3 (no biases) already converted to phase 3."""
    n1, n2 = getattr(blk, "norm1", None), getattr(blk, "norm2", None)
    attn, mlp = getattr(blk, "attn", None), getattr(blk, "mlp", None)
    if n1 is None or n2 is None or attn is None or mlp is None or not hasattr(blk, "adaLN_modulation"):
        return False
    qkv = getattr(attn, "qkv_x", None)
    C = n1.weight.numel() if isinstance(getattr(n1, "weight", None), torch.Tensor) else 0
    return (isinstance(qkv, Fp8LinearF8) and getattr(mlp, "_fp8", False) and mlp.w12.bias is None and
            mlp.w3.bias is None and isinstance(getattr(n2, "weight", None), torch.Tensor) and
            n2.weight.numel() == C and C > 0 and C % 4 == 0 and C <= BWD_MAX_C and qkv.in_features == C)


def _fused_block_forward(blk, x, y, c, pos, mask=None):
    """FlattenDiTBlock.forward's lever-K branch (JiT_T2I.py:201-207) with each norm site's output cast in the norm:
    site 1 hands qkv_x h's e4m3 bytes (through Fp8NormLinearF8), site 2 and the MLP run as fp8_res_mod_rmsnorm_mlp.
    The same operations, in the same order, as that branch over mod_rmsnorm / res_mod_rmsnorm and the phase-3
    linears, so the outputs and gradients are the same bits; h is never written in bf16. Bound to the block as its
    forward (a method, so that a deep copy of the model, e.g. an EMA copy, runs its own modules)."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = blk.adaLN_modulation(c).chunk(6, dim=-1)
    qkv = blk.attn.qkv_x
    marker = torch.empty(x.shape, dtype=torch.bfloat16, device="meta")
    qkv._gpic_norm = (marker, x, blk.norm1.weight, shift_msa, scale_msa, _norm_eps(blk.norm1))
    try:
        a = blk.attn(marker, y, pos, mask)
    finally:
        qkv.__dict__.pop("_gpic_norm", None)
    x, out = fp8_res_mod_rmsnorm_mlp(x, a, gate_msa, blk.norm2.weight, shift_mlp, scale_mlp, _norm_eps(blk.norm2),
                                     blk.mlp.w12.weight, blk.mlp.w3.weight)
    return x + gate_mlp * out


def convert_fused_norm(net):
    """Route each phase-3 image block's norm sites through the producer-fused kernels (after convert_native(phase=3)):
    the block's forward becomes its lever-K branch with h's cast folded into the norm, and its qkv_x an
    Fp8NormLinearF8. Parameters and state-dict keys are unchanged. Returns the number of blocks rewired."""
    n = 0
    for blk in getattr(net, "blocks", []):
        if not fused_norm_ok(blk) or getattr(blk, "_gpic_fused_norm", False):
            continue
        blk.attn.qkv_x.__class__ = Fp8NormLinearF8
        blk.forward = types.MethodType(_fused_block_forward, blk)
        blk._gpic_fused_norm = True
        n += 1
    return n
