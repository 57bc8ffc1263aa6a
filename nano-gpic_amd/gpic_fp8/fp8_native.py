"""Native FP8 linear path for MI355X (gfx950): the module / autograd API of nano-gpic's
baselines/PixelGen/src/models/layers/fp8_native.py, over hand-written HIP kernels (libgpic_fp8.so, C ABI in
include/gpic_fp8.h) instead of Triton kernels and torch._scaled_mm.

Numerics (the reference's rules, fp8_native.py:24-49):
- tensorwise scaling with the current amax (no state across steps): amax = max |x| over the non-NaN elements,
  a = max(amax, 1e-12), scale = 448 / a and dequant = a / 448, both IEEE-rounded fp32 divisions;
- q = e4m3fn(min(max(x * scale, -448), 448)), round to nearest even: bit-exact with the reference's cast;
- the GEMM C = bf16(sa * sb * sum_k A q_k B q_k) with fp32 accumulation (MFMA), the optional bias added afterwards in
  bf16 (fp8_native.py:189-190), fused into the GEMM epilogue with the same two roundings;
- the SwiGLU roundings of fp8_native.py:55-58 and 88-94, with this build's sigmoid (see the C header).

Phases (convert_native / convert_fp8 recipes):
- phase 1 ("native"): forward GEMMs in FP8, backward in bf16 -- as the reference;
- phase 2 ("native2"): the MLP as one function with FP8 dgrads, bf16 wgrads -- as the reference;
- phase 3 ("native3", an extension): every forward, dgrad and wgrad GEMM of qkv_x, proj, w12 and w3 in FP8. The
  forward keeps the e4m3 bytes of its inputs for the wgrad instead of the bf16 inputs; the wgrad GEMM reads them and
  the output gradient's bytes as they are (fp8_gemm_mn: K, the token index, is their row index), so the activations
  and gradients are cast flat, with no transposed copies.
"""
from typing import Optional

import ctypes

import torch

from . import _lib as L

E4 = torch.float8_e4m3fn
FMAX = 448.0          # the largest finite e4m3fn value
TINY = 1e-12          # an all-zero tensor keeps scale FMAX / TINY: its values stay 0


def _r16(n):
    return (n + 15) // 16 * 16


def _prep(x):
    """x as a contiguous, 16-byte aligned bf16 or fp32 tensor (other float dtypes are widened to fp32 exactly as the
    reference's in-kernel .to(tl.float32) does)."""
    if x.dtype not in L.DTYPE_CODE:
        x = x.float()
    return L.aligned(x.contiguous())


def _prep_rows(t, min_cols):
    """A 2-D tensor whose rows are unit-stride, 16-byte aligned and with a row stride that is a multiple of 8 elements;
    else a contiguous aligned copy."""
    if t.stride(-1) != 1 or t.stride(0) % 8 != 0 or t.stride(0) < min_cols or t.data_ptr() % 16 != 0:
        t = L.aligned(t.contiguous())
    return t


# ------------------------------------------------------------------------------------------------ casts

@L.custom_op("gpic::fp8_tcast")
def tcast(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x (any float dtype) -> e4m3 (contiguous, x's shape) and its tensorwise dequantization scale amax / 448 [1] fp32.
    (fp8_native.py:114-122)"""
    L.require_gpu(x)
    xc = _prep(x)
    q = torch.empty(x.shape, dtype=E4, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    with L.on_device(x.device):
        ws = L.cast_workspace(x.device)
        L.check(L.lib().gpic_fp8_tcast(xc.data_ptr(), L.DTYPE_CODE[xc.dtype], xc.numel(), q.data_ptr(), s.data_ptr(),
                                       ws.data_ptr(), L.stream_ptr(x.device)), "gpic_fp8_tcast")
    return q, s


@tcast.register_fake
def _(x):
    return x.new_empty(x.shape, dtype=E4), x.new_empty(1, dtype=torch.float32)


@L.custom_op("gpic::fp8_tcast_t")
def tcast_t(x: torch.Tensor, want_q: bool = True) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """x [R, C] (any float dtype, C % 16 == 0) -> (q [R, C] e4m3, or an empty tensor when want_q is False;
    qt [C, R16] e4m3 = q transposed, R16 = R rounded up to 16, zero bytes in columns R..R16-1; dequant [1] fp32).
    The same bytes and scale as tcast(x) (and as the reference's tcast(x.t().contiguous()), fp8_native.py:259)."""
    L.require_gpu(x)
    if x.dim() != 2 or x.shape[1] % 16:
        raise ValueError(f"tcast_t needs a 2-D tensor with a multiple of 16 columns, got {tuple(x.shape)}")
    xc = _prep(x)
    R, C = xc.shape
    q = torch.empty((R, C) if want_q else (0,), dtype=E4, device=x.device)
    qt = torch.empty(C, _r16(R), dtype=E4, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    with L.on_device(x.device):
        ws = L.cast_workspace(x.device)
        L.check(L.lib().gpic_fp8_tcast_t(xc.data_ptr(), L.DTYPE_CODE[xc.dtype], R, C, q.data_ptr() if want_q else None,
                                         qt.data_ptr(), qt.shape[1], s.data_ptr(), ws.data_ptr(),
                                         L.stream_ptr(x.device)), "gpic_fp8_tcast_t")
    return q, qt, s


@tcast_t.register_fake
def _(x, want_q=True):
    R, C = x.shape
    return (x.new_empty((R, C) if want_q else (0,), dtype=E4), x.new_empty(C, _r16(R), dtype=E4),
            x.new_empty(1, dtype=torch.float32))


@L.custom_op("gpic::fp8_tcast_heads")
def tcast_heads(o: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """The attention output o [B, H, N, D] (D % 16 == 0) -> (q [B, N, H D] e4m3, dequant [1] fp32): the bytes and scale
    tcast(o.transpose(1, 2).reshape(B, N, H D)) gives -- proj's input at JiT_T2I.py:183-185 -- read from o in its own
    layout (either of those scaled_dot_product_attention's backends write: [B, H, N, D] or [B, N, H, D] in memory), so
    the head-merging copy is never made. An extension of the reference, which casts the copy (fp8_native.py:3-6,
    114-122). A bf16 o whose rows are not 16-byte aligned is made contiguous first; another dtype takes that copy and
    tcast."""
    L.require_gpu(o)
    if o.dim() != 4 or o.shape[3] % 16:
        raise ValueError(f"tcast_heads needs o [B, H, N, D] with D % 16 == 0, got {tuple(o.shape)}")
    B, H, N, D = o.shape
    if o.dtype != torch.bfloat16:
        return L.call(tcast, o.transpose(1, 2).reshape(B, N, H * D))
    # a dimension of extent 1 takes stride 0 (its stride never multiplies a nonzero index)
    st = [0 if e == 1 else s for e, s in zip(o.shape, o.stride())]
    if (o.numel() and (st[3] not in (0, 1) or any(s % 8 or s < 0 for s in st[:3]) or o.data_ptr() % 16)):
        o = L.aligned(o.contiguous())
        st = [0 if e == 1 else s for e, s in zip(o.shape, o.stride())]
    q = torch.empty(B, N, H * D, dtype=E4, device=o.device)
    s = torch.empty(1, dtype=torch.float32, device=o.device)
    with L.on_device(o.device):
        ws = L.cast_workspace(o.device)
        L.check(L.lib().gpic_fp8_tcast_heads(o.data_ptr() if o.numel() else None, B, H, N, D, st[0], st[1], st[2],
                                             q.data_ptr() if o.numel() else None, s.data_ptr(), ws.data_ptr(),
                                             L.stream_ptr(o.device)), "gpic_fp8_tcast_heads")
    return q, s


@tcast_heads.register_fake
def _(o):
    B, H, N, D = o.shape
    return o.new_empty(B, N, H * D, dtype=E4), o.new_empty(1, dtype=torch.float32)


@L.custom_op("gpic::fp8_tcast_t_group")
def tcast_t_group(xs: list[torch.Tensor]) -> list[torch.Tensor]:
    """tcast_t of each 2-D tensor in xs, in one call: [q0, qt0, s0, q1, qt1, s1, ...], the same bytes and scales as
    tcast_t(x) for each x. bf16 tensors that fit the device together (a d12 block's four weights) are cast in one
    launch (gpic_fp8_tcast_t_group), each with its own amax. An extension of the reference, whose linears cast their
    weights one at a time inside each forward (fp8_native.py:187,245,248): the weight casts of a block, done together
    before it runs, for fp8_linear_f8(..., wcast=) and fp8_mlp_f8(..., w12cast=, w3cast=)."""
    if not xs:
        return []
    L.require_gpu(*xs)
    dev = xs[0].device
    if any(x.device != dev for x in xs):
        raise ValueError("tcast_t_group: every tensor must be on the same device")
    for x in xs:
        if x.dim() != 2 or x.shape[1] % 16:
            raise ValueError(f"tcast_t_group needs 2-D tensors with a multiple of 16 columns, got {tuple(x.shape)}")
    xc = [_prep(x) for x in xs]
    if len({x.dtype for x in xc}) != 1:   # one dtype per call: mixed lists widen to fp32, as tcast_t would read them
        xc = [L.aligned(x.float().contiguous()) for x in xc]
    out = []
    for x in xc:
        R, C = x.shape
        out += [torch.empty(R, C, dtype=E4, device=dev), torch.empty(C, _r16(R), dtype=E4, device=dev),
                torch.empty(1, dtype=torch.float32, device=dev)]
    n = len(xc)
    arr = lambda t, v: (t * n)(*v)
    with L.on_device(dev):
        ws = L.cast_workspace(dev)
        L.check(L.lib().gpic_fp8_tcast_t_group(
            n, arr(ctypes.c_void_p, [x.data_ptr() for x in xc]), L.DTYPE_CODE[xc[0].dtype],
            arr(ctypes.c_int64, [x.shape[0] for x in xc]), arr(ctypes.c_int64, [x.shape[1] for x in xc]),
            arr(ctypes.c_void_p, [out[3 * i].data_ptr() for i in range(n)]),
            arr(ctypes.c_void_p, [out[3 * i + 1].data_ptr() for i in range(n)]),
            arr(ctypes.c_int64, [out[3 * i + 1].shape[1] for i in range(n)]),
            arr(ctypes.c_void_p, [out[3 * i + 2].data_ptr() for i in range(n)]), ws.data_ptr(),
            L.stream_ptr(dev)), "gpic_fp8_tcast_t_group")
    return out


@tcast_t_group.register_fake
def _(xs):
    out = []
    for x in xs:
        R, C = x.shape
        out += [x.new_empty(R, C, dtype=E4), x.new_empty(C, _r16(R), dtype=E4), x.new_empty(1, dtype=torch.float32)]
    return out


class WeightCast(tuple):
    """A weight's (q, qt, dequant) from weight_casts, which also records the weight it was cast from (its storage
    pointer and version counter, which every in-place update such as an optimizer step advances), so that a cast
    kept past an update of the weight is refused instead of feeding the GEMMs stale bytes."""
    src = None


def weight_casts(*ws):
    """The (q, qt, dequant) triples of tcast_t_group(ws), one per weight, in order (WeightCast tuples)."""
    o = L.call(tcast_t_group, list(ws))
    out = []
    for i, w in enumerate(ws):
        c = WeightCast(o[3 * i:3 * i + 3])
        c.src = (w.data_ptr(), w._version)
        out.append(c)
    return out


def _swiglu_prep(z):
    L.require_gpu(z)
    if z.dim() != 2 or z.shape[1] % 2 or (z.shape[1] // 2) % 8:
        raise ValueError(f"the SwiGLU kernels need z [M, 2H] with H % 8 == 0, got {tuple(z.shape)}")
    if z.dtype != torch.bfloat16:
        raise ValueError(f"the SwiGLU kernels take bf16 z (w12's output), got {z.dtype}")
    return _prep_rows(z, z.shape[1])


@L.custom_op("gpic::fp8_swiglu_tcast")
def swiglu_tcast(z: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """z [M, 2H] bf16 (w12's output) -> silu(z1) * z2 as e4m3 [M, H] and its tensorwise scale [1] fp32.
    (fp8_native.py:130-144). gpic_fp8_swiglu_tcast_t with qt = NULL: the single pass, which holds up to 96 MiB of the
    product on chip and streams the rest through the temporary bf16 buffer; with single-pass casts disabled, the
    product written to the buffer by the amax pass and cast flat. The same bytes either way."""
    zc = _swiglu_prep(z)
    M, H2 = zc.shape
    H = H2 // 2
    q = torch.empty(M, H, dtype=E4, device=z.device)
    s = torch.empty(1, dtype=torch.float32, device=z.device)
    a = torch.empty(M, H, dtype=torch.bfloat16, device=z.device)
    with L.on_device(z.device):
        ws = L.cast_workspace(z.device)
        L.check(L.lib().gpic_fp8_swiglu_tcast_t(zc.data_ptr(), M, H, zc.stride(0), a.data_ptr(), q.data_ptr(),
                                                q.stride(0), None, 0, s.data_ptr(), ws.data_ptr(),
                                                L.stream_ptr(z.device)), "gpic_fp8_swiglu_tcast_t")
    return q, s


@swiglu_tcast.register_fake
def _(z):
    M, H2 = z.shape
    return z.new_empty(M, H2 // 2, dtype=E4), z.new_empty(1, dtype=torch.float32)


@L.custom_op("gpic::fp8_swiglu_tcast_t")
def swiglu_tcast_t(z: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """swiglu_tcast plus the transposed bytes qt [H, M16] (zero past M): the K-major operand of w3's FP8 wgrad."""
    zc = _swiglu_prep(z)
    M, H2 = zc.shape
    H = H2 // 2
    if H % 16:
        raise ValueError(f"swiglu_tcast_t needs H % 16 == 0, got H = {H}")
    q = torch.empty(M, H, dtype=E4, device=z.device)
    qt = torch.empty(H, _r16(M), dtype=E4, device=z.device)
    s = torch.empty(1, dtype=torch.float32, device=z.device)
    # the product a goes through HBM once (written by the amax pass, read by the cast) instead of being recomputed
    a = torch.empty(M, H, dtype=torch.bfloat16, device=z.device)
    with L.on_device(z.device):
        ws = L.cast_workspace(z.device)
        L.check(L.lib().gpic_fp8_swiglu_tcast_t(zc.data_ptr(), M, H, zc.stride(0), a.data_ptr(), q.data_ptr(),
                                                q.stride(0), qt.data_ptr(), qt.shape[1], s.data_ptr(), ws.data_ptr(),
                                                L.stream_ptr(z.device)), "gpic_fp8_swiglu_tcast_t")
    return q, qt, s


@swiglu_tcast_t.register_fake
def _(z):
    M, H2 = z.shape
    return (z.new_empty(M, H2 // 2, dtype=E4), z.new_empty(H2 // 2, _r16(M), dtype=E4),
            z.new_empty(1, dtype=torch.float32))


def _bwd_prep(z, da):
    zc = _swiglu_prep(z)
    M, H2 = zc.shape
    if da.shape != (M, H2 // 2) or da.dtype != torch.bfloat16:
        raise ValueError(f"da must be bf16 [{M}, {H2 // 2}], got {da.dtype} {tuple(da.shape)}")
    L.require_gpu(da)
    return zc, _prep_rows(da, H2 // 2)


def _swiglu_bwd(z, da, want_dz):
    zc, dac = _bwd_prep(z, da)
    M, H2 = zc.shape
    dz = torch.empty(M, H2, dtype=torch.bfloat16, device=z.device) if want_dz else None
    dq = torch.empty(M, H2, dtype=E4, device=z.device)
    s = torch.empty(1, dtype=torch.float32, device=z.device)
    with L.on_device(z.device):
        ws = L.cast_workspace(z.device)
        L.check(L.lib().gpic_fp8_swiglu_bwd(zc.data_ptr(), dac.data_ptr(), M, H2 // 2, zc.stride(0), dac.stride(0),
                                            L.ptr(dz), dq.data_ptr(), s.data_ptr(), ws.data_ptr(),
                                            L.stream_ptr(z.device)), "gpic_fp8_swiglu_bwd")
    return dz, dq, s


@L.custom_op("gpic::fp8_swiglu_bwd")
def swiglu_bwd(z: torch.Tensor, da: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """z [M, 2H] bf16, da [M, H] bf16 -> dz [M, 2H] bf16, dz as e4m3 [M, 2H] and its tensorwise scale [1] fp32.
    (fp8_native.py:153-166)"""
    return _swiglu_bwd(z, da, True)


@swiglu_bwd.register_fake
def _(z, da):
    M, H2 = z.shape
    return z.new_empty(M, H2), z.new_empty(M, H2, dtype=E4), z.new_empty(1, dtype=torch.float32)


@L.custom_op("gpic::fp8_swiglu_bwd_q")
def swiglu_bwd_q(z: torch.Tensor, da: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """swiglu_bwd without dz in memory: (dzq [M, 2H] e4m3, scale [1] fp32), the same bytes -- for phase 3, whose w12
    wgrad takes dzq instead of dz (an extension of the reference). One single-pass launch holds up to 80 MiB of dz on
    chip and computes the rest from z and da twice (for the amax, then for the cast); with single-pass casts disabled,
    an amax pass and a cast pass that recomputes dz."""
    _, dq, s = _swiglu_bwd(z, da, False)
    return dq, s


@swiglu_bwd_q.register_fake
def _(z, da):
    M, H2 = z.shape
    return z.new_empty(M, H2, dtype=E4), z.new_empty(1, dtype=torch.float32)


@L.custom_op("gpic::fp8_swiglu_bwd_t")
def swiglu_bwd_t(z: torch.Tensor, da: torch.Tensor,
                 want_dz: bool = True) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """swiglu_bwd plus the transposed bytes dzqt [2H, M16] (zero past M): the K-major operand of w12's FP8 wgrad.
    want_dz=False returns an empty dz and never writes it: dzq and dzqt (the same bytes) are cast from dz recomputed
    from z and da, which moves less memory than writing dz and reading it back."""
    zc, dac = _bwd_prep(z, da)
    M, H2 = zc.shape
    dz = torch.empty(M if want_dz else 0, H2, dtype=torch.bfloat16, device=z.device)
    dq = torch.empty(M, H2, dtype=E4, device=z.device)
    dqt = torch.empty(H2, _r16(M), dtype=E4, device=z.device)
    s = torch.empty(1, dtype=torch.float32, device=z.device)
    with L.on_device(z.device):
        ws = L.cast_workspace(z.device)
        L.check(L.lib().gpic_fp8_swiglu_bwd_t(zc.data_ptr(), dac.data_ptr(), M, H2 // 2, zc.stride(0), dac.stride(0),
                                              dz.data_ptr() if want_dz else None, dq.data_ptr(), dqt.data_ptr(),
                                              dqt.shape[1], s.data_ptr(),
                                              ws.data_ptr(), L.stream_ptr(z.device)), "gpic_fp8_swiglu_bwd_t")
    return dz, dq, dqt, s


@swiglu_bwd_t.register_fake
def _(z, da, want_dz=True):
    M, H2 = z.shape
    return (z.new_empty(M if want_dz else 0, H2), z.new_empty(M, H2, dtype=E4), z.new_empty(H2, _r16(M), dtype=E4),
            z.new_empty(1, dtype=torch.float32))


# ------------------------------------------------------------------------------------------------ GEMM

def _gemm_operand(t, name):
    if t.dtype != E4 or t.dim() != 2:
        raise ValueError(f"{name} must be a 2-D float8_e4m3fn tensor, got {t.dtype} {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) % 16 or t.stride(0) < t.shape[1] or t.data_ptr() % 16:
        t = L.aligned(t.contiguous())
    return t


@L.custom_op("gpic::fp8_gemm")
def fp8_gemm(a: torch.Tensor, sa: torch.Tensor, b: torch.Tensor, sb: torch.Tensor,
             bias: Optional[torch.Tensor] = None, fast: bool = True) -> torch.Tensor:
    """a [M, K] e4m3, b [N, K] e4m3 (both K-contiguous), sa / sb [1] fp32 dequantization scales ->
    C [M, N] bf16 = bf16(sa * sb * a @ b^T), then bf16(C + bias) when bias [N] is given.
    Replaces torch._scaled_mm(a, b.t(), scale_a=sa, scale_b=sb, out_dtype=bf16) of _mm (fp8_native.py:175-178) and the
    bias add of _Fp8Linear.forward (:189-190). `fast` (use_fast_accum) changes nothing: MFMA accumulates in fp32."""
    L.require_gpu(a, b, sa, sb, bias)
    a = _gemm_operand(a, "a")
    b = _gemm_operand(b, "b")
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"fp8_gemm: a is [{M}, {K}] but b is {tuple(b.shape)}")
    if K % 16 or N % 16:
        raise ValueError(f"fp8_gemm needs K % 16 == 0 and N % 16 == 0, got M={M} N={N} K={K}")
    if sa.dtype != torch.float32 or sa.shape != (1,):
        sa = sa.to(torch.float32).reshape(1)
    if sb.dtype != torch.float32 or sb.shape != (1,):
        sb = sb.to(torch.float32).reshape(1)
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} elements, got {bias.numel()}")
        bias = bias if bias.data_ptr() % 8 == 0 else bias.clone()
    c = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    with L.on_device(a.device):
        nws = L.gemm_workspace_bytes(a.device, M, N, K)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=a.device) if nws else None
        L.check(L.lib().gpic_fp8_gemm(a.data_ptr(), a.stride(0), sa.data_ptr(), b.data_ptr(), b.stride(0),
                                      sb.data_ptr(), L.ptr(bias), c.data_ptr(), c.stride(0), M, N, K, int(fast),
                                      L.ptr(ws), nws, L.stream_ptr(a.device)), "gpic_fp8_gemm")
    return c


@fp8_gemm.register_fake
def _(a, sa, b, sb, bias=None, fast=True):
    return a.new_empty(a.shape[0], b.shape[0], dtype=torch.bfloat16)


def _gemm_operand_mn(t, name):
    if t.dtype != E4 or t.dim() != 2:
        raise ValueError(f"{name} must be a 2-D float8_e4m3fn tensor, got {t.dtype} {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) % 16 or t.stride(0) < t.shape[1] or t.data_ptr() % 16:
        t = L.aligned(t.contiguous())
    return t


@L.custom_op("gpic::fp8_gemm_mn")
def fp8_gemm_mn(a: torch.Tensor, sa: torch.Tensor, b: torch.Tensor, sb: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a [K, M] e4m3, b [K, N] e4m3 (both with K as the row index), sa / sb [1] fp32 ->
    C [M, N] bf16 = bf16(sa * sb * a^T @ b) (then bf16(C + bias)). The FP8 weight gradient from the untransposed
    bytes of the output gradient (a) and the input (b): the same bytes as fp8_gemm(a.t(), sa, b.t(), sb) without the
    transposed copies. An extension of the reference, whose wgrads are bf16 (fp8_native.py:202, 264-265)."""
    L.require_gpu(a, b, sa, sb, bias)
    a = _gemm_operand_mn(a, "a")
    b = _gemm_operand_mn(b, "b")
    K, M = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"fp8_gemm_mn: a is [{K}, {M}] but b is {tuple(b.shape)}")
    if M % 16 or N % 16:
        raise ValueError(f"fp8_gemm_mn needs M % 16 == 0 and N % 16 == 0, got M={M} N={N} K={K}")
    if K * max(a.stride(0), b.stride(0)) >= 2 ** 31:
        # past the kernel's 32-bit load offsets: the K-major kernel on the transposed bytes (K padded with zeros to a
        # multiple of 16) gives the same bits
        k16 = (K + 15) // 16 * 16

        def kmajor(t):
            u = torch.zeros(t.shape[1], k16, dtype=torch.uint8, device=t.device)
            u[:, :K] = t.view(torch.uint8).t()
            return u.view(E4)
        return L.call(fp8_gemm, kmajor(a), sa, kmajor(b), sb, bias, False)
    if sa.dtype != torch.float32 or sa.shape != (1,):
        sa = sa.to(torch.float32).reshape(1)
    if sb.dtype != torch.float32 or sb.shape != (1,):
        sb = sb.to(torch.float32).reshape(1)
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
        if bias.numel() != N:
            raise ValueError(f"bias must have {N} elements, got {bias.numel()}")
        bias = bias if bias.data_ptr() % 8 == 0 else bias.clone()
    c = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    with L.on_device(a.device):
        nws = L.gemm_workspace_bytes(a.device, M, N, K)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=a.device) if nws else None
        L.check(L.lib().gpic_fp8_gemm_mn(a.data_ptr(), a.stride(0), sa.data_ptr(), b.data_ptr(), b.stride(0),
                                         sb.data_ptr(), L.ptr(bias), c.data_ptr(), c.stride(0), M, N, K,
                                         L.ptr(ws), nws, L.stream_ptr(a.device)), "gpic_fp8_gemm_mn")
    return c


@fp8_gemm_mn.register_fake
def _(a, sa, b, sb, bias=None):
    return a.new_empty(a.shape[1], b.shape[1], dtype=torch.bfloat16)


def _mm(xq, sx, wq, sw, fast=True):
    """[M, K] e4m3 x [N, K] e4m3 (each with its tensorwise scale) -> [M, N] bf16 (fp8_native.py:175-178)."""
    return L.call(fp8_gemm, xq, sx, wq, sw, None, fast)


# ------------------------------------------------------------------------------------------------ autograd

class _Fp8Linear(torch.autograd.Function):
    """fp8_native.py:181-204: FP8 forward GEMM; bf16 dgrad and wgrad from the saved bf16 input and weight."""
    @staticmethod
    def forward(ctx, x, w, b):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        xq, sx = L.call(tcast, x2)
        wq, sw = L.call(tcast, w)
        y = L.call(fp8_gemm, xq, sx, wq, sw, None if b is None else b.to(torch.bfloat16))
        ctx.save_for_backward(x2, w)
        ctx.has_b, ctx.shape, ctx.wdt = b is not None, shape, w.dtype
        return y.view(*shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, w = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        dx = (dy2 @ w.to(torch.bfloat16)).view(ctx.shape)
        dw = (dy2.t() @ x2).to(ctx.wdt)
        db = dy2.sum(0).to(ctx.wdt) if ctx.has_b else None
        return dx, dw, db


class _Fp8LinearF8(torch.autograd.Function):
    """Phase 3: forward, dgrad and wgrad GEMMs all in FP8. The forward keeps x's e4m3 bytes (the wgrad's B operand,
    read with the tokens as its K rows) and w's transposed bytes (the dgrad's B operand) instead of bf16 copies."""
    @staticmethod
    def forward(ctx, x, w, b, wcast=None):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        xq, sx = L.call(tcast, x2)
        wq, wqt, sw = L.call(tcast_t, w) if wcast is None else wcast
        y = L.call(fp8_gemm, xq, sx, wq, sw, None if b is None else b.to(torch.bfloat16))
        ctx.save_for_backward(xq, sx, wqt, sw)
        ctx.has_b, ctx.shape, ctx.wdt = b is not None, shape, w.dtype
        return y.view(*shape[:-1], w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        xq, sx, wqt, sw = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        dx = L.call(fp8_gemm, dyq, sdy, wqt, sw, None, False).view(ctx.shape)     # [M, N] . [K, N]^T
        dw = L.call(fp8_gemm_mn, dyq, sdy, xq, sx).to(ctx.wdt)                   # [M, N]^T . [M, K]
        db = dy2.sum(0).to(ctx.wdt) if ctx.has_b else None
        return dx, dw, db, None


class _Fp8HeadsLinearF8(torch.autograd.Function):
    """_Fp8LinearF8 on x = o.transpose(1, 2).reshape(B, N, H D) for the attention output o [B, H, N, D] (proj,
    JiT_T2I.py:183-185): x's e4m3 bytes come from tcast_heads(o), so x itself is never written; the same GEMMs and
    saved bytes as _Fp8LinearF8, and the gradient of o is dx viewed back as [B, H, N, D] (what the transpose and
    reshape give in autograd), so every output and gradient is the same bits as fp8_linear_f8 on the copy."""
    @staticmethod
    def forward(ctx, o, w, b, wcast=None):
        B, H, N, D = o.shape
        xq, sx = L.call(tcast_heads, o)
        xq = xq.view(B * N, H * D)
        wq, wqt, sw = L.call(tcast_t, w) if wcast is None else wcast
        y = L.call(fp8_gemm, xq, sx, wq, sw, None if b is None else b.to(torch.bfloat16))
        ctx.save_for_backward(xq, sx, wqt, sw)
        ctx.has_b, ctx.shape, ctx.wdt = b is not None, (B, H, N, D), w.dtype
        return y.view(B, N, w.shape[0])

    @staticmethod
    def backward(ctx, dy):
        xq, sx, wqt, sw = ctx.saved_tensors
        B, H, N, D = ctx.shape
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        dx = L.call(fp8_gemm, dyq, sdy, wqt, sw, None, False)                      # [M, N] . [K, N]^T
        do = dx.view(B, N, H, D).transpose(1, 2)
        dw = L.call(fp8_gemm_mn, dyq, sdy, xq, sx).to(ctx.wdt)                     # [M, N]^T . [M, K]
        db = dy2.sum(0).to(ctx.wdt) if ctx.has_b else None
        return do, dw, db, None


class _SwiGLUw3(torch.autograd.Function):
    """y = w3(silu(z1) * z2), the product written as FP8 rows for the GEMM (fp8_native.py:207-232)."""
    @staticmethod
    def forward(ctx, z, w3):
        shape = z.shape
        z2d = z.reshape(-1, shape[-1])
        aq, sa = L.call(swiglu_tcast, z2d)
        wq, sw = L.call(tcast, w3)
        y = _mm(aq, sa, wq, sw)
        ctx.save_for_backward(z2d, aq, sa, w3)
        ctx.shape, ctx.wdt = shape, w3.dtype
        return y.view(*shape[:-1], w3.shape[0])

    @staticmethod
    def backward(ctx, dy):
        z, aq, sa, w3 = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        da = dy2 @ w3.to(torch.bfloat16)
        dw3 = (dy2.t() @ (aq.to(torch.float32) * sa).to(torch.bfloat16)).to(ctx.wdt)
        z1, z2 = z.chunk(2, dim=-1)
        z1f = z1.float()
        sg = torch.sigmoid(z1f)
        sl = (z1f * sg).to(torch.bfloat16)
        dz2 = da * sl
        dz1 = (da.float() * z2.float() * (sg * (1 + z1f * (1 - sg)))).to(torch.bfloat16)
        return torch.cat([dz1, dz2], dim=-1).view(ctx.shape), dw3


class _Fp8MLP(torch.autograd.Function):
    """Phase 2 (fp8_native.py:235-266): the whole SwiGLU MLP, FP8 forward GEMMs and FP8 dgrads of w3 and w12; the
    SwiGLU backward kernel writes dz in bf16 (w12's weight gradient) and its FP8 copy (w12's dgrad); weight
    gradients in bf16. The weights' FP8 copies for the dgrads are the transposed casts."""
    @staticmethod
    def forward(ctx, x, w12, w3):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        xq, sx = L.call(tcast, x2)
        w12q, s12 = L.call(tcast, w12)
        z = _mm(xq, sx, w12q, s12)
        aq, sa = L.call(swiglu_tcast, z)
        w3q, s3 = L.call(tcast, w3)
        y = _mm(aq, sa, w3q, s3)
        ctx.save_for_backward(x2, z, aq, sa, w12, w3)
        ctx.shape, ctx.dt = shape, (w12.dtype, w3.dtype)
        return y.view(*shape[:-1], w3.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, z, aq, sa, w12, w3 = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        _, w3tq, s3t = L.call(tcast_t, w3, False)                  # [H, C]: the dgrad's B operand
        da = _mm(dyq, sdy, w3tq, s3t, fast=False)          # [M, H]
        dz, dzq, sdz = L.call(swiglu_bwd, z, da)
        _, w12tq, s12t = L.call(tcast_t, w12, False)               # [C, 2H]
        dx = _mm(dzq, sdz, w12tq, s12t, fast=False)        # [M, C]
        dw12 = (dz.t() @ x2).to(ctx.dt[0])
        dw3 = (dy2.t() @ (aq.to(torch.float32) * sa).to(torch.bfloat16)).to(ctx.dt[1])
        return dx.view(ctx.shape), dw12, dw3


class _Fp8MLPF8(torch.autograd.Function):
    """Phase 3: the SwiGLU MLP with every GEMM in FP8 -- forward, both dgrads and both wgrads. The forward saves x's
    and the SwiGLU product's e4m3 bytes (the wgrads' B operands, read with the tokens as K rows), z, and the weights'
    transposed bytes (the dgrads' B operands)."""
    @staticmethod
    def forward(ctx, x, w12, w3, w12cast=None, w3cast=None):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        xq, sx = L.call(tcast, x2)
        w12q, w12qt, s12 = L.call(tcast_t, w12) if w12cast is None else w12cast
        z = L.call(fp8_gemm, xq, sx, w12q, s12)
        aq, sa = L.call(swiglu_tcast, z)
        w3q, w3qt, s3 = L.call(tcast_t, w3) if w3cast is None else w3cast
        y = L.call(fp8_gemm, aq, sa, w3q, s3)
        ctx.save_for_backward(xq, sx, z, aq, sa, w12qt, s12, w3qt, s3)
        ctx.shape, ctx.dt = shape, (w12.dtype, w3.dtype)
        return y.view(*shape[:-1], w3.shape[0])

    @staticmethod
    def backward(ctx, dy):
        xq, sx, z, aq, sa, w12qt, s12, w3qt, s3 = ctx.saved_tensors
        dy2 = dy.reshape(-1, dy.shape[-1]).to(torch.bfloat16)
        dyq, sdy = L.call(tcast, dy2)
        da = L.call(fp8_gemm, dyq, sdy, w3qt, s3, None, False)           # [M, H]
        dw3 = L.call(fp8_gemm_mn, dyq, sdy, aq, sa)                      # [M, C]^T . [M, H] = [C, H]
        dzq, sdz = L.call(swiglu_bwd_q, z, da)                           # dz itself is not needed: never written
        dx = L.call(fp8_gemm, dzq, sdz, w12qt, s12, None, False)         # [M, C]
        dw12 = L.call(fp8_gemm_mn, dzq, sdz, xq, sx)                     # [M, 2H]^T . [M, C] = [2H, C]
        return dx.view(ctx.shape), dw12.to(ctx.dt[0]), dw3.to(ctx.dt[1]), None, None


def fp8_mlp(x, w12, w3):
    with torch.autocast("cuda", enabled=False):
        return _Fp8MLP.apply(x.to(torch.bfloat16), w12, w3)


def fp8_linear(x, w, b=None):
    with torch.autocast("cuda", enabled=False):
        return _Fp8Linear.apply(x.to(torch.bfloat16), w, b)


def fp8_swiglu_w3(z, w3):
    with torch.autocast("cuda", enabled=False):
        return _SwiGLUw3.apply(z.to(torch.bfloat16), w3)


def _check_cast(name, w, c):
    if c is not None and (len(c) != 3 or c[0].shape != w.shape or c[1].shape[0] != w.shape[1]):
        raise ValueError(f"{name}: a (q, qt, dequant) triple of tcast_t(weight) [{tuple(w.shape)}] expected")
    src = getattr(c, "src", None)
    if src is not None and src != (w.data_ptr(), w._version):
        raise ValueError(f"{name} was cast from another weight, or before the weight's last update: cast it again "
                         "(weight_casts) after every in-place change of the weight")
    return c


def fp8_linear_f8(x, w, b=None, wcast=None):
    """Phase 3 fp8_linear: FP8 dgrad and wgrad as well. wcast: w's (q, qt, dequant) from weight_casts (the same bytes
    tcast_t(w) would give, cast beforehand with the block's other weights), else w is cast here. A wcast must come
    from w's current values: cast again after every update of w (an optimizer step). A WeightCast (weight_casts)
    that was cast from another tensor or before w's last in-place update is refused; of a plain tuple only the
    shapes are checked. The check reads w's version counter, which in-place ops on w advance (torch.optim's updates,
    made under no_grad); writes through w.data do not (w.data has a counter of its own), so cast again after those."""
    with torch.autocast("cuda", enabled=False):
        return _Fp8LinearF8.apply(x.to(torch.bfloat16), w, b, _check_cast("wcast", w, wcast))


def fp8_heads_linear_f8(o, w, b=None, wcast=None):
    """Phase 3 fp8_linear_f8 applied to the attention output o [B, H, N, D] as proj takes it: the same result and
    gradients as fp8_linear_f8(o.transpose(1, 2).reshape(B, N, H D), w, b) without that copy (its e4m3 bytes come from
    tcast_heads(o)). wcast: as fp8_linear_f8's."""
    if o.dim() != 4:
        raise ValueError(f"fp8_heads_linear_f8 needs o [B, H, N, D], got {tuple(o.shape)}")
    if o.shape[1] * o.shape[3] != w.shape[1]:
        raise ValueError(f"o {tuple(o.shape)} merges to {o.shape[1] * o.shape[3]} features, w has {w.shape[1]}")
    with torch.autocast("cuda", enabled=False):
        return _Fp8HeadsLinearF8.apply(o.to(torch.bfloat16), w, b, _check_cast("wcast", w, wcast))


def fp8_mlp_f8(x, w12, w3, w12cast=None, w3cast=None):
    """Phase 3 fp8_mlp: every GEMM of the SwiGLU MLP in FP8. w12cast / w3cast: as fp8_linear_f8's wcast."""
    with torch.autocast("cuda", enabled=False):
        return _Fp8MLPF8.apply(x.to(torch.bfloat16), w12, w3, _check_cast("w12cast", w12, w12cast),
                               _check_cast("w3cast", w3, w3cast))


class Fp8Linear(torch.nn.Linear):
    """nn.Linear with the FP8 forward GEMM (the same parameters and state-dict keys)."""
    def forward(self, x):
        return fp8_linear(x, self.weight, self.bias)


class Fp8LinearF8(torch.nn.Linear):
    """nn.Linear with FP8 forward, dgrad and wgrad GEMMs (phase 3; the same parameters and state-dict keys)."""
    def forward(self, x):
        return fp8_linear_f8(x, self.weight, self.bias)


def _fp8_ok(lin):
    """An nn.Linear the FP8 GEMM can take: in and out features multiples of 16 (fp8.py:35's rule)."""
    return type(lin) is torch.nn.Linear and lin.in_features % 16 == 0 and lin.out_features % 16 == 0


def _convert_block(blk, phase, attn_names):
    """One block's attention linears `attn_names` and its SwiGLU MLP (w12, w3), as convert_native describes."""
    n = 0
    mlp = blk.mlp
    mlp_ok = _fp8_ok(mlp.w12) and _fp8_ok(mlp.w3) and mlp.w12.out_features % 32 == 0
    if phase >= 2:
        lin_cls = Fp8LinearF8 if phase >= 3 else Fp8Linear
        mlp_fn = fp8_mlp_f8 if phase >= 3 else fp8_mlp
        for name in attn_names:
            lin = getattr(blk.attn, name, None)
            if _fp8_ok(lin):
                lin.__class__ = lin_cls
                n += 1
        if mlp_ok and not getattr(mlp, "_fp8", False):
            mlp._fp8 = True
            mlp.forward = (lambda m, f: (lambda x: f(x, m.w12.weight, m.w3.weight)))(mlp, mlp_fn)
            n += 2
        return n
    for parent, name in [(blk.attn, a) for a in attn_names] + [(mlp, "w12")]:
        lin = getattr(parent, name, None)
        if _fp8_ok(lin):
            lin.__class__ = Fp8Linear
            n += 1
    if mlp_ok and not getattr(mlp, "_fp8", False):
        mlp._fp8 = True
        mlp.forward = (lambda m: (lambda x: fp8_swiglu_w3(m.w12(x), m.w3.weight)))(mlp)
        n += 1
    return n


def convert_native(net, phase=1, text=False, fused_norm=False, fused_heads=False):
    """Phase 1: the image blocks' qkv_x, proj, w12 to Fp8Linear and their SwiGLU's w3 GEMM to the fused path. Phase 2:
    qkv_x and proj as in phase 1, the MLP as one fused FP8 function with FP8 dgrads. Phase 3: qkv_x and proj to
    Fp8LinearF8, the MLP as one function with every GEMM in FP8. Returns the count of GEMMs converted
    (fp8_native.py:290-317).
    text=True (an extension: the reference's native recipes convert the image blocks only, fp8_native.py:294, while its
    torchao filter also takes the text-refine blocks, fp8.py:31) converts, in the same phase, the image blocks' kv_y
    (over the text tokens) and the text-refine blocks' attention qkv, proj and SwiGLU MLP (JiT_T2I.py:131,227,231,274):
    linears of M = batch x text tokens, which the same kernels serve.
    fused_norm=True (phase 3 only; an extension: the reference's lever K, JiT_T2I.py:201-207, and its FP8 linears stay
    separate) also rewires each image block's forward so its two norm sites write h's e4m3 bytes for qkv_x and the
    MLP directly (gpic_fp8.norm.convert_fused_norm); the GEMM count is unchanged.
    fused_heads=True (phase 3 only; an extension: the reference casts the head-merged copy of the attention output,
    JiT_T2I.py:183-185) also makes each converted attention's proj cast the attention output in its own layout
    (gpic_fp8.heads.convert_fused_heads): the head-merging copy is never made; the GEMM count is unchanged."""
    if fused_norm and phase != 3:
        raise ValueError("fused_norm needs phase 3 (the fused norm consumers run every GEMM in FP8)")
    if fused_heads and phase != 3:
        raise ValueError("fused_heads needs phase 3 (the attention output's fused cast feeds the phase-3 proj)")
    n = 0
    for blk in getattr(net, "blocks", []):
        n += _convert_block(blk, phase, ("qkv_x", "proj", "kv_y") if text else ("qkv_x", "proj"))
    if text:
        for blk in getattr(net, "text_refine_blocks", []):
            n += _convert_block(blk, phase, ("qkv", "proj"))
    if fused_norm:
        from .norm import convert_fused_norm
        convert_fused_norm(net)
    if fused_heads:
        from .heads import convert_fused_heads
        convert_fused_heads(net)
    return n


def reference(x, w, b=None):
    """The tensorwise FP8 forward in plain torch ops (tests); fp8_native.py:320-331 as written, including its eager
    FMAX / a (torch computes it as reciprocal(a) * 448, which can differ from the kernels' IEEE 448 / a in the last
    bit of the scale)."""
    def q(t):
        a = t.float().abs().amax().clamp_min(TINY)
        return (t.float() * (FMAX / a)).clamp(-FMAX, FMAX).to(E4), a / FMAX
    x2 = x.reshape(-1, x.shape[-1])
    xq, sx = q(x2)
    wq, sw = q(w)
    y = (xq.float() * sx) @ (wq.float() * sw).t()
    if b is not None:
        y = y + b.float()
    return y.to(torch.bfloat16).view(*x.shape[:-1], w.shape[0])
