"""CPU oracle for nano-gpic's native FP8 linear path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the checker
(or as the timed CPU baseline). The product package (nano-gpic_amd/gpic_fp8) never imports it and has no CPU fallback.

The byte-level work (amax, scales, e4m3 rounding, the SwiGLU roundings) is scalar C in fp8_oracle.c, loaded with
ctypes; the GEMM is a float64 numpy matmul of the dequantized operands. bf16 tensors travel as numpy uint16 arrays of
their bit patterns. Each function names the reference lines (baselines/PixelGen/src/models/layers/fp8_native.py)
it restates.

How each function is pinned (tests/test_oracle.py):
  e4m3 / cast   torch CPU .to(float8_e4m3fn) on every bf16 value x every scale in a sweep, on every e4m3 rounding
                boundary +-1 ulp, and on 2^22 random fp32 values; the OCP spec's decoded value of all 256 bytes;
                the committed fixtures in tests/golden (written by tests/golden/make_golden.py with torch ops only).
  amax / scales closed forms (max |x| by numpy; torch.div for the IEEE divisions), the transpose invariant and the
                power-of-two scale invariant.
  swiglu        the eager torch expression of fp8_native.py:226-231 with torch.sigmoid, within 1 bf16 ulp (and
                equal for >99.9% of values); the exp against math.exp to <= 2 fp32 ulp on every bf16 input.
  tcast_heads   the cast of o in its own order, permuted: the scale is the same for any order of the elements and
                the bytes are elementwise, so byte (b N + n, h D + d) is byte (b, h, n, d) of tcast(o).
  mm            exact small-integer operands with power-of-two scales (bf16-exact sums), identity / one-hot B,
                and torch's fp32 matmul of the same dequantized operands.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")
_lib = None

FMAX = 448.0
TINY = 1e-12

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64


def build():
    """Compile fp8_oracle.c into liboracle.so (gcc, via the Makefile next to it)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO) or os.path.getmtime(_SO) < os.path.getmtime(os.path.join(_HERE, "fp8_oracle.c")):
            build()
        L = ctypes.CDLL(_SO)
        L.gpo_e4m3.restype = ctypes.c_uint8
        L.gpo_e4m3.argtypes = [ctypes.c_float]
        L.gpo_e4m3_n.argtypes = [_f32p, _i64, _u8p]
        L.gpo_e4m3_to_f32.restype = ctypes.c_float
        L.gpo_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.gpo_amax_bf16.restype = ctypes.c_uint32
        L.gpo_amax_bf16.argtypes = [_u16p, _i64]
        L.gpo_amax_f32.restype = ctypes.c_uint32
        L.gpo_amax_f32.argtypes = [_f32p, _i64]
        L.gpo_scales.argtypes = [ctypes.c_uint32, _f32p, _f32p]
        L.gpo_cast_bf16.argtypes = [_u16p, _i64, ctypes.c_float, _u8p]
        L.gpo_cast_f32.argtypes = [_f32p, _i64, ctypes.c_float, _u8p]
        L.gpo_tcast_bf16.argtypes = [_u16p, _i64, _u8p, _f32p, _u32p]
        L.gpo_tcast_f32.argtypes = [_f32p, _i64, _u8p, _f32p, _u32p]
        L.gpo_exp.restype = ctypes.c_float
        L.gpo_exp.argtypes = [ctypes.c_float]
        L.gpo_sigmoid.restype = ctypes.c_float
        L.gpo_sigmoid.argtypes = [ctypes.c_float]
        L.gpo_swiglu1.restype = ctypes.c_uint16
        L.gpo_swiglu1.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.gpo_swiglu_tcast.argtypes = [_u16p, _i64, _i64, _i64, _u8p, _i64, _f32p, _u32p]
        L.gpo_swiglu_bwd1.argtypes = [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_uint16, _u16p, _u16p]
        L.gpo_swiglu_bwd.argtypes = [_u16p, _u16p, _i64, _i64, _i64, _i64, _u16p, _i64, _u8p, _f32p, _u32p]
        L.gpo_mod_rmsnorm.argtypes = [_u16p, _u16p, _u16p, _i64, _f32p, _u16p, _i64, _u16p, _i64, _i64, _i64, _i64,
                                      ctypes.c_float, _u16p, _u16p, _f32p]
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t)


# ---------------------------------------------------------------- bf16 helpers (bit patterns as uint16)

def bf16_to_f32(h):
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f):
    """RNE, NaN -> quiet NaN (torch's rule)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def e4m3_to_f32(q):
    """Decode e4m3fn bytes (vectorised restatement of gpo_e4m3_to_f32)."""
    q = np.asarray(q, dtype=np.uint8)
    s = (q >> 7).astype(np.int32)
    e = ((q >> 3) & 15).astype(np.int32)
    m = (q & 7).astype(np.float64)
    v = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e.astype(np.float64) - 10))
    v = np.where((e == 15) & (q & 7 == 7), np.nan, v)
    return np.where(s == 1, -v, v).astype(np.float32)


# ---------------------------------------------------------------- the cast (fp8_native.py:33-49, 105-122)

def e4m3(x):
    """Elementwise e4m3fn RNE of fp32 values (no scaling, no clamp)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, dtype=np.uint8)
    lib().gpo_e4m3_n(_p(x, _f32p), x.size, _p(q, _u8p))
    return q


def scales(amax_bits):
    """(scale, dequant) from the amax bits: scale = RN(448 / max(a, 1e-12)), dequant = RN(a / 448)."""
    s, d = ctypes.c_float(), ctypes.c_float()
    lib().gpo_scales(ctypes.c_uint32(int(amax_bits)), ctypes.byref(s), ctypes.byref(d))
    return np.float32(s.value), np.float32(d.value)


def amax_bits(x):
    """max |x| as fp32 bits; x: uint16 (bf16 bits) or float32 array."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        return int(lib().gpo_amax_bf16(_p(x, _u16p), x.size))
    x = x.astype(np.float32, copy=False)
    return int(lib().gpo_amax_f32(_p(x, _f32p), x.size))


def cast(x, scale):
    """q = e4m3(clamp(RN(x * scale), +-448)) elementwise; x: uint16 (bf16 bits) or float32, contiguous."""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, dtype=np.uint8)
    if x.dtype == np.uint16:
        lib().gpo_cast_bf16(_p(x, _u16p), x.size, ctypes.c_float(scale), _p(q, _u8p))
    else:
        x = x.astype(np.float32, copy=False)
        lib().gpo_cast_f32(_p(x, _f32p), x.size, ctypes.c_float(scale), _p(q, _u8p))
    return q


def tcast(x):
    """tcast (fp8_native.py:114-122): x -> (e4m3 bytes like x, dequant scale fp32, amax fp32 bits)."""
    x = np.ascontiguousarray(x)
    q = np.empty(x.shape, dtype=np.uint8)
    d, am = ctypes.c_float(), ctypes.c_uint32()
    if x.dtype == np.uint16:
        lib().gpo_tcast_bf16(_p(x, _u16p), x.size, _p(q, _u8p), ctypes.byref(d), ctypes.byref(am))
    else:
        x = x.astype(np.float32, copy=False)
        lib().gpo_tcast_f32(_p(x, _f32p), x.size, _p(q, _u8p), ctypes.byref(d), ctypes.byref(am))
    return q, np.float32(d.value), int(am.value)


# ---------------------------------------------------------------- SwiGLU (fp8_native.py:52-98, 130-172)

def tcast_heads(o):
    """The attention output's cast as proj reads it (JiT_T2I.py:183-185: x = attention(q, k, v);
    x.transpose(1, 2).reshape(B, N, C); tcast(x) in proj, fp8_native.py:114-122,187): o [B, H, N, D] bf16 bits ->
    (e4m3 bytes [B N, H D], dequant, amax bits)."""
    B, H, N, D = o.shape
    return tcast(np.ascontiguousarray(o.transpose(0, 2, 1, 3)).reshape(B * N, H * D))


def sigmoid(x):
    L = lib()
    return np.array([L.gpo_sigmoid(float(v)) for v in np.ravel(x)], dtype=np.float32)


def exp(x):
    L = lib()
    return np.array([L.gpo_exp(float(v)) for v in np.ravel(x)], dtype=np.float32)


def swiglu_product(z):
    """a = bf16(bf16(z1 * sigmoid(z1)) * z2) for z [M, 2H] bf16 bits -> [M, H] bf16 bits."""
    z = np.ascontiguousarray(z, dtype=np.uint16)
    M, H2 = z.shape
    H = H2 // 2
    table = swiglu_table()
    # a depends on (z1, z2); sl = bf16(z1 * sigmoid(z1)) is a function of z1 alone, tabulated over all bf16 values
    sl = bf16_to_f32(table[z[:, :H]])
    return f32_to_bf16(sl * bf16_to_f32(z[:, H:]))


_TABLE = None


def swiglu_table():
    """sl = bf16(z1 * sigmoid(z1)) for every bf16 bit pattern z1 (65536 entries), from the C restatement."""
    global _TABLE
    if _TABLE is None:
        L = lib()
        one = 0x3F80  # z2 = 1.0: a = bf16(sl * 1) = sl
        _TABLE = np.array([L.gpo_swiglu1(h, one) for h in range(65536)], dtype=np.uint16)
    return _TABLE


def swiglu_tcast(z):
    """swiglu_tcast (fp8_native.py:130-144): z [M, 2H] bf16 bits -> (aq [M, H] bytes, dequant, amax bits)."""
    z = np.ascontiguousarray(z, dtype=np.uint16)
    M, H2 = z.shape
    H = H2 // 2
    q = np.empty((M, H), dtype=np.uint8)
    d, am = ctypes.c_float(), ctypes.c_uint32()
    lib().gpo_swiglu_tcast(_p(z, _u16p), M, H, H2, _p(q, _u8p), H, ctypes.byref(d), ctypes.byref(am))
    return q, np.float32(d.value), int(am.value)


def swiglu_bwd(z, da):
    """swiglu_bwd (fp8_native.py:153-166): z [M, 2H], da [M, H] bf16 bits -> (dz bits, dzq bytes, dequant, amax)."""
    z = np.ascontiguousarray(z, dtype=np.uint16)
    da = np.ascontiguousarray(da, dtype=np.uint16)
    M, H2 = z.shape
    H = H2 // 2
    dz = np.empty((M, H2), dtype=np.uint16)
    dzq = np.empty((M, H2), dtype=np.uint8)
    d, am = ctypes.c_float(), ctypes.c_uint32()
    lib().gpo_swiglu_bwd(_p(z, _u16p), _p(da, _u16p), M, H, H2, H, _p(dz, _u16p), H2, _p(dzq, _u8p),
                         ctypes.byref(d), ctypes.byref(am))
    return dz, dzq, np.float32(d.value), int(am.value)


# ---------------------------------------------------------------- the norm sites' producer (fused_norm.py:64-91)

def mod_rmsnorm(x, w, shift, scale, ntok, eps, a=None, gate=None):
    """res_mod_rmsnorm's forward (a, gate given) or mod_rmsnorm's (fused_norm.py:64-91) in this build's arithmetic:
    x, a [rows, C] bf16 bits; w [C] fp32; gate, shift, scale [B, C] bf16 bits (row b serves rows b * ntok ..);
    returns (x_new bits or None, h bits, rstd fp32)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    rows, C = x.shape
    w = np.ascontiguousarray(w, dtype=np.float32)
    sh = np.ascontiguousarray(shift, dtype=np.uint16)
    sc = np.ascontiguousarray(scale, dtype=np.uint16)
    h = np.empty((rows, C), dtype=np.uint16)
    rstd = np.empty(rows, dtype=np.float32)
    if a is not None:
        a = np.ascontiguousarray(a, dtype=np.uint16)
        gate = np.ascontiguousarray(gate, dtype=np.uint16)
        xn = np.empty((rows, C), dtype=np.uint16)
        ap, gp, xp = _p(a, _u16p), _p(gate, _u16p), _p(xn, _u16p)
    else:
        xn, ap, gp, xp = None, None, None, None
    lib().gpo_mod_rmsnorm(_p(x, _u16p), ap, gp, C, _p(w, _f32p), _p(sh, _u16p), C, _p(sc, _u16p), C, rows, ntok, C,
                          ctypes.c_float(eps), xp, _p(h, _u16p), _p(rstd, _f32p))
    return xn, h, rstd


def mod_rmsnorm_q(x, w, shift, scale, ntok, eps, a=None, gate=None):
    """The norm followed by h's tcast: (x_new or None, h, rstd, hq bytes, dequant)."""
    xn, h, rstd = mod_rmsnorm(x, w, shift, scale, ntok, eps, a, gate)
    hq, d, _ = tcast(h)
    return xn, h, rstd, hq, d


# ---------------------------------------------------------------- the scaled GEMM (fp8_native.py:175-178, 320-331)

def mm64(aq, sa, bq, sb):
    """C = (sa * A) @ (sb * B)^T in float64 for A [M, K], B [N, K] e4m3 bytes: the scaled-matmul value that
    torch._scaled_mm rounds (fp8_native.py:178; reference() at :328 does the same product in fp32)."""
    a = e4m3_to_f32(aq).astype(np.float64) * np.float64(sa)
    b = e4m3_to_f32(bq).astype(np.float64) * np.float64(sb)
    return a @ b.T


def mm(aq, sa, bq, sb, bias=None):
    """_mm then the bias add of _Fp8Linear.forward (fp8_native.py:188-190): y = bf16(C); y = bf16(y + bf16(b))."""
    y = f32_to_bf16(mm64(aq, sa, bq, sb).astype(np.float32))
    if bias is not None:
        y = f32_to_bf16(bf16_to_f32(y) + bf16_to_f32(np.asarray(bias, dtype=np.uint16))[None, :])
    return y


def rel_fro(x, ref):
    """Relative Frobenius error |x - ref|_F / |ref|_F (the north-star GEMM tolerance is 1e-2)."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / (den if den > 0 else 1.0))


def linear_forward(x, w, bias=None):
    """_Fp8Linear.forward (fp8_native.py:183-195) on bf16 bits: x [M, K], w [N, K] (uint16 or float32)."""
    xq, sx, _ = tcast(x)
    wq, sw, _ = tcast(w)
    return mm(xq, sx, wq, sw, bias)


# ---------------------------------------------------------------- the same path in torch CPU ops (the CPU baseline)
#
# A restatement of the reference's plain-torch path (fp8_native.py:320-331, reference()) with the production cast's
# division rule (fp8_native.py:40-49: IEEE 448 / amax via torch.div, never the eager 448.0 / a), the SwiGLU product
# and backward as the reference's eager expressions (fp8_native.py:55-58, 226-231, torch.sigmoid), on torch CPU
# tensors: what bench.py times on the host's cores as the CPU baseline. Inputs are NaN-free (torch's amax propagates
# NaN, the kernels' ignores it). Pinned against the C restatement above (tests/test_oracle.py): the same bytes and
# scales for the casts and the product cast, dz within one bf16 ulp.

def torch_tcast(x):
    """tcast on a CPU tensor: (e4m3 tensor, dequant [1] fp32)."""
    import torch
    a = x.float().abs().amax().clamp_min(TINY).reshape(1)
    fmax = torch.tensor([FMAX], dtype=torch.float32)
    q = (x.float() * torch.div(fmax, a)).clamp(-FMAX, FMAX).to(torch.float8_e4m3fn)
    return q, torch.div(a, fmax)


def torch_mm(aq, sa, bq, sb):
    """_mm on CPU tensors as reference() computes it: the fp32 product of the dequantized operands, rounded to bf16."""
    import torch
    return ((aq.float() * sa) @ (bq.float() * sb).t()).to(torch.bfloat16)


def torch_swiglu_tcast(z):
    """swiglu_tcast on a CPU bf16 tensor z [M, 2H]: a = bf16(bf16(z1 sigmoid(z1)) z2), then its tcast."""
    import torch
    z1, z2 = z.float().chunk(2, dim=-1)
    sl = (z1 * torch.sigmoid(z1)).to(torch.bfloat16)
    return torch_tcast((sl.float() * z2).to(torch.bfloat16))


def torch_swiglu_bwd(z, da):
    """swiglu_bwd on CPU bf16 tensors (the eager backward of fp8_native.py:226-231): (dz, dzq, dequant)."""
    import torch
    z1, z2 = z.float().chunk(2, dim=-1)
    sg = torch.sigmoid(z1)
    dz2 = da * (z1 * sg).to(torch.bfloat16)
    dz1 = (da.float() * z2 * (sg * (1 + z1 * (1 - sg)))).to(torch.bfloat16)
    dz = torch.cat([dz1, dz2], dim=-1)
    dzq, s = torch_tcast(dz)
    return dz, dzq, s
