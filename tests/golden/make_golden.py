"""Writes tests/golden/golden.npz: small seeded inputs of the FP8 path and their expected outputs, computed with
torch CPU operations only (independent of oracle/ and of the HIP kernels).

The reference holds no golden vectors for this path (its tests live outside the checkout), so these vectors restate
its rules (baselines/PixelGen/src/models/layers/fp8_native.py) with torch's own routines:
  cast     amax = x.abs().amax(); a = clamp_min(amax, 1e-12); scale = torch.div(448, a) and dequant = torch.div(a, 448)
           (IEEE divisions, as the kernel's div_rn, :43-44,49); q = (x * scale).clamp(+-448).to(float8_e4m3fn) (:47)
  swiglu   sl = (z1 * sigmoid(z1)).bf16; a = (sl * z2).bf16 (:55-58), then the cast
  bwd      the eager expression of :226-231 (= the kernel's :88-94), then the cast of dz
  gemm     exact: small-integer e4m3 operands, power-of-two scales -> the fp32 sums are exact, C = bf16(sum * s)
  linear   reference() (:320-331) with IEEE scales: bf16(fp32 matmul of the dequantized operands + bias)
bf16 arrays are stored as uint16 bit patterns, e4m3 as uint8 bytes. Run: python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
E4 = torch.float8_e4m3fn


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def bytes8(t):
    return t.contiguous().view(torch.uint8).numpy().copy()


def tcast(x):
    xf = x.float()
    a = torch.clamp_min(xf.abs().amax(), 1e-12) if xf.numel() else torch.tensor(1e-12)
    scale = torch.div(torch.tensor(448.0), a)
    deq = torch.div(a, torch.tensor(448.0))
    q = (xf * scale).clamp(-448.0, 448.0).to(E4)
    return q, deq.reshape(1)


def main():
    g = torch.Generator().manual_seed(1234)
    out = {}
    # flat casts
    x = torch.randn(96, 128, generator=g)
    cols = torch.randperm(128, generator=g)[:3]
    x[:, cols] *= 50.0
    x = x.to(torch.bfloat16)
    q, d = tcast(x)
    out.update(cast_bf16_x=bits16(x), cast_bf16_q=bytes8(q), cast_bf16_s=d.numpy())

    x = (torch.randn(37, 23, generator=g) * 3).to(torch.bfloat16)          # 851 elements: a tail of 3
    q, d = tcast(x)
    out.update(cast_tail_x=bits16(x), cast_tail_q=bytes8(q), cast_tail_s=d.numpy())

    w = torch.randn(64, 80, generator=g) / 80 ** 0.5                        # an fp32 (DDP master) weight
    q, d = tcast(w)
    out.update(cast_f32_x=w.numpy(), cast_f32_q=bytes8(q), cast_f32_s=d.numpy())

    # wide dynamic range: one large value pushes most elements into e4m3's subnormal range and its ties
    x = (torch.randn(512, generator=g) * torch.exp2(torch.randint(-12, 2, (512,), generator=g).float()))
    x[7] = 3000.0
    x = x.to(torch.bfloat16)
    q, d = tcast(x)
    out.update(cast_range_x=bits16(x), cast_range_q=bytes8(q), cast_range_s=d.numpy())

    z = torch.zeros(16, 16, dtype=torch.bfloat16)
    q, d = tcast(z)
    out.update(cast_zero_q=bytes8(q), cast_zero_s=d.numpy())

    # cast + transposed copy (rows padded to 16 with zero bytes)
    x = torch.randn(40, 48, generator=g).to(torch.bfloat16)
    q, d = tcast(x)
    qt = torch.zeros(48, 48, dtype=torch.uint8)
    qt[:, :40] = q.view(torch.uint8).t()
    out.update(cast_t_x=bits16(x), cast_t_q=bytes8(q), cast_t_qt=qt.numpy(), cast_t_s=d.numpy())

    # SwiGLU product cast
    z = (torch.randn(24, 128, generator=g) * 3).to(torch.bfloat16)
    z1, z2 = z.float().chunk(2, dim=-1)
    sl = (z1 * torch.sigmoid(z1)).to(torch.bfloat16)
    a = (sl.float() * z2).to(torch.bfloat16)
    q, d = tcast(a)
    out.update(swiglu_z=bits16(z), swiglu_a=bits16(a), swiglu_q=bytes8(q), swiglu_s=d.numpy())

    # SwiGLU backward (the eager expression)
    da = (torch.randn(24, 64, generator=g) * 0.1).to(torch.bfloat16)
    z1b, z2b = z.chunk(2, dim=-1)
    z1f = z1b.float()
    sg = torch.sigmoid(z1f)
    slb = (z1f * sg).to(torch.bfloat16)
    dz2 = da * slb
    dz1 = (da.float() * z2b.float() * (sg * (1 + z1f * (1 - sg)))).to(torch.bfloat16)
    dz = torch.cat([dz1, dz2], dim=-1)
    q, d = tcast(dz)
    out.update(bwd_da=bits16(da), bwd_dz=bits16(dz), bwd_dzq=bytes8(q), bwd_s=d.numpy())

    # exact GEMM: integers in [-8, 8] are exact e4m3 values; power-of-two scales; K = 160 (not a multiple of 128)
    A = torch.randint(-8, 9, (72, 160), generator=g).float()
    B = torch.randint(-8, 9, (48, 160), generator=g).float()
    sa, sb = 2.0 ** -3, 2.0 ** -2
    C = (A @ B.t()) * (sa * sb)                                              # exact in fp32
    bias = (torch.randn(48, generator=g)).to(torch.bfloat16)
    Cb = C.to(torch.bfloat16)
    out.update(gemm_a=bytes8(A.to(E4)), gemm_b=bytes8(B.to(E4)), gemm_sa=np.float32([sa]), gemm_sb=np.float32([sb]),
               gemm_c=bits16(Cb), gemm_bias=bits16(bias), gemm_cbias=bits16((Cb.float() + bias.float()).to(torch.bfloat16)))

    # linear forward (reference() with IEEE scales)
    x = torch.randn(128, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(192, 256, generator=g) / 16).to(torch.bfloat16)
    b = (torch.randn(192, generator=g) * 0.1).to(torch.bfloat16)
    xq, sx = tcast(x)
    wq, sw = tcast(w)
    y = ((xq.float() * sx) @ (wq.float() * sw).t() + b.float()).to(torch.bfloat16)
    out.update(lin_x=bits16(x), lin_w=bits16(w), lin_b=bits16(b), lin_y=bits16(y))

    np.savez_compressed(OUT, **out)
    print(OUT, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
