"""Checks shared by the GPU parity tests: bit views of bf16 / e4m3 tensors and the GEMM bounds against the float64
scaled product of the same e4m3 operands (the reference's scaled-matmul semantics, fp8_native.py:175-178,320-331)."""
import numpy as np
import torch

E4 = torch.float8_e4m3fn


def bits(t):
    """bf16 tensor -> numpy uint16 bit patterns (host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def qb(t):
    """e4m3 tensor -> numpy uint8 bytes (host)."""
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def assert_bf16_bits_equal(x, y):
    """Two arrays of bf16 bit patterns equal bit for bit, except that a NaN may be encoded with another payload or
    sign (the NaNs must sit at the same positions)."""
    nx = (x & 0x7FFF) > 0x7F80
    ny = (y & 0x7FFF) > 0x7F80
    assert np.array_equal(nx, ny), f"NaN at different positions: {(nx != ny).sum()}"
    diff = (x != y) & ~nx
    assert not diff.any(), f"{diff.sum()} bf16 values differ"


def rel(x, ref):
    x, ref = x.double(), ref.double()
    return (torch.linalg.norm(x - ref) / torch.linalg.norm(ref)).item()


def ref_fp32(a, sa, b, sb):
    """(a * sa) @ (b * sb)^T in fp32 on the GPU (no TF32) for a [M, K], b [N, K] e4m3."""
    torch.backends.cuda.matmul.allow_tf32 = False
    return (a.float() * float(sa)) @ (b.float() * float(sb)).t()


# The FP8 MFMA (v_mfma_*_f8f6f4) does not sum the products of one instruction exactly: with a few large products in
# a block (activations with x50 outlier channels) the result of a single 32 x 32 x 64 instruction (K = 64) was measured
# up to 1.6e-4 of the sum of |terms| away from the exact sum, and hipBLASLt's FP8 GEMM gives the same errors on the
# same operands; the 16 x 16 x 128 form the GEMM now uses (K = 128 per instruction) showed the same largest errors as
# two 32 x 32 x 64 instructions on the same random and outlier blocks. Data without such outliers stays within 2^-16
# of the sum of |terms|. OUTLIER_SLACK is the allowance for operands with outlier channels (3x the largest error
# measured).
OUTLIER_SLACK = 2.0 ** -11


def assert_elementwise(c, a, sa, b, sb, rows=None, slack=2.0 ** -16):
    """Every element of c = bf16(sa sb a b^T) (a [M, K], b [N, K], e4m3) within one bf16 rounding of the exact
    product (2^-8 relative) plus an accumulation allowance (`slack` times the sum of |terms|: the fp32 accumulation
    order and the MFMA's own summation of each block of products), computed in float64. `rows`: check only these
    rows of c (a long index tensor), for products too large to redo whole."""
    if rows is not None:
        a = a[rows]
        c = c[rows]
    af = a.double() * float(sa)
    bf = b.double() * float(sb)
    exact = af @ bf.t()
    bound = exact.abs() * 2.0 ** -8 + (af.abs() @ bf.abs().t()) * slack
    err = (c.double() - exact).abs()
    bad = (err > bound).sum().item()
    assert bad == 0, f"{bad} elements out of bounds; worst excess {(err - bound).max().item():.3g}"


def sample_rows(m, n, seed):
    """n distinct row indices of [0, m) (all of them when n >= m), including the first and the last."""
    g = torch.Generator().manual_seed(seed)
    if n >= m:
        return torch.arange(m)
    r = torch.randperm(m, generator=g)[:n]
    r[0], r[1] = 0, m - 1
    return torch.unique(r)


# The single-pass casts write their tagged partial maxima from byte 28672 of the cast workspace (one 64-bit word per
# workgroup, the call tag in the high half), count partials a workgroup had to compute from x itself at byte 36864,
# keep the last call's tag (the epoch) at byte 36868, the groups of 32 workgroups of a call that are done folding at
# byte 36872 and each group's count of its workgroups done from byte 40960, one word every 128 bytes (cast.hip:
# kOnceTagged, kOnceFallback, kOnceEpoch, kOnceDone, kOnceGroupDone).
ONCE_WORD0, ONCE_FALLBACK, ONCE_EPOCH, ONCE_DONE = 28672 // 8, 36864 // 4, 36868 // 4, 36872 // 4
ONCE_GROUP_DONE = [(40960 + 128 * g) // 4 for g in range(32)]


def once_state(dev):
    """(workgroup 0's tagged partial word, the count of partials computed by waiters) after the stream's work."""
    from gpic_fp8 import _lib as L
    ws = L.cast_workspace(dev)
    torch.cuda.synchronize()
    w0 = int(ws.view(torch.int64)[ONCE_WORD0].item())
    # after a single-pass call the epoch holds its tag (the high half of workgroup 0's word) and the counter is back to 0
    assert int(ws[ONCE_DONE].item()) == 0 and not ws[ONCE_GROUP_DONE].any()
    assert int(ws[ONCE_EPOCH].item()) & 0xffffffff == (w0 >> 32) & 0xffffffff or w0 == 0
    return w0, int(ws[ONCE_FALLBACK].item())
