"""The drop-in autograd API on the GPU: Fp8Linear / fp8_linear / fp8_swiglu_w3 / fp8_mlp (phases 1 and 2, as the
reference) and the phase-3 all-FP8 functions, against the golden vectors and against fp32 autograd of the same
dequantized formulas (tolerance 1e-2 relative Frobenius), plus convert_native on a small model."""
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

import gpic_fp8 as G

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
TOL = 1e-2


def rel(x, ref):
    x, ref = x.float(), ref.float()
    return (torch.linalg.norm(x - ref) / torch.linalg.norm(ref)).item()


def deq(q, s):
    return q.float() * s


@pytest.fixture(autouse=True)
def no_tf32():
    torch.backends.cuda.matmul.allow_tf32 = False


def test_linear_forward_golden(dev):
    with np.load(GOLD, allow_pickle=False) as g:
        t = {k: torch.from_numpy(g[k].view(np.int16)).view(torch.bfloat16).to(dev)
             for k in ("lin_x", "lin_w", "lin_b", "lin_y")}
    y = G.fp8_linear(t["lin_x"], t["lin_w"], t["lin_b"])
    assert rel(y, t["lin_y"]) < 5e-3
    y3 = G.fp8_linear_f8(t["lin_x"], t["lin_w"], t["lin_b"])
    assert torch.equal(y, y3)                               # phases share the forward bit for bit


def test_linear_phase1_backward_is_the_references(dev):
    """Phase 1 backward = bf16 matmuls of the saved bf16 input and weight (fp8_native.py:198-204)."""
    x = torch.randn(4, 64, 256, device=dev, dtype=torch.bfloat16, requires_grad=True)
    w = (torch.randn(512, 256, device=dev) / 16).requires_grad_()           # fp32 master weight (DDP)
    b = torch.zeros(512, device=dev, requires_grad=True)
    y = G.fp8_linear(x, w, b)
    assert y.dtype == torch.bfloat16 and y.shape == (4, 64, 512)
    dy = torch.randn_like(y)
    y.backward(dy)
    dy2 = dy.reshape(-1, 512)
    assert torch.equal(x.grad, (dy2 @ w.detach().to(torch.bfloat16)).view(4, 64, 256))
    assert torch.equal(w.grad, (dy2.t() @ x.detach().reshape(-1, 256)).float())
    assert torch.equal(b.grad, dy2.sum(0).float())


def test_linear_phase3_all_fp8(dev):
    M, K, N = 1024, 512, 768
    x = torch.randn(M, K, device=dev).to(torch.bfloat16).requires_grad_()
    w = (torch.randn(N, K, device=dev) / K ** 0.5).to(torch.bfloat16).requires_grad_()
    b = (torch.randn(N, device=dev) * 0.1).to(torch.bfloat16).requires_grad_()
    y = G.fp8_linear_f8(x, w, b)
    dy = (torch.randn(M, N, device=dev) * 0.1).to(torch.bfloat16)
    y.backward(dy)
    # the same quantized operands, fp32 products
    xq, sx = G.tcast(x.detach())
    wq, sw = G.tcast(w.detach())
    dyq, sdy = G.tcast(dy)
    assert rel(x.grad, deq(dyq, sdy) @ deq(wq, sw)) < 4e-3
    assert rel(w.grad, deq(dyq, sdy).t() @ deq(xq, sx)) < 4e-3
    # the wgrad from the untransposed bytes is bit for bit the TN GEMM of the transposed bytes
    assert torch.equal(w.grad, G.fp8_gemm(G.tcast_t(dy)[1], sdy, G.tcast_t(x.detach())[1], sx))
    assert torch.equal(b.grad, dy.sum(0).to(torch.bfloat16))
    # and close to the unquantized bf16 gradients
    assert rel(x.grad, dy.float() @ w.detach().float()) < 0.1


def _mlp_ref(x, w12, w3):
    """fp32 autograd of the SwiGLU MLP with the FP8 forward's quantization points (for the phase-3 gradients)."""
    xf = x.float().requires_grad_()
    w12f = w12.float().requires_grad_()
    w3f = w3.float().requires_grad_()
    z = xf @ w12f.t()
    z1, z2 = z.chunk(2, -1)
    y = (torch.nn.functional.silu(z1) * z2) @ w3f.t()
    return xf, w12f, w3f, y


@pytest.mark.parametrize("fn", ["fp8_mlp", "fp8_mlp_f8"])
def test_mlp_phases(dev, fn):
    M, C, H = 1024, 256, 1024
    x = torch.randn(M, C, device=dev).to(torch.bfloat16).requires_grad_()
    w12 = (torch.randn(2 * H, C, device=dev) / C ** 0.5).to(torch.bfloat16).requires_grad_()
    w3 = (torch.randn(C, H, device=dev) / H ** 0.5).to(torch.bfloat16).requires_grad_()
    y = getattr(G, fn)(x, w12, w3)
    dy = (torch.randn(M, C, device=dev) * 0.1).to(torch.bfloat16)
    y.backward(dy)
    xf, w12f, w3f, yf = _mlp_ref(x.detach(), w12.detach(), w3.detach())
    yf.backward(dy.float())
    assert rel(y, yf) < 0.1                     # e4m3 inputs: a few percent from the bf16 / fp32 model
    assert rel(x.grad, xf.grad) < 0.15
    assert rel(w12.grad, w12f.grad) < 0.15
    assert rel(w3.grad, w3f.grad) < 0.15
    # both phases run the same forward bit for bit
    y_other = (G.fp8_mlp_f8 if fn == "fp8_mlp" else G.fp8_mlp)(x.detach(), w12.detach(), w3.detach())
    assert torch.equal(y.detach(), y_other)


def test_mlp_phase3_grads_match_quantized_formula(dev):
    """Each phase-3 gradient equals the fp32 product of the very e4m3 operands it was given."""
    M, C, H = 512, 256, 512
    x = torch.randn(M, C, device=dev).to(torch.bfloat16).requires_grad_()
    w12 = (torch.randn(2 * H, C, device=dev) / C ** 0.5).to(torch.bfloat16).requires_grad_()
    w3 = (torch.randn(C, H, device=dev) / H ** 0.5).to(torch.bfloat16).requires_grad_()
    y = G.fp8_mlp_f8(x, w12, w3)
    dy = (torch.randn(M, C, device=dev) * 0.1).to(torch.bfloat16)
    y.backward(dy)
    xq, sx = G.tcast(x.detach())
    w12q, s12 = G.tcast(w12.detach())
    z = G.fp8_gemm(xq, sx, w12q, s12)
    aq, sa = G.swiglu_tcast(z)
    w3q, s3 = G.tcast(w3.detach())
    dyq, sdy = G.tcast(dy)
    da = G.fp8_gemm(dyq, sdy, G.tcast_t(w3.detach(), False)[1], s3)
    assert rel(w3.grad, deq(dyq, sdy).t() @ deq(aq, sa)) < 4e-3
    _, dzq, sdz = G.swiglu_bwd(z, da)
    assert rel(x.grad, deq(dzq, sdz) @ deq(w12q, s12)) < 4e-3
    assert rel(w12.grad, deq(dzq, sdz).t() @ deq(xq, sx)) < 4e-3
    # the wgrads from the untransposed bytes are bit for bit the TN GEMMs of the transposed bytes
    assert torch.equal(w3.grad, G.fp8_gemm(G.tcast_t(dy)[1], sdy, G.swiglu_tcast_t(z)[1], sa))
    assert torch.equal(w12.grad, G.fp8_gemm(G.swiglu_bwd_t(z, da)[2], sdz, G.tcast_t(x.detach())[1], sx))


def _np_bf16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _np_q(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def _bf16_matmul64(a, b):
    """bf16(a @ b) with a, b float arrays, the product in float64: the reference's bf16 GEMMs (fp8_native.py:202,225,
    264-265) up to their accumulation order."""
    from oracle import oracle as O
    return O.bf16_to_f32(O.f32_to_bf16((np.asarray(a, np.float64) @ np.asarray(b, np.float64)).astype(np.float32)))


def _deq(q, s):
    from oracle import oracle as O
    return O.e4m3_to_f32(q).astype(np.float64) * np.float64(s)


def _orel(x, ref):
    from oracle import oracle as O
    return O.rel_fro(x.detach().float().cpu().numpy(), ref)


def test_swiglu_w3_phase1_against_oracle(dev):
    """_SwiGLUw3 (fp8_native.py:207-232). Forward: the product cast and w3's cast are the oracle's bytes and scales
    (the kernels reproduce them bit for bit) and y is within the elementwise bound of the oracle's float64 scaled
    product of those bytes. Backward: exactly the reference's eager formulas (:221-232) on the saved tensors, and
    within 1e-2 of the oracle's float64 restatement (dz within one bf16 ulp of the oracle's swiglu_bwd, whose
    sigmoid is this build's)."""
    from oracle import oracle as O
    M, C, H = 512, 256, 1024
    g = torch.Generator(device=dev).manual_seed(31)
    z = (torch.randn(M, 2 * H, generator=g, device=dev) * 2).to(torch.bfloat16).requires_grad_()
    w3 = (torch.randn(C, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16).requires_grad_()
    dy = (torch.randn(M, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    y = G.fp8_swiglu_w3(z, w3)
    zb, w3b = _np_bf16(z), _np_bf16(w3)
    oaq, osa, _ = O.swiglu_tcast(zb)
    o3q, os3, _ = O.tcast(w3b)
    aq, sa = G.swiglu_tcast(z.detach())
    w3q, s3 = G.tcast(w3.detach())
    assert np.array_equal(_np_q(aq), oaq) and sa.item() == osa
    assert np.array_equal(_np_q(w3q), o3q) and s3.item() == os3
    ref = O.mm64(oaq, osa, o3q, os3)
    assert _orel(y, ref) < 4e-3
    from parity import assert_elementwise
    assert_elementwise(y, aq, sa.item(), w3q, s3.item())
    y.backward(dy)
    # the reference's eager backward, written out (fp8_native.py:221-232)
    zd, w3d = z.detach(), w3.detach()
    da = dy @ w3d.to(torch.bfloat16)
    dw3 = (dy.t() @ (aq.to(torch.float32) * sa).to(torch.bfloat16)).to(w3.dtype)
    z1, z2 = zd.chunk(2, dim=-1)
    z1f = z1.float()
    sg = torch.sigmoid(z1f)
    dz2 = da * (z1f * sg).to(torch.bfloat16)
    dz1 = (da.float() * z2.float() * (sg * (1 + z1f * (1 - sg)))).to(torch.bfloat16)
    assert torch.equal(z.grad, torch.cat([dz1, dz2], dim=-1))
    assert torch.equal(w3.grad, dw3)
    # against the oracle: da, dw3 in float64, dz from the oracle's swiglu_bwd of that da
    dyf = O.bf16_to_f32(_np_bf16(dy))
    oda = O.f32_to_bf16(_bf16_matmul64(dyf, O.bf16_to_f32(w3b)))
    assert np.abs(O.bf16_to_f32(_np_bf16(da)) - O.bf16_to_f32(oda)).max() <= 2.0 ** -7 * np.abs(O.bf16_to_f32(oda)).max()
    odz, _, _, _ = O.swiglu_bwd(zb, _np_bf16(da))
    diff = np.abs(_np_bf16(z.grad).astype(np.int32) - odz.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    odw3 = _bf16_matmul64(dyf.T, _deq(oaq, osa))
    assert _orel(w3.grad, odw3) < 1e-2


@pytest.mark.parametrize("phase", [2, 3])
def test_mlp_against_oracle_chain(dev, phase):
    """_Fp8MLP (phase 2, fp8_native.py:235-266) and the all-FP8 _Fp8MLPF8 (phase 3): output and every gradient
    within 1e-2 relative Frobenius of the oracle's chain on the same inputs -- tcast, mm, swiglu_tcast, mm forward;
    tcast(dy), tcast(w3^T), mm (da), swiglu_bwd, tcast(w12^T), mm (dx) backward; the wgrads as the reference's bf16
    products (phase 2) or as float64 scaled products of the e4m3 bytes (phase 3). Every intermediate is the
    oracle's own."""
    from oracle import oracle as O
    M, C, H = 512, 256, 512
    g = torch.Generator(device=dev).manual_seed(32 + phase)
    x = torch.randn(M, C, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    w12 = (torch.randn(2 * H, C, generator=g, device=dev) / C ** 0.5).to(torch.bfloat16).requires_grad_()
    w3 = (torch.randn(C, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16).requires_grad_()
    dy = (torch.randn(M, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    y = (G.fp8_mlp if phase == 2 else G.fp8_mlp_f8)(x, w12, w3)
    y.backward(dy)
    xb, w12b, w3b, dyb = _np_bf16(x), _np_bf16(w12), _np_bf16(w3), _np_bf16(dy)
    # forward chain
    oxq, osx, _ = O.tcast(xb)
    o12q, os12, _ = O.tcast(w12b)
    oz = O.mm(oxq, osx, o12q, os12)                                  # [M, 2H] bf16
    oaq, osa, _ = O.swiglu_tcast(oz)
    o3q, os3, _ = O.tcast(w3b)
    assert _orel(y, O.mm64(oaq, osa, o3q, os3)) < 1e-2
    # backward chain
    odyq, osdy, _ = O.tcast(dyb)
    o3tq, os3t, _ = O.tcast(np.ascontiguousarray(w3b.T))            # [H, C]
    oda = O.mm(odyq, osdy, o3tq, os3t)                               # [M, H]
    odz, odzq, osdz, _ = O.swiglu_bwd(oz, oda)
    o12tq, os12t, _ = O.tcast(np.ascontiguousarray(w12b.T))         # [C, 2H]
    assert _orel(x.grad, O.mm64(odzq, osdz, o12tq, os12t)) < 1e-2
    if phase == 2:
        odw12 = _bf16_matmul64(O.bf16_to_f32(odz).T, O.bf16_to_f32(xb))
        odw3 = _bf16_matmul64(O.bf16_to_f32(dyb).T, _deq(oaq, osa))
    else:
        odw12 = _deq(odzq, osdz).T @ _deq(oxq, osx)
        odw3 = _deq(odyq, osdy).T @ _deq(oaq, osa)
    assert _orel(w12.grad, odw12) < 1e-2
    assert _orel(w3.grad, odw3) < 1e-2


def test_mlp_phase2_wiring_exact(dev):
    """Phase 2's backward, operation by operation (fp8_native.py:255-266), recomputed from the same kernels on the
    same tensors: dx is the FP8 dgrad of swiglu_bwd's dzq with w12's transposed bytes, dw12 the bf16 product dz^T x,
    dw3 the bf16 product dy^T bf16(aq sa) -- all bit for bit."""
    M, C, H = 512, 256, 512
    g = torch.Generator(device=dev).manual_seed(35)
    x = torch.randn(M, C, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    w12 = (torch.randn(2 * H, C, generator=g, device=dev) / C ** 0.5).to(torch.bfloat16).requires_grad_()
    w3 = (torch.randn(C, H, generator=g, device=dev) / H ** 0.5).to(torch.bfloat16).requires_grad_()
    dy = (torch.randn(M, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    G.fp8_mlp(x, w12, w3).backward(dy)
    xd, w12d, w3d = x.detach(), w12.detach(), w3.detach()
    xq, sx = G.tcast(xd)
    w12q, s12 = G.tcast(w12d)
    z = G.fp8_gemm(xq, sx, w12q, s12)
    aq, sa = G.swiglu_tcast(z)
    dyq, sdy = G.tcast(dy)
    _, w3tq, s3t = G.tcast_t(w3d, False)
    da = G.fp8_gemm(dyq, sdy, w3tq, s3t, None, False)
    dz, dzq, sdz = G.swiglu_bwd(z, da)
    _, w12tq, s12t = G.tcast_t(w12d, False)
    assert torch.equal(x.grad, G.fp8_gemm(dzq, sdz, w12tq, s12t, None, False))
    assert torch.equal(w12.grad, (dz.t() @ xd).to(w12.dtype))
    assert torch.equal(w3.grad, (dy.t() @ (aq.to(torch.float32) * sa).to(torch.bfloat16)).to(w3.dtype))
    # the transposed bytes are the reference's tcast(w.t().contiguous()) (fp8_native.py:259,262)
    q3t, s3t2 = G.tcast(w3d.t().contiguous())
    assert torch.equal(q3t.view(torch.uint8), w3tq.view(torch.uint8)) and s3t2.item() == s3t.item()


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.qkv_x = nn.Linear(d, 3 * d, bias=False)
        self.proj = nn.Linear(d, d)

    def forward(self, x):
        q, k, v = self.qkv_x(x).chunk(3, -1)
        a = torch.softmax((q.float() @ k.float().transpose(-1, -2)) / q.shape[-1] ** 0.5, -1)
        return self.proj((a @ v.float()).to(x.dtype))


class _MLP(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.w12 = nn.Linear(d, 8 * d, bias=False)
        self.w3 = nn.Linear(4 * d, d, bias=False)

    def forward(self, x):
        x1, x2 = self.w12(x).chunk(2, -1)
        return self.w3(torch.nn.functional.silu(x1) * x2)


class _Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = _Attn(d)
        self.mlp = _MLP(d)

    def forward(self, x):
        x = x + self.attn(x)
        return x + self.mlp(x)


class _Net(nn.Module):
    def __init__(self, d, n):
        super().__init__()
        self.blocks = nn.ModuleList(_Block(d) for _ in range(n))

    def forward(self, x):
        for b in self.blocks:
            x = b(x)
        return x


@pytest.mark.parametrize("recipe", ["native", "native2", "native3"])
def test_convert_and_train_step(dev, recipe):
    torch.manual_seed(0)
    net = _Net(128, 2).to(dev).to(torch.bfloat16)
    ref = _Net(128, 2).to(dev).to(torch.bfloat16)
    ref.load_state_dict(net.state_dict())
    assert G.convert_fp8(net, recipe) == 8
    x = torch.randn(4, 64, 128, device=dev).to(torch.bfloat16)
    y, yr = net(x), ref(x)
    assert rel(y, yr) < 0.1
    y.float().square().mean().backward()
    yr.float().square().mean().backward()
    for (n, p), (_, pr) in zip(net.named_parameters(), ref.named_parameters()):
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
        assert rel(p.grad, pr.grad) < 0.25, n


class _XAttn(nn.Module):
    """Image attention with the text cross-attention keys / values (qkv_x, kv_y, proj: JiT_T2I.py:130-136)."""
    def __init__(self, d):
        super().__init__()
        self.qkv_x = nn.Linear(d, 3 * d, bias=False)
        self.kv_y = nn.Linear(d, 2 * d, bias=False)
        self.proj = nn.Linear(d, d)

    def forward(self, x, y):
        q, k, v = self.qkv_x(x).chunk(3, -1)
        ky, vy = self.kv_y(y).chunk(2, -1)
        k, v = torch.cat([k, ky], 1), torch.cat([v, vy], 1)
        a = torch.softmax((q.float() @ k.float().transpose(-1, -2)) / q.shape[-1] ** 0.5, -1)
        return self.proj((a @ v.float()).to(x.dtype))


class _TAttn(_Attn):
    """TextRefineAttention's linears are named qkv and proj (JiT_T2I.py:227,231)."""
    def __init__(self, d):
        super().__init__(d)
        self.qkv = self.qkv_x
        del self.qkv_x

    def forward(self, x):
        q, k, v = self.qkv(x).chunk(3, -1)
        a = torch.softmax((q.float() @ k.float().transpose(-1, -2)) / q.shape[-1] ** 0.5, -1)
        return self.proj((a @ v.float()).to(x.dtype))


class _XBlock(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = _XAttn(d)
        self.mlp = _MLP(d)

    def forward(self, x, y):
        x = x + self.attn(x, y)
        return x + self.mlp(x)


class _TBlock(_Block):
    def __init__(self, d):
        super().__init__(d)
        self.attn = _TAttn(d)


class _TNet(nn.Module):
    def __init__(self, d, n):
        super().__init__()
        self.blocks = nn.ModuleList(_XBlock(d) for _ in range(n))
        self.text_refine_blocks = nn.ModuleList(_TBlock(d) for _ in range(1))

    def forward(self, x, y):
        for b in self.text_refine_blocks:
            y = b(y)
        for b in self.blocks:
            x = b(x, y)
        return x


def test_convert_text_blocks_and_train_step(dev):
    """Recipe native3+text: the image blocks' kv_y and the text-refine block's qkv, proj and MLP run on the FP8
    kernels as well, at a text length (51 tokens, M = 204 rows) that is no multiple of 16; outputs and every
    gradient close to the bf16 model's."""
    torch.manual_seed(1)
    net = _TNet(128, 2).to(dev).to(torch.bfloat16)
    ref = _TNet(128, 2).to(dev).to(torch.bfloat16)
    ref.load_state_dict(net.state_dict())
    assert G.convert_fp8(net, "native3+text") == 2 * 5 + 4
    assert type(net.blocks[0].attn.kv_y) is G.Fp8LinearF8 and type(net.text_refine_blocks[0].attn.qkv) is G.Fp8LinearF8
    x = torch.randn(4, 64, 128, device=dev).to(torch.bfloat16)
    y = torch.randn(4, 51, 128, device=dev).to(torch.bfloat16)
    out, outr = net(x, y), ref(x, y)
    assert rel(out, outr) < 0.1
    out.float().square().mean().backward()
    outr.float().square().mean().backward()
    for (n, p), (_, pr) in zip(net.named_parameters(), ref.named_parameters()):
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
        assert rel(p.grad, pr.grad) < 0.25, n
