"""The attention output's producer-fused cast (tcast_heads, gpic_fp8_tcast_heads) and its consumers: proj's FP8
linear on the attention output (fp8_heads_linear_f8) and the converter route (convert_native(fused_heads=True),
recipes "+heads" / "+fused"). Every result is held bit for bit to the unfused computation -- the head-merging copy
o.transpose(1, 2).reshape(B, N, H D) cast by tcast and fed to fp8_linear_f8 -- and the cast also to the oracle."""
import copy

import numpy as np
import pytest
import torch

import attn_blocks as AB
import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture
def knob():
    yield
    L.set_single_pass(True, -1)


def merged(o):
    B, H, N, D = o.shape
    return o.transpose(1, 2).reshape(B, N, H * D)


def same_cast(o):
    """tcast_heads(o) against tcast of the copy: the same bytes and scale."""
    q, s = G.tcast_heads(o)
    qr, sr = G.tcast(merged(o))
    B, H, N, D = o.shape
    assert q.shape == (B, N, H * D) and q.dtype == G.E4
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)), "bytes differ from the copy's cast"
    assert torch.equal(s, sr), (s.item(), sr.item())
    return q, s


def flash_layout(B, H, N, D, dev, seed, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(B, H, N, D, generator=g, device=dev) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("B,H,N,D", [
    (2, 4, 24, 64),       # a few KiB: the 256-thread single pass
    (8, 16, 256, 64),     # 4 MiB
    (128, 16, 256, 64),   # d12, one GPU's 32768 tokens (64 MiB): the wide single pass
    (128, 28, 256, 64),   # d18 (112 MiB): the wide kernel's hybrid (part streamed twice)
    (3, 3, 7, 16),        # odd head and token counts: every division of the source index by a non-power of two
    (2, 5, 33, 128),
    (1, 1, 9, 32),        # extents of 1
    (48, 16, 512, 64),    # 48 MiB: the 256-thread kernel's limit before the wide one
    (48, 16, 513, 64),    # just past it: the wide kernel
    (100, 16, 512, 64),   # 100 MiB: all that the wide kernel holds on 256 CUs
    (100, 16, 513, 64),   # just past it: a hybrid streaming one group of words twice
])
def test_flash_layout_equals_copy_cast(dev, B, H, N, D):
    """o as scaled_dot_product_attention's flash backend writes it ([B, H, N, D] in memory)."""
    same_cast(flash_layout(B, H, N, D, dev, B * H + N + D))


def test_other_layouts(dev):
    """[B, N, H, D] in memory (the efficient backend: the call is the flat cast of o), a D-slice of a wider tensor
    (token stride 2 D), heads and batches interleaved, and an unaligned o (made contiguous first)."""
    B, H, N, D = 4, 8, 40, 64
    x = torch.randn(B, N, H, D, device=dev).to(torch.bfloat16)
    same_cast(x.transpose(1, 2))
    wide = torch.randn(B, H, N, 2 * D, device=dev).to(torch.bfloat16)
    same_cast(wide[..., :D])
    same_cast(wide[..., D:])
    hb = torch.randn(H, B, N, D, device=dev).to(torch.bfloat16)
    same_cast(hb.transpose(0, 1))
    flat = torch.randn(B * H * N * D + 8, device=dev).to(torch.bfloat16)
    same_cast(flat[8:].view(B, H, N, D))
    same_cast(flat[4:4 + B * H * N * D].view(B, H, N, D))          # 8-byte offset: not 16-byte aligned


def test_against_oracle(dev):
    o = flash_layout(3, 6, 50, 64, dev, 7)
    q, s = G.tcast_heads(o)
    oq, od, _ = O.tcast_heads(o.view(torch.int16).cpu().numpy().view(np.uint16))
    assert s.item() == od
    assert np.array_equal(q.view(torch.uint8).cpu().numpy().reshape(oq.shape), oq)


@pytest.mark.parametrize("enabled,wait", [(False, -1), (True, 0)])
def test_two_pass_and_zero_wait_agree(dev, knob, enabled, wait):
    """The two-pass path (forced) and the single pass computing every other partial itself (zero wait) give the same
    bytes as the default path, at the d12 size and a small one."""
    for shape in ((128, 16, 256, 64), (3, 3, 7, 16)):
        o = flash_layout(*shape, dev, 11)
        q0, s0 = G.tcast_heads(o)
        L.set_single_pass(enabled, wait)
        q1, s1 = same_cast(o)
        L.set_single_pass(True, -1)
        assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8)) and torch.equal(s0, s1)


def test_nan_inf_outliers_and_empty(dev):
    """NaN is ignored by the amax and inf saturates, as in tcast; an outlier sets the scale wherever it lies; an empty
    o writes only the scale of a zero amax."""
    o = flash_layout(4, 8, 64, 64, dev, 3)
    o[1, 3, 17, 5] = float("nan")
    o[2, 0, 63, 63] = float("inf")
    o[3, 7, 0, 0] = -float("inf")
    same_cast(o)
    o = flash_layout(4, 8, 64, 64, dev, 4)
    o[0, 5, 31, 40] = 3072.0                                       # exact in bf16
    q, s = same_cast(o)
    assert s.item() == np.float32(np.float32(3072.0) / np.float32(448.0))
    q, s = G.tcast_heads(torch.empty(0, 8, 64, 64, device=dev, dtype=torch.bfloat16))
    assert q.shape == (0, 64, 512) and s.item() == np.float32(np.float32(1e-12) / np.float32(448.0))


def test_heads_linear_equals_linear_on_copy(dev):
    """fp8_heads_linear_f8(o, w, b) against fp8_linear_f8 on the head-merged copy, with o from
    scaled_dot_product_attention (flash backend) inside autograd: the output and the gradients of q, k, v, w, b bit
    for bit."""
    torch.manual_seed(2)
    B, H, N, D = 8, 16, 256, 64
    C = H * D
    qkv = [torch.randn(B, H, N, D, device=dev).to(torch.bfloat16).requires_grad_() for _ in range(3)]
    w = (torch.randn(C, C, device=dev) / C ** 0.5).to(torch.bfloat16).requires_grad_()
    b = (torch.randn(C, device=dev) * 0.1).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(B, N, C, device=dev).to(torch.bfloat16)
    outs = []
    for fused in (True, False):
        ts = [t.detach().clone().requires_grad_() for t in (*qkv, w, b)]
        o = torch.nn.functional.scaled_dot_product_attention(*ts[:3])
        y = G.fp8_heads_linear_f8(o, ts[3], ts[4]) if fused else G.fp8_linear_f8(merged(o), ts[3], ts[4])
        y.backward(dy)
        outs.append([y] + [t.grad for t in ts])
    for a, r in zip(*outs):
        assert torch.equal(a.view(torch.int16), r.view(torch.int16))
    with pytest.raises(ValueError, match="features"):
        G.fp8_heads_linear_f8(qkv[0].detach(), w[:, :512].contiguous())


def _nets(C, heads, n, dev):
    torch.manual_seed(5)
    net = AB.Net(C, heads, n).to(dev).to(torch.bfloat16)
    for blk in net.blocks:
        with torch.no_grad():
            blk.norm1.weight.add_(0.1 * torch.randn_like(blk.norm1.weight))
            blk.norm2.weight.add_(0.1 * torch.randn_like(blk.norm2.weight))
            blk.adaLN_modulation[0].weight.mul_(5.0)
    return net, copy.deepcopy(net)


def _run(net, x, c, mask):
    x = x.clone().requires_grad_()
    y = net(x, c, mask)
    y.backward(torch.ones_like(y) * 0.01)
    return [y, x.grad] + [p.grad for p in net.parameters()]


@pytest.mark.parametrize("recipe,C,heads", [("native3+heads", 1024, 16), ("native3+fused", 1024, 16),
                                             ("native3+fused", 896, 14)])
@pytest.mark.parametrize("masked", [False, True])
def test_converted_model_takes_the_heads_path(dev, recipe, C, heads, masked):
    """convert_fp8(net, recipe) against "native3" on the same weights: the output and every gradient bit for bit,
    with and without a key mask (scaled_dot_product_attention then writes o as [B, N, H, D] or [B, H, N, D]), while
    every proj takes the attention output directly. C = 896 is the d11 width (14 heads of 64)."""
    B, N = 8, 256
    net_u, net_f = _nets(C, heads, 2, dev)
    assert G.convert_fp8(net_u, "native3") == 8 and G.convert_fp8(net_f, recipe) == 8
    x = torch.randn(B, N, C, device=dev).to(torch.bfloat16)
    c = torch.randn(B, 1, C, device=dev).to(torch.bfloat16)
    mask = None
    if masked:
        mask = torch.ones(B, 1, 1, N, dtype=torch.bool, device=dev)
        mask[:, :, :, N - 40:] = False
    ru, rf = _run(net_u, x, c, mask), _run(net_f, x, c, mask)
    for a, r in zip(rf, ru):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           r.view(torch.int16) if r.dtype == torch.bfloat16 else r)
    assert all(type(b.attn.proj) is G.Fp8HeadsLinearF8 and b.attn.proj.heads_calls == 1 for b in net_f.blocks)
    if recipe == "native3+fused":
        assert all(type(b.attn.qkv_x) is G.Fp8NormLinearF8 for b in net_f.blocks)


def test_deep_copy_of_a_converted_model_runs_its_own_modules(dev):
    """A deep copy of a native3+fused model (as an EMA copy is made) gives the original's bits on the same weights,
    and after its own weights change only the copy's output changes: its rebound forwards use the copy's modules."""
    C, heads, B, N = 512, 8, 2, 64
    net, _ = _nets(C, heads, 2, dev)
    G.convert_fp8(net, "native3+fused")
    twin = copy.deepcopy(net)
    x = torch.randn(B, N, C, device=dev).to(torch.bfloat16)
    c = torch.randn(B, 1, C, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y0, y1 = net(x, c), twin(x, c)
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
        for b in twin.blocks:
            b.attn.proj.weight.mul_(0.5)
            b.mlp.w3.weight.mul_(0.5)
        y2, y3 = net(x, c), twin(x, c)
    assert torch.equal(y2.view(torch.int16), y0.view(torch.int16)) and not torch.equal(y3, y0)
    assert all(b.attn.proj.heads_calls == 2 for b in twin.blocks)


def test_compiled_converted_model_runs(dev):
    """torch.compile of a native3+fused model (as the reference compiles its blocks): the norm sites stay fused (the
    custom ops are traced opaque), the attention output takes the head-merging copy and the plain phase-3 proj (the
    pending result exists in eager mode only), and the output and gradients agree with the eager model's within the
    roundings the compiler may fuse differently (the block's elementwise ops)."""
    C, heads, B, N = 512, 8, 2, 64
    net, twin = _nets(C, heads, 2, dev)
    G.convert_fp8(net, "native3+fused")
    G.convert_fp8(twin, "native3+fused")
    comp = torch.compile(twin)
    x = torch.randn(B, N, C, device=dev).to(torch.bfloat16)
    c = torch.randn(B, 1, C, device=dev).to(torch.bfloat16)
    re, rc = _run(net, x, c, None), _run(comp, x, c, None)
    rel = lambda a, b: (torch.linalg.norm(a.float() - b.float()) / torch.linalg.norm(b.float())).item()
    for a, b in zip(rc, re):
        assert rel(a, b) < 1e-2
    assert all(b.attn.proj.heads_calls == 0 for b in twin.blocks)
    assert all(b.attn.proj.heads_calls == 1 for b in net.blocks)
