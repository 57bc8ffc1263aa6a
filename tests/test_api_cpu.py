"""Host-side logic of the drop-in API: the converters (GEMM counts, state-dict keys, phases), the torchao recipe
guard, the op registrations and fake kernels, the refusal of CPU tensors, and the reference() helper."""
import copy
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

import gpic_fp8 as G
from gpic_fp8 import fp8_native as F

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


class Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.qkv_x = nn.Linear(d, 3 * d, bias=False)
        self.kv_y = nn.Linear(d, 2 * d, bias=False)
        self.proj = nn.Linear(d, d)


class SwiGLU(nn.Module):
    """baselines/PixelGen/src/models/layers/swiglu.py:4-15"""
    def __init__(self, d, h):
        super().__init__()
        self.w12 = nn.Linear(d, 2 * h, bias=False)
        self.w3 = nn.Linear(h, d, bias=False)

    def forward(self, x):
        x1, x2 = self.w12(x).chunk(2, dim=-1)
        return self.w3(torch.nn.functional.silu(x1) * x2)


class Block(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = Attn(d)
        self.mlp = SwiGLU(d, 4 * d)
        self.adaLN_modulation = nn.Sequential(nn.Linear(d, 6 * d))


class TextAttn(nn.Module):
    """TextRefineAttention's linears (JiT_T2I.py:227,231)"""
    def __init__(self, d):
        super().__init__()
        self.qkv = nn.Linear(d, 3 * d, bias=False)
        self.proj = nn.Linear(d, d)


class TextBlock(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = TextAttn(d)
        self.mlp = SwiGLU(d, 4 * d)
        self.adaLN_modulation = nn.Sequential(nn.Linear(d, 6 * d))


class Net(nn.Module):
    def __init__(self, d=32, n=3):
        super().__init__()
        self.blocks = nn.ModuleList(Block(d) for _ in range(n))
        self.text_refine_blocks = nn.ModuleList(TextBlock(d) for _ in range(1))


@pytest.mark.parametrize("phase,per_block", [(1, 4), (2, 4), (3, 4)])
def test_convert_native_counts_and_keys(phase, per_block):
    net = Net()
    keys = set(net.state_dict())
    assert G.convert_native(net, phase=phase) == 3 * per_block
    assert set(net.state_dict()) == keys
    assert G.convert_native(net, phase=phase) == 0          # idempotent
    lin = {1: G.Fp8Linear, 2: G.Fp8Linear, 3: G.Fp8LinearF8}[phase]
    for b in net.blocks:
        assert type(b.attn.qkv_x) is lin and type(b.attn.proj) is lin
        assert type(b.attn.kv_y) is nn.Linear and type(b.adaLN_modulation[0]) is nn.Linear
        assert b.mlp._fp8
        assert (type(b.mlp.w12) is G.Fp8Linear) == (phase == 1)
    for b in net.text_refine_blocks:                          # image blocks only (fp8_native.py:294)
        assert type(b.attn.qkv) is nn.Linear and type(b.attn.proj) is nn.Linear and not getattr(b.mlp, "_fp8", False)


@pytest.mark.parametrize("phase,per_block,per_text", [(1, 5, 4), (2, 5, 4), (3, 5, 4)])
def test_convert_native_text_blocks(phase, per_block, per_text):
    """text=True: the image blocks' kv_y and the text-refine blocks' qkv, proj and MLP as well, in the same phase;
    state-dict keys unchanged; idempotent; adaLN untouched; a linear whose features are not multiples of 16 stays."""
    net = Net()
    net.text_refine_blocks[0].attn.odd = nn.Linear(32, 24)
    keys = set(net.state_dict())
    assert G.convert_native(net, phase=phase, text=True) == 3 * per_block + per_text
    assert set(net.state_dict()) == keys
    assert G.convert_native(net, phase=phase, text=True) == 0
    lin = {1: G.Fp8Linear, 2: G.Fp8Linear, 3: G.Fp8LinearF8}[phase]
    for b in net.blocks:
        assert type(b.attn.qkv_x) is lin and type(b.attn.kv_y) is lin and type(b.adaLN_modulation[0]) is nn.Linear
    t = net.text_refine_blocks[0]
    assert type(t.attn.qkv) is lin and type(t.attn.proj) is lin and t.mlp._fp8
    assert type(t.adaLN_modulation[0]) is nn.Linear and type(t.attn.odd) is nn.Linear


def test_convert_fp8_recipes(capsys):
    for recipe, n in (("native", 12), ("native2", 12), ("native3", 12), ("native3+text", 19)):
        assert G.convert_fp8(Net(), recipe) == n
    out = capsys.readouterr().out
    assert "GEMMs of the image blocks converted" in out and "GEMMs of the image and text blocks converted" in out
    net = Net()
    keys = {k: v.clone() for k, v in net.state_dict().items()}
    for recipe in ("tensorwise", "rowwise", "native4"):
        with pytest.raises(ValueError, match="native"):
            G.convert_fp8(net, recipe)
    # a refused recipe leaves the model untouched
    assert all(type(m) is nn.Linear for m in net.modules() if isinstance(m, nn.Linear))
    assert all(torch.equal(v, keys[k]) for k, v in net.state_dict().items())


def test_fp8_filter():
    net = Net(d=32)
    names = {n for n, m in net.named_modules() if G.fp8_filter(m, n)}
    assert "blocks.0.attn.qkv_x" in names and "text_refine_blocks.0.mlp.w3" in names
    assert not any("adaLN" in n for n in names)
    assert not G.fp8_filter(nn.Linear(24, 32), "blocks.0.x")


def test_ops_registered_with_reference_schemas():
    assert str(torch.ops.gpic.fp8_tcast.default._schema).startswith("gpic::fp8_tcast(Tensor x) -> (Tensor, Tensor)")
    assert "gpic::fp8_swiglu_tcast(Tensor z)" in str(torch.ops.gpic.fp8_swiglu_tcast.default._schema)
    assert "gpic::fp8_swiglu_bwd(Tensor z, Tensor da)" in str(torch.ops.gpic.fp8_swiglu_bwd.default._schema)


def test_fake_kernels_shapes():
    m = torch.empty(40, 48, device="meta", dtype=torch.bfloat16)
    q, s = torch.ops.gpic.fp8_tcast(m)
    assert q.shape == (40, 48) and q.dtype == torch.float8_e4m3fn and s.shape == (1,)
    q, qt, s = torch.ops.gpic.fp8_tcast_t(m)
    assert qt.shape == (48, 48)
    z = torch.empty(8, 64, device="meta", dtype=torch.bfloat16)
    q, s = torch.ops.gpic.fp8_swiglu_tcast(z)
    assert q.shape == (8, 32)
    dz, dq, s = torch.ops.gpic.fp8_swiglu_bwd(z, torch.empty(8, 32, device="meta", dtype=torch.bfloat16))
    assert dz.shape == (8, 64) and dq.dtype == torch.float8_e4m3fn
    a = torch.empty(8, 32, device="meta", dtype=torch.float8_e4m3fn)
    b = torch.empty(16, 32, device="meta", dtype=torch.float8_e4m3fn)
    c = torch.ops.gpic.fp8_gemm(a, torch.empty(1, device="meta"), b, torch.empty(1, device="meta"))
    assert c.shape == (8, 16) and c.dtype == torch.bfloat16


def test_cpu_tensors_are_refused():
    x = torch.randn(16, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        G.tcast(x)
    with pytest.raises(RuntimeError, match="GPU only"):
        G.fp8_linear(x, torch.randn(16, 16))


def test_reference_helper_matches_golden():
    """reference() (plain torch, CPU-capable) is within bf16 rounding of the IEEE-scale golden linear."""
    with np.load(GOLD, allow_pickle=False) as g:
        x = torch.from_numpy(g["lin_x"].view(np.int16)).view(torch.bfloat16)
        w = torch.from_numpy(g["lin_w"].view(np.int16)).view(torch.bfloat16)
        b = torch.from_numpy(g["lin_b"].view(np.int16)).view(torch.bfloat16)
        y = torch.from_numpy(g["lin_y"].view(np.int16)).view(torch.bfloat16)
    r = G.reference(x, w, b).float()
    assert torch.linalg.norm(r - y.float()) / torch.linalg.norm(y.float()) < 1e-2


class RMSNorm(nn.Module):
    """baselines/PixelGen/src/models/layers/rmsnorm.py: weight and variance_epsilon"""
    def __init__(self, d, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.variance_epsilon = eps


class NormBlock(Block):
    """FlattenDiTBlock's modules (JiT_T2I.py:189-198): norm1, attn, norm2, mlp, adaLN_modulation"""
    def __init__(self, d):
        super().__init__(d)
        self.norm1, self.norm2 = RMSNorm(d), RMSNorm(d)


class NormNet(nn.Module):
    def __init__(self, d=32, n=3):
        super().__init__()
        self.blocks = nn.ModuleList(NormBlock(d) for _ in range(n))
        self.text_refine_blocks = nn.ModuleList(TextBlock(d) for _ in range(1))


def test_convert_fused_norm():
    """native3+norm: the same GEMMs as native3, state-dict keys unchanged, each image block's qkv_x an
    Fp8NormLinearF8 and its forward rewired (idempotent); blocks without norm sites, and the text blocks, keep
    phase 3's plain linears; fused_norm outside phase 3 is refused."""
    net = NormNet()
    net.blocks.append(Block(32))                      # no norm1 / norm2: converted to phase 3, not rewired
    keys = set(net.state_dict())
    assert G.convert_fp8(net, "native3+norm") == 4 * 4
    assert set(net.state_dict()) == keys
    for b in net.blocks[:3]:
        assert type(b.attn.qkv_x) is G.Fp8NormLinearF8 and b._gpic_fused_norm and "forward" in b.__dict__
        assert type(b.attn.proj) is G.Fp8LinearF8 and b.mlp._fp8
    last = net.blocks[3]
    assert type(last.attn.qkv_x) is G.Fp8LinearF8 and "forward" not in last.__dict__
    assert G.convert_fused_norm(net) == 0
    twin = copy.deepcopy(net)                          # e.g. an EMA copy: its forwards run its own modules
    for b, t in zip(net.blocks[:3], twin.blocks[:3]):
        assert t.forward.__self__ is t and b.forward.__self__ is b
    assert G.convert_fp8(NormNet(), "native3+text+norm") == 3 * 5 + 4
    with pytest.raises(ValueError, match="phase 3"):
        G.convert_native(NormNet(), phase=2, fused_norm=True)
    wide = NormNet(d=4096, n=1)                         # wider than the norm's backward takes: not rewired
    G.convert_native(wide, phase=3, fused_norm=True)
    assert type(wide.blocks[0].attn.qkv_x) is G.Fp8LinearF8


def test_fp8_norm_linear_without_pending_norm_is_a_linear():
    """Fp8NormLinearF8 called without a pending norm is Fp8LinearF8 (here: refuses CPU tensors the same way), and
    a pending norm handed to another tensor raises."""
    lin = nn.Linear(32, 96, bias=False)
    lin.__class__ = G.Fp8NormLinearF8
    x = torch.randn(2, 8, 32, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        lin(x)
    marker = torch.empty(2, 8, 32, device="meta")
    lin._gpic_norm = (marker, x, torch.ones(32), x, x, 1e-6)
    with pytest.raises(RuntimeError, match="another tensor"):
        lin(x)
    assert "_gpic_norm" not in lin.__dict__


@pytest.mark.parametrize("res", [False, True])
def test_norm_reference_helper_close_to_oracle(res):
    """gpic_fp8.norm.reference (the model's eager ops, fused_norm.py:305-313, on CPU) agrees with the oracle's norm
    within the bf16 roundings the eager ops take separately (x + gate * a and n * (1 + scale) + shift rounded per
    operation instead of fused)."""
    from oracle import oracle as O
    B, N, C, eps = 2, 24, 896, 1e-6
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    a = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    gate = (torch.randn(B, 1, C, generator=g) * 0.5).to(torch.bfloat16)
    sh = (torch.randn(B, 1, C, generator=g) * 0.1).to(torch.bfloat16)
    sc = (torch.randn(B, 1, C, generator=g) * 0.1).to(torch.bfloat16)
    w = 1 + 0.1 * torch.randn(C, generator=g)
    xs, h = G.norm_reference(x, a, gate, w, sh, sc, eps, res)
    u = lambda t, r: t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(r, C)
    oxn, oh, _ = O.mod_rmsnorm(u(x, B * N), w.numpy(), u(sh, B), u(sc, B), N, eps, u(a, B * N) if res else None,
                               u(gate, B) if res else None)
    hf = torch.from_numpy(O.bf16_to_f32(oh)).view(B, N, C)
    assert (h.float() - hf).abs().max() <= 2 ** -6 * hf.abs().max()
    assert torch.linalg.norm(h.float() - hf) / torch.linalg.norm(hf) < 1e-2
    if res:
        xf = torch.from_numpy(O.bf16_to_f32(oxn)).view(B, N, C)
        assert torch.linalg.norm(xs.float() - xf) / torch.linalg.norm(xf) < 1e-2


def test_norm_width_checks_before_any_work():
    """A norm wider than the backward kernel takes (C > 2048) refuses gradients in the forward, before any kernel; with
    no gradient wanted it goes on to the (GPU-only) forward; widths that are no multiple of 4 are refused."""
    B, N, C = 1, 4, 2560
    x = torch.randn(B, N, C, dtype=torch.bfloat16)
    m = torch.zeros(B, 1, C, dtype=torch.bfloat16)
    w = torch.ones(C)
    with pytest.raises(ValueError, match="at most 2048"):
        G.mod_rmsnorm(x.clone().requires_grad_(), w, m, m, 1e-6)
    with pytest.raises(ValueError, match="at most 2048"):
        G.fp8_mod_rmsnorm_linear(x, w.clone().requires_grad_(), m, m, 1e-6, torch.zeros(16, C, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU only"):
        G.mod_rmsnorm(x, w, m, m, 1e-6)
    with pytest.raises(RuntimeError, match="GPU only"):   # (the device is checked first)
        G.res_mod_rmsnorm_q(x[..., :6], x[..., :6], m[..., :6], w[:6], m[..., :6], m[..., :6], 1e-6, True, True)


# ------------------------------------------------------------------------------------------------ attention output

def test_pending_heads_keeps_only_the_merge_pending():
    """The attention output handed back by a converted attention: transpose(1, 2) then reshape to [B, N, H D] stay
    pending; any other use gives exactly the eager tensor (attributes, methods, operators, torch functions)."""
    from gpic_fp8.heads import _PendingHeads
    o = torch.randn(2, 3, 5, 16)
    eager = o.transpose(1, 2).reshape(2, 5, 48)
    p = _PendingHeads(o, 0)
    t = p.transpose(1, 2)
    assert isinstance(t, _PendingHeads) and t.stage == 1
    assert isinstance(p.transpose(-3, -2), _PendingHeads)
    for shape in ((2, 5, 48), ((2, 5, 48),), (2, 5, -1), (torch.Size([2, 5, 48]),)):
        m = t.reshape(*shape)
        assert isinstance(m, _PendingHeads) and m.stage == 2 and torch.equal(m.materialize(), eager)
    assert torch.equal(t.reshape(10, 48), eager.reshape(10, 48))                 # another reshape: eager result
    assert torch.equal(p.transpose(2, 3), o.transpose(2, 3))                     # another transpose: eager result
    m = t.reshape(2, 5, 48)
    assert m.shape == eager.shape and m.dtype == o.dtype
    assert torch.equal(torch.add(m, 1), eager + 1) and torch.equal(m * 2, eager * 2) and torch.equal(2 * m, eager * 2)
    assert torch.equal(m[0], eager[0]) and torch.equal(-m, -eager)
    assert torch.equal(p + 0, o) and torch.equal(t.contiguous(), o.transpose(1, 2).contiguous())


def _sdpa_net(d=32, heads=2, n=2):
    import attn_blocks as AB

    class _B(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = AB.SdpaAttn(d, heads)
            self.mlp = SwiGLU(d, 4 * d)

    class _N(nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = nn.ModuleList(_B() for _ in range(n))
            self.text_refine_blocks = nn.ModuleList(TextBlock(d) for _ in range(1))
    return _N()


def test_convert_fused_heads(monkeypatch):
    """native3+heads: the same GEMMs and state-dict keys as native3; each attention whose forward calls
    scaled_dot_product_attention as `attention` gets an Fp8HeadsLinearF8 proj and a rebound forward (idempotent);
    attentions without such a forward keep phase 3's proj; outside phase 3 the option is refused. The rebound
    forward hands proj the attention output itself (fp8_heads_linear_f8 on o [B, H, N, D]) and reads every other
    global name from its module at call time. GEMMs stand in as plain linears (no GPU here)."""
    import attn_blocks as AB
    from gpic_fp8 import heads as HD
    net = _sdpa_net()
    ref = _sdpa_net()
    ref.load_state_dict(net.state_dict())
    keys = set(net.state_dict())
    assert G.convert_fp8(net, "native3+heads") == 2 * 4
    assert set(net.state_dict()) == keys
    for b in net.blocks:
        assert type(b.attn.proj) is G.Fp8HeadsLinearF8 and type(b.attn.qkv_x) is G.Fp8LinearF8
        assert b.attn._gpic_fused_heads and "forward" in b.attn.__dict__
    assert type(net.text_refine_blocks[0].attn.proj) is nn.Linear                 # image blocks only without text
    assert G.convert_fused_heads(net) == 0
    twin = copy.deepcopy(net)                          # e.g. an EMA copy: its forwards run its own modules
    for b, t in zip(net.blocks, twin.blocks):
        assert t.attn.forward.__self__ is t.attn and b.attn.forward.__self__ is b.attn
    with pytest.raises(ValueError, match="phase 3"):
        G.convert_native(_sdpa_net(), phase=2, fused_heads=True)
    plain = Net(n=1)                                                             # stand-in attention with no forward
    G.convert_native(plain, phase=3, fused_heads=True)
    assert type(plain.blocks[0].attn.proj) is G.Fp8LinearF8
    assert G.convert_fp8(_sdpa_net(), "native3+text+heads") == 2 * 4 + 4

    seen = []
    lin = lambda x, w, b=None, wcast=None: torch.nn.functional.linear(x, w, b)

    def heads_lin(o, w, b=None):
        seen.append(tuple(o.shape))
        B, H, N, D = o.shape
        return torch.nn.functional.linear(o.transpose(1, 2).reshape(B, N, H * D), w, b)
    monkeypatch.setattr(F, "fp8_linear_f8", lin)
    monkeypatch.setattr(HD, "fp8_linear_f8", lin)
    monkeypatch.setattr(HD, "fp8_heads_linear_f8", heads_lin)
    x = torch.randn(3, 7, 32)
    for b, r in zip(net.blocks, ref.blocks):
        assert torch.allclose(b.attn(x, None, None), r.attn(x, None, None), rtol=1e-6, atol=1e-6)
    assert seen == [(3, 2, 7, 16)] * 2 and [b.attn.proj.heads_calls for b in net.blocks] == [1, 1]
    g = net.blocks[0].attn._gpic_forward.__globals__
    assert g["nn"] is AB.nn and g["attention"] is not AB.attention
    monkeypatch.setattr(AB, "_gpic_probe", 5, raising=False)
    assert g["_gpic_probe"] == 5                                                 # module globals read live


def test_eager_calls_skip_the_dispatcher(monkeypatch):
    """The path's own calls (L.call) run an op's function directly in eager mode and the registered custom op while
    torch.compile traces; every op of the package is registered for it; any other callable is called as it is."""
    from gpic_fp8 import _lib as L
    from gpic_fp8 import norm as NM
    ops = [F.tcast, F.tcast_t, F.tcast_heads, F.tcast_t_group, F.swiglu_tcast, F.swiglu_tcast_t, F.swiglu_bwd,
           F.swiglu_bwd_q, F.swiglu_bwd_t, F.fp8_gemm, F.fp8_gemm_mn, NM.res_mod_rmsnorm_q, NM.res_mod_rmsnorm_bwd_k,
           NM.res_mod_rmsnorm_fwd, NM.res_mod_rmsnorm_bwd]
    assert all(op in L._IMPL for op in ops) and len(L._IMPL) == len(ops)
    seen = []
    monkeypatch.setitem(L._IMPL, F.tcast, lambda x: seen.append("direct") or "direct")
    x = torch.randn(4, 16)
    assert L.call(F.tcast, x) == "direct"
    monkeypatch.setattr(torch.compiler, "is_compiling", lambda: True)
    with pytest.raises(RuntimeError, match="GPU only"):     # the registered op (its kernel refuses CPU tensors)
        L.call(F.tcast, x)
    assert L.call(lambda t: "stand-in", x) == "stand-in" and seen == ["direct"]


def test_reference_norm_op_schemas():
    """The reference's norm ops exist under its names with its schemas (fused_norm.py:151-153,180-183), beside this
    build's own (the cast folded in)."""
    fwd = str(torch.ops.gpic.res_mod_rmsnorm_fwd.default._schema)
    bwd = str(torch.ops.gpic.res_mod_rmsnorm_bwd.default._schema)
    assert fwd.startswith("gpic::res_mod_rmsnorm_fwd(Tensor x, Tensor a, Tensor gate, Tensor w, Tensor shift, "
                          "Tensor scale, float eps, bool has_res) -> (Tensor, Tensor, Tensor)"), fwd
    assert bwd.startswith("gpic::res_mod_rmsnorm_bwd(Tensor dh, Tensor dxn, Tensor xn, Tensor a, Tensor gate, Tensor w, "
                          "Tensor scale, Tensor rstd, bool has_res, bool has_dxn) -> (Tensor, Tensor, Tensor, Tensor, "
                          "Tensor, Tensor)"), bwd
