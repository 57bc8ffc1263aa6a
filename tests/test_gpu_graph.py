"""The casts and the phase-3 linear under CUDA/HIP graph capture and replay, and a converted block under
torch.compile(mode="reduce-overhead") (cudagraph trees), as the reference runs its blocks with lever X
(baselines/PixelGen/src/utils/fsdp_setup.py:92-98,143-145).

A single-pass cast tags its partial maxima with a call number that the kernels read from, and advance in, the
workspace on the device, so each replay of a captured cast takes a new number: the replays below alternate inputs
whose maxima differ by orders of magnitude, with a zero wait bound (a partial not yet published is read again or
computed, never waited for), so a word left by the previous replay under a repeated number would give a wrong amax.
Every replay is checked against the oracle (bytes and scale bit for bit) and against the eager call."""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def qb(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


@pytest.fixture
def knob():
    yield
    L.set_single_pass(True, -1)


def fill(t, seed, scale):
    g = torch.Generator(device=t.device).manual_seed(seed)
    t.copy_((torch.randn(t.shape, generator=g, device=t.device) * scale).to(t.dtype))


# (flat x, transposed w) shapes: config 2's single pass and the [32768 x 3072] dY of qkv (flat hybrid), with a
# weight-shaped transposing cast and a larger transposing hybrid
SHAPES = [((32768, 1024), (3072, 1024)), ((32768, 3072), (32768, 3072))]


@pytest.mark.parametrize("xs,ws", SHAPES)
@pytest.mark.parametrize("wait", [-1, 0])
def test_casts_replayed(dev, knob, xs, ws, wait):
    """tcast and tcast_t captured on a stream that has already cast (its workspace and epoch exist), replayed 4 times
    on that stream with new values copied into the static inputs (maxima alternating between ~1e3 and ~1e-3), with
    eager casts between the replays on the same stream (ordered after the replay: they share its workspace) and on
    the default stream (another workspace): every replay equals the oracle."""
    L.set_single_pass(True, wait)
    x = torch.empty(xs, dtype=torch.bfloat16, device=dev)
    w = torch.empty(ws, dtype=torch.bfloat16, device=dev)
    fill(x, 1, 1.0)
    fill(w, 2, 1.0)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(2):
            G.tcast(x)
            G.tcast_t(w)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        q, sx = G.tcast(x)
        wq, wqt, sw = G.tcast_t(w)
    other = torch.randn(4096, 1024, device=dev).to(torch.bfloat16)
    for rep, scale in enumerate((1e3, 1e-3, 3e2, 2e-3)):
        fill(x, 10 + rep, scale)
        fill(w, 20 + rep, 1.0 / scale)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()                     # the graph's casts use the capture stream's workspace: replayed there,
            G.tcast(other)                 # then eager work on the same workspace, in stream order
        G.tcast(other)
        torch.cuda.synchronize()
        oq, od, _ = O.tcast(bits(x))
        assert sx.item() == od, (rep, sx.item(), od)
        assert np.array_equal(qb(q), oq), f"replay {rep}: x bytes differ"
        oq, od, _ = O.tcast(bits(w))
        assert sw.item() == od, (rep, sw.item(), od)
        assert np.array_equal(qb(wq), oq), f"replay {rep}: w bytes differ"
        r16 = (ws[0] + 15) // 16 * 16
        assert wqt.shape == (ws[1], r16)
        assert np.array_equal(qb(wqt)[:, :ws[0]], oq.T)


@pytest.mark.parametrize("M", [2048, 16384])
@pytest.mark.parametrize("wait", [-1, 0])
def test_swiglu_casts_replayed(dev, knob, M, wait):
    """The single-pass SwiGLU casts (the product cast and the backward's dz cast, H = 4096) captured on a stream that
    has already run them and replayed 4 times with new z and da copied in (maxima alternating by orders of magnitude),
    eager SwiGLU casts between the replays on the same stream: every replay equals the eager result of the same
    inputs through the forced two-pass path. M = 2048 holds everything on chip; M = 16384 is a hybrid of both (the
    product streamed through the op's buffer, dz computed twice); M = 2048 also against the oracle."""
    H = 4096
    L.set_single_pass(True, wait)
    z = torch.empty(M, 2 * H, dtype=torch.bfloat16, device=dev)
    da = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    fill(z, 1, 1.0)
    fill(da, 2, 0.01)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(2):
            G.swiglu_tcast(z)
            G.swiglu_bwd_q(z, da)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        aq, sa = G.swiglu_tcast(z)
        dq, sd = G.swiglu_bwd_q(z, da)
    zo = torch.randn(1024, 2 * H, device=dev).to(torch.bfloat16)
    dao = torch.randn(1024, H, device=dev).to(torch.bfloat16)
    for rep, scale in enumerate((1e2, 1e-2, 3e1, 2e-2)):
        fill(z, 10 + rep, scale)
        fill(da, 20 + rep, 1e-2 / scale)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
            G.swiglu_tcast(zo)             # eager work on the graph's workspace, in stream order
            G.swiglu_bwd_q(zo, dao)
        torch.cuda.synchronize()
        L.set_single_pass(False, -1)
        raq, rsa = G.swiglu_tcast(z)
        rdq, rsd = G.swiglu_bwd_q(z, da)
        L.set_single_pass(True, wait)
        assert sa.item() == rsa.item() and torch.equal(aq.view(torch.uint8), raq.view(torch.uint8)), f"replay {rep}"
        assert sd.item() == rsd.item() and torch.equal(dq.view(torch.uint8), rdq.view(torch.uint8)), f"replay {rep}"
        if M == 2048:
            oq, od, _ = O.swiglu_tcast(bits(z))
            assert sa.item() == od and np.array_equal(qb(aq), oq), f"replay {rep}: product bytes differ"


def test_cast_captured_on_a_new_stream(dev, knob):
    """A stream with no workspace yet: the workspace is created during the capture (from the capture's memory pool,
    its zero fill recorded as a kernel node that clears it again on each replay) and every replay still matches the
    oracle."""
    L.set_single_pass(True, 0)
    x = torch.empty(8192, 1024, dtype=torch.bfloat16, device=dev)
    fill(x, 3, 1.0)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.graph(g, stream=s):
        q, sx = G.tcast(x)
        q2, sx2 = G.tcast(x)             # two calls in one graph: consecutive numbers within a replay
    for rep, scale in enumerate((5.0, 1e-4, 7e3)):
        fill(x, 30 + rep, scale)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        oq, od, _ = O.tcast(bits(x))
        for qq, ss in ((q, sx), (q2, sx2)):
            assert ss.item() == od and np.array_equal(qb(qq), oq), f"replay {rep}"


def test_linear_fwd_bwd_replayed(dev, knob):
    """One fp8_linear_f8 forward + backward (phase 3: FP8 forward, dgrad and wgrad; tcast, tcast_t, GEMM, MN-major
    wgrad) captured whole, replayed 3 times with new inputs and output gradients: output and gradients bit-identical
    to the eager computation on the same values, which matches the oracle's GEMM of the same bytes."""
    L.set_single_pass(True, 0)
    M, K, N = 4096, 1024, 3072
    x = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    w = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
    dy = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    fill(x, 4, 1.0)
    fill(w, 5, K ** -0.5)
    fill(dy, 6, 0.1)
    xs = x.clone().requires_grad_()
    ws = w.clone().requires_grad_()
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):                      # warm-up on the capture stream, as torch.cuda.graph asks
        for _ in range(2):
            G.fp8_linear_f8(xs, ws).backward(dy)
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    xs.grad = ws.grad = None
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = G.fp8_linear_f8(xs, ws)
        y.backward(dy)
    for rep, scale in enumerate((1.0, 1e-3, 40.0)):
        with torch.no_grad():
            fill(x, 40 + rep, scale)
            fill(w, 50 + rep, K ** -0.5 / scale)
            fill(dy, 60 + rep, 0.1 * scale)
            xs.copy_(x)
            ws.copy_(w)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        xe = x.clone().requires_grad_()
        we = w.clone().requires_grad_()
        ye = G.fp8_linear_f8(xe, we)
        ye.backward(dy)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ye.view(torch.int16)), f"replay {rep}: y"
        assert torch.equal(xs.grad.view(torch.int16), xe.grad.view(torch.int16)), f"replay {rep}: dx"
        assert torch.equal(ws.grad.view(torch.int16), we.grad.view(torch.int16)), f"replay {rep}: dw"
        # the forward against the oracle: casts bit for bit, the GEMM within the tolerance of the scaled matmul
        oxq, osx, _ = O.tcast(bits(x))
        owq, osw, _ = O.tcast(bits(w))
        ref = O.mm64(oxq, osx, owq, osw)
        assert O.rel_fro(y.detach().float().cpu().numpy(), ref) < 4e-3


class _Attn(torch.nn.Module):
    def __init__(self, c):
        super().__init__()
        self.qkv_x = torch.nn.Linear(c, 3 * c, bias=False)
        self.proj = torch.nn.Linear(c, c)


class _SwiGLU(torch.nn.Module):
    def __init__(self, c, h):
        super().__init__()
        self.w12 = torch.nn.Linear(c, 2 * h, bias=False)
        self.w3 = torch.nn.Linear(h, c, bias=False)

    def forward(self, x):
        z = self.w12(x)
        z1, z2 = z.chunk(2, -1)
        return self.w3(torch.nn.functional.silu(z1) * z2)


class _Block(torch.nn.Module):
    """The linears of a JiT-T2I block in the reference's module structure (attn.qkv_x, attn.proj, mlp.w12, mlp.w3),
    with a stand-in for attention (the q slice)."""
    def __init__(self, c, h):
        super().__init__()
        self.attn = _Attn(c)
        self.mlp = _SwiGLU(c, h)

    def forward(self, x):
        # one add outside the FP8 ops: a fused chain of adds would round once in the compiled code and once per add
        # eagerly, which is not what is tested here
        c = x.shape[-1]
        return self.attn.proj(self.attn.qkv_x(x)[..., :c]) + self.mlp(x)


class _Net(torch.nn.Module):
    def __init__(self, c, h):
        super().__init__()
        self.blocks = torch.nn.ModuleList([_Block(c, h)])

    def forward(self, x):
        return self.blocks[0](x)


@pytest.mark.timeout(900)
def test_compiled_block_reduce_overhead_matches_eager(dev, knob):
    """A block converted with recipe native3, compiled with mode="reduce-overhead" (cudagraph trees: warm-up, record,
    replays), against the same converted block run eagerly on the same weights: output and every gradient equal to
    the bit on each of 4 steps with new inputs (the FP8 ops are opaque to the compiler and deterministic)."""
    torch.manual_seed(0)
    C, H, B, T = 256, 512, 4, 256
    ref = _Net(C, H).to(dev).to(torch.bfloat16)
    net = _Net(C, H).to(dev).to(torch.bfloat16)
    net.load_state_dict(ref.state_dict())
    assert G.convert_fp8(ref, "native3") == 4 and G.convert_fp8(net, "native3") == 4
    from torch._dynamo.utils import counters
    counters.clear()
    block = net.blocks[0]
    block.compile(mode="reduce-overhead")
    for step in range(4):
        g = torch.Generator(device=dev).manual_seed(100 + step)
        x = (torch.randn(B, T, C, generator=g, device=dev) * (1 + 10 * step)).to(torch.bfloat16)
        dy = (torch.randn(B, T, C, generator=g, device=dev) * 0.1).to(torch.bfloat16)
        xe = x.clone().requires_grad_()
        xc = x.clone().requires_grad_()
        ye = ref(xe)
        ye.backward(dy)
        yc = net(xc)
        yc.backward(dy)
        torch.cuda.synchronize()
        assert torch.equal(yc.view(torch.int16), ye.view(torch.int16)), f"step {step}: y"
        assert torch.equal(xc.grad.view(torch.int16), xe.grad.view(torch.int16)), f"step {step}: dx"
        for (n, p), (_, pe) in zip(net.named_parameters(), ref.named_parameters()):
            assert torch.equal(p.grad.view(torch.int16), pe.grad.view(torch.int16)), f"step {step}: {n}"
            p.grad = None
            pe.grad = None
    assert not counters["inductor"].get("cudagraph_skips"), dict(counters["inductor"])
