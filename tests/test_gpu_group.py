"""The grouped transposing cast (gpic_fp8_tcast_t_group): the same bytes and scales as tcast_t on each tensor, one
launch where the tensors fit the device together and the per-tensor calls where they do not; and the phase-3 linear
and MLP with their weights cast beforehand, bit for bit the same as casting them inside."""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture
def knob():
    yield
    L.set_single_pass(True, -1)


def qb(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def tensors(dev, shapes, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for i, (r, c) in enumerate(shapes):
        x = torch.randn(r, c, generator=g, device=dev) * 10.0 ** (i % 5 - 2)   # maxima 4 orders apart
        out.append(x.to(dtype))
    return out


D12 = [(3072, 1024), (1024, 1024), (8192, 1024), (1024, 4096)]
GROUPS = [
    D12,                                            # one launch, one tile per workgroup (1024 tiles)
    D12 + [(2048, 1024)],                           # one launch, two tiles per workgroup
    [(1000, 272), (33, 16), (4100, 1040)],          # ragged rows and columns, partial tiles
    [(16, 16)],                                     # one tensor, one workgroup
    [(5376, 1792), (1792, 1792), (14336, 1792), (1792, 7168)],   # d18: too large together, per-tensor calls
    [(64, 32)] * 9,                                 # more than the 8 a launch takes
    [(256, 64), (0, 64), (128, 32)],                # an empty tensor: per-tensor calls
]


@pytest.mark.parametrize("shapes", GROUPS, ids=lambda s: f"{len(s)}x{s[0][0]}x{s[0][1]}")
@pytest.mark.parametrize("wait", [-1, 0, None])
def test_group_matches_per_tensor(dev, knob, shapes, wait):
    """Every (q, qt, dequant) equals tcast_t's, bit for bit; with a zero wait bound every partial not yet published is
    computed by the waiting workgroup from its own tensor (the ranged fold's index within the tensor); with the single
    pass switched off (None) the group makes the two-pass per-tensor calls."""
    L.set_single_pass(wait is not None, -1 if wait is None else wait)
    xs = tensors(dev, shapes, 5)
    if len(xs) > 2 and xs[2].numel():
        xs[2][0, 0] = float("nan")                  # a NaN leaves that tensor's amax (and no other's) unchanged
    got = G.weight_casts(*xs)
    for x, (q, qt, s) in zip(xs, got):
        q0, qt0, s0 = G.tcast_t(x)
        assert torch.equal(s, s0), (tuple(x.shape), s.item(), s0.item())
        assert np.array_equal(qb(q), qb(q0)) and np.array_equal(qb(qt), qb(qt0)), tuple(x.shape)


def test_group_matches_oracle(dev, knob):
    """The d12 weights' group against the oracle's cast (bytes and scale) and its transpose."""
    xs = tensors(dev, D12, 7)
    for x, (q, qt, s) in zip(xs, G.weight_casts(*xs)):
        oq, od, _ = O.tcast(x.view(torch.int16).cpu().numpy().view(np.uint16))
        assert np.float32(s.item()) == od
        assert np.array_equal(qb(q), oq)
        R = x.shape[0]
        qtn = qb(qt)
        assert np.array_equal(qtn[:, :R], oq.T) and not qtn[:, R:].any()


def test_group_fp32_and_mixed(dev, knob):
    """fp32 weights (per-tensor calls) and a bf16 / fp32 mix (read as fp32) give tcast_t's bytes."""
    xs = tensors(dev, D12[:2], 9, torch.float32) + tensors(dev, D12[2:3], 9)
    for x, (q, qt, s) in zip(xs, G.weight_casts(*xs)):
        q0, qt0, s0 = G.tcast_t(x)
        assert torch.equal(s, s0) and np.array_equal(qb(q), qb(q0)) and np.array_equal(qb(qt), qb(qt0))


def test_linear_and_mlp_with_weight_casts(dev, knob):
    """fp8_linear_f8 / fp8_mlp_f8 with the weights cast beforehand (one grouped call) equal the calls that cast them
    inside: outputs and every gradient bit for bit."""
    g = torch.Generator(device=dev).manual_seed(11)
    M, C, H = 4096, 1024, 4096
    def bf(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16)
    base = {"x1": bf(M, C), "x2": bf(M, C), "w": bf(3 * C, C, std=C ** -0.5), "w12": bf(2 * H, C, std=C ** -0.5),
            "w3": bf(C, H, std=H ** -0.5), "d1": bf(M, 3 * C, std=0.1), "d2": bf(M, C, std=0.1)}
    res = []
    for pre in (False, True):
        t = {k: v.clone().requires_grad_(k in ("x1", "x2", "w", "w12", "w3")) for k, v in base.items()}
        if pre:
            cw, c12, c3 = G.weight_casts(t["w"], t["w12"], t["w3"])
            y1 = G.fp8_linear_f8(t["x1"], t["w"], wcast=cw)
            y2 = G.fp8_mlp_f8(t["x2"], t["w12"], t["w3"], w12cast=c12, w3cast=c3)
        else:
            y1 = G.fp8_linear_f8(t["x1"], t["w"])
            y2 = G.fp8_mlp_f8(t["x2"], t["w12"], t["w3"])
        torch.autograd.backward([y1, y2], [t["d1"], t["d2"]])
        res.append([y1, y2] + [t[k].grad for k in ("x1", "x2", "w", "w12", "w3")])
    for a, b in zip(*res):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_weight_cast_shape_checked(dev):
    w = torch.zeros(64, 32, dtype=torch.bfloat16, device=dev)
    x = torch.zeros(16, 32, dtype=torch.bfloat16, device=dev)
    (c,) = G.weight_casts(torch.zeros(32, 64, dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):
        G.fp8_linear_f8(x, w, wcast=c)


def test_stale_weight_cast_refused(dev):
    """A WeightCast taken before an in-place update of its weight (an optimizer step), or taken from another tensor of
    the same shape, is refused; cast again, it is accepted and gives tcast_t's result; a plain (q, qt, dequant) tuple is
    checked by shape only."""
    g = torch.Generator(device=dev).manual_seed(3)
    w = (torch.randn(64, 32, generator=g, device=dev) / 32 ** 0.5).to(torch.bfloat16)
    x = torch.randn(16, 32, generator=g, device=dev).to(torch.bfloat16)
    (c,) = G.weight_casts(w)
    y0 = G.fp8_linear_f8(x, w, wcast=c)
    with torch.no_grad():
        w.mul_(2.0)                                   # the update
    with pytest.raises(ValueError, match="last update"):
        G.fp8_linear_f8(x, w, wcast=c)
    with pytest.raises(ValueError, match="another weight"):
        G.fp8_linear_f8(x, w.clone(), wcast=G.weight_casts(w)[0])
    (c2,) = G.weight_casts(w)
    y1 = G.fp8_linear_f8(x, w, wcast=c2)
    assert torch.equal(y1.view(torch.int16), G.fp8_linear_f8(x, w).view(torch.int16))
    # w x 2: the same bytes with twice the scale, so exactly twice the output (power-of-two scaling rounds exactly)
    assert torch.equal(y1.view(torch.int16), (y0.float() * 2).to(torch.bfloat16).view(torch.int16))
    assert torch.equal(G.fp8_linear_f8(x, w, wcast=tuple(c)).view(torch.int16), y0.view(torch.int16))


@pytest.mark.parametrize("wait", [-1, 0])
def test_group_replayed(dev, knob, wait):
    """The grouped cast captured in a graph on a stream that has already cast, replayed 4 times with new values
    (maxima alternating between ~1e3 and ~1e-3) copied into its inputs, each replay followed on that stream by eager
    tcast_t calls: every replay gives their bytes and scales."""
    L.set_single_pass(True, wait)
    xs = tensors(dev, D12, 13)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.tcast_t_group(xs)   # the stream's workspace exists before the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = G.tcast_t_group(xs)
    for rep in range(4):
        new = tensors(dev, D12, 100 + rep)
        with torch.cuda.stream(s):
            for x, y in zip(xs, new):
                x.copy_(y * (1e3 if rep % 2 else 1e-3))
            graph.replay()
            got = [t.clone() for t in out]
            ref = [G.tcast_t(x) for x in xs]
        torch.cuda.synchronize()
        for i, (q0, qt0, s0) in enumerate(ref):
            assert torch.equal(got[3 * i + 2], s0), (rep, i)
            assert np.array_equal(qb(got[3 * i]), qb(q0)) and np.array_equal(qb(got[3 * i + 1]), qb(qt0)), (rep, i)
