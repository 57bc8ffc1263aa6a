"""Benchmark of the MI355X FP8 linear path (one GPU).

Workload (BASELINE.json metric "FP8 GEMM TFLOP/s + % FP8 MFMA peak, d12 block fwd+bwd @32768 tok", configs 3 + 4):
one step = the forward and backward of a width-1024 (d12) JiT-T2I image block's four FP8 linears at one GPU's share
of a step (128 images x 256 tokens = 32768 tokens), through the drop-in autograd API with every GEMM in FP8
(recipe "native3"): qkv_x (1024 -> 3072), proj (1024 -> 1024), and the SwiGLU MLP w12 (1024 -> 8192) + w3
(4096 -> 1024) -- 12 FP8 GEMMs (forward, dgrad, wgrad) = 3.2985 TFLOP, plus every cast, SwiGLU and transposing
kernel the path runs. Inputs are seeded synthetic tensors already in HBM: X ~ N(0,1), W ~ N(0, 1/K), dY ~ N(0, 1e-2),
bf16. value = 3.2985 TFLOP / measured step time.

Also measured live: the 12 GEMM launches alone (the roofline's dominant kernel, HIP events on the launch stream),
the config-2 cast ([32768 x 1024] bf16 -> e4m3, GB/s of algorithmic bytes), hipBLASLt's FP8 GEMM on the same 12
shapes via torch._scaled_mm (a comparator only), the MFMA rate the device sustains at 100% issue on real, random
and constant e4m3 operands (tests/hip/mfma_ceiling.hip: the power-limited ceiling the GEMM's fraction is read against),
and the CPU baseline (the oracle, a bounded sample).

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-compare]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-gpic_amd"))
sys.path.insert(0, ROOT)

METRIC = "FP8 GEMM TFLOP/s + % FP8 MFMA peak, d12 block fwd+bwd @32768 tok"
PEAK_FP8_TFLOPS = 5000.0      # MI355X dense FP8 MFMA (AMD spec)
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
M_TOK, C, H = 32768, 1024, 4096


def gemm_shapes(M=M_TOK, C=C, H=H):
    """(name, M, N, K) of the 12 GEMMs of one block's fwd + bwd (output [M, N], reduction K)."""
    lin = {"qkv": (C, 3 * C), "proj": (C, C), "w12": (C, 2 * H), "w3": (H, C)}
    out = []
    for name, (k, n) in lin.items():
        out.append((f"{name}.fwd", M, n, k))
        out.append((f"{name}.dgrad", M, k, n))
        out.append((f"{name}.wgrad", n, k, M))
    return out


def flops(shapes):
    return sum(2.0 * m * n * k for _, m, n, k in shapes)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-compare", action="store_true")
    p.add_argument("--copy-probe", action="store_true",
                   help="only copy a 1 GiB buffer (the known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--traffic", action="store_true",
                   help="only run each of the 12 GEMM shapes once, in the printed order (one counter row per shape)")
    p.add_argument("--cast-traffic", action="store_true",
                   help="only run the casts once each, in the printed order (one counter row per dispatch): config 2 "
                        "warm and with L2 / MALL flushed, an fp32 weight-shaped cast, the d12 SwiGLU casts, the "
                        "weights' grouped cast and the attention output's head-merging cast")
    p.add_argument("--step-only", type=int, default=0, metavar="N",
                   help="only run the d12 step N times (for a kernel-by-kernel trace of one step)")
    return p.parse_args()


def make_inputs(dev, seed=0, C=C, H=H, outliers=0.0, M=M_TOK):
    """The block's inputs: X ~ N(0,1), W ~ N(0, 1/K), dY ~ N(0, 1e-2), bf16. With `outliers`, that fraction of the
    activation channels (the same columns in every X) is scaled by 50 before the bf16 rounding (config 5)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    cols = torch.randperm(C, generator=g, device=dev)[:round(outliers * C)]

    def bf(*shape, std=1.0):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16)

    def act():
        x = torch.randn(M, C, generator=g, device=dev)
        x[:, cols] *= 50.0
        return x.to(torch.bfloat16)

    t = {
        "x_qkv": act(), "x_proj": act(), "x_mlp": act(),
        "w_qkv": bf(3 * C, C, std=C ** -0.5), "w_proj": bf(C, C, std=C ** -0.5),
        "w12": bf(2 * H, C, std=C ** -0.5), "w3": bf(C, H, std=H ** -0.5),
        "dy_qkv": bf(M, 3 * C, std=0.1), "dy_proj": bf(M, C, std=0.1), "dy_mlp": bf(M, C, std=0.1),
    }
    for k in ("x_qkv", "x_proj", "x_mlp", "w_qkv", "w_proj", "w12", "w3"):
        t[k].requires_grad_(True)
    return t


def step(G, t):
    """The block's four weights are cast together first (one launch; the same bytes as casting each inside its
    linear), then the FP8 linears fwd + bwd."""
    import torch
    c_qkv, c_proj, c12, c3 = G.weight_casts(t["w_qkv"], t["w_proj"], t["w12"], t["w3"])
    y1 = G.fp8_linear_f8(t["x_qkv"], t["w_qkv"], wcast=c_qkv)
    y2 = G.fp8_linear_f8(t["x_proj"], t["w_proj"], wcast=c_proj)
    y3 = G.fp8_mlp_f8(t["x_mlp"], t["w12"], t["w3"], w12cast=c12, w3cast=c3)
    torch.autograd.backward([y1, y2, y3], [t["dy_qkv"], t["dy_proj"], t["dy_mlp"]])


def config2_input(dev):
    """Config 2: X [32768 x 1024] fp32 N(0,1) (seed 1), 1% of the columns x50, rounded once to bf16."""
    import torch
    gx = torch.Generator().manual_seed(1)
    xc = torch.randn(M_TOK, C, generator=gx)
    cols = torch.randperm(C, generator=gx)[:round(0.01 * C)]
    xc[:, cols] *= 50.0
    return xc.to(torch.bfloat16).to(dev)


def cast_traffic(G, dev):
    """Each cast once, for counter collection (one row per dispatch, in this order): config 2 (a warm-up call, then a
    warm one, then one after a 512 MB write that flushes L2 / MALL), an fp32 weight [3072 x 1024] (DDP weights are
    fp32), the dY of qkv [32768 x 3072] (the step's largest flat cast), the d12 SwiGLU casts of the step: the
    product cast of z [32768 x 8192] and the backward's dz cast, the step's four bf16 weights in one grouped
    transposing cast, and the attention output's cast with its head merge folded in (tcast_heads of o
    [128 x 16 x 256 x 64] as the flash backend writes it, [B, H, N, D] in memory)."""
    import torch
    xc = config2_input(dev)
    flush = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    w32 = torch.randn(3 * C, C, generator=g, device=dev) * C ** -0.5
    z = torch.randn(M_TOK, 2 * H, generator=g, device=dev).to(torch.bfloat16)
    da = (torch.randn(M_TOK, H, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    dqkv = (torch.randn(M_TOK, 3 * C, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    wts = [(torch.randn(r, c, generator=g, device=dev) * c ** -0.5).to(torch.bfloat16)
           for r, c in ((3 * C, C), (C, C), (2 * H, C), (C, H))]
    o = torch.randn(M_TOK // 256, 16, 256, C // 16, generator=g, device=dev).to(torch.bfloat16)
    order = []
    for name, fn in (("config2 warm-up", lambda: G.tcast(xc)), ("config2 warm", lambda: G.tcast(xc)),
                     ("flush", lambda: flush.fill_(1)), ("config2 flushed", lambda: G.tcast(xc)),
                     ("fp32 weight [3072 x 1024]", lambda: G.tcast(w32)),
                     ("qkv dY [32768 x 3072]", lambda: G.tcast(dqkv)),
                     ("swiglu product cast z [32768 x 8192]", lambda: G.swiglu_tcast(z)),
                     ("swiglu backward dz cast", lambda: G.swiglu_bwd_q(z, da)),
                     ("d12 weights, grouped transposing cast", lambda: G.tcast_t_group(wts)),
                     ("attention output [128 x 16 x 256 x 64] (tcast_heads)", lambda: G.tcast_heads(o))):
        fn()
        torch.cuda.synchronize()
        order.append(name)
    print(json.dumps({"cast_order": order}), flush=True)


def time_region(fn, steps, warmup):
    """ms per call of fn, HIP events on the current stream around `steps` calls after `warmup` untimed ones."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def time_device(fn, steps, warmup):
    """ms per call of fn on the device alone: the calls are issued while filler work (elementwise passes over a
    1 GiB buffer) holds the stream, and the events bracket the calls, so the host's issue time does not show -- the
    time a host that issues ahead of the GPU would see. The filler is doubled until it outlasts the issuing (checked:
    its event has not completed when the last call is issued); None if it never does."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    issue_ms = (time.perf_counter() - t0) * 1e3
    torch.cuda.synchronize()
    buf = torch.empty(1 << 28, device="cuda")
    buf.mul_(1.0)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    buf.mul_(1.0)
    e.record()
    torch.cuda.synchronize()
    n = max(4, int(2.0 * steps * issue_ms / max(s.elapsed_time(e), 1e-3)) + 1)
    for _ in range(4):
        for _ in range(n):
            buf.mul_(1.0)
        s.record()
        for _ in range(steps):
            fn()
        ahead = not s.query()
        e.record()
        torch.cuda.synchronize()
        if ahead:
            return s.elapsed_time(e) / steps
        n *= 2
    return None


def gemm_operands(G, dev, shapes):
    """e4m3 operands of each shape in the layout the step gives them: forward and dgrad GEMMs K-major (a [M, K],
    b [N, K]: fp8_gemm); wgrads MN-major, the untransposed output gradient and input over the tokens (a [K, M],
    b [K, N]: fp8_gemm_mn)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(1)
    ops = []
    for name, m, n, k in shapes:
        mn = name.endswith(".wgrad")
        a = (torch.randn(*((k, m) if mn else (m, k)), generator=g, device=dev)).to(torch.bfloat16)
        b = (torch.randn(*((k, n) if mn else (n, k)), generator=g, device=dev) / k ** 0.5).to(torch.bfloat16)
        aq, sa = G.tcast(a)
        bq, sb = G.tcast(b)
        ops.append((mn, aq, sa, bq, sb))
        del a, b
    return ops


def run_gemm(G, op):
    mn, aq, sa, bq, sb = op
    if mn:
        return G.fp8_gemm_mn(aq, sa, bq, sb)
    return G.fp8_gemm(aq, sa, bq, sb, None, False)


def gemm_sclk(fn, seconds=1.5, samples=3):
    """The shader clock while fn (one pass of the 12 GEMMs) runs back to back for about `seconds`: `amd-smi metric
    --clock` read `samples` times from a helper thread after the first 0.3 s, the mean over every XCD's GFX clock and
    every sample, in MHz. None when amd-smi is missing or its output cannot be read (the figure is then not reported)."""
    import shutil
    import subprocess
    import threading
    import torch
    exe = shutil.which("amd-smi")
    if exe is None:
        return None
    idx = torch.cuda.current_device()
    vals, stop = [], threading.Event()

    def sample():
        time.sleep(0.3)
        for _ in range(samples):
            if stop.is_set():
                return
            try:
                r = subprocess.run([exe, "metric", "-g", str(idx), "--clock", "--json"], capture_output=True, text=True,
                                   timeout=5)
                d = json.loads(r.stdout)
                d = d["gpu_data"][0] if isinstance(d, dict) and "gpu_data" in d else (d[0] if isinstance(d, list) else d)
                clk = d["clock"]
                vals.extend(float(v["clk"]["value"]) for k, v in clk.items() if k.startswith("gfx"))
            except Exception:   # a missing or changed output format: no figure
                return

    t = threading.Thread(target=sample, daemon=True)
    t0 = time.perf_counter()
    t.start()
    n = 0
    while (time.perf_counter() - t0 < seconds or t.is_alive()) and n < 100000:
        fn()
        n += 1
        if n % 20 == 0:
            torch.cuda.synchronize()   # keep the queue short so the clock is read while GEMMs run
    stop.set()
    torch.cuda.synchronize()
    t.join(timeout=15)
    return round(sum(vals) / len(vals), 1) if vals else None


def norm_sites(G, dev, B=128, N=256, eps=1e-6):
    """The two norm sites of a d12 block over one GPU's 32768 tokens: fused (the norm kernel writes h's e4m3 bytes
    and scale; h never exists in bf16) against unfused (the norm writes bf16 h, then tcast reads it), device time, with
    the bytes each design moves (HBM minimum: x, a read, x_new, h / hq written; 4 bytes of rstd per row)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16)
    a = torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16)
    mod = (torch.randn(B, 1, 6 * C, generator=g, device=dev) * 0.2).to(torch.bfloat16)
    sh, sc, gate = mod[..., :C], mod[..., C:2 * C], mod[..., 2 * C:3 * C]
    w = 1 + 0.1 * torch.randn(C, generator=g, device=dev)
    q = G.res_mod_rmsnorm_q
    t = {
        "site1_fused": time_device(lambda: q(x, x, x, w, sh, sc, eps, False, False), 20, 3),
        "site1_unfused": time_device(lambda: G.tcast(q(x, x, x, w, sh, sc, eps, False, True, False)[1]), 20, 3),
        "site2_fused": time_device(lambda: q(x, a, gate, w, sh, sc, eps, True, False), 20, 3),
        "site2_unfused": time_device(lambda: G.tcast(q(x, a, gate, w, sh, sc, eps, True, True, False)[1]), 20, 3),
    }
    n, rows = B * N * C, B * N
    by = {"site1_fused": n * 3 + rows * 4, "site1_unfused": n * 7 + rows * 4,
          "site2_fused": n * 7 + rows * 4, "site2_unfused": n * 11 + rows * 4}
    out = {"workload": f"d12 norm sites over {rows} tokens (C {C}): site 1 RMSNorm + modulation, site 2 residual add + "
                       "RMSNorm + modulation; fused: h's e4m3 + scale from the norm kernel, unfused: the norm writes bf16 "
                       "h, tcast reads it (device time)"}
    for k, ms in t.items():
        out[k + "_us"] = round(ms * 1e3, 2) if ms else None
        out[k + "_bytes"] = by[k]
        out[k + "_GBs"] = round(by[k] / ms / 1e6, 1) if ms else None
    for site in ("site1", "site2"):
        if t[site + "_fused"] and t[site + "_unfused"]:
            out[site + "_speedup"] = round(t[site + "_unfused"] / t[site + "_fused"], 3)
            out[site + "_fused_frac_hbm"] = round(by[site + "_fused"] / t[site + "_fused"] / 1e6 / PEAK_HBM_GBS, 4)
    return out


def heads_site(G, dev, B=128, N=256):
    """The attention output feeding proj in a d12 block over one GPU's 32768 tokens (16 heads of 64), as the flash
    backend of scaled_dot_product_attention writes it ([B, H, N, D] in memory): fused (tcast_heads reads o in its own
    layout and writes proj's e4m3 input) against unfused (the head-merging copy o.transpose(1, 2).reshape(B, N, C),
    then tcast), device time, with the bytes each moves (fused: o read, e4m3 written; unfused: o read and written by
    the copy, read again and cast)."""
    import torch
    H = 16
    D = C // H
    g = torch.Generator(device=dev).manual_seed(13)
    o = torch.randn(B, H, N, D, generator=g, device=dev).to(torch.bfloat16)
    t = {"fused": time_device(lambda: G.tcast_heads(o), 20, 3),
         "unfused": time_device(lambda: G.tcast(o.transpose(1, 2).reshape(B, N, C)), 20, 3)}
    n = B * N * C
    by = {"fused": n * 3, "unfused": n * 7}
    out = {"workload": f"d12 attention output [{B} x {H} x {N} x {D}] bf16 ([B, H, N, D] in memory) -> proj's e4m3 "
                       "input [32768 x 1024] + scale: tcast_heads (fused) against the head-merging copy then tcast "
                       "(device time)"}
    for k, ms in t.items():
        out[k + "_us"] = round(ms * 1e3, 2) if ms else None
        out[k + "_bytes"] = by[k]
        out[k + "_GBs"] = round(by[k] / ms / 1e6, 1) if ms else None
    if t["fused"] and t["unfused"]:
        out["speedup"] = round(t["unfused"] / t["fused"], 3)
        out["fused_frac_hbm"] = round(by["fused"] / t["fused"] / 1e6 / PEAK_HBM_GBS, 4)
    return out


def norm_block(G, dev, B=128, N=256, eps=1e-6, steps=20):
    """The d12 block's two norm sites with the FP8 linears they feed, fwd + bwd over 32768 tokens (site 1 -> qkv_x,
    site 2 -> the SwiGLU MLP; every GEMM FP8): fused (the norm kernel writes h's e4m3 bytes, h never exists in bf16:
    fp8_mod_rmsnorm_linear, fp8_res_mod_rmsnorm_mlp) against unfused (mod_rmsnorm / res_mod_rmsnorm write bf16 h,
    then fp8_linear_f8 / fp8_mlp_f8 cast it). Both give the same bits; ms per step, alternating runs."""
    import torch
    g = torch.Generator(device=dev).manual_seed(12)

    def bf(*shape, std=1.0, grad=True):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(grad)

    x, a = bf(B, N, C), bf(B, N, C)
    mod = bf(B, 1, 6 * C, std=0.2)
    wn1 = (1 + 0.1 * torch.randn(C, generator=g, device=dev)).requires_grad_()
    wn2 = (1 + 0.1 * torch.randn(C, generator=g, device=dev)).requires_grad_()
    wqkv, w12, w3 = bf(3 * C, C, std=C ** -0.5), bf(2 * H, C, std=C ** -0.5), bf(C, H, std=H ** -0.5)
    dy1, dy3, dxn = bf(B, N, 3 * C, std=0.1, grad=False), bf(B, N, C, std=0.1, grad=False), \
        bf(B, N, C, std=0.1, grad=False)

    def run(fused):
        sh1, sc1, sh2, sc2, g2 = (mod[..., i * C:(i + 1) * C] for i in range(5))
        if fused:
            y1 = G.fp8_mod_rmsnorm_linear(x, wn1, sh1, sc1, eps, wqkv)
            xn, y3 = G.fp8_res_mod_rmsnorm_mlp(x, a, g2, wn2, sh2, sc2, eps, w12, w3)
        else:
            y1 = G.fp8_linear_f8(G.mod_rmsnorm(x, wn1, sh1, sc1, eps), wqkv)
            xn, h2 = G.res_mod_rmsnorm(x, a, g2, wn2, sh2, sc2, eps)
            y3 = G.fp8_mlp_f8(h2, w12, w3)
        torch.autograd.backward([y1, xn, y3], [dy1, dxn, dy3])

    t = {"fused": [], "unfused": []}
    for _ in range(2):
        for k in ("fused", "unfused"):
            t[k].append(time_region(lambda: run(k == "fused"), steps, 3))
    f, u = min(t["fused"]), min(t["unfused"])
    return {"workload": f"d12 block: both norm sites and the FP8 linears they feed (qkv_x, SwiGLU MLP), fwd + bwd over "
                        f"{B * N} tokens; fused: the norm kernels write h's e4m3 bytes; unfused: bf16 h, then the "
                        f"linears cast it (ms per step, best of 2 alternating runs of {steps})",
            "fused_ms": round(f, 4), "unfused_ms": round(u, 4), "saved_us": round((u - f) * 1e3, 1)}


def block_producers(G, dev, B=128, N=256, heads=16, eps=1e-6, steps=10):
    """A d12 block's lever-K forward + backward over 32768 tokens (JiT_T2I.py:201-207 with the attention of :166-186
    minus the q / k norms and the rotary embedding): both norm sites, qkv_x, scaled_dot_product_attention (flash
    backend), proj (with bias), the residual and the SwiGLU MLP, every GEMM FP8. Fused (recipe native3+fused's path):
    the norm kernels write h's e4m3 bytes and proj casts the attention output in its own layout; unfused (native3's):
    the norms write bf16 h, the attention output is copied to [B, N, C], and the linears cast both. The same bits
    either way; ms per step, best of 2 alternating runs."""
    import torch
    D = C // heads
    g = torch.Generator(device=dev).manual_seed(14)

    def bf(*shape, std=1.0, grad=True):
        return (torch.randn(*shape, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(grad)

    x = bf(B, N, C)
    mod = bf(B, 1, 6 * C, std=0.2)
    wn1 = (1 + 0.1 * torch.randn(C, generator=g, device=dev)).requires_grad_()
    wn2 = (1 + 0.1 * torch.randn(C, generator=g, device=dev)).requires_grad_()
    wqkv, wproj, bproj = bf(3 * C, C, std=C ** -0.5), bf(C, C, std=C ** -0.5), bf(C, std=0.1)
    w12, w3 = bf(2 * H, C, std=C ** -0.5), bf(C, H, std=H ** -0.5)
    dy = bf(B, N, C, std=0.1, grad=False)

    def run(fused):
        sh1, sc1, g1, sh2, sc2, g2 = (mod[..., i * C:(i + 1) * C] for i in range(6))
        if fused:
            qkv = G.fp8_mod_rmsnorm_linear(x, wn1, sh1, sc1, eps, wqkv)
        else:
            qkv = G.fp8_linear_f8(G.mod_rmsnorm(x, wn1, sh1, sc1, eps), wqkv)
        q, k, v = (t.contiguous() for t in qkv.view(B, N, 3, heads, D).permute(2, 0, 3, 1, 4))
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v)
        if fused:
            a = G.fp8_heads_linear_f8(o, wproj, bproj)
            xn, y = G.fp8_res_mod_rmsnorm_mlp(x, a, g1, wn2, sh2, sc2, eps, w12, w3)
        else:
            a = G.fp8_linear_f8(o.transpose(1, 2).reshape(B, N, C), wproj, bproj)
            xn, h2 = G.res_mod_rmsnorm(x, a, g1, wn2, sh2, sc2, eps)
            y = G.fp8_mlp_f8(h2, w12, w3)
        (xn + g2 * y).backward(dy)

    t = {"fused": [], "unfused": []}
    for _ in range(2):
        for k in ("fused", "unfused"):
            t[k].append(time_region(lambda: run(k == "fused"), steps, 2))
    f, u = min(t["fused"]), min(t["unfused"])
    return {"workload": f"d12 lever-K block fwd + bwd over {B * N} tokens ({heads} heads of {D}; attention by "
                        "scaled_dot_product_attention, no q / k norms or rotary embedding): native3+fused's path "
                        "(norm sites writing h's e4m3 bytes, proj casting the attention output in its own layout) "
                        f"against native3's (ms per step, best of 2 alternating runs of {steps})",
            "fused_ms": round(f, 4), "unfused_ms": round(u, 4), "saved_us": round((u - f) * 1e3, 1)}


def mfma_ceiling(G, dev):
    """The FP8 MFMA rate the device sustains at 100% issue (tests/hip/mfma_ceiling.hip: every SIMD issuing MFMAs back to
    back, no memory traffic), measured live, in the 16 x 16 x 128 form the GEMM uses on three kinds of operands -- the
    e4m3 bytes of an N(0, 1) tensor as a GEMM sees them ("tcast_randn"), uniformly random bytes ("random"), constant
    bytes ("const") -- and in the 32 x 32 x 64 form on the first ("tcast_randn_32x32x64"). Operands whose bits toggle
    draw enough power that the clock drops below the 2.4 GHz of the published peak. Each figure is the better of two
    runs (the first one also lets the clock settle). None if the measurement library has not been built."""
    import ctypes
    import torch
    path = os.path.join(ROOT, "tests", "hip", "libmfma_ceiling.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    d = ctypes.c_double
    lib.gpic_probe_mfma_ceiling.argtypes = ([ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int] +
                                            [ctypes.POINTER(d)] * 4)
    g = torch.Generator(device=dev).manual_seed(11)
    q = G.tcast(torch.randn(4096, 4096, generator=g, device=dev).to(torch.bfloat16))[0].view(torch.uint8)
    out = {}
    for name, shape, rnd, src in (("tcast_randn", 16, 0, q), ("random", 16, 1, None), ("const", 16, 0, None),
                                  ("tcast_randn_32x32x64", 32, 0, q)):
        best = None
        for _ in range(2):
            ms, tf, ghz, busy = d(), d(), d(), d()
            if lib.gpic_probe_mfma_ceiling(shape, rnd, None if src is None else src.data_ptr(),
                                           0 if src is None else src.numel(), 8000, ms, tf, ghz, busy) != 0:
                return None
            if best is None or tf.value > best[0]:
                best = (tf.value, ghz.value, busy.value)
        out[name] = {"TFLOPs": round(best[0], 1), "clock_GHz": round(best[1], 3), "mfma_busy": round(best[2], 4)}
    return out


def hbm_floor(dev, read_bytes, write_bytes, runs=15):
    """How long one launch takes just to read `read_bytes` from HBM, just to write `write_bytes`, and to do both with a
    cast's traffic pattern (each workgroup writing as soon as its own reads are in), with L2 / MALL flushed before each
    launch as for the cast (tests/hip/hbm_floor.hip; the best of its launch shapes, median of `runs` event-timed
    launches). A single-pass cast moves the same bytes and must also agree on the maximum across the chip before its
    first write, so the read-and-write launch is a floor under it. None if the measurement library has not been
    built."""
    import ctypes
    import torch
    path = os.path.join(ROOT, "tests", "hip", "libhbm_floor.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.gpic_probe_hbm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                   ctypes.c_void_p]
    lib.gpic_probe_hbm_groups.argtypes = [ctypes.c_int, ctypes.c_uint64]
    lib.gpic_probe_hbm_rw.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    src = torch.ones(read_bytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty(write_bytes // 4, dtype=torch.float32, device=dev)
    out = torch.empty(max(lib.gpic_probe_hbm_groups(2, read_bytes), 1), dtype=torch.int32, device=dev)
    flush = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    shapes = {0: "1024 threads x 16 words", 1: "512 x 16", 2: "256 x 8", 3: "512 x 32"}
    best = {}
    calls = {"read": lambda cfg: lib.gpic_probe_hbm(1, cfg, src.data_ptr(), read_bytes, out.data_ptr(), st),
             "write": lambda cfg: lib.gpic_probe_hbm(0, cfg, dst.data_ptr(), write_bytes, None, st),
             "read_write": lambda cfg: lib.gpic_probe_hbm_rw(cfg, src.data_ptr(), read_bytes, dst.data_ptr(), st)}
    for key, call in calls.items():
        for cfg in shapes:
            times = []
            for _ in range(runs):
                flush.fill_(1)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                if call(cfg) != 0:
                    return None
                e1.record()
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1e3)
            us = sorted(times)[len(times) // 2]
            if key not in best or us < best[key][0]:
                best[key] = (us, shapes[cfg])
    del flush, src, dst
    r, w, rw = best["read"], best["write"], best["read_write"]
    return {"read_us": round(r[0], 2), "read_shape": r[1], "read_GBs": round(read_bytes / r[0] / 1e3, 1),
            "write_us": round(w[0], 2), "write_shape": w[1], "write_GBs": round(write_bytes / w[0] / 1e3, 1),
            "read_write_us": round(rw[0], 2), "read_write_shape": rw[1],
            "read_write_GBs": round((read_bytes + write_bytes) / rw[0] / 1e3, 1)}


def gemm_source_sha():
    """Hash of gemm.hip's code: each line with its // comment and trailing blanks removed, blank lines dropped, so
    that comment edits do not make the measured traffic look stale."""
    import hashlib
    import re
    with open(os.path.join(ROOT, "nano-gpic_amd", "csrc", "gemm.hip")) as f:
        lines = [re.sub(r"\s*//.*$", "", ln).rstrip() for ln in f]
    return hashlib.sha256("\n".join(ln for ln in lines if ln).encode()).hexdigest()[:16]


def gemm_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (profiles/gemm_d12_traffic.json), or None when that summary was measured on another version of the GEMM source
    than the one built here (its recorded hash differs): a stale figure is not reported."""
    tpath = os.path.join(ROOT, "profiles", "gemm_d12_traffic.json")
    if not os.path.exists(tpath):
        return None
    with open(tpath) as f:
        t = json.load(f)
    if t.get("gemm_source_sha") != gemm_source_sha():
        return None
    return t.get("traffic_bytes_per_launch")


def cpu_threads():
    """Threads for the CPU baseline: the CPUs this process may run on, capped by OMP_NUM_THREADS where the host sets
    it (the GPU boxes grant each job a share of their cores and set it to that share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model():
    """The host CPU's model string as lscpu reports it (its "Model name", and "BIOS Model name" when that says more),
    else /proc/cpuinfo's."""
    import subprocess
    names = []
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "BIOS Model name") and v.strip() and v.strip() not in names:
                names.append(v.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    if not names:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        names.append(line.split(":", 1)[1].strip())
                        break
        except OSError:
            pass
    return " / ".join(names) or None


def median_s(fn, runs):
    """Median wall time in seconds of `runs` calls of fn after one warm-up call."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(runs=3, sample_tokens=None):
    """The reference path on the host's cores in torch CPU ops (the oracle's torch restatement: reference()'s fp32
    product of dequantized e4m3 operands, the casts with IEEE scales, the eager SwiGLU expressions): config 1 at full
    size, and the d12 block step of this benchmark (every GEMM in FP8, as on the GPU) at the GPU's size, all 32768
    tokens (`sample_tokens` to run fewer); median of `runs` timed runs after a warm-up, with all the threads this
    process is granted."""
    import torch
    from oracle import oracle as O
    threads = cpu_threads()
    torch.set_num_threads(threads)

    g = torch.Generator().manual_seed(0)                    # config 1: X [4096 x 768], W [768 x 768]
    X = torch.randn(4096, 768, generator=g).to(torch.bfloat16)
    W = (torch.randn(768, 768, generator=g) / 768 ** 0.5).to(torch.bfloat16)

    def config1():
        xq, sx = O.torch_tcast(X)
        wq, sw = O.torch_tcast(W)
        return O.torch_mm(xq, sx, wq, sw)
    c1 = median_s(config1, max(runs, 7))

    Ms = sample_tokens or M_TOK
    g = torch.Generator().manual_seed(0)

    def bf(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    x = {k: bf(Ms, C) for k in ("qkv", "proj", "mlp")}
    w = {"qkv": bf(3 * C, C, std=C ** -0.5), "proj": bf(C, C, std=C ** -0.5)}
    w12, w3 = bf(2 * H, C, std=C ** -0.5), bf(C, H, std=H ** -0.5)
    dy = {"qkv": bf(Ms, 3 * C, std=0.1), "proj": bf(Ms, C, std=0.1), "mlp": bf(Ms, C, std=0.1)}
    mm, tc = O.torch_mm, O.torch_tcast

    def step():
        for k in ("qkv", "proj"):
            xq, sx = tc(x[k])
            wq, sw = tc(w[k])
            mm(xq, sx, wq, sw)                                   # forward
            dyq, sdy = tc(dy[k])
            mm(dyq, sdy, wq.t(), sw)                             # dgrad (w's bytes transposed)
            mm(dyq.t(), sdy, xq.t(), sx)                         # wgrad
        xq, sx = tc(x["mlp"])
        w12q, s12 = tc(w12)
        w3q, s3 = tc(w3)
        z = mm(xq, sx, w12q, s12)
        aq, sa = O.torch_swiglu_tcast(z)
        mm(aq, sa, w3q, s3)
        dyq, sdy = tc(dy["mlp"])
        da = mm(dyq, sdy, w3q.t(), s3)
        mm(dyq.t(), sdy, aq.t(), sa)                             # dw3
        _, dzq, sdz = O.torch_swiglu_bwd(z, da)
        mm(dzq, sdz, w12q.t(), s12)                              # dx
        mm(dzq.t(), sdz, xq.t(), sx)                             # dw12

    sec = median_s(step, runs)
    fl = flops(gemm_shapes(M=Ms))
    return {"value": round(fl / sec / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"d12 block fwd+bwd FP8 linear path (the step of this benchmark, every GEMM FP8) on {Ms} of the "
                      f"{M_TOK} tokens (the GPU's configuration{'' if Ms == M_TOK else ', sampled'}) in torch CPU ops "
                      f"(reference()'s fp32 product of dequantized e4m3 operands, IEEE-scaled casts, eager SwiGLU); "
                      f"median of {runs} runs after a warm-up",
            "tokens": Ms, "ms_per_step": round(sec * 1e3, 1), "gemm_tflop_per_step": round(fl / 1e12, 4),
            "config1_ms": round(c1 * 1e3, 2),
            "config1_workload": "X [4096 x 768] . W [768 x 768] seed 0: two casts + fp32 product -> bf16 (4.83 GFLOP)",
            "config1_gflops": round(2.0 * 4096 * 768 * 768 / c1 / 1e9, 1),
            "threads": threads, "os_cpu_count": os.cpu_count(), "cpu_model": cpu_model()}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import gpic_fp8 as G
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_each_way": src.numel() * 4, "launches": 3}), flush=True)
        return

    if args.cast_traffic:
        cast_traffic(G, dev)
        return

    if args.traffic:
        shapes = gemm_shapes()
        ops = gemm_operands(G, dev, shapes)
        for op in ops:
            run_gemm(G, op)
            torch.cuda.synchronize()
        print(json.dumps({"gemm_order": [name for name, *_ in shapes]}), flush=True)
        return

    # ---- the step: the whole FP8 linear path of a d12 block, fwd + bwd
    t = make_inputs(dev)

    def run():
        for v in t.values():
            v.grad = None
        step(G, t)

    if args.step_only:
        for _ in range(args.step_only):
            run()
        torch.cuda.synchronize()
        print(json.dumps({"steps_run": args.step_only}), flush=True)
        return

    shapes = gemm_shapes()
    fl = flops(shapes)
    ms = time_region(run, args.steps, args.warmup)

    # ---- the 12 GEMM launches alone (dominant kernel), same shapes
    ops = gemm_operands(G, dev, shapes)

    def gemms():
        for op in ops:
            run_gemm(G, op)

    gemm_ms = time_region(gemms, max(args.steps, 10), 3)
    sclk = gemm_sclk(gemms)   # after the timed passes: the reading does not touch them
    per_shape = {}
    for (name, m, n, k), op in zip(shapes, ops):
        tm = time_region(lambda: run_gemm(G, op), 10, 2)
        per_shape[name] = {"M": m, "N": n, "K": k, "us": round(tm * 1e3, 1),
                           "tflops": round(2.0 * m * n * k / tm / 1e9, 1)}

    # ---- config 2: the cast alone
    xc = config2_input(dev)
    cast_ms = time_region(lambda: G.tcast(xc), 50, 10)
    cast_bytes = xc.numel() * 3 + 4
    # the same with L2 / MALL flushed before each call (a 512 MB write between the timed launches)
    flush = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device=dev)
    cold = []
    for _ in range(20):
        flush.fill_(1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        G.tcast(xc)
        e1.record()
        e1.synchronize()
        cold.append(e0.elapsed_time(e1))
    cast_cold_ms = sorted(cold)[len(cold) // 2]
    del flush
    # the floor under any single-pass cast of config 2: one launch reading its 64 MiB, one writing its 32 MiB
    floor = hbm_floor(dev, xc.numel() * 2, xc.numel())

    # ---- the other casts: an fp32 weight-shaped tensor (DDP keeps fp32 weights) and the d12 SwiGLU casts of the step,
    # as device time (short kernels: Python's issue time would show in a back-to-back loop)
    gc = torch.Generator(device=dev).manual_seed(3)
    w32 = torch.randn(3 * C, C, generator=gc, device=dev) * C ** -0.5
    w32_ms = time_device(lambda: G.tcast(w32), 20, 3)
    z = torch.randn(M_TOK, 2 * H, generator=gc, device=dev).to(torch.bfloat16)
    da = (torch.randn(M_TOK, H, generator=gc, device=dev) * 0.1).to(torch.bfloat16)
    sw_ms = time_device(lambda: G.swiglu_tcast(z), 10, 2)
    swb_ms = time_device(lambda: G.swiglu_bwd_q(z, da), 10, 2)
    del z, da
    w32_bytes = w32.numel() * 5 + 4
    # product cast, min: read z, write q; as built: the single pass holds 384 KiB of the product per CU and writes and
    # reads back the rest
    sw_held = min(M_TOK * H * 2, 384 * 1024 * torch.cuda.get_device_properties(dev).multi_processor_count)
    sw_min = M_TOK * H * 5
    sw_moved = sw_min + 2 * (M_TOK * H * 2 - sw_held)
    # backward dz cast, min: read z, da, write dzq; as built: the single pass holds 320 KiB of dz per CU (read once)
    # and reads z and da twice for the rest
    swb_held = min(M_TOK * H * 4, 320 * 1024 * torch.cuda.get_device_properties(dev).multi_processor_count)
    swb_min = M_TOK * H * 8
    swb_moved = swb_min + (M_TOK * H * 4 - swb_held) * 6 // 4

    # ---- the norm sites' producer with the cast folded in: site 1 (RMSNorm + modulation -> qkv_x) and site 2 (x + gate
    # * a, RMSNorm + modulation -> the MLP) at d12, h's e4m3 bytes from the norm kernel (fused) against the norm
    # writing bf16 h and tcast(h) reading it back (unfused), device time
    norm = norm_sites(G, dev)
    nblock = norm_block(G, dev)
    # ---- the attention output's producer: proj's e4m3 input read from o [B, H, N, D] in its own layout
    heads = heads_site(G, dev)
    # ---- a whole lever-K block with both producers fused against native3's path
    pblock = block_producers(G, dev)

    # ---- config 5: the d18 block (C = 1792, H = 7168) with 1% outlier activation channels, fwd + bwd
    C18, H18 = 1792, 7168
    t18 = make_inputs(dev, seed=5, C=C18, H=H18, outliers=0.01)

    def run18():
        for v in t18.values():
            v.grad = None
        step(G, t18)

    fl18 = flops(gemm_shapes(M_TOK, C18, H18))
    ms18 = time_region(run18, 5, 2)
    del t18

    # ---- a text-refine block's linears (recipe native3+text): 128 captions x 51.5 tokens = 6592 rows, fwd + bwd
    MT = 6592
    tt = make_inputs(dev, seed=7, M=MT)

    def run_text():
        for v in tt.values():
            v.grad = None
        step(G, tt)

    fl_t = flops(gemm_shapes(MT))
    ms_t = time_region(run_text, 10, 3)
    # Its kernels are short (12-60 us GEMMs): Python's autograd issues a step in about as long as the GPU runs it, so
    # the wall time above depends on the host CPU; the device time is measured with the launches queued ahead.
    ms_t_dev = time_device(run_text, 10, 0)
    # and captured in a CUDA graph, as the reference runs its blocks (reduce-overhead): the same step replayed, its
    # gradients checked bit for bit against an eager step's
    ms_t_graph = None
    try:
        run_text()
        ref = {k: v.grad.clone() for k, v in tt.items() if v.grad is not None}
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(3):
                run_text()
        torch.cuda.current_stream(dev).wait_stream(side)
        for v in tt.values():
            v.grad = None
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(G, tt)
        graph.replay()
        torch.cuda.synchronize()
        if all(torch.equal(tt[k].grad.view(torch.int16), r.view(torch.int16)) for k, r in ref.items()):
            ms_t_graph = time_region(graph.replay, 10, 3)
        del graph
    except RuntimeError as e:   # reported as null, with the reason on stderr
        print(f"text block graph capture failed: {e}", file=sys.stderr, flush=True)
    del tt

    # ---- comparator: hipBLASLt FP8 GEMM (torch._scaled_mm) on the same shapes
    hip = None
    if not args.no_compare:
        try:
            # hipBLASLt takes A row-major and B column-major: the wgrads get transposed copies (outside the timing)
            tn = [(aq.t().contiguous(), sa, bq.t().contiguous(), sb) if mn else (aq, sa, bq, sb)
                  for mn, aq, sa, bq, sb in ops]

            def blaslt():
                for aq, sa, bq, sb in tn:
                    torch._scaled_mm(aq, bq.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
            hip_ms = time_region(blaslt, max(args.steps, 10), 3)
            hip = {"gemm_tflops": round(fl / hip_ms / 1e9, 1), "gemm_ms": round(hip_ms, 4)}
        except Exception as e:     # a comparator only
            hip = {"error": f"{type(e).__name__}: {str(e)[:200]}"}
    del ops

    ceiling = mfma_ceiling(G, dev)
    cpu = None if args.no_cpu else cpu_baseline()
    gemm_tflops = fl / gemm_ms / 1e9
    traffic = gemm_traffic()
    out = {
        "metric": METRIC,
        "value": round(fl / ms / 1e9, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {"workload": "d12 JiT-T2I image block, FP8 linear path fwd+bwd (recipe native3: qkv_x, proj, "
                               "w12+SwiGLU+w3; 12 FP8 GEMMs + all casts), one GPU's 32768 tokens",
                   "tokens": M_TOK, "width": C, "swiglu_hidden": H, "gemm_tflop_per_step": round(fl / 1e12, 4)},
        "pct_fp8_peak": round(100.0 * fl / ms / 1e9 / PEAK_FP8_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": PEAK_FP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_FP8_TFLOPS, 4), "traffic": traffic,
                     "kernel": "gemm_tn_kernel (K-major fwd / dgrad, MN-major wgrad instances; + split-K reduce)",
                     "launches_per_step": len(shapes),
                     "avg_launch_us": round(gemm_ms * 1e3 / len(shapes), 1), "gemm_ms_per_step": round(gemm_ms, 4),
                     "per_shape": per_shape,
                     "mfma_ceiling": ceiling,
                     "frac_of_data_ceiling": round(gemm_tflops / ceiling["tcast_randn"]["TFLOPs"], 4) if ceiling else None,
                     # the same against the peak at the shader clock amd-smi reported while the 12 GEMMs ran
                     "sclk_mhz_during_gemms": sclk,
                     "peak_at_sclk": round(PEAK_FP8_TFLOPS * sclk / 2400.0, 1) if sclk else None,
                     "frac_at_sclk": round(gemm_tflops / (PEAK_FP8_TFLOPS * sclk / 2400.0), 4) if sclk else None},
        "cast": {"workload": "config 2: [32768 x 1024] bf16 -> e4m3 + amax + scale, L2 / MALL flushed before each "
                             "call (a 512 MB write; median of 20); the warm figures are back-to-back calls",
                 "us": round(cast_cold_ms * 1e3, 2), "achieved_GBs": round(cast_bytes / cast_cold_ms / 1e6, 1),
                 "peak_GBs": PEAK_HBM_GBS, "frac": round(cast_bytes / cast_cold_ms / 1e6 / PEAK_HBM_GBS, 4),
                 "algorithmic_bytes": cast_bytes, "us_warm": round(cast_ms * 1e3, 2),
                 "frac_warm": round(cast_bytes / cast_ms / 1e6 / PEAK_HBM_GBS, 4),
                 # launches that only read the 64 MiB, only write the 32 MiB, or do both without the cast's
                 # cross-chip maximum, flushed the same way: the last is a floor under any single pass
                 "hbm_floor": floor,
                 "frac_of_floor": round(floor["read_write_us"] / (cast_cold_ms * 1e3), 4) if floor else None},
        "cast_fp32_weight": {"workload": "fp32 [3072 x 1024] -> e4m3 + amax + scale (a DDP weight)",
                             "us": round(w32_ms * 1e3, 2) if w32_ms else None, "algorithmic_bytes": w32_bytes,
                             "achieved_GBs": round(w32_bytes / w32_ms / 1e6, 1) if w32_ms else None},
        "swiglu": {"workload": "d12 SwiGLU casts: product cast of z [32768 x 8192] and the backward's dz cast "
                               "(z, da [32768 x 4096]), device time",
                   "fwd_us": round(sw_ms * 1e3, 1) if sw_ms else None, "fwd_min_bytes": sw_min,
                   "fwd_moved_bytes": sw_moved,
                   "fwd_GBs_moved": round(sw_moved / sw_ms / 1e6, 1) if sw_ms else None,
                   "fwd_frac_min": round(sw_min / sw_ms / 1e6 / PEAK_HBM_GBS, 4) if sw_ms else None,
                   "bwd_us": round(swb_ms * 1e3, 1) if swb_ms else None, "bwd_min_bytes": swb_min,
                   "bwd_moved_bytes": swb_moved,
                   "bwd_GBs_moved": round(swb_moved / swb_ms / 1e6, 1) if swb_ms else None,
                   "bwd_frac_min": round(swb_min / swb_ms / 1e6 / PEAK_HBM_GBS, 4) if swb_ms else None},
        "norm_sites": norm,
        "norm_block": nblock,
        "heads_site": heads,
        "block_producers": pblock,
        "d18_block": {"workload": "config 5: d18 block (C 1792, H 7168), 1% outlier channels x50, fwd+bwd, native3",
                      "ms": round(ms18, 4), "gemm_tflop": round(fl18 / 1e12, 4),
                      "tflops": round(fl18 / ms18 / 1e9, 1)},
        "text_block": {"workload": "text-refine block linears (qkv, proj, SwiGLU MLP) fwd+bwd, native3+text, "
                                   f"M = {MT} (128 captions x 51.5 tokens)", "ms": round(ms_t, 4),
                       "gemm_tflop": round(fl_t / 1e12, 4), "tflops": round(fl_t / ms_t / 1e9, 1),
                       "device_ms": round(ms_t_dev, 4) if ms_t_dev else None,
                       "device_tflops": round(fl_t / ms_t_dev / 1e9, 1) if ms_t_dev else None,
                       "graph_ms": round(ms_t_graph, 4) if ms_t_graph else None,
                       "graph_tflops": round(fl_t / ms_t_graph / 1e9, 1) if ms_t_graph else None},
        "hipblaslt_compare": hip,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
