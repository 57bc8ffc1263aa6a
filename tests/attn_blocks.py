"""Stand-in modules for the attention-output tests: an attention whose forward calls scaled_dot_product_attention by
the module-level name `attention` and hands proj the head-merged output (the shape of JiT_T2I.py:8,183-186), and a
block / net around it with the lever-K norm sites (JiT_T2I.py:201-207), so that the converters' fused paths can be
compared with the plain phase-3 conversion on the same weights."""
import torch
import torch.nn as nn

import gpic_fp8 as G

attention = torch.nn.functional.scaled_dot_product_attention


class RMSNorm(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.variance_epsilon = 1e-6


class SdpaAttn(nn.Module):
    """qkv_x (no bias) -> q, k, v [B, H, N, D] -> attention -> o.transpose(1, 2).reshape(B, N, C) -> proj."""
    def __init__(self, d, heads):
        super().__init__()
        self.num_heads = heads
        self.qkv_x = nn.Linear(d, 3 * d, bias=False)
        self.proj = nn.Linear(d, d)

    def forward(self, x, y, pos, mask=None):
        B, N, C = x.shape
        qkv = self.qkv_x(x).reshape(B, N, 3, self.num_heads, C // self.num_heads).permute(2, 0, 3, 1, 4)
        q, k, v = qkv[0].contiguous(), qkv[1].contiguous(), qkv[2].contiguous()
        x = attention(q, k, v) if mask is None else attention(q, k, v, attn_mask=mask)
        x = x.transpose(1, 2).reshape(B, N, C)
        return self.proj(x)


class MLP(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.w12 = nn.Linear(d, 2 * h, bias=False)
        self.w3 = nn.Linear(h, d, bias=False)

    def forward(self, x):
        x1, x2 = self.w12(x).chunk(2, dim=-1)
        return self.w3(torch.nn.functional.silu(x1) * x2)


class Block(nn.Module):
    def __init__(self, d, heads):
        super().__init__()
        self.norm1 = RMSNorm(d)
        self.attn = SdpaAttn(d, heads)
        self.norm2 = RMSNorm(d)
        self.mlp = MLP(d, 4 * d)
        self.adaLN_modulation = nn.Sequential(nn.Linear(d, 6 * d, bias=True))

    def forward(self, x, y, c, pos, mask=None):
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.adaLN_modulation(c).chunk(6, dim=-1)
        h = G.mod_rmsnorm(x, self.norm1.weight, shift_msa, scale_msa, self.norm1.variance_epsilon)
        x, h = G.res_mod_rmsnorm(x, self.attn(h, y, pos, mask), gate_msa, self.norm2.weight, shift_mlp, scale_mlp,
                                 self.norm2.variance_epsilon)
        return x + gate_mlp * self.mlp(h)


class Net(nn.Module):
    def __init__(self, d, heads, n):
        super().__init__()
        self.blocks = nn.ModuleList(Block(d, heads) for _ in range(n))

    def forward(self, x, c, mask=None):
        for b in self.blocks:
            x = b(x, None, c, None, mask)
        return x
