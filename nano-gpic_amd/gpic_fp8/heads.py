"""The attention output's producer-fused cast, reachable from a converted model.

At JiT_T2I.py:183-185 (and TextRefineAttention, :261-263) the attention's forward computes
    x = attention(q, k, v)                      # scaled_dot_product_attention: o [B, H, N, D]
    x = x.transpose(1, 2).reshape(B, N, C)      # a copy whenever o is [B, H, N, D] in memory (the flash backend)
    x = self.proj(x)                            # the FP8 linear: tcast(x), then the GEMM
convert_fused_heads (after convert_native(phase=3)) makes the first two lines hand proj the attention output itself,
and proj (Fp8HeadsLinearF8) casts it with tcast_heads: the head-merging copy is never made and proj's e4m3 input is
read straight from o (fp8_heads_linear_f8: the same bits as the copy's cast and the same GEMMs). The attention's own
forward runs unchanged: the converter rebinds only the name `attention` it calls (the reference imports
torch.nn.functional.scaled_dot_product_attention under that name, attention_op.py:4), to a wrapper whose result keeps
the transpose and the reshape pending (_PendingHeads) until proj takes them. Any other use of that result gives the
tensor eager code would have had, so a forward that does something else with it computes what it always did.
The route is eager only: while torch.compile traces a converted attention it traces the class's own forward (and
the wrapper would return the attention output itself), so a compiled model takes the head-merging copy and the plain
phase-3 proj."""
import builtins
import types

import torch
from torch.utils._pytree import tree_map

from .fp8_native import Fp8LinearF8, fp8_heads_linear_f8, fp8_linear_f8

SDPA = torch.nn.functional.scaled_dot_product_attention


class _PendingHeads:
    """The attention output o [B, H, N, D] with stage 0 (o), 1 (o.transpose(1, 2)) or 2 (that, reshaped to
    [B, N, H D]) of the layout change still to do. transpose(1, 2) at stage 0 and reshape to [B, N, H D] at stage 1
    stay pending; every other attribute, method, operator or torch function is applied to the real tensor of the
    stage (made by the same ops on o, once)."""
    __slots__ = ("o", "stage", "_t")

    def __init__(self, o, stage):
        self.o, self.stage, self._t = o, stage, None

    def materialize(self):
        if self._t is None:
            o = self.o
            t = o if self.stage == 0 else o.transpose(1, 2)
            self._t = t if self.stage < 2 else t.reshape(o.shape[0], o.shape[2], o.shape[1] * o.shape[3])
        return self._t

    def transpose(self, d0, d1):
        if self.stage == 0 and isinstance(d0, int) and isinstance(d1, int) and {d0 % 4, d1 % 4} == {1, 2}:
            return _PendingHeads(self.o, 1)
        return self.materialize().transpose(d0, d1)

    def reshape(self, *shape):
        dims = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list, torch.Size)) else shape
        if self.stage == 1 and _merges(self.o, dims):
            return _PendingHeads(self.o, 2)
        return self.materialize().reshape(*shape)

    def __getattr__(self, name):
        return getattr(self.materialize(), name)

    @classmethod
    def __torch_function__(cls, func, types_, args=(), kwargs=None):
        real = lambda a: a.materialize() if isinstance(a, _PendingHeads) else a
        return func(*tree_map(real, args), **tree_map(real, kwargs or {}))


def _forward_operator(name):
    def op(self, *args):
        real = [a.materialize() if isinstance(a, _PendingHeads) else a for a in args]
        return getattr(self.materialize(), name)(*real)
    op.__name__ = name
    return op


for _name in ("__add__", "__radd__", "__sub__", "__rsub__", "__mul__", "__rmul__", "__truediv__", "__rtruediv__",
              "__matmul__", "__rmatmul__", "__neg__", "__getitem__", "__len__", "__iter__", "__bool__", "__float__"):
    setattr(_PendingHeads, _name, _forward_operator(_name))


def _merges(o, dims):
    """Whether reshape(dims) of o.transpose(1, 2) is the merge into [B, N, H D] (one -1 allowed, as torch allows)."""
    B, H, N, D = o.shape
    if not all(isinstance(d, int) for d in dims) or len(dims) != 3 or list(dims).count(-1) > 1:
        return False
    known = 1
    for d in dims:
        if d != -1:
            known *= d
    dims = tuple(d if d != -1 else (o.numel() // known if known else -1) for d in dims)
    return dims == (B, N, H * D)


class Fp8HeadsLinearF8(Fp8LinearF8):
    """The proj of an attention converted with convert_fused_heads: an Fp8LinearF8 (the same parameters and
    state-dict keys) that takes a pending merged attention output through fp8_heads_linear_f8 (its e4m3 input cast
    from o directly); any other input as Fp8LinearF8. heads_calls counts the calls that took the heads path."""
    heads_calls = 0

    def forward(self, x):
        if isinstance(x, _PendingHeads):
            if x.stage == 2 and x._t is None:
                self.heads_calls += 1
                return fp8_heads_linear_f8(x.o, self.weight, self.bias)
            x = x.materialize()
        return fp8_linear_f8(x, self.weight, self.bias)


def _pending_attention(real):
    def attention(q, k, v, *args, **kwargs):
        o = real(q, k, v, *args, **kwargs)
        # (while torch.compile traces, the output as it is: the forward then computes what it always did, through the
        # plain FP8 linear)
        if (isinstance(o, torch.Tensor) and o.dim() == 4 and o.shape[3] % 16 == 0 and
                not torch.compiler.is_compiling()):
            return _PendingHeads(o, 0)
        return o
    return attention


class _Globals(dict):
    """A function's globals with some names bound anew; every other name is read from the module's own dict at the
    time of the call (so later changes of the module's flags are seen)."""
    def __init__(self, base, **bound):
        super().__init__(bound)
        self.base = base
        self["__builtins__"] = base.get("__builtins__", builtins)

    def __missing__(self, key):
        return self.base[key]


def fused_heads_ok(attn):
    """An attention module whose forward calls scaled_dot_product_attention by the global name `attention`
    (JiT_T2I.py:8,183) and whose proj is a phase-3 FP8 linear (convert_native(phase=3))."""
    fwd = getattr(type(attn), "forward", None)
    proj = getattr(attn, "proj", None)
    return (isinstance(fwd, types.FunctionType) and "attention" in fwd.__code__.co_names and
            fwd.__globals__.get("attention") is SDPA and isinstance(proj, Fp8LinearF8) and
            proj.in_features % 16 == 0)


def _rebound(cls):
    """cls.forward with its global name `attention` bound to the pending wrapper."""
    fwd = cls.forward
    g = _Globals(fwd.__globals__, attention=_pending_attention(SDPA))
    f = types.FunctionType(fwd.__code__, g, fwd.__name__, fwd.__defaults__, fwd.__closure__)
    f.__kwdefaults__ = fwd.__kwdefaults__
    return f


def _heads_forward(attn, *args, **kwargs):
    """A converted attention's forward: in eager mode its class's forward with `attention` rebound; while
    torch.compile traces, its class's forward itself (the tracer is given the function with the module's own globals)."""
    if torch.compiler.is_compiling():
        return type(attn).forward(attn, *args, **kwargs)
    return attn._gpic_forward(attn, *args, **kwargs)


def convert_fused_heads(net):
    """Route the attention output feeding proj through tcast_heads in every block attention fused_heads_ok accepts
    (the image blocks' attn; the text-refine blocks' when their proj was converted, convert_native(text=True)).
    Parameters and state-dict keys are unchanged. Returns the number of attentions rewired."""
    n = 0
    for blk in list(getattr(net, "blocks", [])) + list(getattr(net, "text_refine_blocks", [])):
        attn = getattr(blk, "attn", None)
        if attn is None or getattr(attn, "_gpic_fused_heads", False) or not fused_heads_ok(attn):
            continue
        attn.proj.__class__ = Fp8HeadsLinearF8
        attn._gpic_forward = _rebound(type(attn))
        attn.forward = types.MethodType(_heads_forward, attn)
        attn._gpic_fused_heads = True
        n += 1
    return n
