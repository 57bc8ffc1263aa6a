"""Recipe dispatcher of the FP8 path (baselines/PixelGen/src/utils/fp8.py:13-56): "native" / "native2" convert the
image blocks with convert_native (phase 1 / 2), "native3" with every GEMM in FP8 (phase 3), "native3+text" also the
image blocks' kv_y and the text-refine blocks' linears (phase 3, convert_native(text=True)); "+norm" also routes the
image blocks' norm sites through the producer-fused kernels (convert_native(fused_norm=True)), "+heads" the attention
output feeding each converted proj (convert_native(fused_heads=True)), "+fused" both. Every other recipe name selects
a torchao Float8Linear recipe in the reference;
this build implements the native recipes only and refuses the others with a ValueError.
"""
import torch

from .fp8_native import convert_native

KEEP = ("adaLN_modulation",)
# recipe -> (phase, text, fused_norm, fused_heads)
NATIVE = {"native": (1, False, False, False), "native2": (2, False, False, False), "native3": (3, False, False, False),
          "native3+text": (3, True, False, False), "native3+norm": (3, False, True, False),
          "native3+text+norm": (3, True, True, False), "native3+heads": (3, False, False, True),
          "native3+text+heads": (3, True, False, True), "native3+fused": (3, False, True, True),
          "native3+text+fused": (3, True, True, True)}


def fp8_filter(mod, fqn):
    """The linears the torchao recipes convert (fp8.py:28-35): every nn.Linear of blocks.* and text_refine_blocks.*
    except adaLN_modulation, when in and out features are multiples of 16. convert_native(text=True) takes the same
    set of linears of the attention and MLP modules."""
    if not isinstance(mod, torch.nn.Linear):
        return False
    if not (fqn.startswith("blocks.") or fqn.startswith("text_refine_blocks.")):
        return False
    if any(k in fqn for k in KEEP):
        return False
    return mod.in_features % 16 == 0 and mod.out_features % 16 == 0


def convert_fp8(net, recipe):
    """Swap the blocks' Linear layers of net for FP8 ones (the same parameters and state-dict keys) and return the
    number of GEMMs converted. Only the native recipes exist here; another name raises ValueError before anything is
    changed."""
    if recipe not in NATIVE:
        raise ValueError(f"FP8 recipe {recipe!r} is not available: this build implements the MI355X-native recipes "
                         f"{sorted(NATIVE)} only (the reference's other recipes are torchao's Float8Linear)")
    keys = set(net.state_dict())
    phase, text, fused_norm, fused_heads = NATIVE[recipe]
    n = convert_native(net, phase=phase, text=text, fused_norm=fused_norm, fused_heads=fused_heads)
    if set(net.state_dict()) != keys:
        raise RuntimeError("FP8 conversion changed the state-dict keys")
    where = "image and text blocks" if text else "image blocks"
    print(f"FP8 ({recipe}, MI355X native): {n} GEMMs of the {where} converted", flush=True)
    return n
