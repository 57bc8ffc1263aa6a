"""Recipe dispatcher of the FP8 path (baselines/PixelGen/src/utils/fp8.py:13-56): "native" / "native2" convert the
image blocks with convert_native (phase 1 / 2), "native3" with every GEMM in FP8 (phase 3), "native3+text" also the
image blocks' kv_y and the text-refine blocks' linears (phase 3, convert_native(text=True)). Any other recipe name is
a torchao Float8Linear recipe in the reference; torchao is not part of this build and such a recipe raises ImportError.
"""
import os
import sys

import torch

from .fp8_native import convert_native

_PATH = os.environ.get("GPIC_TORCHAO_PATH", "")
KEEP = ("adaLN_modulation",)
NATIVE = {"native": (1, False), "native2": (2, False), "native3": (3, False), "native3+text": (3, True)}


def _torchao():
    if _PATH and _PATH not in sys.path:
        sys.path.insert(0, _PATH)
    try:
        import torchao  # noqa: F401
    except ImportError as e:
        raise ImportError("torchao recipes need torchao (set GPIC_TORCHAO_PATH); the MI355X-native recipes are "
                          f"{sorted(NATIVE)}") from e


def fp8_filter(mod, fqn):
    """The linears the torchao recipes convert (fp8.py:28-35): every nn.Linear of blocks.* and text_refine_blocks.*
    except adaLN_modulation, when in and out features are multiples of 16."""
    if not isinstance(mod, torch.nn.Linear):
        return False
    if not (fqn.startswith("blocks.") or fqn.startswith("text_refine_blocks.")):
        return False
    if any(k in fqn for k in KEEP):
        return False
    return mod.in_features % 16 == 0 and mod.out_features % 16 == 0


def convert_fp8(net, recipe):
    """Swap the blocks' Linear layers of net for FP8 ones (the same parameters and state-dict keys). Returns the
    number of GEMMs (native recipes) or Linear layers (torchao recipes) converted."""
    if recipe in NATIVE:
        keys = set(net.state_dict())
        phase, text = NATIVE[recipe]
        n = convert_native(net, phase=phase, text=text)
        assert set(net.state_dict()) == keys, "FP8 conversion changed the state-dict keys"
        where = "image and text blocks" if text else "image blocks"
        print(f"FP8 ({recipe}, MI355X native): {n} GEMMs of the {where} converted", flush=True)
        return n
    _torchao()
    from torchao.float8 import convert_to_float8_training, Float8LinearConfig
    cfg = Float8LinearConfig.from_recipe_name(recipe)
    keys = set(net.state_dict())
    convert_to_float8_training(net, config=cfg, module_filter_fn=fp8_filter)
    assert set(net.state_dict()) == keys, "FP8 conversion changed the state-dict keys"
    n = sum(1 for m in net.modules() if type(m).__name__ == "Float8Linear")
    print(f"FP8 ({recipe}, lever F8): {n} Linear layers of the blocks converted", flush=True)
    return n
