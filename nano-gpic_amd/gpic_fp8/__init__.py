"""gpic_fp8: nano-gpic's native FP8 linear path (JiT-T2I) for MI355X / gfx950.

The API of baselines/PixelGen/src/models/layers/fp8_native.py and src/utils/fp8.py, computed by hand-written HIP
kernels in libgpic_fp8.so (C ABI: include/gpic_fp8.h). GPU only: no CPU fallback.
"""
from .fp8_native import (E4, FMAX, TINY, Fp8Linear, Fp8LinearF8, convert_native, fp8_gemm, fp8_gemm_mn,
                         fp8_heads_linear_f8, fp8_linear, fp8_linear_f8, fp8_mlp, fp8_mlp_f8, fp8_swiglu_w3, reference,
                         swiglu_bwd, swiglu_bwd_q, swiglu_bwd_t, swiglu_tcast, swiglu_tcast_t, tcast, tcast_heads,
                         tcast_t, tcast_t_group, weight_casts, _mm)
from .fp8 import KEEP, convert_fp8, fp8_filter
from .heads import Fp8HeadsLinearF8, convert_fused_heads
from .norm import (Fp8NormLinearF8, convert_fused_norm, fp8_mod_rmsnorm_linear, fp8_res_mod_rmsnorm_mlp,
                   mod_rmsnorm, res_mod_rmsnorm, res_mod_rmsnorm_bwd, res_mod_rmsnorm_fwd, res_mod_rmsnorm_q)
from .norm import reference as norm_reference

__all__ = ["E4", "FMAX", "TINY", "Fp8Linear", "Fp8LinearF8", "convert_native", "convert_fp8", "fp8_filter", "KEEP",
           "fp8_gemm", "fp8_gemm_mn", "fp8_linear", "fp8_linear_f8", "fp8_mlp", "fp8_mlp_f8", "fp8_swiglu_w3", "reference",
           "swiglu_bwd", "swiglu_bwd_q", "swiglu_bwd_t", "swiglu_tcast", "swiglu_tcast_t", "tcast", "tcast_t", "tcast_t_group",
           "weight_casts", "_mm",
           "mod_rmsnorm", "res_mod_rmsnorm", "res_mod_rmsnorm_q", "norm_reference", "fp8_mod_rmsnorm_linear",
           "fp8_res_mod_rmsnorm_mlp", "Fp8NormLinearF8", "convert_fused_norm", "tcast_heads", "fp8_heads_linear_f8",
           "Fp8HeadsLinearF8", "convert_fused_heads", "res_mod_rmsnorm_fwd", "res_mod_rmsnorm_bwd"]
