"""ctypes binding of libbaracuda_kernels.so (the C ABI in include/baracuda_kernels.h).

Loading fails loudly: there is no CPU fallback for any entry point.  Build the
library first with ``python -m baracuda_amd.build``.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbaracuda_kernels.so"

i32, i64, f32, vp, sz = C.c_int32, C.c_int64, C.c_float, C.c_void_p, C.c_size_t

# name -> (restype, argtypes); mirrors include/baracuda_kernels.h one to one.
_SIGS: dict[str, tuple] = {}


def _sig(name, res, *args):
    _SIGS[name] = (res, list(args))


_RCR_CAN = (i32, i32, i32, vp, i64, vp, i64, vp, i64, vp, i64)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_run", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64, vp, i64, f32, f32, vp, sz, vp)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_can_implement", i32, *_RCR_CAN)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_i32_run", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64, vp, sz, vp)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_i32_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_s8_rcr_gfx950_i32_can_implement", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64)
_sig("baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_run", i32, i32, i32, i32, vp, i64, vp, i64, vp, vp, vp, i64, vp, sz, vp)
_sig("baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_w8a8_rcr_gfx950_bf16_can_implement", i32, i32, i32, i32, vp, i64, vp, i64, vp, vp, vp, i64)
_sig("baracuda_kernels_quantized_linear_w8a8_f32_gfx950_run", i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, sz, vp)
_sig("baracuda_kernels_quantized_linear_w8a8_f32_gfx950_can_implement", i32, i32, i32, i32, vp, vp, vp, vp, vp)
_sig("baracuda_kernels_quantized_linear_w8a8_f64_gfx950_run", i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, sz, vp)
_sig("baracuda_kernels_quantized_linear_w8a8_f64_gfx950_can_implement", i32, i32, i32, i32, vp, vp, vp, vp, vp)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_run", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64, vp, i64, f32, f32, vp, sz, vp)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_can_implement", i32, *_RCR_CAN)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_run", i32, i32, i32, i32, vp, i64, vp, i64, f32, f32, vp, i64, vp, sz, vp)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_bf16_can_implement", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_run", i32, i32, i32, i32, vp, i64, vp, i64, f32, vp, i64, vp, sz, vp)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_fp8_e4m3_rcr_gfx950_f32_can_implement", i32, i32, i32, i32, vp, i64, vp, i64, vp, i64)
for _t in ("f32", "f16", "bf16"):
    _sig(f"baracuda_kernels_gemv_dense_m1_{_t}_run", i32, i32, i32, i32, i32, i32, f32, f32,
         vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, sz, vp)
    _sig(f"baracuda_kernels_gemv_dense_m1_{_t}_can_implement", i32, i32, i32, i32, i32, i32,
         i64, i64, i64, i64, i64, i64)
    _sig(f"baracuda_kernels_gemv_dense_m1_{_t}_workspace_size", sz, i32, i32, i32, i32, i32)
    _sig(f"baracuda_kernels_gather_rows_{_t}_run", i32, vp, vp, vp, i64, i64, i64, vp)
    _sig(f"baracuda_kernels_gather_rows_{_t}_can_implement", i32, i64, i64, i64)
    _sig(f"baracuda_kernels_gather_rows_{_t}_workspace_size", sz, i64, i64, i64)
_sig("baracuda_kernels_gemv_s8w_m1_bf16_gfx950_run", i32, i32, i32, vp, vp, i64, vp, vp, vp, sz, vp)
_sig("baracuda_kernels_gemv_s8w_m1_bf16_gfx950_workspace_size", sz, i32, i32)
_sig("baracuda_kernels_gemv_s8w_m1_bf16_gfx950_can_implement", i32, i32, i32, i64)
_sig("baracuda_kernels_moe_s8_grouped_bf16_gfx950_run", i32, vp, vp, vp, vp, vp, vp, vp, vp,
     i32, i32, i32, i32, i32, vp, vp, vp, sz, vp)
_sig("baracuda_kernels_moe_s8_grouped_bf16_gfx950_can_implement", i32, i32, i32, i32, i32, i32)
_sig("baracuda_kernels_moe_s8_grouped_bf16_gfx950_workspace_size", sz, i32, i32, i32, i32, i32)
_sig("baracuda_kernels_moe_s8_grouped_i32_gfx950_run", i32, vp, vp, vp, vp, vp, vp, vp,
     i32, i32, i32, i32, i32, vp)
_sig("baracuda_kernels_moe_s8_grouped_i32_gfx950_can_implement", i32, i32, i32, i32, i32, i32)

for _t in ("f32", "f64"):
    _sig(f"baracuda_kernels_dynamic_range_quantize_per_token_sym_{_t}_s8_run", i32, i32, i32, i32, i32,
         vp, vp, vp, vp, sz, vp)
    _sig(f"baracuda_kernels_dynamic_range_quantize_per_token_sym_{_t}_s8_can_implement", i32, i32, i32,
         i32, i32, vp, vp, vp)
_sig("baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_run", i32, i32, i32, i32, i32,
     vp, vp, vp, vp, sz, vp)
_sig("baracuda_kernels_dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_can_implement", i32, i32, i32,
     i32, i32, vp, vp, vp)

_RCR_RUN = (i32, i32, i32, vp, i64, vp, i64, vp, i64, vp, i64)
for _e in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
    for _b in ("f32", "i32"):
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_s8_rcr_gfx950_run", i32, *_RCR_RUN, vp, f32, f32, vp, sz, vp)
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_s8_rcr_gfx950_workspace_size", sz, i32, i32, i32)
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_s8_rcr_gfx950_can_implement", i32, *_RCR_RUN, vp)
        _sig(f"baracuda_kernels_gemm_s8_rrr_gfx950_{_e}_{_b}_run", i32, *_RCR_RUN, vp, f32, f32, vp, sz, vp)
        _sig(f"baracuda_kernels_gemm_s8_rrr_gfx950_{_e}_{_b}_can_implement", i32, *_RCR_RUN)
_sig("baracuda_kernels_gemm_s8_rrr_gfx950_run", i32, *_RCR_RUN, f32, f32, vp, sz, vp)
_sig("baracuda_kernels_gemm_u8_rcr_gfx950_run", i32, *_RCR_RUN, f32, f32, vp, sz, vp)
_sig("baracuda_kernels_gemm_u8_rcr_gfx950_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_u8_rcr_gfx950_can_implement", i32, *_RCR_RUN)
for _e in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
    for _b in ("f32", "i32"):
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_u8_rcr_gfx950_run", i32, *_RCR_RUN, vp, f32, f32, vp, sz, vp)
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_u8_rcr_gfx950_workspace_size", sz, i32, i32, i32)
        _sig(f"baracuda_kernels_gemm_{_e}_{_b}bias_u8_rcr_gfx950_can_implement", i32, *_RCR_RUN, vp)
_sig("baracuda_kernels_gemm_u8_rrr_gfx950_run", i32, *_RCR_RUN, f32, f32, vp, sz, vp)
_sig("baracuda_kernels_gemm_u8_rrr_gfx950_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_u8_rrr_gfx950_can_implement", i32, *_RCR_RUN)
_sig("baracuda_kernels_gemm_u8_rrr_gfx950_noalloc_run", i32, *_RCR_RUN, f32, f32, vp)
for _e in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
    for _b in ("f32", "i32"):
        _sig(f"baracuda_kernels_gemm_u8_rrr_gfx950_{_e}_{_b}_run", i32, *_RCR_RUN, vp, f32, f32, vp, sz, vp)
        _sig(f"baracuda_kernels_gemm_u8_rrr_gfx950_{_e}_{_b}_can_implement", i32, *_RCR_RUN)
_sig("baracuda_kernels_gemm_s8_rrr_gfx950_workspace_size", sz, i32, i32, i32)
_sig("baracuda_kernels_gemm_s8_rrr_gfx950_can_implement", i32, *_RCR_RUN)

for _enc in ("e4m3", "e5m2"):
    for _lay in ("rcr", "rrr"):
        _pre = f"baracuda_kernels_gemm_fp8_{_enc}_{_lay}_gfx950"
        if (_enc, _lay) != ("e4m3", "rcr"):
            _sig(f"{_pre}_run", i32, *_RCR_RUN, f32, f32, vp, sz, vp)
            _sig(f"{_pre}_workspace_size", sz, i32, i32, i32)
            _sig(f"{_pre}_can_implement", i32, *_RCR_RUN)
        for _e in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
            _sig(f"{_pre}_{_e}_run", i32, *_RCR_RUN, vp, f32, f32, vp, sz, vp)
            _sig(f"{_pre}_{_e}_can_implement", i32, *_RCR_RUN)

for _i in ("", "i64idx_"):
    for _t in ("f32", "f64", "f16", "bf16"):
        _sig(f"baracuda_kernels_embedding_{_i}{_t}_run", i32, i64, i32, i32, i64, vp, vp, vp, vp, sz, vp)
        _sig(f"baracuda_kernels_embedding_{_i}{_t}_can_implement", i32, i64, i32, i32, i64, vp, vp, vp)

for _t in ("bf16", "f16"):
    _sig(f"baracuda_kernels_moe_wmma_{_t}_run", i32, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32,
         i32, vp, sz, vp)
    _sig(f"baracuda_kernels_moe_wmma_{_t}_can_implement", i32, i32, i32, i32, i32, i32, i32)
_sig("baracuda_te_fp8_format_e4m3", i32)
_sig("baracuda_te_fp8_format_e5m2", i32)
_sig("baracuda_te_fp8_max_representable", f32, i32)
_sig("baracuda_te_fused_cast_amax_run", i32, vp, vp, vp, vp, i32, i64, i32, i32, vp)
_sig("baracuda_te_fused_cast_amax_can_implement", i32, vp, vp, vp, vp, i32, i64, i32, i32)
_sig("baracuda_te_dequant_run", i32, vp, vp, vp, i64, i32, i32, vp)
_sig("baracuda_te_dequant_can_implement", i32, vp, vp, vp, i64, i32, i32)
_sig("baracuda_te_recipe_update_run", i32, vp, vp, vp, i32, i32, i32, vp)
_sig("baracuda_te_recipe_update_can_implement", i32, vp, vp, vp, i32, i32, i32)
_sig("baracuda_te_recipe_init_run", i32, vp, vp, vp, i32, vp)
_sig("baracuda_te_recipe_init_can_implement", i32, vp, vp, vp, i32)

SYMBOLS = tuple(_SIGS)

_lib = None


class Lib:
    """Attribute access to every exported entry point, typed."""

    def __init__(self, path: Path = LIB_PATH):
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with `python -m baracuda_amd.build` "
                "(the gfx950 kernels have no CPU fallback)")
        self._dll = C.CDLL(str(path))
        for name, (res, args) in _SIGS.items():
            fn = getattr(self._dll, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name.replace("baracuda_kernels_", ""), fn)
        self.path = path


def lib() -> Lib:
    global _lib
    if _lib is None:
        _lib = Lib()
    return _lib
