"""C-ABI boundary checks that need no GPU: every declared symbol is exported
with the declared name, and the host-side validation (can_implement /
workspace_size / empty problems / Plan.select) behaves like the reference."""
import re
from pathlib import Path

import pytest

from baracuda_amd import ffi
from baracuda_amd import plans as P

HDR = Path(__file__).resolve().parents[1] / "include" / "baracuda_kernels.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HDR.read_text(), flags=re.S)
    names = set(re.findall(r"\b(baracuda_(?:kernels|te)_\w+)\s*\(", text))
    for tag_macro, body, sufs in (
            ("BK_GEMV_DENSE_DECL", "gemv_dense_m1_{}", ("run", "can_implement", "workspace_size")),
            ("BK_GATHER_DECL", "gather_rows_{}", ("run", "can_implement", "workspace_size")),
            ("BK_QUANT_DECL", "dynamic_range_quantize_per_token_sym_{}_s8", ("run", "can_implement"))):
        for tag in re.findall(tag_macro + r"\((\w+)\)", text):
            for suf in sufs:
                names.add(f"baracuda_kernels_{body.format(tag)}_{suf}")
    for enc, lay in re.findall(r"BK_FP8_DECL\((\w+), (\w+)\)", text):
        for suf in ("run", "workspace_size", "can_implement"):
            names.add(f"baracuda_kernels_gemm_fp8_{enc}_{lay}_gfx950_{suf}")
    for enc, lay in re.findall(r"BK_FP8_BIAS_DECL4\((\w+), (\w+)\)", text):
        for epi in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
            for suf in ("run", "can_implement"):
                names.add(f"baracuda_kernels_gemm_fp8_{enc}_{lay}_gfx950_{epi}_{suf}")
    for tag in re.findall(r"BK_MOE_WMMA_DECL\((\w+)\)", text):
        for suf in ("run", "can_implement"):
            names.add(f"baracuda_kernels_moe_wmma_{tag}_{suf}")
    for tag in re.findall(r"BK_EMBED_DECL\((\w+)\)", text):
        for suf in ("run", "can_implement"):
            names.add(f"baracuda_kernels_{tag}_{suf}")
    for epi, bias in re.findall(r"BK_S8_RCR_BIAS_DECL\((\w+), (\w+)\)", text):
        for suf in ("run", "workspace_size", "can_implement"):
            names.add(f"baracuda_kernels_gemm_{epi}_{bias}_s8_rcr_gfx950_{suf}")
    for epi, bias in re.findall(r"BK_U8_RCR_BIAS_DECL\((\w+), (\w+)\)", text):
        for suf in ("run", "workspace_size", "can_implement"):
            names.add(f"baracuda_kernels_gemm_{epi}_{bias}_u8_rcr_gfx950_{suf}")
    for epi, bias in re.findall(r"BK_U8_RRR_BIAS_DECL\((\w+), (\w+)\)", text):
        for suf in ("run", "can_implement"):
            names.add(f"baracuda_kernels_gemm_u8_rrr_gfx950_{epi}_{bias}_{suf}")
    for epi, bias in re.findall(r"BK_S8_RRR_BIAS_DECL\((\w+), (\w+)\)", text):
        for suf in ("run", "can_implement"):
            names.add(f"baracuda_kernels_gemm_s8_rrr_gfx950_{epi}_{bias}_{suf}")
    return {n for n in names if "_TAG_" not in n and "##" not in n and "_EPI_" not in n
            and "_NAME_" not in n and "_ENC_" not in n and "wmma_TAG" not in n}


def test_header_and_binding_agree():
    assert _declared() == set(ffi.SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = ffi.lib()
    import ctypes
    dll = ctypes.CDLL(str(lib.path))
    for name in _declared():
        assert hasattr(dll, name), name


def test_gemv_can_implement_rejection_table():
    # gemv_dense_smoke.rs:401-432, same argument tuples and expectations.
    L = ffi.lib()
    for tag in ("f32", "f16", "bf16"):
        can = getattr(L, f"gemv_dense_m1_{tag}_can_implement")
        assert can(1, 6, 4, 1, 0, 4, 6, 6, 0, 0, 0) == 0
        assert can(2, 6, 4, 1, 0, 4, 6, 6, 0, 0, 0) == 2
        assert can(1, 6, 4, 1, 1, 4, 6, 6, 0, 0, 0) == 2
        assert can(1, 6, 4, 1, 0, 3, 6, 6, 0, 0, 0) == 2
        assert can(1, 6, 4, 1, 0, 4, 5, 6, 0, 0, 0) == 2
        assert can(1, 6, 4, 1, 0, 4, 6, 5, 0, 0, 0) == 2
        assert can(1, 6, 4, 2, 0, 4, 6, 6, 0, 0, 0) == 2
        assert can(1, 6, 4, 2, 0, 4, 6, 6, 4, 0, 6) == 0
        assert can(1, -1, 4, 1, 0, 4, 6, 6, 0, 0, 0) == 2
        assert getattr(L, f"gemv_dense_m1_{tag}_workspace_size")(1, 6, 4, 1, 0) == 0


def test_gemv_empty_problem_returns_ok_without_launch():
    # gemv_dense.cu:190: m == 0 / n == 0 / batch == 0 -> 0, no launch, null pointers allowed.
    L = ffi.lib()
    assert L.gemv_dense_m1_f32_run(0, 6, 4, 1, 0, 1.0, 0.0, None, 4, 0, None, 6, 0, None, 6, 0, None, 0, None) == 0
    assert L.gemv_dense_m1_bf16_run(1, 0, 4, 1, 0, 1.0, 0.0, None, 4, 0, None, 1, 0, None, 1, 0, None, 0, None) == 0
    assert L.gemv_s8w_m1_bf16_gfx950_run(0, 4096, None, None, 4096, None, None, None, 0, None) == 0


def test_gather_can_implement_and_empty():
    L = ffi.lib()
    for tag in ("f32", "f16", "bf16"):
        assert getattr(L, f"gather_rows_{tag}_can_implement")(3, 4, 1) == 0
        assert getattr(L, f"gather_rows_{tag}_can_implement")(0, 4, 1) == 2
        assert getattr(L, f"gather_rows_{tag}_can_implement")(3, 4, -1) == 2
        assert getattr(L, f"gather_rows_{tag}_workspace_size")(3, 4, 1) == 0
        # n == 0 is a valid no-op; null pointers with n > 0 are invalid
        assert getattr(L, f"gather_rows_{tag}_run")(None, None, None, 3, 4, 0, None) == 0
        assert getattr(L, f"gather_rows_{tag}_run")(None, None, None, 3, 4, 1, None) == 2


def test_gemm_invalid_problems_rejected_before_launch():
    L = ffi.lib()
    # non-positive extents -> 2 (baracuda_int8_rrr_sm80.cuh:321)
    assert L.gemm_s8_rcr_gfx950_can_implement(0, 4, 4, None, 4, None, 4, None, 0, None, 4) == 2
    assert L.gemm_s8_rcr_gfx950_can_implement(4, 4, 4, None, 3, None, 4, None, 0, None, 4) == 2
    assert L.gemm_s8_rcr_gfx950_can_implement(4, 4, 4, None, 4, None, 4, None, 0, None, 4) == 0
    assert L.gemm_s8_rcr_gfx950_run(4, 4, 4, None, 4, None, 4, None, 0, None, 4, 1.0, 0.0, None, 0, None) == 2
    assert L.gemm_s8_rcr_gfx950_i32_run(-1, 4, 4, None, 4, None, 4, None, 4, None, 0, None) == 2
    assert L.gemm_w8a8_rcr_gfx950_bf16_can_implement(8, 8, 8, None, 8, None, 8, None, None, None, 7) == 2
    assert L.gemm_fp8_e4m3_rcr_gfx950_can_implement(1, 1, 0, None, 1, None, 1, None, 0, None, 1) == 2
    assert L.gemm_fp8_e4m3_rcr_gfx950_bf16_workspace_size(16, 16, 16) == 0
    assert L.quantized_linear_w8a8_f32_gfx950_can_implement(-1, 2, 2, None, None, None, None, None) == 2
    assert L.quantized_linear_w8a8_f32_gfx950_run(0, 2, 2, None, None, None, None, None, None, 0, None) == 0
    assert L.quantized_linear_w8a8_f64_gfx950_can_implement(-1, 2, 2, None, None, None, None, None) == 2
    assert L.quantized_linear_w8a8_f64_gfx950_run(0, 2, 2, None, None, None, None, None, None, 0, None) == 0
    assert L.quantized_linear_w8a8_f64_gfx950_run(2, 2, 2, None, None, None, None, None, None, 0, None) == 2



def test_rrr_and_bias_can_implement():
    # gemm_s8_rrr_sm80.cu:44-52: positive extents, lda >= K, ldb >= N, ldd >= N.
    L = ffi.lib()
    assert L.gemm_s8_rrr_gfx950_can_implement(4, 8, 16, None, 16, None, 8, None, 0, None, 8) == 0
    assert L.gemm_s8_rrr_gfx950_can_implement(4, 8, 16, None, 16, None, 7, None, 0, None, 8) == 2
    assert L.gemm_s8_rrr_gfx950_can_implement(4, 8, 16, None, 15, None, 8, None, 0, None, 8) == 2
    assert L.gemm_s8_rrr_gfx950_can_implement(0, 8, 16, None, 16, None, 8, None, 0, None, 8) == 2
    assert L.gemm_s8_rrr_gfx950_workspace_size(64, 64, 64) == 0
    # the u8 RRR family's optional pre-pass workspace: whole tiles only
    assert L.gemm_u8_rrr_gfx950_workspace_size(64, 64, 64) == 0
    assert L.gemm_u8_rrr_gfx950_workspace_size(512, 256, 200) == 0
    assert L.gemm_u8_rrr_gfx950_workspace_size(512, 768, 384) == (512 + 768) * 4 + 512 * 384 + 384 * 768
    for epi in ("bias", "bias_relu", "bias_gelu", "bias_silu"):
        for bt in ("f32", "i32"):
            assert getattr(L, f"gemm_s8_rrr_gfx950_{epi}_{bt}_can_implement")(
                4, 8, 16, None, 16, None, 8, None, 0, None, 8) == 0
            # run refuses a missing bias before launching anything
            assert getattr(L, f"gemm_s8_rrr_gfx950_{epi}_{bt}_run")(
                4, 8, 16, None, 16, None, 8, None, 0, None, 8, None, 1.0, 0.0, None, 0, None) == 2
            rcr = f"gemm_{epi}_{bt}bias_s8_rcr_gfx950_"
            assert getattr(L, rcr + "can_implement")(4, 8, 16, None, 16, None, 16, None, 0, None, 8, None) == 0
            assert getattr(L, rcr + "can_implement")(4, 8, 16, None, 16, None, 15, None, 0, None, 8, None) == 2
            assert getattr(L, rcr + "workspace_size")(4, 8, 16) == 0
            assert getattr(L, rcr + "run")(4, 8, 16, None, 16, None, 16, None, 0, None, 8, None,
                                           1.0, 0.0, None, 0, None) == 2



def test_embedding_can_implement_and_empty():
    # baracuda_embedding.cuh:513-556: negative extents -> 2, N == 0 -> 0 before
    # the pointer check, null pointers -> 2.
    L = ffi.lib()
    for i in ("", "i64idx_"):
        for t in ("f32", "f64", "f16", "bf16"):
            can = getattr(L, f"embedding_{i}{t}_can_implement")
            run = getattr(L, f"embedding_{i}{t}_run")
            assert can(4, 10, 8, -(2 ** 31), None, None, None) == 0
            assert can(-1, 10, 8, 0, None, None, None) == 2
            assert can(4, -1, 8, 0, None, None, None) == 2
            assert can(4, 10, -8, 0, None, None, None) == 2
            assert run(0, 10, 8, 0, None, None, None, None, 0, None) == 0
            assert run(-1, 10, 8, 0, None, None, None, None, 0, None) == 2
            assert run(3, 10, 8, 0, None, None, None, None, 0, None) == 2



def test_te_shim_argument_checks():
    # baracuda_te_shim.cu can_implement / run guards (status 1 = invalid).
    L = ffi.lib()
    assert L.baracuda_te_fp8_format_e4m3() == 0 and L.baracuda_te_fp8_format_e5m2() == 1
    assert L.baracuda_te_fp8_max_representable(0) == 448.0
    assert L.baracuda_te_fp8_max_representable(1) == 57344.0
    assert L.baracuda_te_fp8_max_representable(7) == 1.0
    can = L.baracuda_te_fused_cast_amax_can_implement
    assert can(None, None, None, None, 0, 16, 0, 2) == 0
    assert can(None, None, None, None, -1, 16, 0, 2) == 1
    assert can(None, None, None, None, 0, -1, 0, 2) == 1
    assert can(None, None, None, None, 0, 16, 2, 0) == 1
    assert can(None, None, None, None, 0, 16, 1, 3) == 1
    assert L.baracuda_te_fused_cast_amax_run(None, None, None, None, 0, 16, 0, 0, None) == 1
    assert L.baracuda_te_dequant_can_implement(None, None, None, 16, 1, 2) == 0
    assert L.baracuda_te_dequant_can_implement(None, None, None, 16, 1, -1) == 1
    assert L.baracuda_te_dequant_run(None, None, None, 16, 0, 0, None) == 1
    upd = L.baracuda_te_recipe_update_can_implement
    assert upd(None, None, None, 8, 7, 0) == 0
    assert upd(None, None, None, 8, 8, 0) == 1
    assert upd(None, None, None, 0, 0, 0) == 1
    assert upd(None, None, None, 8193, 0, 0) == 1
    assert L.baracuda_te_recipe_init_can_implement(None, None, None, 8192) == 0
    assert L.baracuda_te_recipe_init_can_implement(None, None, None, 0) == 1
    assert L.baracuda_te_recipe_init_run(None, None, None, 8, None) == 1
    with pytest.raises(P.TeInvalidArgument):
        P.Fp8Recipe(P.Fp8Format.E4M3, 0, device="cpu")


def test_quantize_can_implement():
    # baracuda_quantize_compose.cuh:320-330 checks (N > 65535 accepted here).
    L = ffi.lib()
    for f in (L.dynamic_range_quantize_per_token_sym_f32_s8_can_implement,
              L.dynamic_range_quantize_per_token_sym_f64_s8_can_implement,
              L.dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_can_implement):
        assert f(4, 8, -127, 127, None, None, None) == 0
        assert f(-1, 8, -127, 127, None, None, None) == 2
        assert f(4, 8, 5, 3, None, None, None) == 2
        assert f(4, 8, -5, 0, None, None, None) == 2
        assert f(100000, 8, -127, 127, None, None, None) == 0
    assert L.dynamic_range_quantize_per_token_sym_f32_s8_run(0, 8, -127, 127, None, None, None, None, 0, None) == 0
    assert L.dynamic_range_quantize_per_token_sym_f32_s8_run(2, 8, -127, 127, None, None, None, None, 0, None) == 2


def test_moe_can_implement():
    L = ffi.lib()
    for t in ("bf16", "f16"):   # moe_wmma.cu:189-209
        assert getattr(L, f"moe_wmma_{t}_can_implement")(8, 2, 64, 64, 64, 1) == 0
        assert getattr(L, f"moe_wmma_{t}_can_implement")(2, 3, 64, 64, 64, 0) == 2
        assert getattr(L, f"moe_wmma_{t}_can_implement")(2048, 2, 64, 64, 64, 0) == 3
        assert getattr(L, f"moe_wmma_{t}_run")(None, None, None, None, None, None, None, None,
                                                8, 2, 64, 64, 64, 1, None, 0, None) == 2
    # moe_wmma.cu:177-187
    assert L.moe_s8_grouped_bf16_gfx950_can_implement(8, 2, 8192, 14336, 4096) == 0
    assert L.moe_s8_grouped_bf16_gfx950_can_implement(2, 3, 16, 16, 16) == 2
    assert L.moe_s8_grouped_bf16_gfx950_can_implement(2048, 2, 16, 16, 16) == 3
    assert L.moe_s8_grouped_bf16_gfx950_can_implement(8, 2, 0, 16, 16) == 2


def test_plan_select_and_sku():
    plan = P.IntGemmPlan.select(P.IntGemmDescriptor(4096, 4096, 4096, output=P.ElementKind.Bf16))
    sku = plan.sku()
    assert sku.arch == P.ArchSku.Gfx950 and sku.layout == P.LayoutSku.Rcr
    pg = plan.precision_guarantee()
    assert pg.accumulator == P.ElementKind.I32 and pg.bit_stable_on_same_hardware and pg.deterministic
    assert plan.workspace_size() == 0
    with pytest.raises(P.InvalidProblem):
        P.IntGemmPlan.select(P.IntGemmDescriptor(0, 1, 1))
    rrr = P.IntGemmPlan.select(P.IntGemmDescriptor(8, 8, 8, layout=P.LayoutSku.Rrr,
                                                   epilogue=P.EpilogueKind.BiasGelu,
                                                   bias_element=P.ElementKind.I32))
    assert rrr.sku().layout == P.LayoutSku.Rrr and rrr.sku().bias_element == P.ElementKind.I32
    assert rrr.workspace_size() == 0
    assert P.IntGemmPlan.select(P.IntGemmDescriptor(8, 8, 8)).sku().bias_element is None
    with pytest.raises(P.Unsupported):   # raw accumulator is RCR / Identity only
        P.IntGemmPlan.select(P.IntGemmDescriptor(8, 8, 8, layout=P.LayoutSku.Rrr, output=P.ElementKind.I32))
    with pytest.raises(P.Unsupported):
        P.IntGemmPlan.select(P.IntGemmDescriptor(8, 8, 8, epilogue=P.EpilogueKind.Bias,
                                                 bias_element=P.ElementKind.F16))
    f = P.Fp8GemmPlan.select(P.Fp8GemmDescriptor(2048, 14336, 4096, output=P.ElementKind.Bf16))
    assert f.sku().element == P.ElementKind.Fp8E4M3 and f.workspace_size() == 0
    with pytest.raises(P.InvalidProblem):
        P.GemvDensePlan.select(P.GemvDenseDescriptor(n=4, k=4, m=2), __import__("torch").float32)
    with pytest.raises(P.Unsupported):
        P.MoeS8GroupedPlan.select(2048, 2, 16, 16, 16)


def test_tail_split_workspace_sizes():
    # the optional split-K workspace of a partial last round: whole rounds, a
    # last round more than half full, or K too short take none
    assert P.IntGemmPlan.select(P.IntGemmDescriptor(4296, 4096, 4096, output=P.ElementKind.Bf16)
                                ).workspace_size() == 16 * 16 * 65536 * 4
    # M % 256 in [1, 64] (N % 16 == 0) whose last row of tiles would start
    # another round (or M <= 64) runs the last-rows pass, no workspace; so
    # does M % 256 in [65, 128] when K % 512 == 0 (the staged last rows)
    for m in (4097, 4112, 4128, 4160, 1, 16, 64, 65, 100, 128, 4192, 4224):
        assert P.IntGemmPlan.select(P.IntGemmDescriptor(m, 4096, 4096, output=P.ElementKind.Bf16)
                                    ).workspace_size() == 0
    # ... and K % 512 != 0 leaves those to the split when a workspace is given
    assert P.IntGemmPlan.select(P.IntGemmDescriptor(4192, 4096, 3968, output=P.ElementKind.Bf16)
                                ).workspace_size() == 16 * 15 * 65536 * 4
    assert P.IntGemmPlan.select(P.IntGemmDescriptor(512, 512, 8192, output=P.ElementKind.I32)
                                ).workspace_size() == 4 * 32 * 65536 * 4
    # whole rounds, or a last round more than half full, or K too short: no workspace
    for m, n, k in ((4096, 4096, 4096), (4352, 2048, 4096), (256, 256, 128), (4000, 4096, 4096)):
        assert P.IntGemmPlan.select(P.IntGemmDescriptor(m, n, k, output=P.ElementKind.Bf16)).workspace_size() == 0
