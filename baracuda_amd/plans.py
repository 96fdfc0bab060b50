"""Host-side mirror of baracuda's Plan surface for this path, over the C ABI.

Mirrors (names, argument meaning, error behaviour):
  IntGemmPlan   crates/baracuda-kernels/src/gemm/int_gemm.rs:48-654
  Fp8GemmPlan   crates/baracuda-kernels/src/gemm/fp8_gemm.rs:36-767
  GemvDensePlan crates/baracuda-kernels/src/gemm/gemv_dense.rs:55-412
  GemmSku / PrecisionGuarantee  crates/baracuda-cutlass/src/types.rs:271-370
  ArchSku       crates/baracuda-kernel-vocab/src/layout.rs:43-52 (+ Gfx950)
gather_rows has no Plan in the reference (callers use the FFI directly,
crates/baracuda-kernels/tests/capture_replay_gather_gemv.rs:73-79); it is
exposed here as a function.  Every plan's ``run`` issues exactly one C-ABI
call on the given stream (torch's current stream by default), never
allocates and never synchronises.

Device buffers are torch tensors (plumbing only: the arithmetic is the HIP
library's).  Shapes are validated against the descriptor before the call.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Optional

import torch

from .ffi import lib


# ---- vocabulary ------------------------------------------------------------
class ArchSku(enum.Enum):
    Sm80 = "sm80"
    Sm89 = "sm89"
    Sm90a = "sm90a"
    Gfx950 = "gfx950"


class LayoutSku(enum.Enum):
    Rrr = "rrr"
    Rcr = "rcr"


class EpilogueKind(enum.Enum):
    Identity = "identity"
    Bias = "bias"
    BiasRelu = "bias_relu"
    BiasGelu = "bias_gelu"
    BiasSilu = "bias_silu"


class ElementKind(enum.Enum):
    F64 = "f64"
    S8 = "s8"
    U8 = "u8"
    I32 = "i32"
    F32 = "f32"
    F16 = "f16"
    Bf16 = "bf16"
    Fp8E4M3 = "fp8_e4m3"
    Fp8E5M2 = "fp8_e5m2"
    U32 = "u32"


class BackendKind(enum.Enum):
    Bespoke = "bespoke"


class MathPrecision(enum.Enum):
    Int8 = "int8"
    Fp8E4M3 = "fp8_e4m3"
    Fp8E5M2 = "fp8_e5m2"
    F64 = "f64"
    F32 = "f32"
    F16 = "f16"
    Bf16 = "bf16"


@dataclass(frozen=True)
class PrecisionGuarantee:
    math_precision: MathPrecision
    accumulator: ElementKind
    bit_stable_on_same_hardware: bool
    deterministic: bool


@dataclass(frozen=True)
class GemmSku:
    arch: ArchSku
    layout: LayoutSku
    epilogue: EpilogueKind
    element: ElementKind
    output: ElementKind
    bias_element: Optional[ElementKind] = None

    def precision_guarantee(self) -> PrecisionGuarantee:
        # types.rs:296-369: int8 accumulates in i32 and is bit-stable; the
        # gfx950 FP8 MFMA path is deterministic (fixed per-tile K order, no
        # atomics) and therefore also bit-stable on the same hardware.
        if self.element in (ElementKind.S8, ElementKind.U8):
            return PrecisionGuarantee(MathPrecision.Int8, ElementKind.I32, True, True)
        mp = MathPrecision.Fp8E5M2 if self.element == ElementKind.Fp8E5M2 else MathPrecision.Fp8E4M3
        return PrecisionGuarantee(mp, ElementKind.F32, True, True)


# ---- errors (status codes, crates/baracuda-kernels-sys/src/lib.rs:19-27) ----
class KernelError(RuntimeError):
    status = -1


class Misaligned(KernelError):
    status = 1


class InvalidProblem(KernelError):
    status = 2


class Unsupported(KernelError):
    status = 3


class WorkspaceTooSmall(KernelError):
    status = 4


class LaunchFailed(KernelError):
    status = 5


_STATUS = {1: Misaligned, 2: InvalidProblem, 3: Unsupported, 4: WorkspaceTooSmall, 5: LaunchFailed}


def check(status: int, what: str) -> None:
    if status != 0:
        raise _STATUS.get(status, KernelError)(f"{what}: status {status}")


def _ptr(t: Optional[torch.Tensor]):
    """Device address of a GPU tensor; a host tensor is rejected here rather
    than handed to a kernel, which would fault on the host address."""
    if t is None:
        return None
    if not t.is_cuda:
        raise InvalidProblem("operand tensors must be on the GPU")
    return t.data_ptr()


def _nbytes(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise InvalidProblem(msg)


def _vec(t: Optional[torch.Tensor], n: int, dtype, what: str) -> None:
    """A dense 1-D vector of exactly n elements: the kernels index it as
    contiguous memory, so a strided view would be read (or written) wrongly."""
    _need(t is not None, f"{what} is required")
    _need(t.dim() == 1 and t.is_contiguous() and t.numel() == n and t.dtype == dtype,
          f"{what} must be a contiguous 1-D {dtype} vector of {n} elements")


def _ld(t: torch.Tensor) -> int:
    _need(t.dim() == 2 and t.stride(1) == 1, "operand must be a 2-D row-major view")
    return t.stride(0)


# ---- int8 GEMM -------------------------------------------------------------
@dataclass(frozen=True)
class IntGemmDescriptor:
    m: int
    n: int
    k: int
    layout: LayoutSku = LayoutSku.Rcr
    epilogue: EpilogueKind = EpilogueKind.Identity
    output: ElementKind = ElementKind.S8     # S8 / U8 (the element, reference), I32 or Bf16 (W8A8)
    bias_element: ElementKind = ElementKind.F32   # BiasElementKind for Bias* epilogues: F32 / I32
    element: ElementKind = ElementKind.S8    # operand element (IntElement): S8, or U8 (RRR only)


class IntGemmPlan:
    """int_gemm.rs IntGemmPlan: select / can_implement / workspace_size / sku / run.

    RCR (int_gemm.rs:73-85, CUTLASS arm) and RRR (:86-124, bespoke arm) for S8
    and U8 operands (U8 takes a U8 output, sat_u8).  S8 output: D = sat_s8(rne(act(alpha*acc + beta*C + bias[n]))) for
    the Identity and Bias / BiasRelu / BiasGelu / BiasSilu epilogues, bias f32
    or i32 [N].  RCR additionally offers I32 (raw accumulator) and Bf16 (W8A8
    per-token x per-channel dequant, needs scale_a / scale_b) with Identity."""

    def __init__(self, desc: IntGemmDescriptor, sku: GemmSku):
        self.desc, self._sku = desc, sku

    @classmethod
    def select(cls, desc: IntGemmDescriptor) -> "IntGemmPlan":
        if desc.m <= 0 or desc.n <= 0 or desc.k <= 0:
            raise InvalidProblem("int GEMM problem must have positive M, N, K")
        if desc.element == ElementKind.U8:
            # U8 operands take a U8 output in both layouts: RCR is the CUTLASS
            # arm (plan.rs:2273-2346, 2570-2915), RRR the bespoke one
            # (int_gemm.rs:93-101).
            if desc.output != ElementKind.U8:
                raise Unsupported("U8 int GEMM has a U8 output")
            has_bias = desc.epilogue != EpilogueKind.Identity
            if has_bias and desc.bias_element not in (ElementKind.F32, ElementKind.I32):
                raise Unsupported(f"bias element {desc.bias_element}")
            return cls(desc, GemmSku(ArchSku.Gfx950, desc.layout, desc.epilogue, ElementKind.U8, ElementKind.U8,
                                     desc.bias_element if has_bias else None))
        if desc.element != ElementKind.S8:
            raise Unsupported(f"int GEMM element {desc.element}: S8 / U8 only")
        if desc.output not in (ElementKind.S8, ElementKind.I32, ElementKind.Bf16):
            raise Unsupported(f"int8 GEMM output {desc.output}")
        if desc.output != ElementKind.S8 and (desc.layout != LayoutSku.Rcr or
                                              desc.epilogue != EpilogueKind.Identity):
            raise Unsupported("I32 / Bf16 outputs are RCR with the Identity epilogue")
        has_bias = desc.epilogue != EpilogueKind.Identity
        if has_bias and desc.bias_element not in (ElementKind.F32, ElementKind.I32):
            raise Unsupported(f"bias element {desc.bias_element}")
        return cls(desc, GemmSku(ArchSku.Gfx950, desc.layout, desc.epilogue, ElementKind.S8, desc.output,
                                 desc.bias_element if has_bias else None))

    def sku(self) -> GemmSku:
        return self._sku

    def precision_guarantee(self) -> PrecisionGuarantee:
        return self._sku.precision_guarantee()

    def _symbol(self, suffix: str):
        d, L = self.desc, lib()
        if d.output == ElementKind.I32:
            return getattr(L, f"gemm_s8_rcr_gfx950_i32_{suffix}")
        if d.output == ElementKind.Bf16:
            return getattr(L, f"gemm_w8a8_rcr_gfx950_bf16_{suffix}")
        epi, bt = d.epilogue.value, d.bias_element.value
        if d.element == ElementKind.U8 and d.layout == LayoutSku.Rcr:
            if d.epilogue == EpilogueKind.Identity:
                return getattr(L, f"gemm_u8_rcr_gfx950_{suffix}")
            return getattr(L, f"gemm_{epi}_{bt}bias_u8_rcr_gfx950_{suffix}")
        if d.element == ElementKind.U8:
            if d.epilogue == EpilogueKind.Identity:
                return getattr(L, f"gemm_u8_rrr_gfx950_{suffix}")
            if suffix == "workspace_size":   # one requirement for the whole u8 family
                return getattr(L, "gemm_u8_rrr_gfx950_workspace_size")
            return getattr(L, f"gemm_u8_rrr_gfx950_{epi}_{bt}_{suffix}")
        if d.layout == LayoutSku.Rcr:
            if d.epilogue == EpilogueKind.Identity:
                return getattr(L, f"gemm_s8_rcr_gfx950_{suffix}")
            return getattr(L, f"gemm_{epi}_{bt}bias_s8_rcr_gfx950_{suffix}")
        if d.epilogue == EpilogueKind.Identity:
            return getattr(L, f"gemm_s8_rrr_gfx950_{suffix}")
        if suffix == "workspace_size":
            return None
        return getattr(L, f"gemm_s8_rrr_gfx950_{epi}_{bt}_{suffix}")

    def workspace_size(self) -> int:
        f = self._symbol("workspace_size")
        return 0 if f is None else f(self.desc.m, self.desc.n, self.desc.k)

    def can_implement(self, a, b, d, c=None, bias=None) -> None:
        desc = self.desc
        _need(tuple(a.shape) == (desc.m, desc.k), "A shape mismatch with descriptor (M, K)")
        if desc.layout == LayoutSku.Rcr:
            _need(tuple(b.shape) == (desc.n, desc.k), "B shape mismatch with descriptor ([N, K] = col-major [K, N])")
        else:
            _need(tuple(b.shape) == (desc.k, desc.n), "B shape mismatch with descriptor (K, N) (row-major)")
        _need(tuple(d.shape) == (desc.m, desc.n), "D shape mismatch with descriptor (M, N)")
        want = {ElementKind.S8: torch.int8, ElementKind.U8: torch.uint8, ElementKind.I32: torch.int32,
                ElementKind.Bf16: torch.bfloat16}[desc.output]
        op = torch.uint8 if desc.element == ElementKind.U8 else torch.int8
        _need(a.dtype == op and b.dtype == op and d.dtype == want, "dtype mismatch")
        if c is not None:
            _need(tuple(c.shape) == (desc.m, desc.n) and c.dtype == op, "C shape mismatch")
        if desc.epilogue != EpilogueKind.Identity:
            bdt = torch.float32 if desc.bias_element == ElementKind.F32 else torch.int32
            _need(bias is not None, "Bias* epilogue needs a bias vector")
            _need(bias.dim() == 1 and bias.numel() >= desc.n and bias.dtype == bdt and bias.is_contiguous(),
                  "bias must be a contiguous 1-D [N] vector of the descriptor's bias element")

    def run(self, a, b, d, c=None, alpha=1.0, beta=0.0, scale_a=None, scale_b=None,
            bias=None, workspace=None, stream=None) -> None:
        self.can_implement(a, b, d, c, bias)
        desc, L, s = self.desc, lib(), _stream(stream)
        if desc.output in (ElementKind.S8, ElementKind.U8):
            # beta is passed as given: with c None the RCR SKUs read D in place
            # (CUTLASS, gemm_s8_rcr_sm80.cu:87-89), the RRR SKUs skip the term.
            args = [desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                    _ptr(c), _ld(c) if c is not None else 0, _ptr(d), _ld(d)]
            if desc.epilogue != EpilogueKind.Identity:
                args.append(_ptr(bias))
            st = self._symbol("run")(*args, alpha, beta, _ptr(workspace), _nbytes(workspace), s)
        elif desc.output == ElementKind.I32:
            st = L.gemm_s8_rcr_gfx950_i32_run(desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                                              _ptr(d), _ld(d), _ptr(workspace), _nbytes(workspace), s)
        else:
            _vec(scale_a, desc.m, torch.float32, "W8A8 scale_a")
            _vec(scale_b, desc.n, torch.float32, "W8A8 scale_b")
            st = L.gemm_w8a8_rcr_gfx950_bf16_run(desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                                                 _ptr(scale_a), _ptr(scale_b), _ptr(d), _ld(d),
                                                 _ptr(workspace), _nbytes(workspace), s)
        check(st, "IntGemmPlan::run")


# ---- FP8 GEMM --------------------------------------------------------------
_FP8_ENC = {ElementKind.Fp8E4M3: "e4m3", ElementKind.Fp8E5M2: "e5m2"}


@dataclass(frozen=True)
class Fp8GemmDescriptor:
    m: int
    n: int
    k: int
    layout: LayoutSku = LayoutSku.Rcr
    epilogue: EpilogueKind = EpilogueKind.Identity
    output: ElementKind = ElementKind.Fp8E4M3   # the operand encoding (reference), or Bf16 / F32
    element: ElementKind = ElementKind.Fp8E4M3  # operand encoding: Fp8E4M3 or Fp8E5M2


class Fp8GemmPlan:
    """fp8_gemm.rs Fp8GemmPlan (:104-750): {E4M3, E5M2} x {RCR, RRR} x {Identity,
    Bias, BiasRelu, BiasGelu, BiasSilu}, fp8 out in the operand encoding:
    D = sat_fp8(act(alpha*acc + beta*dequant(C) [+ bias[n]])), bias f32 [N].
    E4M3 RCR Identity also offers Bf16 (scale_a*scale_b*acc) and F32 outputs."""

    def __init__(self, desc: Fp8GemmDescriptor, sku: GemmSku):
        self.desc, self._sku = desc, sku

    @classmethod
    def select(cls, desc: Fp8GemmDescriptor) -> "Fp8GemmPlan":
        if desc.m <= 0 or desc.n <= 0 or desc.k <= 0:
            raise InvalidProblem("FP8 GEMM problem must have positive M, N, K")
        if desc.element not in _FP8_ENC:
            raise Unsupported(f"FP8 GEMM operand element {desc.element}")
        if desc.output in (ElementKind.Bf16, ElementKind.F32):
            if (desc.element, desc.layout, desc.epilogue) != (ElementKind.Fp8E4M3, LayoutSku.Rcr,
                                                               EpilogueKind.Identity):
                raise Unsupported("Bf16 / F32 outputs are E4M3 RCR with the Identity epilogue")
        elif desc.output != desc.element:
            raise Unsupported("fp8 output must use the operand encoding")
        bias = ElementKind.F32 if desc.epilogue != EpilogueKind.Identity else None
        return cls(desc, GemmSku(ArchSku.Gfx950, desc.layout, desc.epilogue, desc.element, desc.output, bias))

    def sku(self) -> GemmSku:
        return self._sku

    def precision_guarantee(self) -> PrecisionGuarantee:
        return self._sku.precision_guarantee()

    def workspace_size(self) -> int:
        return 0

    def _prefix(self) -> str:
        d = self.desc
        return f"gemm_fp8_{_FP8_ENC[d.element]}_{d.layout.value}_gfx950"

    def run(self, a, b, d, c=None, alpha=1.0, beta=0.0, scale_a=1.0, scale_b=1.0, bias=None,
            workspace=None, stream=None) -> None:
        desc, L, s = self.desc, lib(), _stream(stream)
        bshape = (desc.n, desc.k) if desc.layout == LayoutSku.Rcr else (desc.k, desc.n)
        _need(tuple(a.shape) == (desc.m, desc.k) and tuple(b.shape) == bshape
              and tuple(d.shape) == (desc.m, desc.n), "shape mismatch with descriptor")
        _need(a.element_size() == 1 and b.element_size() == 1, "FP8 operands are 1-byte")
        if desc.output == desc.element:
            _need(d.element_size() == 1, "D must be 1-byte fp8")
            if c is None:
                beta = 0.0
            else:
                _need(tuple(c.shape) == (desc.m, desc.n) and c.element_size() == 1, "C shape mismatch")
            args = [desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                    _ptr(c), _ld(c) if c is not None else 0, _ptr(d), _ld(d)]
            if desc.epilogue == EpilogueKind.Identity:
                fn = getattr(L, f"{self._prefix()}_run")
            else:
                _need(bias is not None and bias.dtype == torch.float32 and bias.numel() >= desc.n
                      and bias.is_contiguous(), "Bias* epilogue needs a contiguous f32 [N] bias")
                fn = getattr(L, f"{self._prefix()}_{desc.epilogue.value}_run")
                args.append(_ptr(bias))
            st = fn(*args, alpha, beta, _ptr(workspace), 0, s)
        elif desc.output == ElementKind.Bf16:
            _need(d.dtype == torch.bfloat16, "D must be bf16")
            st = L.gemm_fp8_e4m3_rcr_gfx950_bf16_run(desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                                                     scale_a, scale_b, _ptr(d), _ld(d), _ptr(workspace), 0, s)
        else:
            _need(d.dtype == torch.float32, "D must be f32")
            st = L.gemm_fp8_e4m3_rcr_gfx950_f32_run(desc.m, desc.n, desc.k, _ptr(a), _ld(a), _ptr(b), _ld(b),
                                                    alpha, _ptr(d), _ld(d), _ptr(workspace), 0, s)
        check(st, "Fp8GemmPlan::run")


# ---- GEMV m = 1 ------------------------------------------------------------
_GEMV_TAG = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


@dataclass(frozen=True)
class GemvDenseDescriptor:
    n: int
    k: int
    batch: int = 1
    m: int = 1
    layout: int = 0   # RRR


class GemvDensePlan:
    """gemv_dense.rs GemvDensePlan<T> (RRR, strided batch, stride_b == 0 broadcast)."""

    def __init__(self, desc: GemvDenseDescriptor, dtype: torch.dtype):
        self.desc, self.dtype = desc, dtype

    @classmethod
    def select(cls, desc: GemvDenseDescriptor, dtype: torch.dtype) -> "GemvDensePlan":
        if dtype not in _GEMV_TAG:
            raise Unsupported(f"gemv_dense_m1 dtype {dtype}")
        if desc.m < 0 or desc.n < 0 or desc.k < 0 or desc.batch < 0 or desc.m > 1 or desc.layout != 0:
            raise InvalidProblem("gemv_dense_m1 descriptor")
        return cls(desc, dtype)

    def _fn(self, suffix):
        return getattr(lib(), f"gemv_dense_m1_{_GEMV_TAG[self.dtype]}_{suffix}")

    def workspace_size(self) -> int:
        d = self.desc
        return self._fn("workspace_size")(d.m, d.n, d.k, d.batch, d.layout)

    def can_implement(self, lda, ldb, ldd, stride_a, stride_b, stride_d) -> None:
        d = self.desc
        check(self._fn("can_implement")(d.m, d.n, d.k, d.batch, d.layout, lda, ldb, ldd,
                                        stride_a, stride_b, stride_d), "GemvDensePlan::can_implement")

    def run(self, a, b, d, *, lda, stride_a, ldb, stride_b, ldd, stride_d, alpha=1.0, beta=0.0,
            workspace=None, stream=None) -> None:
        desc = self.desc
        for t in (a, b, d):
            _need(t.dtype == self.dtype, "dtype mismatch")
        st = self._fn("run")(desc.m, desc.n, desc.k, desc.batch, desc.layout, alpha, beta,
                             _ptr(a), lda, stride_a, _ptr(b), ldb, stride_b, _ptr(d), ldd, stride_d,
                             _ptr(workspace), _nbytes(workspace), _stream(stream))
        check(st, "GemvDensePlan::run")


class GemvS8wPlan:
    """New SKU of the gemv_dense_m1 family: int8 weight-only m=1 decode GEMV."""

    def __init__(self, n: int, k: int):
        self.n, self.k = n, k

    @classmethod
    def select(cls, n: int, k: int) -> "GemvS8wPlan":
        if n < 0 or k < 0:
            raise InvalidProblem("gemv_s8w_m1 extents")
        return cls(n, k)

    def run(self, x, w, scale, d, stream=None) -> None:
        _need(w.dtype == torch.int8 and tuple(w.shape) == (self.n, self.k), "W must be int8 [N, K]")
        _vec(x, self.k, torch.bfloat16, "GEMV x")
        _vec(scale, self.n, torch.float32, "GEMV scale")
        _vec(d, self.n, torch.bfloat16, "GEMV d")
        ldw = _ld(w) if self.k > 0 else 1
        st = lib().gemv_s8w_m1_bf16_gfx950_run(self.n, self.k, _ptr(x), _ptr(w), ldw, _ptr(scale),
                                               _ptr(d), None, 0, _stream(stream))
        check(st, "GemvS8wPlan::run")


# ---- gather_rows (direct FFI in the reference) ------------------------------
_GATHER_TAG = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def gather_rows(dest: torch.Tensor, table: torch.Tensor, idx: torch.Tensor, stream=None) -> None:
    """dest[r,:] = table[idx[r],:] (idx uint32, out-of-range -> zeros)."""
    _need(table.dim() == 2 and table.is_contiguous() and dest.is_contiguous(), "contiguous 2-D table/dest")
    _need(idx.dtype == torch.uint32 and idx.is_contiguous(), "idx must be contiguous uint32")
    V, H = table.shape
    n = idx.numel()
    _need(dest.numel() == n * H and dest.dtype == table.dtype, "dest must be [n, H] of table.dtype")
    fn = getattr(lib(), f"gather_rows_{_GATHER_TAG[table.dtype]}_run")
    check(fn(_ptr(dest), _ptr(table), _ptr(idx), V, H, n, _stream(stream)), "gather_rows")


# ---- embedding forward -----------------------------------------------------
PADDING_DISABLED = -(2 ** 31)   # embedding/mod.rs:57 (kPaddingDisabled)
_EMBED_TAG = {torch.float32: "f32", torch.float64: "f64", torch.float16: "f16", torch.bfloat16: "bf16"}
_EMBED_KIND = {torch.float32: ElementKind.F32, torch.float64: ElementKind.F64,
               torch.float16: ElementKind.F16, torch.bfloat16: ElementKind.Bf16}


@dataclass(frozen=True)
class EmbeddingDescriptor:
    num_embeddings: int
    embedding_dim: int
    num_indices: int
    padding_idx: Optional[int] = None
    element: ElementKind = ElementKind.F32


@dataclass(frozen=True)
class KernelSku:
    op: str
    element: ElementKind
    aux_element: Optional[ElementKind]
    arch: ArchSku
    backend: BackendKind
    precision_guarantee: PrecisionGuarantee


class EmbeddingPlan:
    """embedding.rs EmbeddingPlan (:90-360): out[n,:] = weight[idx[n],:], zero rows
    for padding_idx and for negative / out-of-range indices; weight {f32, f64,
    f16, bf16}, indices i32 or i64 (chosen by the index tensor at run time)."""

    def __init__(self, desc: EmbeddingDescriptor, sku: KernelSku):
        self.desc, self._sku = desc, sku

    @classmethod
    def select(cls, desc: EmbeddingDescriptor) -> "EmbeddingPlan":
        if desc.num_embeddings < 0 or desc.embedding_dim < 0 or desc.num_indices < 0:
            raise InvalidProblem("EmbeddingPlan: num_embeddings / embedding_dim / num_indices "
                                 "must be non-negative")
        if desc.element not in (ElementKind.F32, ElementKind.F64, ElementKind.F16, ElementKind.Bf16):
            raise Unsupported("EmbeddingPlan: only f32, f64, f16, bf16")
        mp = MathPrecision.F64 if desc.element == ElementKind.F64 else MathPrecision.F32
        pg = PrecisionGuarantee(mp, desc.element, True, True)
        return cls(desc, KernelSku("embedding", desc.element, ElementKind.I32, ArchSku.Gfx950,
                                   BackendKind.Bespoke, pg))

    def sku(self) -> KernelSku:
        return self._sku

    def precision_guarantee(self) -> PrecisionGuarantee:
        return self._sku.precision_guarantee

    def workspace_size(self) -> int:
        return 0

    def can_implement(self, weight, indices, output) -> None:
        d = self.desc
        _need(tuple(weight.shape) == (d.num_embeddings, d.embedding_dim),
              "EmbeddingPlan: weight shape mismatch with descriptor")
        _need(indices.dim() == 1 and indices.shape[0] == d.num_indices,
              "EmbeddingPlan: indices.shape[0] mismatch with descriptor")
        _need(tuple(output.shape) == (d.num_indices, d.embedding_dim),
              "EmbeddingPlan: output shape must be [num_indices, embedding_dim]")
        _need(weight.dtype in _EMBED_KIND and _EMBED_KIND[weight.dtype] == d.element and
              output.dtype == weight.dtype, "EmbeddingPlan: element type mismatch")
        _need(indices.dtype in (torch.int32, torch.int64), "EmbeddingPlan: indices must be i32 or i64")
        _need(weight.is_contiguous() and indices.is_contiguous() and output.is_contiguous(),
              "EmbeddingPlan: tensors must be contiguous")

    def run(self, weight, indices, output, workspace=None, stream=None) -> None:
        self.can_implement(weight, indices, output)
        d = self.desc
        if d.num_indices == 0 or d.embedding_dim == 0:
            return
        pad = PADDING_DISABLED if d.padding_idx is None else d.padding_idx
        ix = "i64idx_" if indices.dtype == torch.int64 else ""
        fn = getattr(lib(), f"embedding_{ix}{_EMBED_TAG[weight.dtype]}_run")
        check(fn(d.num_indices, d.num_embeddings, d.embedding_dim, pad, _ptr(weight), _ptr(indices),
                 _ptr(output), _ptr(workspace), 0, _stream(stream)), "EmbeddingPlan::run")


# ---- grouped MoE int8 -------------------------------------------------------
class MoeS8GroupedPlan:
    """Grouped int8 expert GEMM with the moe_wmma routing contract (new SKU)."""

    def __init__(self, num_experts, topk, size_m, size_n, size_k):
        self.E, self.topk, self.size_m, self.n, self.k = num_experts, topk, size_m, size_n, size_k

    @classmethod
    def select(cls, num_experts, topk, size_m, size_n, size_k) -> "MoeS8GroupedPlan":
        check(lib().moe_s8_grouped_bf16_gfx950_can_implement(num_experts, topk, size_m, size_n, size_k),
              "MoeS8GroupedPlan::select")
        return cls(num_experts, topk, size_m, size_n, size_k)

    def workspace_size(self) -> int:
        """Always 0, as the reference's MoE plans (`moe/mod.rs:295`); a
        workspace passed to `run` anyway is ignored."""
        return int(lib().moe_s8_grouped_bf16_gfx950_workspace_size(self.E, self.topk, self.size_m, self.n, self.k))

    def run(self, x, w, sorted_token_ids, expert_ids, out, expert_counts, expert_offsets,
            scale_a, scale_w, topk_weights=None, workspace=None, stream=None) -> None:
        _need(x.dtype == torch.int8 and w.dtype == torch.int8 and out.dtype == torch.bfloat16, "dtypes")
        _need(w.numel() == self.E * self.n * self.k and x.shape[-1] == self.k, "shapes")
        _need(x.is_contiguous() and w.is_contiguous() and out.is_contiguous(), "x, w, out contiguous")
        _need(out.numel() >= self.size_m * self.n, "out too small")
        _vec(sorted_token_ids, self.size_m, torch.int32, "sorted_token_ids")
        _vec(expert_ids, self.size_m, torch.int32, "expert_ids")
        _vec(expert_counts, self.E, torch.int32, "expert_counts")
        _vec(expert_offsets, self.E + 1, torch.int32, "expert_offsets")
        _vec(scale_a, x.numel() // self.k, torch.float32, "scale_a")
        _vec(scale_w, self.E * self.n, torch.float32, "scale_w")
        if topk_weights is not None:
            _vec(topk_weights, self.size_m, torch.float32, "topk_weights")
        st = lib().moe_s8_grouped_bf16_gfx950_run(
            _ptr(x), _ptr(w), _ptr(sorted_token_ids), _ptr(expert_ids), _ptr(topk_weights), _ptr(out),
            _ptr(expert_counts), _ptr(expert_offsets), self.E, self.topk, self.size_m, self.n, self.k,
            _ptr(scale_a), _ptr(scale_w), _ptr(workspace), _nbytes(workspace), _stream(stream))
        check(st, "MoeS8GroupedPlan::run")

    def run_i32(self, x, w, sorted_token_ids, expert_ids, out, expert_counts, expert_offsets,
                stream=None) -> None:
        """The int32-accumulator SKU: out[id, n] = acc (int32 [size_m, N]),
        input row = id / topk; the same kernel as `run` without its epilogue."""
        _need(x.dtype == torch.int8 and w.dtype == torch.int8 and out.dtype == torch.int32, "dtypes")
        _need(w.numel() == self.E * self.n * self.k and x.shape[-1] == self.k, "shapes")
        _need(x.is_contiguous() and w.is_contiguous() and out.is_contiguous(), "x, w, out contiguous")
        _need(out.numel() >= self.size_m * self.n, "out too small")
        _vec(sorted_token_ids, self.size_m, torch.int32, "sorted_token_ids")
        _vec(expert_ids, self.size_m, torch.int32, "expert_ids")
        _vec(expert_counts, self.E, torch.int32, "expert_counts")
        _vec(expert_offsets, self.E + 1, torch.int32, "expert_offsets")
        st = lib().moe_s8_grouped_i32_gfx950_run(
            _ptr(x), _ptr(w), _ptr(sorted_token_ids), _ptr(expert_ids), _ptr(out),
            _ptr(expert_counts), _ptr(expert_offsets), self.E, self.topk, self.size_m, self.n, self.k,
            _stream(stream))
        check(st, "MoeS8GroupedPlan::run_i32")


# ---- per-token dynamic quantization + quantized_linear ----------------------
def dynamic_range_quantize_per_token_sym(x, scale, q, qmin=-127, qmax=127, stream=None) -> None:
    """DynamicRangeQuantizePlan (baracuda_quantize_compose.cuh:143-203): per row,
    scale = max|x|/qmax (1 for an all-zero row), q = clamp(rne(x/scale))."""
    _need(x.dim() == 2 and x.is_contiguous() and q.is_contiguous(), "x, q contiguous [N, D]")
    n, d = x.shape
    _need(tuple(q.shape) == (n, d) and q.dtype == torch.int8, "q must be int8 [N, D]")
    _need(scale.dim() == 1 and scale.is_contiguous() and scale.numel() == n,
          "scale must be a contiguous 1-D [N] vector")
    L = lib()
    if x.dtype == torch.float32:
        _need(scale.dtype == torch.float32, "f32 input takes an f32 scale")
        fn = L.dynamic_range_quantize_per_token_sym_f32_s8_run
    elif x.dtype == torch.float64:
        _need(scale.dtype == torch.float64, "f64 input takes an f64 scale")
        fn = L.dynamic_range_quantize_per_token_sym_f64_s8_run
    elif x.dtype == torch.bfloat16:
        _need(scale.dtype == torch.float32, "bf16 input takes an f32 scale")
        fn = L.dynamic_range_quantize_per_token_sym_bf16_s8_gfx950_run
    else:
        raise Unsupported(f"quantize input dtype {x.dtype}")
    check(fn(n, d, qmin, qmax, _ptr(x), _ptr(scale), _ptr(q), None, 0, _stream(stream)),
          "dynamic_range_quantize_per_token_sym")


@dataclass(frozen=True)
class QuantizedLinearDescriptor:
    m: int
    c_out: int
    k: int
    q_min: int = -127
    q_max: int = 127


class QuantizedLinearPlan:
    """quantized_linear.rs QuantizedLinearPlan (:142-386): two launches on one
    stream -- per-token activation quantization into caller scratch, then the
    W8A8 GEMM with the (sa*sw)*acc dequant epilogue.  f32 / f64 activation ->
    f32 / f64 output with scales of the same type (the reference's SKUs);
    bf16 activation -> bf16 output, f32 scales (gfx950)."""

    def __init__(self, desc: QuantizedLinearDescriptor):
        self.desc = desc

    @classmethod
    def select(cls, desc: QuantizedLinearDescriptor) -> "QuantizedLinearPlan":
        if desc.m < 0 or desc.c_out < 0 or desc.k < 0:
            raise InvalidProblem("quantized_linear extents")
        if desc.q_min > desc.q_max or desc.q_max <= 0:
            raise InvalidProblem("quantized_linear q range")
        return cls(desc)

    def workspace_size(self) -> int:
        return 0

    def run(self, activation, weight_q, weight_scale, output, act_q_scratch, act_scale_scratch,
            stream=None) -> None:
        d = self.desc
        if d.m * d.c_out == 0 or d.k == 0:
            return
        _need(tuple(activation.shape) == (d.m, d.k) and tuple(weight_q.shape) == (d.c_out, d.k),
              "activation [M,K], weight_q [C_out,K]")
        _need(tuple(output.shape) == (d.m, d.c_out), "output [M, C_out]")
        dynamic_range_quantize_per_token_sym(activation, act_scale_scratch, act_q_scratch,
                                             d.q_min, d.q_max, stream)
        L, s = lib(), _stream(stream)
        if activation.dtype == torch.float32:
            _need(output.dtype == torch.float32 and weight_scale.dtype == torch.float32, "f32 output/scales")
            st = L.quantized_linear_w8a8_f32_gfx950_run(d.m, d.c_out, d.k, _ptr(weight_q), _ptr(act_q_scratch),
                                                         _ptr(act_scale_scratch), _ptr(weight_scale),
                                                         _ptr(output), None, 0, s)
        elif activation.dtype == torch.float64:
            # quantized_linear.rs:166-171 f64 arm: f64 activation, scales and output.
            _need(output.dtype == torch.float64 and weight_scale.dtype == torch.float64 and
                  act_scale_scratch.dtype == torch.float64, "f64 output / scales")
            st = L.quantized_linear_w8a8_f64_gfx950_run(d.m, d.c_out, d.k, _ptr(weight_q), _ptr(act_q_scratch),
                                                         _ptr(act_scale_scratch), _ptr(weight_scale),
                                                         _ptr(output), None, 0, s)
        elif activation.dtype == torch.bfloat16:
            _need(output.dtype == torch.bfloat16 and weight_scale.dtype == torch.float32, "bf16 output, f32 scales")
            st = L.gemm_w8a8_rcr_gfx950_bf16_run(d.m, d.c_out, d.k, _ptr(act_q_scratch), d.k, _ptr(weight_q),
                                                 _ld(weight_q), _ptr(act_scale_scratch), _ptr(weight_scale),
                                                 _ptr(output), _ld(output), None, 0, s)
        else:
            raise Unsupported(f"quantized_linear activation dtype {activation.dtype}")
        check(st, "QuantizedLinearPlan::run")


# ---- FP8 delayed-scaling quantizer (transformer-engine shim) -----------------
class TeInvalidArgument(KernelError):
    """The shim's status 1 (baracuda-transformer-engine Error::ShimInvalidArgument)."""
    status = 1


def _te_check(status: int, what: str) -> None:
    if status == 1:
        raise TeInvalidArgument(f"{what}: status 1")
    if status == 5:
        raise LaunchFailed(f"{what}: status 5")
    if status != 0:
        raise KernelError(f"{what}: status {status}")


class Fp8Format(enum.Enum):
    """baracuda-transformer-engine lib.rs Fp8Format (FFI tags 0 / 1)."""
    E4M3 = 0
    E5M2 = 1

    def max_representable(self) -> float:
        return 448.0 if self is Fp8Format.E4M3 else 57344.0


_TE_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


class Fp8Recipe:
    """lib.rs Fp8Recipe: amax history ring + device scale / scale_inv scalars.

    new() zeroes the history and sets scale = scale_inv = 1; each cast folds
    max|x| into history[write_pos]; update_after_pass() publishes
    scale = max_repr / max(history) and advances write_pos (wrapping)."""

    def __init__(self, fmt: Fp8Format, history_len: int, device="cuda:0", stream=None):
        if history_len <= 0 or history_len > 8192:
            raise TeInvalidArgument("amax history length must be in 1..=8192")
        self.format, self.history_len, self.write_pos = fmt, history_len, 0
        self.amax_history = torch.empty(history_len, dtype=torch.float32, device=device)
        self.scale = torch.empty(1, dtype=torch.float32, device=device)
        self.scale_inv = torch.empty(1, dtype=torch.float32, device=device)
        _te_check(lib().baracuda_te_recipe_init_run(_ptr(self.amax_history), _ptr(self.scale),
                                                    _ptr(self.scale_inv), history_len, _stream(stream)),
                  "Fp8Recipe::new")

    def update_after_pass(self, stream=None) -> None:
        _te_check(lib().baracuda_te_recipe_update_run(_ptr(self.amax_history), _ptr(self.scale),
                                                      _ptr(self.scale_inv), self.history_len,
                                                      self.write_pos, self.format.value, _stream(stream)),
                  "Fp8Recipe::update_after_pass")
        self.write_pos = (self.write_pos + 1) % self.history_len

    def scale_host(self) -> float:
        torch.cuda.synchronize()
        return float(self.scale.item())

    def scale_inv_host(self) -> float:
        torch.cuda.synchronize()
        return float(self.scale_inv.item())


class Fp8CastPlan:
    """lib.rs Fp8CastPlan: output = sat_fp8(input * scale), amax folded into the recipe."""

    @classmethod
    def select(cls) -> "Fp8CastPlan":
        return cls()

    def run(self, inp: torch.Tensor, out: torch.Tensor, recipe: Fp8Recipe, stream=None) -> None:
        if inp.numel() != out.numel():
            raise TeInvalidArgument("Fp8CastPlan::run: input.len() != output.len()")
        if inp.numel() == 0:
            raise TeInvalidArgument("Fp8CastPlan::run: empty input")
        _need(inp.dtype in _TE_DTYPE and out.element_size() == 1 and inp.is_contiguous()
              and out.is_contiguous(), "Fp8CastPlan: f32/f16/bf16 contiguous input, 1-byte output")
        _te_check(lib().baracuda_te_fused_cast_amax_run(
            _ptr(inp), _ptr(out), _ptr(recipe.scale), _ptr(recipe.amax_history), recipe.write_pos,
            inp.numel(), recipe.format.value, _TE_DTYPE[inp.dtype], _stream(stream)), "Fp8CastPlan::run")


class Fp8DequantPlan:
    """lib.rs Fp8DequantPlan: output = dec(input) * scale_inv."""

    @classmethod
    def select(cls) -> "Fp8DequantPlan":
        return cls()

    def run(self, inp: torch.Tensor, out: torch.Tensor, recipe: Fp8Recipe, stream=None) -> None:
        if inp.numel() != out.numel():
            raise TeInvalidArgument("Fp8DequantPlan::run: input.len() != output.len()")
        if inp.numel() == 0:
            raise TeInvalidArgument("Fp8DequantPlan::run: empty input")
        _need(out.dtype in _TE_DTYPE and inp.element_size() == 1 and inp.is_contiguous()
              and out.is_contiguous(), "Fp8DequantPlan: 1-byte input, f32/f16/bf16 contiguous output")
        _te_check(lib().baracuda_te_dequant_run(
            _ptr(inp), _ptr(out), _ptr(recipe.scale_inv), inp.numel(), recipe.format.value,
            _TE_DTYPE[out.dtype], _stream(stream)), "Fp8DequantPlan::run")


# ---- float MoE (moe_wmma) ----------------------------------------------------
class MoeVariant(enum.Enum):
    """moe/mod.rs:68-76."""
    ScalarGguf = "scalar_gguf"
    Wmma = "wmma"
    WmmaGguf = "wmma_gguf"


@dataclass(frozen=True)
class MoeDescriptor:
    """moe/mod.rs:80-100 MoeDescriptor (d_model = size_k, d_expert = size_n)."""
    num_tokens: int
    num_experts: int
    top_k: int
    d_model: int
    d_expert: int
    variant: MoeVariant = MoeVariant.Wmma
    element: ElementKind = ElementKind.Bf16
    is_prefill: bool = True


class MoePlan:
    """moe/mod.rs:218- MoePlan for the Wmma variant over bf16 / f16 experts:
    out[sorted_token_ids[p], n] = T(sum_k x[in_row, k] * w[e, n, k] [* topk_weights])."""

    def __init__(self, desc: MoeDescriptor):
        self.desc = desc

    @classmethod
    def select(cls, desc: MoeDescriptor) -> "MoePlan":
        if (desc.num_tokens < 0 or desc.num_experts <= 0 or desc.top_k <= 0 or desc.d_model <= 0
                or desc.d_expert <= 0):
            raise InvalidProblem("MoePlan: non-positive dims")
        if desc.variant != MoeVariant.Wmma:
            raise Unsupported("gfx950 MoePlan implements the Wmma variant (GGUF blocks are out of scope)")
        if desc.element not in (ElementKind.Bf16, ElementKind.F16):
            raise Unsupported("MoePlan Wmma: bf16 or f16 elements")
        size_m = max(desc.num_tokens * desc.top_k, 1)
        check(getattr(lib(), f"moe_wmma_{desc.element.value}_can_implement")(
            desc.num_experts, desc.top_k, size_m, desc.d_expert, desc.d_model, int(desc.is_prefill)),
            "MoePlan::select")
        return cls(desc)

    def workspace_size(self) -> int:
        return 0

    def run(self, x, w, sorted_token_ids, expert_ids, out, expert_counts, expert_offsets,
            topk_weights=None, stream=None) -> None:
        d = self.desc
        dt = torch.bfloat16 if d.element == ElementKind.Bf16 else torch.float16
        _need(x.dtype == dt and w.dtype == dt and out.dtype == dt, "MoePlan: element type mismatch")
        _need(w.numel() == d.num_experts * d.d_expert * d.d_model and x.shape[-1] == d.d_model,
              "MoePlan: shapes")
        size_m = sorted_token_ids.numel()
        if size_m == 0:
            return
        st = getattr(lib(), f"moe_wmma_{d.element.value}_run")(
            _ptr(x), _ptr(w), _ptr(sorted_token_ids), _ptr(expert_ids), _ptr(topk_weights), _ptr(out),
            _ptr(expert_counts), _ptr(expert_offsets), d.num_experts, d.top_k, size_m, d.d_expert,
            d.d_model, int(d.is_prefill), None, 0, _stream(stream))
        check(st, "MoePlan::run")
