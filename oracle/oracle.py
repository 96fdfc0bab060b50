"""ctypes/numpy front end of the CPU parity oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product (baracuda_amd/).
Each function forwards to the C restatement in oracle.c, which cites the
reference file:line it follows.  ``build()`` compiles liboracle.so with gcc.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIB_PATH


def _L():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
        vp, i64, f32, f64, i32 = C.c_void_p, C.c_int64, C.c_float, C.c_double, C.c_int
        sig = {
            "bo_f32_to_bf16_bits": (C.c_uint16, [f32]),
            "bo_bf16_bits_to_f32": (f32, [C.c_uint16]),
            "bo_f32_to_f16_bits": (C.c_uint16, [f32]),
            "bo_f16_bits_to_f32": (f32, [C.c_uint16]),
            "bo_e4m3_to_f32": (f32, [C.c_uint8]),
            "bo_f32_to_e4m3_satfinite": (C.c_uint8, [f32]),
            "bo_f64_to_i32_as": (C.c_int32, [f64]),
            "bo_sat_cast_s8": (C.c_int8, [f32]),
            "bo_contraction_s8_i32": (None, [i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64]),
            "bo_contraction_f64": (None, [i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64]),
            "bo_gemm_s8_rcr_i32": (None, [i64, i64, i64, vp, i64, vp, i64, vp, i64, i64, i64, i32]),
            "bo_gemm_s8_rcr_s8": (None, [i64, i64, i64, vp, i64, vp, i64, vp, i64, vp, i64, f32, f32]),
            "bo_gemm_s8_epi": (None, [i64, i64, i64, vp, i64, vp, i64, i64, vp, i64, vp,
                                      C.c_int, vp, i64, f32, f32]),
            "bo_erf_as7126": (f32, [f32]),
            "bo_gemm_u8_epi": (None, [i64, i64, i64, vp, i64, vp, i64, i64, vp, i64, vp,
                                      C.c_int, vp, i64, f32, f32]),
            "bo_e5m2_to_f32": (f32, [C.c_uint8]),
            "bo_f32_to_e5m2_satfinite": (C.c_uint8, [f32]),
            "bo_gemm_fp8_f64": (None, [C.c_int, i64, i64, i64, vp, i64, vp, i64, i64, vp, i64, i64, i64, i32]),
            "bo_fp8_epilogue": (None, [C.c_int, i64, i64, vp, i64, vp, i64, vp, C.c_int, f32, f32, vp, i64]),
            "bo_te_cast_amax": (None, [vp, i64, f32, C.c_int, vp, vp]),
            "bo_te_dequant": (None, [vp, i64, f32, C.c_int, vp]),
            "bo_moe_grouped_f64": (None, [vp, vp, vp, vp, i32, i32, vp, i64, i64, vp]),
            "bo_embedding": (None, [vp, vp, vp, i64, i64, i64, i64, i64, i64]),
            "bo_gemm_w8a8_rcr_bf16": (None, [i64, i64, i64, vp, i64, vp, i64, vp, vp, vp, i64, i64, i64, i32]),
            "bo_gemm_fp8_e4m3_rcr_f64": (None, [i64, i64, i64, vp, i64, vp, i64, vp, i64, i64, i64, i32]),
            "bo_gemm_fp8_e4m3_rcr_f32": (None, [i64, i64, i64, vp, i64, vp, i64, vp, i64]),
            "bo_gemv_dense_m1_f64": (None, [i64, i64, i64, vp, i64, vp, i64, i64, vp, vp, i64, f64, f64]),
            "bo_gemv_s8w_m1_f64": (None, [i64, i64, vp, vp, i64, vp, i32]),
            "bo_gather_rows": (None, [vp, vp, vp, i64, i64, i64, i64]),
            "bo_moe_expert_offsets": (None, [vp, i64, C.c_int32, vp, vp]),
            "bo_quantize_per_token_sym": (None, [vp, i64, i64, C.c_int32, C.c_int32, vp, vp]),
            "bo_moe_s8_grouped_i32": (None, [vp, vp, vp, vp, C.c_int32, C.c_int32, i64, i64, i64, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype, fn.argtypes = res, args
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data


# ---- scalar codecs, vectorised over numpy arrays ---------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = _L().bo_f32_to_bf16_bits
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def e4m3_table() -> np.ndarray:
    f = _L().bo_e4m3_to_f32
    return np.array([f(i) for i in range(256)], dtype=np.float32)


def e4m3_to_f32(b) -> np.ndarray:
    return e4m3_table()[np.asarray(b, dtype=np.uint8)]


def f32_to_e4m3(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    f = _L().bo_f32_to_e4m3_satfinite
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint8).reshape(x.shape)


def f32_to_bf16_bits_fast(x) -> np.ndarray:
    """Vectorised restatement of the same RNE rule (checked against the C one)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---- contractions -----------------------------------------------------------
def contraction_s8_i32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """oracle.rs eval_contraction: a [M,K] (any strides), b [K,N] (any strides)."""
    a = np.asarray(a, dtype=np.int8)
    b = np.asarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.int32)
    sa = [s // a.itemsize for s in a.strides]
    sb = [s // b.itemsize for s in b.strides]
    _L().bo_contraction_s8_i32(m, n, k, _p(a), sa[0], sa[1], _p(b), sb[0], sb[1], _p(out), n)
    return out


def contraction_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    m, k = a.shape
    n = b.shape[1]
    out = np.zeros((m, n), dtype=np.float64)
    _L().bo_contraction_f64(m, n, k, _p(a), a.strides[0] // 8, a.strides[1] // 8,
                            _p(b), b.strides[0] // 8, b.strides[1] // 8, _p(out), n)
    return out


def gemm_s8_rcr_i32(a, b, rows=None, nthreads=1) -> np.ndarray:
    """A [M,K] int8, B [N,K] int8 (col-major [K,N]); returns acc int32 [len(rows), N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    r0, r1 = rows if rows is not None else (0, m)
    out = np.zeros((m, n), dtype=np.int32)
    _L().bo_gemm_s8_rcr_i32(m, n, k, _p(a), k, _p(b), k, _p(out), n, r0, r1, nthreads)
    return out[r0:r1]


def gemm_s8_rcr_s8(a, b, alpha, beta=0.0, c=None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    d = np.zeros((m, n), dtype=np.int8)
    cp = None if c is None else np.ascontiguousarray(c, dtype=np.int8)
    _L().bo_gemm_s8_rcr_s8(m, n, k, _p(a), k, _p(b), k, None if cp is None else _p(cp), n,
                           _p(d), n, alpha, beta)
    return d


ACTS = {None: 0, "relu": 1, "gelu": 2, "silu": 3}


def gemm_s8_epi(a, b, layout, alpha, beta=0.0, c=None, bias=None, act=None) -> np.ndarray:
    """int8-out GEMM with optional C, bias [N] (any numeric dtype, read as f32)
    and activation. layout "rcr": b is [N, K]; "rrr": b is [K, N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    if layout == "rcr":
        n = b.shape[0]
        sbk, sbn = 1, k
    elif layout == "rrr":
        n = b.shape[1]
        sbk, sbn = n, 1
    else:
        raise ValueError(layout)
    d = np.zeros((m, n), dtype=np.int8)
    cp = None if c is None else np.ascontiguousarray(c, dtype=np.int8)
    bp = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.float32))
    _L().bo_gemm_s8_epi(m, n, k, _p(a), k, _p(b), sbk, sbn, None if cp is None else _p(cp), n,
                        None if bp is None else _p(bp), ACTS[act], _p(d), n, alpha, beta)
    return d


FP8_FMT = {"e4m3": 0, "e5m2": 1}


def e5m2_table() -> np.ndarray:
    f = _L().bo_e5m2_to_f32
    return np.array([f(i) for i in range(256)], dtype=np.float32)


def fp8_to_f32(b, fmt: str) -> np.ndarray:
    t = e4m3_table() if fmt == "e4m3" else e5m2_table()
    return t[np.asarray(b, dtype=np.uint8)]


def f32_to_fp8(x, fmt: str) -> np.ndarray:
    f = _L().bo_f32_to_e4m3_satfinite if fmt == "e4m3" else _L().bo_f32_to_e5m2_satfinite
    x = np.asarray(x, dtype=np.float32)
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint8).reshape(x.shape)


def gemm_fp8_f64(a_bits, b_bits, fmt: str, layout: str = "rcr", rows=None, nthreads=1) -> np.ndarray:
    """Exact f64 accumulator; layout "rcr": b is [N, K]; "rrr": b is [K, N]."""
    a = np.ascontiguousarray(a_bits, dtype=np.uint8)
    b = np.ascontiguousarray(b_bits, dtype=np.uint8)
    m, k = a.shape
    if layout == "rcr":
        n, sbk, sbn = b.shape[0], 1, k
    else:
        n, sbk, sbn = b.shape[1], b.shape[1], 1
    r0, r1 = rows if rows is not None else (0, m)
    acc = np.zeros((r1 - r0, n), dtype=np.float64)
    _L().bo_gemm_fp8_f64(FP8_FMT[fmt], m, n, k, _p(a), k, _p(b), sbk, sbn, _p(acc), n, r0, r1, nthreads)
    return acc


def fp8_epilogue(acc, fmt: str, alpha, beta=0.0, c=None, bias=None, act=None) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.float64)
    m, n = acc.shape
    d = np.zeros((m, n), dtype=np.uint8)
    cp = None if c is None else np.ascontiguousarray(c, dtype=np.uint8)
    bp = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _L().bo_fp8_epilogue(FP8_FMT[fmt], m, n, _p(acc), n, None if cp is None else _p(cp), n,
                         None if bp is None else _p(bp), ACTS[act], alpha, beta, _p(d), n)
    return d


def te_cast_amax(x_f32, scale: float, fmt: str):
    """fused_cast_amax on f32-widened input: (fp8 bits, amax)."""
    x = np.ascontiguousarray(x_f32, dtype=np.float32).ravel()
    out = np.zeros(x.size, dtype=np.uint8)
    amax = np.zeros(1, dtype=np.float32)
    _L().bo_te_cast_amax(_p(x), x.size, scale, FP8_FMT[fmt], _p(out), _p(amax))
    return out, float(amax[0])


def te_dequant_f32(bits, scale_inv: float, fmt: str) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint8).ravel()
    y = np.zeros(b.size, dtype=np.float32)
    _L().bo_te_dequant(_p(b), b.size, scale_inv, FP8_FMT[fmt], _p(y))
    return y


TE_MAX_REPR = {"e4m3": 448.0, "e5m2": 57344.0}


def te_recipe_update(history, fmt: str, write_pos: int):
    """recipe_update_kernel: (scale, scale_inv, new history) in f32."""
    h = np.asarray(history, dtype=np.float32).copy()
    amax = np.float32(0.0)
    for v in h:
        if v > amax:
            amax = v
    if not amax > 0:
        amax = np.float32(1.0)
    if not np.isfinite(amax):
        amax = np.float32(TE_MAX_REPR[fmt])
    mr = np.float32(TE_MAX_REPR[fmt])
    scale, scale_inv = np.float32(mr / amax), np.float32(amax / mr)
    h[write_pos] = 0.0
    return float(scale), float(scale_inv), h


PADDING_DISABLED = -(2 ** 31)


def embedding(weight, idx, padding_idx=None) -> np.ndarray:
    """weight [V, D] (any 2/4/8-byte dtype), idx i32 or i64 [N] -> [N, D]."""
    weight = np.ascontiguousarray(weight)
    idx = np.ascontiguousarray(idx)
    assert idx.dtype in (np.int32, np.int64)
    V, D = weight.shape
    out = np.empty((idx.shape[0], D), dtype=weight.dtype)
    pad = PADDING_DISABLED if padding_idx is None else padding_idx
    _L().bo_embedding(_p(out), _p(weight), _p(idx), idx.itemsize, idx.shape[0], V, D,
                      weight.itemsize, pad)
    return out


def gemm_u8_epi(a, b, layout, alpha, beta=0.0, c=None, bias=None, act=None) -> np.ndarray:
    """u8 twin of gemm_s8_epi (u8 operands, C and output)."""
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    m, k = a.shape
    if layout == "rcr":
        n, sbk, sbn = b.shape[0], 1, k
    else:
        n, sbk, sbn = b.shape[1], b.shape[1], 1
    d = np.zeros((m, n), dtype=np.uint8)
    cp = None if c is None else np.ascontiguousarray(c, dtype=np.uint8)
    bp = None if bias is None else np.ascontiguousarray(np.asarray(bias).astype(np.float32))
    _L().bo_gemm_u8_epi(m, n, k, _p(a), k, _p(b), sbk, sbn, None if cp is None else _p(cp), n,
                        None if bp is None else _p(bp), ACTS[act], _p(d), n, alpha, beta)
    return d


def moe_grouped_f64(x_f32, w_f32, sorted_ids, offsets, topk, topk_w=None, out_rows=None) -> np.ndarray:
    """Float MoE reference: x [rows, K], w [E, N, K] (f32 values), f64 out [out_rows, N]."""
    x = np.ascontiguousarray(x_f32, dtype=np.float32)
    w = np.ascontiguousarray(w_f32, dtype=np.float32)
    sid = np.ascontiguousarray(sorted_ids, dtype=np.int32)
    off = np.ascontiguousarray(offsets, dtype=np.int32)
    E, n, k = w.shape
    rows = out_rows if out_rows is not None else int(sid.max()) + 1
    out = np.full((rows, n), np.nan)
    tw = None if topk_w is None else np.ascontiguousarray(topk_w, dtype=np.float32)
    _L().bo_moe_grouped_f64(_p(x), _p(w), _p(sid), _p(off), E, topk, None if tw is None else _p(tw), n, k, _p(out))
    return out


def erf_as7126(x: float) -> float:
    return _L().bo_erf_as7126(x)


def gemm_w8a8_bf16(a, w, sa, sw, rows=None, nthreads=1) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    sa = np.ascontiguousarray(sa, dtype=np.float32)
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    m, k = a.shape
    n = w.shape[0]
    r0, r1 = rows if rows is not None else (0, m)
    d = np.zeros((m, n), dtype=np.uint16)
    _L().bo_gemm_w8a8_rcr_bf16(m, n, k, _p(a), k, _p(w), k, _p(sa), _p(sw), _p(d), n, r0, r1, nthreads)
    return d[r0:r1]


def gemm_fp8_e4m3_f64(a_bits, b_bits, rows=None, nthreads=1) -> np.ndarray:
    a = np.ascontiguousarray(a_bits, dtype=np.uint8)
    b = np.ascontiguousarray(b_bits, dtype=np.uint8)
    m, k = a.shape
    n = b.shape[0]
    r0, r1 = rows if rows is not None else (0, m)
    acc = np.zeros((m, n), dtype=np.float64)
    _L().bo_gemm_fp8_e4m3_rcr_f64(m, n, k, _p(a), k, _p(b), k, _p(acc), n, r0, r1, nthreads)
    return acc[r0:r1]


def gemm_fp8_e4m3_f32(a_bits, b_bits) -> np.ndarray:
    a = np.ascontiguousarray(a_bits, dtype=np.uint8)
    b = np.ascontiguousarray(b_bits, dtype=np.uint8)
    m, k = a.shape
    n = b.shape[0]
    acc = np.zeros((m, n), dtype=np.float32)
    _L().bo_gemm_fp8_e4m3_rcr_f32(m, n, k, _p(a), k, _p(b), k, _p(acc), n)
    return acc


def gemv_dense_m1_f64(a, b, d_init, n, k, batch, stride_a, ldb, stride_b, stride_d, alpha, beta):
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    d_init = np.ascontiguousarray(d_init, dtype=np.float64)
    d = d_init.copy()
    _L().bo_gemv_dense_m1_f64(n, k, batch, _p(a), stride_a, _p(b), ldb, stride_b, _p(d_init), _p(d),
                              stride_d, alpha, beta)
    return d


def gemv_s8w_m1_f64(x_bf16_bits, w, nthreads=1) -> np.ndarray:
    x = np.ascontiguousarray(x_bf16_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.int8)
    n, k = w.shape
    acc = np.zeros(n, dtype=np.float64)
    _L().bo_gemv_s8w_m1_f64(n, k, _p(x), _p(w), k, _p(acc), nthreads)
    return acc


def gather_rows(table: np.ndarray, idx: np.ndarray) -> np.ndarray:
    table = np.ascontiguousarray(table)
    idx = np.ascontiguousarray(idx, dtype=np.uint32)
    V, H = table.shape
    dest = np.full((idx.size, H), 0x5A, dtype=np.uint8).view(table.dtype).reshape(idx.size, H) \
        if table.dtype.itemsize == 1 else np.empty((idx.size, H), dtype=table.dtype)
    _L().bo_gather_rows(_p(dest), _p(table), _p(idx), V, H, idx.size, table.dtype.itemsize)
    return dest


def quantize_per_token_sym(x, qmin=-127, qmax=127):
    """Returns (q int8 [N,D], scale f32 [N]); x is read as f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, d = x.shape
    q = np.zeros((n, d), dtype=np.int8)
    s = np.zeros(n, dtype=np.float32)
    _L().bo_quantize_per_token_sym(_p(x), n, d, qmin, qmax, _p(s), _p(q))
    return q, s


def moe_expert_offsets(expert_ids: np.ndarray, num_experts: int):
    e = np.ascontiguousarray(expert_ids, dtype=np.int32)
    counts = np.zeros(num_experts, dtype=np.int32)
    offs = np.zeros(num_experts + 1, dtype=np.int32)
    _L().bo_moe_expert_offsets(_p(e), e.size, num_experts, _p(counts), _p(offs))
    return counts, offs


def moe_s8_grouped_i32(x, w, sorted_ids, offsets, topk, size_m) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    s = np.ascontiguousarray(sorted_ids, dtype=np.int32)
    o = np.ascontiguousarray(offsets, dtype=np.int32)
    E, n, k = w.shape
    acc = np.zeros((size_m, n), dtype=np.int32)
    _L().bo_moe_s8_grouped_i32(_p(x), _p(w), _p(s), _p(o), E, topk, size_m, n, k, _p(acc))
    return acc


def scalar(name):
    return getattr(_L(), name)
