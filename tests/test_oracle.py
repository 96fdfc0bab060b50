"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Every oracle function is checked against something it was not written from:
the reference's own hand-computed vectors, a library routine (torch / numpy
casts and int64 matmul), closed forms, or brute force on tiny inputs.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from oracle.inputs import int8_uniform, moe_routing, rng
from tests.golden import __file__ as _g  # noqa: F401  (package marker)

GOLD = __import__("pathlib").Path(__file__).resolve().parent / "golden"


# ---- scalar codecs -----------------------------------------------------------
def _specials():
    vals = [0.0, -0.0, 1.0, -1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40, -1e-45,
            float("inf"), float("-inf"), 65504.0, 65520.0, 448.0, 464.0, 2 ** -6, 2 ** -9, 2 ** -10]
    g = rng(11)
    rnd = np.concatenate([g.standard_normal(4000) * 10 ** g.uniform(-8, 8, 4000),
                          g.uniform(-500, 500, 4000)]).astype(np.float32)
    return np.concatenate([np.array(vals, np.float32), rnd])


def test_bf16_rne_matches_torch_cast():
    # oracle.rs:397-404 vs torch's f32->bf16 (round to nearest even).
    x = _specials()
    got = O.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(O.f32_to_bf16_bits_fast(x), got)


def test_bf16_nan_stays_quiet_nan():
    nan = np.array([np.float32("nan"), np.uint32(0x7f800001).view(np.float32)], np.float32)
    b = O.f32_to_bf16_bits(nan)
    assert all(math.isnan(v) for v in O.bf16_bits_to_f32(b))
    assert all((v & 0x0040) for v in b)


def test_bf16_ties_to_even_closed_form():
    # 1 + 2^-8 is exactly half an ulp above 1.0 -> stays 1.0 (even); 1 + 3*2^-8 -> rounds up.
    assert O.scalar("bo_f32_to_bf16_bits")(1.0 + 2 ** -8) == 0x3F80
    assert O.scalar("bo_f32_to_bf16_bits")(1.0 + 3 * 2 ** -8) == 0x3F82


def test_f16_matches_numpy_cast():
    x = _specials()
    x = x[np.isfinite(x)]
    got = np.array([O.scalar("bo_f32_to_f16_bits")(float(v)) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([O.scalar("bo_f16_bits_to_f32")(int(v)) for v in want], np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


def test_e4m3_decode_table_matches_torch_float8_e4m3fn():
    # OCP E4M3 spec decode vs torch.float8_e4m3fn, all 256 codes.
    got = O.e4m3_table()
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert nan.sum() == 2 and np.nanmax(got) == 448.0


def test_e4m3_encode_matches_torch_in_range_and_saturates():
    x = _specials()
    x = x[np.isfinite(x)]
    inr = np.abs(x) <= 448.0
    got = O.f32_to_e4m3(x[inr])
    want = torch.from_numpy(x[inr]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)
    over = O.f32_to_e4m3(np.array([449.0, 1e6, -1e30, np.inf, -np.inf], np.float32))
    assert list(over) == [0x7E, 0x7E, 0xFE, 0x7E, 0xFE]
    # brute force: every code round-trips through decode -> encode
    tab = O.e4m3_table()
    codes = [c for c in range(256) if not math.isnan(tab[c])]
    back = O.f32_to_e4m3(tab[codes])
    for c, b in zip(codes, back):
        assert b == c or (tab[c] == 0.0 and tab[b] == 0.0)


def test_rust_as_i32_semantics():
    f = O.scalar("bo_f64_to_i32_as")
    assert f(float("nan")) == 0
    assert f(3e9) == 2 ** 31 - 1 and f(-3e9) == -(2 ** 31)
    assert f(-2.9) == -2 and f(2.9) == 2


def test_sat_cast_s8_round_half_even_and_clamp():
    f = O.scalar("bo_sat_cast_s8")
    assert [f(v) for v in (0.5, 1.5, 2.5, -0.5, -2.5, 126.6, 200.0, -300.0)] == [0, 2, 2, 0, -2, 127, 127, -128]


# ---- contraction (oracle.rs eval_contraction) ---------------------------------
def test_contraction_reference_hand_vector():
    # oracle.rs:2433-2480: [[1,2,3],[4,5,6]] . [[10,11],[12,13],[14,15]].
    lhs = np.array([[1, 2, 3], [4, 5, 6]], np.float64)
    rhs = np.array([[10, 11], [12, 13], [14, 15]], np.float64)
    assert O.contraction_f64(lhs, rhs).tolist() == [[76, 82], [184, 199]]
    # rhs stored transposed ([N,K] row-major) read through physical strides
    rhs_t = np.ascontiguousarray(rhs.T).T
    assert O.contraction_f64(lhs, rhs_t).tolist() == [[76, 82], [184, 199]]
    assert O.contraction_s8_i32(lhs.astype(np.int8), rhs.astype(np.int8)).tolist() == [[76, 82], [184, 199]]


def test_contraction_matches_golden_config1():
    z = np.load(GOLD / "config1_s8_rcr_256.npz")
    # B is [N,K] row-major == column-major [K,N]: pass the [K,N] view.
    got = O.contraction_s8_i32(z["a"], z["b"].T)
    assert np.array_equal(got, z["c"])
    assert np.array_equal(O.gemm_s8_rcr_i32(z["a"], z["b"]), z["c"])
    assert np.array_equal(O.gemm_s8_rcr_i32(z["a"], z["b"], nthreads=4), z["c"])


@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 5, 7), (100, 70, 50), (64, 64, 32)])
def test_gemm_i32_brute_force(shape):
    m, n, k = shape
    g = rng(sum(shape))
    a, b = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    want = np.array([[sum(int(a[i, t]) * int(b[j, t]) for t in range(k)) for j in range(n)] for i in range(m)])
    assert np.array_equal(O.gemm_s8_rcr_i32(a, b), want)


def test_gemm_s8_sat_epilogue_reference_pattern():
    # int8_smoke.rs:159-172 inputs, alpha = 0.125, beta = 0.
    m = n = k = 128
    a = ((np.arange(m * k) * 7) % 15 - 7).astype(np.int8).reshape(m, k)
    b = ((np.arange(k * n) * 11) % 13 - 6).astype(np.int8).reshape(n, k)   # col-major [K,N]
    acc = a.astype(np.int64) @ b.astype(np.int64).T
    want = np.clip(np.rint(np.float32(0.125) * acc.astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(O.gemm_s8_rcr_s8(a, b, 0.125), want)
    c = ((np.arange(m * n) * 3) % 9 - 4).astype(np.int8).reshape(m, n)
    z = np.float32(0.125) * acc.astype(np.float32) + np.float32(0.5) * c.astype(np.float32)
    assert np.array_equal(O.gemm_s8_rcr_s8(a, b, 0.125, 0.5, c), np.clip(np.rint(z), -128, 127).astype(np.int8))


def test_erf_as7126_against_libm():
    # A&S 7.1.26 has |error| <= 1.5e-7; f32 evaluation adds a few ulp.
    xs = np.linspace(-6, 6, 2001, dtype=np.float32)
    err = max(abs(O.erf_as7126(float(x)) - math.erf(float(x))) for x in xs)
    assert err < 1e-6
    assert O.erf_as7126(0.0) == 0.0 and O.erf_as7126(-2.0) == -O.erf_as7126(2.0)


def _mk_bias(n, kind):
    # int8_rrr_smoke.rs bias patterns: f32 ((j%5)-2)*0.5, i32 ((j%5)-2)*2.
    j = np.arange(n)
    return ((j % 5) - 2) * 0.5 if kind == "f32" else ((j % 5) - 2) * 2


@pytest.mark.parametrize("act", [None, "relu", "gelu", "silu"])
@pytest.mark.parametrize("shape", [(64, 64, 32), (100, 70, 50)])
def test_gemm_s8_epi_closed_forms(act, shape):
    m, n, k = shape
    g = rng(m + n + k)
    a, bt = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    c = int8_uniform(g, (m, n))
    bias = _mk_bias(n, "f32")
    acc = a.astype(np.int64) @ bt.astype(np.int64).T
    z = (np.float32(0.125) * acc.astype(np.float32) + np.float32(0.5) * c.astype(np.float32)
         + bias.astype(np.float32)).astype(np.float32)
    if act == "relu":
        z = np.maximum(z, np.float32(0))
    elif act == "gelu":
        z = np.float32(0.5) * z * (1 + np.vectorize(math.erf)(z / math.sqrt(2))).astype(np.float32)
    elif act == "silu":
        z = (z / (1 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    want = np.clip(np.rint(z), -128, 127).astype(np.int8)
    rcr = O.gemm_s8_epi(a, bt, "rcr", 0.125, 0.5, c, bias, act)
    rrr = O.gemm_s8_epi(a, np.ascontiguousarray(bt.T), "rrr", 0.125, 0.5, c, bias, act)
    assert np.array_equal(rcr, rrr)               # layout only changes indexing
    diff = np.abs(rcr.astype(int) - want.astype(int))
    if act in (None, "relu"):
        assert diff.max() == 0
    else:                                         # approximated erf / f32 exp
        assert diff.max() <= 1 and (diff != 0).mean() < 0.01
    # no bias, no C: the plain int8 epilogue
    assert np.array_equal(O.gemm_s8_epi(a, bt, "rcr", 0.125), O.gemm_s8_rcr_s8(a, bt, 0.125))


def test_w8a8_bf16_epilogue_against_torch():
    g = rng(2)
    m, n, k = 64, 96, 160
    a, w = int8_uniform(g, (m, k)), int8_uniform(g, (n, k))
    sa = g.uniform(0.005, 0.02, m).astype(np.float32)
    sw = g.uniform(0.001, 0.01, n).astype(np.float32)
    acc = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    y = (sa[:, None] * sw[None, :]).astype(np.float32) * acc
    want = torch.from_numpy(y).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.gemm_w8a8_bf16(a, w, sa, sw), want)
    assert np.array_equal(O.gemm_w8a8_bf16(a, w, sa, sw, rows=(5, 9), nthreads=2), want[5:9])


def test_fp8_gemm_against_numpy():
    g = rng(3)
    m, n, k = 40, 24, 96
    a = O.f32_to_e4m3(g.standard_normal((m, k)).astype(np.float32))
    b = O.f32_to_e4m3(g.standard_normal((n, k)).astype(np.float32))
    da, db = O.e4m3_to_f32(a).astype(np.float64), O.e4m3_to_f32(b).astype(np.float64)
    assert np.allclose(O.gemm_fp8_e4m3_f64(a, b), da @ db.T, rtol=0, atol=1e-9)
    # f32 K-ascending (fp8_e4m3_rcr_smoke.rs:51-76) vs an explicit float32 loop
    want = np.zeros((m, n), np.float32)
    for t in range(k):
        want += (da[:, t:t + 1].astype(np.float32) * db[:, t].astype(np.float32)[None, :])
    assert np.array_equal(O.gemm_fp8_e4m3_f32(a, b), want)


def test_gemv_dense_f64_against_numpy():
    g = rng(4)
    n, k, batch = 37, 19, 3
    a = g.standard_normal(batch * k)
    b = g.standard_normal(k * n)          # stride_b = 0: GQA broadcast
    d0 = g.standard_normal(batch * n)
    got = O.gemv_dense_m1_f64(a, b, d0, n, k, batch, k, n, 0, n, 0.5, 0.25)
    want = 0.5 * (a.reshape(batch, k) @ b.reshape(k, n)) + 0.25 * d0.reshape(batch, n)
    assert np.allclose(got.reshape(batch, n), want, rtol=1e-12, atol=1e-12)


def test_gemv_s8w_against_numpy():
    g = rng(4)
    n, k = 33, 1000
    w = int8_uniform(g, (n, k))
    xb = O.f32_to_bf16_bits_fast(g.standard_normal(k).astype(np.float32))
    want = w.astype(np.float64) @ O.bf16_bits_to_f32(xb).astype(np.float64)
    assert np.allclose(O.gemv_s8w_m1_f64(xb, w, nthreads=3), want, rtol=1e-13, atol=1e-12)


def test_gather_rows_reference_golden_and_oob():
    z = np.load(GOLD / "wte_gather.npz")
    assert np.array_equal(O.gather_rows(z["table"], z["idx"]), z["expected"])
    t = np.arange(20, dtype=np.uint16).reshape(5, 4)
    got = O.gather_rows(t, np.array([4, 5, 0, 99], np.uint32))
    assert got.tolist() == [[16, 17, 18, 19], [0, 0, 0, 0], [0, 1, 2, 3], [0, 0, 0, 0]]


def test_moe_routing_offsets_and_grouped_gemm():
    E, topk, tokens, n, k = 8, 2, 64, 24, 40
    sorted_ids, expert_ids = moe_routing(tokens, E, topk, seed=5)
    counts, offs = O.moe_expert_offsets(expert_ids, E)
    assert np.array_equal(counts, np.bincount(expert_ids, minlength=E))
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(counts)]))
    g = rng(6)
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    got = O.moe_s8_grouped_i32(x, w, sorted_ids, offs, topk, tokens * topk)
    for p, e in zip(sorted_ids, expert_ids):
        want = w[e].astype(np.int64) @ x[p // topk].astype(np.int64)
        assert np.array_equal(got[p], want)


def test_moe_expert_offsets_skip_out_of_range_ids():
    # ids outside [0, E) are not counted (and never index past the counters)
    E = 4
    ids = np.array([0, 0, 1, -1, 3, 7, 4, 3, 1 << 20], dtype=np.int32)
    counts, offs = O.moe_expert_offsets(ids, E)
    assert counts.tolist() == [2, 1, 0, 2]
    assert offs.tolist() == [0, 2, 3, 3, 5]
    counts, offs = O.moe_expert_offsets(np.full(9, E, dtype=np.int32), E)
    assert counts.tolist() == [0] * E and offs.tolist() == [0] * (E + 1)


def test_moe_routing_is_zipf_and_topk_distinct():
    sorted_ids, expert_ids = moe_routing(4096, 8, 2, seed=5)
    assert sorted(sorted_ids.tolist()) == list(range(8192))
    pair_e = np.empty(8192, np.int32)
    pair_e[sorted_ids] = expert_ids
    assert np.all(pair_e[0::2] != pair_e[1::2])
    cnt = np.bincount(expert_ids, minlength=8)
    assert cnt[0] > cnt[7] * 2


# ---- per-token dynamic quantization (baracuda_quantize_compose.cuh:143-203) --
def _np_quant(x, qmin, qmax):
    x = x.astype(np.float32)
    m = np.abs(x).max(axis=1)
    s = np.where(m > 0, m / np.float32(qmax), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / s).astype(np.float32)
    q = np.clip(np.rint((x * inv[:, None]).astype(np.float32)), qmin, qmax).astype(np.int8)
    return q, s


def test_quantize_per_token_reference_fixture():
    # quantized_linear_smoke.rs:95-101 activation (two rows, per-token ranges).
    a = np.array([[0.5, -0.3, 0.8, 1.2, -0.4, 0.6, 0.9, -0.7],
                  [4.0, -2.5, 1.8, -3.2, 2.1, -1.4, 0.9, 3.6]], np.float32)
    q, s = O.quantize_per_token_sym(a)
    assert s.tolist() == [np.float32(1.2) / np.float32(127), np.float32(4.0) / np.float32(127)]
    assert q[0, 3] == 127 and q[1, 0] == 127          # the row max maps to qmax
    wq, ws = _np_quant(a, -127, 127)
    assert np.array_equal(q, wq) and np.array_equal(s, ws)


@pytest.mark.parametrize("qmin,qmax", [(-127, 127), (-128, 127), (-20, 20)])
def test_quantize_per_token_against_numpy(qmin, qmax):
    g = rng(17)
    x = (g.standard_normal((40, 333)) * 10 ** g.uniform(-3, 3, (40, 1))).astype(np.float32)
    x[3] = 0.0                    # all-zero row -> scale 1, q 0
    x[5, 7] = 1e4                 # one dominant value
    q, s = O.quantize_per_token_sym(x, qmin, qmax)
    wq, ws = _np_quant(x, qmin, qmax)
    assert np.array_equal(q, wq) and np.array_equal(s, ws)
    assert s[3] == 1.0 and not q[3].any()


# ---- embedding ---------------------------------------------------------------
# embedding_smoke.rs cases: (V, D, weight(i), idx, padding_idx).
EMBED_REF_CASES = [
    (5, 4, lambda i: i * 0.25 + 1.0, [1, 3, 0], None, np.float32),
    (5, 3, lambda i: i * -0.5 + 2.0, [4, 2, 0, 1], None, np.float64),
    (5, 4, lambda i: i + 1.0, [0, 2, 4, -1], 0, np.float32),
    (4, 3, lambda i: i * 0.5 - 1.0, [3, 0, 1], None, np.float16),
]


@pytest.mark.parametrize("case", range(len(EMBED_REF_CASES)))
@pytest.mark.parametrize("idx_dtype", [np.int32, np.int64])
def test_embedding_reference_cases(case, idx_dtype):
    V, D, f, idx, pad, dt = EMBED_REF_CASES[case]
    w = np.array([f(i) for i in range(V * D)], dtype=dt).reshape(V, D)
    got = O.embedding(w, np.array(idx, dtype=idx_dtype), pad)
    want = np.zeros((len(idx), D), dt)
    for r, v in enumerate(idx):
        if v != pad and 0 <= v < V:
            want[r] = w[v]
    assert got.tobytes() == want.tobytes()


def test_embedding_padding_literal():
    # embedding_f32_padding_idx_zeros_row written out: weight[i] = i + 1.
    w = (np.arange(20, dtype=np.float32) + 1).reshape(5, 4)
    got = O.embedding(w, np.array([0, 2, 4, -1], np.int32), 0)
    assert got.tolist() == [[0] * 4, [9, 10, 11, 12], [17, 18, 19, 20], [0] * 4]
    # the i32 sentinel never matches a valid row; a huge i64 index is out of range
    big = np.array([2 ** 40, 3, -(2 ** 31)], np.int64)
    assert O.embedding(w, big).tolist() == [[0] * 4, [13, 14, 15, 16], [0] * 4]


# ---- e5m2 / FP8 epilogue -------------------------------------------------------
def test_e5m2_decode_table_matches_torch_float8_e5m2():
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e5m2).float().numpy()
    got = O.e5m2_table()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])     # includes +-inf at 0x7c / 0xfc


def test_e5m2_encode_matches_torch_in_range_and_saturates():
    x = _specials()
    x = x[np.isfinite(x) & (np.abs(x) <= 57344.0)]
    want = torch.from_numpy(x).to(torch.float8_e5m2).view(torch.uint8).numpy()
    assert np.array_equal(O.f32_to_fp8(x, "e5m2"), want)
    # satfinite: beyond max-finite (incl. the values RNE would send to inf) -> 0x7b
    sat = np.array([61440.0, 1e6, np.inf, -70000.0, -np.inf], np.float32)
    assert O.f32_to_fp8(sat, "e5m2").tolist() == [0x7B, 0x7B, 0x7B, 0xFB, 0xFB]
    assert O.f32_to_fp8(np.array([np.nan], np.float32), "e5m2")[0] & 0x7F == 0x7F
    # ties to even on the 2^-16 subnormal grid and at a normal midpoint
    assert O.f32_to_fp8(np.array([2 ** -17, 3 * 2 ** -17, 1.125, 1.375], np.float32), "e5m2").tolist() == \
        [0x00, 0x02, 0x3C, 0x3E]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("act", [None, "relu", "gelu", "silu"])
def test_fp8_gemm_and_epilogue_closed_forms(fmt, act):
    m, n, k = 37, 29, 45
    g = rng(9)
    a = O.f32_to_fp8(g.standard_normal((m, k)).astype(np.float32), fmt)
    bt = O.f32_to_fp8(g.standard_normal((n, k)).astype(np.float32), fmt)
    c = O.f32_to_fp8(g.standard_normal((m, n)).astype(np.float32), fmt)
    fa, fb = O.fp8_to_f32(a, fmt).astype(np.float64), O.fp8_to_f32(bt, fmt).astype(np.float64)
    acc = O.gemm_fp8_f64(a, bt, fmt, "rcr")
    assert np.array_equal(acc, fa @ fb.T)
    assert np.array_equal(O.gemm_fp8_f64(a, np.ascontiguousarray(bt.T), fmt, "rrr"), acc)
    assert np.array_equal(O.gemm_fp8_f64(a, bt, fmt, rows=(5, 9)), acc[5:9])
    bias = (((np.arange(n) % 5) - 2) * 0.5).astype(np.float32)
    z = (np.float32(0.25) * acc.astype(np.float32) + np.float32(0.5) * O.fp8_to_f32(c, fmt)
         + bias).astype(np.float32)
    if act == "relu":
        z = np.maximum(z, np.float32(0))
    elif act == "gelu":
        z = (np.float32(0.5) * z * (1 + np.vectorize(math.erf)(z / math.sqrt(2)))).astype(np.float32)
    elif act == "silu":
        z = (z / (1 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    want = O.f32_to_fp8(z, fmt)
    got = O.fp8_epilogue(acc, fmt, 0.25, 0.5, c, bias, act)
    if act in (None, "relu"):
        assert np.array_equal(got, want)
    else:   # approximated erf / f32 exp: at most one grid step, rarely
        step = np.abs(O.fp8_to_f32(got, fmt) - O.fp8_to_f32(want, fmt))
        assert (step > 0).mean() < 0.02


# ---- FP8 delayed-scaling quantizer -------------------------------------------
@pytest.mark.parametrize("fmt,tdt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_te_cast_matches_torch_in_range(fmt, tdt):
    g = rng(4)
    x = (g.standard_normal(5000) * 3).astype(np.float32)
    x[17] = np.nan
    s = 7.5
    bits, amax = O.te_cast_amax(x, s, fmt)
    xs = (x * np.float32(s)).astype(np.float32)
    ok = np.isfinite(xs) & (np.abs(xs) <= O.TE_MAX_REPR[fmt])
    want = torch.from_numpy(xs[ok]).to(tdt).view(torch.uint8).numpy()
    assert np.array_equal(bits[ok], want)
    assert bits[17] & 0x7F == 0x7F                      # NaN stays NaN
    assert amax == np.nanmax(np.abs(x))                 # NaN never wins the max
    big = O.te_cast_amax(np.array([1e6, -1e6], np.float32), 1.0, fmt)[0]
    assert big.tolist() == ([0x7E, 0xFE] if fmt == "e4m3" else [0x7B, 0xFB])   # satfinite


def test_te_recipe_scale_formula_reference_cases():
    # recipe_scale_compute_smoke.rs: amax 10 (e4m3) -> 44.8, amax 100 (e5m2)
    # -> 573.44, empty history -> amax floored at 1 -> scale = 448.
    s, si, h = O.te_recipe_update([0, 0, 10.0, 0], "e4m3", 2)
    assert abs(s - 44.8) / 44.8 < 1e-6 and abs(s * si - 1) < 1e-6 and h[2] == 0
    s, si, _ = O.te_recipe_update([100.0], "e5m2", 0)
    assert abs(s - 573.44) / 573.44 < 1e-6
    assert O.te_recipe_update([0.0] * 8, "e4m3", 0)[:2] == (448.0, float(np.float32(1.0) / np.float32(448.0)))
    assert O.te_recipe_update([np.inf], "e4m3", 0)[:2] == (1.0, 1.0)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_te_dequant_is_decode_times_scale_inv(fmt):
    b = np.arange(256, dtype=np.uint8)
    y = O.te_dequant_f32(b, 0.125, fmt)
    ref = O.fp8_to_f32(b, fmt) * np.float32(0.125)
    both_nan = np.isnan(y) & np.isnan(ref)
    assert np.array_equal(y[~both_nan], ref[~both_nan])


@pytest.mark.parametrize("act", [None, "relu", "gelu", "silu"])
def test_gemm_u8_epi_closed_forms(act):
    m, n, k = 37, 45, 70
    g = rng(12)
    a = g.integers(0, 256, (m, k), dtype=np.uint8)
    b = g.integers(0, 256, (k, n), dtype=np.uint8)
    c = g.integers(0, 256, (m, n), dtype=np.uint8)
    bias = (g.standard_normal(n) * 30).astype(np.float32)
    acc = a.astype(np.int64) @ b.astype(np.int64)
    alpha = 1.0 / 2048
    z = (np.float32(alpha) * acc.astype(np.float32) + np.float32(0.5) * c.astype(np.float32) + bias).astype(np.float32)
    if act == "relu":
        z = np.maximum(z, np.float32(0))
    elif act == "gelu":
        z = (np.float32(0.5) * z * (1 + np.vectorize(math.erf)(z / math.sqrt(2)))).astype(np.float32)
    elif act == "silu":
        z = (z / (1 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    want = np.clip(np.rint(z), 0, 255).astype(np.uint8)
    got = O.gemm_u8_epi(a, b, "rrr", alpha, 0.5, c, bias, act)
    assert np.array_equal(got, O.gemm_u8_epi(a, np.ascontiguousarray(b.T), "rcr", alpha, 0.5, c, bias, act))
    diff = np.abs(got.astype(int) - want.astype(int))
    if act in (None, "relu"):
        assert diff.max() == 0
    else:
        assert diff.max() <= 1 and (diff != 0).mean() < 0.01


def test_moe_grouped_f64_against_numpy():
    g = rng(21)
    E, topk, tokens, n, k = 4, 2, 24, 9, 13
    sid, eid = moe_routing(tokens, E, topk, seed=3)
    off = np.concatenate([[0], np.cumsum(np.bincount(eid, minlength=E))]).astype(np.int32)
    x = g.standard_normal((tokens, k)).astype(np.float32)
    w = g.standard_normal((E, n, k)).astype(np.float32)
    got = O.moe_grouped_f64(x, w, sid, off, topk, out_rows=tokens * topk)
    for p in range(len(sid)):
        tok, e = sid[p], eid[p]
        assert np.allclose(got[tok], w[e].astype(np.float64) @ x[tok // topk].astype(np.float64), rtol=1e-12)
    # with topk_weights the input row is the pair id and the result is scaled
    xp = g.standard_normal((tokens * topk, k)).astype(np.float32)
    tw = g.random(tokens * topk).astype(np.float32)
    got = O.moe_grouped_f64(xp, w, sid, off, topk, tw, out_rows=tokens * topk)
    for p in range(len(sid)):
        tok, e = sid[p], eid[p]
        assert np.allclose(got[tok], (w[e].astype(np.float64) @ xp[tok].astype(np.float64)) * tw[tok], rtol=1e-12)
