"""GPU parity of the grouped int8 MoE GEMM (routing contract of moe_wmma)."""
import numpy as np
import pytest
import torch

from baracuda_amd import plans as P
from oracle import oracle as O
from oracle.inputs import int8_uniform, moe_routing, rng
from tests.gpu_util import dev, host_bits16, sync

pytestmark = pytest.mark.gpu


def _run(tokens, E, topk, n, k, seed, topk_w=False, pairs_check=None, routing=None, ws_bytes=None,
         inputs=None):
    sorted_ids, expert_ids = routing if routing is not None else moe_routing(tokens, E, topk, seed=seed)
    size_m = tokens * topk
    g = rng(seed + 100)
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    sa = g.uniform(0.005, 0.02, tokens).astype(np.float32)
    sw = g.uniform(0.001, 0.01, E * n).astype(np.float32)
    tw = g.uniform(0.1, 1.0, size_m).astype(np.float32) if topk_w else None
    # topk_weights form reads input row = pair id: expand x and its per-row scales
    xin = x if not topk_w else np.repeat(x, topk, axis=0)
    sa_in = sa if not topk_w else np.repeat(sa, topk)
    out = torch.zeros((size_m, n), dtype=torch.bfloat16, device="cuda:0")
    counts = torch.zeros(E, dtype=torch.int32, device="cuda:0")
    offs = torch.zeros(E + 1, dtype=torch.int32, device="cuda:0")
    plan = P.MoeS8GroupedPlan.select(E, topk, size_m, n, k)
    ws = None
    if ws_bytes is not None:
        # contents on entry must not matter
        ws = torch.full(((ws_bytes or plan.workspace_size()) // 4,), -123456, dtype=torch.int32, device="cuda:0")
    plan.run(dev(xin), dev(w), dev(sorted_ids), dev(expert_ids), out, counts, offs, dev(sa_in), dev(sw),
             topk_weights=dev(tw) if tw is not None else None, workspace=ws)
    sync()
    c_ref, o_ref = O.moe_expert_offsets(expert_ids, E)
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(offs.cpu().numpy(), o_ref)
    got = host_bits16(out)
    pairs = range(size_m) if pairs_check is None else pairs_check
    pair_e = np.empty(size_m, np.int32)
    pair_e[sorted_ids] = expert_ids
    for p in pairs:
        e, t = pair_e[p], p // topk
        acc = (w[e].astype(np.int64) @ x[t].astype(np.int64)).astype(np.float32)
        y = (sa[t] * sw[e * n:(e + 1) * n]).astype(np.float32) * acc
        if tw is not None:
            y = (y * tw[p]).astype(np.float32)
        assert np.array_equal(got[p], O.f32_to_bf16_bits_fast(y)), p
    if inputs is not None:
        inputs.update(x=x, w=w, sa=sa, sw=sw, pair_e=pair_e)
    return got


def test_moe_small_all_pairs(gpu):
    print("case: moe small", flush=True)
    _run(tokens=300, E=8, topk=2, n=272, k=384, seed=5)


def test_moe_dma_path_all_pairs(gpu):
    # N % 256 == 0 and K % 128 == 0: the LDS-DMA grouped kernel.
    print("case: moe dma path", flush=True)
    _run(tokens=700, E=8, topk=2, n=512, k=384, seed=9)


def test_moe_dma_path_topk_weights(gpu):
    _run(tokens=200, E=4, topk=2, n=256, k=256, seed=10, topk_w=True)


def test_moe_ragged_k_and_topk_weights(gpu):
    print("case: moe ragged k, topk weights", flush=True)
    _run(tokens=100, E=5, topk=3, n=100, k=200, seed=6, topk_w=True)


def test_moe_oracle_grouped_agrees(gpu):
    # the oracle's grouped restatement and the bf16 check above agree on i32 accumulators
    sorted_ids, expert_ids = moe_routing(64, 4, 2, seed=7)
    _, offs = O.moe_expert_offsets(expert_ids, 4)
    g = rng(8)
    x, w = int8_uniform(g, (64, 128)), int8_uniform(g, (4, 64, 128))
    acc = O.moe_s8_grouped_i32(x, w, sorted_ids, offs, 2, 128)
    pair_e = np.empty(128, np.int32)
    pair_e[sorted_ids] = expert_ids
    assert np.array_equal(acc[5], w[pair_e[5]].astype(np.int64) @ x[2].astype(np.int64))


def test_moe_config5_full_size_sampled(gpu):
    # 8 experts, hidden 4096, ffn 14336, 4096 tokens top-2 Zipf(1.1).
    print("case: moe config5", flush=True)
    pairs = [0, 1, 2, 8191, 4095] + list(rng(51).integers(0, 8192, 27))
    _run(tokens=4096, E=8, topk=2, n=14336, k=4096, seed=5, pairs_check=pairs)


def test_moe_config5_whole_output_sums(gpu):
    # Config 5 over all 8192 x 14336 outputs, size-independent: each output is
    # bf16((sa[t] * sw[e, n]) * acc), so v = out / (sa[t] * sw[e, n]) (f64)
    # is acc within a relative 2^-8 (bf16 rounding) plus f32 slack.  Row sums
    # of v against x[t] . sum_n W[e][n, :] and, per expert, column sums of v
    # over its pairs against W[e] . sum_t x[t] (exact integers), each within
    # 1.01 * 2^-8 * the sum of |v|.  Every pair and every column is checked;
    # a missing, misplaced or mis-scaled row or tile moves a sum far beyond
    # that bound.
    print("case: moe config5 whole-output sums", flush=True)
    tokens, E, topk, n, k = 4096, 8, 2, 14336, 4096
    inp = {}
    got = _run(tokens=tokens, E=E, topk=topk, n=n, k=k, seed=5, pairs_check=[0, 8191], inputs=inp)
    x, w, sa, sw, pair_e = inp["x"], inp["w"], inp["sa"], inp["sw"], inp["pair_e"]
    out = (got.astype(np.uint32) << 16).view(np.float32)
    tok = np.arange(tokens * topk) // topk
    sw2 = sw.reshape(E, n)
    tol = 1.01 * 2.0 ** -8
    x64 = x.astype(np.int64)
    for e in range(E):
        pe = np.nonzero(pair_e == e)[0]
        if pe.size == 0:
            continue
        scale = (sa[tok[pe]].astype(np.float32)[:, None] * sw2[e][None, :]).astype(np.float64)
        v = out[pe].astype(np.float64) / scale
        we = w[e].astype(np.int64)
        row_exact = x64[tok[pe]] @ we.sum(0)
        assert np.all(np.abs(v.sum(1) - row_exact) <= tol * np.abs(v).sum(1)), e
        col_exact = we @ x64[tok[pe]].sum(0)
        assert np.all(np.abs(v.sum(0) - col_exact) <= tol * np.abs(v).sum(0)), e


@pytest.mark.parametrize("E", [1, 8, 63, 64, 65, 300])
def test_expert_counting_any_order(gpu, E):
    # Counts / offsets from unsorted expert ids: the ballot path (E <= 64) and
    # the atomic path (E > 64) against the oracle's count + scan.  Ids outside
    # [0, E) (undefined in the reference, which indexes counts with them) are
    # skipped here; the oracle is fed the in-range ids.
    size_m, n, k = 2000, 16, 32
    g = rng(E)
    expert_ids = g.integers(-2, E + 2, size_m).astype(np.int32)
    sorted_ids = np.arange(size_m, dtype=np.int32)
    x, w = int8_uniform(g, (size_m, k)), int8_uniform(g, (E, n, k))
    sa = np.ones(size_m, dtype=np.float32)
    sw = np.ones(E * n, dtype=np.float32)
    out = torch.zeros((size_m, n), dtype=torch.bfloat16, device="cuda:0")
    counts = torch.full((E,), -7, dtype=torch.int32, device="cuda:0")
    offs = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda:0")
    P.MoeS8GroupedPlan.select(E, 1, size_m, n, k).run(dev(x), dev(w), dev(sorted_ids), dev(expert_ids), out,
                                                      counts, offs, dev(sa), dev(sw))
    sync()
    valid = expert_ids[(expert_ids >= 0) & (expert_ids < E)]
    c_ref, o_ref = O.moe_expert_offsets(valid, E)
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(offs.cpu().numpy(), o_ref)
    assert np.array_equal(c_ref, np.bincount(valid, minlength=E))


def _block_routing(counts, seed):
    # top-1 routing with exact per-expert row counts, tokens shuffled
    tokens = sum(counts)
    pair_expert = np.repeat(np.arange(len(counts), dtype=np.int32), counts)
    rng(seed).shuffle(pair_expert)
    order = np.argsort(pair_expert, kind="stable").astype(np.int32)
    return tokens, (order, pair_expert[order].astype(np.int32))


def test_moe_dma_partial_tile_boundaries(gpu):
    # Last tiles of 1, 128 and 129 rows (the first two leave the second half
    # of the wave grid with padding rows only), a full tile, an empty expert.
    print("case: moe partial tile boundaries", flush=True)
    tokens, routing = _block_routing([257, 128, 0, 129, 256], seed=12)
    _run(tokens=tokens, E=5, topk=1, n=512, k=256, seed=12, routing=routing)


def test_moe_dma_path_many_experts(gpu):
    # 80 experts (the LDS-counter path of the offsets kernel) on the LDS-DMA
    # GEMM: mostly single partial tiles, some experts empty.
    print("case: moe 80 experts", flush=True)
    _run(tokens=600, E=80, topk=2, n=256, k=256, seed=21)


def test_moe_dma_tile_list_not_multiple_of_8(gpu):
    # 43 m-tiles x 3 n-tiles = 129 tiles: the XCD regroup pads the list to
    # 136 and the surplus ids exit; sampled pairs over every expert.
    print("case: moe tile list 129", flush=True)
    counts = [256] * 40 + [200, 3, 129]
    tokens, routing = _block_routing(counts, seed=16)
    _run(tokens=tokens, E=len(counts), topk=1, n=768, k=256, seed=16, routing=routing,
         pairs_check=list(range(0, tokens, 37)) + [tokens - 1])


def test_moe_workspace_is_ignored(gpu):
    # workspace_size() is 0; a workspace passed anyway changes nothing
    print("case: moe workspace ignored", flush=True)
    assert P.MoeS8GroupedPlan.select(8, 2, 1400, 512, 384).workspace_size() == 0
    _run(tokens=700, E=8, topk=2, n=512, k=384, seed=9, ws_bytes=1 << 20)


@pytest.mark.parametrize("n", [1280, 2304])
def test_moe_dma_ragged_n_blocks(gpu, n):
    # n-tiles in blocks of 4 with a narrower last block (5 = 4 + 1, 9 = 4 + 4 + 1)
    print(f"case: moe n blocks n={n}", flush=True)
    tokens, routing = _block_routing([300, 0, 41, 513, 256], seed=n)
    _run(tokens=tokens, E=5, topk=1, n=n, k=384, seed=n, routing=routing)


def test_moe_dma_no_valid_rows(gpu):
    # every expert id out of range: no tiles (S = 0) on the LDS-DMA path;
    # counts / offsets zero and the output untouched
    print("case: moe dma no valid rows", flush=True)
    E, size_m, n, k = 4, 300, 256, 128
    g = rng(99)
    x, w = int8_uniform(g, (size_m, k)), int8_uniform(g, (E, n, k))
    out = torch.full((size_m, n), 3.0, dtype=torch.bfloat16, device="cuda:0")
    counts = torch.full((E,), -1, dtype=torch.int32, device="cuda:0")
    offs = torch.full((E + 1,), -1, dtype=torch.int32, device="cuda:0")
    ids = np.full(size_m, E + 3, dtype=np.int32)
    P.MoeS8GroupedPlan.select(E, 1, size_m, n, k).run(
        dev(x), dev(w), dev(np.arange(size_m, dtype=np.int32)), dev(ids), out, counts, offs,
        dev(np.ones(size_m, np.float32)), dev(np.ones(E * n, np.float32)))
    sync()
    assert torch.all(counts == 0) and torch.all(offs == 0)
    assert torch.all(out == 3.0)


def _moe_i32(x, w, sorted_ids, expert_ids, E, topk, size_m, n, k):
    out = torch.full((size_m, n), -7, dtype=torch.int32, device="cuda:0")
    counts = torch.zeros(E, dtype=torch.int32, device="cuda:0")
    offs = torch.zeros(E + 1, dtype=torch.int32, device="cuda:0")
    P.MoeS8GroupedPlan.select(E, topk, size_m, n, k).run_i32(
        x, w, dev(sorted_ids), dev(expert_ids), out, counts, offs)
    sync()
    return out


@pytest.mark.parametrize("case", ["dma", "general", "boundaries"])
def test_moe_i32_all_pairs_vs_oracle(gpu, case):
    # The int32-accumulator SKU against the oracle's grouped restatement
    # (bo_moe_s8_grouped_i32, baracuda_moe.cuh:1121-1162) on every pair: the
    # LDS-DMA kernel, the general kernel (N off the 256 grid, K tail) and
    # last tiles of 1 / 128 / 129 rows with an empty expert.
    print(f"case: moe i32 {case}", flush=True)
    if case == "dma":
        tokens, E, topk, n, k = 700, 8, 2, 512, 384
        sorted_ids, expert_ids = moe_routing(tokens, E, topk, seed=9)
    elif case == "general":
        tokens, E, topk, n, k = 300, 8, 3, 272, 200
        sorted_ids, expert_ids = moe_routing(tokens, E, topk, seed=6)
    else:
        tokens, (sorted_ids, expert_ids) = _block_routing([257, 128, 0, 129, 256], seed=12)
        E, topk, n, k = 5, 1, 512, 256
    size_m = tokens * topk
    g = rng(size_m + n)
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    got = _moe_i32(dev(x), dev(w), sorted_ids, expert_ids, E, topk, size_m, n, k).cpu().numpy()
    _, offs = O.moe_expert_offsets(expert_ids, E)
    want = O.moe_s8_grouped_i32(x, w, sorted_ids, offs, topk, size_m)
    assert np.array_equal(got, want)


def test_moe_config5_i32_whole_output_exact_and_bf16_epilogue(gpu):
    # BASELINE.json config 5 (8 experts, 4096 tokens top-2 Zipf(1.1), N 14336,
    # K 4096) through the int32 SKU, over all 8192 x 14336 accumulators:
    #  - every pair's row sum equals x[t] . sum_n W[e][n, :] exactly and, per
    #    expert, every column sum over its pairs equals W[e] . sum_t x[t]
    #    exactly (int64 on the left; f64 on the right, exact since every
    #    partial sum is an integer below 2^53);
    #  - one pair in every (expert, 256-row tile), and the last pair of every
    #    expert's last (partial) tile, equal int64 dot products in full;
    #  - the bf16 SKU's whole output equals bf16_rne((sa[t] * sw[e, n]) *
    #    f32(acc)) bit for bit (its epilogue over the same accumulators).
    print("case: moe config5 i32 whole output", flush=True)
    tokens, E, topk, n, k = 4096, 8, 2, 14336, 4096
    size_m = tokens * topk
    sorted_ids, expert_ids = moe_routing(tokens, E, topk, seed=5)
    g = rng(105)
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    sa = g.uniform(0.005, 0.02, tokens).astype(np.float32)
    sw = g.uniform(0.001, 0.01, E * n).astype(np.float32)
    xd, wd = dev(x), dev(w)
    acc = _moe_i32(xd, wd, sorted_ids, expert_ids, E, topk, size_m, n, k)
    pair_e = np.empty(size_m, np.int32)
    pair_e[sorted_ids] = expert_ids
    pe_d = torch.from_numpy(pair_e.astype(np.int64)).cuda()
    tok_d = torch.arange(size_m, device="cuda:0") // topk
    x64 = xd.to(torch.float64)
    # rows: acc[p, :].sum() == x[t] . wsum[e]
    row_got = acc.to(torch.int64).sum(1)
    wsum = torch.stack([wd[e].to(torch.float64).sum(0) for e in range(E)])     # [E, K]
    row_exact = (x64[tok_d] * wsum[pe_d]).sum(1)
    assert torch.equal(row_got, row_exact.to(torch.int64))
    # columns, per expert: sum over its pairs of acc[p, n] == W[e][n] . sum x[t_p]
    for e in range(E):
        sel = torch.nonzero(pe_d == e).flatten()
        if sel.numel() == 0:
            continue
        col_got = acc[sel].to(torch.int64).sum(0)
        xs = x64[tok_d[sel]].sum(0)
        col_exact = wd[e].to(torch.float64) @ xs
        assert torch.equal(col_got, col_exact.to(torch.int64)), e
    # sampled pairs in full: one per (expert, tile) + each expert's last pair
    _, offs = O.moe_expert_offsets(expert_ids, E)
    acc_h = acc.cpu().numpy()
    pick = []
    gp = rng(55)
    for e in range(E):
        o0, o1 = int(offs[e]), int(offs[e + 1])
        for t0 in range(o0, o1, 256):
            pick.append(int(gp.integers(t0, min(t0 + 256, o1))))
        if o1 > o0:
            pick.append(o1 - 1)
    assert len(pick) >= 37 + E
    for s in pick:
        p = int(sorted_ids[s])
        e, t = pair_e[p], p // topk
        want = w[e].astype(np.int64) @ x[t].astype(np.int64)
        assert np.array_equal(acc_h[p].astype(np.int64), want), (s, p, e)
    # the bf16 SKU over the same inputs: its epilogue applied to these accumulators
    out = torch.zeros((size_m, n), dtype=torch.bfloat16, device="cuda:0")
    counts = torch.zeros(E, dtype=torch.int32, device="cuda:0")
    offs_d = torch.zeros(E + 1, dtype=torch.int32, device="cuda:0")
    sa_d, sw_d = dev(sa), dev(sw).view(E, n)
    P.MoeS8GroupedPlan.select(E, topk, size_m, n, k).run(xd, wd, dev(sorted_ids), dev(expert_ids), out,
                                                         counts, offs_d, sa_d, dev(sw))
    sync()
    scale = sa_d[tok_d][:, None] * sw_d[pe_d]                 # f32, rounded once
    want_bf16 = (scale * acc.to(torch.float32)).to(torch.bfloat16)
    assert torch.equal(out.view(torch.int16), want_bf16.view(torch.int16))


# ---- decode-sized MoE (size_m <= 64, K % 512 == 0: moe_rows_staged_kernel;
# 3-6 pairs with K % 1024 == 0: moe_row_kernel); no offsets kernel, the
# counts and offsets written by the decode kernels (checked in _run) --
@pytest.mark.parametrize("case", [(1, 8, 2, 512, 1024, False), (3, 8, 2, 256, 512, True), (16, 8, 2, 512, 2048, False),
                                  (32, 8, 2, 256, 512, True), (4, 8, 2, 6144, 512, False),
                                  (2, 8, 2, 12288, 512, True), (21, 4, 3, 256, 1536, False),
                                  (2, 8, 2, 512, 1024, False), (4, 8, 2, 1024, 4096, True), (3, 4, 2, 256, 3072, False),
                                  (6, 1, 1, 256, 2048, False), (3, 8, 2, 512, 1024, True)])
def test_moe_decode_all_pairs(gpu, case):
    # every pair bit-exact against the per-pair W8A8 formula; size_m 2 to 64
    # (16- or 32-row blocks), 16 / 32 / 64 columns per workgroup; the row
    # kernel at 4 / 6 pairs (1 or 2 KiB per batch, with and without
    # topk_weights) and with 6 rows on one expert (3 passes of 2 rows); 8
    # pairs on the staged kernel
    tokens, E, topk, n, k, tw = case
    print(f"case: moe decode {case}", flush=True)
    _run(tokens=tokens, E=E, topk=topk, n=n, k=k, seed=tokens * 7 + n, topk_w=tw)


def test_moe_decode_i32_vs_oracle_empty_and_invalid_experts(gpu):
    # int32 SKU on the decode pass against the oracle's grouped restatement:
    # 16 experts, most empty, some pairs routed to out-of-range ids (not
    # counted, their output rows untouched)
    tokens, E, topk, n, k = 20, 16, 3, 512, 1024
    size_m = tokens * topk
    g = rng(41)
    pair_e = g.integers(0, 4, size_m).astype(np.int32) * 5     # experts 0, 5, 10, 15
    pair_e[[3, 17, 40]] = E + 2                                   # out of range
    order = np.argsort(pair_e, kind="stable").astype(np.int32)
    sorted_ids, expert_ids = order, pair_e[order]
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    got = _moe_i32(dev(x), dev(w), sorted_ids, expert_ids, E, topk, size_m, n, k).cpu().numpy()
    _, offs = O.moe_expert_offsets(expert_ids, E)
    want = O.moe_s8_grouped_i32(x, w, sorted_ids, offs, topk, size_m)
    valid = pair_e < E
    assert np.array_equal(got[valid], want[valid])
    assert np.all(got[~valid] == -7)


def test_moe_decode_one_expert_takes_all_rows(gpu):
    # all 64 pairs on one expert: the largest segment the decode pass takes
    tokens, routing = _block_routing([0, 64, 0], seed=3)
    print("case: moe decode one expert", flush=True)
    _run(tokens=tokens, E=3, topk=1, n=512, k=512, seed=4, routing=routing)


@pytest.mark.parametrize("size_m", [6, 60])
@pytest.mark.parametrize("E", [1, 8, 65])
def test_expert_counting_decode(gpu, E, size_m):
    # Decode launches count in-kernel (one ballot per expert): unsorted ids
    # with some outside [0, E), counts and offsets against the oracle's count
    # and scan of the in-range ids (row kernel at 6 pairs, staged at 60).
    n, k = 256, 1024
    g = rng(E * 100 + size_m)
    expert_ids = g.integers(-2, E + 2, size_m).astype(np.int32)
    sorted_ids = np.arange(size_m, dtype=np.int32)
    x, w = int8_uniform(g, (size_m, k)), int8_uniform(g, (E, n, k))
    out = torch.zeros((size_m, n), dtype=torch.bfloat16, device="cuda:0")
    counts = torch.full((E,), -7, dtype=torch.int32, device="cuda:0")
    offs = torch.full((E + 1,), -7, dtype=torch.int32, device="cuda:0")
    P.MoeS8GroupedPlan.select(E, 1, size_m, n, k).run(dev(x), dev(w), dev(sorted_ids), dev(expert_ids), out,
                                                      counts, offs, dev(np.ones(size_m, np.float32)),
                                                      dev(np.ones(E * n, np.float32)))
    sync()
    valid = expert_ids[(expert_ids >= 0) & (expert_ids < E)]
    c_ref, o_ref = O.moe_expert_offsets(valid, E)
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(offs.cpu().numpy(), o_ref)


def test_moe_decode_row_kernel_i32_vs_oracle(gpu):
    # int32 SKU on the row kernel (6 pairs, one out of range: not counted,
    # its output row untouched) against the oracle's grouped restatement
    tokens, E, topk, n, k = 6, 8, 1, 512, 2048
    g = rng(77)
    pair_e = np.array([3, 3, 0, 7, E + 1, 3], np.int32)
    order = np.argsort(pair_e, kind="stable").astype(np.int32)
    sorted_ids, expert_ids = order, pair_e[order]
    x, w = int8_uniform(g, (tokens, k)), int8_uniform(g, (E, n, k))
    got = _moe_i32(dev(x), dev(w), sorted_ids, expert_ids, E, topk, tokens, n, k).cpu().numpy()
    _, offs = O.moe_expert_offsets(expert_ids, E)
    want = O.moe_s8_grouped_i32(x, w, sorted_ids, offs, topk, tokens)
    valid = pair_e < E
    assert np.array_equal(got[valid], want[valid])
    assert np.all(got[~valid] == -7)


def test_moe_decode_row_blocks_of_one_expert(gpu):
    # 30 of 32 pairs on one expert: 16-row blocks (blockIdx.z), the second
    # holding 14 rows, the other experts' second blocks empty
    tokens, routing = _block_routing([0, 30, 2], seed=8)
    print("case: moe decode two row blocks", flush=True)
    _run(tokens=tokens, E=3, topk=1, n=512, k=1024, seed=9, routing=routing)
