"""GPU parity of the bandwidth kernels against the CPU oracle: alignment
(bit-exact), silu_and_mul, moe_sum, and the activation quantisers
(bit-exact). Each call goes through the C ABI via the package's ops."""

import numpy as np
import pytest
import torch

from flaggems_sglang import _capi, ops  # noqa: F401
from flaggems_sglang.ops import fused_moe as fm
from oracle import moe_ref

pytestmark = pytest.mark.gpu


def _routing(M, E, k, seed, device, hot=(), bias=0.0, scoring="softmax"):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(M, E, generator=g)
    if hot:
        logits[:, list(hot)] += bias
    w, ids = moe_ref.route(logits, k, scoring)
    return w, ids


ALIGN_CASES = [
    # (M, k, E, block)
    (1, 2, 8, 16), (7, 2, 8, 16), (33, 4, 16, 32), (64, 2, 8, 16),
    (1, 8, 128, 64), (16, 8, 128, 64), (256, 8, 128, 64), (2048, 8, 128, 64),
    (8192, 8, 128, 64), (4096, 8, 256, 16), (1024, 8, 64, 32),
    (300, 3, 1024, 16), (5, 1, 1, 7), (8192, 2, 8, 128),
    # decode sizes around the one-wave kernel's limit of 64 slots
    (8, 8, 256, 16), (3, 8, 256, 64), (4, 8, 64, 32), (32, 2, 8, 256),
    (13, 5, 64, 8),
]


@pytest.mark.parametrize("single_wg", [False, True], ids=["default", "one_wg"])
@pytest.mark.parametrize("M,k,E,B", ALIGN_CASES + [(5000, 3, 1024, 16), (4097, 1, 64, 64)])
def test_align_bit_exact(gpu, M, k, E, B, single_wg):
    """Both the multi-workgroup path (>= 4096 slots, with scratch) and the
    one-workgroup path, bit for bit against the oracle."""
    w, ids = _routing(M, E, k, seed=M + k + E + B, device=gpu)
    if M > 100:
        ids[::97, 0] = -1          # dropped slots inside the chunks
        ids[5::101, -1] = E + 3
    s, eids, npp = fm.moe_align_block_size(ids.to(gpu), E, B,
                                           _single_workgroup=single_wg)
    rs, reids, rnpp = moe_ref.align(ids.numpy(), E, B)
    torch.cuda.synchronize()
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(eids.cpu().numpy(), reids)


@pytest.mark.parametrize("skew", [False, True])
def test_align_qwen3_skewed_block64(gpu, skew):
    hot = (3, 17, 31, 45, 59, 73, 87, 101)
    for M in (1, 16, 256, 2048, 8192):
        _, ids = _routing(M, 128, 8, seed=M + 2048 + 768 + 128 + 8, device=gpu,
                          hot=hot if skew else (), bias=2.0)
        s, eids, npp = fm.moe_align_block_size(ids.to(gpu), 128, 64)
        rs, reids, rnpp = moe_ref.align(ids.numpy(), 128, 64)
        assert int(npp.item()) == rnpp, M
        assert np.array_equal(s.cpu().numpy(), rs), M
        assert np.array_equal(eids.cpu().numpy(), reids), M


@pytest.mark.parametrize("numel", [64, 63, 65])
def test_align_small_dropped_ids(gpu, numel):
    """Decode-sized inputs with dropped (-1) and out-of-range ids, one expert
    holding most slots, against the oracle."""
    g = np.random.default_rng(numel)
    raw = g.integers(-1, 20, size=(numel,), dtype=np.int32)  # E = 16: 16..19 out of range
    raw[::3] = 5
    ids = torch.from_numpy(raw.reshape(numel, 1))
    s, eids, npp = fm.moe_align_block_size(ids.to(gpu), 16, 8)
    rs, reids, rnpp = moe_ref.align(raw.reshape(numel, 1), 16, 8)
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(eids.cpu().numpy(), reids)


def test_align_edge_cases(gpu):
    # empty input
    ids = torch.zeros((0, 2), dtype=torch.int32, device=gpu)
    s, eids, npp = fm.moe_align_block_size(ids, 4, 8)
    rs, reids, rnpp = moe_ref.align(np.zeros((0, 2), np.int32), 4, 8)
    assert int(npp.item()) == rnpp == 0
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(eids.cpu().numpy(), reids)
    # out-of-range ids are dropped, all slots on one expert, repeated ids
    raw = np.array([[-1, 3], [7, 3], [3, 3], [0, 100]], dtype=np.int32)
    s, eids, npp = fm.moe_align_block_size(torch.from_numpy(raw).to(gpu), 4, 4)
    rs, reids, rnpp = moe_ref.align(raw, 4, 4)
    assert int(npp.item()) == rnpp
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(eids.cpu().numpy(), reids)


def test_align_deterministic(gpu):
    _, ids = _routing(8192, 128, 8, seed=11, device=gpu)
    ids = ids.to(gpu)
    first = fm.moe_align_block_size(ids, 128, 64)[0].cpu()
    for _ in range(3):
        assert torch.equal(fm.moe_align_block_size(ids, 128, 64)[0].cpu(), first)


def _ulp_diff_bf16(a, b):
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    # map sign-magnitude to a monotone integer line
    ai = torch.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = torch.where(bi < 0, -(bi & 0x7FFF), bi)
    return (ai - bi).abs()


@pytest.mark.parametrize("rows,n", [(1, 256), (7, 3072), (513, 768), (64, 14336)])
def test_silu_and_mul(gpu, rows, n):
    g = torch.Generator().manual_seed(rows + n)
    x = (torch.randn(rows, 2 * n, generator=g) * 3).to(torch.bfloat16)
    out = fm.silu_and_mul(x.to(gpu)).cpu()
    ref = moe_ref.silu_and_mul(x)
    assert _ulp_diff_bf16(out, ref).max() <= 1


@pytest.mark.parametrize("m,k,K", [(1, 2, 4096), (33, 8, 2048), (4096, 2, 1024),
                                   (5, 1, 128)])
def test_moe_sum(gpu, m, k, K):
    g = torch.Generator().manual_seed(m + k + K)
    y = torch.randn(m, k, K, generator=g).to(torch.bfloat16)
    out = fm.moe_sum(y.to(gpu)).cpu()
    ref = moe_ref.moe_sum(y)
    assert _ulp_diff_bf16(out, ref).max() <= 1


@pytest.mark.parametrize("rows,cols,group", [(1, 128, 128), (37, 7168, 128), (512, 2048, 128),
                                            (5, 1024, 512), (9, 256, 32), (3, 64, 8)])
def test_quant_fp8_group_bit_exact(gpu, rows, cols, group):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(torch.bfloat16)
    x[0, :5] = 0.0
    if rows > 1:
        x[1, :group] = 0.0  # all-zero group: scale = 1e-10/448
    q, s = fm.per_token_group_quant_fp8(x.to(gpu), group)
    rq, rsc = moe_ref.quant_fp8_group(x, group)
    assert torch.equal(s.cpu(), rsc)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))


@pytest.mark.parametrize("rows,cols", [(1, 128), (37, 3584), (300, 2560), (5, 520),
                                       (9, 8192), (1030, 520), (2048, 8192)])
def test_quant_int8_token_bit_exact(gpu, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(torch.bfloat16)
    if rows > 1:
        x[1] = 0.0
    q, s = fm.per_token_quant_int8(x.to(gpu))
    rq, rsc = moe_ref.quant_int8_token(x)
    assert torch.equal(s.cpu(), rsc)
    assert torch.equal(q.cpu(), rq)


# ----------------------------------------------------------------- gating ---
@pytest.mark.parametrize("M,E,k,scoring,dtype,renorm", [
    (1, 8, 2, "softmax", torch.float32, True),
    (333, 8, 2, "softmax", torch.float32, True),
    (257, 128, 8, "softmax", torch.bfloat16, True),
    (100, 256, 8, "sigmoid", torch.float32, True),
    (64, 1024, 16, "softmax", torch.float32, False),
    (17, 60, 64 - 4, "sigmoid", torch.bfloat16, False),
    (0, 16, 4, "softmax", torch.float32, True),
])
def test_topk_gating(gpu, M, E, k, scoring, dtype, renorm):
    """ids bit-exact against the oracle's ranking (logit descending, ties to
    the lower id); weights to fp32 rounding."""
    g = torch.Generator().manual_seed(M + E + k)
    logits = torch.randn(M, E, generator=g).to(dtype)
    if M > 3:
        logits[3, :] = logits[3, 0]          # every logit tied
        logits[2, 5 % E] = logits[2, 1 % E]  # one tie
    x = torch.empty(M, 8, device=gpu)
    w, ids = fm.fused_topk(x, logits.to(gpu), k, renormalize=renorm,
                           scoring_func=scoring)
    rw, rids = moe_ref.topk_gating(logits, k, scoring=scoring, renormalize=renorm)
    assert torch.equal(ids.cpu(), rids)
    assert torch.allclose(w.cpu(), rw, rtol=2e-6, atol=1e-7)


def test_topk_gating_feeds_fused_moe(gpu):
    """Gating kernel -> fused MoE equals the torch-routed path."""
    M, K, N, E, k = 96, 256, 128, 8, 2
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * N, K, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    w2 = (torch.randn(E, K, N, generator=g, device=gpu) * 0.1).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g, device=gpu)
    tw, ti = fm.fused_topk(x, logits, k)
    rw, ri = moe_ref.route(logits.cpu(), k)
    assert torch.equal(ti.cpu(), ri)
    a = fm.fused_moe(x, w1, w2, tw, ti)
    b = fm.fused_moe(x, w1, w2, rw.to(gpu), ri.to(gpu))
    assert (a.float() - b.float()).abs().max() <= 2e-2 * b.float().abs().max()


# ------------------------------------------------------- routing format ---
@pytest.mark.parametrize("M,k,E,drop", [
    (1, 2, 8, False), (7, 2, 8, False), (33, 4, 16, True), (64, 8, 256, False),
    (700, 8, 128, True), (1024, 8, 64, False),
    # >= 4096 slots: the multi-workgroup alignment path
    (600, 8, 128, False), (4096, 2, 8, True), (2048, 8, 256, False),
    (0, 2, 8, False), (5, 3, 1022, False),
])
def test_standard_topk_to_routing_bit_exact(gpu, M, k, E, drop):
    """The GPU routing conversion equals the oracle's loop restatement of
    ops/fused_moe.py:126-139 (gate_scal, topk_indx, gate_indx, hist) and of
    compute_expt_data_torch (tile tables) bit for bit, and the compat path's
    inverse rebuilds the per-token routing."""
    w, ids = _routing(M, E, k, M * 7 + k + E, "cpu")
    ids = ids.clone()
    if drop and M:
        ids[::3, -1] = -1
    rd, gi, si = fm.standard_topk_to_routing(w.to(gpu), ids.to(gpu), E)
    gate_scal, topk_indx, gate_indx, hist = moe_ref.topk_to_routing(w, ids, E)
    assert np.array_equal(rd.gate_scal.cpu().numpy(), gate_scal)
    assert np.array_equal(gi.src_indx.cpu().numpy(), topk_indx)
    assert np.array_equal(gi.dst_indx.cpu().numpy(), gate_indx)
    assert np.array_equal(si.src_indx.cpu().numpy(), gate_indx)
    assert np.array_equal(rd.expt_hist.cpu().numpy(), hist)
    assert rd.n_expts_tot == E and rd.n_expts_act == k
    raw, pad, pid = moe_ref.expt_data(hist, E, M * k)
    ed = rd.expt_data
    assert np.array_equal(ed.hist.cpu().numpy(), hist)
    assert np.array_equal(ed.token_offs_raw.cpu().numpy(), raw)
    for bm in moe_ref.ROUTING_BLOCK_MS:
        assert np.array_equal(ed.token_offs_pad[bm].cpu().numpy(), pad[bm])
        assert np.array_equal(ed.block_pid_map[bm].cpu().numpy(), pid[bm])
    if M:
        # the inverse (fgs_moe_routing_to_topk) rebuilds the row-sorted
        # routing, unrouted slots as -1 (they sit past the histogram's total)
        tw, ti = fm._routing_to_topk(rd, gi, M)
        _, _, _, rid, rwt = moe_ref.routing_order(gate_scal, topk_indx, hist, M * k, 1)
        assert np.array_equal(ti.cpu().numpy().reshape(-1), rid)
        assert np.array_equal(tw.cpu().numpy().reshape(-1), rwt)
        key = torch.where((ids >= 0) & (ids < E), ids.long(), torch.full_like(ids.long(), -1))
        sid, order = torch.sort(key, dim=1)
        assert torch.equal(ti.cpu().long(), sid)
        assert torch.equal(tw.cpu(), torch.gather(w, 1, order))


@pytest.mark.parametrize("M,k,E,bad", [(9, 4, 16, None), (300, 8, 128, None),
                                       (64, 2, 8, "over"), (64, 2, 8, "neg"),
                                       (64, 2, 8, "src")])
def test_routing_to_topk_bit_exact_with_bad_tuples(gpu, M, k, E, bad):
    """fgs_moe_routing_to_topk against the oracle's routing_order on tuples a
    caller may get wrong: a histogram summing past the gate count, negative
    counts, gather entries out of range (clamped / skipped, never read or
    written out of bounds)."""
    w, ids = _routing(M, E, k, M + k + E, "cpu")
    gate_scal, topk_indx, _, hist = moe_ref.topk_to_routing(w, ids, E)
    hist, topk_indx = hist.copy(), topk_indx.copy()
    if bad == "over":
        hist[0] += 40
    elif bad == "neg":
        hist[1] = -5
    elif bad == "src":
        topk_indx[3] = M * k + 7
        topk_indx[5] = -2
    _, _, _, rid, rwt = moe_ref.routing_order(gate_scal, topk_indx, hist, M * k, 1)
    written = rid != -7
    lib = _capi.load()
    dev = lambda a: torch.from_numpy(a).to(gpu)
    gs, src, hs = dev(gate_scal), dev(topk_indx), dev(hist)
    tw = torch.full((M * k,), 9.0, device=gpu)
    ti = torch.full((M * k,), -7, dtype=torch.int32, device=gpu)
    _capi.check(lib.fgs_moe_routing_to_topk(gs.data_ptr(), src.data_ptr(), hs.data_ptr(), M,
                                            k, E, tw.data_ptr(), ti.data_ptr(), None),
                "routing_to_topk")
    torch.cuda.synchronize()
    assert np.array_equal(ti.cpu().numpy(), rid)
    assert np.array_equal(tw.cpu().numpy()[written], rwt[written])
