"""Pins the CPU oracle (oracle/) before any GPU result is compared with it.

Each oracle function is checked against something that does not restate its
own formula: hand-worked known answers, the reference's own routing steps
re-run with torch library ops, float64 brute force, the OCP e4m3 code table
decoded from the bit layout, and exact invariants (permutations, scaling,
expert relabelling, token subsets). CPU only.
"""

import math

import numpy as np
import pytest
import torch

from flaggems_sglang import testing
from oracle import moe_ref


# ------------------------------------------------------------ alignment ---
def test_align_known_answer_small():
    # ids per token: t0 -> (2, 0), t1 -> (0, 1), t2 -> (2, 1); E=3, B=4.
    ids = np.array([[2, 0], [0, 1], [2, 1]], dtype=np.int32)
    s, e, npp = moe_ref.align(ids, 3, 4)
    S = 6  # sentinel = numel
    assert npp == 12
    assert s.tolist() == [1, 2, S, S, 3, 5, S, S, 0, 4, S, S, S, S, S]
    assert e.tolist() == [0, 1, 2]


def test_align_known_answer_unused_expert_block1():
    ids = np.array([[3, 1]], dtype=np.int32)
    s, e, npp = moe_ref.align(ids, 4, 1)
    assert npp == 2 and s.tolist() == [1, 0] and e.tolist() == [1, 3]


def test_align_known_answer_dropped_and_empty():
    ids = np.array([[-1, 0], [5, 0]], dtype=np.int32)  # -1 and 5 not routed (E=2)
    s, e, npp = moe_ref.align(ids, 2, 2)
    assert npp == 2 and s[:2].tolist() == [1, 3] and (s[2:] == 4).all()
    assert e.tolist() == [0, -1, -1]  # max_padded = 4 + 2*(2-1) = 6
    s, e, npp = moe_ref.align(np.zeros((0, 2), np.int32), 3, 4)
    assert npp == 0 and (s == 0).all() and (e == -1).all()


def _reference_routing_steps(topk_weights, topk_ids, n_expts_tot):
    """The reference's conversion steps (ops/fused_moe.py:130-139) run with
    torch library ops: per-row sort, stable argsort, gather, histc. The
    argsort key relabels ids outside [0, E) as E (the one change the
    restatement makes, for slots the reference's callers never produce:
    they must sit behind expert E-1, outside every token_offs_raw range);
    ids in range are the reference's own keys."""
    expt_indx_2d, sort_indices = torch.sort(topk_ids, dim=1)
    expt_scal = torch.gather(topk_weights, 1, sort_indices).reshape(-1)
    expt_indx = expt_indx_2d.reshape(-1).to(torch.int32)
    key = torch.where((expt_indx >= 0) & (expt_indx < n_expts_tot), expt_indx,
                      torch.full_like(expt_indx, n_expts_tot))
    topk_indx = torch.argsort(key, stable=True)
    gate_scal = expt_scal[topk_indx]
    hist = torch.histc(expt_indx.float(), bins=n_expts_tot,
                       max=n_expts_tot - 1).int()
    return topk_indx, gate_scal, hist


@pytest.mark.parametrize("M,k,E,B", [(1, 2, 8, 16), (7, 2, 8, 16),
                                     (33, 4, 16, 32), (257, 8, 128, 64),
                                     (64, 8, 256, 16), (100, 1, 3, 5)])
def test_align_matches_reference_stable_order(M, k, E, B):
    g = torch.Generator().manual_seed(M + k + E + B)
    logits = torch.randn(M, E, generator=g)
    w, ids = moe_ref.route(logits, k)
    s, eids, npp = moe_ref.align(ids.numpy(), E, B)
    topk_indx, gate_scal, hist = _reference_routing_steps(w, ids.long(), E)
    valid = s[s < M * k]
    # same per-expert token sequence as the reference's stable argsort
    assert np.array_equal(valid // k, topk_indx.numpy() // k)
    # the gathered gate scales are the reference's gate_scal bit for bit
    assert torch.equal(w.reshape(-1)[torch.from_numpy(valid).long()], gate_scal)
    # per-expert padded segments
    padded = (hist.numpy() + B - 1) // B * B
    off = np.concatenate([[0], np.cumsum(padded)])
    assert npp == off[-1]
    for e in range(E):
        seg = s[off[e]:off[e + 1]]
        c = hist[e].item()
        assert (ids.numpy().reshape(-1)[seg[:c]] == e).all()
        assert (np.diff(seg[:c]) > 0).all()
        assert (seg[c:] == M * k).all()
        assert (eids[off[e] // B:off[e + 1] // B] == e).all()
    assert (eids[npp // B:] == -1).all()


@pytest.mark.parametrize("M,k,E,drop", [(1, 2, 8, False), (9, 4, 16, False),
                                          (33, 4, 16, True), (100, 8, 128, True),
                                          (64, 8, 256, False)])
def test_topk_to_routing_matches_reference_steps(M, k, E, drop):
    """The loop restatement equals the reference's conversion re-run with
    torch library ops (sort, stable argsort, gather, histc), including slots
    marked -1 (not routed), which go behind the last expert."""
    g = torch.Generator().manual_seed(M * 31 + k + E)
    w, ids = moe_ref.route(torch.randn(M, E, generator=g), k)
    ids = ids.long()
    if drop:
        ids[::3, 0] = -1
    gate_scal, topk_indx, gate_indx, hist = moe_ref.topk_to_routing(w, ids, E)
    r_indx, r_scal, r_hist = _reference_routing_steps(w, ids, E)
    assert np.array_equal(topk_indx, r_indx.numpy())
    assert np.array_equal(gate_scal, r_scal.numpy())
    assert np.array_equal(hist, r_hist.numpy())
    assert np.array_equal(gate_indx, torch.argsort(r_indx, stable=True).numpy())


def test_topk_to_routing_dropped_known_answer_round_trip():
    """Hand-worked: ids [[2, -1], [0, 1], [1, 3]], E = 4. Row-sorted flat ids
    [-1, 2, 0, 1, 1, 3]; the unrouted slot (flat 0) goes last:
    topk_indx [2, 3, 4, 1, 5, 0], hist [1, 2, 1, 1]. routing_order gives
    every slot back its id (-1 for flat 0: past the histogram's total) and
    weight, and the padded order of align() on the row-sorted ids."""
    w = torch.tensor([[0.25, 0.75], [0.5, 0.5], [0.125, 0.875]])
    ids = torch.tensor([[2, -1], [0, 1], [1, 3]])
    gate_scal, topk_indx, gate_indx, hist = moe_ref.topk_to_routing(w, ids, 4)
    assert topk_indx.tolist() == [2, 3, 4, 1, 5, 0]
    assert hist.tolist() == [1, 2, 1, 1]
    assert gate_indx.tolist() == [5, 3, 0, 1, 2, 4]
    assert gate_scal.tolist() == [0.5, 0.5, 0.125, 0.25, 0.875, 0.75]
    s, e, npp, rid, rw = moe_ref.routing_order(gate_scal, topk_indx, hist, 6, 2)
    assert rid.tolist() == [-1, 2, 0, 1, 1, 3]  # row-sorted: token 0 is [-1, 2]
    assert rw.tolist() == [0.75, 0.25, 0.5, 0.5, 0.125, 0.875]
    s_ref, e_ref, npp_ref = moe_ref.align(np.array([[-1, 2], [0, 1], [1, 3]]), 4, 2)
    assert npp == npp_ref == 8 and s.tolist() == s_ref.tolist()
    assert e.tolist() == e_ref.tolist()


@pytest.mark.parametrize("M,k,E,B", [(1, 2, 8, 16), (33, 4, 16, 32), (100, 8, 128, 64),
                                     (257, 2, 8, 256), (64, 8, 256, 1)])
def test_routing_order_inverts_topk_to_routing(M, k, E, B):
    """Round trip: routing_order(topk_to_routing(w, ids)) gives the row-sorted
    (weights, ids) back bit for bit, and its padded order equals align() of
    the row-sorted ids (align is pinned separately), dropped slots included."""
    g = torch.Generator().manual_seed(M + k + E + B)
    w, ids = moe_ref.route(torch.randn(M, E, generator=g), k)
    ids = ids.long()
    ids[::5, -1] = -1
    gate_scal, topk_indx, _, hist = moe_ref.topk_to_routing(w, ids, E)
    s, e, npp, rid, rw = moe_ref.routing_order(gate_scal, topk_indx, hist, M * k, B)
    sid, order = torch.sort(ids, dim=1)
    sw = torch.gather(w, 1, order)
    assert rid.tolist() == sid.reshape(-1).tolist()
    assert torch.equal(torch.from_numpy(rw), sw.reshape(-1))
    s_ref, e_ref, npp_ref = moe_ref.align(sid.numpy(), E, B)
    assert npp == npp_ref and s.tolist() == s_ref.tolist() and e.tolist() == e_ref.tolist()


def test_routing_order_clamps_a_bad_histogram():
    """Counts summing past n_gates are cut at n_gates; negative counts read
    as 0; out-of-range src entries become pads."""
    src = np.array([3, 0, 9, 1], dtype=np.int32)
    s, e, npp, rid, rw = moe_ref.routing_order(np.ones(4, np.float32), src, [-2, 3, 5], 4, 2)
    # h = [0, 3, 1]: expert 1 reads positions 0..2, expert 2 position 3
    assert npp == 6 and s[:6].tolist() == [3, 0, 4, 4, 1, 4]
    assert e.tolist() == [1, 1, 2]  # max_padded = 4 + 3 * 1 = 7: three blocks
    assert rid.tolist() == [1, 2, -7, 1]  # slot 2 is never named by src


def test_expt_data_known_answer():
    """Hand-worked tables: hist [3, 0, 17, 16] over 36 gates."""
    raw, pad, pid = moe_ref.expt_data([3, 0, 17, 16], 4, 36)
    assert raw.tolist() == [0, 3, 3, 20, 36]
    # max tiles: ceil((36 - 4 + 1) / 16) + 4 - 1 = 6
    assert pad[16].tolist() == [0, 1, 1, 3, 4]
    assert pid[16].tolist() == [0, 2, (1 << 16) + 2, 3, -1, -1]
    assert pad[32].tolist() == [0, 1, 1, 2, 3]
    assert pid[32].tolist() == [0, 2, 3, -1, -1, -1]
    assert pad[128].tolist() == [0, 1, 1, 2, 3]
    # fewer gates than experts: the table is n_gates long
    raw, pad, pid = moe_ref.expt_data([1, 0, 1], 3, 2)
    assert pid[16].tolist() == [0, 2]


@pytest.mark.parametrize("M,k,E", [(7, 2, 8), (257, 8, 128), (1024, 8, 64),
                                   (3, 8, 256)])
def test_expt_data_agrees_with_alignment(M, k, E):
    """The tile tables describe the alignment kernel's blocks: for each block
    size B, token_offs_pad * B are the padded segment offsets of
    moe_align_block_size(B), the tile -> expert map is its expert_ids, and the
    table bound holds every tile."""
    g = torch.Generator().manual_seed(M + k + E)
    w, ids = moe_ref.route(torch.randn(M, E, generator=g), k)
    hist = np.bincount(ids.numpy().reshape(-1), minlength=E)
    raw, pad, pid = moe_ref.expt_data(hist, E, M * k)
    assert np.array_equal(raw, np.concatenate([[0], np.cumsum(hist)]))
    for B in moe_ref.ROUTING_BLOCK_MS:
        s, eids, npp = moe_ref.align(ids.numpy(), E, B)
        assert pad[B][-1] * B == npp
        tiles = pad[B][-1]
        assert tiles <= len(pid[B]) == moe_ref.routing_max_tiles(M * k, E)
        assert np.array_equal(pid[B][:tiles] & 0xFFFF, eids[:tiles])
        for t in range(tiles):
            e, b = pid[B][t] & 0xFFFF, pid[B][t] >> 16
            assert pad[B][e] + b == t and b * B < hist[e]
        assert (pid[B][tiles:] == -1).all()


# ---------------------------------------------------------------- gating ---
def test_topk_gating_known_answers():
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.0], [0.5, -1.0, 2.0, 2.0]])
    w, ids = moe_ref.topk_gating(logits, 2)
    assert ids.tolist() == [[1, 2], [2, 3]]          # equal logits: lower id first
    assert torch.allclose(w, torch.full((2, 2), 0.5))  # equal scores, renormalised
    w, ids = moe_ref.topk_gating(logits, 3, renormalize=False)
    sm = torch.softmax(logits, -1)
    assert ids.tolist() == [[1, 2, 0], [2, 3, 0]]
    assert torch.allclose(w, torch.gather(sm, 1, ids.long()))
    w, ids = moe_ref.topk_gating(logits, 1, scoring="sigmoid", renormalize=False)
    assert ids.tolist() == [[1], [2]]
    assert torch.allclose(w[:, 0], torch.sigmoid(torch.tensor([3.0, 2.0])))


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_topk_gating_equals_reference_routing(scoring):
    """Without ties, ranking logits = ranking scores: same experts, same
    order and weights as the reference tests' torch.topk routing (route)."""
    g = torch.Generator().manual_seed(11)
    logits = torch.randn(200, 64, generator=g)
    w1, i1 = moe_ref.topk_gating(logits, 8, scoring=scoring)
    w2, i2 = moe_ref.route(logits, 8, scoring=scoring)
    assert torch.equal(i1, i2)
    assert torch.allclose(w1, w2, rtol=1e-6, atol=1e-7)


# -------------------------------------------------------------- silu*mul ---
def test_silu_and_mul_closed_form_float64():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(64, 256, generator=g) * 4).to(torch.bfloat16)
    got = moe_ref.silu_and_mul(x).float().numpy()
    xd = x.double().numpy()
    gd, ud = xd[:, :128], xd[:, 128:]
    want = gd * ud / (1.0 + np.exp(-gd))
    # one bf16 rounding of the exact value: relative error <= 2^-8
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-30)


def test_silu_and_mul_special_cases():
    x = torch.tensor([[0.0, 20.0, -30.0, 3.0, 2.0, 1.0]], dtype=torch.bfloat16)
    out = moe_ref.silu_and_mul(x).float()[0]
    assert out[0] == 0.0                      # silu(0) * u = 0
    assert abs(out[1] - 40.0) < 0.2           # silu(g) * u -> g * u, large g
    assert abs(out[2]) < 1e-10                # silu(g) -> 0 for very negative g


# ------------------------------------------------------------ quantisers ---
def _e4m3fn_decode(code: int) -> float:
    """OCP FP8 E4M3 (fn): 1 sign, 4 exponent (bias 7), 3 mantissa bits,
    subnormals, no infinities, S.1111.111 = NaN."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return math.nan
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_fp8_code_table_matches_ocp_layout():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float().tolist()
    for c in range(256):
        want = _e4m3fn_decode(c)
        if math.isnan(want):
            assert math.isnan(vals[c])
        else:
            assert vals[c] == want, c
    assert max(v for v in vals if not math.isnan(v)) == 448.0


def test_fp8_cast_is_round_to_nearest_even():
    table = sorted({_e4m3fn_decode(c) for c in range(256)} - {math.nan},
                   key=float)
    table = np.array([v for v in table if not math.isnan(v)])
    g = torch.Generator().manual_seed(1)
    x = (torch.rand(4000, generator=g) * 2 - 1) * 460
    x = torch.clamp(x, -448, 448)
    got = x.to(torch.float8_e4m3fn).float().numpy()
    for xi, gi in zip(x.numpy(), got):
        d = np.abs(table - xi)
        best = table[d == d.min()]
        if len(best) == 1:
            assert gi == best[0]
        else:  # tie: even mantissa (the candidate whose code is even)
            codes = [c for c in range(256) if _e4m3fn_decode(c) in best]
            even = [_e4m3fn_decode(c) for c in codes if c % 2 == 0]
            assert gi in even


def test_fp8_group_quant_roundtrip_and_amax():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(16, 512, generator=g) * 3).to(torch.bfloat16)
    q, s = moe_ref.quant_fp8_group(x, 128)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (16, 4)
    xf = x.float().reshape(16, 4, 128)
    assert torch.equal(s, xf.abs().amax(-1) / 448.0)
    deq = moe_ref.dequant_fp8_group(q, s, 128).reshape(16, 4, 128)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 above the subnormal range
    err = (deq - xf).abs()
    bound = 2.0 ** -4 * xf.abs() + 2.0 ** -10 * s[..., None]
    assert (err <= bound).all()
    # the group's amax element maps to +-448 exactly
    qa = q.float().reshape(16, 4, 128).abs().amax(-1)
    assert (qa == 448.0).all()


def test_int8_token_quant_roundtrip():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(8, 256, generator=g)).to(torch.bfloat16)
    q, s = moe_ref.quant_int8_token(x)
    xf = x.float()
    assert torch.equal(s, xf.abs().amax(-1) / 127.0)
    assert ((q.float() * s[:, None] - xf).abs() <= s[:, None] / 2 * (1 + 1e-6)).all()
    assert (q.abs().amax(-1) == 127).all()
    # round half to even on exact ties
    t = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5]], dtype=torch.bfloat16)
    q2, s2 = moe_ref.quant_int8_token(t)
    assert s2.item() == 1.0 and q2.tolist() == [[127, 0, 2, 2, 0]]


def test_weight_quantisers():
    g = torch.Generator().manual_seed(4)
    w = torch.randn(256, 384, generator=g) * 0.02
    q, s = moe_ref.quant_weight_fp8_block(w)
    assert s.shape == (2, 3)
    assert torch.allclose(s, w.reshape(2, 128, 3, 128).abs().amax((1, 3)) / 448)
    deq = moe_ref.dequant_weight_fp8_block(q, s)
    sb = s.repeat_interleave(128, 0).repeat_interleave(128, 1)
    assert ((deq - w).abs() <= 2.0 ** -4 * w.abs() + 2.0 ** -10 * sb).all()
    qi, si = moe_ref.quant_weight_int8_channel(w)
    assert ((qi.float() * si[:, None] - w).abs() <= si[:, None] / 2 * 1.000001).all()


# ------------------------------------------------------------- fused MoE ---
def _brute_force_moe(x, w1, w2, tw, tid, act="silu", b1=None, b2=None,
                     alpha=1.0, limit=0.0, on_input=False, gamma_first=False):
    """Token-by-token float64 MoE (no intermediate rounding); activations
    written from their textbook definitions with math.erf / exp."""
    x = x.double().numpy()
    w1 = w1.double().numpy()
    w2 = w2.double().numpy()
    N = w2.shape[2]
    out = np.zeros((x.shape[0], x.shape[1]))
    for t in range(x.shape[0]):
        for j in range(tid.shape[1]):
            e = int(tid[t, j])
            h = w1[e] @ x[t]
            if b1 is not None:
                h = h + b1[e].double().numpy()
            gam = float(tw[t, j])
            if on_input and (act != "swiglu" or gamma_first):
                h = h * gam
            gte, up = h[:N], h[N:]
            if act == "gelu":
                a = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in gte]) * up
            elif act == "swiglu":
                if limit > 0:
                    gte = np.minimum(gte, limit)
                    up = np.clip(up, -limit, limit)
                a = gte / (1.0 + np.exp(-alpha * gte)) * (up + 1.0)
                if on_input and not gamma_first:
                    a = a * gam
            else:
                a = gte / (1.0 + np.exp(-gte)) * up
            y = w2[e] @ a
            if b2 is not None:
                y = y + b2[e].double().numpy()
            out[t] += (1.0 if on_input else gam) * y
    return out


def _inputs(M, K, N, E, k, seed, scale=0.1):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * N, K, generator=g) * scale).to(torch.bfloat16)
    w2 = (torch.randn(E, K, N, generator=g) * scale).to(torch.bfloat16)
    w, ids = moe_ref.route(torch.randn(M, E, generator=g), k)
    return x, w1, w2, w, ids


@pytest.mark.parametrize("M,K,N,E,k", [(5, 32, 48, 4, 2), (9, 64, 16, 6, 3)])
def test_moe_matches_float64_brute_force(M, K, N, E, k):
    x, w1, w2, w, ids = _inputs(M, K, N, E, k, seed=M + K + N + E + k)
    got = moe_ref.fused_moe(x, w1, w2, w, ids).double().numpy()
    want = _brute_force_moe(x, w1, w2, w, ids)
    # three bf16 roundings on the way (h, a, y) plus the output rounding
    assert np.allclose(got, want, rtol=3e-2, atol=3e-2 * np.abs(want).max())


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_moe_activations_and_biases_match_float64_brute_force(act):
    M, K, N, E, k = 7, 64, 32, 4, 2
    x, w1, w2, w, ids = _inputs(M, K, N, E, k, seed=21)
    g = torch.Generator().manual_seed(22)
    b1 = b2 = None
    kw = {}
    if act == "swiglu":
        b1 = torch.randn(E, 2 * N, generator=g) * 0.5
        b2 = torch.randn(E, K, generator=g) * 0.5
        kw = dict(alpha=1.702, limit=1.5)  # a limit the activations do reach
    got = moe_ref.fused_moe(x, w1, w2, w, ids, activation=act, b1=b1, b2=b2,
                            **kw).double().numpy()
    want = _brute_force_moe(x, w1, w2, w, ids, act=act, b1=b1, b2=b2, **kw)
    assert np.allclose(got, want, rtol=3e-2, atol=3e-2 * np.abs(want).max())


def test_swiglu_router_weight_on_input_after_activation():
    """With the router weight on the input, the bias variant scales the fused
    swiglu's output (matmul_ogs's gammas act on its epilogue's result); the
    brute force with the weight applied to g and u first fails the same
    tolerance, so the test pins the placement."""
    M, K, N, E, k = 7, 64, 32, 4, 2
    x, w1, w2, w, ids = _inputs(M, K, N, E, k, seed=23)
    g = torch.Generator().manual_seed(24)
    b1 = torch.randn(E, 2 * N, generator=g) * 0.5
    b2 = torch.randn(E, K, generator=g) * 0.5
    kw = dict(alpha=1.702, limit=1.5)
    got = moe_ref.fused_moe(x, w1, w2, w, ids, activation="swiglu", b1=b1, b2=b2,
                            apply_router_weight_on_input=True, **kw).double().numpy()
    want = _brute_force_moe(x, w1, w2, w, ids, act="swiglu", b1=b1, b2=b2,
                            on_input=True, **kw)
    other = _brute_force_moe(x, w1, w2, w, ids, act="swiglu", b1=b1, b2=b2,
                             on_input=True, gamma_first=True, **kw)
    tol = 3e-2 * np.abs(want).max()
    assert np.allclose(got, want, rtol=3e-2, atol=tol)
    assert not np.allclose(got, other, rtol=3e-2, atol=tol)


def test_gelu_and_mul_closed_form():
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(32, 128, generator=g) * 3).to(torch.bfloat16)
    got = moe_ref.gelu_and_mul(x).double().numpy()
    xd = x.double().numpy()
    gd, ud = xd[:, :64], xd[:, 64:]
    want = 0.5 * gd * (1.0 + np.vectorize(math.erf)(gd / math.sqrt(2.0))) * ud
    # one bf16 rounding, plus fp32 cancellation in 1 + erf(g) for g << 0
    # (absolute, at most an fp32 ulp of 1 times |g * u|)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 2.0 ** -22 * np.abs(gd * ud))
    # gelu(1) = Phi(1) = 0.8413447460685429; gelu(0) = 0; gelu(-6) ~ 0
    t = torch.tensor([[1.0, 0.0, -6.0, 1.0, 5.0, 5.0]], dtype=torch.bfloat16)
    o = moe_ref.gelu_and_mul(t).float()[0]
    assert abs(o[0] - 0.8413447460685429) < 4e-3 and o[1] == 0.0 and abs(o[2]) < 1e-7


def test_swiglu_identities():
    g = torch.Generator().manual_seed(5)
    a = torch.randn(1000, generator=g) * 4
    b = torch.randn(1000, generator=g) * 4
    # alpha = 1, no clamp: silu(g) * (u + 1) (torch library silu)
    assert torch.allclose(moe_ref.swiglu(a, b),
                          torch.nn.functional.silu(a) * (b + 1), rtol=1e-6, atol=1e-6)
    # alpha = 1.702: g * sigmoid(1.702 g), the GPT-OSS gate
    assert torch.allclose(moe_ref.swiglu(a, b, alpha=1.702),
                          a * torch.sigmoid(1.702 * a) * (b + 1), rtol=1e-6, atol=1e-6)
    # limit clamps the gate from above only and the linear part both ways
    o = moe_ref.swiglu(torch.tensor([10.0, -10.0, 3.0]), torch.tensor([-10.0, 10.0, 0.0]),
                       alpha=1.0, limit=7.0)
    want = [7.0 * (1 / (1 + math.exp(-7.0))) * (-6.0),
            -10.0 * (1 / (1 + math.exp(10.0))) * 8.0,
            3.0 * (1 / (1 + math.exp(-3.0)))]
    assert np.allclose(o.numpy(), want, rtol=1e-6)


def test_moe_top1_unit_weight_is_plain_mlp():
    x, w1, w2, _, _ = _inputs(6, 32, 24, 1, 1, seed=5)
    ones = torch.ones(6, 1)
    zeros = torch.zeros(6, 1, dtype=torch.int32)
    got = moe_ref.fused_moe(x, w1, w2, ones, zeros).double()
    xd, w1d, w2d = x.double(), w1[0].double(), w2[0].double()
    h = xd @ w1d.t()
    a = torch.nn.functional.silu(h[:, :24]) * h[:, 24:]
    want = a @ w2d.t()
    assert torch.allclose(got, want, rtol=3e-2, atol=3e-2 * want.abs().max())


def test_moe_exact_invariants():
    x, w1, w2, w, ids = _inputs(12, 64, 32, 5, 2, seed=6)
    base = moe_ref.fused_moe(x, w1, w2, w, ids)
    # permuting tokens permutes the output rows
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(0))
    assert torch.equal(moe_ref.fused_moe(x[perm], w1, w2, w[perm], ids[perm]),
                       base[perm])
    # relabelling experts changes nothing
    relabel = torch.tensor([3, 0, 4, 1, 2])
    inv = torch.argsort(relabel)
    assert torch.equal(
        moe_ref.fused_moe(x, w1[inv], w2[inv], w, relabel[ids.long()].int()), base)
    # doubling the gate weights doubles the output exactly (fp32 sum, bf16 out)
    assert torch.equal(moe_ref.fused_moe(x, w1, w2, 2 * w, ids).float(),
                       2 * base.float())
    # a token subset equals the same rows of the full result
    sub = [11, 0, 5]
    assert torch.equal(moe_ref.fused_moe(x, w1, w2, w, ids, tokens=sub), base[sub])
    # on-input gating with unit top-1 weights equals output gating
    ones = torch.ones(12, 1)
    a1 = moe_ref.fused_moe(x, w1, w2, ones, ids[:, :1])
    a2 = moe_ref.fused_moe(x, w1, w2, ones, ids[:, :1],
                           apply_router_weight_on_input=True)
    assert torch.equal(a1, a2)


def test_moe_slot_order_and_dropped_slots():
    x, w1, w2, w, ids = _inputs(8, 64, 32, 4, 2, seed=7)
    base = moe_ref.fused_moe(x, w1, w2, w, ids)
    swapped = moe_ref.fused_moe(x, w1, w2, w.flip(1), ids.flip(1))
    assert torch.allclose(swapped.float(), base.float(), atol=1e-2, rtol=1e-2)
    # a slot routed to an out-of-range expert contributes nothing
    ids2 = ids.clone()
    ids2[:, 1] = -1
    w1only = w.clone()
    w1only[:, 1] = 0
    assert torch.equal(moe_ref.fused_moe(x, w1, w2, w, ids2),
                       moe_ref.fused_moe(x, w1, w2, w1only, ids))


# ------------------------------------- quantised modes, float64 brute force ---
def _e4m3_table():
    vals = sorted({_e4m3fn_decode(c) for c in range(256) if not math.isnan(_e4m3fn_decode(c))})
    return np.array(vals)


def _e4m3_round(v):
    """Nearest e4m3fn value of float64 v (|v| <= 448), ties to the even code,
    from the OCP code table (pinned above), not torch's cast."""
    table = _e4m3_table()
    even = {_e4m3fn_decode(c) for c in range(256) if c % 2 == 0}
    out = np.empty_like(v)
    for i, x in np.ndenumerate(v):
        d = np.abs(table - x)
        best = table[d == d.min()]
        out[i] = best[0] if len(best) == 1 else [b for b in best if b in even][0]
    return out


def _bf16(v):
    return torch.from_numpy(np.asarray(v, dtype=np.float32)).to(torch.bfloat16).double().numpy()


def _bruteforce_quant_moe(x, w1q, w2q, s1, s2, w, ids, mode):
    """The w8a8 layer in float64 with explicit loops over tokens, slots and
    scale blocks: weights dequantised element by element (fp8: scale block
    [r // 128, c // 128] of the [rows, cols] weight; int8: scale of output row
    r), activations quantised by the definitions (scale = max(amax, 1e-10) /
    448 per 1x128 group, or / 127 per row, in fp32; fp8 codes by the OCP
    table, int8 round half to even), GEMM1 output rounded to bf16, silu*up
    rounded to bf16, re-quantised, GEMM2 rounded to bf16, weighted fp64 sum
    rounded to bf16."""
    xd = x.float().double().numpy()
    T, K = xd.shape
    N = w2q.shape[2]
    out = np.zeros((T, K))

    def deq(q, sc, e):
        qd = q[e].float().double().numpy()
        R, C = qd.shape
        sd = sc[e].double().numpy()
        dq = np.empty((R, C))
        for r in range(R):
            if mode == "fp8":
                for cb in range(C // 128):
                    dq[r, cb * 128:(cb + 1) * 128] = qd[r, cb * 128:(cb + 1) * 128] * sd[r // 128, cb]
            else:
                dq[r] = qd[r] * sd[r]
        return dq

    def qdq(row):
        row = row.copy()
        if mode == "fp8":
            for g in range(len(row) // 128):
                seg = row[g * 128:(g + 1) * 128]
                sc = np.float32(max(np.float32(np.abs(seg).max()), np.float32(1e-10))) / np.float32(448.0)
                q = _e4m3_round(np.clip((seg.astype(np.float32) / sc).astype(np.float64), -448, 448))
                row[g * 128:(g + 1) * 128] = q * np.float64(sc)
            return row
        sc = np.float32(max(np.float32(np.abs(row).max()), np.float32(1e-10))) / np.float32(127.0)
        q = np.clip(np.round((row.astype(np.float32) / sc).astype(np.float64)), -127, 127)
        return q * np.float64(sc)

    cache = {}
    for t in range(T):
        xq = qdq(xd[t])
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            if e not in cache:
                cache[e] = (deq(w1q, s1, e), deq(w2q, s2, e))
            W13, W2 = cache[e]
            h = _bf16(W13 @ xq)
            g, u = h[:N], h[N:]
            a = _bf16(g / (1.0 + np.exp(-g)) * u)
            y = _bf16(W2 @ qdq(a))
            out[t] += float(w[t, j]) * y
    return _bf16(out)


def _quant_case(mode, K, N, E, seed):
    x, w1, w2, w, ids = _inputs(10, K, N, E, 2, seed=seed, scale=0.05)
    quant = moe_ref.quant_weight_fp8_block if mode == "fp8" else moe_ref.quant_weight_int8_channel
    q1 = [quant(w1[e]) for e in range(E)]
    q2 = [quant(w2[e]) for e in range(E)]
    w1q, w2q = torch.stack([a for a, _ in q1]), torch.stack([a for a, _ in q2])
    s1, s2 = torch.stack([b for _, b in q1]), torch.stack([b for _, b in q2])
    # scales that differ strongly between blocks / rows, so an operand's
    # scale read at the wrong index moves the result
    g = torch.Generator().manual_seed(seed)
    s1 = s1 * (0.5 + 3 * torch.rand(s1.shape, generator=g))
    s2 = s2 * (0.5 + 3 * torch.rand(s2.shape, generator=g))
    return x, w1q, w2q, s1, s2, w, ids


def _close_to_bruteforce(got, want):
    diff = np.abs(got.float().double().numpy() - want)
    return float(diff.sum() / np.abs(want).sum()), float(diff.max())


@pytest.mark.parametrize("mode", ["fp8", "int8"])
def test_quantised_oracle_matches_float64_bruteforce(mode):
    """oracle.fused_moe(mode=fp8|int8) against the float64 brute force on
    non-square shapes (fp8: a 4 x 3 block grid for W13, 3 x 2 for W2; int8:
    2N != K rows), where a scale read along the wrong axis cannot even be
    applied. The two differ only where the fp32 and fp64 sums round a bf16
    intermediate to neighbouring values (then the re-quantised element may
    move by one grid step)."""
    x, w1q, w2q, s1, s2, w, ids = _quant_case(mode, 384, 256, 3, 21)
    got = moe_ref.fused_moe(x, w1q, w2q, w, ids, mode=mode, w1_scale=s1, w2_scale=s2)
    want = _bruteforce_quant_moe(x, w1q, w2q, s1, s2, w, ids, mode)
    mean_rel, _ = _close_to_bruteforce(got, want)
    assert mean_rel <= 1e-4, mean_rel


@pytest.mark.parametrize("mode", ["fp8", "int8"])
def test_quantised_bruteforce_rejects_a_scale_axis_swap(mode, monkeypatch):
    """On a square shape (2N = K, a 2 x 2 fp8 block grid) a scale applied
    along the wrong axis keeps its shape; planted in the oracle's weight
    dequantisation, the brute-force comparison above rejects it."""
    x, w1q, w2q, s1, s2, w, ids = _quant_case(mode, 256, 128, 3, 22)
    want = _bruteforce_quant_moe(x, w1q, w2q, s1, s2, w, ids, mode)
    honest = moe_ref.fused_moe(x, w1q, w2q, w, ids, mode=mode, w1_scale=s1, w2_scale=s2)
    assert _close_to_bruteforce(honest, want)[0] <= 1e-4

    def swapped(mode_, a1, a2, sc1, sc2, e):
        a, b = a1[e].cpu(), a2[e].cpu()
        if mode_ == "fp8":
            return (moe_ref.dequant_weight_fp8_block(a, sc1[e].cpu().t().contiguous()),
                    moe_ref.dequant_weight_fp8_block(b, sc2[e].cpu()))
        return a.float() * sc1[e].cpu().float()[None, :], b.float() * sc2[e].cpu().float()[:, None]

    monkeypatch.setattr(moe_ref, "_expert_weights", swapped)
    bad = moe_ref.fused_moe(x, w1q, w2q, w, ids, mode=mode, w1_scale=s1, w2_scale=s2)
    assert _close_to_bruteforce(bad, want)[0] > 5e-2


def test_moe_quantised_modes_track_bf16():
    x, w1, w2, w, ids = _inputs(16, 256, 128, 4, 2, seed=8, scale=0.05)
    base = moe_ref.fused_moe(x, w1, w2, w, ids).float()
    q1 = [moe_ref.quant_weight_fp8_block(w1[e]) for e in range(4)]
    q2 = [moe_ref.quant_weight_fp8_block(w2[e]) for e in range(4)]
    fp8 = moe_ref.fused_moe(
        x, torch.stack([a for a, _ in q1]), torch.stack([a for a, _ in q2]), w,
        ids, mode="fp8", w1_scale=torch.stack([b for _, b in q1]),
        w2_scale=torch.stack([b for _, b in q2])).float()
    i1 = [moe_ref.quant_weight_int8_channel(w1[e]) for e in range(4)]
    i2 = [moe_ref.quant_weight_int8_channel(w2[e]) for e in range(4)]
    int8 = moe_ref.fused_moe(
        x, torch.stack([a for a, _ in i1]), torch.stack([a for a, _ in i2]), w,
        ids, mode="int8", w1_scale=torch.stack([b for _, b in i1]),
        w2_scale=torch.stack([b for _, b in i2])).float()
    for q in (fp8, int8):
        rel = (q - base).abs().sum() / base.abs().sum()
        assert rel < 0.08, rel


@pytest.mark.parametrize("mode", ["fp8", "int8"])
def test_quantised_tolerance_model(mode):
    """The fp8 / int8 elementwise bound absorbs GEMM1 results perturbed at
    the fp8 MFMA's accumulation precision (W13 scales times 1 + 2^-14: about
    2 % of the bf16 intermediate moves by an ulp and its re-quantisation
    flips grid points), and still rejects a 10 % error planted in one
    128-column weight-scale block of W2."""
    x, w1, w2, w, ids = _inputs(64, 512, 256, 4, 2, seed=9, scale=0.1)
    qf = moe_ref.quant_weight_fp8_block if mode == "fp8" else moe_ref.quant_weight_int8_channel
    q1 = [qf(w1[e]) for e in range(4)]
    q2 = [qf(w2[e]) for e in range(4)]
    W1, S1 = torch.stack([a for a, _ in q1]), torch.stack([b for _, b in q1])
    W2, S2 = torch.stack([a for a, _ in q2]), torch.stack([b for _, b in q2])
    tol = testing.TOL[mode]
    ref, mag = moe_ref.fused_moe(x, W1, W2, w, ids, mode=mode, w1_scale=S1,
                                 w2_scale=S2, return_mag=True)
    out2 = moe_ref.fused_moe(x, W1, W2, w, ids, mode=mode, w1_scale=S1 * (1 + 2.0 ** -14),
                             w2_scale=S2)
    assert not torch.equal(out2, ref)
    ok, _, mean_rel = moe_ref.compare(out2, ref, tol["atol"], tol["rtol"], mag)
    assert ok and mean_rel < tol["mean_rel"]
    S2bad = S2.clone()
    if mode == "fp8":
        S2bad[:, 0, :] *= 1.1   # output columns 0..127
    else:
        S2bad[:, :128] *= 1.1
    bad = moe_ref.fused_moe(x, W1, W2, w, ids, mode=mode, w1_scale=S1, w2_scale=S2bad)
    ok, _, _ = moe_ref.compare(bad, ref, tol["atol"], tol["rtol"], mag)
    assert not ok


def test_compare_helper():
    a = torch.tensor([1.0, 2.0, 3.0])
    ok, mx, mr = moe_ref.compare(a + 0.01, a, atol=2e-2, rtol=0)
    assert ok and abs(mx - 0.01) < 1e-6 and abs(mr - 0.005) < 1e-6
    ok, _, _ = moe_ref.compare(a + 0.5, a, atol=2e-2, rtol=1e-2)
    assert not ok


@pytest.mark.parametrize("plant", ["scale_2pct", "neighbour_scale"])
def test_regression_bound_rejects_one_wrong_scale(monkeypatch, plant):
    """DeepSeek-shaped contraction (K = 7168: 56 k blocks of 128): the fp8
    regression bound (testing.REGRESSION) rejects an output computed with one
    wrong activation scale -- block 17's scale 2 % off, which the tolerance
    contract (testing.TOL) lets through, or replaced by block 18's -- and
    still accepts GEMM1 results perturbed at the fp8 MFMA's accumulation
    precision (W13 scales times 1 + 2^-14). The planted error lives in the
    oracle."""
    M, K, N, E, k = 16, 7168, 256, 4, 2
    x, w1, w2, w, ids = _inputs(M, K, N, E, k, seed=31, scale=0.02)
    q1 = [moe_ref.quant_weight_fp8_block(w1[e]) for e in range(E)]
    q2 = [moe_ref.quant_weight_fp8_block(w2[e]) for e in range(E)]
    W1, S1 = torch.stack([a for a, _ in q1]), torch.stack([b for _, b in q1])
    W2, S2 = torch.stack([a for a, _ in q2]), torch.stack([b for _, b in q2])
    kw = dict(mode="fp8", w2_scale=S2)
    ref, mag = moe_ref.fused_moe(x, W1, W2, w, ids, return_mag=True, w1_scale=S1, **kw)
    tol, reg = testing.TOL["fp8"], testing.REGRESSION["fp8"]

    noisy = moe_ref.fused_moe(x, W1, W2, w, ids, w1_scale=S1 * (1 + 2.0 ** -14), **kw)
    assert not torch.equal(noisy, ref)
    st = testing.regression_stats(noisy, ref, mag)
    assert st["mean_rel"] <= reg["mean_rel"] and st["max_ulp_mag"] <= reg["ulp_mag"], st

    good = moe_ref.quant_fp8_group

    def wrong_scale(a, group=128):
        q, sc = good(a, group)
        if a.shape[-1] == K:  # the GEMM1 input: x
            sc = sc.clone()
            if plant == "scale_2pct":
                sc[:, 17] *= 1.02
            else:
                sc[:, 17] = sc[:, 18]
        return q, sc

    monkeypatch.setattr(moe_ref, "quant_fp8_group", wrong_scale)
    bad = moe_ref.fused_moe(x, W1, W2, w, ids, w1_scale=S1, **kw)
    ok, _, mean_rel = moe_ref.compare(bad, ref, tol["atol"], tol["rtol"], mag)
    if plant == "scale_2pct":
        assert ok and mean_rel <= tol["mean_rel"]  # the contract alone passes it
    st = testing.regression_stats(bad, ref, mag)
    assert st["mean_rel"] > reg["mean_rel"] and st["max_ulp_mag"] > reg["ulp_mag"], st
