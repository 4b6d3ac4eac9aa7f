"""GPU parity of the fused MoE against the CPU oracle.

Shapes: the reference's own test shapes (tests/accuracy_utils.py:114-131,
seed M+K+N+E+topk as in tests/test_fused_moe.py:66, weights randn*0.1),
compared on every token as the reference compares them, and the five
measured layer configurations at full size. Those compare a sample of
tokens chosen so that every row block the GEMMs run (each expert's last,
partly filled block included) holds at least one sampled row: each output
row depends only on its own token, so the oracle computes exactly those
rows (weights stay on the GPU; only touched experts are copied to the
host).

Tolerance: |res - ref| <= atol + rtol*s elementwise, where s is the
magnitude sum_j |w_j * y_j| of the top-k terms an output sums (outputs that
cancel towards 0 keep the rounding error of their terms; fp8 / int8 add a
sixteenth of the absolute GEMM2 dot product, the scale on which the
re-quantised intermediate's grid-point flips move y), and
sum|res - ref| / sum|ref| <= mean_rel, with (atol, rtol, mean_rel) =
(2e-2, 1e-2, 1e-2) for bf16 and (5e-2, 2e-2, 5e-2) for fp8 / int8 against
the dequantising oracle.
"""

import pytest
import torch

import flaggems_sglang
from flaggems_sglang import _capi, testing
from flaggems_sglang.ops import fused_moe as fm
from oracle import moe_ref

pytestmark = pytest.mark.gpu


# (case, mode, max_abs, max ulps of |ref|, max ulps of the term magnitude,
# mean_rel) of every check; conftest writes them out when FGS_PARITY_LOG
# names a file
PARITY = []


def _check(res, ref, mode, what="", ulp_mag=None):
    """``ref`` is the oracle's output or its (output, term magnitude) pair.

    Two bars: the tolerance contract (elementwise ``atol + rtol * s`` and
    ``mean_rel``, ``testing.TOL``) and the regression bound
    (``testing.REGRESSION``: about ten times the error this build measures,
    so that a plausible kernel bug -- one wrong activation scale among 56
    k blocks -- fails); ``ulp_mag`` replaces the latter's term-magnitude
    bound for one check."""
    tol = testing.TOL[mode]
    reg = testing.REGRESSION[mode]
    mag = None
    if isinstance(ref, tuple):
        ref, mag = ref
    ok, max_abs, mean_rel = moe_ref.compare(res, ref, tol["atol"], tol["rtol"], mag)
    st = testing.regression_stats(res, ref, mag)
    PARITY.append(dict(case=what, mode=mode, **st))
    print(f"{what} max_abs={max_abs:.4g} ulp(ref)={st['max_ulp_ref']:.3g} "
          f"ulp(mag)={st['max_ulp_mag']:.3g} mean_rel={mean_rel:.4g}")
    assert ok, f"{what}: elementwise tolerance failed (max_abs={max_abs})"
    assert mean_rel <= tol["mean_rel"], f"{what}: mean_rel={mean_rel}"
    assert mean_rel <= reg["mean_rel"], f"{what}: mean_rel={mean_rel} (regression bound)"
    bound = reg["ulp_mag"] if ulp_mag is None else ulp_mag
    assert st["max_ulp_mag"] <= bound, \
        f"{what}: {st['max_ulp_mag']:.3g} ulps of the term magnitude"


def _sample(M, n=24):
    if M <= n:
        return list(range(M))
    g = torch.Generator().manual_seed(M)
    idx = torch.randperm(M, generator=g)[: n - 2].tolist()
    return sorted(set(idx + [0, M - 1]))


def _ref_inputs(M, K, N, E, topk, device, scale=0.1):
    torch.manual_seed(M + K + N + E + topk)
    g = torch.Generator(device=device).manual_seed(M + K + N + E + topk)
    x = torch.randn(M, K, generator=g, device=device).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * N, K, generator=g, device=device) * scale).to(torch.bfloat16)
    w2 = (torch.randn(E, K, N, generator=g, device=device) * scale).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g, device=device, dtype=torch.float32)
    w, ids = moe_ref.route(logits.cpu(), topk)
    return x, w1, w2, w.to(device), ids.to(device)


def _per_slot_ref(x, w1, w2, w, ids, ascending=False, **kw):
    """The oracle's rows of an uncombined call: row (t, r) is token t's r-th
    slot alone (top-1 with its weight), bf16(w * y) -- slots in the given
    order, or in ascending expert id (the routing tuple's order)."""
    ids, w = ids.long().cpu(), w.cpu()
    if ascending:
        order = torch.argsort(ids, dim=1)
        ids, w = torch.gather(ids, 1, order), torch.gather(w, 1, order)
    xr = x.repeat_interleave(ids.shape[1], dim=0)
    return moe_ref.fused_moe(xr, w1, w2, w.reshape(-1, 1), ids.reshape(-1, 1).int(),
                             return_mag=True, **kw)


@pytest.mark.parametrize("shape", testing.REF_SHAPES_SMALL + testing.REF_SHAPES_LARGE,
                         ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_fused_moe_reference_shapes(gpu, shape):
    """Every output element of every token, as the reference's own test
    compares them (tests/test_fused_moe.py:98-110)."""
    M, K, N, E, topk = shape
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    res = flaggems_sglang.fused_moe(x, w1, w2, w, ids)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, return_mag=True)
    assert res.shape == (M, K)
    _check(res.cpu(), ref, "bf16", f"ref-shape {shape}")


@pytest.mark.parametrize("shape", testing.REF_SHAPES_SMALL,
                         ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_fused_moe_input_gate(gpu, shape):
    M, K, N, E, topk = shape
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    res = flaggems_sglang.fused_moe(x, w1, w2, w, ids,
                                    apply_router_weight_on_input=True)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, apply_router_weight_on_input=True,
                            return_mag=True)
    _check(res.cpu(), ref, "bf16", f"input-gate {shape}")


def _row_sorted(w, ids):
    """Each token's slots by ascending expert id (the routing tuple's flat
    order, ops/fused_moe.py:130), as (weights, ids) on the same device."""
    sid, order = torch.sort(ids.long(), dim=1)
    return torch.gather(w, 1, order), sid.to(torch.int32)


@pytest.mark.parametrize("on_input", [False, True], ids=["out-gate", "in-gate"])
@pytest.mark.parametrize("shape", testing.REF_SHAPES_SMALL + testing.REF_SHAPES_LARGE,
                         ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_triton_kernel_fused_experts_compat(gpu, shape, on_input):
    """Reference signature and layouts: w1 [E, K, 2N], w2 [E, N, K] and the
    (RoutingData, GatherIndx, ScatterIndx) routing format, consumed directly
    (fgs_moe_fused_routed). Every token against the oracle, and bit for bit
    against fused_moe on the same routing in the tuple's slot order (same
    kernels, same row order, same slot order in the sum)."""
    M, K, N, E, topk = shape
    if on_input and shape not in testing.REF_SHAPES_SMALL:
        pytest.skip("the reference tests the input gate on its small shapes only")
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    w1_ref = w1.transpose(1, 2).contiguous()
    w2_ref = w2.transpose(1, 2).contiguous()
    rd, gi, si = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    res = flaggems_sglang.triton_kernel_fused_experts(
        x, w1_ref, w2_ref, rd, gi, si, apply_router_weight_on_input=on_input)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, apply_router_weight_on_input=on_input,
                            return_mag=True)
    _check(res.cpu(), ref, "bf16", f"compat {shape} on_input={on_input}")
    sw, sids = _row_sorted(w, ids)
    res_native = flaggems_sglang.fused_moe(x, w1, w2, sw, sids,
                                           apply_router_weight_on_input=on_input)
    assert torch.equal(res, res_native)


@pytest.mark.parametrize("M", [1, 48])
def test_triton_kernel_fused_experts_dropped_slot(gpu, M):
    """A tuple from standard_topk_to_routing with unrouted slots (-1: they go
    behind the last expert, outside every token_offs_raw range) gives what
    fused_moe gives for the same slots, bit for bit, and the inverse hands
    the -1 back (M=1: the one-token schedule, where GEMM1 finds each
    gathered position's expert from the histogram)."""
    K, N, E, topk = 256, 512, 8, 2
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    ids = ids.clone()
    ids[::4, 0] = -1
    rd, gi, si = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    tw, ti = fm._routing_to_topk(rd, gi, M)
    sw, sids = _row_sorted(w, ids)
    assert torch.equal(ti, sids) and torch.equal(tw, sw)
    res = flaggems_sglang.triton_kernel_fused_experts(
        x, w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous(), rd, gi, si)
    assert torch.equal(res, flaggems_sglang.fused_moe(x, w1, w2, sw, sids))
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, return_mag=True)
    _check(res.cpu(), ref, "bf16", "compat dropped slots")


@pytest.mark.parametrize("mode", ["fp8", "int8", "bf16"])
@pytest.mark.parametrize("M", [1, 3, 300])
def test_fused_routed_quantised_bit_identical(gpu, mode, M):
    """fgs_moe_fused_routed with fp8 / int8 / bf16 weights (one token: the
    direct schedule; more: the routing-order kernel in place of the
    alignment) gives fused_moe's bits on the same routing in the tuple's
    slot order, dropped slots included."""
    K, N, E, topk = 512, 256, 16, 4
    cfg = testing.MoEConfig("t", K, N, E, topk, (M,), mode=mode)
    wts = testing.make_weights(K, N, E, mode, 0.05, device=gpu)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=M + 5)
    ti = ti.clone()
    ti[::2, 1] = -1
    rd, gi, _ = flaggems_sglang.standard_topk_to_routing(tw, ti, E)
    qm = {"bf16": None, "fp8": _capi.QMODE_FP8_BLOCK, "int8": _capi.QMODE_INT8_CHANNEL}[mode]
    res = fm._fused_routed(x, wts.w1, wts.w2, rd, gi, qmode=qm, w1_scale=wts.w1_scale,
                           w2_scale=wts.w2_scale)
    sw, sids = _row_sorted(tw, ti)
    ref = flaggems_sglang.fused_moe(x, wts.w1, wts.w2, sw, sids, **wts.kwargs(cfg.mode))
    assert torch.equal(res, ref)


@pytest.mark.parametrize("sched", [_capi.FLAG_FORCE_DECODE, _capi.FLAG_FORCE_PREFILL, 0],
                         ids=["decode", "prefill", "auto"])
@pytest.mark.parametrize("shape", [(1, 128, 256, 8, 2), (96, 256, 512, 16, 4),
                                   (700, 512, 256, 8, 2), (1000, 1024, 384, 4, 2),
                                   (3000, 768, 640, 8, 3)])
def test_schedules_agree(gpu, shape, sched):
    M, K, N, E, topk = shape
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    res = fm.fused_moe(x, w1, w2, w, ids, _flags=sched)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, tokens=_sample(M, 64), return_mag=True)
    _check(res.cpu()[_sample(M, 64)], ref, "bf16", f"sched {sched} {shape}")


@pytest.mark.parametrize("cfg", range(_capi.TILED_CONFIGS))
@pytest.mark.parametrize("shape", [(40, 256, 256, 4, 2), (300, 512, 384, 8, 3),
                                   (1500, 1024, 1024, 8, 2)])
def test_tiled_configs(gpu, shape, cfg):
    """Every LDS-tiled configuration, forced, on shapes that leave partial
    and empty row blocks."""
    M, K, N, E, topk = shape
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    res = fm.fused_moe(x, w1, w2, w, ids, _flags=_capi.flag_tile(cfg))
    toks = _sample(M, 64)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, "bf16", f"tile {cfg} {shape}")


_QUANT_TILES = [("fp8", c) for c in range(_capi.TILED_CONFIGS)] + \
               [("int8", c) for c in range(_capi.TILED_CONFIGS)]


@pytest.mark.parametrize("mode,cfg", _QUANT_TILES, ids=[f"{m}-{c}" for m, c in _QUANT_TILES])
@pytest.mark.parametrize("shape", [(300, 512, 512, 8, 3), (1500, 1024, 768, 8, 2)])
def test_tiled_configs_quantised(gpu, shape, mode, cfg):
    """fp8 (128x128 block scales) and int8 (per-channel) tiled kernels, each
    configuration forced, against the dequantising oracle."""
    M, K, N, E, topk = shape
    seed = M + K + N + E + topk
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=seed)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=seed)
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=_capi.flag_tile(cfg),
                       **wts.kwargs(mode))
    toks = _sample(M, 32)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode,
                            w1_scale=wts.w1_scale, w2_scale=wts.w2_scale,
                            tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, mode, f"{mode} tile {cfg} {shape}")


@pytest.mark.parametrize("mode", ["fp8", "int8"])
def test_quantised_schedules_agree(gpu, mode):
    """Streaming and tiled kernels of a quantised mode on the same inputs:
    both match the oracle; int8, which sums exactly in int32 before the same
    dequantisation, also matches bit for bit (fp8's streaming and tiled
    MFMA shapes round their k-block partials differently here)."""
    M, K, N, E, topk = 700, 1024, 512, 8, 2
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=7)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=7)
    dec = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=_capi.FLAG_FORCE_DECODE,
                       **wts.kwargs(mode))
    pre = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=_capi.FLAG_FORCE_PREFILL,
                       **wts.kwargs(mode))
    toks = _sample(M, 32)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode,
                            w1_scale=wts.w1_scale, w2_scale=wts.w2_scale,
                            tokens=toks, return_mag=True)
    _check(dec.cpu()[toks], ref, mode, f"{mode} decode")
    _check(pre.cpu()[toks], ref, mode, f"{mode} prefill")
    if mode == "int8":
        assert torch.equal(dec, pre), "int8: streaming and tiled schedules differ"


# ------------------------------------------------------ one-token decode ---
# M = 1 runs the direct-row schedule: no alignment, slot j is row tile j
# (its expert topk_ids[j]); GEMM2 folds the weighted top-k sum
# (FLAG_FOLD_SUM forces it) or leaves it to moe_sum (FLAG_SEPARATE_SUM).
# Covered: both GEMM2 forms for every mode, top-k
# of 2, odd (3: idle waves), above the 16 waves (20: slots dealt round
# robin), 64, 128 and 192 output column tiles of 16 (below 192 the fold runs
# two slots per MFMA on 8-column workgroups: odd top-k 7 leaves a pair's
# second slot absent, top-k 32 is its 16-pair limit), dropped slots and the
# router weight on the input.
@pytest.mark.parametrize("mode", ["bf16", "fp8", "int8"])
@pytest.mark.parametrize("K,N,E,topk", [(3072, 256, 8, 2), (3072, 256, 32, 3),
                                        (3072, 256, 64, 20), (1024, 512, 16, 4),
                                        (2048, 256, 64, 7), (1024, 256, 64, 32)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("variant", ["plain", "dropped", "on_input"])
@pytest.mark.parametrize("fold", [True, False], ids=["folded", "separate"])
def test_single_token(gpu, mode, K, N, E, topk, variant, fold):
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=K + N + E + topk)
    x, tw, ti = testing.make_tokens(1, K, E, topk, device=gpu, seed=K + E + topk)
    if variant == "dropped":
        ti = ti.clone()
        ti[0, 0] = -1
        if topk > 2:
            ti[0, -1] = E + 2
    on_input = variant == "on_input"
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, apply_router_weight_on_input=on_input,
                       _flags=_capi.FLAG_FOLD_SUM if fold else _capi.FLAG_SEPARATE_SUM,
                       **wts.kwargs(mode))
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, apply_router_weight_on_input=on_input,
                            return_mag=True)
    _check(res.cpu(), ref, mode, f"M=1 {mode} {(K, N, E, topk)} {variant}")


# An fp8 token's GEMMs quantise x and the GEMM1 output themselves, an int8
# token's GEMM2 the GEMM1 output (per-token scales; x keeps its quantiser);
# with FLAG_SEPARATE_QUANT the quantiser kernels do. Same arithmetic, so the
# outputs are bit-identical (both GEMM2 forms; top-k 20 deals slots to the
# folded GEMM2's waves in turn, top-k 64 is the on-the-fly limit).
@pytest.mark.parametrize("mode", ["fp8", "int8"])
@pytest.mark.parametrize("K,N,E,topk", [(3072, 256, 8, 2), (3072, 256, 32, 3),
                                        (3072, 256, 64, 20), (1024, 512, 16, 4),
                                        (1024, 256, 64, 64), (7168, 2048, 16, 8)],
                         ids=lambda v: str(v))
@pytest.mark.parametrize("fold", [True, False], ids=["folded", "separate"])
def test_single_token_quant_fold(gpu, mode, K, N, E, topk, fold):
    sched = _capi.FLAG_FOLD_SUM if fold else _capi.FLAG_SEPARATE_SUM
    qm = _capi.QMODE_FP8_BLOCK if mode == "fp8" else _capi.QMODE_INT8_CHANNEL
    expect = " qfold" if mode == "fp8" else " qfold_a2"
    assert _capi.schedule(1, K, N, E, topk, qm, sched).endswith(expect)
    assert "qfold" not in _capi.schedule(1, K, N, E, topk, qm,
                                         sched | _capi.FLAG_SEPARATE_QUANT)
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=K + N + E + topk + 7)
    x, tw, ti = testing.make_tokens(1, K, E, topk, device=gpu, seed=K + E + topk + 7)
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=sched, **wts.kwargs(mode))
    sep = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=sched | _capi.FLAG_SEPARATE_QUANT,
                       **wts.kwargs(mode))
    assert torch.equal(res, sep), "on-the-fly quantisation differs from the quantisers"
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, return_mag=True)
    _check(res.cpu(), ref, mode, f"M=1 qfold {mode} {(K, N, E, topk)}")


def test_single_token_deterministic(gpu):
    wts = testing.make_weights(3072, 256, 8, "bf16", 0.1, device=gpu, seed=5)
    x, tw, ti = testing.make_tokens(1, 3072, 8, 2, device=gpu, seed=5)
    a = fm.fused_moe(x, wts.w1, wts.w2, tw, ti)
    for _ in range(3):
        assert torch.equal(fm.fused_moe(x, wts.w1, wts.w2, tw, ti), a)


# --------------------------------------------------------- stage profiler ---
def test_stage_profiler_modes(gpu):
    """Mode 1 times every stage; mode 2 only GEMM1 through GEMM2 and mode 3
    only GEMM1, the other stages reading 0 (events of earlier calls are not
    mixed in)."""
    import ctypes
    lib = _capi.load()
    x, w1, w2, w, ids = _ref_inputs(300, 256, 128, 8, 2, gpu)
    stage = (ctypes.c_float * 6)()
    lib.fgs_moe_profile_read(stage, 6)
    try:
        for mode in (1, 2, 3):
            lib.fgs_moe_profile_enable(mode)
            for _ in range(3):
                fm.fused_moe(x, w1, w2, w, ids)
            lib.fgs_moe_profile_enable(0)
            assert lib.fgs_moe_profile_read(stage, 6) == 3
            got = dict(zip(_capi.PROFILE_STAGES, list(stage)))
            assert got["gemm1"] > 0, got
            if mode == 1:
                assert got["align"] > 0 and got["moe_sum"] > 0, got
            else:
                assert got["align"] == 0 and got["quant_x"] == 0 and got["moe_sum"] == 0, got
            assert (got["gemm2"] > 0) == (mode != 3), got
    finally:
        lib.fgs_moe_profile_enable(0)
        lib.fgs_moe_profile_read(stage, 6)


# ------------------------------------------------------------ k-split GEMM2 ---
@pytest.mark.parametrize("mode", ["bf16", "int8"])
@pytest.mark.parametrize("shape", [(3328, 1024, 2048, 8, 2), (3328, 1024, 4608, 8, 2),
                                   (832, 1024, 2048, 8, 8)],
                         ids=["top2", "top2_long_k", "top8"])
def test_gemm2_k_split(gpu, shape, mode):
    """Shapes whose GEMM2 grid (about 30 row blocks x 4 column tiles) is
    split in two over k: fp32 partials of the 4-wave kernel (k row <= 8 KiB)
    or of the 8-wave one (bf16 at N=4608), reduced with the top-k sum in
    fixed order."""
    M, K, N, E, topk = shape
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=M + K + N)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=M + K + N)
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, **wts.kwargs(mode))
    toks = _sample(M, 32)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, mode, f"k-split {shape} {mode}")


@pytest.mark.parametrize("mode", ["bf16", "int8"])
@pytest.mark.parametrize("shape", [(4096, 4096, 512, 8, 2), (3500, 4096, 1024, 8, 2),
                                   (2600, 2048, 768, 16, 3)],
                         ids=["rem8_S4", "rem_S2", "E16_top3"])
def test_gemm2_tail_split(gpu, shape, mode):
    """GEMM2 of 256-row blocks over 1 to 8 rounds of the CUs runs on the
    4-wave kernel with its last round's tiles split over k into pieces whose
    fp32 partials a fixup kernel adds in order (M=4096 top-2 over 8 experts:
    about 36 row blocks x 16 column tiles = 72 tiles per XCD, the last 8 in 4
    pieces each)."""
    M, K, N, E, topk = shape
    wts = testing.make_weights(K, N, E, mode, 0.05, device=gpu, seed=M + K + N + 1)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=M + K + N + 1)
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, **wts.kwargs(mode))
    toks = _sample(M, 24)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, mode, f"tail split {shape} {mode}")
    # every token: the fixed-up tiles cover whole column ranges, so compare
    # all rows against a second, deterministic call
    again = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, **wts.kwargs(mode))
    assert torch.equal(res, again)


def _routing_with_counts(counts, device, seed):
    """Top-2 routing giving expert e exactly counts[e] slots: token t takes
    entries t and M + t of the expert-sorted slot list (distinct experts while
    no count exceeds M), weights from a seeded softmax pair."""
    total = sum(counts)
    assert total % 2 == 0 and max(counts) <= total // 2
    M = total // 2
    slots = torch.cat([torch.full((c,), e, dtype=torch.int32) for e, c in enumerate(counts)])
    ids = torch.stack([slots[:M], slots[M:]], 1)
    g = torch.Generator().manual_seed(seed)
    w = torch.softmax(torch.randn(M, 2, generator=g), dim=1)
    return w.to(device), ids.to(device)


_REMAINDER_CASES = [("bf16", 256, 1), ("bf16", 128, 1), ("int8", 256, 1), ("fp8", 256, 1),
                    ("bf16", 256, 2), ("bf16", 128, 2), ("int8", 256, 2)]


@pytest.mark.parametrize("mode,N,full", _REMAINDER_CASES,
                         ids=[f"{m}-{n}-{f}" for m, n, f in _REMAINDER_CASES])
def test_block_remainders(gpu, mode, N, full):
    """256-row tiles (the 4-wave kernel) on experts whose last block holds
    1, 8, 31..33, 63..65 or 200 rows after `full` or `full` + 1 full blocks
    -- the partially filled 32-row MFMA blocks and the all-pad ones the
    kernel skips -- every token checked (N=128: a GEMM2 of two k stages, the
    ring depth; full=2: ~690 rows per expert, where GEMM2 issues its
    activation rows rather than its weight rows a stage early). fp8 (the
    8-wave kernel): blocks of up to 160 rows run its compact 4-slot ring,
    fuller ones the 3-slot ring over all 256 rows, so its remainders
    straddle that edge."""
    K, E = 512, 10
    rem = [1, 8, 31, 32, 33, 63, 64, 65, 200, 1]
    if mode == "fp8":
        rem = [1, 33, 128, 159, 160, 161, 200, 255, 65, 8]
    counts = [256 * (full + e % 2) + r for e, r in enumerate(rem)]
    w, ids = _routing_with_counts(counts, gpu, seed=N)
    M = ids.shape[0]
    wts = testing.make_weights(K, N, E, mode, 0.05, device=gpu, seed=K + N + 7)
    g = torch.Generator(device=gpu).manual_seed(N + 11)
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.bfloat16)
    res = fm.fused_moe(x, wts.w1, wts.w2, w, ids, _flags=_capi.flag_tile(0),
                       **wts.kwargs(mode))
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, w, ids, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, return_mag=True)
    # fp8 checks all ~2500 tokens: GEMM1's bf16 output is requantised to
    # fp8, where a one-step flip against the oracle's rounding is 32 bf16
    # ulps of that element; over this many rows one reaches 5 ulps of the
    # term magnitude, so this check's bound is 8 (sampled checks keep 4)
    _check(res.cpu(), ref, mode, f"block remainders N={N} {mode}",
           ulp_mag=8.0 if mode == "fp8" else None)
    again = fm.fused_moe(x, wts.w1, wts.w2, w, ids, _flags=_capi.flag_tile(0),
                         **wts.kwargs(mode))
    assert torch.equal(res, again)


@pytest.mark.parametrize("mode,K,N", [("bf16", 512, 256), ("int8", 512, 256), ("fp8", 512, 256),
                                      ("fp8", 1024, 512)])
def test_tiled_configs_bit_identical(gpu, mode, K, N):
    """Every tiled configuration -- 256/128/64/32/160-row blocks, the 4-wave
    kernel, the fp8 tile's compact and full rings -- computes each output
    element with the same operations in the same order (per 128-byte k
    stage the same MFMA k steps, then the same scale fold), so on the same
    inputs all of them give the same bits; blocks holding 1..255 rows after
    full ones (the ring edge at 160 included) exercise every partial-block
    path. A layout or indexing slip in any one configuration breaks this
    even where it stays inside the oracle tolerance."""
    rem = [1, 33, 128, 159, 160, 161, 200, 255, 65, 8]
    counts = [256 * (1 + e % 2) + r for e, r in enumerate(rem)]
    w, ids = _routing_with_counts(counts, gpu, seed=N)
    M = ids.shape[0]
    wts = testing.make_weights(K, N, len(counts), mode, 0.05, device=gpu, seed=K + N + 7)
    g = torch.Generator(device=gpu).manual_seed(N + 11)
    x = torch.randn(M, K, generator=g, device=gpu).to(torch.bfloat16)
    outs = [fm.fused_moe(x, wts.w1, wts.w2, w, ids, _flags=_capi.flag_tile(cfg), **wts.kwargs(mode))
            for cfg in range(_capi.TILED_CONFIGS)]
    for cfg in range(1, _capi.TILED_CONFIGS):
        assert torch.equal(outs[0], outs[cfg]), f"{mode} K={K} N={N}: tile 0 vs tile {cfg}"


# ------------------------------------------------- activations and biases ---
_SCHEDS = [_capi.FLAG_FORCE_DECODE, _capi.FLAG_FORCE_PREFILL]


@pytest.mark.parametrize("sched", _SCHEDS, ids=["decode", "prefill"])
@pytest.mark.parametrize("shape", [(5, 256, 128, 4, 2), (600, 512, 384, 8, 2),
                                   (1, 3072, 128, 4, 2)])
def test_gelu_activation(gpu, shape, sched):
    """activation="gelu": exact-erf gelu(gate) * up in GEMM1's epilogue
    (sgl_kernel gelu_and_mul, ops/fused_moe.py:219-220)."""
    M, K, N, E, topk = shape
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    res = fm.fused_moe(x, w1, w2, w, ids, activation="gelu", _flags=sched)
    toks = _sample(M, 48)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, tokens=toks, return_mag=True,
                            activation="gelu")
    _check(res.cpu()[toks], ref, "bf16", f"gelu {shape}")
    # the reference-signature entry point takes the same activation
    routing, gather, scatter = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    res2 = flaggems_sglang.triton_kernel_fused_experts(
        x, w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous(),
        routing, gather, scatter, activation="gelu")
    _check(res2.cpu()[toks], ref, "bf16", f"gelu compat {shape}")


def _interleave_rows(w):
    """[gate block | linear block] rows -> g0, u0, g1, u1, ... (the layout
    matmul_ogs's fused swiglu reads)."""
    n = w.shape[-2] // 2 if w.ndim == 3 else w.shape[-1] // 2
    if w.ndim == 2:
        return torch.stack([w[:, :n], w[:, n:]], dim=2).reshape(w.shape)
    return torch.stack([w[:, :n], w[:, n:]], dim=2).reshape(w.shape)


def _bias_inputs(M, K, N, E, topk, device):
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, device)
    g = torch.Generator(device=device).manual_seed(M + 1)
    b1 = torch.randn(E, 2 * N, generator=g, device=device) * 0.5
    b2 = torch.randn(E, K, generator=g, device=device) * 0.5
    return x, w1, w2, b1, b2, w, ids


@pytest.mark.parametrize("on_input", [False, True], ids=["gammas_out", "gammas_in"])
@pytest.mark.parametrize("sched", _SCHEDS, ids=["decode", "prefill"])
@pytest.mark.parametrize("shape", [(7, 256, 128, 4, 2), (500, 512, 256, 8, 2),
                                   (1, 3072, 128, 4, 2), (1, 256, 128, 4, 3)])
def test_bias_swiglu(gpu, shape, sched, on_input):
    """Bias variant (ops/fused_moe.py:235-325): GEMM1 + b1 with swiglu(alpha,
    limit) fused, GEMM2 + b2, on interleaved gate/linear rows."""
    M, K, N, E, topk = shape
    x, w1, w2, b1, b2, w, ids = _bias_inputs(M, K, N, E, topk, gpu)
    res = fm.fused_moe_with_bias(x, _interleave_rows(w1), _interleave_rows(b1), w2,
                                 b2, w, ids, apply_router_weight_on_input=on_input,
                                 gemm1_alpha=1.702, gemm1_clamp_limit=7.0,
                                 _flags=sched)
    toks = _sample(M, 48)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, tokens=toks, return_mag=True,
                            activation="swiglu", b1=b1, b2=b2, alpha=1.702,
                            limit=7.0, apply_router_weight_on_input=on_input)
    _check(res.cpu()[toks], ref, "bf16", f"bias swiglu {shape}")


# Quantised weights in the bias variant (what the reference's w1_pcg / w2_pcg
# precision configs carry into matmul_ogs, :296-301): fp8 with 128x128 block
# scales on gate-then-linear rows, int8 with per-channel scales on interleaved
# rows (scales de-interleaved with the rows); both schedules (M=1 the direct
# rows with the folded sum and on-the-fly quantisation), the router weight on
# either side. The interpretation of a precision config is parity unpinned
# (triton_kernels is absent); the arithmetic is the oracle's dequantising MoE
# with the bias variant's swiglu.
@pytest.mark.parametrize("mode", ["fp8", "int8"])
@pytest.mark.parametrize("on_input", [False, True], ids=["gammas_out", "gammas_in"])
@pytest.mark.parametrize("sched", _SCHEDS, ids=["decode", "prefill"])
@pytest.mark.parametrize("shape", [(1, 3072, 256, 8, 2), (7, 512, 256, 4, 2),
                                   (300, 1024, 512, 8, 2)])
def test_bias_swiglu_quantised(gpu, shape, sched, on_input, mode):
    M, K, N, E, topk = shape
    wts = testing.make_weights(K, N, E, mode, 0.1, device=gpu, seed=K + N + E + M)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=K + E + M)
    g = torch.Generator(device=gpu).manual_seed(M + 3)
    b1 = torch.randn(E, 2 * N, generator=g, device=gpu) * 0.5
    b2 = torch.randn(E, K, generator=g, device=gpu) * 0.5
    kw = dict(apply_router_weight_on_input=on_input, gemm1_alpha=1.702,
              gemm1_clamp_limit=7.0, _flags=sched)
    if mode == "fp8":
        res = fm.fused_moe_with_bias(x, wts.w1, b1, wts.w2, b2, tw, ti, interleaved=False,
                                     **wts.kwargs(mode), **kw)
    else:
        q = wts.kwargs(mode)
        q["w1_scale"] = _interleave_rows(wts.w1_scale)
        res = fm.fused_moe_with_bias(x, _interleave_rows(wts.w1), _interleave_rows(b1),
                                     wts.w2, b2, tw, ti, **q, **kw)
    toks = _sample(M, 48)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=mode, w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, tokens=toks, return_mag=True,
                            activation="swiglu", b1=b1, b2=b2, alpha=1.702, limit=7.0,
                            apply_router_weight_on_input=on_input)
    _check(res.cpu()[toks], ref, mode, f"bias swiglu {mode} {shape}")


def test_bias_quantised_reference_signature(gpu):
    """int8 weights through triton_kernel_fused_experts_with_bias: the
    reference's layouts, per-column scales from the precision configs'
    ``weight_scale``; fp8 there is rejected (its 128-column scale blocks mix
    interleaved gate and linear columns), and so is fp8 with interleaved rows
    in fused_moe_with_bias."""
    M, K, N, E, topk = 64, 512, 256, 8, 2
    wts = testing.make_weights(K, N, E, "int8", 0.1, device=gpu, seed=17)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=17)
    g = torch.Generator(device=gpu).manual_seed(5)
    b1 = torch.randn(E, 2 * N, generator=g, device=gpu) * 0.5
    b2 = torch.randn(E, K, generator=g, device=gpu) * 0.5
    w1_ref = _interleave_rows(wts.w1).transpose(1, 2).contiguous()
    w2_ref = wts.w2.transpose(1, 2).contiguous()
    pcg1 = _NS(weight_scale=_interleave_rows(wts.w1_scale))
    pcg2 = _NS(weight_scale=wts.w2_scale)
    routing, gather, scatter = flaggems_sglang.standard_topk_to_routing(tw, ti, E)
    res = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        x, w1_ref, pcg1, _interleave_rows(b1), w2_ref, pcg2, b2, routing, gather,
        scatter, gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode="int8", w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, return_mag=True, activation="swiglu",
                            b1=b1, b2=b2, alpha=1.702, limit=7.0)
    _check(res.cpu(), ref, "int8", "bias compat int8")
    f8 = testing.make_weights(K, N, E, "fp8", 0.1, device=gpu, seed=17)
    with pytest.raises(NotImplementedError, match="interleaved"):
        flaggems_sglang.triton_kernel_fused_experts_with_bias(
            x, f8.w1.transpose(1, 2).contiguous(), _NS(weight_scale=f8.w1_scale), b1,
            f8.w2.transpose(1, 2).contiguous(), _NS(weight_scale=f8.w2_scale), b2,
            routing, gather, scatter)
    with pytest.raises(NotImplementedError, match="interleaved"):
        fm.fused_moe_with_bias(x, f8.w1, b1, f8.w2, b2, tw, ti, **f8.kwargs("fp8"))


def test_bias_reference_signature(gpu):
    """triton_kernel_fused_experts_with_bias with the reference's layouts
    (w1 [E, K, 2N] interleaved columns, w2 [E, N, K]) and routing format;
    scatter_indx=None returns the un-combined rows."""
    M, K, N, E, topk = 64, 256, 128, 8, 2
    x, w1, w2, b1, b2, w, ids = _bias_inputs(M, K, N, E, topk, gpu)
    w1_ref = _interleave_rows(w1).transpose(1, 2).contiguous()
    w2_ref = w2.transpose(1, 2).contiguous()
    routing, gather, scatter = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    res = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        x, w1_ref, None, _interleave_rows(b1), w2_ref, None, b2, routing, gather,
        scatter, gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    ref = moe_ref.fused_moe(x, w1, w2, w, ids, return_mag=True, activation="swiglu",
                            b1=b1, b2=b2, alpha=1.702, limit=7.0)
    _check(res.cpu(), ref, "bf16", "bias compat")
    rows = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        x, w1_ref, None, _interleave_rows(b1), w2_ref, None, b2, routing, gather,
        None, gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    assert rows.shape == (M * topk, K)
    _check(rows.cpu(), _per_slot_ref(x, w1, w2, w, ids, ascending=True, activation="swiglu",
                                     b1=b1, b2=b2, alpha=1.702, limit=7.0),
           "bf16", "bias compat uncombined")
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation"):
        flaggems_sglang.triton_kernel_fused_experts_with_bias(
            x, w1_ref, None, b1, w2_ref, None, b2, routing, gather, scatter,
            activation="gelu")


class _NS:
    def __init__(self, **kw):
        self.__dict__.update(kw)


@pytest.mark.parametrize("variant", ["standard", "routing_tuple", "no_combine", "bias"])
def test_fused_moe_flagos_adapter(gpu, variant):
    """The SGLang runner adapter (ops/fused_moe.py:328-422) on native-layout
    layer weights, duck-typed runner config / layer / dispatch output."""
    M, K, N, E, topk = 40, 256, 128, 8, 2
    x, w1, w2, b1, b2, w, ids = _bias_inputs(M, K, N, E, topk, gpu)
    cfg = _NS(num_experts=E, activation="silu", apply_router_weight_on_input=False,
              no_combine=variant == "no_combine", routed_scaling_factor=2.0,
              gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    obj = _NS(runner=_NS(config=cfg))
    layer = _NS(w13_weight=w1, w2_weight=w2)
    if variant == "bias":
        layer = _NS(w13_weight=_interleave_rows(w1), w2_weight=w2,
                    w13_weight_bias=_interleave_rows(b1), w2_weight_bias=b2)
    topk_output = _NS(topk_weights=w, topk_ids=ids)
    if variant == "routing_tuple":
        topk_output = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    out = fm.fused_moe_flagos(obj, layer, _NS(hidden_states=x, topk_output=topk_output))
    res = out.hidden_states
    if variant == "bias":
        ref, mag = moe_ref.fused_moe(x, w1, w2, w, ids, return_mag=True,
                                     activation="swiglu", b1=b1, b2=b2, alpha=1.702,
                                     limit=7.0)
    else:
        ref, mag = moe_ref.fused_moe(x, w1, w2, w, ids, return_mag=True)
    if variant == "no_combine":
        assert res.shape == (M, topk, K)
        _check(res.reshape(M * topk, K).cpu(), _per_slot_ref(x, w1, w2, w, ids), "bf16",
               "flagos no_combine")
    else:
        _check(res.cpu(), ((ref.float() * 2.0).to(torch.bfloat16), mag * 2.0), "bf16",
               f"flagos {variant}")


def test_dropped_slots_and_routed_scaling(gpu):
    x, w1, w2, w, ids = _ref_inputs(16, 256, 128, 4, 2, gpu)
    ids2 = ids.clone()
    ids2[::3, 1] = -1  # slot not routed (e.g. expert owned by another rank)
    res = flaggems_sglang.fused_moe(x, w1, w2, w, ids2, routed_scaling_factor=2.5)
    ref, mag = moe_ref.fused_moe(x, w1, w2, w, ids2, return_mag=True)
    _check(res.cpu(), ((ref.float() * 2.5).to(torch.bfloat16), mag * 2.5), "bf16",
           "dropped+scaled")


def test_deterministic(gpu):
    x, w1, w2, w, ids = _ref_inputs(300, 512, 256, 8, 2, gpu)
    a = flaggems_sglang.fused_moe(x, w1, w2, w, ids)
    for _ in range(2):
        assert torch.equal(flaggems_sglang.fused_moe(x, w1, w2, w, ids), a)


def test_zero_tokens(gpu):
    x, w1, w2, w, ids = _ref_inputs(4, 128, 128, 4, 2, gpu)
    out = flaggems_sglang.fused_moe(x[:0], w1, w2, w[:0], ids[:0])
    assert out.shape == (0, 128)


# ------------------------------------------------ measured configurations ---
_WEIGHTS = {}


def _weights(cfg, device):
    key = cfg.name.replace("_skewed", "")
    if key not in _WEIGHTS:
        _WEIGHTS.clear()
        torch.cuda.empty_cache()
        _WEIGHTS[key] = testing.make_weights(cfg.K, cfg.N, cfg.E, cfg.mode,
                                             cfg.w_scale, device=device)
    return _WEIGHTS[key]


# every M the benchmark reports, for every configuration
CONFIG_CASES = [("small", 64)] + [
    (name, m) for name in ("mixtral", "qwen3", "qwen3_skewed", "qwen2_int8",
                           "deepseek_fp8")
    for m in testing.CONFIGS[name].Ms
]


_QMODE = {"bf16": _capi.QMODE_BF16, "fp8": _capi.QMODE_FP8_BLOCK,
          "int8": _capi.QMODE_INT8_CHANNEL}
_TILE_ROWS = {0: 256, 1: 128, 2: 64, 3: 32, 4: 160}


def _schedule_block(M, cfg):
    """Rows per GEMM row block of the schedule a call of this shape runs."""
    sched = _capi.schedule(M, cfg.K, cfg.N, cfg.E, cfg.topk, _QMODE[cfg.mode])
    if sched.startswith("tiled"):
        return _TILE_ROWS[int(sched.split("cfg=")[1].split()[0])]
    if sched.startswith("stream"):
        return 16 * int(sched.split("mt=")[1].split()[0])
    return None  # one token: no alignment


def block_cover_tokens(topk_ids, E, block):
    """Tokens whose slots hit every half of every row block of the padded
    expert order (the alignment of ``block`` rows; the halves are the
    128-row tiles fp8's GEMM2 runs on 256-row blocks): for each half that
    holds a live row, the token of its last live row -- for an expert's
    last, partly filled block that is the row next to the padding."""
    ids = topk_ids.cpu().numpy()
    numel, topk = ids.size, ids.shape[1]
    s, _, npp = moe_ref.align(ids, E, block)
    half = max(block // 2, 1)
    toks = set()
    for b in range(0, npp, half):
        seg = s[b:b + half]
        live = seg[seg < numel]
        if live.size:
            toks.add(int(live[-1]) // topk)
    return toks


@pytest.mark.parametrize("name,M", CONFIG_CASES, ids=[f"{n}-M{m}" for n, m in CONFIG_CASES])
def test_fused_moe_configs(gpu, name, M):
    cfg = testing.CONFIGS[name]
    wts = _weights(cfg, gpu)
    x, tw, ti = testing.make_tokens(M, cfg.K, cfg.E, cfg.topk, cfg.scoring,
                                    cfg.hot_experts, cfg.hot_bias, device=gpu,
                                    seed=M + cfg.K + cfg.N + cfg.E + cfg.topk)
    res = flaggems_sglang.fused_moe(x, wts.w1, wts.w2, tw, ti, **wts.kwargs(cfg.mode))
    toks = _sample(M, 8 if cfg.mode == "fp8" else 16)
    block = _schedule_block(M, cfg)
    if M == max(cfg.Ms) and block is not None:
        cover = block_cover_tokens(ti, cfg.E, block)
        toks = sorted(set(toks) | cover)
        print(f"{name} M={M}: {len(toks)} tokens cover every half of the "
              f"{block}-row blocks")
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode=cfg.mode,
                            w1_scale=wts.w1_scale, w2_scale=wts.w2_scale,
                            tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, cfg.mode, f"{name} M={M}")


def test_release_config_weights():
    _WEIGHTS.clear()
    torch.cuda.empty_cache()


# -------------------------------------------------------- uncombined rows ---
@pytest.mark.parametrize("M,K,N,E,topk", [(9, 256, 128, 8, 2), (33, 256, 512, 16, 4)])
def test_uncombined_rows_per_slot(gpu, M, K, N, E, topk):
    """``scatter_indx=None`` (the adapter's ``no_combine``) returns one row per
    (token, slot), token-major, a token's slots in ascending expert id (the
    routing tuple's order): row (t, r) is the r-th smallest expert's gated
    output, bf16(w * y). Compared row by row with the oracle run on that one
    slot, so any permutation of the rows fails. matmul_ogs without a scatter
    index would leave rows in expert-sorted order, but the reference then
    views them as [num_tokens, hidden] (ops/fused_moe.py:232), which cannot
    hold M * topk rows: the reference's own order is not observable (parity
    unpinned)."""
    x, w1, w2, w, ids = _ref_inputs(M, K, N, E, topk, gpu)
    w1_ref = w1.transpose(1, 2).contiguous()
    w2_ref = w2.transpose(1, 2).contiguous()
    rd, gi, _ = flaggems_sglang.standard_topk_to_routing(w, ids, E)
    rows = flaggems_sglang.triton_kernel_fused_experts(x, w1_ref, w2_ref, rd, gi, None)
    assert rows.shape == (M * topk, K)
    ref = _per_slot_ref(x, w1, w2, w, ids, ascending=True)
    _check(rows.cpu(), ref, "bf16", f"uncombined rows {(M, K, N, E, topk)}")
    # a swap of two slots' rows is caught
    swapped = rows.view(M, topk, K).flip(1).reshape(M * topk, K).cpu()
    ok, _, _ = moe_ref.compare(swapped, ref[0], 2e-2, 1e-2, ref[1])
    assert not ok


@pytest.mark.parametrize("sched", [_capi.FLAG_FORCE_DECODE, _capi.FLAG_FORCE_PREFILL, 0],
                         ids=["decode", "prefill", "auto"])
def test_int8_wider_than_8192(gpu, sched):
    """int8 w8a8 with an intermediate wider than a wave's quantiser rows
    (N = 9216 > 8192: the GEMM2 input quantiser takes a workgroup per row)."""
    M, K, N, E, topk = 96, 512, 9216, 4, 2
    wts = testing.make_weights(K, N, E, "int8", 0.05, device=gpu, seed=11)
    x, tw, ti = testing.make_tokens(M, K, E, topk, device=gpu, seed=11)
    res = fm.fused_moe(x, wts.w1, wts.w2, tw, ti, _flags=sched, **wts.kwargs("int8"))
    toks = _sample(M, 16)
    ref = moe_ref.fused_moe(x, wts.w1, wts.w2, tw, ti, mode="int8", w1_scale=wts.w1_scale,
                            w2_scale=wts.w2_scale, tokens=toks, return_mag=True)
    _check(res.cpu()[toks], ref, "int8", f"int8 N=9216 sched {sched}")
