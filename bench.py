#!/usr/bin/env python3
"""Fused-MoE benchmark on one MI355X.

A step is one fused-MoE layer call (alignment, GEMM1 + silu, GEMM2 + top-k
weight, top-k sum) on the Mixtral-8x7B-shaped bf16 layer at M=4096 tokens,
with every input already resident in HBM. Prints ONE JSON line:

* ``value``: TFLOP/s of the whole layer at M=4096 (FLOPs = 6*M*topk*K*N),
  ``ms_per_step`` = ms/layer;
* ``roofline``: the dominant kernel (largest stage time, measured with HIP
  events the library records around each stage on the launch stream, over
  the timed calls) against MI355X's peak, with the HBM bytes per launch
  rocprofv3 counted (``traffic``, ``profiles/traffic_<cfg>.json``) and the
  MFMA-busy fraction (``profiles/mfma_<cfg>.json``);
* ``cpu_baseline``: the repo's CPU torch reference (oracle/) on a bounded
  sample of the headline layer, on this host's cores;
* ``rows``: one compact row per (configuration, M) -- field names in
  ``row_fields`` -- for every configuration of
  flaggems_sglang.testing.CONFIGS: ms/layer, TFLOP/s, GB/s, both roofline
  fractions, the dominant GEMM with its own fraction, counter traffic and
  MFMA busy where profiled, the CPU oracle's time on a token sample of the
  same inputs, the parity of that sample against the GPU output (max abs,
  mean rel, within tolerance) and whether the alignment of that routing is
  bit-exact. ``ref_bench`` is the reference's own benchmark
  (benchmark/test_fused_moe.py:53-73): ``triton_kernel_fused_experts`` on the
  routing tuple at (M, 1280, 3072, 64, 8), with ``fused_moe`` on the same
  inputs timed beside it (``ref_fields``).

Options: ``--config`` picks another headline configuration (its largest M
unless ``--m``), ``--no-sweep`` / ``--no-configs`` / ``--no-cpu`` skip those
legs (profiling runs).
"""

import argparse
import json
import os
import statistics
import sys
import time

# the CPU oracle's worker threads sleep as soon as a parallel region ends,
# so they never compete with the host thread that launches the timed calls
os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "flaggems-sglang_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = ("fused-MoE ms/layer, TFLOP/s & HBM GB/s (% roofline) at M=1..4096, "
          "1 GPU")
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 5000.0, "int8": 5000.0}
FLUSH_BYTES = 512 << 20  # > MALL (256 MB): flush between steps when small
SPIN_CYCLES = 400_000    # ~0.2 ms of GPU spin ahead of each flushed call
OTHER_CONFIGS = ("ref_bench", "deepseek_fp8", "qwen3", "qwen3_skewed", "qwen2_int8",
                 "small")
ROW_FIELDS = ("M", "ms", "tflops", "gbs", "frac_hbm", "frac_mfma", "dom", "dom_frac",
              "traffic", "mfma_busy", "cpu_ms", "cpu_tokens", "max_abs", "mean_rel",
              "parity", "align_bitexact")
# ref_bench rows: the reference-signature call, then fused_moe on the same inputs
REF_FIELDS = ROW_FIELDS + ("ms_fused_moe", "sig_over_fused_moe")
CPU_SAMPLE = 4  # tokens the per-row CPU oracle runs on
# untimed calls ahead of each row: the first tens of calls after a new
# weight set run a few % slow (measured: 30 flushed one-token calls 0.0516
# ms, the next 30 0.0477)
SWEEP_WARMUP = 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="mixtral")
    ap.add_argument("--m", type=int, default=None, help="headline M")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the sweep over the other configurations")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sweep-steps", type=int, default=10)
    ap.add_argument("--flags", type=lambda v: int(v, 0), default=0,
                    help="schedule flags passed to the op (FGS_FLAG_* of "
                         "include/fgs_moe.h; a tuning aid)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (the reference "
                         "kernel for scaling FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--summarize", nargs="+", metavar=("DIR", "CFG:M"),
                    help="no GPU work: turn the rocprofv3 CSV output under DIR "
                         "into profiles/moe_kernels_<cfg>_m<M>.md, "
                         "traffic_<cfg>.json and mfma_<cfg>.json")
    return ap.parse_args()


def calibrate_copy():
    """A plain device-to-device copy of known size: its FETCH_SIZE and
    WRITE_SIZE readings give the counter-to-byte factor for the traffic
    figures (read 1 GiB, write 1 GiB per launch)."""
    import torch

    n = 1 << 30
    src = torch.ones(n // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "torch copy_", "bytes_read": n,
                      "bytes_written": n, "launches": 3}), flush=True)


def make_config_weights(cfg, dev):
    """The configuration's weights. ref_bench keeps the reference's layout
    (w1 [E, K, 2N], w2 [E, N, K], randn * 0.1, as its benchmark builds them);
    the others the SGLang layout of flaggems_sglang.testing.make_weights."""
    import torch

    from flaggems_sglang import testing

    if cfg.name != "ref_bench":
        return testing.make_weights(cfg.K, cfg.N, cfg.E, cfg.mode, cfg.w_scale, device=dev)
    g = torch.Generator(device=dev).manual_seed(cfg.K + cfg.N + cfg.E)
    w1 = torch.empty((cfg.E, cfg.K, 2 * cfg.N), dtype=torch.bfloat16, device=dev)
    w2 = torch.empty((cfg.E, cfg.N, cfg.K), dtype=torch.bfloat16, device=dev)
    for e in range(cfg.E):
        w1[e] = (torch.randn((cfg.K, 2 * cfg.N), generator=g, device=dev) *
                 cfg.w_scale).to(torch.bfloat16)
        w2[e] = (torch.randn((cfg.N, cfg.K), generator=g, device=dev) *
                 cfg.w_scale).to(torch.bfloat16)
    return testing.MoEWeights(w1, w2)


class Layer:
    """One configuration's weights plus a token batch, ready to call.

    ``ref_sig``: the call is the reference's entry point,
    ``triton_kernel_fused_experts(x, w1, w2, routing_data, gather_indx,
    scatter_indx)`` on reference-layout weights with the routing tuple built
    (untimed) by standard_topk_to_routing, as the reference's benchmark
    builds it (benchmark/test_fused_moe.py:26-50)."""

    def __init__(self, cfg, weights, M, device, flags=0, ref_sig=False):
        import flaggems_sglang
        from flaggems_sglang import testing

        self.cfg, self.w, self.M, self.flags, self.ref_sig = cfg, weights, M, flags, ref_sig
        self.x, self.tw, self.ti = testing.make_tokens(
            M, cfg.K, cfg.E, cfg.topk, cfg.scoring, cfg.hot_experts,
            cfg.hot_bias, device=device, seed=M + cfg.K + cfg.N + cfg.E + cfg.topk)
        self.kw = weights.kwargs(cfg.mode)
        self.flops = testing.layer_flops(M, cfg)
        self.bytes = testing.layer_bytes(M, cfg.K, cfg.N, cfg.topk, cfg.mode,
                                         self.ti, cfg.E)
        self.touched = int(self.ti.unique().numel())
        if ref_sig:
            self.routing = flaggems_sglang.standard_topk_to_routing(self.tw, self.ti, cfg.E)

    def native_weights(self):
        """w1 [E, 2N, K], w2 [E, K, N]: for ref_bench the contiguous copies
        the reference-signature entry converts once and caches."""
        if self.cfg.name == "ref_bench":
            from flaggems_sglang.ops import fused_moe as fm

            return fm._native_layout(self.w.w1), fm._native_layout(self.w.w2)
        return self.w.w1, self.w.w2

    def __call__(self):
        import flaggems_sglang

        if self.ref_sig:
            return flaggems_sglang.triton_kernel_fused_experts(
                self.x, self.w.w1, self.w.w2, *self.routing)
        w1, w2 = self.native_weights()
        return flaggems_sglang.fused_moe(self.x, w1, w2, self.tw, self.ti,
                                         _flags=self.flags, **self.kw)


def time_layer(layer, steps, warmup, flush, profile_timed=False):
    """Times `steps` calls (after `warmup`), returns (ms/call, stage ms).

    With `profile_timed` the library's events around GEMM1 (profile mode 3:
    the two boundaries of stage 2) are recorded during the timed calls
    themselves (the headline: its roofline comes from the same launches it
    times; each event costs the call ~12 us, so only GEMM1's two are
    recorded there), and a second, untimed pass with every stage boundary
    gives the other stages.
    Otherwise the timed calls run with the profiler off and that second pass
    gives the whole per-stage split (the sweep).
    """
    import ctypes

    import torch

    from flaggems_sglang import _capi

    lib = _capi.load()
    scratch = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda") if flush else None
    for _ in range(warmup):
        layer()
    torch.cuda.synchronize()

    def run(n, profile):
        total = 0.0
        lib.fgs_moe_profile_enable(profile)
        if flush:
            # cold weights each step: a 512 MiB write evicts L2 and MALL;
            # only the layer call itself is inside the events. A short GPU
            # spin after the flush keeps the device busy while the host
            # enqueues the call, so host launch time never shows up as an
            # idle gap between the events.
            for _ in range(n):
                scratch.fill_(1)
                if hasattr(torch.cuda, "_sleep"):
                    torch.cuda._sleep(SPIN_CYCLES)
                a = torch.cuda.Event(enable_timing=True)
                b = torch.cuda.Event(enable_timing=True)
                a.record()
                layer()
                b.record()
                torch.cuda.synchronize()
                total += a.elapsed_time(b)
        else:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(n):
                layer()
            torch.cuda.synchronize()
            total = (time.perf_counter() - t0) * 1e3
        lib.fgs_moe_profile_enable(0)
        return total / n

    stage = (ctypes.c_float * 6)()
    lib.fgs_moe_profile_read(stage, 6)  # drop anything recorded before
    ms = run(steps, 3 if profile_timed else 0)
    timed = {}
    if profile_timed and lib.fgs_moe_profile_read(stage, 6) > 0:
        timed = {"gemm1": float(stage[2])}
    run(max(3, min(steps, 10)), 1)
    n = lib.fgs_moe_profile_read(stage, 6)
    stages = dict(zip(_capi.PROFILE_STAGES, [float(v) for v in stage])) if n > 0 else {}
    stages.update(timed)  # GEMM1: from the timed calls
    return ms, stages


def _profile_entry(kind, cfg_name, M, stage):
    """A stage's entry in a committed rocprofv3 summary
    (profiles/<kind>_<cfg>.json, keyed "<cfg>:<M>:<stage>"), or None."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{cfg_name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("by_stage", {}).get(f"{cfg_name}:{M}:{stage}") or None


def dominant(layer, stages):
    """Roofline object for the slowest stage (a GEMM in every config):
    achieved rate of its algorithmic FLOPs or bytes per launch over its
    event-measured average, the peak, and -- where a committed rocprofv3
    summary covers the shape -- the counted HBM bytes per launch and the
    MFMA-busy fraction."""
    cfg = layer.cfg
    name = max(("gemm1", "gemm2"), key=lambda s: stages.get(s, 0.0))
    t = stages[name] * 1e-3
    M, k, K, N = layer.M, cfg.topk, cfg.K, cfg.N
    bw = 2 if cfg.mode == "bf16" else 1
    if name == "gemm1":
        flops = 4.0 * M * k * K * N
        wbytes = layer.touched * 2 * N * K * bw
        io = M * K * bw + M * k * N * 2
    else:
        flops = 2.0 * M * k * K * N
        wbytes = layer.touched * K * N * bw
        io = M * k * N * bw + M * k * K * 2
    alg = wbytes + io
    tflops = flops / t / 1e12
    gbs = alg / t / 1e9
    frac_mfma = tflops / PEAK_TFLOPS[cfg.mode]
    frac_hbm = gbs / PEAK_HBM_GBS
    meas = _profile_entry("traffic", cfg.name, M, name)
    traffic = None if meas is None else round(meas["fetch_bytes"] + meas["write_bytes"])
    mf = _profile_entry("mfma", cfg.name, M, name)
    mfma = frac_mfma >= frac_hbm
    return {"kernel": f"moe_gemm ({name})", "stage": name,
            "bound": "mfma" if mfma else "hbm",
            "achieved": round(tflops if mfma else gbs, 2),
            "peak": PEAK_TFLOPS[cfg.mode] if mfma else PEAK_HBM_GBS,
            "unit": "TFLOP/s" if mfma else "GB/s",
            "frac": round(frac_mfma if mfma else frac_hbm, 4),
            "traffic": traffic, "algorithmic_bytes": round(alg),
            "traffic_ratio": None if traffic is None else round(traffic / alg, 3),
            "mfma_busy": None if mf is None else round(mf["mfma_busy"], 4),
            "avg_ms": round(stages[name], 4)}


def _sample_tokens(M, n=CPU_SAMPLE):
    return sorted({0, M // 3, (2 * M) // 3, M - 1})[:n] if M > n else list(range(M))


def cpu_check(layer, out, cpu_w):
    """The CPU oracle on a token sample of the row's own inputs: its time,
    and its parity against the GPU output of the same call. Returns
    (cpu_ms, tokens, max_abs, mean_rel, ok)."""
    from flaggems_sglang import testing
    from oracle import moe_ref

    cfg = layer.cfg
    toks = _sample_tokens(layer.M)
    x, tw, ti = layer.x.cpu(), layer.tw.cpu(), layer.ti.cpu()
    t0 = time.perf_counter()
    ref, mag = moe_ref.fused_moe(x, cpu_w.w1, cpu_w.w2, tw, ti, mode=cfg.mode,
                                 w1_scale=cpu_w.w1_scale, w2_scale=cpu_w.w2_scale,
                                 tokens=toks, return_mag=True)
    dt = (time.perf_counter() - t0) * 1e3
    tol = testing.TOL[cfg.mode]
    ok, max_abs, mean_rel = moe_ref.compare(out.cpu()[toks], ref, tol["atol"], tol["rtol"],
                                            mag)
    ok = ok and mean_rel <= tol["mean_rel"]
    return dt, len(toks), max_abs, mean_rel, ok


def align_check(layer):
    """moe_align_block_size (HIP) on the row's routing against the oracle's
    C restatement, at the block size the call's schedule uses: bit-exact?"""
    import flaggems_sglang
    from flaggems_sglang import _capi
    from oracle import moe_ref

    cfg = layer.cfg
    qm = {"bf16": _capi.QMODE_BF16, "fp8": _capi.QMODE_FP8_BLOCK,
          "int8": _capi.QMODE_INT8_CHANNEL}[cfg.mode]
    sched = _capi.schedule(layer.M, cfg.K, cfg.N, cfg.E, cfg.topk, qm)
    block = 16
    if sched.startswith("tiled"):
        block = {0: 256, 1: 128, 2: 64, 3: 32, 4: 160}[int(sched.split("cfg=")[1].split()[0])]
    elif sched.startswith("stream"):
        block = 16 * int(sched.split("mt=")[1].split()[0])
    s, e, npp = flaggems_sglang.moe_align_block_size(layer.ti, cfg.E, block)
    rs, re_, rnpp = moe_ref.align(layer.ti.cpu().numpy(), cfg.E, block)
    n = int(npp.item())
    return (n == rnpp and bool((s.cpu().numpy() == rs).all())
            and bool((e.cpu().numpy() == re_).all()))


def rates(layer, ms):
    """ms/layer and the layer's TFLOP/s, GB/s and roofline fractions."""
    t = ms * 1e-3
    tflops = layer.flops / t / 1e12
    gbs = layer.bytes / t / 1e9
    return {"M": layer.M, "ms": round(ms, 4), "tflops": round(tflops, 2),
            "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "frac_mfma": round(tflops / PEAK_TFLOPS[layer.cfg.mode], 4)}


def measure_row(layer, args):
    """GPU part of one row of ROW_FIELDS (timing with the profiler off, the
    stage split from a second pass, the output of one more call for the
    parity check, the alignment check). Returns (row, stages, output)."""
    flush = layer.bytes < FLUSH_BYTES
    ms, stages = time_layer(layer, args.sweep_steps, SWEEP_WARMUP, flush)
    dom = dominant(layer, stages)
    row = {**rates(layer, ms),
           "dom": dom["stage"], "dom_frac": dom["frac"], "traffic": dom["traffic"],
           "mfma_busy": dom["mfma_busy"], "cpu_ms": None, "cpu_tokens": None,
           "max_abs": None, "mean_rel": None, "parity": None,
           "align_bitexact": align_check(layer)}
    return row, stages, layer().cpu()


def cpu_row(row, layer, out, cpu_w):
    """CPU part of a row: the oracle's time and parity on the token sample."""
    cms, n, max_abs, mean_rel, ok = cpu_check(layer, out, cpu_w)
    row.update(cpu_ms=round(cms, 1), cpu_tokens=n, max_abs=round(max_abs, 5),
               mean_rel=float(f"{mean_rel:.3g}"), parity=ok)


def host_weights(cfg, weights):
    """The configuration's weights on the host for the CPU oracle (bf16
    weights as fp32 once, so the oracle's per-expert conversion is free;
    fp8 / int8 stay quantised: the oracle dequantises the experts it
    touches)."""
    from flaggems_sglang import testing

    w1, w2 = weights.w1, weights.w2
    if cfg.name == "ref_bench":
        w1, w2 = w1.transpose(1, 2), w2.transpose(1, 2)
    if cfg.mode == "bf16":
        return testing.MoEWeights(w1.cpu().float(), w2.cpu().float())
    return testing.MoEWeights(w1.cpu(), w2.cpu(), weights.w1_scale.cpu(),
                              weights.w2_scale.cpu())


def sweep_config(cfg, dev, args, weights=None, cpu_w=None, before_cpu=None):
    """Rows of one configuration at each of its M (compact lists in
    ROW_FIELDS / REF_FIELDS order); its weights are freed after.
    `before_cpu` runs between the GPU rows and the CPU oracle's rows."""
    import torch

    t0 = time.perf_counter()
    own = weights is None
    if own:
        weights = make_config_weights(cfg, dev)
        torch.cuda.synchronize()
    log(f"{cfg.name}: weights {weights.nbytes() / 1e9:.2f} GB in "
        f"{time.perf_counter() - t0:.1f}s")
    # every GPU measurement of the configuration first, then the CPU oracle
    rows, done = [], []
    for m in cfg.Ms:
        ref_sig = cfg.name == "ref_bench"
        lay = Layer(cfg, weights, m, dev, args.flags, ref_sig=ref_sig)
        if ref_sig:
            # both paths warm before either is timed
            for sig in (False, True):
                lay.ref_sig = sig
                for _ in range(SWEEP_WARMUP):
                    lay()
        r, st, out = measure_row(lay, args)
        if ref_sig:
            # the same inputs through fused_moe, alternating with the
            # reference-signature call three times each (medians), so a
            # drift of the device state between passes favours neither
            flush = lay.bytes < FLUSH_BYTES
            t_sig, t_nat = [r["ms"]], []
            for sig in (False, True, False, True, False):
                lay.ref_sig = sig
                (t_sig if sig else t_nat).append(
                    time_layer(lay, args.sweep_steps, SWEEP_WARMUP, flush)[0])
            ms_s, ms_n = statistics.median(t_sig), statistics.median(t_nat)
            r.update(**rates(lay, ms_s), ms_fused_moe=round(ms_n, 4),
                     sig_over_fused_moe=round(ms_s / ms_n, 4))
        log(f"{cfg.name} M={m}: {json.dumps(r)} stages={json.dumps(st)}")
        done.append((r, lay, out))
    if before_cpu is not None:
        before_cpu()
    if not args.no_cpu:
        if cpu_w is None:
            cpu_w = host_weights(cfg, weights)
        for r, lay, out in done:
            cpu_row(r, lay, out, cpu_w)
            log(f"{cfg.name} M={lay.M} cpu: {r['cpu_ms']} ms on {r['cpu_tokens']} tokens, "
                f"max_abs={r['max_abs']} mean_rel={r['mean_rel']} parity={r['parity']}")
    fields = REF_FIELDS if cfg.name == "ref_bench" else ROW_FIELDS
    rows = [[r[f] for f in fields] for r, _, _ in done]
    if own:
        del weights
    done = None
    torch.cuda.empty_cache()
    return rows


def cpu_baseline(layer, cpu_w, budget_s=25.0):
    """The repo's CPU torch reference (oracle/) on a bounded token sample of
    the headline layer, on every core this process may use: the median of
    three runs (one when a run takes more than a third of the budget)."""
    import torch

    from oracle import moe_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = layer.cfg
    x, tw, ti = layer.x.cpu(), layer.tw.cpu(), layer.ti.cpu()
    n = min(layer.M, 512)
    toks = list(range(n))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        moe_ref.fused_moe(x, cpu_w.w1, cpu_w.w2, tw, ti, mode=cfg.mode,
                          w1_scale=cpu_w.w1_scale, w2_scale=cpu_w.w2_scale, tokens=toks)
        times.append(time.perf_counter() - t0)
        if times[0] * 3 > budget_s:
            break
    dt = statistics.median(times)
    flops = 6.0 * n * cfg.topk * cfg.K * cfg.N
    return {"value": round(flops / dt / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "ms_per_layer_sample": round(dt * 1e3, 1),
            "sample": f"oracle.moe_ref.fused_moe (torch fp32 on CPU) on the first "
                      f"{n} of {layer.M} tokens of the same {cfg.name} layer, "
                      f"median of {len(times)}"}


# ---------------------------------------------------------------------------
# rocprofv3 output -> committed summaries (no GPU work; run after the passes)

PROFILE_TITLES = {
    "mixtral": "Mixtral-8x7B-shaped bf16 layer",
    "deepseek_fp8": "DeepSeek-V3-shaped fp8 (128x128 block scales) layer",
    "qwen3": "Qwen3-30B-A3B-shaped bf16 layer",
    "qwen3_skewed": "Qwen3-30B-A3B-shaped bf16 layer, skewed routing",
    "qwen2_int8": "Qwen2-57B-A14B-shaped int8 (per-channel) layer",
    "small": "small bf16 layer",
}
STAGE_ORDER = ("align", "quant_x", "gemm1", "quant_a2", "gemm2", "moe_sum")
MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_VALU",
                 "SQ_INSTS_MFMA", "GRBM_GUI_ACTIVE")
N_XCD, N_CU, N_SIMD = 8, 256, 1024


def _template_args(name):
    """Top-level template arguments of a demangled kernel name."""
    inner = name[name.index("<") + 1:]
    depth, args, cur = 0, [], ""
    for ch in inner:
        if ch == "<":
            depth += 1
        elif ch == ">":
            if depth == 0:
                args.append(cur.strip())
                break
            depth -= 1
        elif ch == "," and depth == 0:
            args.append(cur.strip())
            cur = ""
            continue
        cur += ch
    return args


def _kernel_stage(name, after_gemm1):
    """The layer stage a library kernel belongs to (None: not a layer kernel,
    e.g. the flush fill). Quantiser launches before GEMM1 in a call quantise
    x, after it the GEMM1 output."""
    if "fgs::" not in name:
        return None
    if "align" in name or "routing_order" in name:  # the routing tuple's padded order
        return "align"
    if "wide_plan" in name:  # the 4-wave kernel's tile plan, ahead of its GEMM
        return "gemm2" if after_gemm1 else "gemm1"
    if "quant_" in name:
        return "quant_a2" if after_gemm1 else "quant_x"
    if "scale_gather" in name:  # x's scales into the padded row order
        return "quant_x"
    if "gemm2_direct" in name or "tail_fixup" in name:
        return "gemm2"
    if "moe_gemm" in name:
        args = _template_args(name)
        if "gemm_stream" in name:
            g1 = args[3] == "true"
        elif "gemm_wide" in name:
            g1 = args[1] == "true"
        else:
            g1 = args[-1] == "true"
        return "gemm1" if g1 else "gemm2"
    if "moe_sum" in name:
        return "moe_sum"
    if "silu" in name:
        return "silu"
    return None


def _csv_rows(src, sub, kind):
    import csv
    import glob

    files = glob.glob(os.path.join(src, sub, "**", f"*{kind}.csv"), recursive=True)
    if not files:
        return None
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _dispatches(rows, counters=False):
    """[(stage, kernel, value)] in dispatch order; value = duration in ns, or
    {counter: value} for a counter-collection CSV."""
    per = {}
    for r in rows:
        d = per.setdefault(int(r["Dispatch_Id"]), {"name": r["Kernel_Name"]})
        if counters:
            d.setdefault("c", {})[r["Counter_Name"]] = float(r["Counter_Value"])
        else:
            d["v"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    out, after_gemm1 = [], False
    for _, d in sorted(per.items()):
        st = _kernel_stage(d["name"], after_gemm1)
        if st is None:
            continue
        if st in ("align", "gemm2", "moe_sum"):
            after_gemm1 = False  # the next quantiser belongs to the next call
        elif st == "gemm1":
            after_gemm1 = True
        out.append((st, d["name"], d["c"] if counters else d["v"]))
    return out


def _merge_json(path, calibration, entries):
    data = {"by_stage": {}}
    if os.path.exists(path):
        with open(path) as f:
            data = json.load(f)
    if calibration is not None:
        data["calibration"] = calibration
    data.setdefault("by_stage", {}).update(entries)
    data["by_stage"] = dict(sorted(data["by_stage"].items()))
    with open(path, "w") as f:
        json.dump(data, f, indent=1)
        f.write("\n")


def summarize(src, specs, warmup=3):
    """Writes the committed summaries for each CFG:M from the rocprofv3 runs
    under `src`: <cfg>_m<M>_kt (kernel trace), <cfg>_m<M>_FETCH_SIZE /
    _WRITE_SIZE (HBM bytes), <cfg>_m<M>_mfma (MFMA_COUNTERS) and
    cal_FETCH_SIZE / cal_WRITE_SIZE (the 1 GiB copy of --calibrate-copy).
    Each kernel's first `warmup` trace dispatches are dropped."""
    import statistics
    from collections import OrderedDict, defaultdict

    mean = statistics.mean
    cal = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = _csv_rows(src, f"cal_{c}", "counter_collection")
        if rows:
            vals = [float(r["Counter_Value"]) for r in rows
                    if "copyBuffer" in r["Kernel_Name"]]
            cal[c] = mean(vals)
    calibration = None
    if len(cal) == 2:
        calibration = {
            "kernel": "__amd_rocclr_copyBuffer (torch copy_ of 1 GiB)",
            "FETCH_SIZE_KiB": cal["FETCH_SIZE"], "WRITE_SIZE_KiB": cal["WRITE_SIZE"],
            "fetch_factor": (1 << 30) / (cal["FETCH_SIZE"] * 1024),
            "write_factor": (1 << 30) / (cal["WRITE_SIZE"] * 1024)}
    for spec in specs:
        cfg, m = spec.split(":")
        base = f"{cfg}_m{m}"
        kt_rows = _csv_rows(src, base + "_kt", "kernel_trace")
        if kt_rows is None:
            raise SystemExit(f"no kernel trace under {src}/{base}_kt")
        agg = OrderedDict()
        for st, n, v in _dispatches(kt_rows):
            agg.setdefault((st, n), []).append(v)
        for k in agg:
            if len(agg[k]) > warmup:
                agg[k] = agg[k][warmup:]
        keys = sorted(agg, key=lambda k: STAGE_ORDER.index(k[0])
                      if k[0] in STAGE_ORDER else 99)
        tot = sum(sum(v) for v in agg.values())
        bench_kt = (f"python3 bench.py --config {cfg} --m {m} --steps 20 "
                    f"--warmup {warmup} --no-sweep --no-cpu")
        bench_pmc = (f"python3 bench.py --config {cfg} --m {m} --steps 3 "
                     f"--warmup 1 --no-sweep --no-cpu")
        lines = [
            f"# fused-MoE kernels, {PROFILE_TITLES.get(cfg, cfg)}, M={m}", "",
            "Kernel time (rocprofv3 kernel trace of the bench run; each kernel's",
            f"first {warmup} dispatches, the warmup, are left out, leaving the timed",
            "calls and the calls of the untimed stage-split pass; a quantiser before",
            "GEMM1 quantises x, one after it the GEMM1 output). Made by",
            "", f"    rocprofv3 --kernel-trace --stats -f csv -d <dir>/{base}_kt -o run -- {bench_kt}",
            f"    python3 bench.py --summarize <dir> {cfg}:{m}", "",
            "| stage | kernel | calls | avg us | min us | max us | % of GPU time |",
            "|---|---|---|---|---|---|---|"]
        for k in keys:
            v = agg[k]
            lines.append(f"| {k[0]} | `{k[1][:110]}` | {len(v)} | {mean(v) / 1e3:.1f} | "
                         f"{min(v) / 1e3:.1f} | {max(v) / 1e3:.1f} | "
                         f"{100 * sum(v) / tot:.1f} |")
        # per-call stage sums of the kernel trace (several kernels per stage)
        stage_ns = defaultdict(float)
        for k in keys:
            stage_ns[k[0]] += mean(agg[k])

        def by_kernel(sub):
            rows = _csv_rows(src, sub, "counter_collection")
            if rows is None:
                return None
            d = defaultdict(list)
            for st, n, c in _dispatches(rows, counters=True):
                d[(st, n)].append(c)
            return d

        fe, wr = by_kernel(base + "_FETCH_SIZE"), by_kernel(base + "_WRITE_SIZE")
        traffic = {}
        if fe is not None and wr is not None and calibration is not None:
            ff, wf = calibration["fetch_factor"], calibration["write_factor"]
            lines += [
                "", "HBM traffic per dispatch (two counter passes, each scaled by the same",
                "counter's reading for a plain 1 GiB device copy):", "",
                f"    rocprofv3 --pmc FETCH_SIZE -f csv -d <dir>/{base}_FETCH_SIZE -o run -- {bench_pmc}",
                f"    rocprofv3 --pmc WRITE_SIZE -f csv -d <dir>/{base}_WRITE_SIZE -o run -- {bench_pmc}",
                "    rocprofv3 --pmc FETCH_SIZE -f csv -d <dir>/cal_FETCH_SIZE -o run -- "
                "python3 bench.py --calibrate-copy   (and WRITE_SIZE)", "",
                f"Copy calibration: FETCH_SIZE reads {cal['FETCH_SIZE']:.0f} KiB and WRITE_SIZE "
                f"{cal['WRITE_SIZE']:.0f} KiB for 1 GiB",
                f"read + 1 GiB written, so fetch bytes = FETCH_SIZE x 1024 x {ff:.3f} and "
                f"write bytes = WRITE_SIZE x 1024 x {wf:.3f}.", "",
                "| stage | kernel | fetch MB | write MB | avg us | fetch+write GB/s |",
                "|---|---|---|---|---|---|"]
            for k in keys:
                f = mean(c["FETCH_SIZE"] for c in fe[k]) * 1024 * ff if fe.get(k) else 0.0
                w = mean(c["WRITE_SIZE"] for c in wr[k]) * 1024 * wf if wr.get(k) else 0.0
                avg = mean(agg[k])
                lines.append(f"| {k[0]} | `{k[1][:110]}` | {f / 1e6:.1f} | {w / 1e6:.1f} | "
                             f"{avg / 1e3:.1f} | {(f + w) / avg:.0f} |")
                e = traffic.setdefault(f"{cfg}:{m}:{k[0]}", {
                    "kernel": k[1], "avg_ns": 0.0, "fetch_bytes": 0.0, "write_bytes": 0.0})
                if e["kernel"] != k[1]:
                    e["kernel"] += " + " + k[1]
                e["avg_ns"] += avg
                e["fetch_bytes"] += f
                e["write_bytes"] += w
            _merge_json(os.path.join(ROOT, "profiles", f"traffic_{cfg}.json"),
                        calibration, traffic)
        mf = by_kernel(base + "_mfma")
        if mf is not None:
            lines += [
                "", "MFMA utilisation per dispatch (one counter pass):", "",
                f"    rocprofv3 --pmc {' '.join(MFMA_COUNTERS)} -f csv -d <dir>/{base}_mfma "
                f"-o run -- {bench_pmc}", "",
                "mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs):",
                "the fraction of SIMD cycles the matrix pipe is busy (GRBM_GUI_ACTIVE reads",
                "as the sum of the 8 XCDs' active cycles; SQ_VALU_MFMA_BUSY_CYCLES sums the",
                "SIMDs). cu_busy = SQ_BUSY_CU_CYCLES / (GRBM_GUI_ACTIVE / 8 x 256 CUs).",
                "valu_per_mfma = (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA (SQ_INSTS_VALU",
                "counts the MFMA instructions too).", "",
                "| stage | kernel | mfma_busy | cu_busy | valu_per_mfma | MFMA insts | GRBM_GUI_ACTIVE |",
                "|---|---|---|---|---|---|---|"]
            stage_c = {}
            for k in keys:
                if not mf.get(k):
                    continue
                c = {n: mean(d.get(n, 0.0) for d in mf[k]) for n in MFMA_COUNTERS}
                acc = stage_c.setdefault(k[0], dict.fromkeys(MFMA_COUNTERS, 0.0))
                for n in MFMA_COUNTERS:
                    acc[n] += c[n]
                acc.setdefault("kernels", []).append(k[1])
                simd = c["GRBM_GUI_ACTIVE"] / N_XCD * N_SIMD
                busy = c["SQ_VALU_MFMA_BUSY_CYCLES"] / simd if simd else 0.0
                cu = c["SQ_BUSY_CU_CYCLES"] / (c["GRBM_GUI_ACTIVE"] / N_XCD * N_CU) if simd else 0.0
                vpm = ((c["SQ_INSTS_VALU"] - c["SQ_INSTS_MFMA"]) / c["SQ_INSTS_MFMA"]
                       if c["SQ_INSTS_MFMA"] else None)
                lines.append(f"| {k[0]} | `{k[1][:110]}` | {busy:.3f} | {cu:.3f} | "
                             f"{'-' if vpm is None else f'{vpm:.2f}'} | "
                             f"{c['SQ_INSTS_MFMA']:.4g} | {c['GRBM_GUI_ACTIVE']:.4g} |")
            entries = {}
            for st, acc in stage_c.items():
                if not acc["SQ_INSTS_MFMA"]:
                    continue
                simd = acc["GRBM_GUI_ACTIVE"] / N_XCD * N_SIMD
                entries[f"{cfg}:{m}:{st}"] = {
                    "kernel": " + ".join(acc["kernels"]),
                    "avg_ns": stage_ns[st],
                    "mfma_busy": acc["SQ_VALU_MFMA_BUSY_CYCLES"] / simd,
                    "cu_busy": acc["SQ_BUSY_CU_CYCLES"] / (simd / 4),
                    "valu_per_mfma": (acc["SQ_INSTS_VALU"] - acc["SQ_INSTS_MFMA"])
                    / acc["SQ_INSTS_MFMA"],
                    "counters": {n: acc[n] for n in MFMA_COUNTERS}}
            _merge_json(os.path.join(ROOT, "profiles", f"mfma_{cfg}.json"), None, entries)
        with open(os.path.join(ROOT, "profiles", f"moe_kernels_{cfg}_m{m}.md"), "w") as f:
            f.write("\n".join(lines) + "\n")
        log(f"summarized {cfg} M={m}")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the fused-MoE path has no "
              f"multi-GPU part here); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.summarize:
        summarize(args.summarize[0], args.summarize[1:])
        return
    import torch

    from flaggems_sglang import _capi, testing

    _capi.load()
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"device: {props.name} CUs={props.multi_processor_count} "
        f"mem={props.total_memory / 2**30:.0f} GiB")
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = testing.CONFIGS[args.config]
    M = args.m or max(cfg.Ms)
    t0 = time.perf_counter()
    weights = make_config_weights(cfg, dev)
    torch.cuda.synchronize()
    log(f"weights {weights.nbytes() / 1e9:.2f} GB in {time.perf_counter() - t0:.1f}s")

    head = Layer(cfg, weights, M, dev, args.flags, ref_sig=cfg.name == "ref_bench")
    small_ws = head.bytes < FLUSH_BYTES
    timed = {}

    def time_headline():
        timed["ms"], timed["stages"] = time_layer(head, args.steps, args.warmup,
                                                  flush=small_ws, profile_timed=True)
        log(f"headline {cfg.name} M={M}: {timed['ms']:.4f} ms/layer "
            f"stages={timed['stages']}")

    # The headline is timed right after its configuration's GPU sweep rows
    # (before their CPU oracle rows), i.e. on a device in its steady state:
    # timed right after the weights are made, with 5 warmup calls, the same
    # layer measured ~1.8 % slower (2.649 vs 2.602 ms with 50 warmup calls).
    rows = {}
    cpu_w = None if args.no_cpu else host_weights(cfg, weights)
    if not args.no_sweep:
        rows[cfg.name] = sweep_config(cfg, dev, args, weights, cpu_w,
                                      before_cpu=time_headline)
    else:
        time_headline()
    ms, stages = timed["ms"], timed["stages"]
    roof = dominant(head, stages)
    cpu = None
    if cpu_w is not None:
        cpu = cpu_baseline(head, cpu_w)
        log(f"cpu baseline: {cpu}")
    cpu_w = None
    tflops = head.flops / (ms * 1e-3) / 1e12
    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.mode,
        "data": "synthetic (seeded randn activations, randn*0.02 weights, "
                "softmax/sigmoid top-k routing)",
        "config": {"workload": f"{cfg.name} fused-MoE layer, M={M}",
                   "M": M, "K": cfg.K, "N": cfg.N, "E": cfg.E,
                   "topk": cfg.topk, "mode": cfg.mode, "flags": args.flags,
                   "experts_touched": head.touched,
                   "layer_flops": head.flops, "layer_bytes": head.bytes,
                   "gb_s": round(head.bytes / (ms * 1e-3) / 1e9, 1),
                   "cold_cache": small_ws},
        "roofline": roof,
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "cpu_baseline": cpu,
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "host_cores": cores},
    }
    if not args.no_configs and args.config == "mixtral" and args.m is None:
        head = weights = None  # the headline weights go before the next set
        torch.cuda.empty_cache()
        for name in OTHER_CONFIGS:
            rows[name] = sweep_config(testing.CONFIGS[name], dev, args)
    out["row_fields"] = list(ROW_FIELDS)
    out["ref_fields"] = list(REF_FIELDS)
    out["rows"] = rows
    print(json.dumps(out, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
