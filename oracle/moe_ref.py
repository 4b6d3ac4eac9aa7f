"""CPU oracle of the fused-MoE path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product path
(``flaggems_sglang``) never does.

It restates, on the CPU in torch fp32 (plus the C alignment in
``align_ref.c``), what the reference path computes:

* routing: softmax / sigmoid -> top-k -> renormalise
  (reference tests/test_fused_moe.py:37-41);
* alignment: stable expert grouping (src/flaggems_sglang/ops/fused_moe.py:
  130-139), via ``align_ref.c``;
* ``silu_and_mul`` (ops/fused_moe.py:44-63, fp32 math, bf16 store), the
  erf ``gelu_and_mul`` (:219-220) and the bias variant's fused swiglu
  (:274-314; triton_kernels / sgl_kernel are not in the image, their
  published formulas are restated -- parity of those two is pinned by
  closed forms and library identities only);
* the fused expert computation (ops/fused_moe.py:197-232) with the rounding
  points of an unfused pipeline: GEMM1 output rounded to bf16, activation
  rounded to bf16, GEMM2 output rounded to bf16, fp32 weighted top-k sum
  rounded to bf16. ``apply_router_weight_on_input`` puts the gate scale on the
  GEMM1 output rows (:202-203, gammas of the first matmul_ogs call);
* fp8 / int8 w8a8: the reference rejects them (ops/fused_moe.py:170-185); the
  quantisers and dequantising MoE here define them: e4m3fn with 128x128
  weight blocks and 1x128 activation groups (scale = max(amax, 1e-10)/448),
  int8 with per-output-channel weight scales and per-token activation scales
  (scale = max(amax, 1e-10)/127, round half to even);
* the routing-format conversion of ``_standard_topk_to_triton_kernels``
  (ops/fused_moe.py:126-139) in Python loops, and the tile tables of
  ``triton_kernels``' ``compute_expt_data_torch`` (:140; published algorithm
  restated, version unpinned).

How each function is pinned (closed forms, brute force, library routines,
invariants) is listed in tests/test_oracle.py. ``matmul_ogs``'s exact
accumulation order lives in the un-vendored ``triton_kernels`` package and
is not restated: parity of the GEMM arithmetic is to tolerance, not
bit-exact.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

FP8_MAX = 448.0
INT8_MAX = 127.0
QUANT_EPS = 1e-10


def _clib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: run `make -C {_HERE}`")
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_align.restype = ctypes.c_int
        lib.oracle_align.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
        ]
        _lib = lib
    return _lib


# --------------------------------------------------------------- routing ---
def route(logits: torch.Tensor, topk: int, scoring: str = "softmax",
          renormalize: bool = True):
    """``(topk_weights f32 [M, k], topk_ids int32 [M, k])`` from router logits
    (reference tests/test_fused_moe.py:37-41; sigmoid scoring for the
    DeepSeek-shaped config)."""
    logits = logits.float()
    if scoring == "softmax":
        scores = torch.softmax(logits, dim=-1)
    elif scoring == "sigmoid":
        scores = torch.sigmoid(logits)
    else:
        raise ValueError(scoring)
    w, ids = torch.topk(scores, k=topk, dim=-1)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.float(), ids.to(torch.int32)


def topk_gating(logits: torch.Tensor, topk: int, scoring: str = "softmax",
                renormalize: bool = True):
    """The gating kernel's contract: scores = softmax / sigmoid of the fp32
    logits; the top-k experts ranked by logit descending with equal logits
    in ascending id order (a stable descending sort), in rank order; weights
    = their scores, divided by the top-k sum when ``renormalize``. Ranking
    the logits selects the same experts as ranking the scores (both maps are
    monotonic) -- what :func:`route` / the reference's tests do with
    torch.topk -- but leaves no rounding ties."""
    logits = logits.float()
    ids = torch.sort(logits, dim=-1, descending=True, stable=True).indices[:, :topk]
    scores = torch.softmax(logits, dim=-1) if scoring == "softmax" else torch.sigmoid(logits)
    w = torch.gather(scores, 1, ids)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.float(), ids.to(torch.int32)


# ------------------------------------------------------------- alignment ---
def align(topk_ids, num_experts: int, block_size: int):
    """Stable block-padded expert grouping (C restatement in align_ref.c).
    Returns numpy ``(sorted_ids, expert_ids, num_post_pad)``."""
    ids = np.ascontiguousarray(np.asarray(topk_ids, dtype=np.int32).reshape(-1))
    numel = ids.size
    max_padded = numel + num_experts * (block_size - 1)
    sorted_ids = np.empty(max_padded, dtype=np.int32)
    expert_ids = np.empty(max(max_padded // block_size, 1), dtype=np.int32)
    npp = np.zeros(1, dtype=np.int32)
    rc = _clib().oracle_align(
        ids.ctypes.data, numel, num_experts, block_size, sorted_ids.ctypes.data,
        expert_ids.ctypes.data, npp.ctypes.data, max_padded)
    if rc != 0:
        raise ValueError("oracle_align: invalid arguments")
    return sorted_ids, expert_ids[: max_padded // block_size], int(npp[0])


# -------------------------------------------------------- routing format ---
ROUTING_BLOCK_MS = (16, 32, 64, 128)


def topk_to_routing(topk_weights, topk_ids, n_expts_tot: int):
    """The reference's ``_standard_topk_to_triton_kernels`` conversion
    (src/flaggems_sglang/ops/fused_moe.py:126-139) in plain Python loops:

    * :130-131 sort each token's ids ascending, carrying the weights (ties,
      which top-k routing never produces, keep slot order);
    * :133 flatten; :134 stable argsort of the flat ids -> ``topk_indx``,
      with ids outside ``[0, n_expts_tot)`` (slots not routed here) keyed
      behind expert ``n_expts_tot - 1``, in flat order: matmul_ogs reads
      expert e's rows at ``[token_offs_raw[e], token_offs_raw[e+1])`` with
      ``token_offs_raw`` starting at 0 (:140), so no unrouted slot may sit
      ahead of expert 0 (where argsort would put negative ids; the
      reference's callers never pass any);
    * :135 its inverse -> ``gate_indx``; :136 ``gate_scal`` = weights at
      ``topk_indx``;
    * :137-139 ``hist``: ids in ``[0, n_expts_tot)`` counted per expert
      (``histc`` with ``max = n_expts_tot - 1`` ignores the rest).

    Returns numpy arrays ``(gate_scal f32, topk_indx i32, gate_indx i32,
    hist i32)``.
    """
    w = np.asarray(topk_weights, dtype=np.float32)
    ids = np.asarray(topk_ids, dtype=np.int64)
    M, k = ids.shape
    flat_ids, flat_w = [], []
    for t in range(M):
        order = sorted(range(k), key=lambda j: (int(ids[t, j]), j))
        flat_ids += [int(ids[t, j]) for j in order]
        flat_w += [w[t, j] for j in order]
    n = M * k
    topk_indx = sorted(range(n), key=lambda i: (
        flat_ids[i] if 0 <= flat_ids[i] < n_expts_tot else n_expts_tot, i))
    gate_indx = [0] * n
    for p, i in enumerate(topk_indx):
        gate_indx[i] = p
    gate_scal = [flat_w[i] for i in topk_indx]
    hist = [0] * n_expts_tot
    for v in flat_ids:
        if 0 <= v < n_expts_tot:
            hist[v] += 1
    return (np.array(gate_scal, dtype=np.float32).reshape(n),
            np.array(topk_indx, dtype=np.int32).reshape(n),
            np.array(gate_indx, dtype=np.int32).reshape(n),
            np.array(hist, dtype=np.int32))


def routing_order(gate_scal, src_indx, hist, n_gates: int, block: int):
    """What the grouped GEMMs take from a routing tuple (plain Python loops):
    expert e owns the gathered positions ``[raw[e], raw[e] + h[e])`` of
    ``src_indx``, ``raw`` = exclusive sums of the histogram ``h`` -- the
    ``token_offs_raw`` ranges matmul_ogs reads (ops/fused_moe.py:140,
    205-231). ``h`` is the histogram clamped so the ranges stay inside
    ``[0, n_gates)`` (negative counts read as 0, running sums cut at
    ``n_gates``).

    Returns numpy ``(sorted_ids, expert_ids, num_post_pad, ids, weights)``:
    the block-padded order of :func:`align` (expert e's segment lists
    ``src_indx[raw[e] : raw[e] + h[e]]``, pads and out-of-range entries =
    ``n_gates``; ``expert_ids`` per block, -1 past the padded total) and per
    flat slot ``v = src_indx[p]`` its expert (-1 for ``p`` past the
    histogram's total) and weight ``gate_scal[p]``."""
    src = [int(v) for v in np.asarray(src_indx).reshape(-1)]
    gs = np.asarray(gate_scal, dtype=np.float32).reshape(-1)
    E = len(hist)
    h, run = [], 0
    for c in (int(v) for v in hist):
        c = min(max(c, 0), n_gates - run)
        h.append(c)
        run += c
    raw = [0]
    for c in h:
        raw.append(raw[-1] + c)
    padded = [(c + block - 1) // block * block for c in h]
    max_padded = n_gates + E * (block - 1)
    sorted_ids = [n_gates] * max_padded
    expert_ids = [-1] * (max_padded // block)
    pos = 0
    for e in range(E):
        for i in range(h[e]):
            v = src[raw[e] + i]
            sorted_ids[pos + i] = v if 0 <= v < n_gates else n_gates
        for b in range(padded[e] // block):
            expert_ids[pos // block + b] = e
        pos += padded[e]
    ids = np.full(n_gates, -7, dtype=np.int32)  # every slot of a permutation is written
    w = np.zeros(n_gates, dtype=np.float32)
    for p, v in enumerate(src):
        if not 0 <= v < n_gates:
            continue
        e = next((x for x in range(E) if raw[x] <= p < raw[x + 1]), -1)
        ids[v] = e
        w[v] = gs[p]
    return (np.array(sorted_ids, dtype=np.int32), np.array(expert_ids, dtype=np.int32),
            pos, ids, w)


def routing_max_tiles(n_gates: int, n_expts_tot: int) -> int:
    """Tile-table length of ``compute_expt_data_torch``: ``n_gates`` when it
    does not exceed the expert count, else ceil((n_gates - E + 1) / 16) +
    E - 1 (the bound for the smallest block, 16)."""
    if n_gates <= n_expts_tot:
        return n_gates
    return -((-(n_gates - n_expts_tot + 1)) // min(ROUTING_BLOCK_MS)) + n_expts_tot - 1


def expt_data(hist, n_expts_tot: int, n_gates: int):
    """``compute_expt_data_torch(hist, n_expts_tot, n_gates)`` -- the block
    metadata the reference stores in ``RoutingData.expt_data``
    (ops/fused_moe.py:140-143). That function lives in OpenAI's
    ``triton_kernels`` (python/triton_kernels/triton_kernels/routing.py; no
    version is pinned by the reference and the package is absent here); its
    published algorithm, restated:

    * ``token_offs_raw``: [0] + cumulative sum of ``hist`` (E + 1 entries);
    * for each block_m in (16, 32, 64, 128): ``n_tiles = ceil(hist /
      block_m)``, ``token_offs_pad[block_m]`` = [0] + cumulative sum of
      ``n_tiles`` (tile units), and ``block_pid_map[block_m]`` of
      :func:`routing_max_tiles` entries, -1 except tile ``off_e + b`` of
      expert ``e`` (``b < n_tiles[e]``), which holds ``(b << 16) + e``.

    Returns ``(token_offs_raw, {block_m: token_offs_pad},
    {block_m: block_pid_map})`` as int64 numpy arrays.
    """
    hist = [int(h) for h in hist]
    raw = [0]
    for h in hist:
        raw.append(raw[-1] + h)
    max_tiles = routing_max_tiles(n_gates, n_expts_tot)
    pads, maps = {}, {}
    for bm in ROUTING_BLOCK_MS:
        n_tiles = [(h + bm - 1) // bm for h in hist]
        pad = [0]
        for nt in n_tiles:
            pad.append(pad[-1] + nt)
        pid = [-1] * max_tiles
        for e in range(n_expts_tot):
            for b in range(n_tiles[e]):
                pid[pad[e] + b] = (b << 16) + e
        pads[bm] = np.array(pad, dtype=np.int64)
        maps[bm] = np.array(pid, dtype=np.int64)
    return np.array(raw, dtype=np.int64), pads, maps


# --------------------------------------------------------- element-wise ---
def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """bf16(silu(f32 gate) * f32 up) over x = [gate | up]
    (ops/fused_moe.py:58-62)."""
    n = x.shape[-1] // 2
    g = x[..., :n].float()
    u = x[..., n:].float()
    return (g / (1.0 + torch.exp(-g)) * u).to(torch.bfloat16)


def gelu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """bf16(gelu(f32 gate) * f32 up) over x = [gate | up] with the exact
    gelu 0.5*g*(1 + erf(g/sqrt(2))): sgl_kernel's gelu_and_mul, which the
    reference calls for activation="gelu" (ops/fused_moe.py:219-220; the
    function is not in this image, its published formula is restated)."""
    n = x.shape[-1] // 2
    g = x[..., :n].float()
    u = x[..., n:].float()
    return (0.5 * g * (1.0 + torch.erf(g * 0.7071067811865476)) * u).to(torch.bfloat16)


def swiglu(g: torch.Tensor, u: torch.Tensor, alpha: float = 1.0,
           limit: float = 0.0) -> torch.Tensor:
    """The swiglu the bias variant fuses into matmul_ogs
    (ops/fused_moe.py:274-314, triton_kernels.swiglu.swiglu_fn with
    gemm1_alpha / gemm1_clamp_limit; not in this image -- the published
    GPT-OSS formula is restated): with limit > 0, g = min(g, limit) and
    u = clamp(u, -limit, limit); out = g * sigmoid(alpha*g) * (u + 1), fp32
    in, fp32 out (the caller rounds)."""
    g = g.float()
    u = u.float()
    if limit > 0:
        g = torch.clamp(g, max=limit)
        u = torch.clamp(u, min=-limit, max=limit)
    return g * torch.sigmoid(alpha * g) * (u + 1.0)


def moe_sum(y: torch.Tensor) -> torch.Tensor:
    """[M, k, K] -> bf16(fp32 sum over k)."""
    return y.float().sum(dim=1).to(torch.bfloat16)


# ------------------------------------------------------------ quantisers ---
def quant_fp8_group(x: torch.Tensor, group: int = 128):
    """Dynamic per-(row, group) e4m3fn quantisation of a 2D tensor:
    scale = max(amax, 1e-10)/448, q = e4m3fn(clamp(x/scale, +-448))."""
    rows, cols = x.shape
    xg = x.float().reshape(rows, cols // group, group)
    amax = xg.abs().amax(dim=-1)
    scale = torch.clamp(amax, min=QUANT_EPS) / FP8_MAX
    q = torch.clamp(xg / scale[..., None], -FP8_MAX, FP8_MAX)
    return q.to(torch.float8_e4m3fn).reshape(rows, cols), scale


def dequant_fp8_group(q: torch.Tensor, scale: torch.Tensor, group: int = 128):
    rows, cols = q.shape
    return (q.float().reshape(rows, cols // group, group) *
            scale[..., None]).reshape(rows, cols)


def quant_int8_token(x: torch.Tensor):
    """Dynamic per-row int8: scale = max(amax, 1e-10)/127,
    q = clamp(round_half_even(x/scale), -127, 127)."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1)
    scale = torch.clamp(amax, min=QUANT_EPS) / INT8_MAX
    q = torch.clamp(torch.round(xf / scale[:, None]), -INT8_MAX, INT8_MAX)
    return q.to(torch.int8), scale


def quant_weight_fp8_block(w: torch.Tensor, block: int = 128):
    """One expert's [R, C] weight -> (e4m3fn [R, C], fp32 [R/128, C/128]),
    scale = max(block amax, 1e-10)/448."""
    r, c = w.shape
    wb = w.float().reshape(r // block, block, c // block, block)
    amax = wb.abs().amax(dim=(1, 3))
    scale = torch.clamp(amax, min=QUANT_EPS) / FP8_MAX
    q = torch.clamp(wb / scale[:, None, :, None], -FP8_MAX, FP8_MAX)
    return q.to(torch.float8_e4m3fn).reshape(r, c), scale


def dequant_weight_fp8_block(q: torch.Tensor, scale: torch.Tensor,
                             block: int = 128) -> torch.Tensor:
    r, c = q.shape
    return (q.float().reshape(r // block, block, c // block, block) *
            scale[:, None, :, None]).reshape(r, c)


def quant_weight_int8_channel(w: torch.Tensor):
    """One expert's [R, C] weight -> (int8 [R, C], fp32 [R]) per output row."""
    wf = w.float()
    amax = wf.abs().amax(dim=-1)
    scale = torch.clamp(amax, min=QUANT_EPS) / INT8_MAX
    q = torch.clamp(torch.round(wf / scale[:, None]), -INT8_MAX, INT8_MAX)
    return q.to(torch.int8), scale


# ----------------------------------------------------------- fused MoE ---
def _expert_weights(mode, w1, w2, w1_scale, w2_scale, e):
    """fp32 (dequantised) weights of expert e: W13 [2N, K], W2 [K, N].
    Only this expert is copied to the host, so the weights may stay on the
    GPU and be checked at full model size."""
    a, b = w1[e].cpu(), w2[e].cpu()
    if mode == "bf16":
        return a.float(), b.float()
    if mode == "fp8":
        return (dequant_weight_fp8_block(a, w1_scale[e].cpu()),
                dequant_weight_fp8_block(b, w2_scale[e].cpu()))
    if mode == "int8":
        return (a.float() * w1_scale[e].cpu().float()[:, None],
                b.float() * w2_scale[e].cpu().float()[:, None])
    raise ValueError(mode)


def _quant_dequant_act(mode, a: torch.Tensor) -> torch.Tensor:
    """What the w8a8 kernels feed the MFMA: quantise then dequantise."""
    if mode == "bf16":
        return a.float()
    if mode == "fp8":
        q, s = quant_fp8_group(a, 128)
        return dequant_fp8_group(q, s, 128)
    q, s = quant_int8_token(a)
    return q.float() * s[:, None]


def fused_moe(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
              topk_weights: torch.Tensor, topk_ids: torch.Tensor,
              mode: str = "bf16", w1_scale: Optional[torch.Tensor] = None,
              w2_scale: Optional[torch.Tensor] = None,
              apply_router_weight_on_input: bool = False,
              tokens: Optional[Sequence[int]] = None,
              return_mag: bool = False, activation: str = "silu",
              b1: Optional[torch.Tensor] = None, b2: Optional[torch.Tensor] = None,
              alpha: float = 1.0, limit: float = 0.0):
    """Reference fused MoE on CPU tensors (SGLang layout: w1 [E, 2N, K],
    w2 [E, K, N]). Returns bf16 [len(tokens), K] (all tokens by default);
    with ``return_mag`` also the fp32 magnitude sum_j |w_j| * (|y_j| + q_j)
    of the terms each output sums (the scale its rounding errors live on).
    q_j is 2^-8 * (|a| @ |W2|^T) for bf16: fp32 sums in another order round
    an element of the bf16 intermediate a to its neighbour now and then, and
    one such flip moves y_j by up to 2^-8 |a_i W2_ki| whatever the size of
    y_j (outputs that cancel towards 0 included). For fp8 / int8 it is
    2^-2 * (|a_q| @ |W2|^T), a quarter of the absolute dot product behind
    y_j. The GEMM2 input is
    re-quantised from a bf16 intermediate; where the kernel's bf16 value
    differs from this oracle's by an ulp the two round to neighbouring grid
    points, and each such flip moves y_j by one quantisation step (up to
    2^-3 of the element for e4m3) times a weight. The fp8 MFMA sums its
    products with about 14 bits of precision, which makes about 2 % of the
    intermediate differ by an ulp (the same rate as scaling W13 by 1+2^-14
    in this oracle); at that rate this bound is met with a factor ~2 to
    spare, while a 10 % error in one weight-scale block still fails it.

    Every token's output depends only on its own row and routing, so any
    subset of tokens can be checked exactly at full layer size.

    ``activation``: "silu" or "gelu" (unfused pipeline, GEMM1 output rounded
    to bf16 first), or "swiglu" -- the bias variant (ops/fused_moe.py:
    235-325): GEMM1 + ``b1`` [E, 2N] (gate rows then linear rows, like w1)
    with swiglu(alpha, limit) fused (no bf16 rounding before it), GEMM2 +
    ``b2`` [E, K].
    """
    x = x.cpu()
    topk_weights = topk_weights.cpu().float()
    topk_ids = topk_ids.cpu().long()
    if tokens is None:
        tokens = range(x.shape[0])
    tok = torch.as_tensor(list(tokens), dtype=torch.long)
    xs = x[tok]
    ids = topk_ids[tok]
    wts = topk_weights[tok]
    T, k = ids.shape
    K = x.shape[1]
    N = w2.shape[2]
    E = w1.shape[0]
    # x as the GEMM1 kernel sees it (per-token quantisation is row-local, so
    # quantising the subset equals quantising all rows then selecting).
    xq = _quant_dequant_act(mode, xs)
    y = torch.zeros(T, k, K, dtype=torch.float32)
    q = torch.zeros(T, k, K, dtype=torch.float32)
    for e in torch.unique(ids).tolist():
        if e < 0 or e >= E:
            continue
        rows, slots = torch.nonzero(ids == e, as_tuple=True)
        w13e, w2e = _expert_weights(mode, w1, w2, w1_scale, w2_scale, e)
        h = xq[rows] @ w13e.t()
        if b1 is not None:
            h = h + b1[e].cpu().float()
        gam = wts[rows, slots][:, None]
        if apply_router_weight_on_input and activation != "swiglu":
            h = h * gam
        if activation == "swiglu":
            # matmul_ogs applies the input gammas to its fused activation's
            # output (parity unpinned: triton_kernels is absent)
            n = h.shape[1] // 2
            a = swiglu(h[:, :n], h[:, n:], alpha, limit)
            if apply_router_weight_on_input:
                a = a * gam
            a = a.to(torch.bfloat16)
        elif activation == "gelu":
            a = gelu_and_mul(h.to(torch.bfloat16))
        else:
            a = silu_and_mul(h.to(torch.bfloat16))
        aq = _quant_dequant_act(mode, a)
        ye = aq @ w2e.t()
        if b2 is not None:
            ye = ye + b2[e].cpu().float()
        ye = ye.to(torch.bfloat16).float()
        y[rows, slots] = ye
        if return_mag:
            q[rows, slots] = (aq.abs() @ w2e.abs().t()) * (2.0 ** -8 if mode == "bf16"
                                                           else 2.0 ** -2)
    terms = y if apply_router_weight_on_input else y * wts[:, :, None]
    out = terms.sum(dim=1).to(torch.bfloat16)
    if return_mag:
        wq = q if apply_router_weight_on_input else q * wts.abs()[:, :, None]
        return out, terms.abs().sum(dim=1) + wq.sum(dim=1)
    return out


def compare(res: torch.Tensor, ref: torch.Tensor, atol: float, rtol: float,
            mag: Optional[torch.Tensor] = None):
    """Tolerance check used by the parity tests:
    |res - ref| <= atol + rtol * s elementwise, with s = ``mag`` (the
    magnitude of the summed terms, from ``fused_moe(..., return_mag=True)``)
    or |ref|; plus max-abs and mean-rel (sum|res - ref| / sum|ref|) for
    reporting. Using the term magnitude keeps outputs that cancel to ~0
    from being held to a tighter bound than their own rounding allows."""
    r = res.float().cpu()
    f = ref.float().cpu()
    s = f.abs() if mag is None else mag.float().cpu()
    diff = (r - f).abs()
    ok = bool((diff <= atol + rtol * s).all()) and bool(torch.isfinite(r).all())
    max_abs = float(diff.max()) if diff.numel() else 0.0
    mean_rel = float(diff.sum() / f.abs().sum().clamp(min=1e-30)) if diff.numel() else 0.0
    return ok, max_abs, mean_rel
