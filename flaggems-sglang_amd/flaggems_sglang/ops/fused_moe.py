"""Fused Mixture-of-Experts for MI355X (gfx950): host side of the op.

Every entry point validates its tensors, allocates outputs and the one
workspace with the torch caching allocator, and hands plain device pointers
plus torch's current HIP stream to ``libfgs_moe.so`` (include/fgs_moe.h).
All arithmetic runs in the library's HIP kernels; nothing here computes on
the host, and there is no CPU fallback.

Reference interface mirrored: src/flaggems_sglang/ops/fused_moe.py
  - ``triton_kernel_fused_experts``  (:149-232)  -> same name, same flags
  - ``_silu_and_mul_triton``          (:88-116)   -> ``silu_and_mul``
  - ``_standard_topk_to_triton_kernels`` (:119-146) -> ``standard_topk_to_routing``
  - the SGLang-layout call the plugin wrapper makes (:328-422) -> ``fused_moe``
"""

from __future__ import annotations

import logging
import weakref
from dataclasses import dataclass
from typing import Optional

import torch

from flaggems_sglang import _capi

logger = logging.getLogger(__name__)

# Same wording as the reference's assertion messages (ops/fused_moe.py:41).
_UNSUPPORTED_FEATURE_MSG = "{name} is not supported"


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{name} must be a GPU tensor: the fused-MoE kernels run only on "
            "the MI355X (no CPU path)"
        )


class _ConversionCache:
    """Layout conversions of model weights, made once per live weight.

    An entry belongs to the source's root tensor (a view's ``_base``, else
    the tensor itself), matched by object identity, and within it to the
    view's geometry (offset, shape, strides, dtype); it is served while the
    root's version counter and storage are unchanged: an in-place update
    through the tensor (``w.copy_(...)``, ``w.add_(...)``) bumps the version
    and a reassignment of ``param.data`` swaps the storage, and either
    converts again. An update that goes through ``param.data`` in place
    (``param.data.copy_(...)``, what many weight loaders do) changes neither
    and cannot be seen here: after one, call :func:`clear_weight_cache`.
    ``weakref.finalize`` on the root drops its entries when the root is
    garbage-collected, so the cache holds exactly one converted copy per live
    weight -- a model with any number of MoE layers converts each weight
    once -- and never a copy of a dead one. A conversion that returns a view
    of its source (a transposed view that is already contiguous in the other
    order) costs nothing and is not stored: storing it would keep the root
    alive.
    """

    def __init__(self, fn):
        self._fn = fn
        self._roots: dict = {}  # id(root) -> {geometry: (version, converted)}

    def __call__(self, w: torch.Tensor) -> torch.Tensor:
        root = w._base if w._base is not None else w
        geometry = (w.storage_offset(), tuple(w.shape), tuple(w.stride()), w.dtype)
        stamp = (root._version, root.untyped_storage().data_ptr())
        views = self._roots.get(id(root))
        if views is not None:
            hit = views.get(geometry)
            if hit is not None and hit[0] == stamp:
                return hit[1]
        out = self._fn(w)
        if out.untyped_storage().data_ptr() == w.untyped_storage().data_ptr():
            return out  # zero-copy view of the source
        if views is None:
            views = self._roots[id(root)] = {}
            weakref.finalize(root, self._roots.pop, id(root), None)
        views[geometry] = (stamp, out)
        return out

    def __len__(self) -> int:
        return sum(len(v) for v in self._roots.values())

    def clear(self) -> None:
        for views in self._roots.values():
            views.clear()


# --------------------------------------------------------------- routing ---
@dataclass
class ExptData:
    """Block metadata of a routing (the fields of ``triton_kernels.routing.
    ExptData`` that ``compute_expt_data_torch`` fills, ops/fused_moe.py:140):
    ``hist`` int32 ``[E]``; ``token_offs_raw`` int32 ``[E + 1]`` (exclusive
    sums of ``hist``); per block_m in (16, 32, 64, 128) ``token_offs_pad
    [block_m]`` int32 ``[E + 1]`` (exclusive sums of ``ceil(hist /
    block_m)``, in tiles) and ``block_pid_map[block_m]`` int32
    ``[max_tiles]`` (``(b << 16) | e`` for expert e's b-th tile, -1 past the
    last tile)."""

    hist: torch.Tensor
    token_offs_raw: torch.Tensor
    token_offs_pad: dict
    block_pid_map: dict


@dataclass
class RoutingData:
    """Duck-typed stand-in for ``triton_kernels.routing.RoutingData`` with the
    fields the reference builds and reads (ops/fused_moe.py:141-143,
    200-201)."""

    gate_scal: torch.Tensor
    expt_hist: torch.Tensor
    n_expts_tot: int
    n_expts_act: int
    expt_data: Optional[ExptData] = None


@dataclass
class GatherIndx:
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


@dataclass
class ScatterIndx:
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


def standard_topk_to_routing(topk_weights, topk_ids, n_expts_tot):
    """``(topk_weights, topk_ids)`` -> ``(RoutingData, GatherIndx,
    ScatterIndx)`` in the reference's routing format, computed on the GPU
    (``fgs_moe_topk_to_routing``: the stable alignment kernel plus two small
    kernels).

    The result is that of ``_standard_topk_to_triton_kernels``
    (ops/fused_moe.py:119-146): per-token ascending id sort carrying the
    weights (:130-131), stable argsort of the flattened ids (``topk_indx``,
    :134) and its inverse (``gate_indx``, :135), the gathered gate scales
    (:136), the per-expert histogram (:137-139) and the tile tables of
    ``compute_expt_data_torch`` (:140) in ``routing_data.expt_data``
    (:class:`ExptData`). Ids below 0 (slots not routed here) sort ahead of
    expert 0 and ids >= E behind expert E-1, in slot order.
    """
    _require_gpu("topk_ids", topk_ids)
    _require_gpu("topk_weights", topk_weights)
    assert topk_ids.ndim == 2 and topk_weights.shape == topk_ids.shape, (
        "topk_ids / topk_weights must be [M, topk]")
    lib = _capi.load()
    M, k = topk_ids.shape
    E = int(n_expts_tot)
    numel = M * k
    max_tiles = lib.fgs_moe_routing_max_tiles(numel, E)
    ws_bytes = lib.fgs_moe_routing_workspace_bytes(numel, E)
    if max_tiles < 0 or ws_bytes < 0:
        raise ValueError(f"standard_topk_to_routing: n_expts_tot={E} not in [1, 1022]")
    dev = topk_ids.device
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    i32 = dict(dtype=torch.int32, device=dev)
    gate_scal = torch.empty(numel, dtype=torch.float32, device=dev)
    topk_indx = torch.empty(numel, **i32)
    gate_indx = torch.empty(numel, **i32)
    hist = torch.empty(E, **i32)
    offs_raw = torch.empty(E + 1, **i32)
    offs_pad = torch.empty((len(_capi.ROUTING_BLOCK_MS), E + 1), **i32)
    pid_map = torch.empty((len(_capi.ROUTING_BLOCK_MS), max(max_tiles, 1)), **i32)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    _capi.check(
        lib.fgs_moe_topk_to_routing(
            wts.data_ptr(), ids.data_ptr(), M, k, E, gate_scal.data_ptr(),
            topk_indx.data_ptr(), gate_indx.data_ptr(), hist.data_ptr(),
            offs_raw.data_ptr(), offs_pad.data_ptr(), pid_map.data_ptr(),
            max_tiles, ws.data_ptr(), ws_bytes, _stream_ptr(ids)),
        "standard_topk_to_routing",
    )
    bms = _capi.ROUTING_BLOCK_MS
    expt = ExptData(hist, offs_raw,
                    {bm: offs_pad[i] for i, bm in enumerate(bms)},
                    {bm: pid_map[i, :max_tiles] for i, bm in enumerate(bms)})
    routing = RoutingData(gate_scal, hist, E, k, expt)
    return (
        routing,
        GatherIndx(src_indx=topk_indx, dst_indx=gate_indx),
        ScatterIndx(src_indx=gate_indx, dst_indx=topk_indx),
    )


def _routing_args(routing_data, gather_indx, num_tokens):
    """The routing tuple's device arrays as the C ABI takes them:
    ``(gate_scal f32, src_indx int32, expt_hist int32, topk, E)``, each
    contiguous on the GPU."""
    top_k = int(routing_data.n_expts_act)
    gate = routing_data.gate_scal
    src = gather_indx.src_indx
    hist = routing_data.expt_hist
    for name, t in (("routing_data.gate_scal", gate), ("gather_indx.src_indx", src),
                    ("routing_data.expt_hist", hist)):
        _require_gpu(name, t)
    n = num_tokens * top_k
    assert gate.numel() == n and src.numel() == n, (
        "routing tuple does not hold num_tokens * n_expts_act gates")
    E = hist.numel()
    n_tot = getattr(routing_data, "n_expts_tot", E)
    assert int(n_tot) == E, "routing_data.expt_hist must hold n_expts_tot counts"
    return (gate.to(torch.float32).contiguous(), src.to(torch.int32).contiguous(),
            hist.to(torch.int32).contiguous(), top_k, E)


def _routing_to_topk(routing_data, gather_indx, num_tokens):
    """Inverse of :func:`standard_topk_to_routing` on the GPU
    (``fgs_moe_routing_to_topk``, one kernel): per-token ``(topk_weights,
    topk_ids)`` in the row-sorted slot order of the tuple (ids ascending
    within a token, the order of the reference's conversion,
    ops/fused_moe.py:130). Expert e owns the gathered positions of
    ``token_offs_raw`` = exclusive sums of ``expt_hist`` (the ranges
    matmul_ogs reads); positions past the histogram's total come back as id
    -1 (dropped)."""
    gate, src, hist, top_k, E = _routing_args(routing_data, gather_indx, num_tokens)
    n = num_tokens * top_k
    wts = torch.empty(n, dtype=torch.float32, device=src.device)
    ids = torch.empty(n, dtype=torch.int32, device=src.device)
    _capi.check(
        _capi.load().fgs_moe_routing_to_topk(
            gate.data_ptr(), src.data_ptr(), hist.data_ptr(), num_tokens, top_k, E,
            wts.data_ptr(), ids.data_ptr(), _stream_ptr(src)),
        "routing_to_topk",
    )
    return wts.view(num_tokens, top_k), ids.view(num_tokens, top_k)


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor,
               topk: int, renormalize: bool = True,
               scoring_func: str = "softmax"):
    """Router gating on the GPU (HIP kernel, one wave per token): scores
    (softmax or sigmoid of ``gating_output [M, E]``, fp32 or bf16), top-k
    experts ranked by logit (ties: lower id), weights = their scores,
    renormalised to sum 1 when ``renormalize``. Returns ``(topk_weights f32
    [M, topk], topk_ids int32 [M, topk])`` -- the routing the reference's
    tests build with torch ops (tests/test_fused_moe.py:37-41)."""
    _require_gpu("gating_output", gating_output)
    assert gating_output.ndim == 2, "gating_output must be [M, E]"
    assert hidden_states.shape[0] == gating_output.shape[0], "token count mismatch"
    if scoring_func == "softmax":
        scoring = _capi.SCORING_SOFTMAX
    elif scoring_func == "sigmoid":
        scoring = _capi.SCORING_SIGMOID
    else:
        raise ValueError(f"Unsupported scoring function: {scoring_func}")
    logits = gating_output
    if logits.dtype not in (torch.float32, torch.bfloat16):
        logits = logits.float()
    logits = logits.contiguous()
    M, E = logits.shape
    w = torch.empty((M, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((M, topk), dtype=torch.int32, device=logits.device)
    _capi.check(
        _capi.load().fgs_moe_topk_gating(
            logits.data_ptr(), 1 if logits.dtype == torch.bfloat16 else 0, M, E,
            topk, scoring, 1 if renormalize else 0, w.data_ptr(), ids.data_ptr(),
            _stream_ptr(logits)),
        "fused_topk",
    )
    return w, ids


# ------------------------------------------------------------ small ops ---
def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int,
                         block_size: int, _single_workgroup: bool = False):
    """Expert-grouped, block-padded routing order (HIP kernel).

    Returns ``(sorted_ids, expert_ids, num_tokens_post_padded)``; the
    semantics are those of ``fgs_moe_align_block_size`` in include/fgs_moe.h.
    The order inside each expert is the stable order of the reference's
    ``argsort(expt_indx, stable=True)`` (ops/fused_moe.py:134).
    """
    _require_gpu("topk_ids", topk_ids)
    lib = _capi.load()
    ids = topk_ids.to(torch.int32).contiguous()
    numel = ids.numel()
    max_padded = lib.fgs_moe_align_max_padded(numel, num_experts, block_size)
    if max_padded < 0:
        raise ValueError("invalid moe_align_block_size arguments")
    dev = ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max(max_padded // block_size, 1),
                             dtype=torch.int32, device=dev)
    npp = torch.empty(1, dtype=torch.int32, device=dev)
    sc_bytes = 0 if _single_workgroup else max(
        lib.fgs_moe_align_scratch_bytes(numel, num_experts), 0)
    scratch = torch.empty(max(sc_bytes, 1), dtype=torch.uint8, device=dev)
    _capi.check(
        lib.fgs_moe_align_block_size(
            ids.data_ptr(), numel, num_experts, block_size,
            sorted_ids.data_ptr(), expert_ids.data_ptr(), npp.data_ptr(),
            max_padded, scratch.data_ptr() if sc_bytes else None, sc_bytes,
            _stream_ptr(ids)),
        "moe_align_block_size",
    )
    return sorted_ids, expert_ids[: max_padded // block_size], npp


def silu_and_mul(x: torch.Tensor, out: Optional[torch.Tensor] = None):
    """``bf16(silu(gate) * up)`` over ``x = [gate | up]`` (HIP kernel);
    the reference's ``_silu_and_mul_triton`` (ops/fused_moe.py:88-116)."""
    _require_gpu("x", x)
    assert x.dtype == torch.bfloat16, "x must be bfloat16"
    x = x.contiguous()
    n = x.shape[-1] // 2
    rows = x.numel() // x.shape[-1]
    if out is None:
        out = x.new_empty(x.shape[:-1] + (n,))
    _capi.check(
        _capi.load().fgs_moe_silu_and_mul(
            x.data_ptr(), out.data_ptr(), rows, n, _stream_ptr(x)),
        "silu_and_mul",
    )
    return out


def moe_sum(x: torch.Tensor, out: Optional[torch.Tensor] = None):
    """``[M, topk, K] -> [M, K]`` fp32-accumulated sum (HIP kernel)."""
    _require_gpu("x", x)
    assert x.dtype == torch.bfloat16 and x.ndim == 3, "x must be bf16 [M, topk, K]"
    x = x.contiguous()
    m, topk, k = x.shape
    if out is None:
        out = x.new_empty((m, k))
    _capi.check(
        _capi.load().fgs_moe_sum(x.data_ptr(), out.data_ptr(), m, topk, k,
                                 _stream_ptr(x)),
        "moe_sum",
    )
    return out


def per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128):
    """Dynamic 1 x group fp8 (e4m3fn) quantisation (HIP kernel).
    Returns ``(q, scales)`` with ``scales`` fp32 ``[rows, cols/group]``."""
    _require_gpu("x", x)
    assert x.dtype == torch.bfloat16, "x must be bfloat16"
    x = x.contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(x.shape[:-1] + (cols // group_size,), dtype=torch.float32,
                    device=x.device)
    _capi.check(
        _capi.load().fgs_moe_quant_fp8_group(
            x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, cols, group_size,
            _stream_ptr(x)),
        "per_token_group_quant_fp8",
    )
    return q, s


def per_token_quant_int8(x: torch.Tensor):
    """Dynamic per-row int8 quantisation (HIP kernel). Returns
    ``(q, scales)`` with ``scales`` fp32 ``[rows]``."""
    _require_gpu("x", x)
    assert x.dtype == torch.bfloat16, "x must be bfloat16"
    x = x.contiguous()
    cols = x.shape[-1]
    rows = x.numel() // cols
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    _capi.check(
        _capi.load().fgs_moe_quant_int8_token(
            x.data_ptr(), q.data_ptr(), s.data_ptr(), rows, cols,
            _stream_ptr(x)),
        "per_token_quant_int8",
    )
    return q, s


# -------------------------------------------------------------- fused op ---
def _check_unsupported(**flags):
    for name, value in flags.items():
        assert value is None, _UNSUPPORTED_FEATURE_MSG.format(name=name)


def _weight_qmode(w1, w2, use_fp8_w8a8, use_int8_w8a8, per_channel_quant,
                  w1_scale, w2_scale, block_shape) -> int:
    """The weights' quantisation mode from the reference's flag set, with its
    checks (w1 [E, 2N, K], w2 [E, K, N]): bf16; ``use_fp8_w8a8`` with
    ``block_shape=[128, 128]`` (e4m3fn, fp32 block scales ``[E, 2N/128,
    K/128]`` / ``[E, K/128, N/128]``); ``use_int8_w8a8`` with
    ``per_channel_quant`` (int8, fp32 ``[E, 2N]`` / ``[E, K]``)."""
    assert not (use_fp8_w8a8 and use_int8_w8a8), (
        "use_fp8_w8a8 and use_int8_w8a8 are exclusive")
    E, two_n, K = w1.shape
    N = two_n // 2
    if use_fp8_w8a8:
        assert block_shape is not None and list(block_shape) == [128, 128], (
            "use_fp8_w8a8 needs block_shape=[128, 128]")
        assert w1.dtype == torch.float8_e4m3fn and w2.dtype == torch.float8_e4m3fn, (
            "fp8 weights must be float8_e4m3fn")
        assert w1_scale is not None and w2_scale is not None, (
            "use_fp8_w8a8 needs w1_scale and w2_scale")
        assert tuple(w1_scale.shape) == (E, two_n // 128, K // 128), "w1_scale shape"
        assert tuple(w2_scale.shape) == (E, K // 128, N // 128), "w2_scale shape"
        return _capi.QMODE_FP8_BLOCK
    if use_int8_w8a8:
        assert per_channel_quant, "use_int8_w8a8 needs per_channel_quant=True"
        _check_unsupported(block_shape=block_shape)
        assert w1.dtype == torch.int8 and w2.dtype == torch.int8, (
            "int8 weights must be int8")
        assert w1_scale is not None and w2_scale is not None, (
            "use_int8_w8a8 needs w1_scale and w2_scale")
        assert w1_scale.numel() == E * two_n and w2_scale.numel() == E * K, (
            "per-channel scales must be [E, 2N] and [E, K]")
        return _capi.QMODE_INT8_CHANNEL
    assert per_channel_quant is False, _UNSUPPORTED_FEATURE_MSG.format(
        name="per_channel_quant")
    _check_unsupported(w1_scale=w1_scale, w2_scale=w2_scale, block_shape=block_shape)
    assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
    assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
    return _capi.QMODE_BF16


def fused_moe(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    use_fp8_w8a8: bool = False,
    use_int8_w8a8: bool = False,
    per_channel_quant: bool = False,
    global_num_experts: int = -1,
    expert_map: Optional[torch.Tensor] = None,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    a1_scale: Optional[torch.Tensor] = None,
    a2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[list] = None,
    routed_scaling_factor: Optional[float] = None,
    _flags: int = 0,
) -> torch.Tensor:
    """Fused MoE layer on SGLang-layout weights.

    ``hidden_states`` bf16 ``[M, K]``; ``w1`` ``[E, 2N, K]`` (gate rows then
    up rows); ``w2`` ``[E, K, N]``; ``topk_weights`` ``[M, topk]``;
    ``topk_ids`` ``[M, topk]``. Returns bf16 ``[M, K]``::

        out[t] = sum_j w[t,j] * (act(x_t W1g[e]^T) * (x_t W1u[e]^T)) W2[e]^T

    with ``act`` silu, or the exact (erf) gelu for ``activation="gelu"``
    (sgl_kernel's ``gelu_and_mul``, ops/fused_moe.py:219-220).

    Modes: bf16; ``use_fp8_w8a8`` with ``block_shape=[128, 128]`` (e4m3fn
    weights, fp32 block scales ``w1_scale [E, 2N/128, K/128]``,
    ``w2_scale [E, K/128, N/128]``, activations quantised per 1x128 group in
    the call); ``use_int8_w8a8`` with ``per_channel_quant`` (int8 weights,
    fp32 ``w1_scale [E, 2N]``, ``w2_scale [E, K]``, per-token activation
    scales computed in the call). Argument checks follow the reference
    (ops/fused_moe.py:170-195); flags that stay unsupported raise
    ``AssertionError("<name> is not supported")``.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE (gfx950)")
    _check_unsupported(expert_map=expert_map, a1_scale=a1_scale,
                       a2_scale=a2_scale)
    assert inplace is False, "Inplace is not supported"
    if activation not in ("silu", "gelu"):
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")

    assert hidden_states.ndim == 2, "hidden_states must be 2D"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    for name, t in (("hidden_states", hidden_states), ("w1", w1), ("w2", w2),
                    ("topk_weights", topk_weights), ("topk_ids", topk_ids)):
        _require_gpu(name, t)
    assert w1.ndim == 3 and w2.ndim == 3, "w1 and w2 must be 3D"
    E, two_n, K = w1.shape
    N = two_n // 2
    assert hidden_states.shape[1] == K, "hidden size mismatch"
    assert two_n == 2 * N, "w1 must hold 2*N rows"
    assert tuple(w2.shape) == (E, K, N), "intermediate size mismatch"
    M = hidden_states.shape[0]
    assert topk_ids.shape == topk_weights.shape and topk_ids.shape[0] == M, (
        "topk_ids / topk_weights must be [M, topk]")
    topk = topk_ids.shape[1]

    qmode = _weight_qmode(w1, w2, use_fp8_w8a8, use_int8_w8a8, per_channel_quant,
                          w1_scale, w2_scale, block_shape)

    lib = _capi.load()
    flags = int(_flags)
    if apply_router_weight_on_input:
        flags |= _capi.FLAG_ROUTER_WEIGHT_ON_INPUT
    if activation == "gelu":
        flags |= _capi.FLAG_ACT_GELU
    x = hidden_states.contiguous()
    w1 = w1.contiguous()
    w2 = w2.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    ws_bytes = lib.fgs_moe_workspace_bytes(M, K, N, E, topk, qmode, flags)
    if ws_bytes < 0:
        _capi.check(lib.fgs_moe_validate(M, K, N, E, topk, qmode, flags, 0),
                    "fused_moe")
    out = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=x.device)
    stream = _stream_ptr(x)
    if qmode == _capi.QMODE_BF16:
        rc = lib.fgs_moe_fused_bf16(
            x.data_ptr(), w1.data_ptr(), w2.data_ptr(), wts.data_ptr(),
            ids.data_ptr(), M, K, N, E, topk, flags, ws.data_ptr(), ws_bytes,
            out.data_ptr(), stream)
    elif qmode == _capi.QMODE_FP8_BLOCK:
        s1 = w1_scale.to(torch.float32).contiguous()
        s2 = w2_scale.to(torch.float32).contiguous()
        rc = lib.fgs_moe_fused_fp8_block(
            x.data_ptr(), w1.data_ptr(), w2.data_ptr(), s1.data_ptr(),
            s2.data_ptr(), 128, 128, wts.data_ptr(), ids.data_ptr(), M, K, N,
            E, topk, flags, ws.data_ptr(), ws_bytes, out.data_ptr(), stream)
    else:
        s1 = w1_scale.to(torch.float32).contiguous()
        s2 = w2_scale.to(torch.float32).contiguous()
        rc = lib.fgs_moe_fused_int8_channel(
            x.data_ptr(), w1.data_ptr(), w2.data_ptr(), s1.data_ptr(),
            s2.data_ptr(), wts.data_ptr(), ids.data_ptr(), M, K, N, E, topk,
            flags, ws.data_ptr(), ws_bytes, out.data_ptr(), stream)
    _capi.check(rc, "fused_moe")
    if routed_scaling_factor is not None and routed_scaling_factor != 1.0:
        out.mul_(routed_scaling_factor)
    return out


def _fused_routed(hidden_states, w1, w2, routing_data, gather_indx, *,
                  qmode=None, w1_scale=None, w2_scale=None, b1=None, b2=None,
                  alpha=1.0, limit=0.0, activation="silu",
                  apply_router_weight_on_input=False, _flags=0):
    """One fused call on the routing tuple (``fgs_moe_fused_routed``):
    SGLang-layout weights ``w1 [E, 2N, K]`` (gate rows then up / linear
    rows), ``w2 [E, K, N]``; the tuple's gathered order is the GEMMs' row
    order (no top-k reconstruction, no second alignment). ``b1`` / ``b2``
    (both or neither) select the bias variant with swiglu(alpha, limit)."""
    for name, t in (("hidden_states", hidden_states), ("w1", w1), ("w2", w2)):
        _require_gpu(name, t)
    M, K = hidden_states.shape
    E, two_n, Kw = w1.shape
    N = two_n // 2
    assert Kw == K, "hidden size mismatch"
    assert tuple(w2.shape) == (E, K, N), "intermediate size mismatch"
    gate, src, hist, topk, E_r = _routing_args(routing_data, gather_indx, M)
    assert E_r == E, "routing_data.expt_hist must hold one count per expert"
    if qmode is None:
        qmode = _capi.QMODE_BF16
    lib = _capi.load()
    flags = int(_flags)
    if apply_router_weight_on_input:
        flags |= _capi.FLAG_ROUTER_WEIGHT_ON_INPUT
    if activation == "gelu":
        flags |= _capi.FLAG_ACT_GELU
    x = hidden_states.contiguous()
    w1 = w1.contiguous()
    w2 = w2.contiguous()
    ws_bytes = lib.fgs_moe_workspace_bytes(M, K, N, E, topk, qmode, flags)
    if ws_bytes < 0:
        _capi.check(lib.fgs_moe_validate(M, K, N, E, topk, qmode, flags, 0),
                    "fused_moe (routing tuple)")
    out = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=x.device)
    s1 = s2 = None
    if qmode != _capi.QMODE_BF16:
        s1 = w1_scale.to(torch.float32).contiguous()
        s2 = w2_scale.to(torch.float32).contiguous()
    b1f = b2f = None
    if b1 is not None or b2 is not None:
        assert b1 is not None and b2 is not None, (
            "Bias execution requires both w13_bias and w2_bias")
        assert tuple(b1.shape) == (E, two_n) and tuple(b2.shape) == (E, K), (
            "b1 must be [E, 2N] and b2 [E, K]")
        b1f = b1.to(torch.float32).contiguous()
        b2f = b2.to(torch.float32).contiguous()

    def ptr(t):
        return None if t is None else t.data_ptr()

    _capi.check(
        lib.fgs_moe_fused_routed(
            qmode, x.data_ptr(), w1.data_ptr(), w2.data_ptr(), ptr(s1), ptr(s2),
            ptr(b1f), ptr(b2f), float(alpha), float(limit), gate.data_ptr(),
            src.data_ptr(), hist.data_ptr(), M, K, N, E, topk, flags, ws.data_ptr(),
            ws_bytes, out.data_ptr(), _stream_ptr(x)),
        "fused_moe (routing tuple)",
    )
    return out


# ``[E, A, B] -> [E, B, A]`` contiguous, once per weight (the reference
# plugin transposes both weights on every call, ops/fused_moe.py:342-343).
# A weight passed as a transposed view of a native-layout tensor converts
# for free.
_native_layout = _ConversionCache(lambda t: t.transpose(-1, -2).contiguous())


def clear_weight_cache() -> None:
    """Drop every cached weight conversion (the reference-layout transposes
    and the de-interleaved bias-variant weights). Call it after updating
    weights in place through ``param.data`` (``param.data.copy_(...)``),
    which the caches cannot detect; updates through the tensor itself and
    reassignments of ``param.data`` are detected."""
    for cache in (_native_layout, _deinterleaved, _transposed_deinterleaved):
        cache.clear()


def triton_kernel_fused_experts(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    routing_data,
    gather_indx,
    scatter_indx,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    use_fp8_w8a8: bool = False,
    per_channel_quant: bool = False,
    global_num_experts: int = -1,
    expert_map: Optional[torch.Tensor] = None,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    a1_scale: Optional[torch.Tensor] = None,
    a2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[list] = None,
) -> torch.Tensor:
    """Drop-in for the reference's ``triton_kernel_fused_experts``
    (ops/fused_moe.py:149-232): same signature, same argument checks
    (:170-195), reference weight layout ``w1 [E, K, 2N]``, ``w2 [E, N, K]``
    and routing in the reference's format (``routing_data.gate_scal``,
    ``.expt_hist``, ``.n_expts_act``; ``gather_indx.src_indx``).

    ``scatter_indx=None`` (the adapter's ``no_combine``, :371) returns the
    un-combined ``[M * topk, K]`` rows token-major, a token's slots in
    ascending expert id (the routing tuple's order): row ``(t, r)`` is
    ``bf16(w * y)`` of token t's r-th slot. The reference's own row order
    for this case is not observable -- it ends in ``.view(num_tokens,
    hidden_size)`` (:232), which cannot hold ``M * topk`` rows -- so the
    order is parity-unpinned.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE (gfx950)")
    assert use_fp8_w8a8 is False, _UNSUPPORTED_FEATURE_MSG.format(
        name="use_fp8_w8a8")
    assert per_channel_quant is False, _UNSUPPORTED_FEATURE_MSG.format(
        name="per_channel_quant")
    _check_unsupported(expert_map=expert_map, w1_scale=w1_scale,
                       w2_scale=w2_scale, a1_scale=a1_scale, a2_scale=a2_scale,
                       block_shape=block_shape)
    assert inplace is False, "Inplace is not supported"
    assert hidden_states.ndim == 2, "hidden_states must be 2D"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
    assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
    assert hidden_states.shape[-1] == w1.shape[-2], "hidden size mismatch"
    assert w2.shape[-1] == w1.shape[1], "intermediate size mismatch"
    if activation not in ("silu", "gelu"):
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")

    num_tokens, hidden = hidden_states.shape
    w13n = _native_layout(w1)
    w2n = _native_layout(w2)
    if scatter_indx is not None:
        out = _fused_routed(hidden_states, w13n, w2n, routing_data, gather_indx,
                            activation=activation,
                            apply_router_weight_on_input=apply_router_weight_on_input)
        return out.view(num_tokens, hidden)
    # No combine: one row per (token, slot) in the gate (row-sorted) order.
    topk_weights, topk_ids = _routing_to_topk(routing_data, gather_indx,
                                              num_tokens)
    return _uncombined(
        lambda x, tw, ti: fused_moe(
            x, w13n, w2n, tw, ti, activation=activation,
            apply_router_weight_on_input=apply_router_weight_on_input),
        hidden_states, topk_weights, topk_ids)


def _deinterleave_rows(w: torch.Tensor) -> torch.Tensor:
    """Rows ``[g0, u0, g1, u1, ...]`` (dim -2 of ``[E, 2N, K]``, or the last
    dim of a bias ``[E, 2N]``) -> ``[g0..g(N-1), u0..u(N-1)]``."""
    if w.ndim == 2:
        return torch.cat([w[:, 0::2], w[:, 1::2]], dim=1).contiguous()
    return torch.cat([w[:, 0::2, :], w[:, 1::2, :]], dim=1).contiguous()


# interleaved gate/linear weights -> the kernels' [gate block | up block]
# rows, once per weight: native layout, and the reference's [E, K, 2N]
_deinterleaved = _ConversionCache(_deinterleave_rows)
_transposed_deinterleaved = _ConversionCache(
    lambda w: _deinterleave_rows(w.transpose(-1, -2)))


def fused_moe_with_bias(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    b1: torch.Tensor,
    w2: torch.Tensor,
    b2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    apply_router_weight_on_input: bool = False,
    gemm1_alpha: Optional[float] = None,
    gemm1_clamp_limit: Optional[float] = None,
    interleaved: bool = True,
    routed_scaling_factor: Optional[float] = None,
    use_fp8_w8a8: bool = False,
    use_int8_w8a8: bool = False,
    per_channel_quant: bool = False,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[list] = None,
    _flags: int = 0,
) -> torch.Tensor:
    """Fused MoE with biases and the swiglu activation on SGLang-layout
    weights (the computation of ``triton_kernel_fused_experts_with_bias``,
    ops/fused_moe.py:235-325).

    ``w1`` bf16 ``[E, 2N, K]`` with gate and linear rows interleaved
    (``interleaved=True``, the layout matmul_ogs's fused swiglu reads) or
    gate rows then linear rows; ``b1`` ``[E, 2N]`` in the same order;
    ``w2`` ``[E, K, N]``; ``b2`` ``[E, K]``. Per slot::

        g = x W1g^T + b1g;  u = x W1u^T + b1u
        g = min(g, limit);  u = clamp(u, -limit, limit)   (when limit given)
        a = bf16(g * sigmoid(alpha * g) * (u + 1))
        y = bf16(a W2^T + b2);  out = bf16(sum_j w_j * y_j)

    ``gemm1_alpha`` defaults to 1.0 and no clamp is applied without
    ``gemm1_clamp_limit``. With ``apply_router_weight_on_input`` the router
    weight multiplies ``a`` before its bf16 rounding (matmul_ogs applies its
    gammas to the fused activation's output) and ``y`` is not weighted.

    Quantised weights (the reference's ``w1_pcg`` / ``w2_pcg``) take the
    flags and scales of ``fused_moe``: ``use_fp8_w8a8`` with 128x128 block
    scales (gate rows then linear rows only, ``interleaved=False``: the
    reference's interleaved rows would split every 128-row scale block
    between gate and linear rows), or ``use_int8_w8a8`` with per-channel
    scales (``w1_scale [E, 2N]`` in the same row order as ``w1``, so it is
    de-interleaved with it); the biases add to the dequantised outputs.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE_WITH_BIAS (gfx950)")
    assert hidden_states.ndim == 2, "hidden_states must be 2D"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    for name, t in (("hidden_states", hidden_states), ("w1", w1), ("b1", b1),
                    ("w2", w2), ("b2", b2), ("topk_weights", topk_weights),
                    ("topk_ids", topk_ids)):
        _require_gpu(name, t)
    E, two_n, K = w1.shape
    N = two_n // 2
    assert hidden_states.shape[1] == K, "hidden size mismatch"
    assert tuple(w2.shape) == (E, K, N), "intermediate size mismatch"
    assert tuple(b1.shape) == (E, two_n) and tuple(b2.shape) == (E, K), (
        "b1 must be [E, 2N] and b2 [E, K]")
    qmode = _weight_qmode(w1, w2, use_fp8_w8a8, use_int8_w8a8, per_channel_quant,
                          w1_scale, w2_scale, block_shape)
    if qmode == _capi.QMODE_FP8_BLOCK and interleaved:
        raise NotImplementedError(
            "fp8 block scales need w1's gate rows then linear rows (interleaved=False)")
    M = hidden_states.shape[0]
    assert topk_ids.shape == topk_weights.shape and topk_ids.shape[0] == M, (
        "topk_ids / topk_weights must be [M, topk]")
    topk = topk_ids.shape[1]
    if interleaved:
        w1 = _deinterleaved(w1)
        b1 = _deinterleave_rows(b1)
        if qmode == _capi.QMODE_INT8_CHANNEL:
            w1_scale = _deinterleave_rows(w1_scale.reshape(E, two_n))
    alpha = 1.0 if gemm1_alpha is None else float(gemm1_alpha)
    limit = 0.0 if gemm1_clamp_limit is None else float(gemm1_clamp_limit)

    lib = _capi.load()
    flags = int(_flags)
    if apply_router_weight_on_input:
        flags |= _capi.FLAG_ROUTER_WEIGHT_ON_INPUT
    x = hidden_states.contiguous()
    w1 = w1.contiguous()
    w2 = w2.contiguous()
    b1f = b1.to(torch.float32).contiguous()
    b2f = b2.to(torch.float32).contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    ws_bytes = lib.fgs_moe_workspace_bytes(M, K, N, E, topk, qmode, flags)
    if ws_bytes < 0:
        _capi.check(lib.fgs_moe_validate(M, K, N, E, topk, qmode, flags, 0),
                    "fused_moe_with_bias")
    out = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=x.device)
    if qmode == _capi.QMODE_BF16:
        rc = lib.fgs_moe_fused_bf16_bias(
            x.data_ptr(), w1.data_ptr(), b1f.data_ptr(), w2.data_ptr(),
            b2f.data_ptr(), wts.data_ptr(), ids.data_ptr(), M, K, N, E, topk, flags,
            alpha, limit, ws.data_ptr(), ws_bytes, out.data_ptr(), _stream_ptr(x))
    else:
        s1 = w1_scale.to(torch.float32).contiguous()
        s2 = w2_scale.to(torch.float32).contiguous()
        rc = lib.fgs_moe_fused_quant_bias(
            qmode, x.data_ptr(), w1.data_ptr(), b1f.data_ptr(), w2.data_ptr(),
            b2f.data_ptr(), s1.data_ptr(), s2.data_ptr(), wts.data_ptr(),
            ids.data_ptr(), M, K, N, E, topk, flags, alpha, limit, ws.data_ptr(),
            ws_bytes, out.data_ptr(), _stream_ptr(x))
    _capi.check(rc, "fused_moe_with_bias")
    if routed_scaling_factor is not None and routed_scaling_factor != 1.0:
        out.mul_(routed_scaling_factor)
    return out


def _uncombined(fn, hidden_states, topk_weights, topk_ids, **kw):
    """One output row per (token, slot), token-major, slots in the routing
    order: the op on each token repeated topk times with one slot each."""
    top_k = topk_ids.shape[1]
    rep_x = hidden_states.repeat_interleave(top_k, dim=0)
    return fn(rep_x, topk_weights.reshape(-1, 1), topk_ids.reshape(-1, 1), **kw)


def triton_kernel_fused_experts_with_bias(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w1_pcg,
    b1: torch.Tensor,
    w2: torch.Tensor,
    w2_pcg,
    b2: torch.Tensor,
    routing_data,
    gather_indx,
    scatter_indx,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    global_num_experts: int = -1,
    gemm1_alpha: Optional[float] = None,
    gemm1_clamp_limit: Optional[float] = None,
) -> torch.Tensor:
    """Drop-in for the reference's ``triton_kernel_fused_experts_with_bias``
    (ops/fused_moe.py:235-325): same signature and checks, reference layout
    ``w1 [E, K, 2N]`` with interleaved gate/linear columns, ``b1 [E, 2N]``,
    ``w2 [E, N, K]``, ``b2 [E, K]``, reference routing format. The
    precision configs (``w1_pcg`` / ``w2_pcg``) matter for quantised weights:
    int8 ``w1`` / ``w2`` take per-output-column fp32 scales from their
    ``weight_scale`` (``[E, 2N]`` in w1's interleaved column order, ``[E,
    K]``); for bf16 weights they are accepted and ignored. fp8 block scales
    cannot follow the interleaved gate/linear columns (each 128-column block
    holds both), so fp8 weights go through ``fused_moe_with_bias``.
    ``scatter_indx=None`` returns un-combined rows.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE_WITH_BIAS (gfx950)")
    assert inplace is False, "Inplace is not supported"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    if activation != "silu":
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")
    if w1.dtype == torch.float8_e4m3fn or w2.dtype == torch.float8_e4m3fn:
        raise NotImplementedError(
            "fp8 block scales do not follow the interleaved gate/linear columns; "
            "use fused_moe_with_bias with gate rows then linear rows")
    quant = {}
    if w1.dtype == torch.int8 or w2.dtype == torch.int8:
        assert w1.dtype == torch.int8 and w2.dtype == torch.int8, (
            "w1 and w2 must both be int8")
        s1 = getattr(w1_pcg, "weight_scale", None)
        s2 = getattr(w2_pcg, "weight_scale", None)
        assert s1 is not None and s2 is not None, (
            "int8 weights need w1_pcg.weight_scale and w2_pcg.weight_scale")
        E, two_n = w1.shape[0], w1.shape[2]
        quant = dict(use_int8_w8a8=True, per_channel_quant=True,
                     w1_scale=_deinterleave_rows(s1.reshape(E, two_n)),
                     w2_scale=s2)
    else:
        assert w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16, (
            "w1 and w2 must be bfloat16 or int8")
    num_tokens, hidden = hidden_states.shape
    w13n = _transposed_deinterleaved(w1)
    b1n = _deinterleave_rows(b1)
    w2n = _native_layout(w2)
    if scatter_indx is not None:
        out = _fused_routed(
            hidden_states, w13n, w2n, routing_data, gather_indx,
            qmode=_capi.QMODE_INT8_CHANNEL if quant else _capi.QMODE_BF16,
            w1_scale=quant.get("w1_scale"), w2_scale=quant.get("w2_scale"),
            b1=b1n, b2=b2,
            alpha=1.0 if gemm1_alpha is None else float(gemm1_alpha),
            limit=0.0 if gemm1_clamp_limit is None else float(gemm1_clamp_limit),
            apply_router_weight_on_input=apply_router_weight_on_input)
        return out.view(num_tokens, hidden)
    kw = dict(apply_router_weight_on_input=apply_router_weight_on_input,
              gemm1_alpha=gemm1_alpha, gemm1_clamp_limit=gemm1_clamp_limit,
              interleaved=False, **quant)

    def call(x, tw, ti, **k):
        return fused_moe_with_bias(x, w13n, b1n, w2n, b2, tw, ti, **k)

    topk_weights, topk_ids = _routing_to_topk(routing_data, gather_indx,
                                              num_tokens)
    return _uncombined(call, hidden_states, topk_weights, topk_ids, **kw)


@dataclass
class StandardCombineInput:
    """Stand-in for SGLang's ``StandardCombineInput`` (the adapter's return
    type, ops/fused_moe.py:422) when SGLang is not installed."""

    hidden_states: torch.Tensor


def _combine_input_cls():
    try:
        from sglang.srt.layers.moe.token_dispatcher.standard import (
            StandardCombineInput as cls,
        )
        return cls
    except Exception:
        return StandardCombineInput


def fused_moe_flagos(obj, layer, dispatch_output):
    """SGLang runner adapter (the reference's ``fused_moe_flagos``,
    ops/fused_moe.py:328-422) on native-layout weights: ``layer.w13_weight``
    ``[E, 2N, K]`` and ``layer.w2_weight`` ``[E, K, N]`` are used as they are
    (the reference transposes both on every call, :342-343).

    Reads ``obj.runner.config`` (``num_experts``, ``activation``,
    ``apply_router_weight_on_input``, ``no_combine``,
    ``routed_scaling_factor``, ``gemm1_alpha``, ``gemm1_clamp_limit``),
    optional ``layer.w13_weight_bias`` / ``layer.w2_weight_bias`` (both or
    neither: the bias variant with interleaved gate/linear rows), and
    ``dispatch_output.hidden_states`` / ``.topk_output`` (standard
    ``topk_weights`` / ``topk_ids`` or the triton-kernels routing tuple).
    ``no_combine`` returns ``[tokens, topk, hidden]``; the routed scaling
    factor applies to combined outputs only (:408-420).
    """
    cfg = obj.runner.config
    hidden_states = dispatch_output.hidden_states
    topk_output = dispatch_output.topk_output
    routing = None
    if isinstance(topk_output, (tuple, list)) and len(topk_output) == 3 and \
            hasattr(topk_output[0], "gate_scal"):
        routing = topk_output[:2]  # (routing_data, gather_indx)
        topk_weights = topk_ids = None
    else:
        topk_weights, topk_ids = topk_output.topk_weights, topk_output.topk_ids
    no_combine = bool(getattr(cfg, "no_combine", False))
    on_input = bool(getattr(cfg, "apply_router_weight_on_input", False))
    activation = getattr(cfg, "activation", "silu")
    b13 = getattr(layer, "w13_weight_bias", None)
    b2 = getattr(layer, "w2_weight_bias", None)
    if b13 is not None or b2 is not None:
        assert b13 is not None and b2 is not None, (
            "Bias execution requires both w13_bias and w2_bias")
        if activation != "silu":
            raise ValueError(f"Unsupported FusedMoe activation: {activation}")
        w13 = _deinterleaved(layer.w13_weight)
        b13n = _deinterleave_rows(b13)
        alpha = getattr(cfg, "gemm1_alpha", None)
        limit = getattr(cfg, "gemm1_clamp_limit", None)

        def call(x, tw, ti):
            return fused_moe_with_bias(
                x, w13, b13n, layer.w2_weight, b2, tw, ti,
                apply_router_weight_on_input=on_input, gemm1_alpha=alpha,
                gemm1_clamp_limit=limit, interleaved=False)

        def call_routed(x):
            return _fused_routed(
                x, w13, layer.w2_weight, *routing, b1=b13n, b2=b2,
                alpha=1.0 if alpha is None else float(alpha),
                limit=0.0 if limit is None else float(limit),
                apply_router_weight_on_input=on_input)
    else:
        def call(x, tw, ti):
            return fused_moe(x, layer.w13_weight, layer.w2_weight, tw, ti,
                             activation=activation,
                             apply_router_weight_on_input=on_input)

        def call_routed(x):
            return _fused_routed(x, layer.w13_weight, layer.w2_weight, *routing,
                                 activation=activation,
                                 apply_router_weight_on_input=on_input)
    if no_combine:
        if routing is not None:
            topk_weights, topk_ids = _routing_to_topk(*routing, hidden_states.shape[0])
        rows = _uncombined(call, hidden_states, topk_weights, topk_ids)
        output = rows.view(hidden_states.shape[0], topk_ids.shape[1],
                           hidden_states.shape[-1])
    else:
        if routing is not None:
            output = call_routed(hidden_states)
        else:
            output = call(hidden_states, topk_weights, topk_ids)
        scale = getattr(cfg, "routed_scaling_factor", None)
        if scale is not None and scale != 1.0:
            output.mul_(scale)
    return _combine_input_cls()(hidden_states=output)


__all__ = [
    "fused_topk",
    "fused_moe",
    "fused_moe_with_bias",
    "fused_moe_flagos",
    "triton_kernel_fused_experts",
    "triton_kernel_fused_experts_with_bias",
    "moe_align_block_size",
    "silu_and_mul",
    "moe_sum",
    "per_token_group_quant_fp8",
    "per_token_quant_int8",
    "standard_topk_to_routing",
]
