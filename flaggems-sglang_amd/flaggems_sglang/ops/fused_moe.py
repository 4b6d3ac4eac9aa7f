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


# --------------------------------------------------------------- routing ---
@dataclass
class RoutingData:
    """Duck-typed stand-in for ``triton_kernels.routing.RoutingData`` with the
    fields the reference reads (ops/fused_moe.py:141-143, 200-201)."""

    gate_scal: torch.Tensor
    expt_hist: torch.Tensor
    n_expts_tot: int
    n_expts_act: int
    expt_data: object = None


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
    ScatterIndx)`` in the reference's routing format.

    Follows ``_standard_topk_to_triton_kernels`` (ops/fused_moe.py:119-146):
    per-token ascending sort of the ids carrying the weights (:130-131), stable
    argsort of the flattened ids (:134) and its inverse (:135), gathered gate
    scales (:136) and the per-expert histogram (:137-139). The block metadata
    of ``compute_expt_data_torch`` (:140) belongs to ``triton_kernels`` and is
    not produced (``expt_data=None``); nothing in this package reads it.
    """
    expt_indx_2d, sort_indices = torch.sort(topk_ids, dim=1)
    expt_scal = torch.gather(topk_weights, 1, sort_indices).reshape(-1)
    expt_indx = expt_indx_2d.reshape(-1).to(torch.int32)
    topk_indx = torch.argsort(expt_indx, stable=True).to(torch.int32)
    gate_indx = torch.argsort(topk_indx, stable=True).to(torch.int32)
    gate_scal = expt_scal[topk_indx.long()]
    hist = torch.bincount(expt_indx.long(), minlength=n_expts_tot)[
        :n_expts_tot
    ].to(torch.int32)
    routing = RoutingData(gate_scal, hist, n_expts_tot, topk_ids.shape[1])
    return (
        routing,
        GatherIndx(src_indx=topk_indx, dst_indx=gate_indx),
        ScatterIndx(src_indx=gate_indx, dst_indx=topk_indx),
    )


def _routing_to_topk(routing_data, gather_indx, num_tokens):
    """Inverse of :func:`standard_topk_to_routing`: rebuild per-token
    ``(topk_weights, topk_ids)`` (ids ascending within a token, the order the
    reference's conversion produces at ops/fused_moe.py:130)."""
    top_k = int(routing_data.n_expts_act)
    hist = routing_data.expt_hist.to(torch.int64)
    src = gather_indx.src_indx.to(torch.int64)
    n = num_tokens * top_k
    expert_of_pos = torch.repeat_interleave(
        torch.arange(hist.numel(), device=hist.device), hist, output_size=n
    )
    ids = torch.empty(n, dtype=torch.int32, device=src.device)
    wts = torch.empty(n, dtype=torch.float32, device=src.device)
    ids[src] = expert_of_pos.to(torch.int32)
    wts[src] = routing_data.gate_scal.to(torch.float32)
    return wts.view(num_tokens, top_k), ids.view(num_tokens, top_k)


# ------------------------------------------------------------ small ops ---
def moe_align_block_size(topk_ids: torch.Tensor, num_experts: int,
                         block_size: int):
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
    _capi.check(
        lib.fgs_moe_align_block_size(
            ids.data_ptr(), numel, num_experts, block_size,
            sorted_ids.data_ptr(), expert_ids.data_ptr(), npp.data_ptr(),
            max_padded, _stream_ptr(ids)),
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

        out[t] = sum_j w[t,j] * (silu(x_t W1g[e]^T) * (x_t W1u[e]^T)) W2[e]^T

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
    if activation != "silu":
        if activation == "gelu":
            raise NotImplementedError("activation='gelu' is not implemented")
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")
    assert not (use_fp8_w8a8 and use_int8_w8a8), (
        "use_fp8_w8a8 and use_int8_w8a8 are exclusive")

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

    if use_fp8_w8a8:
        assert block_shape is not None and list(block_shape) == [128, 128], (
            "use_fp8_w8a8 needs block_shape=[128, 128]")
        assert w1.dtype == torch.float8_e4m3fn and w2.dtype == torch.float8_e4m3fn, (
            "fp8 weights must be float8_e4m3fn")
        assert w1_scale is not None and w2_scale is not None, (
            "use_fp8_w8a8 needs w1_scale and w2_scale")
        assert tuple(w1_scale.shape) == (E, two_n // 128, K // 128), "w1_scale shape"
        assert tuple(w2_scale.shape) == (E, K // 128, N // 128), "w2_scale shape"
        qmode = _capi.QMODE_FP8_BLOCK
    elif use_int8_w8a8:
        assert per_channel_quant, "use_int8_w8a8 needs per_channel_quant=True"
        _check_unsupported(block_shape=block_shape)
        assert w1.dtype == torch.int8 and w2.dtype == torch.int8, (
            "int8 weights must be int8")
        assert w1_scale is not None and w2_scale is not None, (
            "use_int8_w8a8 needs w1_scale and w2_scale")
        assert w1_scale.numel() == E * two_n and w2_scale.numel() == E * K, (
            "per-channel scales must be [E, 2N] and [E, K]")
        qmode = _capi.QMODE_INT8_CHANNEL
    else:
        assert per_channel_quant is False, _UNSUPPORTED_FEATURE_MSG.format(
            name="per_channel_quant")
        _check_unsupported(w1_scale=w1_scale, w2_scale=w2_scale,
                           block_shape=block_shape)
        assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
        assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
        qmode = _capi.QMODE_BF16

    lib = _capi.load()
    flags = int(_flags)
    if apply_router_weight_on_input:
        flags |= _capi.FLAG_ROUTER_WEIGHT_ON_INPUT
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


_TRANSPOSE_CACHE: dict = {}


def _native_layout(w: torch.Tensor) -> torch.Tensor:
    """``[E, A, B] -> [E, B, A]`` contiguous, cached per weight version so a
    model's weights are transposed once, not on every call (the reference
    plugin transposes on every call, ops/fused_moe.py:342-343)."""
    key = (w.data_ptr(), w._version, tuple(w.shape), tuple(w.stride()), w.dtype)
    hit = _TRANSPOSE_CACHE.get(key)
    if hit is None:
        if len(_TRANSPOSE_CACHE) > 64:
            _TRANSPOSE_CACHE.clear()
        hit = w.transpose(-1, -2).contiguous()
        _TRANSPOSE_CACHE[key] = hit
    return hit


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

    ``scatter_indx=None`` returns the un-combined ``[M * topk, K]`` rows in
    the reference's gate order (the ``no_combine`` case of :371).
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
    topk_weights, topk_ids = _routing_to_topk(routing_data, gather_indx,
                                              num_tokens)
    w13n = _native_layout(w1)
    w2n = _native_layout(w2)
    if scatter_indx is not None:
        out = fused_moe(hidden_states, w13n, w2n, topk_weights, topk_ids,
                        activation=activation,
                        apply_router_weight_on_input=apply_router_weight_on_input)
        return out.view(num_tokens, hidden)
    # No combine: one row per (token, slot) in the gate (row-sorted) order.
    top_k = topk_ids.shape[1]
    rep_x = hidden_states.repeat_interleave(top_k, dim=0)
    flat_ids = topk_ids.reshape(-1, 1)
    flat_w = topk_weights.reshape(-1, 1)
    return fused_moe(rep_x, w13n, w2n, flat_w, flat_ids, activation=activation,
                     apply_router_weight_on_input=apply_router_weight_on_input)


__all__ = [
    "fused_moe",
    "triton_kernel_fused_experts",
    "moe_align_block_size",
    "silu_and_mul",
    "moe_sum",
    "per_token_group_quant_fp8",
    "per_token_quant_int8",
    "standard_topk_to_routing",
]
