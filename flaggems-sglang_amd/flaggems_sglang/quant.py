"""Offline weight preparation for the quantised fused-MoE modes.

These run once per model load (torch ops on whatever device the weights
live on), not per forward call. The layouts are the ones the fused kernels
read (include/fgs_moe.h):

* fp8 w8a8: e4m3fn weights ``[E, R, C]`` with fp32 scales
  ``[E, R/128, C/128]`` per 128x128 block, ``scale = max(amax, 1e-10)/448``;
* int8 w8a8: int8 weights ``[E, R, C]`` with fp32 scales ``[E, R]`` per
  output channel, ``scale = max(amax, 1e-10)/127``, round half to even.

The reference has no quantised path (src/flaggems_sglang/ops/fused_moe.py:
170-185 rejects every quantisation flag), so these layouts follow SGLang's
block-fp8 and channel-int8 MoE weight formats.
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0
INT8_MAX = 127.0
EPS = 1e-10


@torch.no_grad()
def quantize_fp8_block(w: torch.Tensor, block: int = 128):
    """``[E, R, C]`` float -> (e4m3fn ``[E, R, C]``, fp32 ``[E, R/b, C/b]``).
    Processed one expert at a time to bound temporary memory."""
    E, R, C = w.shape
    assert R % block == 0 and C % block == 0, "dims must be multiples of block"
    q = torch.empty((E, R, C), dtype=torch.float8_e4m3fn, device=w.device)
    s = torch.empty((E, R // block, C // block), dtype=torch.float32,
                    device=w.device)
    for e in range(E):
        wb = w[e].float().reshape(R // block, block, C // block, block)
        amax = wb.abs().amax(dim=(1, 3))
        scale = torch.clamp(amax, min=EPS) / FP8_MAX
        qe = torch.clamp(wb / scale[:, None, :, None], -FP8_MAX, FP8_MAX)
        q[e] = qe.to(torch.float8_e4m3fn).reshape(R, C)
        s[e] = scale
    return q, s


@torch.no_grad()
def quantize_int8_channel(w: torch.Tensor):
    """``[E, R, C]`` float -> (int8 ``[E, R, C]``, fp32 ``[E, R]``)."""
    E, R, C = w.shape
    q = torch.empty((E, R, C), dtype=torch.int8, device=w.device)
    s = torch.empty((E, R), dtype=torch.float32, device=w.device)
    for e in range(E):
        wf = w[e].float()
        scale = torch.clamp(wf.abs().amax(dim=-1), min=EPS) / INT8_MAX
        qe = torch.clamp(torch.round(wf / scale[:, None]), -INT8_MAX, INT8_MAX)
        q[e] = qe.to(torch.int8)
        s[e] = scale
    return q, s
