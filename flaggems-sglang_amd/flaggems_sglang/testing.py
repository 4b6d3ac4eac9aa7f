"""Benchmark / test configurations and seeded synthetic inputs.

The shapes are the reference's own fused-MoE test and benchmark shapes
(tests/accuracy_utils.py:114-131, benchmark/attri_util.py:62-70) and the
five layer configurations this port is measured on. Inputs are generated on
the target device with a seeded ``torch.Generator`` (seed convention
``M + K + N + E + topk`` of the reference's tests/test_fused_moe.py:66);
weights use a seed independent of M so one weight set serves a whole sweep.
"""

from __future__ import annotations

import dataclasses
from typing import List, Optional

import torch

from flaggems_sglang import quant


@dataclasses.dataclass(frozen=True)
class MoEConfig:
    name: str
    K: int            # hidden size
    N: int            # per-expert intermediate size
    E: int            # experts
    topk: int
    Ms: tuple         # token counts of the sweep
    mode: str = "bf16"          # "bf16" | "fp8" | "int8"
    scoring: str = "softmax"    # router: "softmax" | "sigmoid"
    w_scale: float = 0.02
    hot_experts: tuple = ()     # experts whose logits get +hot_bias
    hot_bias: float = 0.0


CONFIGS = {
    "small": MoEConfig("small", 1024, 512, 8, 2, (64,)),
    "mixtral": MoEConfig("mixtral", 4096, 14336, 8, 2, (1, 8, 32, 128, 512, 4096)),
    "qwen3": MoEConfig("qwen3", 2048, 768, 128, 8, (1, 16, 256, 2048, 8192)),
    "qwen3_skewed": MoEConfig("qwen3_skewed", 2048, 768, 128, 8,
                              (1, 16, 256, 2048, 8192),
                              hot_experts=(3, 17, 31, 45, 59, 73, 87, 101),
                              hot_bias=2.0),
    "deepseek_fp8": MoEConfig("deepseek_fp8", 7168, 2048, 256, 8,
                              (1, 32, 512, 4096), mode="fp8",
                              scoring="sigmoid"),
    "qwen2_int8": MoEConfig("qwen2_int8", 3584, 2560, 64, 8,
                            (1, 64, 1024, 8192), mode="int8"),
    # the reference's own benchmark (benchmark/test_fused_moe.py:53-73 over
    # benchmark/attri_util.py:62-70): triton_kernel_fused_experts on the
    # routing tuple, weights randn * 0.1 in the reference layout
    "ref_bench": MoEConfig("ref_bench", 1280, 3072, 64, 8,
                           (1, 4, 17, 64, 1024, 2048, 4096), w_scale=0.1),
}

# Reference test shapes (M, K, N, E, topk): tests/accuracy_utils.py:114-131.
REF_SHAPES_SMALL = [(1, 128, 256, 8, 2), (7, 128, 256, 8, 2),
                    (33, 256, 512, 16, 4)]
REF_SHAPES_LARGE = [(m, 1280, 3072, 64, 8) for m in (1, 4, 17, 64, 1024, 2048, 4096)]

# Parity tolerances: |res - ref| <= atol + rtol*|ref| and
# sum|res - ref| / sum|ref| <= mean_rel.
TOL = {
    "bf16": dict(atol=2e-2, rtol=1e-2, mean_rel=1e-2),
    "fp8": dict(atol=5e-2, rtol=2e-2, mean_rel=5e-2),
    "int8": dict(atol=5e-2, rtol=2e-2, mean_rel=5e-2),
}

# Regression bounds of the parity tests, set from the errors measured on
# MI355X over every parity case of the mode: mean_rel (worst measured:
# bf16 2.2e-4 on a single token, <= 4e-5 for 90 % of the cases; fp8 2.5e-3;
# int8 4.2e-5) and the elementwise error in bf16 ulps of the summed terms'
# magnitude (worst measured: bf16 11 on one-term uncombined rows, 2 for
# 90 % of the cases; fp8 1.03; int8 0.5). They catch plausible kernel bugs
# the tolerance contract above lets through: one fp8 activation scale 2 %
# off among 56 k blocks fails them
# (tests/test_oracle.py::test_regression_bound_rejects_one_wrong_scale).
REGRESSION = {
    "bf16": dict(mean_rel=1e-3, ulp_mag=32.0),
    "fp8": dict(mean_rel=1e-2, ulp_mag=4.0),
    "int8": dict(mean_rel=1e-3, ulp_mag=4.0),
}


def ulp_bf16(v: torch.Tensor) -> torch.Tensor:
    """bf16 unit in the last place of |v| (8 significant bits)."""
    v = v.abs().clamp(min=2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(v)) - 7)


def regression_stats(res: torch.Tensor, ref: torch.Tensor,
                     mag: Optional[torch.Tensor] = None) -> dict:
    """max-abs, max error in ulps of |ref| and of the term magnitude ``mag``
    (|ref| when absent), and mean_rel = sum|res - ref| / sum|ref|."""
    r, f = res.float().cpu(), ref.float().cpu()
    diff = (r - f).abs()
    if diff.numel() == 0:
        return dict(max_abs=0.0, max_ulp_ref=0.0, max_ulp_mag=0.0, mean_rel=0.0)
    s = f.abs() if mag is None else mag.float().cpu()
    return dict(max_abs=float(diff.max()),
                max_ulp_ref=float((diff / ulp_bf16(f)).max()),
                max_ulp_mag=float((diff / ulp_bf16(s)).max()),
                mean_rel=float(diff.sum() / f.abs().sum().clamp(min=1e-30)))


@dataclasses.dataclass
class MoEWeights:
    w1: torch.Tensor
    w2: torch.Tensor
    w1_scale: Optional[torch.Tensor] = None
    w2_scale: Optional[torch.Tensor] = None

    def kwargs(self, mode: str) -> dict:
        if mode == "fp8":
            return dict(use_fp8_w8a8=True, block_shape=[128, 128],
                        w1_scale=self.w1_scale, w2_scale=self.w2_scale)
        if mode == "int8":
            return dict(use_int8_w8a8=True, per_channel_quant=True,
                        w1_scale=self.w1_scale, w2_scale=self.w2_scale)
        return {}

    def nbytes(self) -> int:
        n = self.w1.numel() * self.w1.element_size()
        n += self.w2.numel() * self.w2.element_size()
        for s in (self.w1_scale, self.w2_scale):
            if s is not None:
                n += s.numel() * 4
        return n


def make_weights(K: int, N: int, E: int, mode: str = "bf16",
                 w_scale: float = 0.02, device="cuda",
                 seed: Optional[int] = None) -> MoEWeights:
    """SGLang-layout expert weights ``w1 [E, 2N, K]``, ``w2 [E, K, N]``:
    ``randn * w_scale`` in bf16, quantised per expert for fp8 / int8."""
    g = torch.Generator(device=device)
    g.manual_seed(K + N + E if seed is None else seed)
    if mode == "bf16":
        w1 = torch.empty((E, 2 * N, K), dtype=torch.bfloat16, device=device)
        w2 = torch.empty((E, K, N), dtype=torch.bfloat16, device=device)
        for e in range(E):
            w1[e] = (torch.randn((2 * N, K), generator=g, device=device) *
                     w_scale).to(torch.bfloat16)
            w2[e] = (torch.randn((K, N), generator=g, device=device) *
                     w_scale).to(torch.bfloat16)
        return MoEWeights(w1, w2)
    qdt = torch.float8_e4m3fn if mode == "fp8" else torch.int8
    w1 = torch.empty((E, 2 * N, K), dtype=qdt, device=device)
    w2 = torch.empty((E, K, N), dtype=qdt, device=device)
    if mode == "fp8":
        s1 = torch.empty((E, 2 * N // 128, K // 128), device=device)
        s2 = torch.empty((E, K // 128, N // 128), device=device)
        fn = quant.quantize_fp8_block
    else:
        s1 = torch.empty((E, 2 * N), device=device)
        s2 = torch.empty((E, K), device=device)
        fn = quant.quantize_int8_channel
    for e in range(E):
        a = (torch.randn((1, 2 * N, K), generator=g, device=device) *
             w_scale).to(torch.bfloat16)
        q, s = fn(a)
        w1[e], s1[e] = q[0], s[0]
        b = (torch.randn((1, K, N), generator=g, device=device) *
             w_scale).to(torch.bfloat16)
        q, s = fn(b)
        w2[e], s2[e] = q[0], s[0]
    return MoEWeights(w1, w2, s1, s2)


def make_tokens(M: int, K: int, E: int, topk: int, scoring: str = "softmax",
                hot_experts=(), hot_bias: float = 0.0, device="cuda",
                seed: Optional[int] = None, x_scale: float = 1.0):
    """Hidden states ``randn [M, K]`` bf16 and routing from ``randn [M, E]``
    router logits: softmax (or sigmoid) -> top-k -> renormalise
    (reference tests/test_fused_moe.py:37-41)."""
    g = torch.Generator(device=device)
    g.manual_seed(M + K + E + topk if seed is None else seed)
    x = (torch.randn((M, K), generator=g, device=device) * x_scale).to(
        torch.bfloat16)
    logits = torch.randn((M, E), generator=g, device=device, dtype=torch.float32)
    if hot_experts:
        logits[:, list(hot_experts)] += hot_bias
    scores = torch.softmax(logits, -1) if scoring == "softmax" else torch.sigmoid(logits)
    w, ids = torch.topk(scores, topk, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return x, w.float(), ids.to(torch.int32)


def layer_flops(M: int, cfg_or_K, N: int = 0, topk: int = 0) -> float:
    """Algorithmic FLOPs of one layer call: 6*M*topk*K*N (two GEMMs)."""
    if isinstance(cfg_or_K, MoEConfig):
        c = cfg_or_K
        return 6.0 * M * c.topk * c.K * c.N
    return 6.0 * M * topk * cfg_or_K * N


def layer_bytes(M: int, K: int, N: int, topk: int, mode: str,
                topk_ids: torch.Tensor, E: int) -> float:
    """Algorithmic HBM bytes of one layer call: every touched expert's
    weights (and scales) once, x in, out, ids and weights."""
    touched = int(torch.unique(topk_ids).numel())
    bw = 2 if mode == "bf16" else 1
    w = touched * 3 * N * K * bw
    if mode == "fp8":
        w += touched * (3 * N * K // (128 * 128)) * 4
    elif mode == "int8":
        w += touched * (2 * N + K) * 4
    return float(w + M * K * 2 + M * K * 2 + M * topk * 8)


def list_configs() -> List[str]:
    return list(CONFIGS)
