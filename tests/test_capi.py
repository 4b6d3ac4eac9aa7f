"""The C-ABI boundary on the CPU: the library loads, exports every symbol
include/fgs_moe.h declares, and validates arguments on the host (no kernel
is launched by anything here). Also the Python-level argument checks and the
operator registry."""

import ctypes
import os
import re

import pytest
import torch

from flaggems_sglang import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fgs_moe.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fgs_moe_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _capi.load()
    declared = _declared_symbols()
    assert len(declared) >= 13
    for name in declared:
        assert hasattr(lib, name), name
    # the ctypes table covers exactly the header
    assert sorted(_capi.SIGNATURES) == declared


def test_version_and_error_string():
    lib = _capi.load()
    assert lib.fgs_moe_version().decode().startswith("fgs_moe")
    assert isinstance(_capi.last_error(), str)


def test_align_max_padded():
    lib = _capi.load()
    assert lib.fgs_moe_align_max_padded(16, 8, 16) == 16 + 8 * 15
    assert lib.fgs_moe_align_max_padded(-1, 8, 16) == -1
    assert lib.fgs_moe_align_max_padded(4, 0, 16) == -1


@pytest.mark.parametrize(
    "args,code,msg",
    [
        ((1, 4096, 14336, 8, 2, 0, 0), 0, ""),
        ((-1, 4096, 14336, 8, 2, 0, 0), _capi.FGS_EINVAL, "m must be"),
        ((1, 0, 14336, 8, 2, 0, 0), _capi.FGS_EINVAL, "hidden and inter"),
        ((1, 4096, 14336, 0, 2, 0, 0), _capi.FGS_EINVAL, "num_experts"),
        ((1, 4096, 14336, 2000, 2, 0, 0), _capi.FGS_EINVAL, "num_experts"),
        ((1, 4096, 14336, 8, 9, 0, 0), _capi.FGS_EINVAL, "topk"),
        ((1, 4096, 14336, 8, 2, 7, 0), _capi.FGS_EINVAL, "qmode"),
        ((1, 4096, 14336, 8, 2, 0, 0x40), _capi.FGS_EINVAL, "flag"),
        ((1, 4096, 14336, 8, 2, 0, 0x300), _capi.FGS_EINVAL, "excludes"),
        ((1, 4096, 14336, 8, 2, 0, 0x100 | 0x1000), _capi.FGS_EINVAL, "excludes"),
        ((1, 4096, 14336, 8, 2, 0, 0x6000), _capi.FGS_EINVAL, "TILE"),
        ((1, 4096, 14336, 8, 2, 0, 0x5000), 0, ""),
        ((1, 4096, 14336, 8, 2, 0, 0x4000), 0, ""),
        ((1, 4096, 14336, 8, 2, 0, 0x400), 0, ""),
        ((1, 4096, 14336, 8, 2, 0, 0x800), 0, ""),
        ((1, 4096, 14336, 8, 2, 0, 0xC00), _capi.FGS_EINVAL, "exclude each other"),
        ((1, 7168, 2048, 256, 8, 1, 0x1000), 0, ""),
        ((1, 7168, 2048, 256, 8, 1, 0x2000), 0, ""),
        ((1, 4000, 14336, 8, 2, 0, 0), _capi.FGS_EUNSUPPORTED, "multiples"),
        ((1, 3584, 2560, 64, 8, 2, 0), 0, ""),
        ((1, 3584 - 128, 2560, 64, 8, 2, 0), _capi.FGS_EUNSUPPORTED, "multiples"),
        ((1, 9216, 2560, 64, 8, 2, 0), 0, ""),
        ((1, 4096, 14336, 8, 2, 2, 0), 0, ""),
        ((1, 9216, 2560, 64, 8, 0, 0), 0, ""),
    ],
)
def test_validate(args, code, msg):
    lib = _capi.load()
    need = lib.fgs_moe_workspace_bytes(*args)
    rc = lib.fgs_moe_validate(*args, max(need, 0))
    assert rc == code, _capi.last_error()
    if code:
        assert need == -1
        assert msg in _capi.last_error()
    else:
        assert need > 0


def test_validate_workspace_too_small():
    lib = _capi.load()
    need = lib.fgs_moe_workspace_bytes(64, 1024, 512, 8, 2, 0, 0)
    assert lib.fgs_moe_validate(64, 1024, 512, 8, 2, 0, 0, need - 1) == _capi.FGS_EINVAL
    assert "workspace too small" in _capi.last_error()


def test_workspace_grows_with_tokens_and_quant_mode():
    lib = _capi.load()
    a = lib.fgs_moe_workspace_bytes(1, 7168, 2048, 256, 8, 0, 0)
    b = lib.fgs_moe_workspace_bytes(4096, 7168, 2048, 256, 8, 0, 0)
    c = lib.fgs_moe_workspace_bytes(4096, 7168, 2048, 256, 8, 1, 0)
    assert 0 < a < b < c


def test_entry_points_reject_bad_arguments_before_launch():
    """Invalid calls return an error code without touching a device."""
    lib = _capi.load()
    nul = None
    # max_padded below numel + E*(B-1)
    assert lib.fgs_moe_align_block_size(nul, 8, 4, 16, nul, nul, nul, 10, nul, 0,
                                        nul) == -1
    assert "max_padded" in _capi.last_error()
    assert lib.fgs_moe_align_block_size(nul, 8, 0, 16, nul, nul, nul, 100, nul, 0,
                                        nul) == -1
    assert lib.fgs_moe_align_scratch_bytes(100, 8) == 0      # one workgroup
    assert lib.fgs_moe_align_scratch_bytes(65536, 128) == 64 * 128 * 4
    assert lib.fgs_moe_align_scratch_bytes(-1, 8) == -1
    assert lib.fgs_moe_topk_gating(nul, 0, 4, 8, 9, 0, 1, nul, nul, nul) == -1
    assert "topk" in _capi.last_error()
    assert lib.fgs_moe_topk_gating(nul, 0, 4, 2000, 2, 0, 1, nul, nul, nul) == -1
    assert lib.fgs_moe_topk_gating(nul, 0, 4, 8, 2, 5, 1, nul, nul, nul) == -1
    assert lib.fgs_moe_topk_gating(nul, 0, 4, 8, 2, 0, 1, nul, nul, nul) == -1
    assert "null pointer" in _capi.last_error()
    assert lib.fgs_moe_topk_gating(nul, 0, 0, 8, 2, 0, 1, nul, nul, nul) == 0
    assert lib.fgs_moe_silu_and_mul(nul, nul, 4, 12, nul) == -2
    assert lib.fgs_moe_silu_and_mul(nul, nul, 4, 16, nul) == -1  # null pointers
    assert lib.fgs_moe_sum(nul, nul, 4, 0, 16, nul) == -1
    assert lib.fgs_moe_quant_fp8_group(nul, nul, nul, 4, 256, 100, nul) == -2
    assert lib.fgs_moe_quant_int8_token(nul, nul, nul, 4, 12, nul) == -2
    assert lib.fgs_moe_quant_int8_token(nul, nul, nul, 4, 8200, nul) == -1  # null
    need = lib.fgs_moe_workspace_bytes(4, 256, 128, 4, 2, 0, 0)
    rc = lib.fgs_moe_fused_bf16(nul, nul, nul, nul, nul, 4, 256, 128, 4, 2, 0,
                                nul, need, nul, nul)
    assert rc == -1 and "null pointer" in _capi.last_error()
    rc = lib.fgs_moe_fused_fp8_block(nul, nul, nul, nul, nul, 64, 128, nul, nul,
                                     4, 256, 128, 4, 2, 0, nul, need, nul, nul)
    assert rc == -2 and "128x128" in _capi.last_error()
    rc = lib.fgs_moe_fused_int8_channel(nul, nul, nul, nul, nul, nul, nul, 4,
                                        256, 256, 4, 2, 0, nul, 0, nul, nul)
    assert rc == -1 and "workspace" in _capi.last_error()
    # bias variant: swiglu only, both biases, no NaN parameters
    rc = lib.fgs_moe_fused_bf16_bias(nul, nul, nul, nul, nul, nul, nul, 4, 256, 128,
                                     4, 2, _capi.FLAG_ACT_GELU, 1.0, 0.0, nul, need,
                                     nul, nul)
    assert rc == -2 and "swiglu" in _capi.last_error()
    rc = lib.fgs_moe_fused_bf16_bias(nul, nul, nul, nul, nul, nul, nul, 4, 256, 128,
                                     4, 2, 0, 1.0, 0.0, nul, need, nul, nul)
    assert rc == -1 and "b13 and b2" in _capi.last_error()
    rc = lib.fgs_moe_fused_bf16_bias(nul, nul, 16, nul, 16, nul, nul, 4, 256, 128,
                                     4, 2, 0, float("nan"), 0.0, nul, need, nul, nul)
    assert rc == -1 and "NaN" in _capi.last_error()
    # quantised bias variant: fp8 / int8 only, then the bias entry's checks
    rc = lib.fgs_moe_fused_quant_bias(_capi.QMODE_BF16, nul, nul, 16, nul, 16, nul, nul,
                                      nul, nul, 4, 256, 128, 4, 2, 0, 1.0, 0.0, nul, need,
                                      nul, nul)
    assert rc == -1 and "qmode" in _capi.last_error()
    rc = lib.fgs_moe_fused_quant_bias(_capi.QMODE_INT8_CHANNEL, nul, nul, 16, nul, 16, nul,
                                      nul, nul, nul, 4, 256, 128, 4, 2, _capi.FLAG_ACT_GELU,
                                      1.0, 0.0, nul, need, nul, nul)
    assert rc == -2 and "swiglu" in _capi.last_error()
    rc = lib.fgs_moe_fused_quant_bias(_capi.QMODE_FP8_BLOCK, nul, nul, nul, nul, 16, nul,
                                      nul, nul, nul, 4, 256, 128, 4, 2, 0, 1.0, 0.0, nul,
                                      need, nul, nul)
    assert rc == -1 and "b13 and b2" in _capi.last_error()
    need8 = lib.fgs_moe_workspace_bytes(4, 256, 256, 4, 2, _capi.QMODE_INT8_CHANNEL, 0)
    rc = lib.fgs_moe_fused_quant_bias(_capi.QMODE_INT8_CHANNEL, nul, nul, 16, nul, 16, nul,
                                      nul, nul, nul, 4, 256, 256, 4, 2, 0, 1.0, 0.0, nul,
                                      need8, nul, nul)
    assert rc == -1 and "null pointer" in _capi.last_error()
    assert lib.fgs_moe_validate(4, 256, 128, 4, 2, 0, _capi.FLAG_ACT_GELU, need) == 0
    # routing-tuple entry: bias pair, swiglu only, the tuple's arrays
    rc = lib.fgs_moe_fused_routed(0, nul, nul, nul, nul, nul, 16, nul, 1.0, 0.0, 16, 16,
                                  16, 4, 256, 128, 4, 2, 0, nul, need, nul, nul)
    assert rc == -1 and "b13 and b2" in _capi.last_error()
    rc = lib.fgs_moe_fused_routed(0, nul, nul, nul, nul, nul, 16, 16, 1.0, 0.0, 16, 16,
                                  16, 4, 256, 128, 4, 2, _capi.FLAG_ACT_GELU, nul, need,
                                  nul, nul)
    assert rc == -2 and "swiglu" in _capi.last_error()
    rc = lib.fgs_moe_fused_routed(0, nul, nul, nul, nul, nul, nul, nul, 1.0, 0.0, nul, 16,
                                  16, 4, 256, 128, 4, 2, 0, nul, need, nul, nul)
    assert rc == -1 and "null pointer" in _capi.last_error()
    rc = lib.fgs_moe_fused_routed(0, 16, 16, 16, nul, nul, nul, nul, 1.0, 0.0, 16, 16,
                                  16, 4, 256, 128, 4, 2, 0, 256, need - 1, 16, nul)
    assert rc == -1 and "workspace" in _capi.last_error()
    rc = lib.fgs_moe_fused_routed(0, nul, nul, nul, nul, nul, nul, nul, 1.0, 0.0, nul, nul,
                                  nul, 0, 256, 128, 4, 2, 0, nul, need, nul, nul)
    assert rc == 0  # no tokens: nothing read or written
    # routing tuple -> per-slot routing
    assert lib.fgs_moe_routing_to_topk(nul, nul, nul, 4, 0, 8, nul, nul, nul) == -1
    assert lib.fgs_moe_routing_to_topk(nul, nul, nul, 4, 2, 2000, nul, nul, nul) == -1
    assert lib.fgs_moe_routing_to_topk(nul, nul, nul, 4, 2, 8, nul, nul, nul) == -1
    assert lib.fgs_moe_routing_to_topk(nul, nul, nul, 0, 2, 8, nul, nul, nul) == 0


def test_profile_modes():
    """Stage profiler modes 0..3 are accepted (host only); others fail."""
    lib = _capi.load()
    for mode in (1, 2, 3, 0):
        assert lib.fgs_moe_profile_enable(mode) == 0
    assert lib.fgs_moe_profile_enable(4) == _capi.FGS_EINVAL
    assert "profile mode" in _capi.last_error()
    assert lib.fgs_moe_profile_enable(-1) == _capi.FGS_EINVAL


def test_error_codes_map_to_python_exceptions():
    with pytest.raises(ValueError):
        _capi.check(_capi.FGS_EINVAL, "x")
    with pytest.raises(NotImplementedError):
        _capi.check(_capi.FGS_EUNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _capi.check(_capi.FGS_ELAUNCH, "x")
    _capi.check(_capi.FGS_OK, "x")


def test_error_string_is_thread_local():
    import threading

    lib = _capi.load()
    lib.fgs_moe_validate(-1, 1, 1, 1, 1, 0, 0, 0)
    seen = {}

    def other():
        seen["msg"] = _capi.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "m must be" in _capi.last_error()


# ------------------------------------------------------ python boundary ---
def test_registry_surface():
    import flaggems_sglang

    names = flaggems_sglang.all_registered_ops()
    for n in ("fused_moe", "triton_kernel_fused_experts", "moe_align_block_size",
              "silu_and_mul", "moe_sum", "fused_topk", "fused_moe_flagos",
              "triton_kernel_fused_experts_with_bias"):
        assert n in names
        assert getattr(flaggems_sglang, n) is flaggems_sglang.get_op(n)
    assert flaggems_sglang.get_op("nope") is None
    assert flaggems_sglang.device == "cuda"
    assert flaggems_sglang.vendor_name == "amd"


def _cpu_inputs():
    x = torch.randn(4, 256, dtype=torch.bfloat16)
    w1 = torch.randn(4, 256, 256, dtype=torch.bfloat16)
    w2 = torch.randn(4, 256, 128, dtype=torch.bfloat16)
    tw = torch.full((4, 2), 0.5)
    ti = torch.zeros(4, 2, dtype=torch.int32)
    return x, w1, w2, tw, ti


def test_unsupported_flags_keep_reference_messages():
    from flaggems_sglang import fused_moe, triton_kernel_fused_experts

    x, w1, w2, tw, ti = _cpu_inputs()
    with pytest.raises(AssertionError, match="expert_map is not supported"):
        fused_moe(x, w1, w2, tw, ti, expert_map=torch.zeros(4))
    with pytest.raises(AssertionError, match="a1_scale is not supported"):
        fused_moe(x, w1, w2, tw, ti, a1_scale=torch.ones(1))
    with pytest.raises(AssertionError, match="Inplace is not supported"):
        fused_moe(x, w1, w2, tw, ti, inplace=True)
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation"):
        fused_moe(x, w1, w2, tw, ti, activation="relu")
    from flaggems_sglang import triton_kernel_fused_experts_with_bias
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation"):
        triton_kernel_fused_experts_with_bias(x, w1, None, None, w2, None, None,
                                              None, None, None, activation="gelu")
    with pytest.raises(AssertionError, match="Inplace is not supported"):
        triton_kernel_fused_experts_with_bias(x, w1, None, None, w2, None, None,
                                              None, None, None, inplace=True)
    with pytest.raises(AssertionError, match="use_fp8_w8a8 is not supported"):
        triton_kernel_fused_experts(x, w1, w2, None, None, None, use_fp8_w8a8=True)
    with pytest.raises(AssertionError, match="block_shape is not supported"):
        triton_kernel_fused_experts(x, w1, w2, None, None, None, block_shape=[128, 128])


def test_no_cpu_fallback():
    from flaggems_sglang import fused_moe, moe_align_block_size, silu_and_mul

    x, w1, w2, tw, ti = _cpu_inputs()
    with pytest.raises(RuntimeError, match="GPU tensor"):
        fused_moe(x, w1, w2, tw, ti)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        moe_align_block_size(ti, 4, 16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        silu_and_mul(x)


def test_standard_topk_to_routing_needs_gpu():
    """The routing conversion runs on the GPU only (no CPU fallback)."""
    from flaggems_sglang import standard_topk_to_routing

    w = torch.full((3, 2), 0.5)
    ids = torch.zeros(3, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        standard_topk_to_routing(w, ids, 4)


def test_routing_conversion_validation():
    lib = _capi.load()
    assert lib.fgs_moe_routing_max_tiles(36, 4) == 6
    assert lib.fgs_moe_routing_max_tiles(2, 3) == 2
    assert lib.fgs_moe_routing_max_tiles(65536, 128) == (65536 - 128 + 1 + 15) // 16 + 127
    assert lib.fgs_moe_routing_max_tiles(10, 1023) == -1
    ws = lib.fgs_moe_routing_workspace_bytes(36, 4)
    assert ws > 0
    p = 1 << 20  # never dereferenced: validation fails first
    rc = lib.fgs_moe_topk_to_routing(p, p, 9, 4, 4, p, p, p, p, p, p, p, 5, p, ws, None)
    assert rc == _capi.FGS_EINVAL and "max_tiles" in _capi.last_error()
    rc = lib.fgs_moe_topk_to_routing(p, p, 9, 4, 4, p, p, p, p, p, p, p, 6, p, ws - 1, None)
    assert rc == _capi.FGS_EINVAL and "workspace too small" in _capi.last_error()
    rc = lib.fgs_moe_topk_to_routing(p, p, 9, 4, 1023, p, p, p, p, p, p, p, 6, p, ws, None)
    assert rc == _capi.FGS_EINVAL and "num_experts" in _capi.last_error()
    rc = lib.fgs_moe_topk_to_routing(p, None, 9, 4, 4, p, p, p, p, p, p, p, 6, p, ws, None)
    assert rc == _capi.FGS_EINVAL and "null pointer" in _capi.last_error()


def test_weight_cache_one_conversion_per_live_weight():
    """A model with many MoE layers (Qwen3-30B-A3B: 48, DeepSeek-V3: 58, two
    or three converted weights each) converts every weight once, however
    many there are; an in-place update converts again; a freed weight's copy
    is released with it and never served to a new tensor."""
    import gc

    from flaggems_sglang.ops import fused_moe as fm

    calls = []

    def double(t):
        calls.append(1)
        return t * 2

    cache = fm._ConversionCache(double)
    ws = [torch.full((4, 4), float(i)) for i in range(150)]
    first = [cache(w) for w in ws]
    for _ in range(3):
        for w, f in zip(ws, first):
            assert cache(w) is f
    del w  # the loop variable holds the last weight
    assert len(calls) == 150 and len(cache) == 150
    # views of one weight are separate conversions of the same root
    assert torch.equal(cache(ws[1].t()), ws[1].t() * 2)
    assert len(calls) == 151 and len(cache) == 151
    # an in-place update is a new version
    ws[0].add_(1)
    assert torch.equal(cache(ws[0]), torch.full((4, 4), 2.0))
    assert len(calls) == 152
    # dropping weights drops their copies
    del ws[10:]
    gc.collect()
    assert len(cache) == 11
    fresh = [torch.full((4, 4), 7.0) for _ in range(20)]
    for t in fresh:
        assert torch.equal(cache(t), torch.full((4, 4), 14.0))
    assert len(cache) == 31


def test_weight_cache_zero_copy_views_not_stored():
    """A reference-layout weight that is a transposed view of a native-layout
    tensor converts to that tensor's storage without a copy, and is not held
    (holding it would keep the source alive)."""
    from flaggems_sglang.ops import fused_moe as fm

    native = torch.randn(2, 8, 4)
    ref_layout = native.transpose(-1, -2)
    out = fm._native_layout(ref_layout)
    assert out.data_ptr() == native.data_ptr() and torch.equal(out, native)
    before = len(fm._native_layout)
    fm._native_layout(ref_layout)
    assert len(fm._native_layout) == before


def _schedule_in_subprocess(env_extra):
    import subprocess
    import sys

    code = ("import sys; sys.path[:0] = [{!r}, {!r}]\n"
            "from flaggems_sglang import _capi\n"
            "print(_capi.schedule(4096, 4096, 14336, 8, 2))\n").format(
                ROOT, os.path.join(ROOT, "flaggems-sglang_amd"))
    env = {k: v for k, v in os.environ.items() if not k.startswith("FGS_MOE_")}
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                         text=True, check=True)
    return out.stdout.strip()


def test_tuning_knobs_need_the_tuning_switch():
    """Schedule knobs in the environment (here the GEMM2 k split and the
    tail split) change nothing unless FGS_MOE_TUNING=1: the compiled-in
    choices are the product."""
    base = _schedule_in_subprocess({})
    knobs = {"FGS_MOE_KSPLIT": "3", "FGS_MOE_TAIL": "0"}
    assert _schedule_in_subprocess(knobs) == base
    tuned = _schedule_in_subprocess({**knobs, "FGS_MOE_TUNING": "1"})
    assert tuned != base and "ksplit2=3" in tuned


def test_removed_single_token_fused_flag_is_rejected():
    """0x4 (the former single-token fused schedule) is an unknown flag bit."""
    lib = _capi.load()
    assert lib.fgs_moe_validate(1, 256, 128, 4, 2, 0, 0x4, 1 << 30) == _capi.FGS_EINVAL
    assert "unknown flag" in _capi.last_error()


def test_weight_cache_sees_data_reassignment_and_clears_on_request():
    """``param.data = new`` (a new storage) converts again. ``param.data.
    copy_(new)`` bumps neither the version nor the storage, so the cache
    serves the old conversion until clear_weight_cache() drops it."""
    from flaggems_sglang.ops import fused_moe as fm

    p = torch.nn.Parameter(torch.arange(6.0).reshape(1, 2, 3), requires_grad=False)
    first = fm._native_layout(p)
    assert torch.equal(first, p.transpose(-1, -2))
    assert fm._native_layout(p) is first
    p.data = torch.full((1, 2, 3), 5.0)
    assert torch.equal(fm._native_layout(p), torch.full((1, 3, 2), 5.0))
    p.data.copy_(torch.full((1, 2, 3), 9.0))
    assert p._version == 0  # invisible to the version counter
    assert torch.equal(fm._native_layout(p), torch.full((1, 3, 2), 5.0))  # stale
    fm.clear_weight_cache()
    assert torch.equal(fm._native_layout(p), torch.full((1, 3, 2), 9.0))
