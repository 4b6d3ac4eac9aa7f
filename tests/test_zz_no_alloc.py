"""The allocation-free entry point ``fgs_moe_fused_bf16_noalloc`` (the
library's own per-GPU device scratch instead of a caller workspace) against
``fgs_moe_fused_bf16`` with a workspace, through the C ABI.

Both run the same kernels with the same schedule, so the outputs must be
identical bit for bit. Two calls in a row on one GPU share the scratch; the
second, smaller call must not see the first call's leftovers."""

import pytest
import torch

from flaggems_sglang import _capi, testing

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(x, w1, w2, tw, ti, flags=0):
    lib = _capi.load()
    M, K = x.shape
    E, two_n, _ = w1.shape
    k = ti.shape[1]
    ws_bytes = lib.fgs_moe_workspace_bytes(M, K, two_n // 2, E, k, _capi.QMODE_BF16, flags)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    out = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    rc = lib.fgs_moe_fused_bf16(x.data_ptr(), w1.data_ptr(), w2.data_ptr(), tw.data_ptr(),
                                ti.data_ptr(), M, K, two_n // 2, E, k, flags, ws.data_ptr(),
                                ws_bytes, out.data_ptr(), _stream())
    _capi.check(rc, "fgs_moe_fused_bf16")
    return out


def _no_alloc(x, w1, w2, tw, ti, flags=0):
    lib = _capi.load()
    M, K = x.shape
    E, two_n, _ = w1.shape
    out = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    rc = lib.fgs_moe_fused_bf16_noalloc(x.data_ptr(), w1.data_ptr(), w2.data_ptr(),
                                        tw.data_ptr(), ti.data_ptr(), M, K, two_n // 2, E,
                                        ti.shape[1], flags, out.data_ptr(), _stream())
    _capi.check(rc, "fgs_moe_fused_bf16_noalloc")
    return out


# (K, N, E, topk) and two token counts, the second smaller: the tiled
# schedule then the streaming one, streaming then one token (direct rows),
# and a Qwen3-shaped layer at serving batch sizes
CASES = [((1024, 512, 8, 2), 300, 20),
         ((2048, 768, 128, 8), 256, 1),
         ((4096, 1024, 8, 2), 64, 5)]


@pytest.mark.parametrize("shape,m1,m2", CASES, ids=lambda v: str(v))
def test_no_alloc_matches_workspace_entry(gpu, shape, m1, m2):
    K, N, E, k = shape
    wts = testing.make_weights(K, N, E, "bf16", 0.05, device=gpu, seed=K + N + E)
    for m in (m1, m2):
        x, tw, ti = testing.make_tokens(m, K, E, k, device=gpu, seed=m + K + E + k)
        ref = _with_workspace(x, wts.w1, wts.w2, tw, ti)
        got = _no_alloc(x, wts.w1, wts.w2, tw, ti)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"M={m}: differs from the workspace entry point"


def test_no_alloc_rejects_oversize(gpu):
    """A problem whose workspace exceeds the scratch is refused before any
    launch, with the size in the message."""
    lib = _capi.load()
    need = lib.fgs_moe_workspace_bytes(4096, 4096, 14336, 8, 2, _capi.QMODE_BF16, 0)
    assert need > _capi.NOALLOC_SCRATCH_BYTES
    rc = lib.fgs_moe_fused_bf16_noalloc(None, None, None, None, None, 4096, 4096, 14336, 8,
                                        2, 0, None, None)
    assert rc == _capi.FGS_EUNSUPPORTED
    assert str(need) in _capi.last_error()


@pytest.mark.parametrize("m", [300, 1])
def test_no_alloc_under_graph_capture(gpu, m):
    """Captured in a HIP graph after one eager call (the first call on a
    device sets itself up outside the capture) and replayed several times
    with new inputs copied into the captured buffers and eager work in
    between: every replay gives the workspace entry point's bits."""
    K, N, E, k = 1024, 512, 8, 2
    wts = testing.make_weights(K, N, E, "bf16", 0.05, device=gpu, seed=K + N + E + 1)
    x, tw, ti = testing.make_tokens(m, K, E, k, device=gpu, seed=m + 3)
    _no_alloc(x, wts.w1, wts.w2, tw, ti)  # eager set-up call
    torch.cuda.synchronize()
    lib = _capi.load()
    out = torch.empty((m, K), dtype=torch.bfloat16, device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.fgs_moe_fused_bf16_noalloc(x.data_ptr(), wts.w1.data_ptr(), wts.w2.data_ptr(),
                                            tw.data_ptr(), ti.data_ptr(), m, K, N, E, k, 0,
                                            out.data_ptr(), _stream())
    _capi.check(rc, "fgs_moe_fused_bf16_noalloc (captured)")
    for rep in range(4):
        x2, tw2, ti2 = testing.make_tokens(m, K, E, k, device=gpu, seed=100 * rep + m)
        x.copy_(x2)
        tw.copy_(tw2)
        ti.copy_(ti2)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        ref = _with_workspace(x, wts.w1, wts.w2, tw, ti)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager entry point"
