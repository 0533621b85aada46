"""The allocation-free W4A16 entry point (ff_gemm_w4a16_noalloc) against the
workspace entry point it mirrors (ff_gemm_w4a16_ws given the bytes
ff_gemm_w4a16_workspace asks for): bit-identical outputs on consecutive calls
that share the static scratch, the second with a smaller input, plus a tail
row; a split that would exceed the scratch is rejected; captured in a hipGraph,
every replay equals the eager call."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
DEV = "cuda"
FF_TUNE_W4A16_SPLITS = 4


def _case(m, k, n, group, sym, seed):
    from fastforward_amd.linear import Int4
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(BF16).to(DEV)
    op = Int4((torch.randn(n, k, generator=g) * 0.02).to(BF16).to(DEV), group=group, symmetric=sym)
    return x, op


def _both(x, op):
    from fastforward_amd._lib import call, ptr, stream
    m, k = x.shape
    n = op.weight.shape[0]
    need = ctypes.c_int64(0)
    call("ff_gemm_w4a16_workspace", m, n, k, ctypes.byref(need))
    ws = torch.full((max(need.value, 256),), 0x7F, device=DEV, dtype=torch.uint8)
    y_ws = torch.full((m, n), float("nan"), device=DEV, dtype=BF16)
    y_na = torch.full((m, n), float("nan"), device=DEV, dtype=BF16)
    call("ff_gemm_w4a16_ws", ptr(x), k, ptr(op.packed), ptr(op.scales), op.group, ptr(y_ws), n, m, n, k, ptr(ws),
         need.value, stream())
    call("ff_gemm_w4a16_noalloc", ptr(x), k, ptr(op.packed), ptr(op.scales), op.group, ptr(y_na), n, m, n, k,
         stream())
    torch.cuda.synchronize()
    return y_ws, y_na, need.value


def test_noalloc_equals_workspace_entry_point(gpu):
    # two calls in a row that both split k, the second smaller, then a tail row
    for m, k, n, group, sym, seed in ((576, 4096, 6144, 128, True, 1), (100, 1024, 512, 32, False, 2),
                                      (1, 12288, 4096, 128, True, 3)):
        x, op = _case(m, k, n, group, sym, seed)
        y_ws, y_na, need = _both(x, op)
        print(f"noalloc {m}x{k}x{n} g{group}: {need} bytes of scratch", flush=True)
        assert need > 0, "the case must use the scratch"
        assert not torch.isnan(y_na.float()).any()
        assert torch.equal(y_ws, y_na), (m, k, n)


def test_noalloc_rejects_a_split_beyond_the_scratch(gpu):
    from fastforward_amd._lib import call, ptr, stream
    x, op = _case(576, 4096, 6144, 128, True, 4)
    y = torch.empty(576, 6144, device=DEV, dtype=BF16)
    call("ff_set_tuning", FF_TUNE_W4A16_SPLITS, 8)      # 8 x 576 x 6144 x 4 bytes > 32 MiB
    try:
        with pytest.raises(RuntimeError, match="static scratch"):
            call("ff_gemm_w4a16_noalloc", ptr(x), 4096, ptr(op.packed), ptr(op.scales), op.group, ptr(y), 6144,
                 576, 6144, 4096, stream())
    finally:
        call("ff_set_tuning", FF_TUNE_W4A16_SPLITS, 0)
    # and the default choice for the same product runs
    y_ws, y_na, _ = _both(x, op)
    assert torch.equal(y_ws, y_na)


def test_noalloc_under_graph_capture(gpu):
    """The use the entry point exists for: captured in a hipGraph (no allocation,
    no memset node), each replay equals the workspace entry point's eager call
    on the inputs the replay read, with other eager work and synchronisations
    between the replays."""
    from fastforward_amd._lib import call, ptr, stream
    m, k, n = 576, 4096, 6144
    x, op = _case(m, k, n, 128, True, 5)
    y = torch.full((m, n), float("nan"), device=DEV, dtype=BF16)
    g = torch.Generator().manual_seed(6)
    inputs = [torch.randn(m, k, generator=g).to(BF16).to(DEV) for _ in range(3)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # eager call first: the scratch address is taken outside the capture
        call("ff_gemm_w4a16_noalloc", ptr(x), k, ptr(op.packed), ptr(op.scales), op.group, ptr(y), n, m, n, k,
             stream())
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call("ff_gemm_w4a16_noalloc", ptr(x), k, ptr(op.packed), ptr(op.scales), op.group, ptr(y), n, m, n, k,
             stream())
    for rep, xi in enumerate(inputs + inputs[:1]):
        x.copy_(xi)
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        got = y.clone()
        y_ws, y_na, need = _both(x, op)      # eager calls between the replays (they reuse the scratch)
        assert need > 0
        assert torch.equal(got, y_ws), f"replay {rep} differs from the eager workspace call"
        assert torch.equal(y_na, y_ws)
