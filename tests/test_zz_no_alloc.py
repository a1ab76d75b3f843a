"""hn_block_linear_noalloc (the one-call linear on the library's own scratch array) against hn_block_linear (the
same linear on a caller workspace): identical outputs on consecutive calls, the later ones smaller, across the
scale layouts, and under HIP graph capture.  (Problems beyond the scratch size are rejected before any launch:
tests/test_capi.py checks that on the CPU.)"""
import pytest
import torch

from conftest import seeded

pytestmark = pytest.mark.gpu


def noalloc(x, qw, sw, bias, group, kind, sw_rows=1, rounding="half_away", out=None):
    from hy_nomas import _lib

    m, k = x.shape
    n = qw.shape[0]
    if out is None:
        out = torch.empty((m, n), device=x.device, dtype=x.dtype)
    _lib.call("hn_block_linear_noalloc", x.data_ptr(), _lib.dtype_code(x), x.stride(0), m, k, group, _lib.KIND[kind],
              _lib.ROUND[rounding], qw.data_ptr(), qw.stride(0), sw.data_ptr(), sw.stride(0), sw_rows, _lib.ptr(bias),
              _lib.dtype_code(bias) if bias is not None else 0, n, out.data_ptr(), _lib.dtype_code(out), out.stride(0),
              _lib.stream(x))
    return out


def with_workspace(x, qw, sw, bias, group, kind, sw_rows=1, rounding="half_away"):
    from hy_nomas import _lib

    m, k = x.shape
    n = qw.shape[0]
    out = torch.empty((m, n), device=x.device, dtype=x.dtype)
    nbytes = _lib.lib().hn_block_linear_workspace_bytes(m, k, group)
    ws = torch.full((nbytes,), 0x55, device=x.device, dtype=torch.uint8)
    _lib.call("hn_block_linear", x.data_ptr(), _lib.dtype_code(x), x.stride(0), m, k, group, _lib.KIND[kind],
              _lib.ROUND[rounding], qw.data_ptr(), qw.stride(0), sw.data_ptr(), sw.stride(0), sw_rows, _lib.ptr(bias),
              _lib.dtype_code(bias) if bias is not None else 0, n, out.data_ptr(), _lib.dtype_code(out), out.stride(0),
              ws.data_ptr(), nbytes, _lib.stream(x))
    return out


def case(dev, g, m, k, n, layout):
    """(x, qw, sw, bias, group, kind, sw_rows) for a layout: int8 g128, int8 per token, fp8 128x128 blocks."""
    x = (torch.randn(m, k, generator=g) * 2).to(torch.bfloat16).to(dev)
    bias = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    if layout == "fp8_block":
        from hy_nomas import pixelumm

        qw, sblk = pixelumm.quantize_fp8_block(torch.randn(n, k, generator=g) * 0.02)
        return x, qw.to(dev), sblk.to(dev), bias, 128, "fp8", 128
    qw = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).to(dev)
    cols = 1 if layout == "int8_per_token" else k // 128
    sw = (torch.rand(n, cols, generator=g) * 4e-3 + 1e-3).to(dev)
    return x, qw, sw, bias, (k if cols == 1 else 128), "int8", 1


def test_noalloc_matches_the_workspace_entry_point(dev):
    print("hn_block_linear_noalloc vs hn_block_linear: consecutive calls, shrinking", flush=True)
    g = seeded(4096)
    # each call smaller than the one before, so a later call that read stale scratch contents would differ
    for m, k, n, layout in ((3000, 3072, 1536, "int8_g128"), (700, 2048, 768, "int8_per_token"),
                            (513, 1024, 640, "fp8_block"), (37, 256, 384, "int8_g128")):
        x, qw, sw, bias, group, kind, sw_rows = case(dev, g, m, k, n, layout)
        got = noalloc(x, qw, sw, bias, group, kind, sw_rows)
        torch.cuda.synchronize()
        ref = with_workspace(x, qw, sw, bias, group, kind, sw_rows)
        assert torch.equal(got, ref), f"{layout} {m}x{k}x{n}: outputs differ"
        assert got.abs().max().item() > 0


def test_noalloc_rounding_and_repeat(dev):
    """Half-even rounding reaches the quantizer, and a repeated call gives the same result."""
    g = seeded(4097)
    x, qw, sw, bias, group, kind, sw_rows = case(dev, g, 1024, 3072, 3072, "int8_per_token")
    a = noalloc(x, qw, sw, bias, group, kind, sw_rows, "half_even")
    b = with_workspace(x, qw, sw, bias, group, kind, sw_rows, "half_even")
    c = noalloc(x, qw, sw, bias, group, kind, sw_rows, "half_even")
    assert torch.equal(a, b) and torch.equal(a, c)


def test_noalloc_under_graph_capture(dev):
    """The entry point inside a captured HIP graph: one call outside capture first (the first call on a device
    looks up the scratch array's address), then the call captured once and replayed on fresh inputs, with
    eager work and synchronizations between the replays; every replay equals the workspace entry point."""
    print("hn_block_linear_noalloc under graph capture", flush=True)
    g = seeded(4098)
    for layout in ("int8_g128", "int8_per_token", "fp8_block"):
        x, qw, sw, bias, group, kind, sw_rows = case(dev, g, 640, 1024, 768, layout)
        out = torch.empty((x.shape[0], qw.shape[0]), device=dev, dtype=x.dtype)
        noalloc(x, qw, sw, bias, group, kind, sw_rows, out=out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            noalloc(x, qw, sw, bias, group, kind, sw_rows, out=out)
        torch.cuda.synchronize()
        for replay in range(3):
            x.copy_((torch.randn(x.shape, generator=g) * (replay + 1)).to(torch.bfloat16))
            graph.replay()
            torch.cuda.synchronize()
            ref = with_workspace(x, qw, sw, bias, group, kind, sw_rows)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"{layout}: replay {replay} differs from the eager call"
            assert out.abs().max().item() > 0
