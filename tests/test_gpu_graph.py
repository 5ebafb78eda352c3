"""The kernels under HIP graph capture: a captured forward + backward, replayed several times with
new inputs copied in between (eager work and synchronisations between the replays), must give
the same bits as the eager calls on the same inputs after every replay.  The library records no
memset and allocates nothing inside the call; the workspace comes from the caller."""

import pytest
import torch

from velograd_amd import kernels as vk

pytestmark = pytest.mark.gpu


def _eager(x, r, w, gy, gh, eps):
    y, h, inv = vk.fused_rmsnorm_residual_forward(x, r, w, eps)
    dx, dw = vk.fused_rmsnorm_residual_backward(gy, h, w, inv, saved_is_h=True, grad_h=gh)
    return y, h, inv, dx, dw


@pytest.mark.parametrize("dtype,rows,d", [(torch.bfloat16, 7, 5120), (torch.bfloat16, 512, 4096),
                                          (torch.float32, 33, 1000)])
def test_graph_replays_match_eager(dtype, rows, d):
    torch.manual_seed(0)
    eps = 1e-6
    dev = torch.device("cuda", 0)
    mk = lambda: torch.randn(rows, d, device=dev, dtype=dtype)  # noqa: E731
    x, r, gy, gh = mk(), mk(), mk(), mk()
    w = (1 + 0.1 * torch.randn(d, device=dev)).to(dtype)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm up allocator pools and the library on the capture stream
            _eager(x, r, w, gy, gh, eps)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = _eager(x, r, w, gy, gh, eps)

    for rep in range(4):
        torch.manual_seed(100 + rep)
        for t in (x, r, gy, gh):
            t.copy_(torch.randn(rows, d, device=dev, dtype=dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = _eager(x, r, w, gy, gh, eps)
        torch.cuda.synchronize()
        for name, got, want in zip(("y", "h", "inv_rms", "dx", "dweight"), outs, ref):
            assert torch.equal(got, want), f"replay {rep}: {name} differs from the eager call"


def test_graph_replays_of_quantised_forwards_and_rope_match_eager():
    """fp8, MXFP8, MXFP4 forwards and RoPE captured together, replayed with new inputs."""
    torch.manual_seed(1)
    dev = torch.device("cuda", 0)
    rows, d = 300, 2048
    x = torch.randn(rows, d, device=dev, dtype=torch.bfloat16)
    r = torch.randn(rows, d, device=dev, dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(d, device=dev)).to(torch.bfloat16)
    q = torch.randn(2, 64, 8, 128, device=dev, dtype=torch.bfloat16)

    def calls():
        out = list(vk.fused_rmsnorm_residual_forward_fp8(x, r, w, 1e-5))
        out += list(vk.fused_rmsnorm_residual_forward_mx(x, r, w, 1e-5, fmt="e4m3"))
        out += list(vk.fused_rmsnorm_residual_forward_mx(x, r, w, 1e-5, fmt="e2m1"))
        out.append(vk.fused_rope_forward(q)[0])
        return [t.view(torch.uint8) if t.element_size() == 1 else t for t in out]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = calls()
    for rep in range(3):
        for t in (x, r, q):
            t.copy_(torch.randn(t.shape, device=dev, dtype=t.dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = calls()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(outs, ref)):
            assert torch.equal(got, want), f"replay {rep}: output {i} differs from the eager call"


def test_launch_stream_is_torchs_current_stream():
    """The library launches on torch's current stream: the default one, a side stream made
    current, and the capture stream inside torch.cuda.graph."""
    from velograd_amd.kernels import _stream

    dev = torch.device("cuda", 0)
    assert _stream(dev) == torch.cuda.current_stream(dev).cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert _stream(dev) == side.cuda_stream == torch.cuda.current_stream(dev).cuda_stream
        x = torch.randn(64, 4096, device=dev, dtype=torch.bfloat16)
        y, _, _ = vk.fused_rmsnorm_residual_forward(x, None, None, 1e-5)
    side.synchronize()
    ref, _, _ = vk.fused_rmsnorm_residual_forward(x, None, None, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    g = torch.cuda.CUDAGraph()
    seen = []
    with torch.cuda.graph(g):
        seen.append((_stream(dev), torch.cuda.current_stream(dev).cuda_stream))
        yg, _, _ = vk.fused_rmsnorm_residual_forward(x, None, None, 1e-5)
    assert seen[0][0] == seen[0][1]
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(yg, ref)


def test_graph_replays_of_module_forms_and_interleaved_rope_match_eager():
    """The module form (floor), the residual add with the floor, the backward through the fast
    path's outputs, the interleaved RoPE, and the norm + RoPE forward with its one-pass
    backward, captured together and replayed with new inputs."""
    torch.manual_seed(2)
    dev = torch.device("cuda", 0)
    x = torch.randn(64, 4096, device=dev, dtype=torch.bfloat16)
    r = torch.randn(64, 4096, device=dev, dtype=torch.bfloat16)
    g = torch.randn(64, 4096, device=dev, dtype=torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, device=dev)).to(torch.bfloat16)
    q = torch.randn(2, 48, 1024, device=dev, dtype=torch.bfloat16)

    def calls():
        y1, inv1 = vk.rmsnorm_forward(x, w, 1e-6)
        y2, h2, inv2 = vk.fused_rmsnorm_residual_forward(x, r, w, 1e-6, min_mean_sq=1e-12)
        dx, dw = vk.fused_rmsnorm_residual_backward(g, h2, w, inv2, saved_is_h=True)
        qi = vk.fused_rope_interleaved(q, 10000.0)
        qb = vk.fused_rope_interleaved(qi, 10000.0, inverse=True)
        # the attention-branch input: norm + RoPE forward and its one-pass backward
        yr, hr, invr = vk.rmsnorm_rope_forward(x.view(2, 32, 4096), w, 1e-6, 10000.0)
        dxr, dwr = vk.rmsnorm_rope_backward(g.view(2, 32, 4096), hr, w, invr, 10000.0)
        return [y1, inv1, y2, h2, inv2, dx, dw, qi, qb, yr, invr, dxr, dwr]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = calls()
    for rep in range(3):
        for t in (x, r, g, q):
            t.copy_(torch.randn(t.shape, device=dev, dtype=t.dtype))
        x[rep] = 0                       # a floored row in every replay
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = calls()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(outs, ref)):
            assert torch.equal(got, want), f"replay {rep}: output {i} differs from the eager call"
