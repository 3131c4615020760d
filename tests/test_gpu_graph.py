"""HIP-graph capture of the FP8 MLP forward (the sequence bench.py times): every replay,
with the program's own eager work and synchronisations between replays, reproduces the
eager result bit for bit.

The path records no memset nodes (its kernels overwrite every byte they produce, and the
amax partials are plain per-block stores), and all its kernels are deterministic, so
bit-exact agreement is the bar.
"""

import pytest
import torch

from bongard_amd import ops

pytestmark = pytest.mark.gpu


def _mlp_step(x, w_gu, w_d, inter):
    xq = ops.quantize(x, ops.E4M3)
    gq = ops.quantize(w_gu, ops.E4M3)
    dq = ops.quantize(w_d, ops.E4M3)
    H, _, hparts = ops.gemm_geglu(xq.data, xq.meta, gq.data, gq.meta, inter)
    hq = ops.cast_partials(H, hparts, ops.E4M3)
    return ops.gemm(hq.data, ops.E4M3, hq.meta, dq.data, ops.E4M3, dq.meta)


@pytest.mark.parametrize("M,K,I", [(512, 512, 1024), (300, 256, 384)])
def test_mlp_forward_graph_replays(gpu, M, K, I):
    g = torch.Generator(device=gpu).manual_seed(7)
    x = torch.randn(M, K, device=gpu, generator=g).to(torch.bfloat16)
    w_gu = (torch.randn(2 * I, K, device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    w_d = (torch.randn(K, I, device=gpu, generator=g) * 0.014).to(torch.bfloat16)
    inputs = [torch.randn(M, K, device=gpu, generator=g).to(torch.bfloat16) * s
              for s in (1.0, 3.0, 0.25)]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _mlp_step(x, w_gu, w_d, I)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_graph = _mlp_step(x, w_gu, w_d, I)
    torch.cuda.synchronize()

    for rep, xin in enumerate(inputs):
        x.copy_(xin)
        eager = _mlp_step(x, w_gu, w_d, I).clone()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        same = torch.equal(y_graph.view(torch.int16), eager.view(torch.int16))
        print(f"[graph M={M} replay {rep}] identical to eager: {same}", flush=True)
        assert same, f"replay {rep} differs from the eager step"
