"""ltx25_linear_q_noalloc captured in a HIP graph (torch.cuda.CUDAGraph on
the stream the library launches on), the use it exists for: every replay
must reproduce the eager call's output bit for bit, with other calls that
overwrite the library's fixed scratch array run eagerly between the
replays.

The entry point launches only kernels (no allocation, no memset, no host
synchronization), so a capture records the GEMM and, for split-K plans,
its reduction, reading and writing the per-GPU scratch array.
"""
import numpy as np
import pytest
import torch

from gpu_util import make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

# (name, M, K, N, bits, group, bias dtype, epilogue)
CASES = [
    ("mid split-K (128x128 tile)", 256, 2048, 2048, 8, 64, "f32", 1),
    ("M <= 128 kernel, split-K", 126, 8192, 2048, 8, 64, "bf16", 0),
    ("256x256 fused w8 tile", 4096, 2048, 4096, 8, 64, None, 1),
]


def _operands(pkg, M, K, N, bits, group, bias_dt, seed):
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    qw = make_qweight(pkg, rng_normal(rng, (N, K), 0.02), bits, group)[0]
    bias = None
    if bias_dt is not None:
        b = torch.randn((N,), device="cuda", generator=g) * 0.05
        bias = b.to(torch.bfloat16) if bias_dt == "bf16" else b.float()
    return x, qw, bias


@pytest.mark.parametrize("name,M,K,N,bits,group,bias_dt,epi", CASES, ids=[c[0] for c in CASES])
def test_noalloc_linear_replays_in_a_graph(pkg, lib, name, M, K, N, bits, group, bias_dt, epi):
    assert lib.ltx25_init() == 0, pkg.last_error()
    pkg.set_tile(pkg.TILE_AUTO)
    x, qw, bias = _operands(pkg, M, K, N, bits, group, bias_dt, 11)
    # another call of the same plan family, run eagerly between replays: it
    # rewrites the scratch array the captured call uses
    x2, qw2, bias2 = _operands(pkg, M, K, N, bits, group, bias_dt, 12)
    y_eager = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y_other = torch.empty_like(y_eager)
    say(f"noalloc graph {name}: eager")
    pkg.linear_q_noalloc(x, qw, bias, y_eager, M, K, N, epi)
    torch.cuda.synchronize()
    want = y_eager.clone()

    y_graph = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        # a warm-up call on the capture stream, as torch's capture recipe asks
        pkg.linear_q_noalloc(x, qw, bias, y_graph, M, K, N, epi)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    say(f"noalloc graph {name}: capture")
    with torch.cuda.graph(graph):
        pkg.linear_q_noalloc(x, qw, bias, y_graph, M, K, N, epi)
    torch.cuda.synchronize()
    for rep in range(3):
        y_graph.fill_(float("nan"))
        pkg.linear_q_noalloc(x2, qw2, bias2, y_other, M, K, N, epi)   # dirties the scratch
        torch.cuda.synchronize()
        say(f"noalloc graph {name}: replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.view(torch.int16), want.view(torch.int16)), f"replay {rep}"
    # and the eager call is unchanged by the replays
    pkg.linear_q_noalloc(x, qw, bias, y_eager, M, K, N, epi)
    torch.cuda.synchronize()
    assert torch.equal(y_eager.view(torch.int16), want.view(torch.int16))
    del graph
