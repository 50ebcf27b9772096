"""The measurement probes (ltx25_probe_read / ltx25_probe_mfma) on the GPU: the
read probe reads exactly the span it is given (each workgroup's XOR of its
16-byte words checked against numpy), and the MFMA probe runs to completion
at both wave counts and operand kinds."""
import numpy as np
import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks", [(16, 1), (4096, 3), (1 << 20, 7), (5496832, 256)])
def test_probe_read_covers_the_span(pkg, dev, nbytes, blocks):
    rng = np.random.default_rng(nbytes + blocks)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    src = torch.from_numpy(host.view(np.int32).copy()).cuda()
    sink = torch.zeros((blocks,), dtype=torch.int32, device="cuda")
    say(f"probe_read bytes={nbytes} blocks={blocks}")
    pkg.probe_read(src, nbytes, sink, blocks)
    torch.cuda.synchronize()
    n16 = nbytes // 16
    per = (n16 + blocks - 1) // blocks
    want = np.zeros(blocks, np.uint32)
    for b in range(blocks):
        span = host[4 * b * per: 4 * min(n16, (b + 1) * per)]
        want[b] = np.bitwise_xor.reduce(span) if span.size else 0
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


@pytest.mark.parametrize("random", [False, True])
@pytest.mark.parametrize("wps", [1, 2])
def test_probe_mfma_runs(pkg, dev, random, wps):
    out = torch.zeros((256,), dtype=torch.float32, device="cuda")
    say(f"probe_mfma random={random} waves_per_simd={wps}")
    pkg.probe_mfma(100, random, wps, out)
    torch.cuda.synchronize()
