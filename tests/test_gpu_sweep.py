"""A seeded sweep of random linear shapes through the C ABI, against the oracle.

The fixed cases elsewhere pin the reference's own test shapes and the DiT's; this sweep draws
shapes across the routing space instead -- M from 1 to ~700 (one or several 128- and 256-row
tiles, ragged edges), K any multiple of 64, N ragged, w8 / w4, group 64 / 32, no / bf16 /
f32 bias, with and without the GELU epilogue, dense weights too, and the dequant-once arm forced
on for a share of them -- so that a tile, split or edge path no fixed case reaches still meets
the bar: max|y - ref| / max|ref| <= 1e-2 against the f64-accumulated GEMM over the f32
dequantized weight (GELU applied to the f32-rounded reference where asked).
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_f32, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2


def draw(i):
    rng = np.random.default_rng(1000 + i)
    bits, group = [(8, 64), (8, 32), (4, 64), (4, 32), (16, 64)][i % 5]
    M = int(rng.choice([1, 7, 33, 64, 126, 129, 200, 255, 257, 320, 511, 700]))
    K = 64 * int(rng.integers(1, 40))      # the kernels step K by 64 (others are refused)
    N = int(rng.choice([8, 40, 100, 128, 255, 384, 513, 1000, 2050]))
    if bits == 4:
        N = max(8, N - N % 8)
    bias = ["none", "bf16", "f32"][int(rng.integers(0, 3))]
    epi = int(rng.integers(0, 2)) if bits != 16 else 0   # the dense linear has no epilogue
    deq_once = bool(rng.integers(0, 4) == 0) and bits != 16 and M >= 64 and K % 64 == 0
    return M, K, N, bits, group, bias, epi, deq_once


CASES = [draw(i) for i in range(30)]


@pytest.mark.parametrize("M,K,N,bits,group,bias,epi,deq_once", CASES,
                         ids=[f"c{i}" for i in range(len(CASES))])
def test_random_shape_against_oracle(pkg, dev, M, K, N, bits, group, bias, epi, deq_once):
    rng = np.random.default_rng(M * 131 + K * 7 + N)
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    w = rng_normal(rng, (N, K), 0.02)
    b = rng_normal(rng, (N,), 0.01)
    if bias == "bf16":
        b = orc.bf16_to_f32(orc.bf16_rne(b))
        bd = dev_bf16(orc.bf16_rne(b))
    elif bias == "f32":
        bd = dev_f32(b)
    else:
        b, bd = None, None
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"sweep M={M} K={K} N={N} bits={bits} g={group} bias={bias} epi={epi} "
        f"dequant_once={deq_once}")
    if bits == 16:
        wb = orc.bf16_rne(w)
        wf = orc.bf16_to_f32(wb)
        pkg.linear(dev_bf16(x), dev_bf16(wb), bd, y, M, K, N)
    else:
        qw, codes, scales, biases, _ = make_qweight(pkg, w, bits, group)
        wf, _ = orc.dequant(codes, scales, biases, N, K, bits, group)
        try:
            if deq_once:
                pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
            pkg.linear_q(dev_bf16(x), qw, bd, y, M, K, N, epi)
        finally:
            pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    torch.cuda.synchronize()
    ref = orc.linear_f64_d(orc.bf16_to_f32(x), wf, b)
    if epi:
        ref = orc.gelu(ref.astype(np.float32)).astype(np.float64)
    got = host_f32(y)
    assert orc.max_rel(got, ref) <= MAX_REL
