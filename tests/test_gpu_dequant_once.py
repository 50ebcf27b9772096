"""The dequant-once A/B arm (ltx25_set_dequant_once) on the GPU.

The reference's M5 route expands the quantized weight into a bf16 scratch and
runs the dense GEMM over it (src/ltx25-metal-ops.cc:467-502); its test pins
that the expansion and the fused qmm agree with the dense GEMM over the
uploaded dequantized weight at rel-L2 0 (tests/ltx25-qlinear-test.cc:
266-273). Here the expansion is bit-identical to the fused kernel's
in-register dequant and both arms run the same tile, so the bar is
bit-identical outputs, with and without bias and the GELU epilogue, and the
oracle bar on top.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

CASES = [  # M, K, N, bits, group, bias, epilogue
    (320, 4096, 4096, 8, 64, True, 0),     # config 0
    (256, 1024, 3072, 8, 64, False, 1),    # ff_in shape class, GELU fused
    (200, 512, 640, 4, 32, True, 0),
    (64, 2048, 2048, 8, 64, True, 0),      # the arm's M floor
]


@pytest.mark.parametrize("M,K,N,bits,group,has_bias,epi", CASES)
def test_dequant_once_arm_is_bit_identical_to_fused(pkg, dev, M, K, N, bits, group, has_bias,
                                                   epi):
    rng = np.random.default_rng(M * 7 + N)
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    w = rng_normal(rng, (N, K), 0.02)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, bits, group)
    bias = rng_normal(rng, (N,), 0.01) if has_bias else None
    xd = dev_bf16(x)
    bd = dev_f32(bias) if has_bias else None
    outs = []
    try:
        for arm in (False, True):
            pkg.set_dequant_once(arm)
            assert pkg.dequant_once_takes(M, K, N) == arm
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            say(f"linear_q M={M} K={K} N={N} w{bits}g{group} bias={has_bias} epi={epi} "
                f"dequant_once={arm}")
            pkg.linear_q(xd, qw, bd, y, M, K, N, epi)
            torch.cuda.synchronize()
            outs.append(host_bits(y))
    finally:
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    assert np.array_equal(outs[0], outs[1])
    ref = orc.linear_f64(orc.bf16_to_f32(x), orc.bf16_to_f32(wb), bias)
    if epi == 1:
        ref = orc.gelu(ref)
    got = orc.bf16_to_f32(outs[1])
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-2


def test_dequant_once_declines_below_the_mma_floor(pkg):
    pkg.set_dequant_once(True)
    try:
        assert not pkg.dequant_once_takes(63, 4096, 4096)
        assert not pkg.dequant_once_takes(126, 2048, 8)
        assert pkg.dequant_once_takes(64, 4096, 16)
    finally:
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    assert pkg.dequant_once_takes(8160, 4096, 16384)   # AUTO: tall shapes
    assert not pkg.dequant_once_takes(320, 4096, 4096)


TALL_CASES = [  # M, K, N, group, bias dtype, epilogue
    (1000, 1152, 2056, 64, "f32", 1),   # ragged M, N % 256 != 0, GELU, 18 K steps
    (520, 640, 1040, 32, "bf16", 0),    # group 32: two groups per 64-deep step
    (300, 4096, 1024, 64, None, 1),
    (300, 1024, 1030, 64, "f32", 0),    # N % 8 != 0: the template's 256 x 256 tile on both arms
]


@pytest.mark.parametrize("M,K,N,group,bias_kind,epi", TALL_CASES)
def test_fused_tall_tile_is_bit_identical_to_dequant_once(pkg, M, K, N, group, bias_kind, epi):
    """The 256 x 256 tile with w8 codes dequantized in registers once per workgroup
    (dequant-once OFF) against the same tile over the bf16 expansion (ON): identical
    bits, since both feed the MFMAs the same bf16 weights in the same K order; and the
    oracle bar."""
    rng = np.random.default_rng(M + 3 * N + group)
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    qw, codes, scales, biases, wb = make_qweight(pkg, rng_normal(rng, (N, K), 0.02), 8, group)
    bias = rng_normal(rng, (N,), 0.01) if bias_kind else None
    if bias_kind == "bf16":
        bias = orc.bf16_to_f32(orc.bf16_rne(bias))
        bd = dev_bf16(orc.bf16_rne(bias))
    else:
        bd = dev_f32(bias) if bias_kind else None
    xd = dev_bf16(x)
    outs = []
    pkg.set_tile(pkg.TILE_TALL)
    try:
        for arm in (False, True):
            pkg.set_dequant_once(arm)
            route = pkg.linear_route(M, K, N, 8)
            assert route["tile"] == pkg.TILE_TALL and route["dequant_once"] == int(arm)
            say(f"tall tile M={M} K={K} N={N} w8g{group} bias={bias_kind} epi={epi} "
                f"dequant_once={arm}")
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            pkg.linear_q(xd, qw, bd, y, M, K, N, epi)
            torch.cuda.synchronize()
            outs.append(host_bits(y))
    finally:
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
        pkg.set_tile(pkg.TILE_AUTO)
    assert np.array_equal(outs[0], outs[1])
    ref = orc.linear_f64(orc.bf16_to_f32(x), orc.bf16_to_f32(wb), bias)
    if epi == 1:
        ref = orc.gelu(ref)
    got = orc.bf16_to_f32(outs[0])
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-2
