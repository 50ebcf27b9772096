"""The low-rank adapter delta on the GPU, through the C ABI, against the oracle.

Mirrors tests/ltx25-lora-apply-test.cc (layer one, :383-470): every shape of
its table, including the three the published adapters run (the x2
upscaler's rank 32 at 128 tokens over 4096 and 16384 columns, and the
distilled adapter's rank 450), with its bar -- rel-L2 < 2e-2 against f64 over
the unrounded draws -- and the north-star bar against the oracle, which
applies the same bf16 rounding of r: max|y - ref| / max|ref| <= 1e-2. Plus the
shapes that take the element-wise load path, an adapter wider than one launch
(rank > 512), the matrix-core GEMM pair (rank >= 96), the r-first route (many
tokens: r by the dense GEMM, then the fused kernel's second phase), the
empty-shape no-op and A = 0 (y bit-identical).
"""
import zlib

import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, host_bits, say

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2   # normwise max relative error vs the oracle
REL_L2 = 2e-2    # the reference's bar (tests/ltx25-lora-apply-test.cc:456-465)

SHAPES = [
    ("square self-attention projection", 12, 64, 64, 3),
    ("cross-attention key (narrow in)", 8, 32, 64, 3),
    ("cross-attention key (wide in)", 12, 64, 32, 3),
    ("the per-head gate (4 columns out)", 12, 64, 4, 3),
    ("the feed-forward widening", 12, 64, 256, 5),
    ("rank 1", 6, 64, 64, 1),
    ("x2 upscaler: attn projection", 128, 4096, 4096, 32),
    ("x2 upscaler: ff widening", 128, 4096, 16384, 32),
    ("distilled adapter: rank 450", 64, 1024, 1024, 450),
    # beyond the reference's table
    ("odd K, odd N (element-wise loads)", 45, 37, 30, 6),
    ("video tokens, rank 64", 1000, 512, 768, 64),
    ("two launches (rank 600)", 70, 256, 192, 600),
    ("two launches, padded rank (530)", 96, 256, 320, 530),
    ("N not a multiple of 8 (element-wise y)", 40, 128, 4100, 16),
    # the GEMM pair (M >= 256, rank >= 64): rank padded to 64 with zero rows / columns
    ("GEMM pair, rank 128, no padding", 300, 2048, 1024, 128),
    ("GEMM pair, rank 450 padded to 512", 512, 1024, 2048, 450),
    ("GEMM pair, ragged M and N", 777, 512, 1000, 200),
    ("GEMM pair, rank 1000 (split-K second GEMM)", 256, 512, 640, 1000),
    # r first (M >= 512, rank % 8 == 0, rank < 96): r = x . A^T by the dense GEMM, then the
    # fused kernel's second phase reads it
    ("r first: rank 32 at the FFN width", 1024, 4096, 16384, 32),
    ("r first: rank 40, ragged M", 777, 1024, 2048, 40),
    ("r first: rank 8", 600, 512, 1024, 8),
    # N not a multiple of the 512-column super-block stride: the y loads issued four
    # super blocks ahead (ranks up to 64) run past the column split's end
    ("r first: rank 16, ragged N", 640, 1024, 1000, 16),
    ("r first: rank 64, N = 4104", 520, 256, 4104, 64),
]


def draws(tag, M, K, N, rank):
    rng = np.random.default_rng(zlib.crc32(tag.encode()))
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = (rng.standard_normal((rank, K)) * 0.5).astype(np.float32)
    b = (rng.standard_normal((N, rank)) * 0.5).astype(np.float32)
    y = rng.standard_normal((M, N)).astype(np.float32)
    return x, a, b, y


def max_rel(got, ref):
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("what,M,K,N,rank", SHAPES, ids=[s[0] for s in SHAPES])
def test_lora_add_against_oracle_and_f64(pkg, dev, what, M, K, N, rank):
    x, a, b, y0 = draws(what, M, K, N, rank)
    xb, ab, bb, yb = (orc.bf16_rne(t) for t in (x, a, b, y0))
    xd, ad, bd, yd = (dev_bf16(t) for t in (xb, ab, bb, yb))
    say(f"lora_add {what}: M={M} K={K} N={N} rank={rank}")
    assert pkg.lora_on_matrix_cores(M, K, N, rank)
    pkg.lora_add(xd, ad, bd, yd, M, K, N, rank)
    torch.cuda.synchronize()
    got = orc.bf16_to_f32(host_bits(yd))
    ref = orc.bf16_to_f32(orc.lora_add(xb, ab, bb, yb))
    assert max_rel(got, ref) <= MAX_REL, what
    want = y0.astype(np.float64) + (x.astype(np.float64) @ a.T.astype(np.float64)) @ b.T
    assert orc.rel_l2(got, want) < REL_L2, what
    # and it ADDED: y changed where the delta is not negligible
    assert not np.array_equal(host_bits(yd), yb)


def test_lora_zero_adapter_leaves_y_bit_identical(pkg, dev):
    M, K, N, rank = 96, 256, 320, 16
    x, a, b, y0 = draws("zero", M, K, N, rank)
    yb = orc.bf16_rne(y0)
    yd = dev_bf16(yb)
    say("lora_add with A = 0")
    pkg.lora_add(dev_bf16(orc.bf16_rne(x)), torch.zeros((rank, K), dtype=torch.bfloat16,
                                                          device="cuda"),
                 dev_bf16(orc.bf16_rne(b)), yd, M, K, N, rank)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(yd), yb)


def test_lora_empty_shape_is_a_no_op(pkg, dev):
    yb = orc.bf16_rne(np.ones((4, 8), np.float32))
    yd = dev_bf16(yb)
    say("lora_add with M = 0 and rank = 0")
    pkg.lora_add(yd, yd, yd, yd, 0, 8, 8, 4)
    pkg.lora_add(yd, yd, yd, yd, 4, 8, 8, 0)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(yd), yb)
    assert not pkg.lora_on_matrix_cores(0, 8, 8, 4)


def test_lora_is_deterministic(pkg, dev):
    M, K, N, rank = 256, 1024, 2048, 32
    x, a, b, y0 = draws("determinism", M, K, N, rank)
    xd, ad, bd = (dev_bf16(orc.bf16_rne(t)) for t in (x, a, b))
    outs = []
    for i in range(2):
        yd = dev_bf16(orc.bf16_rne(y0))
        say(f"lora_add determinism run {i}")
        pkg.lora_add(xd, ad, bd, yd, M, K, N, rank)
        torch.cuda.synchronize()
        outs.append(host_bits(yd))
    assert np.array_equal(outs[0], outs[1])
