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

F, RF, P = "fused", "rfirst", "pair"
SHAPES = [  # name, M, K, N, rank, the route AUTO takes
    ("square self-attention projection", 12, 64, 64, 3, F),
    ("cross-attention key (narrow in)", 8, 32, 64, 3, F),
    ("cross-attention key (wide in)", 12, 64, 32, 3, F),
    ("the per-head gate (4 columns out)", 12, 64, 4, 3, F),
    ("the feed-forward widening", 12, 64, 256, 5, F),
    ("rank 1", 6, 64, 64, 1, F),
    ("x2 upscaler: attn projection", 128, 4096, 4096, 32, F),
    ("x2 upscaler: ff widening", 128, 4096, 16384, 32, F),
    ("distilled adapter: rank 450", 64, 1024, 1024, 450, F),
    # beyond the reference's table
    ("odd K, odd N (element-wise loads)", 45, 37, 30, 6, F),
    ("video tokens, rank 64", 1000, 512, 768, 64, RF),
    ("two launches (rank 600)", 70, 256, 192, 600, F),
    ("two launches, padded rank (530)", 96, 256, 320, 530, F),
    ("N not a multiple of 8 (element-wise y)", 40, 128, 4100, 16, F),
    # the GEMM pair (M >= 256, rank >= 96): rank padded to 64 with zero rows / columns
    ("GEMM pair, rank 128, no padding", 300, 2048, 1024, 128, P),
    ("GEMM pair, rank 450 padded to 512", 512, 1024, 2048, 450, P),
    ("GEMM pair, ragged M and N", 777, 512, 1000, 200, P),
    ("GEMM pair, rank 1000 (split-K second GEMM)", 256, 512, 640, 1000, P),
    # r first (M >= 512, rank % 8 == 0, rank < 96): r = x . A^T by the dense GEMM, then the
    # fused kernel's second phase reads it
    ("r first: rank 32 at the FFN width", 1024, 4096, 16384, 32, RF),
    ("r first: rank 40, ragged M", 777, 1024, 2048, 40, RF),
    ("r first: rank 8", 600, 512, 1024, 8, RF),
    # N not a multiple of the 512-column super-block stride: the y loads issued four
    # super blocks ahead (ranks up to 64) run past the column split's end
    ("r first: rank 16, ragged N", 640, 1024, 1000, 16, RF),
    ("r first: rank 64, N = 4104", 520, 256, 4104, 64, RF),
    # more rows: r's GEMM covers the CUs with fewer K splits; ragged M, a rank that is not a
    # multiple of 16, K that is not a multiple of 512
    ("r first, 2085 rows: rank 40, K = 2624", 2085, 2624, 1024, 40, RF),
    ("r first, 2112 rows: rank 8, K = 1088", 2112, 1088, 256, 8, RF),
    ("r first, 2048 rows: rank 64, K = 4096", 2048, 4096, 512, 64, RF),
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


ROUTE = {F: 3, RF: 2, P: 1}   # LTX25_LORA_FUSED / _RFIRST / _PAIR


def run_and_check(pkg, what, M, K, N, rank):
    x, a, b, y0 = draws(what, M, K, N, rank)
    xb, ab, bb, yb = (orc.bf16_rne(t) for t in (x, a, b, y0))
    xd, ad, bd, yd = (dev_bf16(t) for t in (xb, ab, bb, yb))
    route = pkg.lora_route(xd, ad, bd, yd, M, K, N, rank)
    pkg.lora_add(xd, ad, bd, yd, M, K, N, rank)
    torch.cuda.synchronize()
    got = orc.bf16_to_f32(host_bits(yd))
    ref = orc.bf16_to_f32(orc.lora_add(xb, ab, bb, yb))
    assert max_rel(got, ref) <= MAX_REL, what
    want = y0.astype(np.float64) + (x.astype(np.float64) @ a.T.astype(np.float64)) @ b.T
    assert orc.rel_l2(got, want) < REL_L2, what
    # and it ADDED: y changed where the delta is not negligible
    assert not np.array_equal(host_bits(yd), yb)
    return route


@pytest.mark.parametrize("what,M,K,N,rank,route", SHAPES, ids=[s[0] for s in SHAPES])
def test_lora_add_against_oracle_and_f64(pkg, dev, what, M, K, N, rank, route):
    say(f"lora_add {what}: M={M} K={K} N={N} rank={rank}")
    assert pkg.lora_on_matrix_cores(M, K, N, rank) == (route == P)
    assert run_and_check(pkg, what, M, K, N, rank) == ROUTE[route]


# the same shapes on every route that can take them (the A/B hook, ltx25_set_lora_route)
FORCED = [s for s in SHAPES if s[0] in (
    "x2 upscaler: attn projection", "distilled adapter: rank 450", "video tokens, rank 64",
    "GEMM pair, ragged M and N", "r first: rank 32 at the FFN width", "r first: rank 16, ragged N")]


@pytest.mark.parametrize("forced", [P, RF, F])
@pytest.mark.parametrize("what,M,K,N,rank,route", FORCED, ids=[s[0] for s in FORCED])
def test_lora_forced_routes_agree(pkg, dev, what, M, K, N, rank, route, forced):
    say(f"lora_add forced {forced}: {what}: M={M} K={K} N={N} rank={rank}")
    pkg.set_lora_route(ROUTE[forced])
    try:
        if forced == RF and rank % 8 != 0:
            # r first needs rank % 8 == 0: refused before any device use, y untouched
            yd = torch.ones((M, N), dtype=torch.bfloat16, device="cuda")
            xd = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
            ad = torch.zeros((rank, K), dtype=torch.bfloat16, device="cuda")
            bd = torch.zeros((N, rank), dtype=torch.bfloat16, device="cuda")
            with pytest.raises(pkg.Ltx25Error) as e:
                pkg.lora_add(xd, ad, bd, yd, M, K, N, rank)
            assert e.value.code == pkg.E_UNSUPPORTED
            return
        assert run_and_check(pkg, what, M, K, N, rank) == ROUTE[forced]
    finally:
        pkg.set_lora_route(pkg.LORA_AUTO)


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


# the reference's caller scratch r ([M][rank]): the r-first route, and the GEMM pair at a
# rank that is a multiple of 64, compute r into it instead of the library's scratch
CALLER_R = [("r first: rank 40, ragged M", 777, 1024, 2048, 40, RF),
            ("r first: rank 56, 2085 rows", 2085, 2624, 512, 56, RF),
            ("GEMM pair, rank 128, no padding", 300, 2048, 1024, 128, P)]


@pytest.mark.parametrize("what,M,K,N,rank,route", CALLER_R, ids=[s[0] for s in CALLER_R])
def test_lora_caller_r_holds_r(pkg, dev, what, M, K, N, rank, route):
    say(f"lora_add with the caller's r: {what}: M={M} K={K} N={N} rank={rank}")
    x, a, b, y0 = draws(what, M, K, N, rank)
    xb, ab, bb, yb = (orc.bf16_rne(t) for t in (x, a, b, y0))
    xd, ad, bd = (dev_bf16(t) for t in (xb, ab, bb))
    assert pkg.lora_route(xd, ad, bd, dev_bf16(yb), M, K, N, rank) == ROUTE[route]
    # the library's scratch, then the caller's r (NaN-filled first): same kernels, same bits
    y_lib = dev_bf16(yb)
    pkg.lora_add(xd, ad, bd, y_lib, M, K, N, rank)
    r = torch.full((M, rank), float("nan"), dtype=torch.bfloat16, device="cuda")
    y_r = dev_bf16(yb)
    pkg.lora_add(xd, ad, bd, y_r, M, K, N, rank, r=r)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y_r), host_bits(y_lib))
    got = orc.bf16_to_f32(host_bits(y_r))
    ref = orc.bf16_to_f32(orc.lora_add(xb, ab, bb, yb))
    assert max_rel(got, ref) <= MAX_REL
    # r = bf16(x . a^T) landed in the caller's buffer
    r_got = orc.bf16_to_f32(host_bits(r))
    r_ref = orc.bf16_to_f32(xb).astype(np.float64) @ orc.bf16_to_f32(ab).astype(np.float64).T
    assert np.isfinite(r_got).all()
    assert max_rel(r_got, r_ref) <= MAX_REL
