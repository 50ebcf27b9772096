"""The int8 tier on the GPU, through the C ABI.

Bit-exact against the oracle: the per-row quantizer, the int32
accumulators, and the bf16 outputs of the fused dequant epilogue (a fixed
f32 sequence). At the full video shape (config 3) the accumulators are
checked on sampled rows against the oracle and on all rows against an
exact float64 GEMM of the same int8 operands. Inside `linear` the tier is
checked as tests/ltx25-i8-gemm-test.cc checks it: taken where its gates say,
within (1e-5, 3e-2) rel-L2 of the bf16 path, and bit-equal to it where
refused.
"""
import os

import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, host_f32, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def i8_run(pkg, xq, sx, wq, sw, bias, M, K, N, want_acc=True):
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda") if want_acc else None
    pkg.i8_gemm(xq, sx, wq, sw, bias, y, acc, M, K, N)
    torch.cuda.synchronize()
    return y, acc


def quantize_rows_dev(pkg, x_dev, M, K):
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    pkg.i8_quantize_rows(x_dev, q, s, M, K)
    torch.cuda.synchronize()
    return q, s


@pytest.mark.parametrize("M,K", [(70, 4096), (9, 20480)])   # 20480: past the register cache
def test_quantize_rows_bit_exact(pkg, M, K):
    say(f"i8 quantize rows M={M} K={K}")
    rng = np.random.default_rng(30 + K)
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    x[4] = 0
    x[5, 17] = orc.bf16_rne(np.array([300.0], np.float32))[0]   # one outlier
    q, s = quantize_rows_dev(pkg, dev_bf16(x), M, K)
    q_ref, s_ref = orc.i8_quantize_rows(x)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


def test_quantize_rows_at_half_integer_quotients(pkg):
    """Values whose quotient v / s sits on or next to a half-integer: the
    quantizer's reciprocal fast path must hand these to the division (ties
    to even, and the nearest integer on either side of a tie)."""
    K = 512
    rows = []
    r0 = np.zeros(K, np.float32)   # amax 127: s = 1 exactly, exact ties
    ties = np.array([2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5, 64.5, -65.5, 100.5], np.float32)
    r0[:ties.size] = ties
    r0[ties.size] = 127.0
    rows.append(r0)
    for amax in (1.0, 0.75, 3.0, 1e-3, 5e4):   # s = amax / 127: quotients next to the ties
        s = np.float32(amax) / np.float32(127.0)
        k = (np.arange(K) % 254) - 127
        r = ((k + 0.5) * s).astype(np.float32)
        r[0] = amax
        rows.append(r)
    # (amax, v) where v * fl(1 / s) rounds to the other side of 63.5 than v / s
    # does (found by an exhaustive search over bf16 values)
    for amax, v in ((27.0, 13.5), (1.6640625, 0.83203125), (91.5, 45.75), (72.0, 36.0),
                    (87.5, 43.75), (15.0625, 7.53125)):
        r = np.zeros(K, np.float32)
        r[0], r[1], r[2] = amax, v, -v
        rows.append(r)
    x = orc.bf16_rne(np.stack(rows))
    M = x.shape[0]
    say(f"i8 quantize rows at half-integer quotients M={M} K={K}")
    q, sc = quantize_rows_dev(pkg, dev_bf16(x), M, K)
    q_ref, s_ref = orc.i8_quantize_rows(x)
    assert np.array_equal(sc.cpu().numpy(), s_ref)
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("N,K,bits,group", [
    (48, 2048, 8, 64), (40, 4096, 8, 32), (33, 4096, 4, 64), (17, 2048, 4, 32),
    (6, 36864, 8, 64),     # w8: 2304 chunks per row, past the register cache
    (4, 69632, 4, 64),     # w4: 2176 chunks per row
])
def test_quantize_qweight_bit_exact(pkg, N, K, bits, group):
    say(f"i8 quantize of a w{bits}g{group} weight N={N} K={K}")
    rng = np.random.default_rng(31 + K + bits)
    qw, codes, scales, biases, wb = make_qweight(pkg, rng_normal(rng, (N, K), 0.02), bits, group)
    wq = torch.empty((N, K), dtype=torch.int8, device="cuda")
    sw = torch.empty((N,), dtype=torch.float32, device="cuda")
    pkg.i8_quantize_qweight(qw, wq, sw, N, K)
    torch.cuda.synchronize()
    q_ref, s_ref = orc.i8_quantize_rows(wb)
    assert np.array_equal(sw.cpu().numpy(), s_ref)
    assert np.array_equal(wq.cpu().numpy(), q_ref)


def test_golden_i8_fixture(pkg):
    g = np.load(os.path.join(GOLDEN, "i8_m32.npz"))
    M, K = g["x_bf16"].shape
    N = g["w_bf16"].shape[0]
    xq, sx = quantize_rows_dev(pkg, dev_bf16(g["x_bf16"]), M, K)
    wq, sw = quantize_rows_dev(pkg, dev_bf16(g["w_bf16"]), N, K)
    assert np.array_equal(xq.cpu().numpy(), g["xq"])
    assert np.array_equal(wq.cpu().numpy(), g["wq"])
    y, acc = i8_run(pkg, xq, sx, wq, sw, dev_f32(g["bias_f32"]), M, K, N)
    assert np.array_equal(acc.cpu().numpy(), g["acc"])
    assert np.array_equal(host_bits(y), g["y_bf16"])


@pytest.mark.parametrize("M,K,N,bias_kind", [
    (64, 256, 64, "none"),
    (200, 512, 300, "f32"),
    (1030, 1024, 130, "bf16"),
    (300, 4096, 4096, "f32"),
])
def test_i8_gemm_bit_exact(pkg, M, K, N, bias_kind):
    say(f"i8 gemm M={M} K={K} N={N} bias={bias_kind}")
    rng = np.random.default_rng(32)
    xq_h = rng.integers(-127, 128, (M, K), dtype=np.int8)
    wq_h = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sx_h = (rng.random(M) * 0.05).astype(np.float32)
    sw_h = (rng.random(N) * 0.001).astype(np.float32)
    bias_h = rng_normal(rng, (N,), 0.5)
    if bias_kind == "none":
        bias_dev, bdt, bias_o = None, 0, None
    elif bias_kind == "f32":
        bias_dev, bdt, bias_o = dev_f32(bias_h), 2, bias_h
    else:
        bb = orc.bf16_rne(bias_h)
        bias_dev, bdt, bias_o = dev_bf16(bb), 1, bb
    y, acc = i8_run(pkg, torch.from_numpy(xq_h).cuda(), dev_f32(sx_h),
                    torch.from_numpy(wq_h).cuda(), dev_f32(sw_h), bias_dev, M, K, N)
    acc_ref = orc.i8_gemm_i32(xq_h, wq_h)
    assert np.array_equal(acc.cpu().numpy(), acc_ref)
    y_ref = orc.i8_epilogue(acc_ref, sx_h, sw_h, bias_o, bdt)
    assert np.array_equal(host_bits(y), y_ref)


@pytest.mark.parametrize("M,K,N,bias_kind", [
    (4100, 1152, 4104, "bf16"),   # 17 x 17 tiles, ragged in M and N: the 256 x 256 int8 tile
    (4100, 1152, 4100, "f32"),    # N % 8 != 0: the template's 256 x 256 tile
    (2304, 640, 8192, "none"),    # 9 x 32 tiles, 5 K steps of 128
])
def test_i8_gemm_tall_tiles_bit_exact(pkg, M, K, N, bias_kind):
    """Shapes whose 256 x 256 tiles fill the GPU: int32 accumulators equal to an exact
    float64 GEMM of the same operands on every row, and every bf16 output equal to the
    oracle's epilogue over those accumulators."""
    say(f"i8 gemm (256 x 256 tiles) M={M} K={K} N={N} bias={bias_kind}")
    rng = np.random.default_rng(38)
    xq_h = rng.integers(-127, 128, (M, K), dtype=np.int8)
    wq_h = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sx_h = (rng.random(M) * 0.05).astype(np.float32)
    sw_h = (rng.random(N) * 0.001).astype(np.float32)
    bias_h = rng_normal(rng, (N,), 0.5)
    if bias_kind == "none":
        bias_dev, bdt, bias_o = None, 0, None
    elif bias_kind == "f32":
        bias_dev, bdt, bias_o = dev_f32(bias_h), 2, bias_h
    else:
        bb = orc.bf16_rne(bias_h)
        bias_dev, bdt, bias_o = dev_bf16(bb), 1, bb
    xq, wq = torch.from_numpy(xq_h).cuda(), torch.from_numpy(wq_h).cuda()
    y, acc = i8_run(pkg, xq, dev_f32(sx_h), wq, dev_f32(sw_h), bias_dev, M, K, N)
    exact = xq.double() @ wq.double().t()
    assert torch.equal(acc.double(), exact)
    del exact
    acc_h = acc.cpu().numpy()
    assert np.array_equal(host_bits(y), orc.i8_epilogue(acc_h, sx_h, sw_h, bias_o, bdt))
    # a small corner of the accumulators against the oracle's own int32 GEMM
    assert np.array_equal(acc_h[-40:, -24:], orc.i8_gemm_i32(xq_h[-40:], wq_h[-24:]))


@pytest.mark.parametrize("N", [4096, 16384])
def test_config3_video_shape(pkg, N):
    say(f"config 3: i8 8160x4096->{N}")
    M, K = 8160, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(33)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn((N, K), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    xq, sx = quantize_rows_dev(pkg, x, M, K)
    wq, sw = quantize_rows_dev(pkg, w, N, K)
    y, acc = i8_run(pkg, xq, sx, wq, sw, None, M, K, N)
    # all rows: exact float64 GEMM over the same int8 operands
    exact = xq.double() @ wq.double().t()
    assert torch.equal(acc.double(), exact)
    del exact
    # sampled rows against the oracle (quantizer, int32 GEMM and epilogue)
    rows = np.array([0, 1, 4095, 8159] + list(np.random.default_rng(34).integers(0, M, 4)))
    x_h = host_bits(x)[rows]
    w_h = host_bits(w)
    q_ref, s_ref = orc.i8_quantize_rows(x_h)
    wq_ref, sw_ref = orc.i8_quantize_rows(w_h)
    assert np.array_equal(xq.cpu().numpy()[rows], q_ref)
    assert np.array_equal(wq.cpu().numpy(), wq_ref)
    acc_ref = orc.i8_gemm_i32(q_ref, wq_ref)
    assert np.array_equal(acc.cpu().numpy()[rows], acc_ref)
    assert np.array_equal(host_bits(y)[rows], orc.i8_epilogue(acc_ref, s_ref, sw_ref))
    # and the tier's stated error against the bf16 product (~1e-2 rel-L2)
    ref = x.float() @ w.float().t()
    r = ((y.float() - ref).norm() / ref.norm()).item()
    assert 1e-5 < r < 3e-2


TIER_SHAPES = [  # tests/ltx25-i8-gemm-test.cc:154-166
    ("attn projection", 8160, 4096, 4096, True),
    ("ff widening", 8160, 4096, 16384, True),
    ("ff narrowing", 8160, 16384, 4096, True),
    ("cross-attn k", 8160, 3840, 4096, True),
    ("short M (refused)", 512, 4096, 4096, False),
    ("shallow K (refused)", 8160, 512, 4096, False),
]


@pytest.mark.parametrize("name,M,K,N,want", TIER_SHAPES, ids=[t[0] for t in TIER_SHAPES])
def test_tier_inside_linear(pkg, name, M, K, N, want):
    say(f"i8 tier inside linear: {name}")
    g = torch.Generator(device="cuda")
    g.manual_seed(35)
    x = (torch.randn((M, K), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    w = (torch.randn((N, K), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    base = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    acc = torch.empty_like(base)
    pkg.set_i8_gemm(False)
    pkg.linear(x, w, None, base, M, K, N)
    pkg.set_i8_gemm(True)
    try:
        assert pkg.i8_takes(M, K, N) == want
        pkg.linear(x, w, None, acc, M, K, N)
        torch.cuda.synchronize()
    finally:
        pkg.set_i8_gemm(False)
    r = ((acc.float() - base.float()).norm() / base.float().norm()).item()
    if want:
        assert 1e-5 < r < 3e-2, f"rel-L2 {r:.3e}"
    else:
        assert r == 0.0


def test_tier_with_gelu_epilogue_bit_exact_accumulators(pkg):
    """linear_q_ex with the GELU epilogue takes the tier (the reference's tier sits under
    ff_in too, src/ltx25-metal-ops.cc:376-391): the tier's own operands re-derived by the
    oracle give the same int32 products, and the output is the oracle's epilogue + GELU
    within one bf16 ulp (the kernel's GELU uses the hardware exp2 / reciprocal)."""
    M, K, N = 1024, 1024, 320
    say(f"i8 tier + GELU inside linear_q_ex {M}x{K}->{N}")
    rng = np.random.default_rng(36)
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K)))
    qw, codes, scales, biases, wb = make_qweight(pkg, rng_normal(rng, (N, K), 0.02))
    bias = rng_normal(rng, (N,), 0.01)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.set_i8_gemm(True)
    try:
        assert pkg.i8_takes(M, K, N)
        assert pkg.linear_route(M, K, N)["i8"] == 1
        pkg.linear_q(dev_bf16(x_bits), qw, dev_f32(bias), y, M, K, N, pkg.EPI_GELU_TANH)
        torch.cuda.synchronize()
    finally:
        pkg.set_i8_gemm(False)
    xq, sx = orc.i8_quantize_rows(x_bits)
    wq, sw = orc.i8_quantize_rows(wb)
    acc = orc.i8_gemm_i32(xq, wq)
    want = orc.bf16_to_f32(orc.i8_epilogue(acc, sx, sw, bias, 2, epilogue=1))
    got = host_f32(y)
    ulp = np.abs(want) * 2.0 ** -7
    assert np.all(np.abs(got - want) <= np.maximum(ulp, 1e-6))
    # GELU was applied: the no-epilogue tier output differs on negative values
    plain = orc.bf16_to_f32(orc.i8_epilogue(acc, sx, sw, bias, 2))
    assert np.mean(np.abs(got - plain) > 0) > 0.3


def test_tier_with_gelu_at_the_ffn_shape(pkg):
    """8160 x 4096 -> 16384 with GELU, tier on: the route says int8, and the result is
    within the tier's stated band of the bf16 route's (tests/ltx25-i8-gemm-test.cc:207-215)."""
    M, K, N = 8160, 4096, 16384
    say(f"i8 tier + GELU at the FFN shape {M}x{K}->{N}")
    g = torch.Generator(device="cuda")
    g.manual_seed(37)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    codes = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    sc = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    qb = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    pkg.quantize_affine(w, codes, sc, qb, N, K, 8, 64)
    del w
    qw = pkg.QWeight(codes, sc, qb, 8, 64)
    base = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    tier = torch.empty_like(base)
    pkg.linear_q(x, qw, None, base, M, K, N, pkg.EPI_GELU_TANH)
    pkg.set_i8_gemm(True)
    try:
        assert pkg.i8_takes(M, K, N)
        assert pkg.linear_route(M, K, N)["i8"] == 1
        pkg.linear_q(x, qw, None, tier, M, K, N, pkg.EPI_GELU_TANH)
        torch.cuda.synchronize()
    finally:
        pkg.set_i8_gemm(False)
    r = ((tier.float() - base.float()).norm() / base.float().norm()).item()
    assert 1e-5 < r < 3e-2, f"rel-L2 {r:.3e}"
