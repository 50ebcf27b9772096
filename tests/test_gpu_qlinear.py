"""The quantized linear on the GPU, through the C ABI, against the oracle.

Mirrors tests/ltx25-qlinear-test.cc: its six cases (:190-197), its negative
control (:274-321), its bias control (:326-384) and its tile-routing bands
(:420-433), plus the DiT's own shapes (configs 0-2). The bars, written per
test:
  - bf16 output vs the oracle's f64-accumulated GEMM over the f32
    dequantized weight: max|y - ref| / max|ref| <= 1e-2;
  - vs the oracle over the bf16 dequantized weight (what the kernel
    multiplies): rel-L2 < 3e-3 (the reference's own bar);
  - quantized vs dense over the GPU-dequantized weight: bit-identical (the
    reference measured rel-L2 0.000e+00 for the same relation).
Full-size shapes are checked on sampled rows against the oracle and on all
rows against a torch fp32 GEMM of the same dequantized operands.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, host_f32, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2      # normwise max relative error, bf16 outputs
REL_L2 = 3e-3       # the reference's rel-L2 bar (tests/ltx25-qlinear-test.cc:191-196)


@pytest.fixture(autouse=True)
def _fp32_reference_matmul():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def run_q(pkg, x_dev, qw, bias, M, K, N, epi=0):
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.linear_q(x_dev, qw, bias, y, M, K, N, epi)
    torch.cuda.synchronize()
    return y


def run_dense(pkg, x_dev, w_dev, bias, M, K, N):
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.linear(x_dev, w_dev, bias, y, M, K, N)
    torch.cuda.synchronize()
    return y


def sample_rows(M, n=16, seed=0):
    rng = np.random.default_rng(seed)
    rows = set([0, M - 1]) | set(rng.integers(0, M, n).tolist())
    return np.array(sorted(rows))


def check_rows_vs_oracle(y_dev, x_f32, w_f32, bias_f32, rows, epilogue=None):
    ref = orc.linear_f64_d(x_f32[rows], w_f32, bias_f32)
    if epilogue == "gelu":
        ref = orc.gelu(ref.astype(np.float32)).astype(np.float64)
    got = host_f32(y_dev)[rows]
    mr = orc.max_rel(got, ref)
    r2 = orc.rel_l2(got, ref)
    assert mr <= MAX_REL, f"max-rel {mr:.3e}"
    assert r2 < REL_L2, f"rel-L2 {r2:.3e}"
    return mr, r2


def check_full_vs_torch(y_dev, x_dev, w_dev_bf16, bias_dev=None, gelu=False):
    ref = x_dev.float() @ w_dev_bf16.float().t()
    if bias_dev is not None:
        ref = ref + bias_dev.float()
    if gelu:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    d = (y_dev.float() - ref).abs().max().item() / ref.abs().max().item()
    r2 = ((y_dev.float() - ref).norm() / ref.norm()).item()
    assert d <= MAX_REL and r2 < REL_L2, f"full matrix: max-rel {d:.3e} rel-L2 {r2:.3e}"


# ---- the reference's six cases ----------------------------------------------------------
REF_CASES = [  # M, N, K, bits, group -- tests/ltx25-qlinear-test.cc:190-197
    (16, 128, 256, 8, 64),
    (192, 128, 256, 8, 64),
    (16, 128, 256, 4, 64),
    (192, 128, 256, 4, 64),
    (192, 128, 256, 4, 32),
    (192, 256, 512, 8, 32),
]


@pytest.mark.parametrize("M,N,K,bits,group", REF_CASES)
def test_reference_cases(pkg, M, N, K, bits, group):
    say(f"reference case M={M} N={N} K={K} w{bits}g{group}")
    rng = np.random.default_rng(7)
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K), 0.05))
    w = rng_normal(rng, (N, K), 0.05)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, bits, group)
    x_dev = dev_bf16(x_bits)
    yq = run_q(pkg, x_dev, qw, None, M, K, N)

    # quantized == dense over the dequantized weight, bit for bit
    w_deq_dev = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(qw, w_deq_dev, N, K)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(w_deq_dev), wb)
    yd = run_dense(pkg, x_dev, w_deq_dev, None, M, K, N)
    assert np.array_equal(host_bits(yq), host_bits(yd))

    xf = orc.bf16_to_f32(x_bits)
    got = host_f32(yq)
    assert orc.rel_l2(got, orc.linear_f64_d(xf, orc.bf16_to_f32(wb))) < REL_L2
    wf, _ = orc.dequant(codes, scales, biases, N, K, bits, group)
    assert orc.max_rel(got, orc.linear_f64_d(xf, wf)) <= MAX_REL
    assert np.abs(got).sum() > 0, "a kernel that never ran also compares equal"


def test_negative_control_one_code_flipped(pkg):
    say("negative control")
    M, N, K = 64, 128, 256
    rng = np.random.default_rng(8)
    x_dev = dev_bf16(orc.bf16_rne(rng_normal(rng, (M, K), 0.05)))
    w = rng_normal(rng, (N, K), 0.05)
    qa, codes, scales, biases, _ = make_qweight(pkg, w, 8, 64)
    bad = codes.copy()
    bad[0, 0] ^= 0xFF
    qb = pkg.QWeight(torch.from_numpy(bad.view(np.uint8).copy()).cuda(), qa.scales, qa.qbias, 8, 64)
    ya = run_q(pkg, x_dev, qa, None, M, K, N)
    yb = run_q(pkg, x_dev, qb, None, M, K, N)
    r = orc.rel_l2(host_f32(yb), host_f32(ya))
    assert r > 0.0, "the result does not depend on the codes"
    # and only column 0 moved
    diff = np.abs(host_f32(yb) - host_f32(ya)).sum(axis=0)
    assert diff[0] > 0 and np.all(diff[1:] == 0)


@pytest.mark.parametrize("bias_kind", ["bf16", "f32"])
def test_bias_is_fused_and_present(pkg, bias_kind):
    say(f"bias control ({bias_kind})")
    M, N, K = 64, 128, 256
    rng = np.random.default_rng(9)
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K), 0.05))
    w = rng_normal(rng, (N, K), 0.05)
    bias = rng_normal(rng, (N,), 0.05) * 4
    if bias_kind == "bf16":
        bias = orc.bf16_to_f32(orc.bf16_rne(bias))
        bias_dev = dev_bf16(orc.bf16_rne(bias))
    else:
        bias_dev = dev_f32(bias)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
    y = run_q(pkg, dev_bf16(x_bits), qw, bias_dev, M, K, N)
    xf = orc.bf16_to_f32(x_bits)
    wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    ref = orc.linear_f64_d(xf, wf, bias)
    got = host_f32(y)
    assert orc.max_rel(got, ref) <= MAX_REL
    assert orc.rel_l2(got, orc.linear_f64_d(xf, orc.bf16_to_f32(wb), bias)) < REL_L2
    # the bias is large enough that dropping it would fail the check above
    assert np.abs(bias).mean() > 0.1 * np.abs(ref).mean()
    assert orc.max_rel(got, ref - bias) > MAX_REL


# ---- tile routing bands (tests/ltx25-qlinear-test.cc:420-433) --------------------------
BANDS = [  # name, M, K, N
    ("small M, shallow K", 512, 4096, 4096),
    ("large M, shallow K (DiT attn)", 2048, 4096, 4096),
    ("large M, deep K", 2048, 12288, 512),
    ("deep K, narrow N (VAE L1)", 2427, 13824, 512),
    ("deep K, wide N (DiT ff_out)", 256, 16384, 4096),
    ("narrow-N guard (conv_out)", 2048, 3456, 48),
    ("narrow-N guard at N=128", 2048, 3456, 128),
    ("N=129, just past the guard", 2048, 3456, 129),
    ("N not a multiple of 512", 2048, 8192, 300),
    ("N not a multiple of 256", 192, 16384, 260),
]


@pytest.mark.parametrize("name,M,K,N", BANDS, ids=[b[0] for b in BANDS])
@pytest.mark.parametrize("quantized", [True, False], ids=["w8g64", "dense"])
def test_routing_bands(pkg, name, M, K, N, quantized):
    say(f"band {name} M={M} K={K} N={N} quantized={quantized}")
    rng = np.random.default_rng(10)
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K), 0.05))
    x_dev = dev_bf16(x_bits)
    w = rng_normal(rng, (N, K), 0.05)
    if quantized:
        qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
        y = run_q(pkg, x_dev, qw, None, M, K, N)
    else:
        wb = orc.bf16_rne(w)
        y = run_dense(pkg, x_dev, dev_bf16(wb), None, M, K, N)
    rows = sample_rows(M)
    check_rows_vs_oracle(y, orc.bf16_to_f32(x_bits), orc.bf16_to_f32(wb), None, rows)
    check_full_vs_torch(y, x_dev, dev_bf16(wb))


def test_unsupported_k_is_refused(pkg):
    x = torch.zeros((16, 81), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((128, 81), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((16, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(pkg.Ltx25Error) as e:
        pkg.linear(x, w, None, y, 16, 81, 128)
    assert e.value.code == pkg.E_UNSUPPORTED


# ---- the DiT's shapes ---------------------------------------------------------------------
def synth_linear(rng, M, K, N, bias=True):
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K), 1.0))
    w = rng_normal(rng, (N, K), 0.02)
    b = rng_normal(rng, (N,), 0.01) if bias else None
    return x_bits, w, b


def test_config0_single_linear_f32_bias(pkg):
    say("config 0: 320x4096->4096 w8g64, f32 bias")
    M, K, N = 320, 4096, 4096
    rng = np.random.default_rng(11)
    x_bits, w, b = synth_linear(rng, M, K, N)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
    x_dev = dev_bf16(x_bits)
    y = run_q(pkg, x_dev, qw, dev_f32(b), M, K, N)
    wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    rows = sample_rows(M, 24)
    check_rows_vs_oracle(y, orc.bf16_to_f32(x_bits), wf, b, rows)
    check_full_vs_torch(y, x_dev, dev_bf16(wb), dev_f32(b))


AUDIO = [("qkv", 2048, 6144), ("out", 2048, 2048), ("ff_up", 2048, 8192), ("ff_down", 8192, 2048)]


@pytest.mark.parametrize("name,K,N", AUDIO, ids=[a[0] for a in AUDIO])
def test_config1_audio_skinny(pkg, name, K, N):
    say(f"config 1: audio {name} 126x{K}->{N}")
    M = 126
    rng = np.random.default_rng(12)
    x_bits, w, b = synth_linear(rng, M, K, N)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
    x_dev = dev_bf16(x_bits)
    y = run_q(pkg, x_dev, qw, dev_f32(b), M, K, N)
    wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    check_rows_vs_oracle(y, orc.bf16_to_f32(x_bits), wf, b, sample_rows(M, 24))
    check_full_vs_torch(y, x_dev, dev_bf16(wb), dev_f32(b))
    y2 = run_q(pkg, x_dev, qw, dev_f32(b), M, K, N)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16)), "split-K is not deterministic"


def test_config2_video_ffn_pair(pkg):
    say("config 2: 8160x4096->16384 GELU ->4096 (quantize on GPU)")
    M, D, H = 8160, 4096, 16384
    g = torch.Generator(device="cuda")
    g.manual_seed(13)
    x = torch.randn((M, D), device="cuda", generator=g).to(torch.bfloat16)
    w1 = torch.randn((H, D), device="cuda", generator=g) * 0.02
    w2 = torch.randn((D, H), device="cuda", generator=g) * 0.02

    def gpu_quant(w):
        N, K = w.shape
        codes = torch.empty((N, K), dtype=torch.uint8, device="cuda")
        sc = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
        qb = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
        pkg.quantize_affine(w, codes, sc, qb, N, K, 8, 64)
        deq = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
        q = pkg.QWeight(codes, sc, qb, 8, 64)
        pkg.dequant(q, deq, N, K)
        return q, deq

    q1, d1 = gpu_quant(w1)
    q2, d2 = gpu_quant(w2)
    h = run_q(pkg, x, q1, None, M, D, H, pkg.EPI_GELU_TANH)
    y = run_q(pkg, h, q2, None, M, H, D)
    rows = sample_rows(M, 12)
    xf = host_f32(x)
    check_rows_vs_oracle(h, xf, host_f32(d1), None, rows, epilogue="gelu")
    check_rows_vs_oracle(y, host_f32(h), host_f32(d2), None, rows)
    check_full_vs_torch(h, x, d1, gelu=True)
    check_full_vs_torch(y, h, d2)


# One joint audio-video block's linear set (config 4), at the real token counts: video 8160,
# audio 126, text 1024. Fused QKV (N = 3 x inner) and text K/V packs, f32 biases where the
# block has them, GELU fused into both ff_in projections. The video launches take the
# dequant-once route (M >= 4096), the text and audio ones the fused kernel.
BLOCK4 = [
    ("v_qkv", 8160, 4096, 12288, True, False), ("v_out", 8160, 4096, 4096, True, False),
    ("v_xkv", 1024, 4096, 8192, True, False), ("v_ff_up", 8160, 4096, 16384, False, True),
    ("v_ff_down", 8160, 16384, 4096, False, False), ("a_qkv", 126, 2048, 6144, True, False),
    ("a_xkv", 1024, 2048, 4096, True, False), ("a_ff_up", 126, 2048, 8192, True, True),
    ("a_ff_down", 126, 8192, 2048, True, False), ("a2v_q", 8160, 4096, 2048, True, False),
    ("a2v_o", 8160, 2048, 4096, True, False), ("v2a_kv", 8160, 4096, 4096, True, False),
]


@pytest.mark.parametrize("name,M,K,N,has_bias,gelu", BLOCK4, ids=[b[0] for b in BLOCK4])
def test_config4_block_linear_set(pkg, name, M, K, N, has_bias, gelu):
    say(f"config 4: {name} {M}x{K}->{N} bias={has_bias} gelu={gelu}")
    g = torch.Generator(device="cuda")
    g.manual_seed(40 + len(name) * 7 + N)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    codes = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    sc = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    qb = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    pkg.quantize_affine(w, codes, sc, qb, N, K, 8, 64)
    q = pkg.QWeight(codes, sc, qb, 8, 64)
    deq = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(q, deq, N, K)
    b = (torch.randn((N,), device="cuda", generator=g) * 0.01) if has_bias else None
    y = run_q(pkg, x, q, b, M, K, N, pkg.EPI_GELU_TANH if gelu else pkg.EPI_NONE)
    bias_h = host_f32(b) if has_bias else None
    check_rows_vs_oracle(y, host_f32(x), host_f32(deq), bias_h, sample_rows(M, 6),
                         epilogue="gelu" if gelu else None)
    check_full_vs_torch(y, x, deq, b, gelu=gelu)


def test_gelu_epilogue_matches_separate_gelu(pkg):
    say("fused GELU epilogue vs linear then gelu")
    M, K, N = 300, 512, 640
    rng = np.random.default_rng(14)
    x_bits, w, b = synth_linear(rng, M, K, N)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
    x_dev = dev_bf16(x_bits)
    fused = run_q(pkg, x_dev, qw, dev_f32(b), M, K, N, pkg.EPI_GELU_TANH)
    wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    check_rows_vs_oracle(fused, orc.bf16_to_f32(x_bits), wf, b, np.arange(M), epilogue="gelu")


def test_golden_qlinear_fixture(pkg):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "qlinear_w8g64_m16.npz"))
    N, K = (int(v) for v in g["w_shape"])
    M = g["x_bf16"].shape[0]
    qw = pkg.QWeight(torch.from_numpy(g["codes"].view(np.uint8).reshape(N, -1).copy()).cuda(),
                     dev_bf16(g["scales"]), dev_bf16(g["biases"]), 8, 64)
    y = run_q(pkg, dev_bf16(g["x_bf16"]), qw, dev_f32(g["bias_f32"]), M, K, N)
    got = host_f32(y)
    assert orc.max_rel(got, g["y_f32"]) <= MAX_REL
    assert orc.rel_l2(got, g["y_f32"]) < REL_L2
