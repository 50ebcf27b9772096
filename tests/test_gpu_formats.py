"""The byte/format kernels on the GPU against the oracle, bit for bit:
dequant-once, the group-affine quantizer, u32 pack/unpack, the loader's
F16 -> bf16 conversion and the standalone bias pass. GELU is floating point
(one bf16 ulp against the oracle's f64 form)."""
import os

import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_bytes, dev_f32, host_bits, host_f32, rng_normal, say

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("bits,group", [(8, 64), (8, 32), (4, 64), (4, 32)])
def test_dequant_bit_exact(pkg, bits, group):
    say(f"dequant w{bits}g{group}")
    N, K = 96, 1024
    rng = np.random.default_rng(20)
    w = rng_normal(rng, (N, K), 0.02)
    codes, scales, biases, _ = orc.quantize_affine(w, bits, group)
    qw = pkg.QWeight(dev_bytes(codes), dev_bf16(scales), dev_bf16(biases), bits, group)
    out = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(qw, out, N, K)
    torch.cuda.synchronize()
    _, wb = orc.dequant(codes, scales, biases, N, K, bits, group)
    assert np.array_equal(host_bits(out), wb)


@pytest.mark.parametrize("bits,group", [(8, 64), (8, 32), (4, 64), (4, 32)])
def test_quantize_affine_bit_exact(pkg, bits, group):
    say(f"quantize w{bits}g{group}")
    N, K = 64, 2048
    rng = np.random.default_rng(21)
    w = rng_normal(rng, (N, K), 0.02)
    w[5, :group] = 0.25                      # constant group: scale 0
    w[6, :] = rng_normal(rng, (K,), 30.0)    # wide range
    codes_ref, scales_ref, biases_ref, _ = orc.quantize_affine(w, bits, group)
    codes = torch.empty((N, K * bits // 8), dtype=torch.uint8, device="cuda")
    sc = torch.empty((N, K // group), dtype=torch.bfloat16, device="cuda")
    qb = torch.empty((N, K // group), dtype=torch.bfloat16, device="cuda")
    pkg.quantize_affine(dev_f32(w), codes, sc, qb, N, K, bits, group)
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), codes_ref.view(np.uint8).reshape(N, -1))
    assert np.array_equal(host_bits(sc), scales_ref)
    assert np.array_equal(host_bits(qb), biases_ref)


def test_quantize_golden_fixtures(pkg):
    for name in ["quantize_w8g64.npz", "quantize_w4g32.npz"]:
        g = np.load(os.path.join(GOLDEN, name))
        bits, group = int(g["bits"]), int(g["group"])
        N, K = g["w"].shape
        codes = torch.empty((N, K * bits // 8), dtype=torch.uint8, device="cuda")
        sc = torch.empty((N, K // group), dtype=torch.bfloat16, device="cuda")
        qb = torch.empty((N, K // group), dtype=torch.bfloat16, device="cuda")
        pkg.quantize_affine(dev_f32(g["w"]), codes, sc, qb, N, K, bits, group)
        torch.cuda.synchronize()
        assert np.array_equal(codes.cpu().numpy(), g["codes"].view(np.uint8).reshape(N, -1)), name
        assert np.array_equal(host_bits(sc), g["scales"]), name
        assert np.array_equal(host_bits(qb), g["biases"]), name


@pytest.mark.parametrize("bits", [8, 4])
def test_pack_unpack_bit_exact(pkg, bits):
    N, K = 33, 512
    rng = np.random.default_rng(22)
    q = rng.integers(0, 1 << bits, (N, K), dtype=np.uint8)
    q_dev = torch.from_numpy(q.copy()).cuda()
    words = torch.empty((N, K * bits // 32), dtype=torch.int32, device="cuda")
    pkg.pack_codes(q_dev, words, N, K, bits)
    back = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    pkg.unpack_codes(words, back, N, K, bits)
    torch.cuda.synchronize()
    assert np.array_equal(words.cpu().numpy().view(np.uint32), orc.pack(q, bits))
    assert np.array_equal(back.cpu().numpy(), q)


def test_f16_to_bf16_all_patterns(pkg):
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    src = torch.from_numpy(bits.view(np.int16).copy()).cuda()
    dst = torch.empty_like(src)
    pkg.f16_to_bf16(src, dst)
    inplace = src.clone()
    pkg.f16_to_bf16(inplace, inplace)
    torch.cuda.synchronize()
    ours = dst.cpu().numpy().view(np.uint16)
    ref = orc.f16_to_bf16(bits)
    finite = ~np.isnan(bits.view(np.float16))
    assert np.array_equal(ours[finite], ref[finite])
    assert np.all(np.isnan(orc.bf16_to_f32(ours[~finite])))
    assert np.array_equal(inplace.cpu().numpy().view(np.uint16), ours)


@pytest.mark.parametrize("M,N", [(64, 128), (7, 100), (126, 6144)])
def test_bias_add_bit_exact(pkg, M, N):
    rng = np.random.default_rng(23)
    y = orc.bf16_rne(rng_normal(rng, (M, N)))
    b = orc.bf16_rne(rng_normal(rng, (N,), 4.0))
    y_dev = dev_bf16(y)
    pkg.bias_add(y_dev, dev_bf16(b), M, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y_dev), orc.bias_add_bf16(y, b))
    # f32 bias: bf16(f32(y) + b)
    bf = rng_normal(rng, (N,), 4.0)
    y_dev = dev_bf16(y)
    pkg.bias_add(y_dev, dev_f32(bf), M, N)
    torch.cuda.synchronize()
    expect = orc.bf16_rne(orc.bf16_to_f32(y) + bf[None, :])
    assert np.array_equal(host_bits(y_dev), expect)


def test_gelu_kernel_within_one_bf16_ulp(pkg):
    g = np.load(os.path.join(GOLDEN, "gelu.npz"))
    x = g["x"]
    xb = orc.bf16_rne(x)
    y = torch.empty((x.size,), dtype=torch.bfloat16, device="cuda")
    pkg.gelu_tanh(dev_bf16(xb), y)
    torch.cuda.synchronize()
    ref = orc.gelu(orc.bf16_to_f32(xb))
    got = host_f32(y)
    ulp = np.abs(orc.bf16_to_f32(orc.bf16_rne(ref))) * 2.0 ** -7
    assert np.all(np.abs(got - ref) <= np.maximum(ulp, 1e-6))
