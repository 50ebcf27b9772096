"""Writes the committed fixtures in this directory from the CPU oracle.

The reference commits no fixtures for this path (its hot-path tests draw
from std::mt19937 at run time, tests/ltx25-qlinear-test.cc:185 and
tests/ltx25-i8-gemm-test.cc:94,168), so these are this build's own: inputs
and oracle outputs at small shapes, regenerated only on purpose. The oracle
itself is pinned independently in tests/test_oracle.py; the fixtures then
pin the oracle against later change and give the GPU tests fixed vectors.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import orc  # noqa: E402


def save(name, **arrays):
    np.savez(os.path.join(HERE, name), **arrays)
    print("wrote", name)


def main():
    # group-affine quantize, w8g64 and w4g32, with a constant group
    for bits, group, seed in [(8, 64, 101), (4, 32, 102)]:
        w = orc.fill_normal(8 * 256, seed, 0.0, 0.02).reshape(8, 256)
        w[3, 64:128] = 0.0173
        codes, scales, biases, deq = orc.quantize_affine(w, bits, group)
        save(f"quantize_w{bits}g{group}.npz", kind="quantize", w=w, bits=bits, group=group,
             codes=codes, scales=scales, biases=biases, deq=deq)

    # a small quantized linear with an f32 bias (config 0's form, shrunk)
    M, K, N = 16, 256, 48
    x = orc.bf16_rne(orc.fill_normal(M * K, 201).reshape(M, K))
    w = orc.fill_normal(N * K, 202, 0.0, 0.02).reshape(N, K)
    bias = orc.fill_normal(N, 203, 0.0, 0.01)
    codes, scales, biases, _ = orc.quantize_affine(w, 8, 64)
    _, wb = orc.dequant(codes, scales, biases, N, K, 8, 64)
    y = orc.linear_f64(orc.bf16_to_f32(x), orc.bf16_to_f32(wb), bias)
    save("qlinear_w8g64_m16.npz", kind="qlinear", x_bf16=x, codes=codes, scales=scales,
         biases=biases, bits=8, group=64, w_shape=np.array([N, K]), w_bf16=wb, bias_f32=bias,
         y_f32=y)

    # int8 tier: per-token x, per-channel w, int32 accumulators, epilogue
    M, K, N = 32, 256, 24
    x = orc.bf16_rne(orc.fill_normal(M * K, 301).reshape(M, K))
    w = orc.bf16_rne(orc.fill_normal(N * K, 302, 0.0, 0.02).reshape(N, K))
    bias = orc.fill_normal(N, 303, 0.0, 0.01)
    xq, sx = orc.i8_quantize_rows(x)
    wq, sw = orc.i8_quantize_rows(w)
    acc = orc.i8_gemm_i32(xq, wq)
    y = orc.i8_epilogue(acc, sx, sw, bias, 2)
    save("i8_m32.npz", kind="i8", x_bf16=x, w_bf16=w, bias_f32=bias, xq=xq, sx=sx, wq=wq,
         sw=sw, acc=acc, y_bf16=y)

    # GELU-tanh over a range
    xg = np.linspace(-8, 8, 4097).astype(np.float32)
    save("gelu.npz", kind="gelu", x=xg, y=orc.gelu(xg))


if __name__ == "__main__":
    main()
