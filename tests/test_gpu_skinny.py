"""The M <= 128 route (skinny.hip) on the GPU, through the C ABI.

A linear with at most 128 tokens takes this kernel unless its weight is large
enough to need more than 3 workgroups per CU: 32 output columns per workgroup, the workgroup's K (up to 2048) split between its 8 waves in runs
of 64-wide chunks, split-K across workgroups above 2048. Its lane mapping
(X chunks swizzled in LDS, a permuted K order shared by both operands, the
codes transposed through LDS, the cross-wave sum) is pinned two ways:

- a selection GEMM: row m of X holds a single 1.0 at column k(m), spread
  over chunks, waves and splits, so y[m][n] = bf16(w[n][k(m)] + bias[n])
  exactly, whatever the summation order -- a wrong swizzle, K permutation,
  operand transpose or reduction index changes bits (the oracle's dequant
  gives the bf16 w, the oracle's rounding the expected bits);
- random data against the oracle (max|y - ref| / max|ref| <= 1e-2) at the
  chunk counts the wave split and split-K make ragged: 1 chunk (7 idle waves),
  7 and 9 chunks, 33 and 97 chunks (uneven splits);
- and the same launch twice gives the same bits.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, host_f32, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2

SELECT = [  # M, K, N, bits, group, bias
    (1, 64, 32, 8, 64, "f32"),
    (7, 2048, 40, 8, 64, "none"),
    (126, 2048, 100, 8, 64, "f32"),
    (128, 2048, 64, 4, 64, "bf16"),
    (126, 2112, 33, 8, 32, "f32"),        # 33 chunks: split 2 (17 + 16)
    (126, 4096, 5, 4, 32, "none"),        # N < 8: element-wise stores; split 2
    (126, 8192, 96, 8, 64, "bf16"),       # the audio ff_down shape class: split 4
    (100, 1024, 2050, 8, 64, "f32"),      # ragged N over many workgroups
    (126, 2048, 72, 16, 64, "f32"),       # dense bf16 weight
    (33, 6208, 48, 16, 64, "none"),       # dense, 97 chunks: split 4 (25, 25, 25, 22)
]


def selection_x(M, K):
    """Row m has a 1.0 at k(m): odd strides walk the chunks and waves."""
    x = np.zeros((M, K), np.float32)
    cols = (np.arange(M) * 97 + 13) % K
    x[np.arange(M), cols] = 1.0
    return x, cols


def make_bias(rng, N, kind):
    b = rng_normal(rng, (N,), 0.05)
    if kind == "bf16":
        b = orc.bf16_to_f32(orc.bf16_rne(b))
        return b, dev_bf16(orc.bf16_rne(b))
    if kind == "f32":
        return b, dev_f32(b)
    return None, None


def run(pkg, xb, w, M, K, N, bits, group, bd, epi=0):
    """-> y, the f32 dequantized weight (the f64 bar's reference), and the
    bf16 weight the GEMM multiplies by (as f32)."""
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    if bits == 16:
        wb = orc.bf16_rne(w)
        pkg.linear(dev_bf16(xb), dev_bf16(wb), bd, y, M, K, N)
        wf = orc.bf16_to_f32(wb)
    else:
        qw, codes, scales, biases, wb = make_qweight(pkg, w, bits, group)
        pkg.linear_q(dev_bf16(xb), qw, bd, y, M, K, N, epi)
        wf, _ = orc.dequant(codes, scales, biases, N, K, bits, group)
    torch.cuda.synchronize()
    return y, wf, orc.bf16_to_f32(wb).reshape(N, K)


@pytest.mark.parametrize("M,K,N,bits,group,bias", SELECT,
                         ids=[f"M{c[0]}-K{c[1]}-N{c[2]}-w{c[3]}g{c[4]}-{c[5]}" for c in SELECT])
def test_selection_gemm_is_bit_exact(pkg, dev, M, K, N, bits, group, bias):
    rng = np.random.default_rng(M * 31 + K + N * 7 + bits)
    x, cols = selection_x(M, K)
    w = rng_normal(rng, (N, K), 0.05)
    b, bd = make_bias(rng, N, bias)
    say(f"skinny selection M={M} K={K} N={N} w{bits}g{group} bias={bias}")
    y, _, w16 = run(pkg, orc.bf16_rne(x), w, M, K, N, bits, group, bd)
    sel = np.asarray(w16, np.float32)[:, cols].T          # [M][N]: w[n][k(m)]
    want = sel + (np.asarray(b, np.float32)[None, :] if b is not None else 0.0)
    assert np.array_equal(host_bits(y), orc.bf16_rne(want.astype(np.float32)))


RAGGED = [  # M, K, N, bits, group, bias, epilogue
    (126, 64, 96, 8, 64, "f32", 0),       # one chunk: waves 1..7 idle
    (126, 448, 200, 4, 64, "bf16", 1),    # 7 chunks
    (126, 576, 128, 8, 32, "none", 1),    # 9 chunks: one wave takes 2
    (126, 2112, 260, 8, 64, "f32", 0),    # 33 chunks: split 2
    (128, 6208, 64, 4, 32, "f32", 0),     # 97 chunks: split 4, uneven
    (64, 2048, 2048, 8, 64, "bf16", 1),
]


@pytest.mark.parametrize("M,K,N,bits,group,bias,epi", RAGGED,
                         ids=[f"M{c[0]}-K{c[1]}-N{c[2]}-w{c[3]}g{c[4]}-{c[5]}-e{c[6]}" for c in RAGGED])
def test_ragged_chunk_counts_against_oracle(pkg, dev, M, K, N, bits, group, bias, epi):
    rng = np.random.default_rng(K * 3 + N)
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    w = rng_normal(rng, (N, K), 0.02)
    b, bd = make_bias(rng, N, bias)
    say(f"skinny ragged M={M} K={K} N={N} w{bits}g{group} bias={bias} epi={epi}")
    y, wf, _ = run(pkg, x, w, M, K, N, bits, group, bd, epi)
    ref = orc.linear_f64_d(orc.bf16_to_f32(x), wf, b)
    if epi:
        ref = orc.gelu(ref.astype(np.float32)).astype(np.float64)
    assert orc.max_rel(host_f32(y), ref) <= MAX_REL


def test_same_launch_twice_gives_the_same_bits(pkg, dev):
    M, K, N = 126, 8192, 2048      # split-K path: partials summed in split order
    rng = np.random.default_rng(5)
    x = dev_bf16(orc.bf16_rne(rng_normal(rng, (M, K))))
    qw, _, _, _, _ = make_qweight(pkg, rng_normal(rng, (N, K), 0.02), 8, 64)
    outs = []
    for i in range(2):
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        say(f"skinny determinism run {i}")
        pkg.linear_q(x, qw, None, y, M, K, N)
        torch.cuda.synchronize()
        outs.append(host_bits(y))
    assert np.array_equal(outs[0], outs[1])
