"""The per-head gate on the attention output (ltx25_gate_heads) on the GPU.

Reference: MetalOps::gate_heads / ltx_gate_heads (src/ltx25-metal-ops.cc:1089-1101;
src/ltx25-kernels.metal:85-103), y[t][h][d] = y * 2 sigmoid(logit[t][h]) stored as bf16,
with the gate expression of the CPU block (src/ltx25-block-ref.cc:113-125). The oracle is
pinned bit-exactly against that CPU code (tests/test_oracle.py). The device evaluates exp
with its own library, which may differ from the host's by an ulp of float, so the bar is:
at most one bf16 ulp anywhere and at least 99.5% of the elements bit-identical; the
special gates (1 at logit 0, 2 at a large logit, 0 past exp's overflow) are exact.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, host_bits, rng_normal, say

pytestmark = pytest.mark.gpu

CASES = [  # tokens, heads, head_dim, misaligned y
    (126, 16, 128, False),     # audio self-attention (inner 2048)
    (1000, 32, 128, False),    # video (inner 4096)
    (37, 5, 100, False),       # head width not a multiple of 8: element-wise path
    (64, 8, 64, True),         # y at a 2-byte offset: element-wise path
    (3, 1, 8, False),
]


def ulp_distance(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # map sign-magnitude bf16 patterns onto a monotone integer line
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(a - b)


@pytest.mark.parametrize("tokens,heads,head_dim,misaligned", CASES)
def test_gate_heads_against_oracle(pkg, dev, tokens, heads, head_dim, misaligned):
    rng = np.random.default_rng(tokens * 31 + heads)
    y = orc.bf16_rne(rng_normal(rng, (tokens, heads * head_dim)))
    lg = orc.bf16_rne(rng_normal(rng, (tokens, heads), 3.0))
    want = orc.gate_heads(y, lg, heads, head_dim)
    if misaligned:
        buf = dev_bf16(np.concatenate([np.zeros(1, np.uint16), y.reshape(-1)]))
        yd = buf[1:]
    else:
        yd = dev_bf16(y)
    say(f"gate_heads tokens={tokens} heads={heads} head_dim={head_dim} misaligned={misaligned}")
    pkg.gate_heads(yd, dev_bf16(lg), heads, tokens, head_dim)
    torch.cuda.synchronize()
    got = host_bits(yd).reshape(tokens, heads * head_dim)
    d = ulp_distance(got, want)
    assert d.max() <= 1
    assert np.mean(d == 0) >= 0.995


def test_gate_heads_special_gates_are_exact(pkg, dev):
    tokens, heads, head_dim = 4, 3, 16
    rng = np.random.default_rng(5)
    y = orc.bf16_rne(rng_normal(rng, (tokens, heads * head_dim)))
    for val in (0.0, 88.0, -100.0):
        lg = orc.bf16_rne(np.full((tokens, heads), val, np.float32))
        yd = dev_bf16(y)
        say(f"gate_heads special logit {val}")
        pkg.gate_heads(yd, dev_bf16(lg), heads, tokens, head_dim)
        torch.cuda.synchronize()
        assert np.array_equal(host_bits(yd).reshape(y.shape), orc.gate_heads(y, lg, heads, head_dim))


def test_gate_heads_empty_is_a_noop(pkg, dev):
    y = torch.ones(8, dtype=torch.bfloat16, device="cuda")
    pkg.gate_heads(y, y, 0, 4, 2)
    pkg.gate_heads(y, y, 2, 0, 2)
    torch.cuda.synchronize()
    assert bool((y == 1).all())
