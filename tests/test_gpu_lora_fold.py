"""The linear with its adapter in one call (ltx25_linear_q_lora), through the
C ABI: the adapter folded into the linear's GEMM where lora_fold_takes says
so -- merged into the expanded weight (w8 codes, K % 128 == 0, aligned A,
rank up to 64), else as extra K -- and the reference's sequence (linear,
lora_add, GELU) elsewhere.

The reference applies the adapter between the linear and the GELU
(src/ltx25-block-metal.cc:639-648). Bars:
  - against the oracle over the same bf16 operands -- f64 products of x and
    the dequantized weight, plus the f64 product of r = bf16(x . A^T) (the
    rounding the reference's lora_add makes) with B, then GELU --
    max|y - ref| / max|ref| <= 1e-2 and rel-L2 < 3e-3 (the fold rounds once
    to bf16, so only that rounding separates it from the f64 result);
  - against the reference's sequence on the GPU (the linear rounded to bf16,
    the delta added and rounded again, then GELU): rel-L2 < 1e-2;
  - where the fold does not take, the call is that sequence, bit for bit.
Large shapes check sampled rows against the oracle and every row against
torch fp32 of the same operands.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
REL_L2_ORACLE = 3e-3
REL_L2_SEQ = 1e-2

# name, M, K, N, rank, bits, group, bias, epilogue, dequant-once mode
CASES = [
    # merged into the expansion
    ("merged: rank 32, f32 bias, GELU", 256, 512, 384, 32, 8, 64, "f32", 1, "on"),
    ("merged: rank 64, bf16 bias", 320, 1024, 1024, 64, 8, 64, "bf16", 0, "on"),
    ("merged: w8g32, rank 48, N = 520 (a partial row tile), GELU", 1024, 1024, 520, 48, 8, 32,
     "bf16", 1, "on"),
    # B copied with its rank padded to a multiple of 8
    ("merged: rank 36 (B padded to 40)", 1024, 512, 256, 36, 8, 64, "f32", 0, "on"),
    # as extra K: w4 codes, rank above 64, an unaligned A, K % 128 != 0
    ("rank 128, f32 bias", 1024, 512, 256, 128, 8, 64, "f32", 0, "on"),
    ("w8g32, rank 200, GELU", 1024, 1024, 512, 200, 8, 32, "bf16", 1, "on"),
    ("rank 450, N = 520, GELU", 1024, 512, 520, 450, 8, 64, None, 1, "on"),
    ("w4g32, rank 100 padded to 128, N = 520, GELU", 300, 768, 520, 100, 4, 32, None, 1, "on"),
    ("split K across the two parts (128 x 128 tile), rank 36", 256, 4096, 512, 36, 8, 64, "f32",
     0, "on"),
    ("rank 1", 192, 256, 256, 1, 8, 64, None, 0, "on"),
    ("rank 96, K = 1088", 512, 1088, 256, 96, 8, 64, "f32", 1, "on"),
    ("256 x 256 tile at the dequant-once threshold", 4096, 1024, 8192, 32, 8, 64, "bf16", 1,
     "auto"),
    ("rank 40, ragged M, K = 2624", 2085, 2624, 512, 40, 8, 64, "f32", 1, "on"),
    # the expansion's [W | B] tail (2112 columns) is wider than one 256-thread
    # block's 2048: written by the tail loop
    ("rank 2100, tail wider than one block", 1024, 256, 256, 2100, 8, 64, "f32", 0, "auto"),
]
MODES = {"on": 1, "auto": 2}


@pytest.fixture(autouse=True)
def _modes(pkg):
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    pkg.set_tile(pkg.TILE_AUTO)


def _operands(pkg, M, K, N, rank, bits, group, bias_kind, seed):
    rng = np.random.default_rng(seed)
    xb = orc.bf16_rne(rng_normal(rng, (M, K)))
    w = rng_normal(rng, (N, K), 0.02)
    qw, codes, scales, biases, wb = make_qweight(pkg, w, bits, group)
    ab = orc.bf16_rne(rng_normal(rng, (rank, K), 0.05))
    bb = orc.bf16_rne(rng_normal(rng, (N, rank), 0.05))
    bias = rng_normal(rng, (N,), 0.01) if bias_kind is not None else None
    if bias_kind == "bf16":
        bias = orc.bf16_to_f32(orc.bf16_rne(bias))
    return xb, qw, wb, ab, bb, bias


def _bias_dev(bias, kind):
    if kind is None:
        return None
    if kind == "bf16":
        return dev_bf16(orc.bf16_rne(bias))
    return dev_f32(bias)


def _oracle_rows(xb, wb, ab, bb, bias, epi, rows):
    """f64 x . W^T + bias + bf16(x . A^T) . B^T (+ GELU) over the given rows."""
    xr = orc.bf16_to_f32(xb[rows])
    pre = orc.linear_f64_d(xr, orc.bf16_to_f32(wb), bias)
    r = orc.bf16_to_f32(orc.bf16_rne(orc.linear_f64(xr, orc.bf16_to_f32(ab))))
    pre = pre + orc.linear_f64_d(r, orc.bf16_to_f32(bb))
    pre = pre.astype(np.float32)
    return orc.gelu(pre) if epi == 1 else pre


def _sequence(pkg, xd, qw, bd, ad, bbd, rank, M, K, N, epi):
    """The reference's order on the GPU: linear, lora_add, then GELU."""
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.linear_q(xd, qw, bd, y, M, K, N)
    pkg.lora_add(xd, ad, bbd, y, M, K, N, rank)
    if epi == 1:
        pkg.gelu_tanh(y, y)
    return y


@pytest.mark.parametrize("name,M,K,N,rank,bits,group,bias_kind,epi,mode", CASES,
                         ids=[c[0] for c in CASES])
def test_fold_against_oracle_and_sequence(pkg, dev, name, M, K, N, rank, bits, group, bias_kind,
                                          epi, mode):
    pkg.set_dequant_once(MODES[mode])
    assert pkg.lora_fold_takes(M, K, N, rank, bits), name
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, bits, group, bias_kind, M + N + rank)
    xd, ad, bbd = dev_bf16(xb), dev_bf16(ab), dev_bf16(bb)
    bd = _bias_dev(bias, bias_kind)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"lora fold {name}: M={M} K={K} N={N} rank={rank} w{bits}g{group}")
    pkg.linear_q_lora(xd, qw, bd, ad, bbd, rank, y, M, K, N, epi)
    torch.cuda.synchronize()
    got = orc.bf16_to_f32(host_bits(y))
    rows = np.arange(M) if M <= 512 else np.unique(np.linspace(0, M - 1, 96).astype(int))
    ref = _oracle_rows(xb, wb, ab, bb, bias, epi, rows)
    assert orc.max_rel(got[rows], ref) <= MAX_REL, name
    assert orc.rel_l2(got[rows], ref) < REL_L2_ORACLE, name
    seq = orc.bf16_to_f32(host_bits(_sequence(pkg, xd, qw, bd, ad, bbd, rank, M, K, N, epi)))
    assert orc.rel_l2(got, seq) < REL_L2_SEQ, name
    # the adapter changed the output (it is not silently dropped)
    plain = torch.empty_like(y)
    pkg.linear_q(xd, qw, bd, plain, M, K, N, epi)
    torch.cuda.synchronize()
    assert orc.rel_l2(orc.bf16_to_f32(host_bits(plain)), got) > 1e-3, name


@pytest.mark.parametrize("M,rank", [(256, 64), (2080, 48)])
def test_fold_a_not_16_byte_aligned(pkg, dev, M, rank):
    """A as a view one element into its storage: the fold pads it first."""
    K, N = 512, 256
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, 8, 64, None, 7)
    store = torch.empty((rank * K + 8,), dtype=torch.bfloat16, device="cuda")
    ad = store[1:1 + rank * K].view(rank, K)
    ad.copy_(dev_bf16(ab))
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"lora fold with a misaligned A, M={M} rank={rank}")
    pkg.linear_q_lora(dev_bf16(xb), qw, None, ad, dev_bf16(bb), rank, y, M, K, N)
    torch.cuda.synchronize()
    got = orc.bf16_to_f32(host_bits(y))
    ref = _oracle_rows(xb, wb, ab, bb, None, 0, np.arange(M))
    assert orc.max_rel(got, ref) <= MAX_REL
    assert orc.rel_l2(got, ref) < REL_L2_ORACLE


@pytest.mark.parametrize("epi", [0, 1])
def test_no_fold_is_the_reference_sequence(pkg, dev, epi):
    """Below the dequant-once threshold (AUTO) the call is linear, lora_add,
    GELU: bit-identical to issuing them one by one."""
    M, K, N, rank = 512, 1024, 2048, 32
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    assert not pkg.lora_fold_takes(M, K, N, rank, 8)
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, 8, 64, "f32", 11)
    xd, ad, bbd, bd = dev_bf16(xb), dev_bf16(ab), dev_bf16(bb), dev_f32(bias)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"lora no-fold sequence epi={epi}")
    pkg.linear_q_lora(xd, qw, bd, ad, bbd, rank, y, M, K, N, epi)
    seq = _sequence(pkg, xd, qw, bd, ad, bbd, rank, M, K, N, epi)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), seq.view(torch.int16))


def test_rank_zero_is_the_linear(pkg, dev):
    M, K, N = 4096, 1024, 2048
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, 8, 8, 64, None, 13)
    xd = dev_bf16(xb)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    want = torch.empty_like(y)
    say("lora fold rank 0")
    pkg.linear_q_lora(xd, qw, None, None, None, 0, y, M, K, N, 1)
    pkg.linear_q(xd, qw, None, want, M, K, N, 1)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_fold_at_the_ffn_shape(pkg, dev):
    """The x2 upscaler's rank-32 adapter on the video FFN up-projection
    (8160 x 4096 -> 16384, GELU): every row against torch fp32 of the same
    bf16 operands, sampled rows against the oracle."""
    M, K, N, rank = 8160, 4096, 16384, 32
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    assert pkg.lora_fold_takes(M, K, N, rank, 8)
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), device="cuda", generator=g) * 0.02
    codes = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    sc = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    qb = torch.empty((N, K // 64), dtype=torch.bfloat16, device="cuda")
    pkg.quantize_affine(w, codes, sc, qb, N, K, 8, 64)
    del w
    qw = pkg.QWeight(codes, sc, qb, 8, 64)
    a = (torch.randn((rank, K), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    b = (torch.randn((N, rank), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    bias = torch.randn((N,), device="cuda", generator=g) * 0.01
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say("lora fold at 8160 x 4096 -> 16384, rank 32, GELU")
    pkg.linear_q_lora(x, qw, bias, a, b, rank, y, M, K, N, 1)
    wd = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(qw, wd, N, K)
    torch.cuda.synchronize()
    r = (x.float() @ a.float().t()).to(torch.bfloat16).float()
    ref = x.float() @ wd.float().t() + bias + r @ b.float().t()
    ref = torch.nn.functional.gelu(ref, approximate="tanh")
    rel = ((y.float() - ref).norm() / ref.norm()).item()
    assert rel < REL_L2_ORACLE, rel
    del ref, r
    rows = np.unique(np.linspace(0, M - 1, 24).astype(int))
    xb = host_bits(x[rows])
    got = orc.bf16_to_f32(host_bits(y[rows]))
    ref_rows = _oracle_rows(xb, host_bits(wd), host_bits(a), host_bits(b),
                            bias.cpu().numpy(), 1, np.arange(len(rows)))
    assert orc.max_rel(got, ref_rows) <= MAX_REL
    assert orc.rel_l2(got, ref_rows) < REL_L2_ORACLE


def _sweep_draw(i):
    """A seeded random fold shape: both forms (merged: w8, rank up to 64,
    K % 128 == 0; extra K otherwise), ragged M and N, groups of 64 and 32, every bias kind,
    with and without GELU, the dequant-once arm forced on so the fold takes."""
    rng = np.random.default_rng(7000 + i)
    bits, group = [(8, 64), (8, 32), (8, 64), (4, 64), (8, 32)][i % 5]
    M = int(rng.choice([130, 256, 333, 512, 700]))
    K = 64 * int(rng.integers(1, 33))
    N = int(rng.choice([64, 200, 384, 520, 1000, 2050]))
    N = max(8, N - N % 8)
    rank = int(rng.choice([1, 8, 12, 16, 24, 32, 40, 48, 56, 64, 72, 96]))
    bias = [None, "bf16", "f32"][int(rng.integers(0, 3))]
    epi = int(rng.integers(0, 2))
    return M, K, N, rank, bits, group, bias, epi


SWEEP = [_sweep_draw(i) for i in range(20)]


@pytest.mark.parametrize("M,K,N,rank,bits,group,bias_kind,epi", SWEEP,
                         ids=[f"s{i}" for i in range(len(SWEEP))])
def test_fold_random_shapes(pkg, dev, M, K, N, rank, bits, group, bias_kind, epi):
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
    assert pkg.lora_fold_takes(M, K, N, rank, bits)
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, bits, group, bias_kind,
                                         M * 7 + K + N + rank)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"lora fold sweep: M={M} K={K} N={N} rank={rank} w{bits}g{group} bias={bias_kind} "
        f"epi={epi}")
    pkg.linear_q_lora(dev_bf16(xb), qw, _bias_dev(bias, bias_kind), dev_bf16(ab), dev_bf16(bb),
                      rank, y, M, K, N, epi)
    torch.cuda.synchronize()
    got = orc.bf16_to_f32(host_bits(y))
    ref = _oracle_rows(xb, wb, ab, bb, bias, epi, np.arange(M))
    assert orc.max_rel(got, ref) <= MAX_REL
    assert orc.rel_l2(got, ref) < REL_L2_ORACLE


def test_fold_forms_agree_and_are_deterministic(pkg, dev):
    """The same adapter through both fold forms: merged into the expansion (A aligned) and as
    extra K (the same A one element into its storage, which the merge does not take). The two
    differ only in where they round (the weight, or r): each is within the oracle's rel-L2 bar,
    so by the triangle inequality they are within twice it of each other; and each call repeats
    bit for bit."""
    M, K, N, rank = 1024, 1024, 768, 32
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, 8, 64, "f32", 11)
    xd, bbd, bd = dev_bf16(xb), dev_bf16(bb), _bias_dev(bias, "f32")
    ad = dev_bf16(ab)
    store = torch.empty((rank * K + 8,), dtype=torch.bfloat16, device="cuda")
    ad_off = store[1:1 + rank * K].view(rank, K)
    ad_off.copy_(ad)
    outs = {}
    for name, a_in in (("merged", ad), ("extra K", ad_off)):
        runs = []
        for _ in range(2):
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            say(f"lora fold forms: {name}")
            pkg.linear_q_lora(xd, qw, bd, a_in, bbd, rank, y, M, K, N, 1)
            torch.cuda.synchronize()
            runs.append(host_bits(y))
        assert np.array_equal(runs[0], runs[1]), name
        outs[name] = orc.bf16_to_f32(runs[0])
    assert not np.array_equal(outs["merged"], outs["extra K"])   # two different roundings
    ref = _oracle_rows(xb, wb, ab, bb, bias, 1, np.arange(M))
    for name, got in outs.items():
        assert orc.max_rel(got, ref) <= MAX_REL, name
        assert orc.rel_l2(got, ref) < REL_L2_ORACLE, name
    assert orc.rel_l2(outs["merged"], outs["extra K"]) < 2 * REL_L2_ORACLE


# rank, K, bits, group, whether the merge into the expansion takes
BOUNDARY = [
    (64, 512, 8, 64, True),     # the largest rank the merge takes
    (65, 512, 8, 64, False),    # one above it: extra K
    (64, 512, 8, 32, True),
    (32, 576, 8, 64, False),    # K % 128 != 0: extra K
    (32, 512, 4, 64, False),    # w4 codes: extra K
]


@pytest.mark.parametrize("rank,K,bits,group,merges", BOUNDARY,
                         ids=[f"r{c[0]}-K{c[1]}-w{c[2]}g{c[3]}" for c in BOUNDARY])
def test_merge_boundary(pkg, dev, rank, K, bits, group, merges):
    """Where the merge takes, an aligned A (merged) and the same A one element into its
    storage (extra K: the merge needs an aligned A) round in different places, so the two
    outputs differ; where it does not take, both calls run the extra-K form and agree bit for
    bit. Each output is within the oracle's bars."""
    M, N = 256, 256
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
    assert pkg.lora_fold_takes(M, K, N, rank, bits)
    xb, qw, wb, ab, bb, bias = _operands(pkg, M, K, N, rank, bits, group, "bf16", rank + K)
    xd, bbd, bd = dev_bf16(xb), dev_bf16(bb), _bias_dev(bias, "bf16")
    ad = dev_bf16(ab)
    store = torch.empty((rank * K + 8,), dtype=torch.bfloat16, device="cuda")
    ad_off = store[1:1 + rank * K].view(rank, K)
    ad_off.copy_(ad)
    ref = _oracle_rows(xb, wb, ab, bb, bias, 1, np.arange(M))
    outs = []
    for a_in in (ad, ad_off):
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        say(f"lora merge boundary: rank={rank} K={K} w{bits}g{group} "
            f"A {'aligned' if a_in is ad else 'one element in'}")
        pkg.linear_q_lora(xd, qw, bd, a_in, bbd, rank, y, M, K, N, 1)
        torch.cuda.synchronize()
        got = host_bits(y)
        assert orc.max_rel(orc.bf16_to_f32(got), ref) <= MAX_REL
        assert orc.rel_l2(orc.bf16_to_f32(got), ref) < REL_L2_ORACLE
        outs.append(got)
    assert np.array_equal(outs[0], outs[1]) != merges
