"""Pins the CPU oracle before anything is compared against it.

Every oracle function is checked against something that is not itself: a
library routine (torch's bf16 cast, numpy's half decoder, numpy float64 and
int64 matmul), a closed form with a known answer (an exactly representable
quantization grid, a half-way rounding case, packed words written out by
hand), or the reference's own compiled CPU code (oracle/_ref, built from the
reference sources by oracle/Makefile). A plausible slip -- swapped scale and
bias, high bits packed first, round-half-even where half-away is meant, a
transposed weight, a dropped bias -- fails at least one of these.
"""
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def torch_bf16_bits(a_f32: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a_f32, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ---- number formats ---------------------------------------------------------------
def test_bf16_rne_matches_torch_including_ties_and_specials():
    rng = np.random.default_rng(1)
    vals = [rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-30, 30, 20000)]
    # exact ties: low half 0x8000 with both parities of the kept LSB
    hi = rng.integers(0, 0x7F7F, 4000, dtype=np.uint32)
    ties = ((hi << 16) | 0x8000).astype(np.uint32).view(np.float32)
    vals.append(ties)
    vals.append(np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45,
                          -1e-45, 1.1754942e-38, 65504.0], np.float32))
    a = np.concatenate(vals).astype(np.float32)
    ours = orc.bf16_rne(a)
    theirs = torch_bf16_bits(a)
    assert np.array_equal(ours, theirs)
    # a tie must go to the even neighbour
    assert orc.bf16_rne(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 0x3F80
    assert orc.bf16_rne(np.array([1.0 + 3 * 2.0 ** -8], np.float32))[0] == 0x3F82
    nan = orc.bf16_rne(np.array([np.nan], np.float32))
    assert np.isnan(orc.bf16_to_f32(nan))[0]


def test_bf16_to_f32_is_the_upper_half():
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(h)
    assert np.array_equal(f.view(np.uint32) >> 16, h.astype(np.uint32))
    assert np.all(f.view(np.uint32) & 0xFFFF == 0)


def test_f16_to_bf16_matches_numpy_half_then_torch():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    f = bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(f)
    ours = orc.f16_to_bf16(bits)
    theirs = torch_bf16_bits(f)
    assert np.array_equal(ours[finite], theirs[finite])
    assert np.all(np.isnan(orc.bf16_to_f32(ours[~finite])))


# ---- packing -----------------------------------------------------------------------
def test_pack_low_bits_first_known_words():
    q8 = np.array([[1, 2, 3, 4, 0xAA, 0xBB, 0xCC, 0xDD]], np.uint8)
    assert orc.pack(q8, 8).tolist() == [[0x04030201, 0xDDCCBBAA]]
    q4 = np.array([[1, 2, 3, 4, 5, 6, 7, 8]], np.uint8)
    assert orc.pack(q4, 4).tolist() == [[0x87654321]]


def test_pack_w8_is_little_endian_u8_and_round_trips():
    rng = np.random.default_rng(2)
    q = rng.integers(0, 256, (7, 64), dtype=np.uint8)
    c = orc.pack(q, 8)
    assert np.array_equal(c.view(np.uint8).reshape(7, 64), q)
    assert np.array_equal(orc.unpack(c, 7, 64, 8), q)
    q4 = rng.integers(0, 16, (5, 64), dtype=np.uint8)
    assert np.array_equal(orc.unpack(orc.pack(q4, 4), 5, 64, 4), q4)


# ---- quantization ------------------------------------------------------------------
def exact_grid(rng, N, K, group, bits):
    """Weights that lie exactly on a bf16-representable affine grid whose
    extremes are present in every group, so quantize must return exactly the
    codes, scales and biases they were built from."""
    qmax = (1 << bits) - 1
    G = K // group
    s = rng.integers(128, 256, (N, G)).astype(np.float64) * 2.0 ** -12
    b = -rng.integers(1, 256, (N, G)).astype(np.float64) * 2.0 ** -12
    q = rng.integers(0, qmax + 1, (N, K))
    q[:, ::group] = 0
    q[:, 1::group] = qmax
    w = (np.repeat(s, group, axis=1) * q + np.repeat(b, group, axis=1)).astype(np.float32)
    assert np.array_equal(w.astype(np.float64),
                          np.repeat(s, group, axis=1) * q + np.repeat(b, group, axis=1))
    return w, q.astype(np.uint8), s.astype(np.float32), b.astype(np.float32)


@pytest.mark.parametrize("bits,group", [(8, 64), (8, 32), (4, 64), (4, 32)])
def test_quantize_exact_grid_round_trip(bits, group):
    rng = np.random.default_rng(3)
    w, q, s, b = exact_grid(rng, 6, 256, group, bits)
    codes, scales, biases, deq = orc.quantize_affine(w, bits, group)
    assert np.array_equal(orc.unpack(codes, 6, 256, bits), q)
    assert np.array_equal(orc.bf16_to_f32(scales), s)
    assert np.array_equal(orc.bf16_to_f32(biases), b)
    assert np.array_equal(deq, w)


def test_quantize_constant_group_has_zero_scale_and_codes():
    w = np.full((2, 128), 0.0123, np.float32)
    w[1, 64:] = -3.5
    codes, scales, biases, deq = orc.quantize_affine(w, 8, 64)
    assert np.all(codes == 0)
    assert np.all(scales == 0)
    assert np.array_equal(orc.bf16_to_f32(biases)[:, 0], orc.bf16_to_f32(orc.bf16_rne(w[:, 0])))
    assert np.array_equal(deq, np.repeat(orc.bf16_to_f32(biases), 64, axis=1))


def test_quantize_rounds_half_away_from_zero():
    # s = 2^-8, b = 0; a value at exactly 10.5 steps must code as 11, 11.5 as 12
    # (round-half-even would give 10 and 12).
    s = 2.0 ** -8
    g = np.arange(64, dtype=np.float64)
    w = np.zeros((1, 64))
    w[0, :] = (g % 2) * 255 * s
    w[0, 2] = 10.5 * s
    w[0, 4] = 11.5 * s
    codes, scales, biases, _ = orc.quantize_affine(w.astype(np.float32), 8, 64)
    assert orc.bf16_to_f32(scales)[0, 0] == np.float32(s)
    q = orc.unpack(codes, 1, 64, 8)[0]
    assert q[2] == 11 and q[4] == 12


def test_quantize_error_bound_on_random_weights():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    codes, scales, biases, deq = orc.quantize_affine(w, 8, 64)
    q = orc.unpack(codes, 64, 512, 8).astype(np.int64)
    scr = np.repeat(orc.bf16_to_f32(scales), 64, axis=1).astype(np.float64)
    lor = np.repeat(orc.bf16_to_f32(biases), 64, axis=1).astype(np.float64)
    err = np.abs(w.astype(np.float64) - deq)
    inner = (q > 0) & (q < 255)
    # an unclamped code is the nearest grid point
    assert np.all(err[inner] <= 0.5 * scr[inner] * (1 + 1e-5) + 1e-9)
    # deq is exactly scale*q + bias in two f32 roundings
    assert np.array_equal(deq, (np.float32(scr) * q.astype(np.float32)).astype(np.float32)
                          + np.float32(lor))
    # scale and bias are the bf16 roundings of (max-min)/255 and min
    grp = w.reshape(64, 8, 64)
    lo, hi = grp.min(axis=2), grp.max(axis=2)
    assert np.array_equal(biases, torch_bf16_bits(lo))
    assert np.array_equal(scales, torch_bf16_bits((hi - lo) / np.float32(255)))


def test_dequant_is_a_single_rounding_fma():
    rng = np.random.default_rng(5)
    for bits, group in [(8, 64), (4, 32)]:
        w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
        codes, scales, biases, _ = orc.quantize_affine(w, bits, group)
        wf, wb = orc.dequant(codes, scales, biases, 16, 256, bits, group)
        q = orc.unpack(codes, 16, 256, bits).astype(np.float64)
        s = np.repeat(orc.bf16_to_f32(scales), group, axis=1).astype(np.float64)
        b = np.repeat(orc.bf16_to_f32(biases), group, axis=1).astype(np.float64)
        exact = s * q + b             # exact in double: 8x8-bit product plus a bf16
        assert np.array_equal(wf, exact.astype(np.float32))
        assert np.array_equal(wb, torch_bf16_bits(wf))


# ---- linear, GELU, bias --------------------------------------------------------------
def test_linear_f64_matches_numpy_float64():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, 200)).astype(np.float32)
    w = rng.standard_normal((13, 200)).astype(np.float32)
    b = rng.standard_normal(13).astype(np.float32)
    ours = orc.linear_f64_d(x, w, b)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.max(np.abs(ours - ref)) <= 1e-12 * np.max(np.abs(ref))
    # not transposed, bias not dropped
    assert np.max(np.abs(orc.linear_f64_d(x, w) - (ref - b))) < 1e-9
    assert np.array_equal(orc.linear_f64(x, w, b), ours.astype(np.float32))


def test_linear_f32_omp_matches_numpy_within_f32_accumulation():
    """The timing baseline's f32 linear: the f64 result up to f32 rounding of
    K products and sums, any thread count the same, bias added, W not
    transposed."""
    rng = np.random.default_rng(16)
    x = rng.standard_normal((11, 300)).astype(np.float32)
    w = rng.standard_normal((17, 300)).astype(np.float32)
    b = rng.standard_normal(17).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    bound = 300 * np.finfo(np.float32).eps * (np.abs(x).astype(np.float64) @
                                             np.abs(w).astype(np.float64).T + np.abs(b))
    one = orc.linear_f32_omp(x, w, b, threads=1)
    assert np.all(np.abs(one - ref) <= bound)
    assert np.array_equal(orc.linear_f32_omp(x, w, b, threads=4), one)
    assert np.max(np.abs(orc.linear_f32_omp(x, w, None, threads=2) - (ref - b))) < 1e-3


def test_fill_normal_is_seeded_standard_normal():
    """The synthetic-data generator: a pure function of the seed, N(0, 1) by
    a Kolmogorov-Smirnov test, and mean / stddev applied as mean + stddev z."""
    from scipy import stats

    a = orc.fill_normal(200000, 7)
    assert np.array_equal(a, orc.fill_normal(200000, 7))
    assert not np.array_equal(a, orc.fill_normal(200000, 8))
    assert stats.kstest(a.astype(np.float64), "norm").pvalue > 1e-3
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    s = orc.fill_normal(1000, 7, 3.0, 0.5)
    assert np.allclose(s, 3.0 + 0.5 * a[:1000], rtol=0, atol=2e-6)


def test_gelu_matches_torch_tanh_gelu():
    x = np.concatenate([np.linspace(-12, 12, 20001), [0.0, -0.0, 1e-30, -1e-30, 50, -50]])
    x = x.astype(np.float32)
    ours = orc.gelu(x)
    theirs = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh")
    theirs = theirs.float().numpy()
    # One ulp, with an absolute floor for the far negative tail: there the
    # reference's 0.5 x (1 + tanh t) cancels in double (1 + tanh t ~ 1e-16)
    # and leaves values of order 1e-16 where torch returns 0.
    ulp = np.spacing(np.abs(theirs).astype(np.float32))
    assert np.all(np.abs(ours - theirs) <= np.maximum(ulp, 1e-15))
    # and it is the tanh form, not the erf form
    erf = torch.nn.functional.gelu(torch.from_numpy(x).double()).float().numpy()
    assert np.max(np.abs(ours - erf)) > 1e-4


def test_bias_add_bf16_matches_torch():
    rng = np.random.default_rng(7)
    y = torch_bf16_bits(rng.standard_normal((5, 24)).astype(np.float32))
    bias = torch_bf16_bits(rng.standard_normal(24).astype(np.float32) * 4)
    ours = orc.bias_add_bf16(y, bias)
    ty = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16).float()
    tb = torch.from_numpy(bias.view(np.int16)).view(torch.bfloat16).float()
    theirs = (ty + tb).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


# ---- the reference's own CPU code (oracle/_ref) ---------------------------------------
ref_only = pytest.mark.skipif(orc.ref() is None, reason="oracle/_ref was not built here")


@ref_only
def test_linear_bit_exact_against_reference_linear_():
    rng = np.random.default_rng(8)
    r = orc.ref()
    for M, K, N, with_bias in [(3, 64, 5, True), (17, 300, 11, False), (8, 1024, 16, True)]:
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32) if with_bias else None
        out = np.empty((M, N), np.float32)
        r.ref_linear(x.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data, M, K, N,
                     out.ctypes.data)
        assert np.array_equal(orc.linear_f64(x, w, b), out)


@ref_only
def test_gelu_bit_exact_against_reference_stream_ff():
    rng = np.random.default_rng(9)
    r = orc.ref()
    rows, cols = 4, 96
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    out = np.empty_like(x)
    r.ref_ff_identity(x.ctypes.data, rows, cols, 1e-6, out.ctypes.data)
    z = x.copy()
    r.ref_rms_norm(z.ctypes.data, rows, cols, 1e-6)
    expect = (x + orc.gelu(z)).astype(np.float32)
    assert np.array_equal(out, expect)


@ref_only
def test_gate_bit_exact_against_reference_attention_gating():
    rng = np.random.default_rng(21)
    r = orc.ref()
    heads, head_dim, rows = 6, 16, 3
    # bf16-representable inputs, so that the oracle's bf16 operands are the reference's floats
    v_b = orc.bf16_to_f32(torch_bf16_bits(rng.standard_normal(heads * head_dim).astype(np.float32)))
    g_b = orc.bf16_to_f32(torch_bf16_bits((rng.standard_normal(heads) * 4).astype(np.float32)))
    out = np.empty((rows, heads * head_dim), np.float32)
    r.ref_gate_identity(v_b.ctypes.data, g_b.ctypes.data, heads, head_dim, rows, out.ctypes.data)
    y = np.tile(torch_bf16_bits(v_b), (rows, 1))
    lg = np.tile(torch_bf16_bits(g_b), (rows, 1))
    got = orc.gate_heads(y, lg, heads, head_dim)
    assert np.array_equal(got, torch_bf16_bits(out))


def test_gate_heads_closed_form_and_special_cases():
    rng = np.random.default_rng(22)
    tokens, heads, head_dim = 5, 4, 24
    y = torch_bf16_bits(rng.standard_normal((tokens, heads * head_dim)).astype(np.float32))
    lg_f = (rng.standard_normal((tokens, heads)) * 3).astype(np.float32)
    lg = torch_bf16_bits(lg_f)
    got = orc.bf16_to_f32(orc.gate_heads(y, lg, heads, head_dim)).astype(np.float64)
    g64 = 2.0 / (1.0 + np.exp(-orc.bf16_to_f32(lg).astype(np.float64)))
    want = orc.bf16_to_f32(y).astype(np.float64) * np.repeat(g64, head_dim, axis=1)
    # one bf16 rounding of a float product: within half an ulp of bf16 (2^-9 relative) plus
    # the float gate's own rounding
    assert np.all(np.abs(got - want) <= np.abs(want) * (2.0 ** -8) + 1e-30)
    # logit 0: gate exactly 1, y unchanged; +88: gate 2, y doubled exactly; -100: exp
    # overflows, the gate is 0 and y becomes a signed zero
    for val, expect in [(0.0, lambda v: v), (88.0, lambda v: 2 * v), (-100.0, lambda v: 0 * v)]:
        lgc = torch_bf16_bits(np.full((tokens, heads), val, np.float32))
        out = orc.bf16_to_f32(orc.gate_heads(y, lgc, heads, head_dim))
        assert np.array_equal(out, expect(orc.bf16_to_f32(y)).astype(np.float32)), val


# ---- int8 tier ------------------------------------------------------------------------
def test_i8_quantize_rows_closed_form():
    rng = np.random.default_rng(10)
    x = torch_bf16_bits(rng.standard_normal((12, 256)).astype(np.float32))
    x[3] = 0                                                 # all-zero row
    q, s = orc.i8_quantize_rows(x)
    xf = orc.bf16_to_f32(x)
    amax = np.max(np.abs(xf), axis=1)
    s_np = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(s, s_np)
    with np.errstate(divide="ignore", invalid="ignore"):
        q_np = np.clip(np.rint(xf / s_np[:, None]), -127, 127)
    q_np[3] = 0
    assert np.array_equal(q.astype(np.float32), q_np)
    assert s[3] == 0 and np.all(q[3] == 0)
    nz = np.arange(12) != 3
    assert np.all(np.max(np.abs(q[nz].astype(np.int32)), axis=1) == 127)
    err = np.abs(xf[nz] - q[nz] * s[nz, None])
    assert np.all(err <= 0.5 * s[nz, None] * (1 + 1e-6))


def test_i8_gemm_matches_numpy_int64():
    rng = np.random.default_rng(11)
    xq = rng.integers(-127, 128, (7, 384), dtype=np.int8)
    wq = rng.integers(-127, 128, (9, 384), dtype=np.int8)
    ref = xq.astype(np.int64) @ wq.astype(np.int64).T
    assert np.array_equal(orc.i8_gemm_i32(xq, wq).astype(np.int64), ref)


def _f32_fma_exact(a, b, c):
    """fmaf(a, b, c) by exact rational arithmetic, or None if the rational
    result is not representable in double (then one rounding to f32 via a
    double is not guaranteed to be correct)."""
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    d = float(exact)
    if Fraction(d) != exact:
        return None
    return np.float32(d)


def test_i8_epilogue_is_one_fma_then_bf16():
    rng = np.random.default_rng(12)
    acc = rng.integers(-2_000_000, 2_000_000, (6, 10)).astype(np.int32)
    sx = (rng.random(6) * 0.03).astype(np.float32)
    sw = (rng.random(10) * 0.0004).astype(np.float32)
    bias = rng.standard_normal(10).astype(np.float32)
    for bias_dtype, b in [(0, None), (2, bias), (1, torch_bf16_bits(bias))]:
        y = orc.i8_epilogue(acc, sx, sw, b, bias_dtype)
        bf = np.zeros(10, np.float32) if b is None else (
            orc.bf16_to_f32(b) if bias_dtype == 1 else bias)
        checked = 0
        for m in range(6):
            for n in range(10):
                sc = np.float32(sx[m] * sw[n])
                v = _f32_fma_exact(np.float32(acc[m, n]), sc, bf[n])
                if v is None:
                    continue
                checked += 1
                assert y[m, n] == torch_bf16_bits(np.array([v], np.float32))[0]
        assert checked >= 50


def test_i8_epilogue_with_gelu_is_the_composition():
    """epilogue 1 = the pinned epilogue's f32 value through the pinned GELU, rounded once;
    epilogue 0 = orc_i8_epilogue bit for bit."""
    rng = np.random.default_rng(13)
    acc = rng.integers(-2_000_000, 2_000_000, (6, 10)).astype(np.int32)
    sx = (rng.random(6) * 0.03).astype(np.float32)
    sw = (rng.random(10) * 0.0004).astype(np.float32)
    bias = rng.standard_normal(10).astype(np.float32)
    assert np.array_equal(orc.i8_epilogue(acc, sx, sw, bias, 2, epilogue=0),
                          orc.i8_epilogue(acc, sx, sw, bias, 2))
    y = orc.i8_epilogue(acc, sx, sw, bias, 2, epilogue=1)
    checked = 0
    for m in range(6):
        for n in range(10):
            v = _f32_fma_exact(np.float32(acc[m, n]), np.float32(sx[m] * sw[n]), bias[n])
            if v is None:
                continue
            checked += 1
            g = orc.gelu(np.array([v], np.float32))
            assert y[m, n] == torch_bf16_bits(g)[0]
    assert checked >= 50
    # and GELU changed something: negative pre-activations shrink toward 0
    assert not np.array_equal(y, orc.i8_epilogue(acc, sx, sw, bias, 2))


# ---- low-rank adapter delta ---------------------------------------------------------------
# The reference's lora test shapes (tests/ltx25-lora-apply-test.cc:394-409), minus the
# three large ones, which the GPU tests cover.
LORA_SMALL = [(12, 64, 64, 3), (8, 32, 64, 3), (12, 64, 32, 3), (12, 64, 4, 3), (12, 64, 256, 5),
              (6, 64, 64, 1)]


def _lora_draws(M, K, N, rank, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    a = (rng.standard_normal((rank, K)) * 0.5).astype(np.float32)
    b = (rng.standard_normal((N, rank)) * 0.5).astype(np.float32)
    y = rng.standard_normal((M, N)).astype(np.float32)
    return x, a, b, y


@pytest.mark.parametrize("M,K,N,rank", LORA_SMALL)
def test_lora_meets_the_reference_tests_f64_bar(M, K, N, rank):
    # The reference's known answer: y + (x @ A^T) @ B^T in f64 over the UNROUNDED draws,
    # rel-L2 < 2e-2 (tests/ltx25-lora-apply-test.cc:410-465).
    x, a, b, y = _lora_draws(M, K, N, rank, 7)
    want = y.astype(np.float64) + (x.astype(np.float64) @ a.T.astype(np.float64)) @ b.T
    got = orc.bf16_to_f32(orc.lora_add(orc.bf16_rne(x), orc.bf16_rne(a), orc.bf16_rne(b),
                                       orc.bf16_rne(y)))
    assert orc.rel_l2(got, want) < 2e-2


@pytest.mark.parametrize("M,K,N,rank", LORA_SMALL + [(33, 96, 40, 17)])
def test_lora_matches_numpy_with_the_same_roundings(M, K, N, rank):
    # numpy float64 matmuls: r rounded to bf16 once, then y + r . B^T rounded once.
    x, a, b, y = (orc.bf16_rne(t) for t in _lora_draws(M, K, N, rank, 11))
    xf, af, bf, yf = (orc.bf16_to_f32(t).astype(np.float64) for t in (x, a, b, y))
    r = orc.bf16_to_f32(orc.bf16_rne((xf @ af.T).astype(np.float32))).astype(np.float64)
    want = orc.bf16_rne((yf + r @ bf.T).astype(np.float32))
    got = orc.lora_add(x, a, b, y)
    # double -> float -> bf16 in both; the only freedom is summation order in f64
    diff = np.abs(orc.bf16_to_f32(got) - orc.bf16_to_f32(want))
    assert np.count_nonzero(diff) <= max(1, got.size // 1000)


def test_lora_zero_a_leaves_y_bit_identical():
    x, a, b, y = (orc.bf16_rne(t) for t in _lora_draws(16, 64, 48, 4, 3))
    got = orc.lora_add(x, np.zeros_like(a), b, y)
    assert np.array_equal(got, y)


def test_lora_rank1_is_an_outer_product_and_adds():
    # rank 1, y = 0: y[m][n] = bf16(bf16(x[m] . a) * b[n]) -- a wrong operand order, a
    # transposed B or an assignment instead of an add each break one of the two checks.
    rng = np.random.default_rng(5)
    M, K, N = 5, 32, 7
    x = orc.bf16_rne(rng.standard_normal((M, K)).astype(np.float32))
    a = orc.bf16_rne(rng.standard_normal((1, K)).astype(np.float32))
    b = orc.bf16_rne(rng.standard_normal((N, 1)).astype(np.float32))
    r = orc.bf16_to_f32(orc.bf16_rne((orc.bf16_to_f32(x).astype(np.float64) @
                                      orc.bf16_to_f32(a)[0].astype(np.float64)).astype(np.float32)))
    want = orc.bf16_rne((r[:, None].astype(np.float64) *
                         orc.bf16_to_f32(b)[:, 0][None, :].astype(np.float64)).astype(np.float32))
    zero = np.zeros((M, N), np.uint16)
    assert np.array_equal(orc.lora_add(x, a, b, zero), want)
    ones = orc.bf16_rne(np.ones((M, N), np.float32))
    got = orc.bf16_to_f32(orc.lora_add(x, a, b, ones))
    assert np.allclose(got, 1.0 + orc.bf16_to_f32(want), rtol=1e-2, atol=1e-2)


# ---- committed fixtures -----------------------------------------------------------------
def test_golden_fixtures_reproduce():
    files = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert files, "no golden fixtures committed"
    for f in files:
        g = np.load(os.path.join(GOLDEN, f), allow_pickle=False)
        kind = str(g["kind"])
        if kind == "quantize":
            codes, scales, biases, deq = orc.quantize_affine(g["w"], int(g["bits"]), int(g["group"]))
            assert np.array_equal(codes, g["codes"]), f
            assert np.array_equal(scales, g["scales"]), f
            assert np.array_equal(biases, g["biases"]), f
            assert np.array_equal(deq, g["deq"]), f
        elif kind == "qlinear":
            wf, wb = orc.dequant(g["codes"], g["scales"], g["biases"], *g["w_shape"],
                                 int(g["bits"]), int(g["group"]))
            assert np.array_equal(wb, g["w_bf16"]), f
            xf = orc.bf16_to_f32(g["x_bf16"])
            bias = g["bias_f32"] if g["bias_f32"].size else None
            out = orc.linear_f64(xf, orc.bf16_to_f32(wb), bias)
            assert np.array_equal(out, g["y_f32"]), f
        elif kind == "i8":
            q, s = orc.i8_quantize_rows(g["x_bf16"])
            assert np.array_equal(q, g["xq"]) and np.array_equal(s, g["sx"]), f
            wq, sw = orc.i8_quantize_rows(g["w_bf16"])
            assert np.array_equal(wq, g["wq"]) and np.array_equal(sw, g["sw"]), f
            acc = orc.i8_gemm_i32(q, wq)
            assert np.array_equal(acc, g["acc"]), f
            y = orc.i8_epilogue(acc, s, sw, g["bias_f32"], 2)
            assert np.array_equal(y, g["y_bf16"]), f
        elif kind == "gelu":
            assert np.array_equal(orc.gelu(g["x"]), g["y"]), f
        else:
            raise AssertionError(f"unknown fixture kind {kind} in {f}")
