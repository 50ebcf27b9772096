"""The measurement probes (ltx25_probe_read / ltx25_probe_mfma) on the GPU: the
read probe reads exactly the span it is given (each workgroup's XOR of its
16-byte words checked against numpy), and the MFMA probe runs to completion
at both wave counts and operand kinds."""
import numpy as np
import pytest
import torch

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks", [(16, 1), (4096, 3), (1 << 20, 7), (5496832, 256)])
def test_probe_read_covers_the_span(pkg, dev, nbytes, blocks):
    rng = np.random.default_rng(nbytes + blocks)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    src = torch.from_numpy(host.view(np.int32).copy()).cuda()
    sink = torch.zeros((blocks,), dtype=torch.int32, device="cuda")
    say(f"probe_read bytes={nbytes} blocks={blocks}")
    pkg.probe_read(src, nbytes, sink, blocks)
    torch.cuda.synchronize()
    n16 = nbytes // 16
    per = (n16 + blocks - 1) // blocks
    want = np.zeros(blocks, np.uint32)
    for b in range(blocks):
        span = host[4 * b * per: 4 * min(n16, (b + 1) * per)]
        want[b] = np.bitwise_xor.reduce(span) if span.size else 0
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)


@pytest.mark.parametrize("random", [False, True])
@pytest.mark.parametrize("wps", [1, 2])
def test_probe_mfma_runs(pkg, dev, random, wps):
    out = torch.zeros((256,), dtype=torch.float32, device="cuda")
    say(f"probe_mfma random={random} waves_per_simd={wps}")
    pkg.probe_mfma(100, random, wps, out)
    torch.cuda.synchronize()


# (M, K, N, k_chunk, splits): the planner's split, forced 2- and 4-way splits, K > 2048
PHASE_CASES = [(126, 2048, 96, 0, 1), (126, 2048, 64, 1024, 2), (100, 2048, 40, 512, 4),
               (126, 8192, 64, 0, 4)]


@pytest.mark.parametrize("M,K,N,k_chunk,splits", PHASE_CASES)
def test_probe_skinny_phases(pkg, dev, M, K, N, k_chunk, splits):
    """The phase-stamp instantiation computes what the linear computes (bit for bit: the
    same sums in the same order, plus clock reads) and writes ordered stamps for every wave
    of every workgroup, the split count included."""
    from gpu_util import make_qweight, rng_normal
    rng = np.random.default_rng(M + K + N + k_chunk)
    qw = make_qweight(pkg, rng_normal(rng, (N, K), 0.02), 8, 64)[0]
    x = torch.from_numpy(rng_normal(rng, (M, K))).to(torch.bfloat16).cuda()
    bias = torch.from_numpy(rng_normal(rng, (N,), 0.1)).cuda()
    tiles = (N + 31) // 32
    nwords = splits * tiles * 8 * 10
    stamps = torch.zeros((nwords + 80,), dtype=torch.int64, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"probe_skinny_phases M={M} K={K} N={N} k_chunk={k_chunk}")
    got_splits = pkg.probe_skinny_phases(x, qw, bias, y, M, K, N, k_chunk, stamps, nwords * 8)
    torch.cuda.synchronize()
    assert got_splits == splits
    want = torch.empty_like(y)
    if k_chunk == 0:
        pkg.linear_q(x, qw, bias, want, M, K, N)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    else:
        # a forced split sums the same products in another order: the oracle's tolerance
        # (bf16 rounding of the f32 sum) against the linear's own result
        pkg.linear_q(x, qw, bias, want, M, K, N)
        torch.cuda.synchronize()
        assert torch.allclose(y.float(), want.float(), rtol=1e-2, atol=1e-2)
    s = stamps.cpu().numpy()
    assert not s[nwords:].any(), "stamps written past splits * tiles * 8 waves"
    s = s[:nwords].reshape(splits * tiles, 8, 10)
    clk = s[..., :6]
    assert (np.diff(clk, axis=-1) >= 0).all(), "shader-clock stamps out of phase order"
    assert (s[..., 7] >= s[..., 6]).all() and (s[..., 6] > 0).all()


def test_probe_skinny_phases_rejects(pkg, dev):
    from gpu_util import make_qweight, rng_normal
    rng = np.random.default_rng(5)
    qw = make_qweight(pkg, rng_normal(rng, (64, 2048), 0.02), 8, 64)[0]
    x = torch.zeros((126, 2048), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((126, 64), dtype=torch.bfloat16, device="cuda")
    stamps = torch.zeros((4 * 2 * 8 * 10,), dtype=torch.int64, device="cuda")
    for k_chunk, nbytes in ((100, stamps.numel() * 8), (4096, stamps.numel() * 8),
                            (512, 2 * 8 * 10 * 8 * 3)):   # 4 splits need 4 x 2 tiles
        with pytest.raises(pkg.Ltx25Error):
            pkg.probe_skinny_phases(x, qw, None, y, 126, 2048, 64, k_chunk, stamps, nbytes)


def _check_tall_stamps(st, tiles):
    s = st.cpu().numpy()
    assert not s[tiles * 64:].any(), "stamps written past tiles * 8 waves"
    s = s[:tiles * 64].reshape(tiles, 8, 8)
    assert (s[..., 5] > 0).all(), "a wave wrote no stamps"
    assert (np.diff(s[..., :5], axis=-1) >= 0).all(), "shader-clock stamps out of phase order"
    assert (s[..., 6] >= s[..., 5]).all()
    assert ((s[..., 7] >> 32) < 8).all()


# (M, K, N, bias dtype): whole tiles, and ragged M and N. K <= 512 keeps the dense linear
# on one K split (the planner splits from 1024 of K), so both sum in the same order.
TALL_PHASE_CASES = [(512, 256, 512, "f32"), (300, 512, 264, "bf16"), (1024, 512, 2048, None)]


@pytest.mark.parametrize("M,K,N,bias_dt", TALL_PHASE_CASES)
def test_probe_tall_phases(pkg, dev, M, K, N, bias_dt):
    """The bf16 tile's phase-stamp instantiation gives the bits the dense linear gives (the
    same sums in the same K order on either tile) and stamps every wave of every tile."""
    rng = np.random.default_rng(M + K + N)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = torch.from_numpy((rng.standard_normal((N, K)) * 0.05).astype(np.float32)).to(
        torch.bfloat16).cuda()
    bias = None
    if bias_dt is not None:
        b = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float32)).cuda()
        bias = b.to(torch.bfloat16) if bias_dt == "bf16" else b
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    st = torch.zeros((tiles * 64 + 64,), dtype=torch.int64, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say(f"probe_tall_phases M={M} K={K} N={N} bias={bias_dt}")
    pkg.probe_tall_phases(x, w, bias, y, M, K, N, pkg.EPI_NONE, st, tiles * 512)
    want = torch.empty_like(y)
    pkg.linear(x, w, bias, want, M, K, N)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    _check_tall_stamps(st, tiles)
    st.zero_()
    pkg.probe_tall_phases(x, w, bias, y, M, K, N, pkg.EPI_GELU_TANH, st, tiles * 512)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    _check_tall_stamps(st, tiles)


@pytest.mark.parametrize("M,K,N", [(512, 256, 512), (300, 384, 264)])
def test_probe_tall_i8_phases(pkg, dev, M, K, N):
    """The int8 tile's phase-stamp instantiation gives the bits ltx25_i8_gemm gives."""
    rng = np.random.default_rng(M * 7 + N)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = torch.from_numpy((rng.standard_normal((N, K)) * 0.05).astype(np.float32)).to(
        torch.bfloat16).cuda()
    xq = torch.empty((M, K), dtype=torch.int8, device="cuda")
    wq = torch.empty((N, K), dtype=torch.int8, device="cuda")
    sx = torch.empty((M,), dtype=torch.float32, device="cuda")
    sw = torch.empty((N,), dtype=torch.float32, device="cuda")
    pkg.i8_quantize_rows(x, xq, sx, M, K)
    pkg.i8_quantize_rows(w, wq, sw, N, K)
    bias = torch.from_numpy((rng.standard_normal(N) * 0.1).astype(np.float32)).cuda()
    tiles = ((M + 255) // 256) * ((N + 255) // 256)
    st = torch.zeros((tiles * 64 + 64,), dtype=torch.int64, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    want = torch.empty_like(y)
    say(f"probe_tall_i8_phases M={M} K={K} N={N}")
    pkg.probe_tall_i8_phases(xq, sx, wq, sw, bias, y, M, K, N, st, tiles * 512)
    pkg.i8_gemm(xq, sx, wq, sw, bias, want, None, M, K, N)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    _check_tall_stamps(st, tiles)


def test_probe_tall_phases_rejects(pkg, dev):
    x = torch.zeros((256, 256), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((256, 256), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((256, 256), dtype=torch.bfloat16, device="cuda")
    st = torch.zeros((64,), dtype=torch.int64, device="cuda")
    with pytest.raises(pkg.Ltx25Error):     # one tile needs 512 bytes of stamps
        pkg.probe_tall_phases(x, w, None, y, 256, 256, 256, pkg.EPI_NONE, st, 511)
    with pytest.raises(pkg.Ltx25Error):     # K not a multiple of 64
        pkg.probe_tall_phases(x, w, None, y, 256, 200, 256, pkg.EPI_NONE, st, 512)
    with pytest.raises(pkg.Ltx25Error):     # unknown epilogue
        pkg.probe_tall_phases(x, w, None, y, 256, 256, 256, 7, st, 512)
