"""Every GEMM route at the same shapes, through the C ABI's tile switch
(ltx25_set_tile, the A/B hook the reference keeps as VPIPE_LTX25_MMA_TILE,
src/ltx25-metal-ops.cc:193-231), and the row slabs that keep each operand of
a launch under 2 GiB (the reference's operand limit, :342-374).

Each forced route is asserted through ltx25_linear_route before it runs, so a
test cannot pass on a route it did not mean to measure. Bars as in
test_gpu_qlinear.py: max|y - ref| / max|ref| <= 1e-2 against the oracle's f64
GEMM over the dequantized weight on sampled rows, rel-L2 < 3e-3 on all rows
against torch fp32 of the same operands; within one route the quantized
weight and its GPU-dequantized bf16 copy give bit-identical outputs.
"""
import numpy as np
import pytest
import torch

import orc
from gpu_util import dev_bf16, dev_f32, host_bits, host_f32, make_qweight, rng_normal, say
from test_gpu_qlinear import check_full_vs_torch, check_rows_vs_oracle, sample_rows

pytestmark = pytest.mark.gpu

SHAPES = [  # name, M, K, N, bias
    ("audio qkv", 126, 2048, 6144, True),
    ("audio ff_down (split K)", 126, 8192, 2048, True),
    ("config 0", 320, 4096, 4096, True),
    ("text kv", 1024, 4096, 8192, True),
    ("ragged M and N", 777, 2048, 1000, False),
    ("N not a multiple of 256", 192, 16384, 260, False),
]
TILES = [("tall", 1), ("mid", 2), ("skinny", 3)]


@pytest.fixture(autouse=True)
def _reset_tile(pkg):
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    pkg.set_tile(pkg.TILE_AUTO)


@pytest.mark.parametrize("tile_name,tile", TILES, ids=[t[0] for t in TILES])
@pytest.mark.parametrize("name,M,K,N,has_bias", SHAPES, ids=[s[0] for s in SHAPES])
def test_forced_tile(pkg, name, M, K, N, has_bias, tile_name, tile):
    rng = np.random.default_rng(40 + M + N)
    x_bits = orc.bf16_rne(rng_normal(rng, (M, K)))
    w = rng_normal(rng, (N, K), 0.02)
    b = rng_normal(rng, (N,), 0.01) if has_bias else None
    qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
    pkg.set_tile(tile)
    route = pkg.linear_route(M, K, N)
    want = tile if (tile != 3 or M <= 128) else route["tile"]
    assert route["tile"] == want, route
    say(f"forced tile {tile_name}: {name} {M}x{K}->{N} route={route}")
    x_dev = dev_bf16(x_bits)
    b_dev = dev_f32(b) if b is not None else None
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.linear_q(x_dev, qw, b_dev, y, M, K, N)
    w_deq = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(qw, w_deq, N, K)
    yd = torch.empty_like(y)
    pkg.linear(x_dev, w_deq, b_dev, yd, M, K, N)
    torch.cuda.synchronize()
    assert pkg.linear_route(M, K, N, bits=16)["tile"] == route["tile"]
    assert np.array_equal(host_bits(y), host_bits(yd)), "quantized and dense differ"
    wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    check_rows_vs_oracle(y, orc.bf16_to_f32(x_bits), wf, b, sample_rows(M, 12))
    check_full_vs_torch(y, x_dev, dev_bf16(wb), b_dev)


@pytest.mark.parametrize("quantized", [False, True], ids=["dense", "w8g64"])
def test_row_slabs_past_2gib(pkg, quantized):
    """X of 2.2 GB: two row slabs, each launch's operands under 2 GiB. Rows on both
    sides of the slab boundary and the last row against the oracle."""
    M, K, N = 270000, 4096, 256
    route = pkg.linear_route(M, K, N, bits=8 if quantized else 16)
    assert route["slabs"] == 2, route
    edge = route["slab_rows"]
    say(f"row slabs: {M}x{K}->{N} quantized={quantized} slab_rows={edge}")
    rng = np.random.default_rng(41)
    w = rng_normal(rng, (N, K), 0.02)
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    if quantized:
        qw, codes, scales, biases, wb = make_qweight(pkg, w, 8, 64)
        pkg.linear_q(x, qw, None, y, M, K, N)
        wf, _ = orc.dequant(codes, scales, biases, N, K, 8, 64)
    else:
        wb = orc.bf16_rne(w)
        pkg.linear(x, dev_bf16(wb), None, y, M, K, N)
        wf = orc.bf16_to_f32(wb)
    torch.cuda.synchronize()
    assert not torch.isnan(y.float()).any(), "rows left unwritten"
    rows = np.array([0, 1, edge - 2, edge - 1, edge, edge + 1, M - 2, M - 1] +
                    list(rng.integers(0, M, 8)))
    xr = orc.bf16_to_f32(host_bits(x[torch.from_numpy(rows).cuda()]))
    ref = orc.linear_f64_d(xr, wf)
    got = host_f32(y)[rows]
    assert orc.max_rel(got, ref) <= 1e-2
    assert orc.rel_l2(got, ref) < 3e-3
