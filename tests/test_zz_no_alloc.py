"""ltx25_linear_q_noalloc, the linear that allocates nothing, against the
entry point it varies (ltx25_linear_q_ex), through the C ABI.

The variant runs the same GEMM plan with its split-K partials in a fixed
per-GPU device array. Its output must be bit-identical to linear_q_ex's on
the same operands (the in-register dequant stands in for the dequant-once
expansion, which produces the same bits). Each pair of calls runs back to
back, the second on a smaller input, so stale partials of the first call
sit in the shared array when the second runs. The device's free memory is
read around every call after set-up (ltx25_init, which resolves this GPU's
copy of the array; the runtime places it in device memory then): the
variant must not change it. As a check that
both entry points are not wrong together, each output is also held to
rel-L2 < 3e-3 against torch fp32 over the same bf16 operands.
"""
import numpy as np
import pytest
import torch

from gpu_util import make_qweight, rng_normal, say

pytestmark = pytest.mark.gpu

# (name, M, K, N, bits, group, bias dtype, epilogue); first of each pair is the larger input
PAIRS = [
    ("mid split-K then skinny split-K",
     (256, 2048, 2048, 8, 64, "f32", 1), (64, 4096, 4096, 8, 64, "bf16", 0)),
    ("skinny split-K then skinny",
     (126, 8192, 2048, 8, 64, "bf16", 0), (126, 2048, 2048, 8, 64, None, 1)),
    ("tall (dequant-once in the entry point) then mid split-K",
     (4096, 4096, 4096, 8, 64, "bf16", 1), (300, 2048, 2048, 8, 64, "f32", 0)),
    ("w4 skinny split-K then w4 mid",
     (126, 4096, 4096, 4, 32, "f32", 0), (192, 2048, 1024, 4, 32, None, 0)),
    # linear_q_ex expands the w4 weight and runs the 16x16x32 tile; the
    # no-allocation call runs the template's fused 32x32x16 w4 tile
    ("w4 tall (dequant-once in the entry point vs fused w4 tile) then w4 mid",
     (1024, 4096, 4096, 4, 32, None, 1), (512, 1024, 2048, 4, 64, "f32", 0)),
]


@pytest.fixture(autouse=True)
def _defaults(pkg, lib):
    torch.backends.cuda.matmul.allow_tf32 = False
    assert lib.ltx25_init() == 0, pkg.last_error()
    pkg.set_i8_gemm(False)
    pkg.set_tile(pkg.TILE_AUTO)
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    yield
    pkg.set_i8_gemm(False)
    pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)


def _operands(pkg, M, K, N, bits, group, bias_dt, seed):
    rng = np.random.default_rng(seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((M, K), device="cuda", generator=g).to(torch.bfloat16)
    w = rng_normal(rng, (N, K), 0.02)
    qw = make_qweight(pkg, w, bits, group)[0]
    bias = None
    if bias_dt is not None:
        b = torch.randn((N,), device="cuda", generator=g) * 0.05
        bias = b.to(torch.bfloat16) if bias_dt == "bf16" else b.float()
    return x, qw, bias


def _torch_ref(pkg, x, qw, bias, M, K, N, epi):
    wd = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.dequant(qw, wd, N, K)
    ref = x.float() @ wd.float().t()
    if bias is not None:
        ref = ref + bias.float()
    if epi == 1:
        ref = torch.nn.functional.gelu(ref, approximate="tanh")
    return ref


def _one(pkg, case, seed):
    M, K, N, bits, group, bias_dt, epi = case
    x, qw, bias = _operands(pkg, M, K, N, bits, group, bias_dt, seed)
    route = pkg.linear_route(M, K, N, bits)
    say(f"no-alloc linear M={M} K={K} N={N} w{bits}g{group} bias={bias_dt} epi={epi} "
        f"route={route}")
    want = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    pkg.linear_q(x, qw, bias, want, M, K, N, epi)
    got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    pkg.linear_q_noalloc(x, qw, bias, got, M, K, N, epi)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
        f"{int((got.view(torch.int16) != want.view(torch.int16)).sum())} outputs differ"
    ref = _torch_ref(pkg, x, qw, bias, M, K, N, epi)
    rel = ((got.float() - ref).norm() / ref.norm()).item()
    assert rel < 3e-3, rel
    return route


@pytest.mark.parametrize("name,first,second", PAIRS, ids=[p[0] for p in PAIRS])
def test_noalloc_matches_linear_q_ex(pkg, name, first, second):
    r1 = _one(pkg, first, 11 + first[0])
    r2 = _one(pkg, second, 23 + second[0])
    # the pair must exercise the shared scratch at least once
    assert r1["splits"] > 1 or r2["splits"] > 1


def test_noalloc_refuses_the_int8_tier(pkg):
    M, K, N = 1024, 2048, 2048
    pkg.set_i8_gemm(True)
    assert pkg.i8_takes(M, K, N)
    x, qw, _ = _operands(pkg, M, K, N, 8, 64, None, 5)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    say("no-alloc linear refuses the int8 tier")
    with pytest.raises(pkg.Ltx25Error) as e:
        pkg.linear_q_noalloc(x, qw, None, y, M, K, N)
    assert e.value.code == pkg.E_UNSUPPORTED
    assert "int8" in str(e.value)


def test_noalloc_scratch_size(pkg):
    assert pkg.noalloc_scratch_bytes() == 32 << 20
