"""The pack reader on the GPU: a synthetic checkpoint in the on-disk format
the reference's loader reads (src/ltx25-dit-weights.cc:195-403) -- u32 codes
with F16 scales and biases, as the quantizer writes them -- bound through
ltx25_pack_bind_qlinear and run through the linear. Bars: the bound weight
dequantizes bit-identically to the oracle's dequant over the F16 -> bf16
(RNE) converted scales and biases; the linear over it meets the north-star
bar against the oracle's f64 GEMM; a dense BF16 weight binds unconverted;
the checkpoint's group is fixed by its first quantized linear."""
import ctypes

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import orc
from gpu_util import dev_bf16, host_bits, rng_normal, say

pytestmark = pytest.mark.gpu


def f16_bits(bf16_bits):
    """bf16 values stored as F16, the way the quantizer writes scales and biases."""
    return orc.bf16_to_f32(bf16_bits).astype(np.float16).view(np.uint16)


def t_u16(bits, dtype):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(dtype)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    rng = np.random.default_rng(21)
    K, N = 1024, 384
    lin = {}
    tensors = {}
    for name, bits, group, sdt in [("blk.0.ff_in", 8, 64, "F16"), ("blk.0.to_q", 8, 64, "F32"),
                                   ("blk.1.to_k", 4, 32, "F16")]:
        w = rng_normal(rng, (N, K), 0.02)
        codes, scales, biases, _ = orc.quantize_affine(w, bits, group)
        if sdt == "F16":
            s_store, b_store = f16_bits(scales), f16_bits(biases)
            s_dev, b_dev = orc.f16_to_bf16(s_store), orc.f16_to_bf16(b_store)
            tensors[name + ".scales"] = t_u16(s_store, torch.float16)
            tensors[name + ".biases"] = t_u16(b_store, torch.float16)
        else:
            tensors[name + ".scales"] = torch.from_numpy(orc.bf16_to_f32(scales))
            tensors[name + ".biases"] = torch.from_numpy(orc.bf16_to_f32(biases))
            s_dev, b_dev = scales, biases   # f32 of a bf16 value rounds back to itself
        tensors[name + ".weight"] = torch.from_numpy(codes.copy())   # U32, as packed
        lin[name] = (bits, group, codes, s_dev, b_dev)
    dense = orc.bf16_rne(rng_normal(rng, (N, K), 0.02))
    tensors["blk.0.gate.weight"] = t_u16(dense, torch.bfloat16)
    lin["blk.0.gate"] = (16, 0, dense, None, None)
    path = str(tmp_path_factory.mktemp("pack") / "dit.safetensors")
    save_file(tensors, path, metadata={"format": "pt"})
    return path, K, N, lin


def dequant_c(pkg, cw, N, K):
    out = torch.empty((N, K), dtype=torch.bfloat16, device="cuda")
    pkg.check(pkg.load().ltx25_dequant(torch.cuda.current_stream().cuda_stream,
                                       ctypes.byref(cw), out.data_ptr(), N, K))
    torch.cuda.synchronize()
    return host_bits(out)


def test_bind_quantized_and_dense_and_run(pkg, dev, checkpoint):
    path, K, N, lin = checkpoint
    rng = np.random.default_rng(3)
    M = 200
    x = orc.bf16_rne(rng_normal(rng, (M, K)))
    xd = dev_bf16(x)
    with pkg.Pack(path) as p:
        for name in ("blk.0.ff_in", "blk.0.to_q", "blk.0.gate"):
            bits, group, codes, s_dev, b_dev = lin[name]
            say(f"pack bind {name}")
            cw = p.bind_qlinear(name, K)
            if bits == 16:
                assert not cw.quantized
                wb = codes
            else:
                assert cw.quantized and cw.bits == bits and cw.group == group
                _, wb = orc.dequant(codes, s_dev, b_dev, N, K, bits, group)
                assert np.array_equal(dequant_c(pkg, cw, N, K), wb), name
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            say(f"linear over {name}")
            pkg.linear_qc(xd, cw, None, y, M, K, N)
            torch.cuda.synchronize()
            got = orc.bf16_to_f32(host_bits(y))
            ref = orc.linear_f64(orc.bf16_to_f32(x), orc.bf16_to_f32(wb))
            assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-2, name
        assert p.group == 64
        # the w4g32 linear is in a checkpoint that already bound group 64
        with pytest.raises(pkg.Ltx25Error, match="group"):
            p.bind_qlinear("blk.1.to_k", K)


def test_bind_w4g32_in_its_own_checkpoint_and_reuse(pkg, dev, checkpoint):
    path, K, N, lin = checkpoint
    bits, group, codes, s_dev, b_dev = lin["blk.1.to_k"]
    with pkg.Pack(path) as p:
        say("pack bind blk.1.to_k (w4g32)")
        cw = p.bind_qlinear("blk.1.to_k", K)
        assert cw.bits == 4 and cw.group == 32 and p.group == 32
        _, wb = orc.dequant(codes, s_dev, b_dev, N, K, bits, group)
        assert np.array_equal(dequant_c(pkg, cw, N, K), wb)
        # read_bf16 returns the same cached device copy the bind used
        ptr, n = p.read_bf16("blk.1.to_k.scales")
        assert ptr == cw.scales and n == N * K // 32
