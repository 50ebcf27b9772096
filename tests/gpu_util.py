"""Moving oracle-format numpy arrays to and from device tensors."""
import sys

import numpy as np
import torch

import orc


def say(msg: str) -> None:
    """Name the case before a GPU step, flushed, so a crash names it."""
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def dev_bf16(bits_u16: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(bits_u16, np.uint16).view(np.int16)
    return torch.from_numpy(a.copy()).view(torch.bfloat16).cuda()


def dev_bytes(a: np.ndarray) -> torch.Tensor:
    b = np.ascontiguousarray(a).view(np.uint8).reshape(a.shape[0], -1)
    return torch.from_numpy(b.copy()).cuda()


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32).copy()).cuda()


def host_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 device tensor -> its uint16 bit patterns."""
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def host_f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def make_qweight(pkg, w_f32: np.ndarray, bits=8, group=64):
    """Quantize on the CPU oracle and upload. Returns (QWeight, codes, scales,
    biases, w_bf16_dequant_bits)."""
    N, K = w_f32.shape
    codes, scales, biases, _ = orc.quantize_affine(w_f32, bits, group)
    _, wb = orc.dequant(codes, scales, biases, N, K, bits, group)
    qw = pkg.QWeight(dev_bytes(codes), dev_bf16(scales), dev_bf16(biases), bits, group)
    return qw, codes, scales, biases, wb


def rng_normal(rng, shape, std=1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(np.float32)
