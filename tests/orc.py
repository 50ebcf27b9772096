"""numpy wrappers over the CPU oracle (oracle/liboracle.so) and, where it was
built, the reference's own CPU code (oracle/_ref/libltx25ref.so).

Test infrastructure: the oracle is the checker the HIP path is compared
against, never a path under test.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")
REF_LIB = os.path.join(ORACLE_DIR, "_ref", "libltx25ref.so")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t

_SIGS = {
    "orc_bf16_rne": (ctypes.c_uint16, [ctypes.c_float]),
    "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_f32_to_bf16_n": (None, [_vp, _vp, _sz]),
    "orc_bf16_to_f32_n": (None, [_vp, _vp, _sz]),
    "orc_f16_to_bf16_n": (None, [_vp, _vp, _sz]),
    "orc_quantize_affine": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "orc_pack_codes": (_i, [_vp, _i, _i, _i, _vp]),
    "orc_unpack_codes": (_i, [_vp, _i, _i, _i, _vp]),
    "orc_dequant": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "orc_linear_f64": (None, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "orc_linear_f64_d": (None, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "orc_linear_f32_omp": (None, [_vp, _vp, _vp, _i, _i, _i, _vp, _i]),
    "orc_gelu_tanh": (None, [_vp, _vp, _sz]),
    "orc_bias_add_bf16": (None, [_vp, _vp, _i, _i]),
    "orc_gate_heads": (None, [_vp, _vp, _i, _i, _i]),
    "orc_lora_add": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_i8_quantize_rows": (None, [_vp, _i, _i, _vp, _vp]),
    "orc_i8_gemm_i32": (None, [_vp, _vp, _i, _i, _i, _vp]),
    "orc_i8_epilogue": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "orc_i8_epilogue_ex": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_fill_normal": (None, [_vp, _sz, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]),
}

_lib = None
_ref = None


def lib():
    """The oracle library, built on first use if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
        l = ctypes.CDLL(ORACLE_LIB)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def ref():
    """The reference's own CPU linear_/GELU, or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        r = ctypes.CDLL(REF_LIB)
        r.ref_linear.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
        r.ref_linear.restype = None
        r.ref_rms_norm.argtypes = [_vp, _i, _i, ctypes.c_double]
        r.ref_rms_norm.restype = None
        r.ref_ff_identity.argtypes = [_vp, _i, _i, ctypes.c_double, _vp]
        r.ref_ff_identity.restype = None
        r.ref_gate_identity.argtypes = [_vp, _vp, _i, _i, _i, _vp]
        r.ref_gate_identity.restype = None
        _ref = r
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- number formats ----------------------------------------------------------
def bf16_rne(a) -> np.ndarray:
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(a), _p(out), a.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_bf16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f16_to_bf16(bits) -> np.ndarray:
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.uint16)
    lib().orc_f16_to_bf16_n(_p(bits), _p(out), bits.size)
    return out


# ---- quantization ------------------------------------------------------------
def quantize_affine(w, bits=8, group=64):
    """-> codes u32 [N][K*bits/32], scales u16 [N][K/g], biases u16, deq f32 [N][K]."""
    w = _c(w, np.float32)
    N, K = w.shape
    codes = np.empty((N, K * bits // 32), np.uint32)
    scales = np.empty((N, K // group), np.uint16)
    biases = np.empty((N, K // group), np.uint16)
    deq = np.empty((N, K), np.float32)
    rc = lib().orc_quantize_affine(_p(w), N, K, bits, group, _p(codes), _p(scales), _p(biases),
                                   _p(deq))
    assert rc == 0
    return codes, scales, biases, deq


def pack(q, bits):
    q = _c(q, np.uint8)
    N, K = q.shape
    codes = np.empty((N, K * bits // 32), np.uint32)
    assert lib().orc_pack_codes(_p(q), N, K, bits, _p(codes)) == 0
    return codes


def unpack(codes, N, K, bits):
    codes = _c(codes, np.uint32)
    q = np.empty((N, K), np.uint8)
    assert lib().orc_unpack_codes(_p(codes), N, K, bits, _p(q)) == 0
    return q


def dequant(codes, scales, biases, N, K, bits=8, group=64):
    """-> (f32 [N][K], bf16 bits [N][K]) of fmaf(scale, q, bias)."""
    codes = _c(codes, np.uint32)
    scales = _c(scales, np.uint16)
    biases = _c(biases, np.uint16)
    wf = np.empty((N, K), np.float32)
    wb = np.empty((N, K), np.uint16)
    assert lib().orc_dequant(_p(codes), _p(scales), _p(biases), N, K, bits, group, _p(wf),
                             _p(wb)) == 0
    return wf, wb


# ---- linear / GELU / bias -----------------------------------------------------
def linear_f64(x, w, bias=None) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), np.float32)
    lib().orc_linear_f64(_p(x), _p(w), _p(b), M, K, N, _p(out))
    return out


def linear_f64_d(x, w, bias=None) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), np.float64)
    lib().orc_linear_f64_d(_p(x), _p(w), _p(b), M, K, N, _p(out))
    return out


def linear_f32_omp(x, w, bias=None, threads=1) -> np.ndarray:
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    M, K = x.shape
    N = w.shape[0]
    out = np.empty((M, N), np.float32)
    lib().orc_linear_f32_omp(_p(x), _p(w), _p(b), M, K, N, _p(out), threads)
    return out


def gelu(a) -> np.ndarray:
    a = _c(a, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().orc_gelu_tanh(_p(a), _p(out), a.size)
    return out


def bias_add_bf16(y, bias) -> np.ndarray:
    y = np.array(y, dtype=np.uint16, copy=True)
    bias = _c(bias, np.uint16)
    M, N = y.shape
    lib().orc_bias_add_bf16(_p(y), _p(bias), M, N)
    return y


def gate_heads(y_bf16, logits_bf16, heads: int, head_dim: int) -> np.ndarray:
    """y [tokens][heads*head_dim] * 2 sigmoid(logits [tokens][heads]) on bf16 bit patterns."""
    y = np.array(y_bf16, dtype=np.uint16, copy=True)
    lg = _c(logits_bf16, np.uint16)
    tokens = lg.shape[0]
    assert y.shape == (tokens, heads * head_dim) and lg.shape == (tokens, heads)
    lib().orc_gate_heads(_p(y), _p(lg), heads, tokens, head_dim)
    return y


def lora_add(x_bf16, a_bf16, b_bf16, y_bf16) -> np.ndarray:
    """y + (x . a^T) . b^T on bf16 bit patterns (uint16); returns the new y."""
    x = _c(x_bf16, np.uint16)
    a = _c(a_bf16, np.uint16)
    b = _c(b_bf16, np.uint16)
    y = np.array(y_bf16, dtype=np.uint16, copy=True)
    M, K = x.shape
    rank = a.shape[0]
    N = b.shape[0]
    lib().orc_lora_add(_p(x), _p(a), _p(b), _p(y), M, K, N, rank)
    return y


# ---- int8 tier -----------------------------------------------------------------
def i8_quantize_rows(x_bf16):
    x = _c(x_bf16, np.uint16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    lib().orc_i8_quantize_rows(_p(x), M, K, _p(q), _p(s))
    return q, s


def i8_gemm_i32(xq, wq) -> np.ndarray:
    xq = _c(xq, np.int8)
    wq = _c(wq, np.int8)
    M, K = xq.shape
    N = wq.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().orc_i8_gemm_i32(_p(xq), _p(wq), M, K, N, _p(acc))
    return acc


def i8_epilogue(acc, sx, sw, bias=None, bias_dtype=0, epilogue=0) -> np.ndarray:
    acc = _c(acc, np.int32)
    sx = _c(sx, np.float32)
    sw = _c(sw, np.float32)
    M, N = acc.shape
    if bias is not None:
        bias = _c(bias, np.uint16 if bias_dtype == 1 else np.float32)
    y = np.empty((M, N), np.uint16)
    if epilogue == 0:
        lib().orc_i8_epilogue(_p(acc), _p(sx), _p(sw), _p(bias), bias_dtype, M, N, _p(y))
    else:
        lib().orc_i8_epilogue_ex(_p(acc), _p(sx), _p(sw), _p(bias), bias_dtype, epilogue, M, N,
                                 _p(y))
    return y


def fill_normal(n, seed, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty((n,), np.float32)
    lib().orc_fill_normal(_p(out), n, seed, mean, std)
    return out


# ---- metrics -------------------------------------------------------------------
def rel_l2(a, b) -> float:
    """The reference's rel-L2 (tests/ltx25-qlinear-test.cc:143-153)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    num = float(np.sum((a - b) ** 2))
    den = float(np.sum(b ** 2))
    return float(np.sqrt(num / den)) if den > 0 else float(np.sqrt(num))


def max_rel(y, ref) -> float:
    """Normwise max relative error max|y - ref| / max|ref| (the 1e-2 bar)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(y - ref))) / (den if den > 0 else 1.0)
