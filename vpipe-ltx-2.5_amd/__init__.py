"""Python binding of the ltx25 quantized-linear C ABI (include/ltx25_qlinear.h).

A thin ctypes layer over libltx25_qlinear.so for tests and the benchmark:
device buffers are torch tensors (plumbing only) whose data pointers are
passed through the C ABI, and every call runs on torch's current stream
unless a stream is given. The HIP library is the only compute path; when it
is missing, load() raises instead of falling back to anything else.

The package directory name is not a Python identifier, so callers import it
by path; ``load_package()`` in __graft_entry__.py and tests/conftest.py do
that.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libltx25_qlinear.so")
HEADER_PATH = os.path.join(HERE, "..", "include", "ltx25_qlinear.h")

OK = 0
E_INVAL = 1
E_UNSUPPORTED = 2
E_HIP = 3
E_NODEV = 4
E_DECLINED = 5

DT_NONE = 0
DT_BF16 = 1
DT_F32 = 2

EPI_NONE = 0
EPI_GELU_TANH = 1

DEQUANT_ONCE_OFF = 0
DEQUANT_ONCE_ON = 1
DEQUANT_ONCE_AUTO = 2

TILE_AUTO = 0
TILE_TALL = 1
TILE_MID = 2
TILE_SKINNY = 3

LORA_AUTO = 0
LORA_NONE = 0
LORA_PAIR = 1
LORA_RFIRST = 2
LORA_FUSED = 3


class QWeightC(ctypes.Structure):
    """ltx25_qweight (mirrors QWeight, src/ltx25-metal-ops.h:45-57)."""

    _fields_ = [
        ("w", ctypes.c_void_p),
        ("codes", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("qbias", ctypes.c_void_p),
        ("bits", ctypes.c_int),
        ("group", ctypes.c_int),
        ("quantized", ctypes.c_int),
    ]


class RouteC(ctypes.Structure):
    """ltx25_route: what a linear runs on (ltx25_linear_route)."""

    _fields_ = [
        ("tile", ctypes.c_int),
        ("i8", ctypes.c_int),
        ("dequant_once", ctypes.c_int),
        ("splits", ctypes.c_int),
        ("slabs", ctypes.c_int),
        ("slab_rows", ctypes.c_int),
        ("scratch_bytes", ctypes.c_size_t),
    ]


class Ltx25Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"ltx25 error {code}: {msg}")
        self.code = code


_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_long = ctypes.c_long

# name -> (restype, argtypes)
SIGNATURES = {
    "ltx25_init": (_i, []),
    "ltx25_last_error": (ctypes.c_char_p, []),
    "ltx25_quant_available": (_i, []),
    "ltx25_linear_q": (_i, [_vp, _vp, ctypes.POINTER(QWeightC), _vp, _i, _vp, _i, _i, _i]),
    "ltx25_linear_q_ex": (_i, [_vp, _vp, ctypes.POINTER(QWeightC), _vp, _i, _vp, _i, _i, _i, _i]),
    "ltx25_linear_q_noalloc": (_i, [_vp, _vp, ctypes.POINTER(QWeightC), _vp, _i, _vp, _i, _i, _i,
                                    _i]),
    "ltx25_noalloc_scratch_bytes": (_sz, []),
    "ltx25_linear": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i]),
    "ltx25_bias_add": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "ltx25_gelu_tanh": (_i, [_vp, _vp, _vp, _sz]),
    "ltx25_gate_heads": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "ltx25_probe_read": (_i, [_vp, _vp, _sz, _vp, _i]),
    "ltx25_probe_mfma": (_i, [_vp, _i, _i, _i, _vp]),
    "ltx25_probe_skinny_phases": (_i, [_vp, _vp, ctypes.POINTER(QWeightC), _vp, _i, _vp, _i, _i,
                                       _i, _i, _vp, _sz, ctypes.POINTER(ctypes.c_int)]),
    "ltx25_probe_tall_phases": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz]),
    "ltx25_probe_tall_i8_phases": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _vp,
                                        _sz]),
    "ltx25_dequant": (_i, [_vp, ctypes.POINTER(QWeightC), _vp, _i, _i]),
    "ltx25_set_dequant_once": (_i, [_i]),
    "ltx25_dequant_once_takes": (_i, [_i, _i, _i]),
    "ltx25_lora_add": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "ltx25_lora_on_matrix_cores": (_i, [_i, _i, _i, _i]),
    "ltx25_set_lora_matrix_cores": (_i, [_i]),
    "ltx25_set_lora_route": (_i, [_i]),
    "ltx25_lora_route": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, ctypes.POINTER(_i)]),
    "ltx25_linear_q_lora": (_i, [_vp, _vp, ctypes.POINTER(QWeightC), _vp, _i, _vp, _vp, _i, _vp,
                                 _i, _i, _i, _i]),
    "ltx25_lora_fold_takes": (_i, [_i, _i, _i, _i, _i]),
    "ltx25_set_tile": (_i, [_i]),
    "ltx25_linear_route": (_i, [_i, _i, _i, _i, ctypes.POINTER(RouteC)]),
    "ltx25_set_i8_gemm": (_i, [_i]),
    "ltx25_i8_takes": (_i, [_i, _i, _i]),
    "ltx25_i8_quantize_rows": (_i, [_vp, _vp, _vp, _vp, _i, _i]),
    "ltx25_i8_quantize_qweight": (_i, [_vp, ctypes.POINTER(QWeightC), _vp, _vp, _i, _i]),
    "ltx25_i8_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i]),
    "ltx25_pack_codes": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "ltx25_unpack_codes": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "ltx25_quantize_affine": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "ltx25_f16_to_bf16": (_i, [_vp, _vp, _vp, _sz]),
    "ltx25_qweight_infer": (_i, [_i, _long, _long, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "ltx25_pack_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "ltx25_pack_close": (None, [_vp]),
    "ltx25_pack_tensor": (_i, [_vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_i),
                               ctypes.POINTER(_long)]),
    "ltx25_pack_metadata": (ctypes.c_char_p, [_vp, ctypes.c_char_p]),
    "ltx25_pack_read_bf16": (_i, [_vp, _vp, ctypes.c_char_p, ctypes.POINTER(_vp),
                                  ctypes.POINTER(_sz)]),
    "ltx25_pack_bind_qlinear": (_i, [_vp, _vp, ctypes.c_char_p, _i, ctypes.POINTER(_i),
                                     ctypes.POINTER(QWeightC), ctypes.c_char_p, _sz]),
    "ltx25_pack_quantizable": (_i, [ctypes.c_char_p, ctypes.c_char_p, _i]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libltx25_qlinear.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().ltx25_last_error().decode()


def check(rc: int) -> None:
    if rc != OK:
        raise Ltx25Error(rc, last_error())


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is not None:
        return stream
    import torch

    return torch.cuda.current_stream().cuda_stream


def bias_dtype_of(bias) -> int:
    if bias is None:
        return DT_NONE
    import torch

    if bias.dtype == torch.bfloat16:
        return DT_BF16
    if bias.dtype == torch.float32:
        return DT_F32
    raise TypeError(f"bias must be bf16 or f32, got {bias.dtype}")


class QWeight:
    """A packed linear weight held in torch device tensors.

    codes: uint8 [N][K*bits/8] (the little-endian bytes of the u32 words),
    scales / qbias: bf16 [N][K/group].
    """

    def __init__(self, codes, scales, qbias, bits: int = 8, group: int = 64):
        self.codes, self.scales, self.qbias = codes, scales, qbias
        self.bits, self.group = bits, group

    def c(self) -> QWeightC:
        return QWeightC(None, _ptr(self.codes), _ptr(self.scales), _ptr(self.qbias),
                        self.bits, self.group, 1)


def dense_weight(w) -> QWeightC:
    return QWeightC(_ptr(w), None, None, None, 0, 0, 0)


def linear_q(x, w: QWeight, bias, y, M: int, K: int, N: int, epilogue: int = EPI_NONE,
             stream=None) -> None:
    cw = w.c()
    check(load().ltx25_linear_q_ex(_stream(stream), _ptr(x), ctypes.byref(cw), _ptr(bias),
                                   bias_dtype_of(bias), _ptr(y), M, K, N, epilogue))


def linear_q_noalloc(x, w: QWeight, bias, y, M: int, K: int, N: int, epilogue: int = EPI_NONE,
                     stream=None) -> None:
    """linear_q that allocates nothing: split-K partials in the library's fixed
    per-GPU scratch (noalloc_scratch_bytes()); overlapping calls on one GPU race."""
    cw = w.c()
    check(load().ltx25_linear_q_noalloc(_stream(stream), _ptr(x), ctypes.byref(cw), _ptr(bias),
                                        bias_dtype_of(bias), _ptr(y), M, K, N, epilogue))


def noalloc_scratch_bytes() -> int:
    return int(load().ltx25_noalloc_scratch_bytes())


def linear_q_lora(x, w: QWeight, bias, a, b, rank: int, y, M: int, K: int, N: int,
                  epilogue: int = EPI_NONE, stream=None) -> None:
    """The linear and its adapter (a [rank][K], b [N][rank]) in one call, the
    adapter added before the epilogue; folded into the GEMM where
    lora_fold_takes says so."""
    cw = w.c()
    check(load().ltx25_linear_q_lora(_stream(stream), _ptr(x), ctypes.byref(cw), _ptr(bias),
                                     bias_dtype_of(bias), _ptr(a), _ptr(b), rank, _ptr(y), M, K,
                                     N, epilogue))


def lora_fold_takes(M: int, K: int, N: int, rank: int, bits: int = 8) -> bool:
    return bool(load().ltx25_lora_fold_takes(M, K, N, rank, bits))


def linear(x, w, bias, y, M: int, K: int, N: int, stream=None) -> None:
    check(load().ltx25_linear(_stream(stream), _ptr(x), _ptr(w), _ptr(bias),
                              bias_dtype_of(bias), _ptr(y), M, K, N))


def bias_add(y, bias, M: int, N: int, stream=None) -> None:
    check(load().ltx25_bias_add(_stream(stream), _ptr(y), _ptr(bias), bias_dtype_of(bias), M, N))


def gelu_tanh(x, y, stream=None) -> None:
    check(load().ltx25_gelu_tanh(_stream(stream), _ptr(x), _ptr(y), x.numel()))


def gate_heads(y, logits, heads: int, tokens: int, head_dim: int, stream=None) -> None:
    check(load().ltx25_gate_heads(_stream(stream), _ptr(y), _ptr(logits), heads, tokens,
                                  head_dim))


def probe_read(src, nbytes: int, sink, blocks: int, stream=None) -> None:
    """The streaming-read ceiling probe (ltx25_probe_read)."""
    check(load().ltx25_probe_read(_stream(stream), _ptr(src), nbytes, _ptr(sink), blocks))


def probe_mfma(iters: int, random: bool, waves_per_simd: int, out, stream=None) -> None:
    """The MFMA-stream ceiling probe (ltx25_probe_mfma)."""
    check(load().ltx25_probe_mfma(_stream(stream), iters, 1 if random else 0, waves_per_simd,
                                  _ptr(out)))


def probe_skinny_phases(x, w: QWeight, bias, y, M: int, K: int, N: int, k_chunk: int, stamps,
                        stamps_bytes: int, stream=None) -> int:
    """One w8 linear on the M <= 128 kernel's phase-stamp instantiation
    (ltx25_probe_skinny_phases); returns the number of K splits."""
    cw = w.c()
    splits = ctypes.c_int(0)
    check(load().ltx25_probe_skinny_phases(_stream(stream), _ptr(x), ctypes.byref(cw), _ptr(bias),
                                           bias_dtype_of(bias), _ptr(y), M, K, N, k_chunk,
                                           _ptr(stamps), stamps_bytes, ctypes.byref(splits)))
    return splits.value


def probe_tall_phases(x, w_bf16, bias, y, M: int, K: int, N: int, epilogue: int, stamps,
                      stamps_bytes: int, stream=None) -> None:
    """The dense bf16 GEMM on the 256 x 256 tile's phase-stamp instantiation
    (ltx25_probe_tall_phases)."""
    check(load().ltx25_probe_tall_phases(_stream(stream), _ptr(x), _ptr(w_bf16), _ptr(bias),
                                         bias_dtype_of(bias), _ptr(y), M, K, N, epilogue,
                                         _ptr(stamps), stamps_bytes))


def probe_tall_i8_phases(xq, sx, wq, sw, bias, y, M: int, K: int, N: int, stamps,
                         stamps_bytes: int, stream=None) -> None:
    """The int8 GEMM on the 256 x 256 tile's phase-stamp instantiation
    (ltx25_probe_tall_i8_phases)."""
    check(load().ltx25_probe_tall_i8_phases(_stream(stream), _ptr(xq), _ptr(sx), _ptr(wq),
                                            _ptr(sw), _ptr(bias), bias_dtype_of(bias), _ptr(y),
                                            M, K, N, _ptr(stamps), stamps_bytes))


def dequant(w: QWeight, out, N: int, K: int, stream=None) -> None:
    cw = w.c()
    check(load().ltx25_dequant(_stream(stream), ctypes.byref(cw), _ptr(out), N, K))


def quantize_affine(w_f32, codes, scales, qbias, N: int, K: int, bits: int = 8,
                    group: int = 64, stream=None) -> None:
    check(load().ltx25_quantize_affine(_stream(stream), _ptr(w_f32), _ptr(codes), _ptr(scales),
                                       _ptr(qbias), N, K, bits, group))


def pack_codes(q, codes, N: int, K: int, bits: int, stream=None) -> None:
    check(load().ltx25_pack_codes(_stream(stream), _ptr(q), _ptr(codes), N, K, bits))


def unpack_codes(codes, q, N: int, K: int, bits: int, stream=None) -> None:
    check(load().ltx25_unpack_codes(_stream(stream), _ptr(codes), _ptr(q), N, K, bits))


def f16_to_bf16(src, dst, stream=None) -> None:
    check(load().ltx25_f16_to_bf16(_stream(stream), _ptr(src), _ptr(dst), src.numel()))


def set_dequant_once(mode) -> None:
    """DEQUANT_ONCE_OFF / _ON / _AUTO (the default); a bool means OFF / ON."""
    check(load().ltx25_set_dequant_once(int(mode)))


def dequant_once_takes(M: int, K: int, N: int) -> bool:
    return bool(load().ltx25_dequant_once_takes(M, K, N))


def lora_add(x, a, b, y, M: int, K: int, N: int, rank: int, r=None, d=None,
             stream=None) -> None:
    """y += (x . a^T) . b^T in place (MetalOps::lora_add). r: optional caller scratch
    [M][rank] (16-byte aligned) that receives r = bf16(x . a^T) on the r-first route and
    on the GEMM pair when rank % 64 == 0; d is unused."""
    check(load().ltx25_lora_add(_stream(stream), _ptr(x), _ptr(a), _ptr(b), _ptr(y), _ptr(r),
                                _ptr(d), M, K, N, rank))


def lora_on_matrix_cores(M: int, K: int, N: int, rank: int) -> bool:
    return bool(load().ltx25_lora_on_matrix_cores(M, K, N, rank))


def set_lora_matrix_cores(on: bool) -> None:
    check(load().ltx25_set_lora_matrix_cores(1 if on else 0))


def set_lora_route(route: int) -> None:
    """LORA_AUTO / LORA_PAIR / LORA_RFIRST / LORA_FUSED for every later lora_add."""
    check(load().ltx25_set_lora_route(route))


def lora_route(x, a, b, y, M: int, K: int, N: int, rank: int) -> int:
    """The LORA_* route lora_add would take; raises when a forced route cannot."""
    r = ctypes.c_int(-1)
    check(load().ltx25_lora_route(_ptr(x), _ptr(a), _ptr(b), _ptr(y), M, K, N, rank,
                                  ctypes.byref(r)))
    return r.value


def set_tile(tile: int) -> None:
    """TILE_AUTO / TILE_TALL / TILE_MID / TILE_SKINNY for every later linear."""
    check(load().ltx25_set_tile(tile))


def linear_route(M: int, K: int, N: int, bits: int = 8) -> dict:
    """The route a linear takes (bits 4 / 8 codes, 16 dense), as a dict."""
    r = RouteC()
    check(load().ltx25_linear_route(M, K, N, bits, ctypes.byref(r)))
    return {f: getattr(r, f) for f, _ in RouteC._fields_}


def set_i8_gemm(on: bool) -> None:
    check(load().ltx25_set_i8_gemm(1 if on else 0))


def i8_takes(M: int, K: int, N: int) -> bool:
    return bool(load().ltx25_i8_takes(M, K, N))


def i8_quantize_rows(x, q, scale, M: int, K: int, stream=None) -> None:
    check(load().ltx25_i8_quantize_rows(_stream(stream), _ptr(x), _ptr(q), _ptr(scale), M, K))


def i8_quantize_qweight(w: QWeight, wq, sw, N: int, K: int, stream=None) -> None:
    cw = w.c()
    check(load().ltx25_i8_quantize_qweight(_stream(stream), ctypes.byref(cw), _ptr(wq), _ptr(sw),
                                           N, K))


def i8_gemm(xq, sx, wq, sw, bias, y, acc, M: int, K: int, N: int, stream=None) -> None:
    check(load().ltx25_i8_gemm(_stream(stream), _ptr(xq), _ptr(sx), _ptr(wq), _ptr(sw),
                               _ptr(bias), bias_dtype_of(bias), _ptr(y), _ptr(acc), M, K, N))


def qweight_infer(K: int, scales_cols: int, codes_cols: int, group: int = 0) -> tuple[int, int]:
    """(bits, group) from packed shapes; raises Ltx25Error when they do not close."""
    b = ctypes.c_int(0)
    g = ctypes.c_int(group)
    check(load().ltx25_qweight_infer(K, scales_cols, codes_cols, ctypes.byref(b), ctypes.byref(g)))
    return b.value, g.value


def _pack_stream(stream):
    """torch's current stream when a device is visible; NULL otherwise, so
    that host-side validation runs (and fails) without touching a device."""
    if stream is not None:
        return stream
    import torch

    return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None


class Pack:
    """An open .safetensors pack (ltx25_pack_*). Device tensors it binds stay
    valid until close()."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(load().ltx25_pack_open(path.encode(), ctypes.byref(h)))
        self._h = h
        self.group = 0   # the checkpoint's group, set by the first quantized bind

    def close(self) -> None:
        if self._h:
            load().ltx25_pack_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, name: str) -> tuple[str, tuple[int, ...]]:
        dt = ctypes.create_string_buffer(16)
        nd = ctypes.c_int(0)
        dims = (ctypes.c_long * 8)()
        check(load().ltx25_pack_tensor(self._h, name.encode(), dt, ctypes.byref(nd), dims))
        return dt.value.decode(), tuple(dims[i] for i in range(nd.value))

    def metadata(self, key: str):
        v = load().ltx25_pack_metadata(self._h, key.encode())
        return None if v is None else v.decode()

    def read_bf16(self, name: str, stream=None) -> tuple[int, int]:
        """(device pointer, element count) of the tensor as bf16."""
        p = ctypes.c_void_p()
        n = ctypes.c_size_t(0)
        check(load().ltx25_pack_read_bf16(self._h, _pack_stream(stream), name.encode(),
                                          ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def bind_qlinear(self, name: str, K: int, stream=None) -> QWeightC:
        """The C weight descriptor of linear `name` (quantized or dense)."""
        out = QWeightC()
        g = ctypes.c_int(self.group)
        miss = ctypes.create_string_buffer(256)
        rc = load().ltx25_pack_bind_qlinear(self._h, _pack_stream(stream), name.encode(), K,
                                            ctypes.byref(g), ctypes.byref(out), miss, 256)
        if rc != OK:
            raise Ltx25Error(rc, last_error() + (f" (missing {miss.value.decode()})"
                                                 if miss.value else ""))
        self.group = g.value
        return out


def pack_quantizable(name: str, dtype: str, ndim: int) -> bool:
    return bool(load().ltx25_pack_quantizable(name.encode(), dtype.encode(), ndim))


def linear_qc(x, cw: QWeightC, bias, y, M: int, K: int, N: int, epilogue: int = EPI_NONE,
              stream=None) -> None:
    """linear over an already-built C weight descriptor (e.g. from Pack.bind_qlinear)."""
    check(load().ltx25_linear_q_ex(_stream(stream), _ptr(x), ctypes.byref(cw), _ptr(bias),
                                   bias_dtype_of(bias), _ptr(y), M, K, N, epilogue))
