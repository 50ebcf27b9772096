"""The C ABI on the host: the library loads, exports every entry point the
header declares, and its host-only logic (argument validation, the int8
tier's shape gates, packed-shape inference) behaves as specified without
touching a device."""
import os
import re
import shutil
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_entry_points():
    names = set()
    for f in os.listdir(INCLUDE):
        if f.endswith(".h"):
            text = open(os.path.join(INCLUDE, f)).read()
            names |= set(re.findall(r"^\s*(?:int|const char\*|void|size_t)\s+(ltx25_\w+)\s*\(", text,
                                    re.M))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_entry_points()
    for must in ["ltx25_init", "ltx25_linear_q", "ltx25_linear", "ltx25_bias_add",
                 "ltx25_set_i8_gemm", "ltx25_i8_takes", "ltx25_i8_gemm",
                 "ltx25_quant_available", "ltx25_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_entry_points():
        assert hasattr(lib, name), f"{name} is declared but not exported"


def test_binding_covers_every_declared_symbol(pkg):
    assert set(declared_entry_points()) == set(pkg.SIGNATURES)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_init_without_a_device_reports_nodev(pkg, lib):
    assert lib.ltx25_init() == pkg.E_NODEV
    assert pkg.last_error()
    assert lib.ltx25_quant_available() == 0


def test_validation_precedes_any_device_use(pkg, lib):
    fake = 0x1000  # never dereferenced: every call below fails validation first
    q = pkg.QWeightC(None, fake, fake, fake, 8, 64, 1)
    import ctypes

    def call(M, K, N, w=q, bias=None, dt=pkg.DT_NONE, epi=0):
        return lib.ltx25_linear_q_ex(None, fake, ctypes.byref(w), bias, dt, fake, M, K, N, epi)

    assert call(16, 100, 128) == pkg.E_INVAL                  # K not a multiple of group
    assert "group" in pkg.last_error()
    assert call(0, 256, 128) == pkg.E_INVAL
    assert call(16, 256, 128, bias=fake, dt=pkg.DT_NONE) == pkg.E_INVAL
    assert call(16, 256, 128, epi=7) == pkg.E_INVAL
    bad_bits = pkg.QWeightC(None, fake, fake, fake, 5, 64, 1)
    assert call(16, 256, 128, w=bad_bits) == pkg.E_INVAL
    bad_group = pkg.QWeightC(None, fake, fake, fake, 8, 48, 1)
    assert call(16, 192, 128, w=bad_group) == pkg.E_INVAL
    no_codes = pkg.QWeightC(None, None, fake, fake, 8, 64, 1)
    assert call(16, 256, 128, w=no_codes) == pkg.E_INVAL
    # dense K=81 (the reference's VAE conv_in) is well-formed but no kernel takes it
    assert lib.ltx25_linear(None, fake, fake, None, 0, fake, 4096, 81, 128) == pkg.E_UNSUPPORTED
    assert lib.ltx25_i8_gemm(None, fake, fake, fake, fake, None, 0, fake, None, 64, 100,
                             64) == pkg.E_UNSUPPORTED
    assert lib.ltx25_pack_codes(None, fake, fake, 4, 6, 8) == pkg.E_INVAL  # 6 codes != words
    assert lib.ltx25_gate_heads(None, None, fake, 2, 2, 8) == pkg.E_INVAL      # null y
    assert lib.ltx25_gate_heads(None, fake + 1, fake, 2, 2, 8) == pkg.E_INVAL  # odd address
    assert lib.ltx25_gate_heads(None, None, None, 0, 2, 8) == pkg.OK           # empty: no-op


def test_dequant_once_and_lora_gates(pkg, lib):
    # AUTO by default: the arm for tall GEMMs only
    assert pkg.dequant_once_takes(8160, 4096, 16384)
    assert pkg.dequant_once_takes(4096, 2048, 8192)
    assert pkg.dequant_once_takes(1024, 4096, 4096)
    assert not pkg.dequant_once_takes(1023, 4096, 4096)
    assert not pkg.dequant_once_takes(126, 2048, 6144)
    try:
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_OFF)
        assert not pkg.dequant_once_takes(8160, 4096, 16384)
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_ON)
        assert pkg.dequant_once_takes(320, 4096, 4096)
        assert not pkg.dequant_once_takes(63, 4096, 4096)     # mma_eligible_'s M floor
        assert not pkg.dequant_once_takes(64, 4096, 15)       # and its N floor
        assert not pkg.dequant_once_takes(64, 100, 64)        # K the tile cannot step
        assert lib.ltx25_set_dequant_once(7) == pkg.E_INVAL
    finally:
        pkg.set_dequant_once(pkg.DEQUANT_ONCE_AUTO)
    # the GEMM pair from rank 96 and 256 tokens (the reference's matrix-core pair)
    assert pkg.lora_on_matrix_cores(8160, 4096, 16384, 450)
    assert pkg.lora_on_matrix_cores(256, 1024, 1024, 96)
    assert not pkg.lora_on_matrix_cores(8160, 4096, 16384, 32)   # one-pass kernel
    assert not pkg.lora_on_matrix_cores(255, 1024, 1024, 450)
    assert not pkg.lora_on_matrix_cores(0, 64, 64, 3)
    assert not pkg.lora_on_matrix_cores(12, 64, 64, 0)
    try:
        pkg.set_lora_matrix_cores(False)
        assert not pkg.lora_on_matrix_cores(8160, 4096, 16384, 450)
    finally:
        pkg.set_lora_matrix_cores(True)
    assert pkg.lora_on_matrix_cores(8160, 4096, 16384, 450)


def test_lora_validation_precedes_any_device_use(pkg, lib):
    fake = 0x1000
    # empty shapes are the reference's no-op (src/ltx25-metal-ops.cc:996): OK, no device use
    assert lib.ltx25_lora_add(None, fake, fake, fake, fake, None, None, 0, 64, 64, 3) == pkg.OK
    assert lib.ltx25_lora_add(None, fake, fake, fake, fake, None, None, 12, 64, 64, -1) == pkg.OK
    assert lib.ltx25_lora_add(None, None, fake, fake, fake, None, None, 12, 64, 64, 3) == pkg.E_INVAL
    assert lib.ltx25_lora_add(None, fake + 1, fake, fake, fake, None, None, 12, 64, 64,
                              3) == pkg.E_INVAL


def test_i8_takes_gates(pkg):
    pkg.set_i8_gemm(False)
    assert not pkg.i8_takes(8160, 4096, 4096)
    pkg.set_i8_gemm(True)
    try:
        # the DiT's projections at a clip's token count (tests/ltx25-i8-gemm-test.cc:155-161)
        assert pkg.i8_takes(8160, 4096, 4096)
        assert pkg.i8_takes(8160, 4096, 16384)
        assert pkg.i8_takes(8160, 16384, 4096)
        assert pkg.i8_takes(8160, 3840, 4096)
        # refused: short M, shallow K (tests/ltx25-i8-gemm-test.cc:164-165)
        assert not pkg.i8_takes(512, 4096, 4096)
        assert not pkg.i8_takes(8160, 512, 4096)
        assert not pkg.i8_takes(8160, 1000, 4096)       # K not a multiple of 128
        assert not pkg.i8_takes(8160, 4096, 8)          # narrow N
    finally:
        pkg.set_i8_gemm(False)


def test_qweight_infer_recovers_bits_and_group(pkg):
    # K = 4096: w8g64 packs 1024 u32 words and 64 scale columns per row
    assert pkg.qweight_infer(4096, 64, 1024) == (8, 64)
    assert pkg.qweight_infer(4096, 128, 512) == (4, 32)
    assert pkg.qweight_infer(4096, 64, 512) == (4, 64)
    assert pkg.qweight_infer(2048, 64, 512, group=32) == (8, 32)
    with pytest.raises(pkg.Ltx25Error):
        pkg.qweight_infer(4096, 64, 1000)                # codes do not close
    with pytest.raises(pkg.Ltx25Error):
        pkg.qweight_infer(4096, 100, 1024)               # group not 32/64
    with pytest.raises(pkg.Ltx25Error):
        pkg.qweight_infer(4096, 128, 1024, group=64)     # second group size in one pack


def test_cpp_facade_compiles():
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    src = "#include \"ltx25_ops.h\"\nint main(){ ltx25::Ops o; ltx25::QWeight w; return w.empty() ? 0 : 1; }\n"
    r = subprocess.run([cxx, "-std=c++17", "-fsyntax-only", "-x", "c++", "-",
                        "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + INCLUDE,
                        "-I" + os.path.join(ROOT, "vpipe-ltx-2.5_amd", "csrc")],
                       input=src, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]


class _Fake:
    """Stands in for a tensor in the host-only route queries: only the
    address is read (for alignment), never dereferenced."""

    def __init__(self, addr):
        self.addr = addr

    def data_ptr(self):
        return self.addr


def test_lora_route_query_and_forcing(pkg):
    al, odd = _Fake(0x10000), _Fake(0x10002)
    r = lambda M, K, N, rank, x=al, a=al, b=al, y=al: pkg.lora_route(x, a, b, y, M, K, N, rank)  # noqa: E731
    assert r(8160, 4096, 16384, 450) == pkg.LORA_PAIR
    assert r(8160, 4096, 16384, 32) == pkg.LORA_RFIRST
    assert r(511, 4096, 16384, 32) == pkg.LORA_FUSED             # too few tokens for r-first
    assert r(8160, 4096, 16384, 36) == pkg.LORA_FUSED            # rank not a multiple of 8
    assert r(8160, 4096, 16384, 32, x=odd) == pkg.LORA_FUSED     # scalar path
    assert r(8160, 4096, 16384, 450, y=odd) == pkg.LORA_FUSED    # pair needs aligned x, y
    assert r(0, 4096, 16384, 32) == pkg.LORA_NONE
    try:
        pkg.set_lora_route(pkg.LORA_FUSED)
        assert r(8160, 4096, 16384, 450) == pkg.LORA_FUSED
        pkg.set_lora_route(pkg.LORA_PAIR)
        assert r(64, 4096, 1024, 16) == pkg.LORA_PAIR
        with pytest.raises(pkg.Ltx25Error) as e:
            r(64, 100, 1024, 16)                                  # K % 64 != 0
        assert e.value.code == pkg.E_UNSUPPORTED
        pkg.set_lora_route(pkg.LORA_RFIRST)
        assert r(64, 4096, 1024, 16) == pkg.LORA_RFIRST
        with pytest.raises(pkg.Ltx25Error):
            r(64, 4096, 1024, 12)                                 # rank % 8 != 0
        import ctypes
        lib = pkg.load()
        # a forced route that cannot take the shape fails before any device use
        assert lib.ltx25_lora_add(None, 0x10000, 0x10000, 0x10000, 0x10000, None, None, 64, 4096,
                                  1024, 12) == pkg.E_UNSUPPORTED
        assert lib.ltx25_set_lora_route(9) == pkg.E_INVAL
        del ctypes
    finally:
        pkg.set_lora_route(pkg.LORA_AUTO)


def test_linear_route_and_tile_switch(pkg, lib):
    r = pkg.linear_route
    # the video GEMMs fill 256 CUs with 256 x 256 tiles; the audio ones take the M <= 128 kernel
    assert r(8160, 4096, 16384)["tile"] == pkg.TILE_TALL
    assert r(8160, 4096, 16384)["dequant_once"] == 1
    assert r(126, 2048, 6144)["tile"] == pkg.TILE_SKINNY
    assert r(126, 8192, 2048)["splits"] > 1
    assert r(320, 4096, 4096)["tile"] == pkg.TILE_MID
    assert r(1024, 4096, 8192, bits=16)["dequant_once"] == 0
    try:
        pkg.set_tile(pkg.TILE_MID)
        assert r(8160, 4096, 16384)["tile"] == pkg.TILE_MID
        pkg.set_tile(pkg.TILE_TALL)
        assert r(126, 2048, 6144)["tile"] == pkg.TILE_TALL
        assert r(126, 2048, 6144)["splits"] == 1
        pkg.set_tile(pkg.TILE_SKINNY)
        assert r(126, 2048, 6144)["tile"] == pkg.TILE_SKINNY
        assert r(8160, 4096, 4096)["tile"] == pkg.TILE_TALL       # SKINNY cannot take M > 128
        assert lib.ltx25_set_tile(7) == pkg.E_INVAL
    finally:
        pkg.set_tile(pkg.TILE_AUTO)


def test_operand_limit_slabs_and_refusal(pkg, lib):
    """Every operand of a launch stays under 2 GiB (32-bit buffer offsets,
    the reference's own limit, src/ltx25-metal-ops.cc:342-374): X and Y
    are cut into row slabs; a weight at the limit is refused before any
    device use."""
    import ctypes

    r = pkg.linear_route
    assert r(8160, 4096, 16384)["slabs"] == 1
    big = r(300000, 4096, 4096, bits=16)        # X is 2.46 GB
    assert big["slabs"] == 2
    assert big["slab_rows"] % 256 == 0
    assert big["slab_rows"] * 4096 * 2 < 2 ** 31
    assert big["slab_rows"] * 2 >= 300000
    # the bf16 expansion of a 2^31-byte weight would not fit: the fused kernel instead
    assert r(8160, 65536, 16384)["dequant_once"] == 0            # w8 codes 1 GiB, bf16 2 GiB
    with pytest.raises(pkg.Ltx25Error) as e:
        r(8160, 32768, 65536)                                    # w8 codes exactly 2 GiB
    assert e.value.code == pkg.E_UNSUPPORTED and "2 GiB" in str(e.value)
    fake = 0x10000
    q = pkg.QWeightC(None, fake, fake, fake, 8, 64, 1)
    assert lib.ltx25_linear_q_ex(None, fake, ctypes.byref(q), None, 0, fake, 8160, 32768, 65536,
                                 0) == pkg.E_UNSUPPORTED
    assert "2 GiB" in pkg.last_error()
    dense = lib.ltx25_linear(None, fake, fake, None, 0, fake, 64, 32768, 32768)   # bf16 W 2 GiB
    assert dense == pkg.E_UNSUPPORTED
    # the int8 tier declines operands it cannot address
    pkg.set_i8_gemm(True)
    try:
        assert pkg.i8_takes(8160, 4096, 16384)
        assert not pkg.i8_takes(600000, 4096, 4096)              # int8 X 2.46 GB
        assert r(8160, 4096, 16384)["i8"] == 1
    finally:
        pkg.set_i8_gemm(False)


def test_noalloc_refuses_the_int8_tier_before_device_use(pkg, lib):
    """The no-allocation linear cannot quantize into library scratch: with
    the tier on and taking the shape it fails before any HIP call."""
    import ctypes

    fake = 0x10000
    q = pkg.QWeightC(None, fake, fake, fake, 8, 64, 1)
    pkg.set_i8_gemm(True)
    try:
        assert pkg.i8_takes(1024, 2048, 2048)
        rc = lib.ltx25_linear_q_noalloc(None, fake, ctypes.byref(q), None, 0, fake, 1024, 2048,
                                        2048, 0)
        assert rc == pkg.E_UNSUPPORTED
        assert "int8" in pkg.last_error()
    finally:
        pkg.set_i8_gemm(False)
    # malformed calls fail validation exactly as linear_q_ex does
    assert lib.ltx25_linear_q_noalloc(None, fake, ctypes.byref(q), None, 0, fake, 16, 100, 128,
                                      0) == pkg.E_INVAL


def test_every_planned_split_fits_the_noalloc_scratch(pkg):
    """Split-K partials of every plan the planner makes for a 256-CU device
    fit the no-allocation linear's 32 MiB: the M <= 128 kernel keeps
    (N / 32) x splits within 3 workgroups per CU, and the 128 x 128 tile
    splits only until its workgroups cover the CUs once."""
    cap = pkg.noalloc_scratch_bytes()
    worst = 0
    for M in [1, 16, 64, 126, 128, 129, 192, 255, 256, 300, 384, 512, 640, 1000, 1024, 2040,
              4080]:
        for N in [64, 260, 1000, 2048, 4096, 6144, 8192, 16384, 32640]:
            for K in [64, 512, 2048, 4096, 8192, 16384, 65536]:
                if N * K * 2 >= 2 ** 31:
                    continue        # a weight the linear refuses
                r = pkg.linear_route(M, K, N, bits=16)
                worst = max(worst, r["scratch_bytes"])
                assert r["scratch_bytes"] <= cap, (M, K, N, r)
    assert worst > cap // 4        # the scan reaches plans near the cap


_ENV_PROBE = r"""
import ctypes, importlib.util, json, os, sys
spec = importlib.util.spec_from_file_location("vpipe_ltx25_amd", sys.argv[1])
pkg = importlib.util.module_from_spec(spec)
sys.modules["vpipe_ltx25_amd"] = pkg
spec.loader.exec_module(pkg)
lib = pkg.load()
before = pkg.linear_route(8160, 4096, 16384)
rc = lib.ltx25_init()
print(json.dumps({
    "init_rc": rc,
    "before": before,
    "big": pkg.linear_route(8160, 4096, 16384),
    "mid_m": pkg.dequant_once_takes(1000, 4096, 4096),
    "i8": pkg.i8_takes(8160, 4096, 4096),
    "lora": pkg.lora_on_matrix_cores(8160, 4096, 16384, 450),
}))
"""


def _env_probe(env_extra):
    env = {k: v for k, v in os.environ.items() if not k.startswith(("VPIPE_LTX25_", "VPIPE_I8"))}
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", _ENV_PROBE,
                          os.path.join(ROOT, "vpipe-ltx-2.5_amd", "__init__.py")],
                         env=env, capture_output=True, text=True, timeout=120, check=True)
    import json

    return json.loads(out.stdout.strip().splitlines()[-1])


def test_init_reads_the_reference_route_knobs():
    """ltx25_init maps the reference's init-time A/B knobs
    (src/ltx25-metal-ops.cc:186-231) and VPIPE_I8_GEMM onto the switches,
    before the device check, so the routes change on any host."""
    base = _env_probe({})
    assert base["big"]["tile"] == 1 and base["big"]["dequant_once"] == 1
    assert base["before"] == base["big"]
    assert not base["mid_m"] and not base["i8"] and base["lora"]

    r = _env_probe({"VPIPE_LTX25_NO_DEQUANT_MMA": "1"})
    assert r["before"]["dequant_once"] == 1 and r["big"]["dequant_once"] == 0

    r = _env_probe({"VPIPE_LTX25_MMA_TILE": "128"})
    assert r["big"]["tile"] == 2
    r = _env_probe({"VPIPE_LTX25_MMA_TILE": "512"})
    assert r["big"]["tile"] == 1
    r = _env_probe({"VPIPE_LTX25_MMA_TILE": "300"})     # not a reference tile: ignored
    assert r["big"] == base["big"]

    r = _env_probe({"VPIPE_LTX25_MMA_MIN_M": "900"})
    assert r["mid_m"]
    r = _env_probe({"VPIPE_LTX25_MMA_MIN_M": "-3"})
    assert not r["mid_m"]

    r = _env_probe({"VPIPE_I8_GEMM": "1"})
    assert r["i8"] and r["big"]["i8"] == 1
    r = _env_probe({"VPIPE_I8_GEMM": "1", "VPIPE_LTX25_NO_MMA": "1"})
    assert not r["i8"] and r["big"]["dequant_once"] == 0 and r["big"]["i8"] == 0

    r = _env_probe({"VPIPE_LTX25_NO_LORA_MMA": "1"})
    assert not r["lora"]


def test_fold_predicate_at_a_rank_wider_than_one_block(pkg):
    """The fold's expansion writes the [W | B] tail in a loop over its
    columns, so the predicate holds at any rank (2100 -> 2112 tail columns,
    wider than one 256-thread block's 2048)."""
    assert pkg.lora_fold_takes(1024, 256, 256, 2100, 8)
    assert pkg.lora_fold_takes(8160, 4096, 16384, 2100, 8)
    assert not pkg.lora_fold_takes(1023, 256, 256, 2100, 8)    # below the dequant-once arm


def test_linear_q_lora_checks_epilogue_and_bias_first(pkg, lib):
    """A bad epilogue or bias dtype is refused before either path touches
    the device (the non-fold path would otherwise write y first)."""
    import ctypes

    fake = 0x1000
    q = pkg.QWeightC(None, fake, fake, fake, 8, 64, 1)
    for M in (64, 8160):     # the sequence, and the fold
        assert lib.ltx25_linear_q_lora(None, fake, ctypes.byref(q), None, pkg.DT_NONE, fake, fake,
                                       32, fake, M, 4096, 4096, 7) == pkg.E_INVAL
        assert "epilogue" in pkg.last_error()
        assert lib.ltx25_linear_q_lora(None, fake, ctypes.byref(q), fake, 9, fake, fake,
                                       32, fake, M, 4096, 4096, 0) == pkg.E_INVAL
        assert "bias" in pkg.last_error()
