"""A C++ program that includes the ltx25::Ops facade (vpipe-ltx-2.5_amd/csrc/
ltx25_ops.h), links libltx25_qlinear.so, and runs Ops::init, linear,
linear_gelu and wait_ok (tests/cpp/consumer.cpp) -- the way the reference's
C++20 plugin code would bind the boundary. Built with the host compiler; run
in a fresh process. On a host without a GPU it must stop at init with the
no-device message; on the GPU its outputs are checked against the oracle."""
import os
import shutil
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vpipe-ltx-2.5_amd")
ORACLE = os.path.join(ROOT, "oracle")
SRC = os.path.join(ROOT, "tests", "cpp", "consumer.cpp")


def build(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    for lib in (os.path.join(PKG, "libltx25_qlinear.so"), os.path.join(ORACLE, "liboracle.so")):
        if not os.path.exists(lib):
            pytest.fail(f"{lib} is not built")
    exe = str(tmp_path / "consumer")
    cmd = [cxx, "-std=c++17", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(PKG, "csrc"), "-I" + ORACLE,
           SRC, "-o", exe, "-L" + PKG, "-lltx25_qlinear", "-L" + ORACLE, "-loracle",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath," + PKG, "-Wl,-rpath," + ORACLE,
           "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_consumer_links_and_stops_at_init_without_a_device(tmp_path):
    exe = build(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 3, r.stdout + r.stderr
    assert r.stdout.startswith("NODEV:")


@pytest.mark.gpu
def test_consumer_runs_the_facade_on_the_gpu(tmp_path):
    exe = build(tmp_path)
    print("[gpu] C++ consumer of ltx25::Ops", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.rstrip().endswith("OK")
