"""The C++ host side (inference-agent_amd/host/ingot_hip_attention.hpp, ingot::HipAttention)
driven as Ingot's forward_batch drives its attention step: chunked prefill then decode steps on
one layer of a 2-layer cache, each compared with the CPU oracle (max|d| <= 2e-3, rel-L2 <=
1e-3), the V cache bits, the untouched layer, and the reference's std::runtime_error behaviour
on range errors. The checks run inside tests/cpp/test_hip_attention (built by build())."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "test_hip_attention")
EXE_BACKEND = os.path.join(ROOT, "tests", "cpp", "test_hip_backend")
EXE_GGUF = os.path.join(ROOT, "tests", "cpp", "test_gguf")


def test_cpp_host_side():
    if not os.path.exists(EXE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    print("[cpp host] running tests/cpp/test_hip_attention", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout


def test_cpp_backend():
    """ingot::HipBackend (host/ingot_hip_backend.hpp): the whole Llama forward in C++ on a small
    synthetic model with F16/Q8_0/Q4_0 weights and tied embeddings, token-by-token decode and a
    40-token chunk then decode, against the CPU oracle forward; the checks and tolerances are in
    tests/cpp/test_hip_backend.cpp."""
    if not os.path.exists(EXE_BACKEND):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    print("[cpp host] running tests/cpp/test_hip_backend", flush=True)
    r = subprocess.run([EXE_BACKEND], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout


def test_cpp_gguf():
    """host/ingot_gguf.hpp: a GGUF file written by the test, mapped, parsed, resolved into the
    model, its weights uploaded once, and run by HipBackend bit-identically to the in-memory
    model; malformed files raise the reference's errors (tests/cpp/test_gguf.cpp)."""
    if not os.path.exists(EXE_GGUF):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    print("[cpp host] running tests/cpp/test_gguf", flush=True)
    r = subprocess.run([EXE_GGUF], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout
