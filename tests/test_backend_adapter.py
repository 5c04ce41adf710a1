"""The MI355X backend binds to Ingot's real Backend interface at compile time:
tests/cpp/backend_adapter.cpp (`HipBackendAdapter : public Backend`, forwarding to
ingot::HipBackend, and the "hip" factory case with make_backend's shape) is compiled with
-fsyntax-only against the reference's own headers (src/backend.h:9-23, src/engine.h,
src/model.h). Skipped where the reference sources are absent (the GPU box)."""
from __future__ import annotations

import os
import subprocess

import pytest

from conftest import PKG, ROOT

REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "backend.h")),
                    reason="reference sources not present on this machine")
def test_hip_backend_adapter_compiles_against_reference_backend():
    src = os.path.join(ROOT, "tests", "cpp", "backend_adapter.cpp")
    cmd = ["/opt/rocm/bin/hipcc", "-fsyntax-only", "-std=c++20", "-Wall", "-Werror", "-Wno-unused-command-line-argument", "-x", "hip",
           "--offload-arch=gfx950", "--cuda-host-only", "-I", REF_SRC, "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(PKG, "host"), src]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
