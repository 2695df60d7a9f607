"""The engine's C++ API on the GPU: tests/cpp/test_hip.cc, built by
__graft_entry__.build() into tests/cpp/bin/test_hip, run against the kernel
pack. It drives BuildEngine / ExecutionContext as the reference's device test
does (tests/cpp/test_cuda.cpp:182-302, 395-606): stem KAT, artifact refusals,
output rebind, a caller-created stream, a spatially dynamic profile with a
graph cache of two (graph counts 1, 2, 2 and eviction), three loaded code
objects, the tuning cache and the FP16 FFN fusions."""

from __future__ import annotations

import subprocess

import pytest

from cutriton_amd import native

TESTS = ("artifact_refusals", "stem_graph_rebind_and_stream", "dynamic_spatial_profile", "tuning_cache",
         "fp16_ffn_fusions")


@pytest.fixture(scope="module")
def test_binary():
    exe = native.CPP_TEST_BIN_DIR / "test_hip"
    if not exe.exists():
        exe = native.build_cpp_gpu_test()
    return exe


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_cpp_api_on_gpu(test_binary, name):
    run = subprocess.run([str(test_binary), str(native.PACK_DIR), name], capture_output=True, text=True, timeout=100)
    assert run.returncode == 0, run.stdout + run.stderr
    assert f"ok {name}" in run.stdout, run.stdout + run.stderr
