"""Build and load the native pieces: the C++ engine library and the Kernel Pack.

``build_all()`` compiles ``csrc/**/*.cc`` (host C++17 against the HIP runtime)
into ``libcutriton_gfx950.so`` beside this file, with the engine's own
re-layout kernels (``csrc/runtime/relayout.hip``, gfx950) embedded as a code
object, and runs the pack producer into ``pack/``. ``library()`` loads the
engine library and raises when it is missing: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY_PATH = PACKAGE_DIR / "libcutriton_gfx950.so"
PACK_DIR = PACKAGE_DIR / "pack"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

CXXFLAGS = (
    "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra",
    "-D__HIP_PLATFORM_AMD__",
    f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", f"-I{ROCM / 'include'}",
)


def _compile(source: Path) -> Path:
    obj = BUILD_DIR / (source.relative_to(CSRC_DIR).as_posix().replace("/", "_") + ".o")
    cmd = ["g++", *CXXFLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"g++ failed for {source}:\n{result.stderr}")
    return obj


# HIP sources compiled for host and gfx950 into the library itself (their
# device symbols are registered with the HIP runtime when it loads).
LIBRARY_HIP_SOURCES = ("runtime/static_scratch.hip",)


def _compile_library_hip(relative: str) -> Path:
    from .kernel_sdk.builder import HIPCC_FLAGS, hipcc

    source = CSRC_DIR / relative
    obj = BUILD_DIR / (relative.replace("/", "_") + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", "-fPIC", f"-I{INCLUDE_DIR}", f"-I{CSRC_DIR}", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source}:\n{result.stderr}")
    return obj


def _embedded_relayout_code() -> Path:
    """Compiles ``relayout.hip`` to a gfx950 code object and compiles that
    object into the library as ``cutriton::kRelayoutCodeObject``."""
    from .kernel_sdk.builder import compile_code_object

    hsaco = BUILD_DIR / "relayout.hsaco"
    compile_code_object(CSRC_DIR / "runtime" / "relayout.hip", hsaco)
    data = hsaco.read_bytes()
    rows = [", ".join(str(b) for b in data[i:i + 32]) for i in range(0, len(data), 32)]
    source = BUILD_DIR / "relayout_code.cc"
    source.write_text(
        "// Generated from csrc/runtime/relayout.hip by cutriton_amd/native.py.\n"
        "#include <cstddef>\n\nnamespace cutriton {\n"
        "extern const unsigned char kRelayoutCodeObject[];\n"
        "extern const std::size_t kRelayoutCodeObjectBytes;\n"
        "alignas(64) const unsigned char kRelayoutCodeObject[] = {\n" + ",\n".join(rows) + "};\n"
        "const std::size_t kRelayoutCodeObjectBytes = sizeof(kRelayoutCodeObject);\n"
        "}  // namespace cutriton\n")
    obj = BUILD_DIR / "relayout_code.o"
    result = subprocess.run(["g++", *CXXFLAGS, "-c", str(source), "-o", str(obj)], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"g++ failed for {source}:\n{result.stderr}")
    return obj


def build_engine_library(jobs: int = 8) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC_DIR.rglob("*.cc"))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        embedded = pool.submit(_embedded_relayout_code)
        device_objects = [pool.submit(_compile_library_hip, relative) for relative in LIBRARY_HIP_SOURCES]
        objects = list(pool.map(_compile, sources)) + [embedded.result()] + [f.result() for f in device_objects]
    staging = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = ["g++", "-shared", "-o", str(staging), *map(str, objects),
           f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(staging, LIBRARY_PATH)
    return LIBRARY_PATH


def build_kernel_pack(jobs: int = 8) -> Path:
    cmd = ["python3", "-m", "cutriton_amd.kernel_sdk.builder", "--output", str(PACK_DIR), "--jobs", str(jobs)]
    result = subprocess.run(cmd, cwd=REPO_DIR, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"kernel pack build failed:\n{result.stdout}\n{result.stderr}")
    return PACK_DIR / "pack.json"


CPP_TEST_DIR = REPO_DIR / "tests" / "cpp"
CPP_TEST_BIN_DIR = CPP_TEST_DIR / "bin"


def build_cpp_gpu_test() -> Path:
    """Compiles tests/cpp/test_hip.cc (the C++ API on the GPU) against the
    engine library into tests/cpp/bin/test_hip. The binary finds the library
    through a run path relative to itself, so it runs from any copy of the
    tree."""
    CPP_TEST_BIN_DIR.mkdir(parents=True, exist_ok=True)
    exe = CPP_TEST_BIN_DIR / "test_hip"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE_DIR}", f"-I{ROCM / 'include'}",
           str(CPP_TEST_DIR / "test_hip.cc"), f"-L{PACKAGE_DIR}", "-lcutriton_gfx950", f"-L{ROCM / 'lib'}",
           "-lamdhip64", "-Wl,-rpath,$ORIGIN/../../../cutriton_amd", f"-Wl,-rpath,{ROCM / 'lib'}",
           "-o", str(exe)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"g++ failed for test_hip.cc:\n{result.stderr}")
    return exe


def build_all(jobs: int = 8) -> None:
    build_engine_library(jobs)
    build_kernel_pack(jobs)
    build_cpp_gpu_test()


_LIBRARY: ctypes.CDLL | None = None


def library() -> ctypes.CDLL:
    """The loaded engine library; raises if it was never built."""
    global _LIBRARY
    if _LIBRARY is None:
        if not LIBRARY_PATH.exists():
            raise RuntimeError(f"{LIBRARY_PATH} is missing: run __graft_entry__.build() first")
        if not (PACK_DIR / "pack.json").exists():
            raise RuntimeError(f"{PACK_DIR / 'pack.json'} is missing: run __graft_entry__.build() first")
        # torch ships its own libamdhip64 under the soname this library needs
        # (libamdhip64.so.7). One process must hold one HIP runtime: load
        # torch's first when torch is installed, so that both bind to it.
        # Loaded the other way round, torch's device initialisation fails.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        _LIBRARY = ctypes.CDLL(str(LIBRARY_PATH))
    return _LIBRARY
