"""Kernel Pack producer for gfx950.

Compiles every HIP source named by the registered specs into one AMDGPU code
object (an ELF, ``binary_format`` ``"hsaco"``), checks that each variant's
symbol is a kernel of that object, and writes ``pack.json`` (schema v2,
ABI v2) with the SHA-256 of every binary. The manifest fields are those the
reference producer writes (``python/cutriton/kernel_sdk/builder.py:69-120``)
plus ``target_arch``; the runtime loader verifies them again.

Usage: ``python -m cutriton_amd.kernel_sdk.builder --output <dir>``.
"""

from __future__ import annotations

import argparse
import hashlib
import importlib
import json
import os
import shutil
import struct
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Any

from .spec import KernelSpec, registered_specs

PACK_SCHEMA_VERSION = 2
ABI_SCHEMA_VERSION = 2
GENERATOR_VERSION = "cutriton-amd-0.1.0"
TARGET_ARCH = "gfx950"
DEFAULT_MODULES = ("cutriton_amd.kernel_specs.resnet", "cutriton_amd.kernel_specs.transformer")
KERNEL_SOURCE_DIR = Path(__file__).resolve().parent.parent / "kernels"

# Every HIP compile of this project: CDNA4 only, -O3, and no packed-FP32
# instructions (v_pk_*_f32 are kept out of the generated code).
HIPCC_FLAGS = (
    f"--offload-arch={TARGET_ARCH}",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def toolchain_id() -> str:
    out = subprocess.run([hipcc(), "--version"], check=True, capture_output=True, text=True).stdout
    first = next((line for line in out.splitlines() if line.startswith("HIP version")), "HIP version unknown")
    return "hipcc " + first.split(":", 1)[-1].strip()


def compile_code_object(source: Path, output: Path) -> None:
    """hipcc device-only compile of one source to an unbundled code object."""
    output.parent.mkdir(parents=True, exist_ok=True)
    cmd = [hipcc(), *HIPCC_FLAGS, "--offload-device-only", "--no-gpu-bundle-output",
           "-I", str(source.parent), str(source), "-o", str(output)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")


def elf_function_symbols(image: bytes) -> set[str]:
    """Names of the FUNC symbols of a 64-bit little-endian ELF image."""
    if image[:4] != b"\x7fELF" or image[4] != 2 or image[5] != 1:
        raise ValueError("not a 64-bit little-endian ELF code object")
    shoff, = struct.unpack_from("<Q", image, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", image, 0x3A)
    sections = [struct.unpack_from("<IIQQQQIIQQ", image, shoff + i * shentsize) for i in range(shnum)]
    names: set[str] = set()
    for _, sh_type, _, _, offset, size, link, _, _, entsize in sections:
        if sh_type not in (2, 11) or entsize == 0:  # SHT_SYMTAB, SHT_DYNSYM
            continue
        str_offset = sections[link][4]
        for i in range(size // entsize):
            st_name, st_info = struct.unpack_from("<IB", image, offset + i * entsize)
            if st_info & 0xF != 2:  # STT_FUNC
                continue
            end = image.index(b"\0", str_offset + st_name)
            names.add(image[str_offset + st_name:end].decode())
    return names


def _entries(spec: KernelSpec, binary: str, digest: str) -> list[dict[str, Any]]:
    arguments = [{"name": a.name, "type": a.type, "source": a.source} for a in spec.arguments]
    grid = list(spec.grid) + [{"kind": "literal", "value": 1}] * (3 - len(spec.grid))
    entries = [
        {
            "kernel_id": spec.kernel_id,
            "op_type": spec.op_type,
            "kernel_version": spec.version,
            "variant_id": v.variant_id,
            "default": v.default,
            "symbol": v.symbol,
            "binary": binary,
            "binary_format": "hsaco",
            "sha256": digest,
            "dtype": spec.dtype,
            "layout": spec.layout,
            "min_compute_capability": spec.min_compute_capability,
            "target_arch": spec.target_arch,
            "num_warps": v.num_warps,
            "num_stages": v.num_stages,
            "shared_memory_bytes": 0,  # every kernel declares its LDS statically
            "arguments": arguments,
            "grid": grid,
            "constraints": list(spec.constraints),
            "tuning": dict(v.meta),
        }
        for v in spec.variants
    ]
    for entry, v in zip(entries, spec.variants):
        if v.scratch_bytes:
            entry["runtime_scratch_bytes"] = v.scratch_bytes
    return entries


def build_pack(output: Path, modules: tuple[str, ...] = DEFAULT_MODULES, jobs: int = 8) -> Path:
    for module in modules:
        importlib.import_module(module)
    specs = registered_specs()
    if not specs:
        raise RuntimeError("no KernelSpec was registered")
    output = Path(output)
    staging = output.with_name(output.name + ".staging")
    if staging.exists():
        shutil.rmtree(staging)
    staging.mkdir(parents=True)
    sources = sorted({spec.source for spec in specs})
    binaries = {src: Path("kernels") / (Path(src).stem + ".hsaco") for src in sources}
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(lambda s: compile_code_object(KERNEL_SOURCE_DIR / s, staging / binaries[s]), sources))
    digests: dict[str, str] = {}
    for src in sources:
        image = (staging / binaries[src]).read_bytes()
        digests[src] = hashlib.sha256(image).hexdigest()
        symbols = elf_function_symbols(image)
        for spec in specs:
            if spec.source != src:
                continue
            missing = [v.symbol for v in spec.variants if v.symbol not in symbols]
            if missing:
                raise RuntimeError(f"{spec.kernel_id}: symbols missing from {src}: {missing}")
    kernels: list[dict[str, Any]] = []
    for spec in sorted(specs, key=lambda s: s.kernel_id):
        kernels.extend(_entries(spec, binaries[spec.source].as_posix(), digests[spec.source]))
    pack = {
        "schema_version": PACK_SCHEMA_VERSION,
        "abi_schema_version": ABI_SCHEMA_VERSION,
        "pack_name": "cutriton_gfx950",
        "pack_version": 1,
        "generator_version": GENERATOR_VERSION,
        "triton_version": toolchain_id(),
        "kernels": kernels,
    }
    (staging / "pack.json").write_text(json.dumps(pack, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    if output.exists():
        shutil.rmtree(output)
    staging.rename(output)
    return output / "pack.json"


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--output", type=Path, required=True)
    parser.add_argument("--module", action="append", dest="modules")
    parser.add_argument("--jobs", type=int, default=8)
    args = parser.parse_args()
    print(build_pack(args.output, tuple(args.modules or DEFAULT_MODULES), args.jobs))


if __name__ == "__main__":
    main()
