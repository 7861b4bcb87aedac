"""Build the gfx950 HIP backend library in-tree.

Compiles every source under runtime_amd/csrc with hipcc for gfx950 into
runtime_amd/_build/*.o (in parallel) and links runtime_amd/libminifield_hip.so;
then builds the measurement probes (csrc/probe) as
runtime_amd/libminifield_probe.so.
Run as `python -m runtime_amd.build` or through __graft_entry__.build().
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PACKAGE = pathlib.Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libminifield_hip.so"
# The measurement probes (streaming-read ceiling, shader clock, LDS and MFMA
# unit rates): a library of their own, not the backend.
PROBE_SRCS = [CSRC / "probe" / "read_ceiling.hip", CSRC / "probe" / "unit_rates.hip"]
PROBE_LIBRARY = PACKAGE / "libminifield_probe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation (wrong results seen
# on this hardware class); hipcc's host pass warns that it does not know the
# feature, which is harmless.
COMMON = [
    "-x", "hip",
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[pathlib.Path]:
    return sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))


def _compile(src: pathlib.Path) -> tuple[pathlib.Path, str]:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *COMMON, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    noise = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line and line.strip()
    )
    return obj, noise


def build(jobs: int | None = None, verbose: bool = False) -> pathlib.Path:
    """Compile and link the library; always rebuilds every object."""
    if not pathlib.Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the HIP backend cannot be built")
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(_compile, srcs))
    for obj, noise in results:
        if noise and verbose:
            print(f"[{obj.name}] {noise}", file=sys.stderr)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
           *[str(obj) for obj, _ in results], "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    tmp = PROBE_LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, *COMMON, "-shared", "-o", str(tmp), *[str(p) for p in PROBE_SRCS]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for the probe library:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, PROBE_LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
