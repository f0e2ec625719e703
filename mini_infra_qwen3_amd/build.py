"""Builds libmi_paged.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950, and
libmi_calib.so (HBM streaming-copy calibration kernels that bench.py reads the data-plane rates
against; not part of the ABI).

Usage: ``python -m mini_infra_qwen3_amd.build`` (also called by ``__graft_entry__.build()``).
Every source is compiled on each call; objects go to ``_build/`` and the libraries next to
this file, where ``mini_infra_qwen3_amd._native`` (and bench.py) load them from.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
CALIB_DIR = PACKAGE_DIR / "csrc_calib"
CALIB_LIBRARY_PATH = PACKAGE_DIR / "libmi_calib.so"
REPO_DIR = PACKAGE_DIR.parent
BUILD_DIR = REPO_DIR / "_build" / "mi_paged"
LIBRARY_PATH = PACKAGE_DIR / "libmi_paged.so"
ARCH = "gfx950"

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
]

# Per-source flags.  exact_attention.hip: the fp64 MFMA accumulators of its prefill kernel in
# ordinary VGPRs (the compiler's default puts them in AGPRs, which at 256 threads per workgroup
# pushes the kernel to one wavefront per SIMD; in VGPRs the cached form fits four).
SOURCE_FLAGS = {
    "exact_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources(directory: Path = CSRC_DIR) -> list[Path]:
    return sorted(directory.glob("*.hip"))


def _compile(src: Path, build_dir: Path, extra: tuple[str, ...]) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, ()), *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True, extra_flags: tuple[str, ...] = (), output: Path | None = None,
          calibration: bool = True) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links libmi_paged.so; returns its path.

    ``extra_flags`` (e.g. ``-DMI_DECODE_PART_BLOCKS=32`` to override a kernel tunable) and
    ``output`` build a variant library elsewhere; the defaults build the in-tree library, and
    then (``calibration``) libmi_calib.so from csrc_calib/.
    """
    if output is None and calibration:
        _link(sources(CALIB_DIR), CALIB_LIBRARY_PATH, BUILD_DIR.with_name("mi_calib"), (), verbose)
    output = LIBRARY_PATH if output is None else Path(output)
    build_dir = BUILD_DIR if output == LIBRARY_PATH else output.parent / "_obj"
    return _link(sources(), output, build_dir, tuple(extra_flags), verbose)


def _link(srcs: list[Path], output: Path, build_dir: Path, extra: tuple[str, ...], verbose: bool) -> Path:
    build_dir.mkdir(parents=True, exist_ok=True)
    if not srcs:
        raise RuntimeError(f"no HIP sources for {output.name}")
    workers = min(len(srcs), 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(lambda src: _compile(src, build_dir, extra), srcs))
    tmp = output.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {output.name} failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, output)
    if verbose:
        print(f"built {output} from {len(srcs)} sources", flush=True)
    return output


if __name__ == "__main__":
    build()
    sys.exit(0)
