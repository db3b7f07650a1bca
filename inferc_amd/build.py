"""Builds the gfx950 backend library ``inferc_amd/libinferc_hip.so`` in-tree.

Every ``csrc/*.hip`` translation unit is compiled by ``hipcc`` for gfx950
only, then linked into one shared library that exports the C-ABI declared in
``include/inferc_hip.h``. Packed-fp32 VALU instructions are disabled
(``-target-feature -packed-fp32-ops``) for all device code.

Usage: ``python -m inferc_amd.build [--jobs N] [--sanitize]``.

``--sanitize`` builds ``libinferc_hip_san.so`` instead (objects under
``_build_san/``): the host code compiled with AddressSanitizer and
UndefinedBehaviorSanitizer (each ``-fsanitize=`` applies to the host pass
only, through ``-Xarch_host``; device code is unchanged). It is for the CPU
tests (``tests/run_sanitized.sh``), which load it through ``INFERC_HIP_LIB``
with the clang ASan runtime preloaded.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libinferc_hip.so"
BUILD_SAN = PKG / "_build_san"
LIB_SAN = PKG / "libinferc_hip_san.so"
# host-pass-only sanitizer flags (compile and link)
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
             "-Xarch_host", "-g"]
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXXFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar kernel arguments arrive in SGPRs at wave launch, so a
    # kernel's first loads need no scalar load of its argument block
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
]


# Sources compiled more than once, each time with other defines (object
# suffix, flags): gemm_tile.hip holds the LDS-tiled GEMM's launcher for one
# tile form and A orientation per compile, so the forms build in parallel.
VARIANTS = {
    "gemm_tile": [(f"_f{f}_t{t}", (f"-DIH_TILE_FORM={f}", f"-DIH_TILE_TA={t}"))
                  for f in range(4) for t in range(2)],
}


def _jobs(sources: list[Path]) -> list[tuple[Path, str, tuple]]:
    """(source, object suffix, extra flags) for every compile."""
    out = []
    for src in sources:
        for suffix, flags in VARIANTS.get(src.stem, [("", ())]):
            out.append((src, suffix, flags))
    return out


def _compile(src: Path, out_dir: Path = BUILD, extra: tuple = (), suffix: str = "") -> Path:
    obj = out_dir / (src.stem + suffix + ".o")
    cmd = [HIPCC, *CXXFLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, sanitize: bool = False) -> Path:
    """Compiles all HIP sources and links the library; returns its path."""
    out_dir, lib = (BUILD_SAN, LIB_SAN) if sanitize else (BUILD, LIB)
    extra = tuple(SAN_FLAGS) if sanitize else ()
    out_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    work = _jobs(sources)
    # the slowest compiles first, so they do not start last
    work.sort(key=lambda w: w[0].stem != "gemm_tile")
    jobs = jobs or min(len(work), os.cpu_count() or 4, 8)
    for stale in out_dir.glob("*.o"):
        stale.unlink()
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda w: _compile(w[0], out_dir, extra + w[2], w[1]), work))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *extra, *map(str, objs), "-o",
           str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} from {len(sources)} sources")
    return lib


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--sanitize", action="store_true",
                    help="host ASan + UBSan build (libinferc_hip_san.so) for the CPU tests")
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True, sanitize=args.sanitize)
    return 0


if __name__ == "__main__":
    sys.exit(main())
