"""Build recipe for libasdsl_hip.so (gfx950 only).

Compiles every ``csrc/*.hip`` with hipcc into ``_build/`` and links the shared
library into ``lib/``.  Run ``python build_hip.py`` or call :func:`build`.
``timeline=True`` (``--timeline``) builds the timing variant
``lib/libasdsl_hip_timeline.so`` (``-DASDSL_WG_TIMELINE``, objects in
``_build_timeline/``): the same kernels, with the decode step's kernels
stamping a per-workgroup wall-clock timeline (``bench.py --decode-timeline``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
LIB = PKG_ROOT / "lib" / "libasdsl_hip.so"
BUILD_TIMELINE = PKG_ROOT / "_build_timeline"
LIB_TIMELINE = PKG_ROOT / "lib" / "libasdsl_hip_timeline.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_ROOT / 'include'}",
    f"-I{CSRC}",
]


# Per-file device code generation options.  The batched GEMVs' exact MFMA
# kernels read every MFMA result right away in fp32 steps; with the results
# in VGPRs instead of AGPRs the four v_accvgpr_read per MFMA go away (the
# 16-column prefetching instance: 3228 -> 2841 instructions).
FILE_FLAGS = {
    "gemv_preq2_batch.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
}


def _compile(src: Path, verbose: bool, build_dir: Path = BUILD, extra: tuple = ()) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, ()), *extra, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns about the device-only target feature; drop that line.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    for line in (res.stderr or "").splitlines():
        if line.strip() and noise not in line and "(ignoring feature)" not in line:
            print(line, file=sys.stderr)
    return obj


def _stale(src: Path, headers: list[Path], build_dir: Path = BUILD) -> bool:
    obj = build_dir / (src.stem + ".o")
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return src.stat().st_mtime > t or any(h.stat().st_mtime > t for h in headers)


def build(verbose: bool = False, incremental: bool = False, timeline: bool = False) -> Path:
    """Compile all HIP sources and link lib/libasdsl_hip.so (timeline=True:
    lib/libasdsl_hip_timeline.so); returns its path.  incremental=True
    recompiles only sources newer than their objects (or any header); the
    default rebuilds everything."""
    build_dir = BUILD_TIMELINE if timeline else BUILD
    lib = LIB_TIMELINE if timeline else LIB
    extra = ("-DASDSL_WG_TIMELINE",) if timeline else ()
    build_dir.mkdir(exist_ok=True)
    lib.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    headers = sorted(CSRC.glob("*.hpp")) + sorted((REPO_ROOT / "include").glob("*.h"))
    todo = [s for s in sources if not incremental or _stale(s, headers, build_dir)]
    with cf.ThreadPoolExecutor(max_workers=min(8, max(1, len(todo)))) as ex:
        list(ex.map(lambda s: _compile(s, verbose, build_dir, extra), todo))
    objs = [build_dir / (s.stem + ".o") for s in sources]
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, incremental="-i" in sys.argv, timeline="--timeline" in sys.argv))
