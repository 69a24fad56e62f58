"""Build the C-ABI shared library ``_lib/libdrama3_moe.so`` for gfx950.

Each ``csrc/*.hip`` / ``*.cpp`` file is compiled to an object with hipcc in
parallel, then linked into one shared library in-tree (it travels with the
repository snapshot; nothing is installed).  ``python -m drama3_amd._build``
or ``__graft_entry__.build()`` runs it.
"""

from __future__ import annotations

import concurrent.futures
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
INCLUDE = PACKAGE.parent.parent / "include"
OUT_DIR = PACKAGE / "_lib"
LIBRARY = OUT_DIR / "libdrama3_moe.so"
ARCH = os.environ.get("DRAMA3_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops stay off: hipcc must not form v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build")
    return path


def sources() -> list[Path]:
    return sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])


# The compiler's per-kernel resource report; every kernel must run without
# per-lane scratch (a register spill or an outlined call that the compiler
# chose not to inline costs the hot loops several microseconds).
RESOURCE_REMARKS = "-Rpass-analysis=kernel-resource-usage"
_FUNCTION = re.compile(r"remark: Function Name: (\S+)")
_SCRATCH = re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")


def scratch_users(remarks: str) -> list[tuple[str, int]]:
    """(function, bytes per lane) for every function the resource remarks
    report with a nonzero scratch size."""
    users, name = [], None
    for line in remarks.splitlines():
        m = _FUNCTION.search(line)
        if m:
            name = m.group(1)
            continue
        m = _SCRATCH.search(line)
        if m and name is not None and int(m.group(1)) > 0:
            users.append((name, int(m.group(1))))
    return users


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, RESOURCE_REMARKS, *extra, "-c", str(src), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{result.stdout}\n{result.stderr}")
    users = scratch_users(result.stderr)
    if users:
        listing = "\n".join(f"  {name}: {size} bytes/lane" for name, size in users)
        raise RuntimeError(f"{src.name}: kernels use per-lane scratch (spills or outlined calls):\n{listing}")


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every source and link the library; returns its path."""
    extra = list(extra_flags or [])
    objdir = OUT_DIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        futures = [pool.submit(_compile, s, objdir / (s.stem + ".o"), extra) for s in srcs]
        for f in futures:
            f.result()
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(objdir / (s.stem + ".o")) for s in srcs]]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
