"""Build ``libtx_hip.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m transformer_optimization_amd.build`` (or ``build()``).
Each ``csrc/*.hip`` file is compiled to an object under ``_build/`` in
parallel, then linked into ``transformer_optimization_amd/_lib/libtx_hip.so``.
The library links the HIP runtime by SONAME (``libamdhip64.so.7``), so when it
is loaded after ``import torch`` it binds to the runtime torch already mapped.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libtx_hip.so"
OBJ_DIR = ROOT / "_build"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

CXXFLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # Packed-FP32 VALU instructions stay disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source flags.  The eager-exact attention must round every product to
# fp32 before converting it to 16 bits, as the eager ops do; fp contraction
# would fold multiply + convert into one v_fma_mix (a single rounding).
EXTRA_FLAGS = {
    "attention.hip": ["-ffp-contract=off"],
}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True, jobs: int | None = None, incremental: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library.

    ``incremental=True`` recompiles only sources (or shared headers) newer
    than their object file."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)

    headers = list(CSRC.glob("*.hpp")) + list(INCLUDE.glob("*.h"))
    newest_header = max((h.stat().st_mtime for h in headers), default=0.0)

    def compile_one(pair):
        src, obj = pair
        if incremental and obj.exists():
            mtime = obj.stat().st_mtime
            if mtime > src.stat().st_mtime and mtime > newest_header:
                return
        cmd = [HIPCC, *CXXFLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print("[build]", " ".join(cmd[:1] + cmd[-3:]), flush=True)
        _run(cmd)

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(compile_one, zip(sources, objs)))

    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    _run(cmd)
    os.replace(tmp, LIB)
    _write_build_info()
    if verbose:
        print(f"[build] wrote {LIB}", flush=True)
    return LIB


def _git(*args: str) -> str | None:
    try:
        out = subprocess.run(["git", "-C", str(ROOT), *args], stdout=subprocess.PIPE,
                             stderr=subprocess.DEVNULL, text=True, timeout=20)
    except (OSError, subprocess.SubprocessError):
        return None
    return out.stdout.strip() if out.returncode == 0 else None


def _write_build_info() -> None:
    """Record the git state the library was built from next to it
    (``_lib/build_info.json``), so that a run on a copy of the tree without
    ``.git`` can still name its commit.  Built artefact, not tracked."""
    import datetime
    import hashlib
    import json
    h = hashlib.sha256()
    for f in sorted([*CSRC.glob("*"), *INCLUDE.glob("*.h")]):
        if f.is_file():
            h.update(str(f.relative_to(ROOT)).encode())
            h.update(f.read_bytes())
    status = _git("status", "--porcelain", "--untracked-files=no")
    info = {
        "git_head": _git("rev-parse", "HEAD"),
        "git_dirty": (bool(status) if status is not None else None),
        "built_utc": datetime.datetime.now(datetime.timezone.utc).isoformat(timespec="seconds"),
        "kernel_sources_sha256": h.hexdigest(),
    }
    (OUT_DIR / "build_info.json").write_text(json.dumps(info, indent=1) + "\n")


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv[1:])
