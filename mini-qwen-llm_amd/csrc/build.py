"""Build libmqk.so (gfx950) in-tree with hipcc.

    python mini-qwen-llm_amd/csrc/build.py            # build
    python mini-qwen-llm_amd/csrc/build.py --verbose  # echo the hipcc lines
    python mini-qwen-llm_amd/csrc/build.py --incremental  # recompile only sources
                                                          # newer than their object

Every translation unit is compiled in parallel, then linked into
``mini-qwen-llm_amd/mqk/libmqk.so`` (the location the ``mqk`` package loads).
The compile flags switch off packed-fp32 instruction selection for the device
pass (``-target-feature -packed-fp32-ops``); hipcc's host pass prints a
harmless "not a recognized feature" warning for it.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent / "mqk"
OUT = PKG / "libmqk.so"
BUILD_DIR = CSRC.parent / "_build"
SOURCES = ["qkv_tile.hip", "qkv_tile_dma.hip", "qkv_decode.hip", "norm_rope.hip", "input_norm.hip", "qkv_f32.hip",
           "w4_gemv.hip", "read_probe.hip", "mqk_api.hip"]
# No kernel may use scratch memory (register spills, or an array the compiler
# could not keep in registers): the compiler's resource-usage remarks of every
# source are checked and the build fails otherwise.
NO_SCRATCH = set(SOURCES)
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _filter(text: str) -> str:
    keep = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
    return "\n".join(keep)


def _scratch_kernels(remarks: str) -> list[str]:
    """Kernels with a non-zero ScratchSize in -Rpass-analysis=kernel-resource-usage output."""
    bad, name = [], None
    for ln in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", ln)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", ln)
        if m and int(m.group(1)) > 0 and name:
            bad.append(f"{name} ({m.group(1)} B/lane)")
    return bad


def _up_to_date(src: str, obj: Path) -> bool:
    """The object is newer than its source and every header of csrc/."""
    if not obj.exists():
        return False
    t = obj.stat().st_mtime
    deps = [CSRC / src, *CSRC.glob("*.h"), CSRC.parent.parent / "include" / "mqk.h", Path(__file__)]
    return all(d.stat().st_mtime < t for d in deps if d.exists())


def _compile(src: str, verbose: bool, incremental: bool = False) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    if incremental and _up_to_date(src, obj):
        return obj
    check = src in NO_SCRATCH
    cmd = [_hipcc(), *COMMON_FLAGS, *(["-Rpass-analysis=kernel-resource-usage"] if check else []),
           "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = res.stdout + res.stderr
    msg = _filter("\n".join(ln for ln in out.splitlines() if "remark:" not in ln)).strip()
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
    if check:
        bad = _scratch_kernels(out)
        if bad:
            raise RuntimeError(f"{src}: kernels use scratch memory (register spills): " + "; ".join(bad))
    if msg and verbose:
        print(msg)
    return obj


def build(verbose: bool = False, incremental: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, incremental), SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + _filter(res.stdout + res.stderr))
    os.replace(tmp, OUT)
    return OUT


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--incremental", action="store_true", help="skip sources whose object is up to date")
    args = ap.parse_args(argv)
    out = build(args.verbose, args.incremental)
    print(f"built {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
