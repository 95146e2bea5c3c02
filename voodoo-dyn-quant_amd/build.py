"""Build libvoodoo_hip.so (gfx950) in-tree.

    python voodoo-dyn-quant_amd/build.py [--jobs N]

Each ``csrc/*.hip`` file is compiled to an object with hipcc in parallel, then
linked into ``voodoo_quant/libvoodoo_hip.so`` next to the Python package that
loads it.  ``csrc/probe/*.hip`` (measurement probes for bench.py, outside the
product's C ABI) becomes ``voodoo_quant/libvq_probe.so``.  Objects go to
``_build/`` (git-ignored).
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT_DIR = ROOT / "_build"
LIB = ROOT / "voodoo_quant" / "libvoodoo_hip.so"
PROBE_LIB = ROOT / "voodoo_quant" / "libvq_probe.so"
ARCH = os.environ.get("VQ_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # never emit packed-fp32 VALU ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Extra hipcc flags per source file.
FILE_FLAGS = {
    # MFMA accumulators in VGPRs: the attention softmax reads and rescales the
    # accumulators with VALU ops, which AGPR accumulators would copy out and
    # back for every key tile (255 v_accvgpr moves per tile)
    "vq_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or Path(cand).exists()):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _link(hipcc: str, objs: list[Path], lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, lib)


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    t0 = time.time()
    OUT_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    probes = sorted((CSRC / "probe").glob("*.hip"))
    objs = [OUT_DIR / (s.stem + ".o") for s in sources]
    probe_objs = [OUT_DIR / ("probe_" + s.stem + ".o") for s in probes]
    with ThreadPoolExecutor(max_workers=jobs or min(8, len(sources) + len(probes))) as ex:
        list(ex.map(lambda so: _run([hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(so[0].name, []), "-c", str(so[0]),
                                     "-o", str(so[1])]),
                    zip(sources + probes, objs + probe_objs)))
    _link(hipcc, objs, LIB)
    if probe_objs:
        _link(hipcc, probe_objs, PROBE_LIB)
    if verbose:
        print(f"built {LIB} (and {PROBE_LIB.name}) in {time.time() - t0:.1f}s")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    build(ap.parse_args().jobs)
