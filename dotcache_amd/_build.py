"""Build ``libdotcache_hip.so`` for gfx950 with hipcc (no GPU needed).

Run as ``python -m dotcache_amd._build``; ``__graft_entry__.build()`` calls
:func:`build`.  The library is written in-tree next to this file so it
travels with the repository snapshot.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libdotcache_hip.so"
SOURCES = ["dc_abi.cpp", "dc_encode.hip", "dc_score_mix.hip", "dc_decode.hip", "dc_decode_mfma.hip", "dc_shortlist.hip",
           "dc_decode_noalloc.hip"]

# -packed-fp32-ops: no v_pk_*_f32 anywhere in the device code.
# -ffp-contract=off: no fused multiply-add, so the encoder's fp32 steps round
# exactly like numpy's.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
# dc_decode_mfma.hip: MFMA results in VGPRs (the VGPR form of the
# instruction) instead of AGPRs, so the score's per-group results and the
# softmax rescale of the accumulators need no AGPR <-> VGPR copies.
PER_FILE = {"dc_encode.hip": ["-ffp-contract=off"],
            "dc_decode_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm 7.x with gfx950 support is required)")


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    # one hipcc per source, all at once (they are independent)
    jobs = []
    for name in SOURCES:
        src = CSRC / name
        if not src.exists():
            continue
        obj = objdir / (name + ".o")
        lang = ["-x", "hip"] if name.endswith(".cpp") else []
        cmd = [hipcc, *COMMON, *PER_FILE.get(name, []), *lang, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
        jobs.append((name, obj, proc))
    objs, failed = [], []
    for name, obj, proc in jobs:
        out, err = proc.communicate()
        if proc.returncode != 0:
            failed.append(f"hipcc failed on {name}:\n{out}\n{err}")
        elif verbose and err.strip():
            print(err, file=sys.stderr)
        objs.append(str(obj))
    if failed:
        raise RuntimeError("\n".join(failed))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
