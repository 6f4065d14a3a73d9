"""Compiles libvmi.so (HIP, gfx950) in-tree with hipcc."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libvmi.so"
# A tuning variant: the same sources with the kernels' real-time stamps on
# (-DVMI_TIMELINE), read by vates_amd.timeline.  Never loaded by the product.
TIMELINE_LIB = PKG / "libvmi_timeline.so"
SOURCES = ["vmi_moe.hip", "vmi_util.hip", "vmi_head.hip", "vmi_accept.hip", "vmi_prefill.hip", "vmi_attn.hip", "vmi_gdn.hip",
           "vmi_peak.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed FP32 instructions stay off: scalar float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source additions.  The prefill GEMMs scale every MFMA result by FMA:
# MFMA results in VGPRs (not accumulation registers) save a copy per value.
SOURCE_FLAGS = {
    "vmi_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libvmi.so)")


def build_library(verbose: bool = False, timeline: bool = False) -> Path:
    """Compiles every source to an object, then links libvmi.so atomically
    (timeline: libvmi_timeline.so, the stamped tuning variant)."""
    objdir = ROOT / "_build" / ("timeline" if timeline else "")
    objdir.mkdir(parents=True, exist_ok=True)
    target = TIMELINE_LIB if timeline else LIB
    extra = ["-DVMI_TIMELINE"] if timeline else []
    cc = hipcc()
    objs = []
    procs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        cmd = [cc, *HIP_FLAGS, *extra, *SOURCE_FLAGS.get(src, []), f"-I{ROOT / 'include'}", "-c", str(CSRC / src),
               "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines() if "packed-fp32-ops" not in l)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed: {' '.join(cmd)}\n{text}")
        if verbose and text.strip():
            print(text)
    tmp = target.with_suffix(".so.tmp")
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}{res.stderr}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    import sys
    print(build_library(verbose=True, timeline="--timeline" in sys.argv[1:]))
