"""Build libttsplat.so (gfx950) from tt-splat_amd/csrc/*.hip with hipcc.

Each source compiles to its own object in parallel, then one shared library is linked next to
this package (ttsplat/libttsplat.so), where the loader looks for it.

Flags
  --offload-arch=gfx950            CDNA4 only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                   no packed-FP32 (v_pk_*_f32) codegen
  -ffp-contract=off (binning.hip)  binning keys are products and sums rounded one by one
  -mllvm -amdgpu-mfma-vgpr-form (splat.hip)
                                   matrix-core results in VGPRs, not accumulator registers
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                       # tt-splat_amd/
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
LIB_NAME = "libttsplat.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
OBJ_DIR = os.path.join(ROOT, "_build")

COMMON = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument", "-I", INCLUDE, "-I", CSRC]
PER_FILE = {"binning.hip": ["-ffp-contract=off"],
            # matrix-core results straight into VGPRs (no accumulator-register copies)
            "splat.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: the ttsplat HIP library cannot be built")
    return exe


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OBJ_DIR, src.replace(".hip", ".o"))
    cmd = [hipcc(), *COMMON, *PER_FILE.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    """Compile every csrc/*.hip and link LIB_PATH.  Always rebuilds.  Returns the .so path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
