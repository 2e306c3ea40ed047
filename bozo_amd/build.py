"""Build libtension_hip.so for gfx950 with hipcc (no GPU needed).

    python -m bozo_amd.build          # always recompiles

Each HIP translation unit is compiled in parallel to an object file under
bozo_amd/_build/, then linked into bozo_amd/lib/libtension_hip.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OBJDIR = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIBNAME = "libtension_hip.so"
ARCH = os.environ.get("TENSION_OFFLOAD_ARCH", "gfx950")

SOURCES = [
    "capi.hip", "exact.hip", "decode.hip",
    "mfma.hip", "mfma_fwd.hip", "mfma_dq.hip", "mfma_dkv.hip", "mfma_bwd_fused.hip", "mfma_global.hip",
    "split.hip", "split_fwd_bf16.hip", "split_dq_bf16.hip", "split_dkv_bf16.hip",
    "split_fwd_f32.hip", "split_dq_f32.hip", "split_dkv_f32.hip",
    "split_fwd_f32v.hip", "split_dq_f32v.hip", "split_dkv_f32v.hip",
    "split_fwd_f16.hip", "split_dq_f16.hip", "split_dkv_f16.hip",
    "tau_export.hip", "graph_bias.hip", "aux_loss.hip",
    "exact_fwd_f32.hip", "exact_dq_f32.hip", "exact_dkv_f32.hip",
    "exact_fwd_f64.hip", "exact_dq_f64.hip", "exact_dkv_f64.hip",
]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # code-object v5 loads under both torch's bundled HIP 7.0 runtime and /opt/rocm 7.2
    "-mcode-object-version=5",
    # no packed-fp32 VALU instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libtension_hip.so)")


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    # the host pass prints a harmless notice about the device-only feature flag
    noise = "packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (r.stderr or "").splitlines() if noise not in ln and ln.strip()]
    if msgs:
        sys.stderr.write("\n".join(msgs) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4, 16)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    out = os.path.join(LIBDIR, LIBNAME)
    tmp = out + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
