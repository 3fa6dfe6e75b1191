"""Ahead-of-time build of libtrnopt_hip.so (the fused Sinkhorn kernels for gfx950) with hipcc.

    python -m trnopt._build            # from trainium-sinkhorn_amd/, or call build() from Python

The library lands in trnopt/_lib/ next to this file (in the source tree, so it ships with the package
directory); nothing is compiled at import time. Two translation units:

* sk_lse_partial.hip -- the MFMA partial (max, sum) kernel, built with -fno-honor-nans -mno-amdgpu-ieee
  (no NaN ever reaches it; this drops the IEEE canonicalisation of every MFMA result before a max), twice:
  the instantiations of kp <= 64 and those of kp 80 to 128, both with MFMA results in VGPRs
  (-amdgpu-mfma-vgpr-form: the epilogue reads them without copies);
* sk_kernels.hip -- packing, finalisation, the on-device loop and the C ABI, built with default NaN
  semantics (the loop state stores NaN for "not checked yet").

Every HIP file is built with -Xclang -target-feature -Xclang -packed-fp32-ops (no packed fp32 VALU).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent                        # trainium-sinkhorn_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
LIB_DIR = PKG / "_lib"
LIB_NAME = "libtrnopt_hip.so"
ARCH = os.environ.get("TRNOPT_HIP_ARCH", "gfx950")

COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]
UNITS = [   # (source, object name, extra flags)
    ("sk_lse_partial.hip", "sk_lse_partial_small", ["-fno-honor-nans", "-mno-amdgpu-ieee", "-DSK_PARTIAL_LARGE=0",
                                                    "-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("sk_lse_partial.hip", "sk_lse_partial_large", ["-fno-honor-nans", "-mno-amdgpu-ieee", "-DSK_PARTIAL_LARGE=1",
                                                    "-mllvm", "-amdgpu-mfma-vgpr-form"]),
    ("sk_kernels.hip", "sk_kernels", []),
    ("sk_median.hip", "sk_median", []),
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build libtrnopt_hip.so)")


def lib_path() -> Path:
    return LIB_DIR / LIB_NAME


def build(verbose: bool = False) -> Path:
    """Compile and link the library (always rebuilds). Returns its path."""
    cc = hipcc()
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="trnopt_build_") as tmp:
        cmds, objs = [], []
        for src, name, extra in UNITS:
            obj = Path(tmp) / (name + ".o")
            cmds.append([cc, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)])
            objs.append(str(obj))
        # the translation units compile independently: one hipcc process each, at most MAX_JOBS at once
        jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", "") or os.cpu_count() or 1)))
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                f.result()
        out_tmp = Path(tmp) / LIB_NAME
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(out_tmp)], verbose)
        # Replace atomically so a process that has the old library mapped keeps a valid file.
        dst = lib_path()
        staged = dst.with_suffix(".so.tmp")
        shutil.copy2(out_tmp, staged)
        os.replace(staged, dst)
    return lib_path()


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
