"""Build ``libawq_w4a16.so`` in-tree with hipcc for gfx950 (no JIT cache, no torch extension).

Usage: ``python -m litevllm_amd.build``.  Each translation unit under ``csrc/`` compiles to
an object in ``_build/`` in parallel, then one link produces the shared library next to this
file, so it travels with the source tree to the GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INC = os.path.join(ROOT, "include")
BUILD_DIR = os.path.join(ROOT, "_build")
OUT = os.path.join(HERE, "libawq_w4a16.so")
ARCH = "gfx950"
SOURCES = ["awq_capi.hip", "awq_dequant.hip", "awq_decode.hip", "awq_decode_misc.hip", "awq_decode_narrow.hip",
           "awq_gemm.hip", "awq_prefill.hip", "awq_moe.hip", "awq_moe_misc.hip", "awq_moe_mfma.hip", "awq_moe_mfma_down.hip",
           "awq_rmsnorm.hip"]

# hipcc's host pass does not know the packed-fp32 target feature and says so: harmless
_NOISE = "is not a recognized feature for this target"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.isfile(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build the HIP library)")


def common_flags(extra: list[str] | None = None) -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        # packed-fp32 VALU forms are kept out of the generated code on purpose
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INC}", f"-I{CSRC}", *(extra or []),
    ]


def compile_cmd(src: str, obj: str, extra: list[str] | None = None) -> list[str]:
    return [hipcc(), *common_flags(extra), "-c", "-o", obj, src]


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if _NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = True, out: str = OUT, sources: list[str] | None = None,
          extra: list[str] | None = None, build_dir: str = BUILD_DIR) -> str:
    """Compile every translation unit (in parallel) and link ``out``."""
    os.makedirs(build_dir, exist_ok=True)
    srcs = [s if os.path.isabs(s) else os.path.join(CSRC, s) for s in (sources or SOURCES)]
    objs = [os.path.join(build_dir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = {ex.submit(_run, compile_cmd(s, o, extra)): s for s, o in zip(srcs, objs)}
        for f in cf.as_completed(futs):
            err = f.result()
            if verbose:
                print(f"[build] compiled {os.path.basename(futs[f])}", flush=True)
                if err.strip():
                    print(err, file=sys.stderr)
    tmp = out + ".tmp"
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    _run(link)
    os.replace(tmp, out)
    if verbose:
        print(f"[build] linked {out}", flush=True)
    return out


if __name__ == "__main__":
    print(build())
