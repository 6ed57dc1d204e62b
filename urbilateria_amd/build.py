"""In-tree build of the HIP libraries for gfx950 (hipcc; no JIT cache, no site-packages)."""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
ARCH = "gfx950"

# -ffp-contract=off: every fused multiply-add is written out (fmaf) where wanted, so the
# reference's separate multiply/add steps stay separate.  Denormals are kept (E8M0 code 0 is
# the f32 subnormal 2^-127).  Packed FP32 instructions are disabled.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

MOE_SOURCES = ["urb_route.hip", "urb_panel.hip", "urb_combine.hip", "urb_gemm.hip", "urb_hy4.hip",
               "urb_decode.hip", "urb_scratch.hip", "urb_dense.hip",
               "urb_block.hip",
               "urb_moe_host.cpp", "urb_residency.cpp"]
SYNTH_SOURCES = ["urb_synth.hip"]


def _hipcc() -> str:
    for c in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.exists(c) or c == "hipcc":
            return c
    return "hipcc"


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({' '.join(cmd)}):\n{err}")
    return err


def _compile(sources, out, verbose=False):
    """Each source to an object in parallel (one hipcc per file), then one link."""
    from concurrent.futures import ThreadPoolExecutor
    srcs = [os.path.join(CSRC, s) for s in sources if os.path.exists(os.path.join(CSRC, s))]
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.basename(s) + ".o") for s in srcs]
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "0") or 0) or os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as pool:
        errs = list(pool.map(lambda so: _run([_hipcc(), *flags, "-c", "-o", so[1], so[0]]),
                             zip(srcs, objs)))
    tmp = out + ".tmp"
    errs.append(_run([_hipcc(), *HIPCC_FLAGS, "-o", tmp, *objs]))
    if verbose:
        for e in errs:
            if e.strip():
                print(e, file=sys.stderr)
    os.replace(tmp, out)


def build(verbose: bool = False) -> None:
    _compile(MOE_SOURCES, os.path.join(HERE, "liburb_moe.so"), verbose)
    _compile(SYNTH_SOURCES, os.path.join(HERE, "liburb_synth.so"), verbose)


if __name__ == "__main__":
    build(verbose=True)
    print("built", os.path.join(HERE, "liburb_moe.so"), os.path.join(HERE, "liburb_synth.so"))
