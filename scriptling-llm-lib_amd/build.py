"""Build libsllm_qmm.so (the C-ABI library) for gfx950 with hipcc, in-tree."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsllm_qmm.so")
# Measurement-only probe (peak int8 MFMA rate), loaded by bench.py, never by the library.
PROBE_LIB = os.path.join(HERE, "libsllm_probe.so")
PROBE_SOURCE = "probe_mfma.hip"

SOURCES = ["qmm_api.hip", "qmm_gemv.hip", "qmm_gemv_q8.hip", "qmm_gemv_q4.hip", "qmm_gemv_q4_1.hip",
           "qmm_gemv_q5.hip", "qmm_gemv_q5k1.hip", "qmm_gemv_q4k.hip", "qmm_gemv_q6k.hip", "qmm_gemv_q2k.hip", "qmm_gemv_q3k.hip", "qmm_gemm.hip", "qmm_pack.hip", "qmm_attn.hip"]

# -ffp-contract=off: every float operation rounds separately, as in the reference.
# -packed-fp32-ops off: no v_pk_*_f32 in the device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


# Per-source additions. The GEMM's MFMA results feed VALU arithmetic directly:
# keeping them in VGPRs (not AGPRs) saves a v_accvgpr_read per value.
EXTRA_FLAGS = {"qmm_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")


def build(verbose: bool = False) -> str:
    """Compile every source to an object (in parallel, under _build/), then link."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in srcs]
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    cmds = [[hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(s, []), *inc, "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(srcs, objs)]
    if verbose:
        for c in cmds:
            print(" ".join(c), flush=True)
    jobs = min(len(cmds), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", LIB + ".tmp"])
    os.replace(LIB + ".tmp", LIB)
    probe = [hipcc, *HIPCC_FLAGS, "-shared", os.path.join(CSRC, PROBE_SOURCE), "-o", PROBE_LIB + ".tmp"]
    if verbose:
        print(" ".join(probe), flush=True)
    _run(probe)
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
