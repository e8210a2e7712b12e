"""Build the gfx950 HIP library in-tree: ``mamba4_amd/libmamba4_memread.so``.

Usage: ``python -m mamba4_amd.build`` (or ``__graft_entry__.build()``).
hipcc cross-compiles for gfx950 without a GPU.  Every HIP source is built
with packed-FP32 instruction selection disabled.  The sources compile in
parallel; the ones with hand-written DPP multiply-adds are also compiled to
assembly and checked by ``check_dpp_hazards`` before the library is
replaced.
"""

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBRARY = os.path.join(HERE, "libmamba4_memread.so")
SOURCES = ["api.hip", "states.hip", "factor.hip", "chunk.hip", "mixer.hip", "order.hip",
           "scan3.hip", "diag.hip", "spd_wide.hip"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]

# Sources whose inline-asm DPP multiply-adds are re-checked on the compiled code.
HAZARD_CHECKED = ["factor.hip"]

# Per-source extra flags.  The factorization accumulates its trailing blocks
# in place with MFMA; keeping MFMA operands and results in VGPRs avoids a
# second copy of those blocks in AGPRs (which would halve the occupancy).
SOURCE_FLAGS = {"factor.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

_NOISE = "is not a recognized feature for this target"


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    stderr = "\n".join(line for line in proc.stderr.splitlines() if _NOISE not in line)
    return proc.returncode, stderr


def build(verbose=False):
    """Compile every source into the shared library; raises on failure."""
    include = ["-I", os.path.join(ROOT, "include")]
    with tempfile.TemporaryDirectory(prefix="m4mr_build_") as tmp:
        jobs = {}
        for src in SOURCES:
            obj = os.path.join(tmp, src.replace(".hip", ".o"))
            jobs[src] = (obj, [hipcc(), *FLAGS, *SOURCE_FLAGS.get(src, []), "-fPIC", "-c",
                               *include, "-o", obj, os.path.join(CSRC, src)])
        asms = {}
        for src in HAZARD_CHECKED:
            asm = os.path.join(tmp, src.replace(".hip", ".s"))
            asms[src] = (asm, [hipcc(), *FLAGS, *SOURCE_FLAGS.get(src, []), "--cuda-device-only",
                               "-S", *include, "-o", asm, os.path.join(CSRC, src)])
        workers = min(8, len(jobs) + len(asms))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            results = {k: pool.submit(_run, cmd) for k, (_, cmd) in jobs.items()}
            asm_results = {k: pool.submit(_run, cmd) for k, (_, cmd) in asms.items()}
            for src, fut in list(results.items()) + list(asm_results.items()):
                rc, stderr = fut.result()
                if rc != 0:
                    raise RuntimeError(f"hipcc failed on {src} ({rc}):\n{stderr}")
                if verbose and stderr.strip():
                    print(stderr, file=sys.stderr)
        check_hazards({src: open(path).read() for src, (path, _) in asms.items()}, verbose)
        out_tmp = os.path.join(tmp, "lib.so")
        rc, stderr = _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", out_tmp,
                           *(obj for obj, _ in jobs.values())])
        if rc != 0:
            raise RuntimeError(f"link failed ({rc}):\n{stderr}")
        _install(out_tmp)
    if verbose:
        print(LIBRARY, flush=True)
    return LIBRARY


def _install(path):
    """Copy the linked library next to the package, replacing it atomically."""
    staging = LIBRARY + ".tmp"
    with open(path, "rb") as src, open(staging, "wb") as dst:
        dst.write(src.read())
    os.chmod(staging, 0o755)
    os.replace(staging, LIBRARY)


def check_hazards(asm_texts, verbose=False):
    """Raise if a hand-written DPP read in the compiled code is unsafe."""
    from mamba4_amd import check_dpp_hazards

    for src, text in asm_texts.items():
        problems = check_dpp_hazards.check(text)
        if problems:
            raise RuntimeError(f"DPP hazard in {src}:\n" + "\n".join(problems[:20]))
        if verbose:
            print(f"{src}: {text.count('v_fmac_f32_dpp')} DPP multiply-adds, no hazards",
                  flush=True)


if __name__ == "__main__":
    build(verbose=True)
