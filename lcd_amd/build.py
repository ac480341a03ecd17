"""Builds ``liblcdhip.so`` (the HIP runtime, DAG inspector and probes) in tree.

Run ``python -m lcd_amd.build``; hipcc cross-compiles for gfx950 without a
GPU.  The packed-FP32 target feature is switched off for every device
compile of this project.
"""

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBRARY = os.path.join(HERE, "liblcdhip.so")
SOURCES = ("lcdhip_runtime.hip", "lcdhip_dag.hip")
DEVICE_FLAGS = ("-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


def hipcc_path():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(found):
        raise RuntimeError("hipcc was not found; a ROCm toolchain is required")
    return found


def build(verbose=False):
    """Compile every HIP source of the package into ``liblcdhip.so``."""
    objects = []
    build_dir = os.path.join(CSRC, "build")
    os.makedirs(build_dir, exist_ok=True)
    common = [
        hipcc_path(), "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
        "-munsafe-fp-atomics", *DEVICE_FLAGS,
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
    ]
    processes = []
    for source in SOURCES:
        obj = os.path.join(build_dir, source.replace(".hip", ".o"))
        objects.append(obj)
        command = common + ["-c", os.path.join(CSRC, source), "-o", obj]
        if verbose:
            print(" ".join(command), flush=True)
        processes.append((source, subprocess.Popen(
            command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
            text=True)))
    for source, process in processes:
        output, _ = process.communicate()
        if process.returncode != 0:
            raise RuntimeError(f"hipcc failed on {source}:\n{output}")
        if verbose and output.strip():
            print(output)
    link = [hipcc_path(), "--offload-arch=gfx950", "-shared", "-fPIC",
            *objects, "-o", LIBRARY, "-lhiprtc"]
    result = subprocess.run(link, stdout=subprocess.PIPE,
                            stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}")
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
