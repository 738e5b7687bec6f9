"""Build libhipq.so (gfx950, hipcc, light_amd/csrc/Makefile) and the host-layer module
_light*.so (g++ + pybind11, light_amd/host/Makefile) in-tree."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")


def build(jobs=8, force=False):
    """Compile every HIP translation unit for gfx950, link light_amd/libhipq.so, then the host module."""
    for d in (CSRC, HOST):
        if force:
            subprocess.run(["make", "-s", "-C", d, "clean"], check=True)
        subprocess.run(["make", "-s", f"-j{jobs}", "-C", d], check=True)
    return os.path.join(HERE, "libhipq.so")


if __name__ == "__main__":
    print(build())
