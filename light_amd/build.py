"""Build libhipq.so (gfx950) in-tree with hipcc via light_amd/csrc/Makefile."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs=8, force=False):
    """Compile every HIP translation unit for gfx950 and link light_amd/libhipq.so."""
    if force:
        subprocess.run(["make", "-s", "-C", CSRC, "clean"], check=True)
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return os.path.join(HERE, "libhipq.so")


if __name__ == "__main__":
    print(build())
