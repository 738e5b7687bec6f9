"""Random arguments through every C-ABI entry point that takes only device pointers, shapes
and dtypes (negative, zero, huge and overflowing sizes; NULL and misaligned pointers): each
call returns a status code, never crashes the process.  Host-side only: on a machine with a
GPU the calls that pass validation would launch on fake pointers, so the test is skipped
there (no device is visible in the CPU suite, where a validated call fails at its first HIP
call).  Run in a child process so a crash is reported, with the call that caused it."""
import ctypes
import os
import subprocess
import sys

import pytest

from light_amd import hipq

pytestmark = pytest.mark.skipif(not os.path.exists(hipq.LIB_PATH), reason="libhipq.so not built")

_CHILD = r"""
import ctypes, random, sys
from light_amd import hipq
L = hipq.lib()
n = ctypes.c_int(0)
if L.hq_device_count(ctypes.byref(n)) == 0 and n.value > 0:
    print("gpu"); sys.exit(0)
SKIP = {"hq_last_error", "hq_device_count", "hq_malloc", "hq_free", "hq_memcpy_h2d", "hq_memcpy_d2h",
        "hq_memcpy_d2d", "hq_memset", "hq_stream_create", "hq_stream_destroy", "hq_stream_synchronize",
        "hq_stream_set_current", "hq_stream_get_current", "hq_trace_start", "hq_trace_stop", "hq_version",
        "hq_debug_moe_block_spin_limit", "hq_set_device", "hq_workspace_release",
        "hq_ceiling_mfma"}  # (host pointers or process state)
rng = random.Random(int(sys.argv[1]))
I64 = [0, 1, -1, 2, 7, 32, 64, 256, 4096, 14336, 1 << 31, (1 << 31) - 1, 1 << 40, 1 << 62, -(1 << 62),
       (1 << 63) - 1, -(1 << 63)]
II = [0, 1, -1, 2, 3, 8, 13, 15, 17, 21, 22, 23, 30, 31, 64, 127, 128, 255, 256, 1 << 30, -(1 << 31), (1 << 31) - 1]
PP = [None, 0x10000, 0x10004, 0x10001]
SZ = [0, 1, 16, 1 << 20, 1 << 40, (1 << 64) - 1]
names = [k for k in hipq.SIGNATURES if k not in SKIP]
for it in range(int(sys.argv[2])):
    name = rng.choice(names)
    res, argt = hipq.SIGNATURES[name]
    args = []
    for a in argt:
        if a is ctypes.c_int64:
            args.append(rng.choice(I64) if rng.random() < 0.8 else rng.randrange(-5, 20000))
        elif a is ctypes.c_int:
            args.append(rng.choice(II) if rng.random() < 0.8 else rng.randrange(-5, 300))
        elif a is ctypes.c_size_t:
            args.append(rng.choice(SZ))
        else:
            args.append(rng.choice(PP))
    sys.stderr.write(f"{name} {args}\n")
    getattr(L, name)(*args)
    hipq.last_error()  # the error text is always a valid C string
print("done")
"""


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_arguments_never_crash(seed):
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.environ.get("PYTHONPATH", "")]), HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sys.executable, "-c", _CHILD, str(seed), "4000"], capture_output=True, text=True, env=env,
                       timeout=300)
    if r.stdout.strip() == "gpu":
        pytest.skip("a GPU is visible: random calls could launch on fake pointers")
    last = r.stderr.strip().splitlines()[-1:] if r.stderr else []
    assert r.returncode == 0 and r.stdout.strip() == "done", f"rc {r.returncode}, last call: {last}"
