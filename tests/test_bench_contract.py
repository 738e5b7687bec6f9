"""CPU checks of bench.py's contract: one GPU only, the step's algorithmic bytes, and weight
rotation past the Infinity Cache.  No GPU is touched."""
import os
import subprocess
import sys
import types

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (standard library only at import time)


def q4k_bytes(N, K):
    """Q4_K as stored: 144-byte blocks of 256 weights along each row."""
    return N * (K // 256) * 144


def test_more_than_one_gpu_is_refused_with_a_message():
    env = dict(os.environ, WORLD_SIZE="1")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, env=env, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_a_second_rank_is_refused_too():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 2
    assert "WORLD_SIZE 2" in r.stderr


def test_step_bytes_are_the_llama3_8b_mlp_weights_plus_x_and_y():
    H, I = 4096, 14336

    def w(N, K):
        return types.SimpleNamespace(raw=np.empty(q4k_bytes(N, K), np.uint8), N=N, K=K)

    gate, up, down = w(I, H), w(I, H), w(H, I)
    # 3 x 14336 x 4096 weights at 4.5 bits, F32 x (4096) in and F32 y (4096) out.
    assert bench.step_bytes(gate, up, down) == 3 * 33_030_144 + 4 * 4096 + 4 * 4096 == 99_123_200


def test_rotated_copies_exceed_the_infinity_cache():
    for nbytes in (1 << 20, 33_030_144, 128 << 20, 300 << 20):
        n = bench.copies_for(nbytes)
        assert n >= 2
        assert n * nbytes >= 2 * bench.MALL_BYTES
