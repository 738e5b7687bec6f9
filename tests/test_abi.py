"""The C ABI library: loads, exports every declared symbol, validates arguments.

No compute call is made (there is no GPU here): every call below fails or
returns before any HIP call, as Light's op layer validates before launching
(ops/matmul_q.go:28-47, ops/int4.go:67-72, ops/moe.go:125-155).
"""
import ctypes
import os
import re

import pytest

from light_amd import hipq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "hipq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(hq_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = hipq.lib()
    decl = _declared()
    assert len(decl) >= 20
    for name in decl:
        assert hasattr(L, name), name
    assert set(decl) == set(hipq.SIGNATURES), set(decl) ^ set(hipq.SIGNATURES)


def test_version_and_no_error():
    assert hipq.lib().hq_version() >= 100
    assert isinstance(hipq.last_error(), str)


def _matmul_q(M, N, K, dt, x=1 << 12, w=1 << 12, out=1 << 12):
    L = hipq.lib()
    return L.hq_matmul_q(x, w, out, M, N, K, dt, None, 0, None)


def test_matmul_q_rejects_unquantized_dtype():
    rc = _matmul_q(1, 4, 256, hipq.F32)
    assert rc == hipq.HQ_EUNSUPPORTED
    msg = hipq.last_error()
    assert msg.startswith("hipq: hq_matmul_q:") and "(code -2)" in msg


@pytest.mark.parametrize("dt,K", [(hipq.Q4_K, 255), (hipq.Q4_K, 128), (hipq.Q6_K, 32), (hipq.Q8_0, 48)])
def test_matmul_q_k_not_block_multiple(dt, K):
    """K % BlockElems != 0 is an error (ops/matmul_q.go:45-47)."""
    assert _matmul_q(1, 4, K, dt) == hipq.HQ_EINVAL
    assert "not a multiple of block size" in hipq.last_error()


def test_matmul_q_empty_is_ok_and_null_is_error():
    assert _matmul_q(0, 4, 256, hipq.Q4_K) == hipq.HQ_OK
    assert _matmul_q(1, 0, 256, hipq.Q4_K) == hipq.HQ_OK
    assert _matmul_q(1, 4, 256, hipq.Q4_K, x=None) == hipq.HQ_EINVAL
    assert _matmul_q(1, 4, 256, hipq.Q4_K, x=(1 << 12) + 4) == hipq.HQ_EINVAL  # misaligned


def test_matmul_q_workspace_too_small():
    L = hipq.lib()
    need = L.hq_matmul_q_ws_bytes(3, 4, 4096, hipq.Q4_K)
    assert need >= 3 * 128 * 36
    rc = L.hq_matmul_q(1 << 12, 1 << 12, 1 << 12, 3, 4, 4096, hipq.Q4_K, 1 << 12, need - 1, None)
    assert rc == hipq.HQ_ENOMEM


def test_int4_validation():
    L = hipq.lib()
    p = 1 << 12
    assert L.hq_int4_matmul(p, hipq.F32, p, p, p, p, 1, 8, 256, 48, None, 0, None) == hipq.HQ_EINVAL
    assert "does not divide" in hipq.last_error()
    assert L.hq_int4_matmul(p, hipq.F32, p, p, p, p, 1, 8, 48, 16, None, 0, None) == hipq.HQ_EUNSUPPORTED
    assert L.hq_int4_matmul(p, hipq.Q4_K, p, p, p, p, 1, 8, 256, 64, None, 0, None) == hipq.HQ_EUNSUPPORTED
    assert L.hq_int4_dequant(p, p, p, p, hipq.F32, 8, 256, 48, 0, None) == hipq.HQ_EINVAL
    assert L.hq_int4_dequant(p, p, p, p, hipq.F16, 8, 256, 64, 0, None) == hipq.HQ_EUNSUPPORTED


def test_moe_validation():
    L = hipq.lib()
    p = 1 << 12
    # rows must be M (per pair) or M/topk (per token) (ops/moe.go:139-147)
    rc = L.hq_moe_gemm_q(p, p, p, p, p, p, None, p, 2, 8, 8, 5, 4, 16, 256, 0, hipq.Q4_K, None, 0, None)
    assert rc == hipq.HQ_EINVAL and "input rows" in hipq.last_error()
    rc = L.hq_moe_gemm_q(p, p, p, p, p, p, None, p, 2, 8, 8, 4, 4, 16, 256, 0, hipq.F32, None, 0, None)
    assert rc == hipq.HQ_EUNSUPPORTED


def test_dequant_validation():
    L = hipq.lib()
    p = 1 << 12
    assert L.hq_dequant(p, p, 100, hipq.Q4_K, hipq.F32, None) == hipq.HQ_EINVAL
    assert L.hq_dequant(p, p, 256, hipq.F32, hipq.F32, None) == hipq.HQ_EUNSUPPORTED
    assert L.hq_quantize_q8_1(p, hipq.F32, p, 1, 33, None) == hipq.HQ_EINVAL


def test_check_raises_with_message():
    with pytest.raises(hipq.HipqError) as e:
        hipq.check(_matmul_q(1, 4, 100, hipq.Q4_K))
    assert e.value.code == hipq.HQ_EINVAL


def test_matmul_q_noalloc_validates_before_any_device_call():
    """The allocation-free entry point checks arguments and its static scratch limit first."""
    L = hipq.lib()
    assert L.hq_matmul_q_noalloc(1 << 12, 1 << 12, 1 << 12, 1, 4, 256, hipq.F32, None) == hipq.HQ_EUNSUPPORTED
    assert L.hq_matmul_q_noalloc(1 << 12, 1 << 12, 1 << 12, 1, 4, 255, hipq.Q4_K, None) == hipq.HQ_EINVAL
    assert L.hq_matmul_q_noalloc(1 << 12, 1 << 12, 1 << 12, 0, 4, 256, hipq.Q4_K, None) == hipq.HQ_OK
    assert L.hq_matmul_q_noalloc(None, 1 << 12, 1 << 12, 1, 4, 256, hipq.Q4_K, None) == hipq.HQ_EINVAL
    # M = 4096, K = 14336 needs 117 MB of bf16 x alone: beyond the 64 MiB scratch.
    need = L.hq_matmul_q_ws_bytes(4096, 4096, 14336, hipq.Q4_K)
    assert need > hipq.NOALLOC_SCRATCH_BYTES
    rc = L.hq_matmul_q_noalloc(1 << 12, 1 << 12, 1 << 12, 4096, 4096, 14336, hipq.Q4_K, None)
    assert rc == hipq.HQ_ENOMEM
    assert "static scratch" in hipq.last_error()
    # The benchmark's M = 512 prefill shapes and every decode shape fit.
    for M, N, K in ((512, 14336, 4096), (512, 4096, 14336), (1, 128256, 4096), (8, 4096, 14336)):
        assert L.hq_matmul_q_ws_bytes(M, N, K, hipq.Q4_K) <= hipq.NOALLOC_SCRATCH_BYTES, (M, N, K)
