"""ctypes binding of libhipq's C ABI (include/hipq.h) for torch device tensors.

This is the Python twin of the cgo stub a Light tree would carry: it passes
raw device pointers, sizes and Light dtype codes across the C ABI and turns a
non-zero return into ``HipqError`` carrying ``hq_last_error()``.  There is no
CPU fallback: if ``libhipq.so`` is missing, importing the op functions raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhipq.so")

# Light dtype.DType codes (dtype/dtype.go:13-37).
F16, BF16, F32 = 0, 1, 2
Q4_0, Q5_0, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K = 13, 15, 17, 18, 21, 22, 23
# Not a Light dtype: the planar load-time repack of Q6_K (hq_repack_q6k).
Q6_K_R = 123
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q8_1: (32, 36), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210)}
NAMES = {F16: "F16", BF16: "BF16", F32: "F32", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q8_1: "Q8_1",
         Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q6_K_R: "Q6_K_R"}

HQ_OK, HQ_EINVAL, HQ_EUNSUPPORTED, HQ_ENOMEM, HQ_EBARRIER = 0, -1, -2, -3, -4
ACT_SILU, ACT_GELU_ERF = 0, 1


class HipqError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_SZ = ctypes.c_size_t

# Every exported symbol with its ctypes signature; tests check this list
# against include/hipq.h.
SIGNATURES = {
    "hq_last_error": (ctypes.c_char_p, []),
    "hq_version": (_I, []),
    "hq_device_count": (_I, [ctypes.POINTER(_I)]),
    "hq_set_device": (_I, [_I]),
    "hq_malloc": (_I, [ctypes.POINTER(_P), _SZ]),
    "hq_free": (_I, [_P]),
    "hq_memcpy_h2d": (_I, [_P, _P, _SZ, _P]),
    "hq_memcpy_d2h": (_I, [_P, _P, _SZ, _P]),
    "hq_memcpy_d2d": (_I, [_P, _P, _SZ, _P]),
    "hq_memset": (_I, [_P, _I, _SZ, _P]),
    "hq_stream_create": (_I, [ctypes.POINTER(_P)]),
    "hq_stream_destroy": (_I, [_P]),
    "hq_stream_synchronize": (_I, [_P]),
    "hq_stream_set_current": (_I, [_P]),
    "hq_stream_get_current": (_P, []),
    "hq_trace_start": (_I, []),
    "hq_trace_stop": (_I, [ctypes.c_char_p, ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_double), _I]),
    "hq_matmul_q_ws_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "hq_matmul_q": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "hq_matmul_q_noalloc": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "hq_workspace_release": (_I, []),
    "hq_matmul_q_gated_ws_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "hq_matmul_q_gated": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _SZ, _P]),
    "hq_matmul_q_gated_act_ws_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "hq_matmul_q_gated_act": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _SZ, _P]),
    "hq_mlp_q_ws_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "hq_mlp_q": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _SZ, _P]),
    "hq_act_bytes": (_SZ, [_I64, _I64]),
    "hq_quantize_act": (_I, [_P, _I, _P, _I64, _I64, _P]),
    "hq_matmul_q_act_ws_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "hq_matmul_q_act": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "hq_dequant": (_I, [_P, _P, _I64, _I, _I, _P]),
    "hq_repack_q6k_bytes": (_SZ, [_I64, _I64]),
    "hq_repack_q6k": (_I, [_P, _P, _I64, _I64, _P]),
    "hq_dequant_rows": (_I, [_P, _P, _I64, _I64, _I, _I, _P]),
    "hq_quantize_q8_1": (_I, [_P, _I, _P, _I64, _I64, _P]),
    "hq_int4_matmul_ws_bytes": (_SZ, [_I64, _I64, _I64, _I, _I]),
    "hq_int4_matmul": (_I, [_P, _I, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "hq_int4_dequant": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _I, _I64, _P]),
    "hq_int4_from_gptq": (_I, [_P, _P, _P, _P, _I64, _I64, _I, _I, _P, _P, _P, _P]),
    "hq_int4_from_awq": (_I, [_P, _P, _P, _I64, _I64, _I, _P, _P, _P, _P]),
    "hq_moe_gemm_q_ws_bytes": (_SZ, [_I64, _I64, _I]),
    "hq_moe_combine": (_I, [_P, _P, _I64, _I64, _I, _P]),
    "hq_moe_gemm_q_combine_ws_bytes": (_SZ, [_I64, _I, _I64, _I64, _I64, _I]),
    "hq_moe_gemm_q_combine": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "hq_moe_route": (_I, [_P, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "hq_moe_sort_ids": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _P]),
    "hq_moe_gemm_q_gated_ws_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I]),
    "hq_moe_gemm_q_gated": (_I, [_P, _P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I,
                                 _P, _SZ, _P]),
    "hq_gather_cols": (_I, [_P, _P, _P, _I64, _I64, _I, _P]),
    "hq_moe_int4_ws_bytes": (_SZ, [_I64, _I, _I64]),
    "hq_moe_int4": (_I, [_P, _I, _P, _I64, _P, _P, _P, _I64, _I, _I64, _I64, _I, _I, _P, _SZ, _P]),
    "hq_moe_route_gated_ws_bytes": (_SZ, [_I64, _I, _I64, _I64, _I64, _I]),
    "hq_moe_block_q_ws_bytes": (_SZ, [_I64, _I, _I64, _I64, _I64, _I]),
    "hq_moe_block_q": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _P,
                            _P, _SZ, _P]),
    "hq_moe_block_q_check": (_I, [_P]),
    "hq_ceiling_read": (_I, [_P, _I64, _I, _I, _P, _P]),
    "hq_ceiling_mfma": (_I, [_I64, _P, _P, _P]),
    "hq_ceiling_mix": (_I, [_I, _I64, _P, _P]),
    "hq_debug_moe_block_spin_limit": (None, [ctypes.c_uint32]),
    "hq_moe_route_gated": (_I, [_P, _P, _P, _P, _I64, _I64, _I, _I, _I64, _I64, _I, _I, _P, _P, _P, _P, _P, _P, _P,
                                _SZ, _P]),
    "hq_moe_gemm_q": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I,
                           _P, _SZ, _P]),
}

_lib = None


def lib():
    """Load libhipq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"libhipq.so not built at {LIB_PATH}: run light_amd.build.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().hq_last_error().decode()


def check(rc):
    if rc != 0:
        raise HipqError(rc, last_error())
    return rc


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _torch_dtype_code(t):
    import torch
    return {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}[t.dtype]


def row_bytes(dt, K):
    be, bb = BLOCK[dt]
    return K // be * bb


# ---------------------------------------------------------------------------
# Ops (device tensors in, device tensors out; all asynchronous on the stream)
# ---------------------------------------------------------------------------

def matmul_q(x, w, N, K, w_dtype, out=None, ws=None, stream=None):
    """out (M, N) f32 = x (M, K) f32 @ dequant(w)^T; w is a uint8 tensor of GGUF blocks."""
    import torch
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_matmul_q(_ptr(x), _ptr(w), _ptr(out), M, N, K, w_dtype, _ptr(ws), ws_bytes, _stream(stream)))
    return out


def matmul_q_gated_act(x, wg, wu, N, K, w_dtype, act=ACT_SILU, out=None, ws=None, stream=None):
    """Prepared activations (uint8, hq_act_bytes(M, N)) of act(x @ dequant(wg)^T) * (x @ dequant(wu)^T)."""
    import torch
    M = x.shape[0]
    if out is None:
        out = torch.empty(lib().hq_act_bytes(M, N), dtype=torch.uint8, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_matmul_q_gated_act(_ptr(x), _ptr(wg), _ptr(wu), _ptr(out), M, N, K, w_dtype, act, _ptr(ws),
                                      ws_bytes, _stream(stream)))
    return out


def matmul_q_noalloc(x, w, N, K, w_dtype, out=None, stream=None):
    """hq_matmul_q on the library's static device scratch (no allocation inside the call)."""
    import torch
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    check(lib().hq_matmul_q_noalloc(_ptr(x), _ptr(w), _ptr(out), M, N, K, w_dtype, _stream(stream)))
    return out


NOALLOC_SCRATCH_BYTES = 64 << 20




def matmul_q_gated(x, wg, wu, N, K, w_dtype, act=ACT_SILU, out=None, ws=None, stream=None):
    """out (M, N) f32 = act(x @ dequant(wg)^T) * (x @ dequant(wu)^T)."""
    import torch
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_matmul_q_gated(_ptr(x), _ptr(wg), _ptr(wu), _ptr(out), M, N, K, w_dtype, act, _ptr(ws),
                                  ws_bytes, _stream(stream)))
    return out


def mlp_q(x, wg, wu, wd, H, I, w_dtype, act=ACT_SILU, out=None, ws=None, stream=None):
    """out (M, H) f32 = (act(x @ wg^T) * (x @ wu^T)) @ wd^T for GGUF weights wg, wu (I, H), wd (H, I)."""
    import torch
    M = x.shape[0]
    if out is None:
        out = torch.empty((M, H), dtype=torch.float32, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_mlp_q(_ptr(x), _ptr(wg), _ptr(wu), _ptr(wd), _ptr(out), M, H, I, w_dtype, act, _ptr(ws),
                         ws_bytes, _stream(stream)))
    return out


def mlp_q_ws_bytes(M, H, I, w_dtype):
    return lib().hq_mlp_q_ws_bytes(M, H, I, w_dtype)


def quantize_act(x, out=None, stream=None):
    """Prepared activations of x (M, K) (planar q8_1) for matmul_q_act."""
    import torch
    M, K = x.shape
    if out is None:
        out = torch.empty(lib().hq_act_bytes(M, K), dtype=torch.uint8, device=x.device)
    check(lib().hq_quantize_act(_ptr(x), _torch_dtype_code(x), _ptr(out), M, K, _stream(stream)))
    return out


def matmul_q_act(act, w, M, N, K, w_dtype, out=None, ws=None, stream=None):
    """out (M, N) f32 from prepared activations and GGUF weight bytes w."""
    import torch
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=w.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_matmul_q_act(_ptr(act), _ptr(w), _ptr(out), M, N, K, w_dtype, _ptr(ws), ws_bytes,
                                _stream(stream)))
    return out


def matmul_q_ws_bytes(M, N, K, w_dtype):
    return lib().hq_matmul_q_ws_bytes(M, N, K, w_dtype)


def matmul_q_gated_ws_bytes(M, N, K, w_dtype):
    return lib().hq_matmul_q_gated_ws_bytes(M, N, K, w_dtype)


def repack_q6k(w, N, K, out=None, stream=None):
    """The Q6_K_R copy (uint8, hq_repack_q6k_bytes(N, K)) of a Q6_K weight (N, K)."""
    import torch
    if out is None:
        out = torch.empty(lib().hq_repack_q6k_bytes(N, K), dtype=torch.uint8, device=w.device)
    check(lib().hq_repack_q6k(_ptr(w), _ptr(out), N, K, _stream(stream)))
    return out


def dequant_rows(src, N, K, src_dtype, out_dtype=F32, out=None, stream=None):
    """(N, K) F32 / BF16 of a weight in any hq_dequant format or Q6_K_R."""
    import torch
    if out is None:
        out = torch.empty((N, K), dtype=torch.float32 if out_dtype == F32 else torch.bfloat16, device=src.device)
    check(lib().hq_dequant_rows(_ptr(src), _ptr(out), N, K, src_dtype, out_dtype, _stream(stream)))
    return out


def dequant(src, n, src_dtype, out_dtype=F32, out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty(n, dtype=torch.float32 if out_dtype == F32 else torch.bfloat16, device=src.device)
    check(lib().hq_dequant(_ptr(src), _ptr(out), n, src_dtype, out_dtype, _stream(stream)))
    return out


def quantize_q8_1(x, out=None, stream=None):
    import torch
    M, K = x.shape
    if out is None:
        out = torch.empty(M * (K // 32) * 36, dtype=torch.uint8, device=x.device)
    check(lib().hq_quantize_q8_1(_ptr(x), _torch_dtype_code(x), _ptr(out), M, K, _stream(stream)))
    return out


def int4_matmul(x, codes, scales, zeros, G, out=None, ws=None, stream=None):
    """y (M, N) at x's dtype = x (M, K) @ W^T, W = s * (code - z) (quant.Int4 layout)."""
    import torch
    M, K = x.shape
    N = codes.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_int4_matmul(_ptr(x), _torch_dtype_code(x), _ptr(codes), _ptr(scales), _ptr(zeros), _ptr(out),
                               M, N, K, G, _ptr(ws), ws_bytes, _stream(stream)))
    return out


def int4_matmul_ws_bytes(M, N, K, G, x_dtype):
    return lib().hq_int4_matmul_ws_bytes(M, N, K, G, x_dtype)


def int4_dequant(codes, scales, zeros, G, out_dtype=F32, out=None, out_offset=0, stream=None):
    import torch
    N = codes.shape[0]
    K = codes.shape[1] * 8
    if out is None:
        out = torch.empty((N, K), dtype=torch.float32 if out_dtype == F32 else torch.bfloat16, device=codes.device)
    check(lib().hq_int4_dequant(_ptr(codes), _ptr(scales), _ptr(zeros), _ptr(out), out_dtype, N, K, G, out_offset,
                                _stream(stream)))
    return out


def int4_from_gptq(qweight, qzeros, scales, group, perm=None, v2=False, stream=None):
    """Canonical (codes U32 (N, K/8), scales, zeros F32 (N, K/G)) from GPTQ qweight (K/8, N) and
    qzeros (K/G, N/8) int32 tensors and F32 scales (K/G, N); perm: I64 (K) for act order."""
    import torch
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    G = K // group
    dev = qweight.device
    codes = torch.empty((N, K // 8), dtype=torch.int32, device=dev)
    so = torch.empty((N, G), dtype=torch.float32, device=dev)
    zo = torch.empty((N, G), dtype=torch.float32, device=dev)
    check(lib().hq_int4_from_gptq(_ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(perm) if perm is not None else None,
                                  K, N, group, 1 if v2 else 0, _ptr(codes), _ptr(so), _ptr(zo), _stream(stream)))
    return codes, so, zo


def int4_from_awq(qweight, qzeros, scales, group, stream=None):
    """Canonical (codes, scales, zeros) from AutoAWQ qweight (K, N/8), qzeros (K/G, N/8) int32
    tensors and F32 scales (K/G, N)."""
    import torch
    K, N = qweight.shape[0], qweight.shape[1] * 8
    G = K // group
    dev = qweight.device
    codes = torch.empty((N, K // 8), dtype=torch.int32, device=dev)
    so = torch.empty((N, G), dtype=torch.float32, device=dev)
    zo = torch.empty((N, G), dtype=torch.float32, device=dev)
    check(lib().hq_int4_from_awq(_ptr(qweight), _ptr(qzeros), _ptr(scales), K, N, group, _ptr(codes), _ptr(so),
                                 _ptr(zo), _stream(stream)))
    return codes, so, zo


def moe_gemm_q(x, w, sorted_pairs, sorted_expts, E, N, K, w_dtype, topk, topk_w=None, out=None, counts=None,
               offsets=None, ws=None, stream=None):
    """Grouped expert qmatmul with Light's MoEGemmQ contract (ops/moe.go:242-265)."""
    import torch
    M = sorted_pairs.numel()
    rows = x.shape[0]
    if rows == M:
        rpp = 1
    elif rows == M // topk:
        rpp = 0
    else:
        raise HipqError(HQ_EINVAL, f"moe_gemm_q: input rows {rows} must be M={M} or M/topk={M // topk}")
    dev = x.device
    if counts is None:
        counts = torch.zeros(E, dtype=torch.int32, device=dev)
    if offsets is None:
        offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    if out is None:
        out = torch.zeros((M, N), dtype=torch.float32, device=dev)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_gemm_q(_ptr(x), _ptr(w), _ptr(sorted_pairs), _ptr(sorted_expts), _ptr(counts),
                              _ptr(offsets), _ptr(topk_w), _ptr(out), topk, out.shape[0], M, rows, E, N, K, rpp,
                              w_dtype, _ptr(ws), ws_bytes, _stream(stream)))
    return out


def moe_combine(pair_out, topk, out=None, stream=None):
    """(M, N) pair rows -> (M/topk, N): slot rows summed in slot order."""
    import torch
    M, N = pair_out.shape
    if out is None:
        out = torch.empty((M // topk, N), dtype=torch.float32, device=pair_out.device)
    check(lib().hq_moe_combine(_ptr(pair_out), _ptr(out), M, N, topk, _stream(stream)))
    return out


def moe_gemm_q_combine(h, w, sorted_pairs, sorted_expts, E, N, K, w_dtype, topk, topk_w=None, out=None,
                       counts=None, offsets=None, ws=None, stream=None):
    """y (T, N) = MoECombine(MoEGemmQ(h, w, routing, topk_w), topk), h per pair (T*topk, K)."""
    import torch
    M = sorted_pairs.numel()
    T = M // topk
    if out is None:
        out = torch.empty((T, N), dtype=torch.float32, device=h.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_gemm_q_combine(_ptr(h), _ptr(w), _ptr(sorted_pairs), _ptr(sorted_expts), _ptr(counts),
                                      _ptr(offsets), _ptr(topk_w), _ptr(out), topk, T, E, N, K, w_dtype, _ptr(ws),
                                      ws_bytes, _stream(stream)))
    return out


def moe_route_gated(probs, x, w, E, I, K, w_dtype, topk, normalize=True, act=ACT_SILU, h=None, counts=None,
                    offsets=None, ws=None, stream=None):
    """MoERoute + the routed gated gate/up: (topk_ids, weights, sorted_pairs, sorted_expts, h (T*topk, I))."""
    import torch
    T = probs.shape[0]
    dev = probs.device
    M = T * topk
    ids = torch.empty((T, topk), dtype=torch.int64, device=dev)
    wt = torch.empty(M, dtype=torch.float32, device=dev)
    sp = torch.empty(M, dtype=torch.int64, device=dev)
    se = torch.empty(M, dtype=torch.int64, device=dev)
    if h is None:
        h = torch.zeros((M, I), dtype=torch.float32, device=dev)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_route_gated(_ptr(probs), _ptr(x), _ptr(w), _ptr(h), T, E, topk, int(bool(normalize)), I, K,
                                   w_dtype, act, _ptr(ids), _ptr(wt), _ptr(sp), _ptr(se), _ptr(counts),
                                   _ptr(offsets), _ptr(ws), ws_bytes, _stream(stream)))
    return ids, wt, sp, se, h


def moe_block_q(probs, x, w_gate_up, w_down, E, H, I, w_dtype, topk, normalize=True, act=ACT_SILU, out=None, h=None,
                counts=None, offsets=None, ws=None, stream=None):
    """The SparseMoE decode block: (y (T, H), topk_ids, weights, sorted_pairs, sorted_expts, h)."""
    import torch
    T = probs.shape[0]
    dev = probs.device
    M = T * topk
    ids = torch.empty((T, topk), dtype=torch.int64, device=dev)
    wt = torch.empty(M, dtype=torch.float32, device=dev)
    sp = torch.empty(M, dtype=torch.int64, device=dev)
    se = torch.empty(M, dtype=torch.int64, device=dev)
    if h is None:
        h = torch.zeros((M, I), dtype=torch.float32, device=dev)
    if out is None:
        out = torch.empty((T, H), dtype=torch.float32, device=dev)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_block_q(_ptr(probs), _ptr(x), _ptr(w_gate_up), _ptr(w_down), _ptr(h), _ptr(out), T, E, topk,
                               int(bool(normalize)), H, I, w_dtype, act, _ptr(ids), _ptr(wt), _ptr(sp), _ptr(se),
                               _ptr(counts), _ptr(offsets), _ptr(ws), ws_bytes, _stream(stream)))
    return out, ids, wt, sp, se, h


def moe_block_q_check(stream=None):
    """Synchronize the stream; raise HipqError(HQ_EBARRIER) if a one-launch MoE block on the
    current device gave up at its grid barrier since the last report."""
    check(lib().hq_moe_block_q_check(_stream(stream)))


def debug_moe_block_spin_limit(limit=1 << 22):
    """Test hook: polls before the one-launch block's barrier gives up (0: at once); also
    re-enables the one launch after a reported failure."""
    lib().hq_debug_moe_block_spin_limit(int(limit))


def moe_int4(x, gate_up, down, topk_ids, weights, topk, G, act=ACT_SILU, out=None, ws=None, stream=None):
    """ops.MoEInt4: x (T, H); gate_up / down: lists of E (codes, scales, zeros) device tensors
    (gate-up (2I, H/8) codes, down (H, I/8)); topk_ids I64 / weights F32 (T*topk)."""
    import torch
    T, H = x.shape
    E = len(gate_up)
    I = down[0][0].shape[1] * 8
    tab = torch.tensor([t.data_ptr() for part in range(3) for t in (gu[part] for gu in gate_up)] +
                       [t.data_ptr() for part in range(3) for t in (dn[part] for dn in down)],
                       dtype=torch.int64).to(x.device)
    xdt = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}[x.dtype]
    if out is None:
        out = torch.empty((T, H), dtype=x.dtype, device=x.device)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_int4(_ptr(x), xdt, _ptr(tab), E, _ptr(topk_ids), _ptr(weights), _ptr(out), T, topk, H, I, G,
                            act, _ptr(ws), ws_bytes, _stream(stream)))
    return out


def moe_route(probs, topk, normalize=True, counts=None, offsets=None, stream=None):
    """ops.MoERoute on the device: (topk_ids (T, topk) I64, weights (T*topk,) F32,
    sorted_pairs, sorted_expts (T*topk,) I64); counts / offsets filled when given."""
    import torch
    T, E = probs.shape
    dev = probs.device
    ids = torch.empty((T, topk), dtype=torch.int64, device=dev)
    w = torch.empty(T * topk, dtype=torch.float32, device=dev)
    sp = torch.empty(T * topk, dtype=torch.int64, device=dev)
    se = torch.empty(T * topk, dtype=torch.int64, device=dev)
    check(lib().hq_moe_route(_ptr(probs), T, E, topk, int(bool(normalize)), _ptr(ids), _ptr(w), _ptr(sp), _ptr(se),
                             _ptr(counts), _ptr(offsets), _stream(stream)))
    return ids, w, sp, se


def moe_sort_ids(ids, E, counts=None, offsets=None, stream=None):
    """Stable ascending expert sort of flat ids on the device: (sorted_pairs, sorted_expts)."""
    import torch
    M = ids.numel()
    sp = torch.empty(M, dtype=torch.int64, device=ids.device)
    se = torch.empty(M, dtype=torch.int64, device=ids.device)
    check(lib().hq_moe_sort_ids(_ptr(ids), M, E, _ptr(sp), _ptr(se), _ptr(counts), _ptr(offsets), _stream(stream)))
    return sp, se


def moe_gemm_q_gated(x, w, sorted_pairs, sorted_expts, E, I, K, w_dtype, topk, act=ACT_SILU, out=None,
                     counts=None, offsets=None, ws=None, stream=None):
    """Routed gated gate/up: w (E, 2I, K) quantized -> h (M, I) = act(g) * u."""
    import torch
    M = sorted_pairs.numel()
    rows = x.shape[0]
    rpp = 1 if rows == M else 0
    dev = x.device
    if counts is None:
        counts = torch.zeros(E, dtype=torch.int32, device=dev)
    if offsets is None:
        offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    if out is None:
        out = torch.zeros((M, I), dtype=torch.float32, device=dev)
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().hq_moe_gemm_q_gated(_ptr(x), _ptr(w), _ptr(sorted_pairs), _ptr(sorted_expts), _ptr(counts),
                                    _ptr(offsets), _ptr(out), topk, out.shape[0], M, rows, E, I, K, rpp, w_dtype, act,
                                    _ptr(ws), ws_bytes, _stream(stream)))
    return out


def moe_gemm_q_gated_ws_bytes(size_m, rows, I, K, w_dtype):
    return lib().hq_moe_gemm_q_gated_ws_bytes(size_m, rows, I, K, w_dtype)


def moe_gemm_q_ws_bytes(rows, K, w_dtype):
    return lib().hq_moe_gemm_q_ws_bytes(rows, K, w_dtype)


def trace_start():
    check(lib().hq_trace_start())


def trace_stop(n_max=32):
    names = ctypes.create_string_buffer(32 * n_max)
    calls = (_I * n_max)()
    us = (ctypes.c_double * n_max)()
    n = lib().hq_trace_stop(names, calls, us, n_max)
    if n < 0:
        raise HipqError(n, last_error())
    out = {}
    for i in range(n):
        nm = names.raw[32 * i:32 * (i + 1)].split(b"\0", 1)[0].decode()
        out[nm] = (calls[i], us[i])
    return out
