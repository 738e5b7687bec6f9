"""The GGUF byte path (light_amd/host/gguf.cpp) on CPU tensors.

Mirrors Light's gguf tests:
  * gguf/gguf_test.go:26-190 -- scalar/array metadata round trip, an F32 tensor, a Q4_0
    tensor whose bytes dequantize to scale * q, bad magic, a missing tensor, the empty file;
  * gguf/validate_test.go:47-127 -- the twelve malformed headers rejected at Open for both a
    sized and an unsized input, tensor data past the end of a sized input, the sized round
    trip;
plus TensorRowMajor's dim reversal (gguf/reader.go:240-265) and the MoE expert loader's
byte-level gate/up fusion (models/llama_gguf.go:173-206).
"""
import struct

import numpy as np
import pytest

import oracle
from _gguf import ARR, BOOL, F32, I64, STR, U8, U32, U64, Writer, gstr, stream, tensor_info
from light_amd import _light as L
from light_amd import synth

U64MAX = 2**64 - 1
I64MAX = 2**63 - 1


def f32b(*vs):
    return np.asarray(vs, "<f4").tobytes()


def q4_0_block(scale, vals):
    """gguf_test.go:174-186: f16 scale, then the low nibble of byte j = vals[j] + 8, high = vals[j+16] + 8."""
    b = struct.pack("<H", int(oracle.half_from_f32(np.float32(scale))))
    return b + bytes(((vals[j] + 8) & 15) | (((vals[j + 16] + 8) & 15) << 4) for j in range(16))


def test_round_trip_scalar():
    w = Writer()
    w.add("general.name", STR, "toy-model")
    w.add("general.architecture_version", U32, 1)
    w.add("block_count", I64, 4)
    w.add("rope_theta", F32, 10000.0)
    w.add("is_quantized", BOOL, True)
    w.add("tokenizer.tokens", ARR, (STR, ["hello", "world"]))
    vals = [1, 2, 3, 4, 5, 6]
    w.add_tensor("weight", [2, 3], 0, f32b(*vals))
    f = L.gguf_open_bytes(w.bytes())
    assert f.version == 3
    assert f.string("general.name") == "toy-model"
    assert f.int64("block_count") == 4
    assert f.int64("general.architecture_version") == 1
    assert f.float64("rope_theta") == 10000.0
    assert f.string("block_count") is None and f.int64("general.name") is None
    m = f.meta
    assert m["is_quantized"] is True
    assert m["tokenizer.tokens"] == ["hello", "world"]
    assert f.key_order == ["general.name", "general.architecture_version", "block_count", "rope_theta",
                           "is_quantized", "tokenizer.tokens", "general.alignment"]
    t = f.load_tensor("weight")
    assert t.dtype == "F32" and t.shape == [2, 3]
    assert t.numpy().ravel().tolist() == vals


def test_every_value_type():
    w = Writer()
    cases = [(0, 200), (1, -100), (2, 60000), (3, -30000), (4, 4_000_000_000), (5, -2_000_000_000), (6, 1.5),
             (7, False), (8, "sé"), (10, 2**63 + 5), (11, -(2**40)), (12, 0.1)]
    for t, v in cases:
        w.add(f"k{t}", t, v)
    w.add("nested", ARR, (ARR, [(U8, [1, 2]), (STR, ["a"])]))
    m = L.gguf_open_bytes(w.bytes()).meta
    for t, v in cases:
        assert m[f"k{t}"] == v, t
    assert m["nested"] == [[1, 2], ["a"]]


def test_quant_tensor_loads_and_dequantizes():
    vals = [(i % 16) - 8 for i in range(32)]
    block = q4_0_block(0.5, vals)
    w = Writer()
    w.add("general.name", STR, "q4-test")
    w.add_tensor("w", [32], 2, block)
    f = L.gguf_open_bytes(w.bytes())
    t = f.load_tensor("w")
    assert t.dtype == "Q4_0" and t.shape == [32]
    raw = t.numpy()
    assert raw.tobytes() == block == f.tensor_bytes("w")
    got = oracle.dequant(oracle.Q4_0, raw, 32)
    np.testing.assert_array_equal(got, np.float32(0.5) * np.asarray(vals, np.float32))


def test_bad_magic():
    with pytest.raises(L.Error, match="bad magic"):
        L.gguf_open_bytes(bytes(32))


def test_bad_version():
    w = Writer(version=1)
    with pytest.raises(L.Error, match=r"version 1 not in \[2, 3\]"):
        L.gguf_open_bytes(w.bytes())
    assert L.gguf_open_bytes(Writer(version=2).bytes()).version == 2


def test_tensor_missing():
    f = L.gguf_open_bytes(Writer().bytes())
    with pytest.raises(L.Error, match='tensor "nope" not found'):
        f.load_tensor("nope")


def test_empty_file():
    f = L.gguf_open_bytes(Writer().bytes())
    assert f.order == []
    assert list(f.meta) == ["general.alignment"] and f.meta["general.alignment"] == 32


def _array_kv(elem, n):
    return gstr("k") + struct.pack("<IIQ", ARR, elem, n)


def _nested():
    b = gstr("deep") + struct.pack("<I", ARR)
    for _ in range(100):
        b += struct.pack("<IQ", ARR, 1)
    return b


MALFORMED = {
    "array count MaxUint64": stream(0, 1, _array_kv(U8, U64MAX)),
    "array of u64 too long": stream(0, 1, _array_kv(U64, 4) + bytes(16)),
    "array of arrays too big": stream(0, 1, _array_kv(ARR, 1 << 40)),
    "kv count MaxUint64": stream(0, U64MAX),
    "tensor count MaxUint64": stream(U64MAX, 0),
    "deep nesting": stream(0, 1, _nested()),
    "huge rank": stream(1, 0, gstr("t") + struct.pack("<I", 2**32 - 1)),
    "dims product overflow": stream(1, 0, tensor_info("t", [1 << 32, 1 << 32], 0)),
    "byte size overflow": stream(1, 0, tensor_info("t", [1 << 62], 0)),
    "offset overflow": stream(1, 0, tensor_info("t", [1], U64MAX - 2)),
    "offset near MaxInt64": stream(1, 0, tensor_info("t", [4], I64MAX - 8)),
    "string length too big": stream(0, 1, struct.pack("<Q", 1 << 29)),
}


@pytest.mark.parametrize("name", sorted(MALFORMED))
@pytest.mark.parametrize("sized", [True, False])
def test_malformed_rejected(name, sized):
    with pytest.raises(L.Error, match="^gguf: "):
        L.gguf_open_bytes(MALFORMED[name], sized)


def test_data_past_end():
    with pytest.raises(L.Error, match="past end"):
        L.gguf_open_bytes(stream(1, 0, tensor_info("t", [1000], 0)))


def test_truncated_inputs_never_crash():
    """Every prefix of a valid file either opens or raises gguf's Error."""
    w = Writer()
    w.add("tokenizer.tokens", ARR, (STR, ["a", "bb", "ccc"]))
    w.add_tensor("a", [8], 0, f32b(*range(8)))
    data = w.bytes()
    for n in range(len(data)):
        for sized in (True, False):
            try:
                L.gguf_open_bytes(data[:n], sized)
            except L.Error:
                pass


def test_sized_round_trip():
    w = Writer()
    w.add("general.name", STR, "toy")
    w.add_tensor("a", [3], 0, f32b(1, 2, 3))
    w.add_tensor("b", [2], 0, f32b(4, 5))
    data = w.bytes()
    for sized in (True, False):
        f = L.gguf_open_bytes(data, sized)
        assert f.order == ["a", "b"]
        assert f.load_tensor("b").numpy().tolist() == [4, 5]
        assert f.info("b").offset == 32 and f.info("b").bytes == 8


def test_alignment_key_moves_data():
    w = Writer()
    w.set_alignment(64)
    w.add("general.alignment", U32, 64)
    w.add_tensor("a", [3], 0, f32b(1, 2, 3))
    w.add_tensor("b", [2], 0, f32b(4, 5))
    f = L.gguf_open_bytes(w.bytes())
    assert f.data_base % 64 == 0 and f.info("b").offset == 64
    assert f.load_tensor("b").numpy().tolist() == [4, 5]


def test_open_file(tmp_path):
    w = Writer()
    w.add_tensor("a", [3], 0, f32b(7, 8, 9))
    p = tmp_path / "m.gguf"
    p.write_bytes(w.bytes())
    f = L.gguf_open(str(p))
    assert f.load_tensor("a").numpy().tolist() == [7, 8, 9]


def test_tensor_row_major():
    """A Linear weight stored [in, out] (ne0 = in) loads as (out, in), bytes unchanged."""
    g = synth.rng(3)
    N, K = 8, 512
    raw = synth.gguf_weight(oracle.Q4_K, N, K, g)
    w = Writer()
    w.add_tensor("blk.0.attn_q.weight", [K, N], 12, raw.tobytes())
    f = L.gguf_open_bytes(w.bytes())
    assert f.info("blk.0.attn_q.weight").dims == [K, N]
    t = f.tensor_row_major("blk.0.attn_q.weight")
    assert t.dtype == "Q4_K" and t.shape == [N, K]
    assert t.numpy().tobytes() == raw.tobytes()
    assert f.load_tensor("blk.0.attn_q.weight").shape == [K, N]


def test_load_experts_fuses_gate_up():
    g = synth.rng(5)
    E, I, H = 4, 256, 512
    gate = synth.gguf_weight(oracle.Q4_K, E * I, H, g)
    up = synth.gguf_weight(oracle.Q4_K, E * I, H, g)
    down = synth.gguf_weight(oracle.Q6_K, E * H, I, g)
    w = Writer()
    w.add_tensor("blk.0.ffn_gate_exps.weight", [H, I, E], 12, gate.tobytes())
    w.add_tensor("blk.0.ffn_up_exps.weight", [H, I, E], 12, up.tobytes())
    w.add_tensor("blk.0.ffn_down_exps.weight", [I, H, E], 14, down.tobytes())
    f = L.gguf_open_bytes(w.bytes())
    gu, dn = L.gguf_load_experts(f, "blk.0.")
    assert gu.dtype == "Q4_K" and gu.shape == [E, 2 * I, H]
    assert dn.dtype == "Q6_K" and dn.shape == [E, H, I]
    slab = gate.nbytes // E
    want = b"".join(gate.tobytes()[e * slab:(e + 1) * slab] + up.tobytes()[e * slab:(e + 1) * slab]
                    for e in range(E))
    assert gu.numpy().tobytes() == want
    assert dn.numpy().tobytes() == down.tobytes()


@pytest.mark.parametrize("dt,code", [("F16", 1), ("BF16", 30)])
def test_load_experts_widens_half(dt, code):
    g = np.random.default_rng(7)
    E, I, H = 2, 3, 4
    vals = g.standard_normal((3, E, I, H)).astype(np.float32)
    if dt == "F16":
        bits = vals.astype(np.float16)
        want = bits.astype(np.float32)
        raw = bits.view(np.uint16)
    else:
        raw = (vals.view(np.uint32) >> 16).astype(np.uint16)
        want = (raw.astype(np.uint32) << 16).view(np.float32)
    w = Writer()
    w.add_tensor("p.ffn_gate_exps.weight", [H, I, E], code, raw[0].tobytes())
    w.add_tensor("p.ffn_up_exps.weight", [H, I, E], code, raw[1].tobytes())
    w.add_tensor("p.ffn_down_exps.weight", [I, H, E], code, raw[2].tobytes())
    f = L.gguf_open_bytes(w.bytes())
    gu, dn = L.gguf_load_experts(f, "p.")
    assert gu.dtype == "F32" and dn.dtype == "F32"
    np.testing.assert_array_equal(gu.numpy(), np.concatenate([want[0], want[1]], axis=1))
    assert dn.shape == [E, H, I]
    np.testing.assert_array_equal(dn.numpy().ravel(), want[2].ravel())


def test_load_experts_errors():
    w = Writer()
    with pytest.raises(L.Error, match="p.ffn_gate_exps.weight missing"):
        L.gguf_load_experts(L.gguf_open_bytes(w.bytes()), "p.")
    w.add_tensor("p.ffn_gate_exps.weight", [2, 2, 2], 0, f32b(*range(8)))
    with pytest.raises(L.Error, match="p.ffn_up_exps.weight missing or mismatched"):
        L.gguf_load_experts(L.gguf_open_bytes(w.bytes()), "p.")
    w.add_tensor("p.ffn_up_exps.weight", [2, 2, 2], 1, bytes(16))
    with pytest.raises(L.Error, match="missing or mismatched"):
        L.gguf_load_experts(L.gguf_open_bytes(w.bytes()), "p.")


def test_ggml_type_codes():
    """ggml type codes (gguf/types.go:61-156) for every format on the path."""
    want = {0: "F32", 1: "F16", 2: "Q4_0", 6: "Q5_0", 8: "Q8_0", 9: "Q8_1", 12: "Q4_K", 13: "Q5_K",
            14: "Q6_K", 30: "BF16"}
    for code, name in want.items():
        assert L.dtype_from_ggml(code) == name
    with pytest.raises(L.Error, match="unsupported ggml type 99"):
        L.dtype_from_ggml(99)


def test_unsized_lying_size_is_an_error_not_an_allocation():
    """On an unsized input a tensor may claim more data than exists; loading it fails as the
    short read of gguf/reader.go:254-264 before anything of the claimed size is allocated."""
    w = Writer()
    w.add_tensor("t", [1 << 44], 0, f32b(1, 2))  # 64 TiB claimed, 8 bytes present
    f = L.gguf_open_bytes(w.bytes(), False)
    for load in (f.load_tensor, f.tensor_row_major, f.tensor_bytes):
        with pytest.raises(L.Error, match="read tensor"):
            load("t")


def test_non_utf8_names_round_trip():
    """GGUF strings are bytes (Go strings): a name that is not UTF-8 is listed and loads."""
    w = Writer()
    name = b"blk.\xff\x80.w"
    w.add_tensor(name, [2], 0, f32b(3, 4))
    f = L.gguf_open_bytes(w.bytes())
    (listed,) = f.order
    assert listed.encode("utf-8", "surrogateescape") == name
    assert f.load_tensor(listed).numpy().tolist() == [3, 4]
    assert f.load_tensor(name).numpy().tolist() == [3, 4]
    assert f.info(listed).name == listed


_FUZZ = r"""
import random, resource, sys
resource.setrlimit(resource.RLIMIT_AS, (4 << 30, 4 << 30))
import numpy as np
from _gguf import ARR, STR, U32, Writer
from light_amd import _light as L
w = Writer()
w.add("general.name", STR, "toy")
w.add("tokenizer.tokens", ARR, (STR, ["a", "bb", "ccc"]))
w.add("n", U32, 7)
w.add_tensor("a", [8], 0, np.arange(8, dtype="<f4").tobytes())
w.add_tensor("b", [32, 2], 2, bytes(range(36)))
w.add_tensor("c", [4], 1, np.arange(4, dtype="<f2").tobytes())
data = bytearray(w.bytes())
rng = random.Random(int(sys.argv[1]))
for it in range(int(sys.argv[2])):
    d = bytearray(data)
    for _ in range(rng.choice((1, 1, 2, 4, 8))):
        i = rng.randrange(len(d)) if rng.random() < 0.5 else rng.randrange(min(len(d), 160))
        d[i] = rng.choice((0, 0xFF, 0x7F, 0x80, rng.randrange(256)))
    for sized in (True, False):
        try:
            f = L.gguf_open_bytes(bytes(d), sized)
        except L.Error:
            continue
        for n in f.order:
            f.info(n)
            try:
                f.load_tensor(n)
            except L.Error:
                pass
print("done")
"""


@pytest.mark.parametrize("seed", [1, 2])
def test_mutated_inputs_never_crash(seed):
    """Random byte mutations of a valid file (header, metadata, tensor table, data): every one
    opens or raises gguf's Error, and every listed tensor loads or raises it -- no crash, no
    other exception and no allocation beyond a 4 GiB address-space cap (run in a child)."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([here, os.path.dirname(here), os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", _FUZZ, str(seed), "5000"], capture_output=True, text=True, env=env,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "done", r.stderr[-2000:]
