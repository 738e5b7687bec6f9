"""A GGUF v3 byte-stream builder for the tests, following the file layout Light's test writer
emits (gguf/writer.go:103-165): header (magic, version, tensor count, KV count), KV entries
(general.alignment appended last unless set), tensor infos with data offsets rounded up to
the alignment, zero padding to the alignment, then the payloads at their offsets."""
import struct

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", U64: "<Q", I64: "<q",
        F64: "<d"}


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t, v):
    if t in _FMT:
        return struct.pack(_FMT[t], v)
    if t == BOOL:
        return b"\x01" if v else b"\x00"
    if t == STR:
        return gstr(v)
    if t == ARR:
        elem, vals = v
        return struct.pack("<IQ", elem, len(vals)) + b"".join(value(elem, e) for e in vals)
    raise ValueError(f"unsupported value type {t}")


class Writer:
    def __init__(self, version=3, align=32):
        self.version, self.align, self.align_set = version, align, False
        self.meta, self.tensors = [], []

    def set_alignment(self, n):
        self.align, self.align_set = n, True

    def add(self, key, t, v):
        self.meta.append((key, t, v))

    def add_tensor(self, name, dims, ggml_type, data):
        self.tensors.append((name, [int(d) for d in dims], ggml_type, bytes(data)))

    def bytes(self):
        meta = list(self.meta)
        if not self.align_set:
            meta.append(("general.alignment", U32, self.align))
        head = struct.pack("<IIQQ", MAGIC, self.version, len(self.tensors), len(meta))
        for k, t, v in meta:
            head += gstr(k) + struct.pack("<I", t) + value(t, v)
        offs, cur = [], 0
        for _, _, _, data in self.tensors:
            cur = -(-cur // self.align) * self.align
            offs.append(cur)
            cur += len(data)
        for (name, dims, dt, _), off in zip(self.tensors, offs):
            head += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", dt, off)
        head += b"\x00" * (-len(head) % self.align)
        body = bytearray()
        for (_, _, _, data), off in zip(self.tensors, offs):
            body += b"\x00" * (off - len(body))
            body += data
        return head + bytes(body)


def stream(n_tensors, n_kv, body=b""):
    """A v3 header with the given counts followed by body (validate_test.go:22-29)."""
    return struct.pack("<IIQQ", MAGIC, 3, n_tensors, n_kv) + body


def tensor_info(name, dims, off, ggml_type=0):
    return gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ggml_type, off)
