"""Writes the golden dequant fixtures from Light's known-answer tests.

The fixtures restate, as data, the hand-built blocks and closed-form expected
values of quant/q4_k_test.go (TestDequantQ4_K :48-87, TestDequantQ4_KMultiBlock
:89-127), quant/q6_k_test.go (TestDequantQ6_K :61-85,
TestDequantQ6_KKnownValues :87-120, TestDequantQ6_KNegativeScale :122-147),
quant/q4_0_test.go (TestDequantQ4_0Basic :44-84, TestDequantQ4_0MultipleBlocks
:86-111), quant/q5_k_test.go (TestDequantQ5_K :63-102, TestDequantQ5_KFifthBit
:104-130) and quant/others_test.go (TestDequantQ8_0 :30-50, TestDequantQ5_0
:105-124).  Blocks are packed with the reference's own builder rules
(buildQ4_KBlock :20-46, buildQ6_KBlock :20-59, buildQ4_0Block :16-29,
buildQ5_KBlock :13-61, buildQ8_0Block / buildQ5_0Block in others_test.go),
restated here; expected values are the tests' closed forms, not outputs of the
oracle.  Where a test states its scale in f32 (0.1, 0.25) the expected value
uses the f16-rounded scale the block stores, times the integer quant: exact in
f32, so the comparison is bit for bit.  Run: python tests/golden/make_golden.py
"""
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def half_bits(v):
    return int(np.float32(v).astype(np.float16).view(np.uint16))


def build_q4_k(d, dmin, sub_scales, sub_mins, quants):
    buf = bytearray(144)
    buf[0:2] = struct.pack("<H", half_bits(d))
    buf[2:4] = struct.pack("<H", half_bits(dmin))
    for j in range(4):
        buf[4 + j] = (sub_scales[j] & 0x3F) | ((sub_scales[j + 4] & 0x30) << 2)
        buf[8 + j] = (sub_mins[j] & 0x3F) | ((sub_mins[j + 4] & 0x30) << 2)
        buf[12 + j] = (sub_scales[j + 4] & 0x0F) | ((sub_mins[j + 4] & 0x0F) << 4)
    for p in range(4):
        for l in range(32):
            buf[16 + p * 32 + l] = (quants[p * 64 + l] & 0x0F) | ((quants[p * 64 + 32 + l] & 0x0F) << 4)
    return bytes(buf)


def build_q6_k(d, scales, raw):
    ql, qh = bytearray(128), bytearray(64)
    for half in range(2):
        for l in range(32):
            y = half * 128
            r1, r2, r3, r4 = (raw[y + l] & 0x3F, raw[y + l + 32] & 0x3F, raw[y + l + 64] & 0x3F,
                              raw[y + l + 96] & 0x3F)
            ql[half * 64 + l] = (r1 & 0x0F) | ((r3 & 0x0F) << 4)
            ql[half * 64 + l + 32] = (r2 & 0x0F) | ((r4 & 0x0F) << 4)
            qh[half * 32 + l] = ((r1 >> 4) & 3) | (((r2 >> 4) & 3) << 2) | (((r3 >> 4) & 3) << 4) | (
                ((r4 >> 4) & 3) << 6)
    return bytes(ql) + bytes(qh) + bytes((s & 0xFF) for s in scales) + struct.pack("<H", half_bits(d))


def cases():
    out = []
    # TestDequantQ4_K: sc_j = j+1, m_j = j, q = (j+1)&15 on sub-block j, d = dmin = 1: y = sc*q - m.
    sc = [j + 1 for j in range(8)]
    mn = [j for j in range(8)]
    q = [((i // 32) + 1) & 0x0F for i in range(256)]
    want = [sc[i // 32] * (sc[i // 32] & 0x0F) - mn[i // 32] for i in range(256)]
    out.append(dict(name="q4_k_known", dtype="Q4_K", n=256, blocks=build_q4_k(1.0, 1.0, sc, mn, q).hex(),
                    want=want, checks="all"))
    # TestDequantQ4_KMultiBlock: two blocks; element 7*32 of each: -1.75 and -7.
    sc = [2 * j for j in range(8)]
    mn = [j for j in range(8)]
    q = [i % 16 for i in range(256)]
    blocks = build_q4_k(0.5, 0.25, sc, mn, q) + build_q4_k(2.0, 1.0, sc, mn, q)
    out.append(dict(name="q4_k_multiblock", dtype="Q4_K", n=512, blocks=blocks.hex(),
                    want={str(7 * 32): -1.75, str(256 + 7 * 32): -7.0}, checks="indexed"))
    # TestDequantQ6_K: raw = 32 everywhere -> 0.
    out.append(dict(name="q6_k_zero", dtype="Q6_K", n=256,
                    blocks=build_q6_k(0.5, [i + 1 for i in range(16)], [32] * 256).hex(), want=[0.0] * 256,
                    checks="all"))
    # TestDequantQ6_KKnownValues: scale 1, d 1, sub-block s holds q = s.
    raw = [(i // 16) + 32 for i in range(256)]
    out.append(dict(name="q6_k_known", dtype="Q6_K", n=256, blocks=build_q6_k(1.0, [1] * 16, raw).hex(),
                    want=[float(i // 16) for i in range(256)], checks="all"))
    # TestDequantQ6_KNegativeScale: scale -3, raw 40 (q = 8), d 0.25 -> -6.
    out.append(dict(name="q6_k_negative_scale", dtype="Q6_K", n=256, blocks=build_q6_k(0.25, [-3] * 16, [40] * 256).hex(),
                    want=[-6.0] * 256, checks="all"))
    # TestDequantQ4_0Basic: d = 0.5, values -8..7 twice.
    vals = [i - 8 for i in range(16)] * 2
    out.append(dict(name="q4_0_basic", dtype="Q4_0", n=32, blocks=build_q4_0(0.5, vals).hex(),
                    want=[0.5 * v for v in vals], checks="all"))
    # TestDequantQ4_0MultipleBlocks: (2.0, all 1) and (3.0, all -2).
    blocks = build_q4_0(2.0, [1] * 32) + build_q4_0(3.0, [-2] * 32)
    out.append(dict(name="q4_0_multiblock", dtype="Q4_0", n=64, blocks=blocks.hex(),
                    want=[2.0] * 32 + [-6.0] * 32, checks="all"))
    # TestDequantQ8_0: d = 0.25, values -16..15.
    vals = [i - 16 for i in range(32)]
    out.append(dict(name="q8_0_others", dtype="Q8_0", n=32, blocks=build_q8_0(0.25, vals).hex(),
                    want=[0.25 * v for v in vals], checks="all"))
    # TestDequantQ5_0: d = f16(0.1), values -16..15.
    d = f16_value(0.1)
    out.append(dict(name="q5_0_others", dtype="Q5_0", n=32, blocks=build_q5_0(0.1, vals).hex(),
                    want=[float(np.float32(d) * np.float32(v)) for v in vals], checks="all"))
    # TestDequantQ5_K: d = dmin = 1, sc_j = j+1, m_j = j, q5 = j+1 on sub-block j.
    sc = [j + 1 for j in range(8)]
    mn = [j for j in range(8)]
    q5 = [(i // 32) + 1 for i in range(256)]
    out.append(dict(name="q5_k_known", dtype="Q5_K", n=256, blocks=build_q5_k(1.0, 1.0, sc, mn, q5).hex(),
                    want=[float(sc[i // 32] * q5[i] - mn[i // 32]) for i in range(256)], checks="all"))
    # TestDequantQ5_KFifthBit: every q5 = 17, scale 2, min 0 -> 34.
    out.append(dict(name="q5_k_fifth_bit", dtype="Q5_K", n=256,
                    blocks=build_q5_k(1.0, 1.0, [2] * 8, [0] * 8, [17] * 256).hex(), want=[34.0] * 256,
                    checks="all"))
    return out


def f16_value(v):
    return float(np.float32(v).astype(np.float16))


def build_q4_0(d, values):
    buf = bytearray(18)
    buf[0:2] = struct.pack("<H", half_bits(d))
    for j in range(16):
        buf[2 + j] = ((values[j] + 8) & 0x0F) | (((values[j + 16] + 8) & 0x0F) << 4)
    return bytes(buf)


def build_q8_0(d, values):
    return struct.pack("<H", half_bits(d)) + bytes(v & 0xFF for v in values)


def build_q5_0(d, values):
    buf = bytearray(22)
    buf[0:2] = struct.pack("<H", half_bits(d))
    qh = 0
    for j in range(16):
        r0, r1 = values[j] + 16, values[j + 16] + 16
        qh |= ((r0 >> 4) & 1) << j
        qh |= ((r1 >> 4) & 1) << (j + 16)
        buf[6 + j] = (r0 & 0x0F) | ((r1 & 0x0F) << 4)
    buf[2:6] = struct.pack("<I", qh)
    return bytes(buf)


def build_q5_k(d, dmin, sub_scales, sub_mins, q5):
    q4 = build_q4_k(d, dmin, sub_scales, sub_mins, [q & 0x0F for q in q5])
    qh = bytearray(32)
    for p in range(4):
        for l in range(32):
            if q5[p * 64 + l] & 0x10:
                qh[l] |= 1 << (2 * p)
            if q5[p * 64 + 32 + l] & 0x10:
                qh[l] |= 1 << (2 * p + 1)
    return q4[:16] + bytes(qh) + q4[16:]


if __name__ == "__main__":
    with open(os.path.join(HERE, "dequant_kat.json"), "w") as f:
        json.dump({"source": "sushvibez/light quant/q4_k_test.go, quant/q6_k_test.go, quant/q4_0_test.go, quant/q5_k_test.go, quant/others_test.go", "cases": cases()}, f,
                  indent=1)
    print("wrote dequant_kat.json")
