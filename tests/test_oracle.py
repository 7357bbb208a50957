"""Pins the CPU oracle (oracle/weft_oracle.c) before any GPU result is
compared with it.  Each check is independent of the oracle's own formula:

  * fp16 / e8m0 conversions against numpy's IEEE float16 and math.ldexp;
  * lookup tables against tests/golden/ggml_tables.json, parsed from the
    reference's ggml-common.h text by tests/golden/make_tables.py;
  * dequantizers by brute force over every code at every position, with the
    expected value built in float64 from the record layout as Weft's own
    encodings declare it (examples/formats/ggml.py) and its dequantize
    kernels compute it (examples/kernels/dequantize/*.py) -- a different
    description from the GGML C the oracle restates;
  * Q8 quantizers by hand-computed known answers (rounding ties, first-index
    maximum, all-zero block) and invariants; the Q4_0 / Q4_1 / MXFP4 / NVFP4
    weight quantizers likewise (inputs on the grid, rounding and tie rules);
  * vec_dot / mul_mat and the fp64 re-accumulation against an independent
    numpy path: dequantize both operands to float64 and take the dot.
GGML itself is not built here: ggml-impl.h includes gguf.h, which the
reference does not vendor.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle as o

GOLDEN = json.loads((Path(__file__).parent / "golden" / "ggml_tables.json").read_text())


# ------------------------------------------------------------ conversions
def test_fp16_to_fp32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    got = o.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_round_to_nearest_even_vs_numpy():
    # every fp16 value, every midpoint between neighbours (ties), their
    # fp32 neighbours, and 2M random bit patterns
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    mids = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    probes = [v.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
              np.nextafter(mids, np.float32(0)), np.float32([65504, 65519.99, 65520, 1e9, 6e-8, 3e-8])]
    rng = np.random.default_rng(0)
    probes.append(rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32))
    x = np.concatenate([np.concatenate([p, -p]) for p in probes]).astype(np.float32)
    finite = ~np.isnan(x)
    with np.errstate(over="ignore"):
        want = x[finite].astype(np.float16).view(np.uint16)
    got = o.fp32_to_fp16(x)
    assert np.array_equal(got[finite], want)
    # NaN keeps its sign and becomes the quiet NaN 0x7E00 (ggml-impl.h:431)
    assert set(np.unique(got[~finite] & 0x7fff)) <= {0x7e00}


def test_e8m0_half_is_two_to_the_e_minus_128():
    for e in range(256):
        assert o.e8m0_half(e) == np.float32(math.ldexp(1.0, e - 128)) or (
            math.ldexp(1.0, e - 128) > 3.4e38)
    assert np.array_equal(o.e8m0_half_table(),
                          np.array([np.float32(math.ldexp(1.0, e - 128)) if e < 255 else np.float32(2.0**127)
                                    for e in range(256)], np.float32))


# ----------------------------------------------------------------- tables
def test_iq2xxs_grid_matches_ggml_table():
    want = np.array([int(x, 16) for x in GOLDEN["iq2xxs_grid"]], np.uint64)
    got = o.iq2xxs_grid().view(np.uint64)
    assert np.array_equal(got, want)
    assert set(np.unique(o.iq2xxs_grid())) == {0x08, 0x19, 0x2b}


def test_iq2xs_grid_matches_ggml_table():
    want = np.array([int(x, 16) for x in GOLDEN["iq2xs_grid"]], np.uint64)
    got = o.iq2xs_grid().view(np.uint64)
    assert np.array_equal(got, want)
    assert set(np.unique(o.iq2xs_grid())) == {0x08, 0x19, 0x2b}


def test_sign_tables_match_ggml():
    assert list(o.ksigns_iq2xs()) == GOLDEN["ksigns_iq2xs"]
    kmask = GOLDEN["kmask_iq2xs"]
    s = o.signs_i8x8().reshape(128, 8)
    for i, ks in enumerate(GOLDEN["ksigns_iq2xs"]):
        assert list(s[i]) == [-1 if ks & kmask[j] else 1 for j in range(8)]
        assert (s[i] < 0).sum() % 2 == 0  # even number of minus signs


def test_kvalues_mxfp4_matches_ggml():
    assert list(o.kvalues_mxfp4()) == GOLDEN["kvalues_mxfp4"]


def test_record_sizes_match_ggml_static_asserts():
    # sizeof expressions of ggml-common.h evaluated with QK4_0 = QK8_0 =
    # QK_MXFP4 = 32, QK_K = 256, K_SCALE_SIZE = 12, ggml_half = 2 bytes
    env = {"ggml_half": 2, "uint8_t": 1, "int16_t": 2, "uint16_t": 2, "float": 4,
           "QK4_0": 32, "QK8_0": 32, "QK_MXFP4": 32, "QK_K": 256, "K_SCALE_SIZE": 12,
           "QK_NVFP4_SUB": 16, "QK_NVFP4": 64, "QK4_1": 32, "QK8_1": 32}
    sizes = {}
    for k, expr in GOLDEN["record_size_asserts"].items():
        e = expr.replace("sizeof", "")
        for name in sorted(env, key=len, reverse=True):
            e = e.replace(name, str(env[name]))
        sizes[k] = eval(e, {"__builtins__": {}})  # arithmetic on literals only
    assert sizes == {"block_q4_0": 18, "block_mxfp4": 17, "block_q8_0": 34, "block_q4_K": 144,
                     "block_q8_K": 292, "block_iq2_xxs": 66, "block_q6_K": 210, "block_q5_K": 176,
                     "block_nvfp4": 36, "block_q4_1": 20, "block_q8_1": 36, "block_iq2_xs": 74}
    assert {k: o.RECORD[k][1] for k in o.RECORD} == {
        "q4_0": 18, "mxfp4": 17, "q8_0": 34, "q4_k": 144, "q8_k": 292, "iq2_xxs": 66, "q6_k": 210, "q5_k": 176,
        "nvfp4": 36, "q4_1": 20, "q8_1": 36, "iq2_xs": 74}


# ------------------------------------------------------------ dequantizers
def _f16(x: float) -> int:
    return int(np.float16(x).view(np.uint16))


D16 = [_f16(v) for v in (0.5, -0.0373, 1.0, 6.0e-8, -3.0e-5, 1234.0)]


def test_dequant_q4_0_brute_force():
    # Weft Q4_0: f16 d, then q: u4[32] grouped(32) bit_layers(16, lo_first):
    # element j < 16 is the low nibble of byte j, j >= 16 the high nibble of
    # byte j-16; value (q - 8) * d (examples/kernels/dequantize/q4_0.py).
    recs, want = [], []
    for dh in D16:
        d = float(np.uint16(dh).view(np.float16))
        for pos in range(32):
            for q in range(16):
                codes = [(pos * 7 + j * 3 + q) % 16 for j in range(32)]
                codes[pos] = q
                b = bytearray(18)
                b[0:2] = dh.to_bytes(2, "little")
                for j in range(16):
                    b[2 + j] = codes[j] | (codes[j + 16] << 4)
                recs.append(bytes(b))
                want.append([np.float32((c - 8) * d) for c in codes])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 18)
    got = o.dequantize("q4_0", w, 32)
    assert np.array_equal(got, np.array(want, np.float32))


def test_dequant_q4_1_brute_force():
    # Weft Q4_1: f16 d, f16 m, q: u4[32] like Q4_0; value q * d + m
    # (examples/kernels/dequantize/q4_1.py, functions/quantization.py:10-11)
    recs, want = [], []
    for i, dh in enumerate(D16):
        mh = D16[(i + 2) % len(D16)]
        d = float(np.uint16(dh).view(np.float16))
        m = float(np.uint16(mh).view(np.float16))
        for pos in range(32):
            for q in range(16):
                codes = [(pos * 5 + j * 7 + q) % 16 for j in range(32)]
                codes[pos] = q
                b = bytearray(20)
                b[0:2] = dh.to_bytes(2, "little")
                b[2:4] = mh.to_bytes(2, "little")
                for j in range(16):
                    b[4 + j] = codes[j] | (codes[j + 16] << 4)
                recs.append(bytes(b))
                want.append([np.float32(np.float32(c * np.float32(d)) + np.float32(m)) for c in codes])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 20)
    got = o.dequantize("q4_1", w, 32)
    assert np.array_equal(got, np.array(want, np.float32))


def test_dequant_iq2_xs_brute_force():
    # examples/kernels/dequantize/iq2_xs.py: per 32-group g, scale byte
    # scales[g] (low nibble: entries 0-1, high: entries 2-3) gives
    # d * (0.5 + s) * 0.25; entry l's u16 word q[4g + l]: grid row = bits
    # 0-8, sign row = bits 9-15.
    grid = np.array([int(x, 16) for x in GOLDEN["iq2xs_grid"]], np.uint64).view(np.uint8).reshape(512, 8)
    ks = GOLDEN["ksigns_iq2xs"]
    rng = np.random.default_rng(4)
    raw = rng.integers(0, 256, (200, 74), dtype=np.uint8)
    raw[:, 0:2] = np.array([np.uint16(D16[i % 6]) for i in range(200)], np.uint16).view(np.uint8).reshape(200, 2)
    want = np.zeros((200, 256), np.float32)
    for r in range(200):
        d = np.float32(raw[r, 0:2].view(np.float16)[0])
        q = raw[r, 2:66].view(np.uint16)
        for gi in range(8):
            sb = int(raw[r, 66 + gi])
            scales = [np.float32(np.float32(d * np.float32(0.5 + (sb & 15))) * np.float32(0.25)),
                      np.float32(np.float32(d * np.float32(0.5 + (sb >> 4))) * np.float32(0.25))]
            for l in range(4):
                word = int(q[4 * gi + l])
                idx, sgn = word & 511, ks[word >> 9]
                for j in range(8):
                    s = np.float32(-1.0 if sgn & (1 << j) else 1.0)
                    want[r, 32 * gi + 8 * l + j] = np.float32(scales[l // 2] * np.float32(grid[idx, j])) * s
    assert np.array_equal(o.dequantize("iq2_xs", raw, 256).view(np.uint32), want.view(np.uint32))


def _pack_q4k_scales(sc, m):
    """6-bit scale/min packing as quantize_row_q4_K_ref writes it."""
    out = [0] * 12
    for j in range(8):
        if j < 4:
            out[j] = sc[j]
            out[j + 4] = m[j]
        else:
            out[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            out[j - 4] |= (sc[j] >> 4) << 6
            out[j] |= (m[j] >> 4) << 6
    return bytes(out)


def test_dequant_q4_k_brute_force():
    # Weft Q4_K: d, dmin, (sc, m) 6-bit x 8, q: u4[256] grouped(64)
    # bit_layers(32, lo_first): element e is byte 32*(e//64) + e%32, low
    # nibble when e%64 < 32; value d*sc*q - dmin*m of sub-block e//32
    # (examples/kernels/dequantize/q4_k.py, functions/quantization.py:14-17).
    rng = np.random.default_rng(7)
    recs, want = [], []
    for trial in range(600):
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        m = [int(v) for v in rng.integers(0, 64, 8)]
        if trial < 64:  # every scale and min value in every sub-block
            sc = [(trial + 7 * s) % 64 for s in range(8)]
            m = [(63 - trial + 5 * s) % 64 for s in range(8)]
        codes = [int(v) for v in rng.integers(0, 16, 256)]
        dh, mh = D16[trial % 6], D16[(trial + 3) % 6]
        d = float(np.uint16(dh).view(np.float16))
        dm = float(np.uint16(mh).view(np.float16))
        qs = bytearray(128)
        for e, c in enumerate(codes):
            byte = 32 * (e // 64) + e % 32
            qs[byte] |= c if e % 64 < 32 else c << 4
        recs.append(dh.to_bytes(2, "little") + mh.to_bytes(2, "little") + _pack_q4k_scales(sc, m) + bytes(qs))
        want.append([np.float32(d * sc[e // 32] * c - dm * m[e // 32]) for e, c in enumerate(codes)])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 144)
    got = o.dequantize("q4_k", w, 256)
    assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32))


def _q6k_record(codes, sc, dh):
    """A Q6_K record from the Weft encoding (examples/formats/ggml.py:114-120):
    ql u4[256] grouped(128) bit_layers(64, lo_first) -> element e of 128-group
    h at byte 64 h + (e % 128) % 64, high nibble when e % 128 >= 64; qh u2[256]
    grouped(128) bit_layers(32, lo_first) -> byte 128 + 32 h + (e % 128) % 32,
    bits 2 ((e % 128) // 32); scales i8[16] grouped(16); d f16 last."""
    b = bytearray(210)
    for e, c in enumerate(codes):
        h, i = e // 128, e % 128
        b[64 * h + i % 64] |= (c & 0xF) << (4 * (i // 64))
        b[128 + 32 * h + i % 32] |= (c >> 4) << (2 * (i // 32))
    b[192:208] = np.array(sc, np.int8).tobytes()
    b[208:210] = dh.to_bytes(2, "little")
    return bytes(b)


def test_dequant_q6_k_brute_force():
    # examples/kernels/dequantize/q6_k.py: q = ql | qh << 4, q -= 32,
    # y = f32(d) * f32(scale[e // 16]) * f32(q), products rounded left to right
    rng = np.random.default_rng(9)
    recs, want = [], []
    for trial in range(640):
        codes = [int(v) for v in rng.integers(0, 64, 256)]
        if trial < 64:  # every code at every position
            codes = [(trial + 13 * e) % 64 for e in range(256)]
        sc = [int(v) for v in rng.integers(-128, 128, 16)]
        if trial < 16:
            sc = [-128, 127, -1, 0, 1, 64, -65, 3] * 2
        dh = D16[trial % 6]
        d = np.float32(np.uint16(dh).view(np.float16))
        recs.append(_q6k_record(codes, sc, dh))
        want.append([(d * np.float32(sc[e // 16])) * np.float32(c - 32) for e, c in enumerate(codes)])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 210)
    got = o.dequantize("q6_k", w, 256)
    assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32))


def test_dequant_q5_k_brute_force():
    # Weft Q5_K (examples/formats/ggml.py:101-110): d, dmin, (sc, m) 6-bit x 8
    # packed as Q4_K's, qh u1[256] bit_layers(32, lo_first) -> byte e % 32,
    # bit e // 32; q u4[256] as Q4_K's; value d*sc*(q | qh << 4) - dmin*m
    # (examples/kernels/dequantize/q5_k.py, functions/quantization.py:14-17)
    rng = np.random.default_rng(11)
    recs, want = [], []
    for trial in range(600):
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        m = [int(v) for v in rng.integers(0, 64, 8)]
        codes = [int(v) for v in rng.integers(0, 32, 256)]
        if trial < 64:  # every scale, min and code value in every position
            sc = [(trial + 7 * s) % 64 for s in range(8)]
            m = [(63 - trial + 5 * s) % 64 for s in range(8)]
            codes = [(trial + 11 * e) % 32 for e in range(256)]
        dh, mh = D16[trial % 6], D16[(trial + 3) % 6]
        d = float(np.uint16(dh).view(np.float16))
        dm = float(np.uint16(mh).view(np.float16))
        qh, qs = bytearray(32), bytearray(128)
        for e, c in enumerate(codes):
            qs[32 * (e // 64) + e % 32] |= (c & 0xF) if e % 64 < 32 else (c & 0xF) << 4
            qh[e % 32] |= (c >> 4) << (e // 32)
        recs.append(dh.to_bytes(2, "little") + mh.to_bytes(2, "little") + _pack_q4k_scales(sc, m) +
                    bytes(qh) + bytes(qs))
        want.append([np.float32(d * sc[e // 32] * c - dm * m[e // 32]) for e, c in enumerate(codes)])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 176)
    got = o.dequantize("q5_k", w, 256)
    assert np.array_equal(got.view(np.uint32), np.array(want, np.float32).view(np.uint32))


def test_dequant_mxfp4_brute_force():
    kv = GOLDEN["kvalues_mxfp4"]
    recs, want = [], []
    for e in list(range(0, 256, 5)) + [1, 2, 127, 254]:
        for q in range(16):
            codes = [(q + 5 * j) % 16 for j in range(32)]
            b = bytearray(17)
            b[0] = e
            for j in range(16):
                b[1 + j] = codes[j] | (codes[j + 16] << 4)
            recs.append(bytes(b))
            with np.errstate(over="ignore"):  # 12 * 2^126 is +-inf in fp32, as in GGML
                want.append([np.float32(kv[c] * math.ldexp(1.0, e - 128)) for c in codes])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 17)
    assert np.array_equal(o.dequantize("mxfp4", w, 32), np.array(want, np.float32))


def _ue4m3_closed_form(c: int) -> float:
    """UE4M3 from the E4M3 bit fields (exponent bias 7, 3 mantissa bits,
    subnormals m * 2^-9), the sign bit ignored, times 1/2; 0x7F is zero."""
    if c & 0x7F in (0, 0x7F):
        return 0.0 if c != 0xFF else 0.5 * math.ldexp(1.875, 8)
    e, m = (c >> 3) & 0xF, c & 7
    return 0.5 * (math.ldexp(m, -9) if e == 0 else math.ldexp(1 + m / 8, e - 7))


def test_ue4m3_decode_matches_e4m3():
    import torch
    tab = o.ue4m3_table()
    e4m3 = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    # the torch E4M3FN decode for every finite positive code, halved
    assert np.array_equal(tab[:127], (0.5 * e4m3).astype(np.float32))
    assert tab[0x7F] == 0.0
    assert [float(tab[c]) for c in range(256)] == [_ue4m3_closed_form(c) for c in range(256)]


def test_ue4m3_encode_rounds_to_nearest_ties_up():
    # GGML's encoder returns 0x7E (448) for any result in exponent 15, so the
    # candidates are codes 1..0x77 plus 256 (code 0x78), which stands for 0x7E
    raw = 2.0 * o.ue4m3_table()[1:0x79].astype(np.float64)   # codes 1..0x78, increasing
    assert (np.diff(raw) > 0).all() and raw[-1] == 256.0
    for c in range(1, 0x78):                                    # exact values round-trip
        assert o.lib().wo_fp32_to_ue4m3(float(raw[c - 1])) == c
    rng = np.random.default_rng(5)
    xs = np.concatenate([np.exp(rng.uniform(np.log(1e-4), np.log(600.0), 4000)),
                         (raw[:-1] + raw[1:]) / 2])             # every midpoint: ties go up
    for x in xs.astype(np.float32):
        x = float(x)
        if 7.5 * 2.0 ** -9 <= x < 2.0 ** -6:
            want = 7      # GGML's subnormal path caps m at 7 below the first normal
        elif x >= 256.0:
            want = 0x7E   # exponent 15: saturated
        elif x < 0.5 * 2.0 ** -9:
            want = 0
        else:
            err = np.abs(raw - x)
            best = np.flatnonzero(err == err.min())
            want = int(best[-1]) + 1
            want = 0x7E if want == 0x78 else want
        assert o.lib().wo_fp32_to_ue4m3(x) == want, x
    assert o.lib().wo_fp32_to_ue4m3(0.0) == 0 and o.lib().wo_fp32_to_ue4m3(-1.0) == 0


def test_dequant_nvfp4_brute_force():
    # Weft NVFP4 (examples/formats/ggml.py:259-263): d u8[4], q u4[64]
    # grouped(16) then bit_layers(8, lo_first): element e of sub-block s = e // 16,
    # i = e % 16 sits in byte 4 + 8 s + i % 8, nibble i // 8; value kv[q] * ue4m3(d[s])
    kv = GOLDEN["kvalues_mxfp4"]
    rng = np.random.default_rng(13)
    recs, want = [], []
    for trial in range(300):
        d = [int(v) for v in rng.integers(0, 256, 4)] if trial >= 64 else [(trial + 61 * s) % 256 for s in range(4)]
        codes = [(trial + 7 * e) % 16 for e in range(64)]
        b = bytearray(36)
        b[0:4] = bytes(d)
        for e, c in enumerate(codes):
            s, i = divmod(e, 16)
            b[4 + 8 * s + i % 8] |= c << (4 * (i // 8))
        recs.append(bytes(b))
        want.append([np.float32(kv[c] * _ue4m3_closed_form(d[e // 16])) for e, c in enumerate(codes)])
    w = np.frombuffer(b"".join(recs), np.uint8).reshape(len(recs), 36)
    assert np.array_equal(o.dequantize("nvfp4", w, 64).view(np.uint32), np.array(want, np.float32).view(np.uint32))


def test_nvfp4_quantizer_picks_scale_and_nearest_codes():
    kv = np.array(GOLDEN["kvalues_mxfp4"], np.float64)
    x = o.seeded_normal(41, (8, 256), 0.02)
    q = o.quantize("nvfp4", x).reshape(-1, 36)
    xs = x.reshape(-1, 4, 16)
    tab = o.ue4m3_table()
    for r in range(q.shape[0]):
        for s in range(4):
            amax = np.float32(np.abs(xs[r, s]).max())
            assert q[r, s] == o.lib().wo_fp32_to_ue4m3(float(np.float32(amax / np.float32(6.0))))
            d = np.float32(tab[q[r, s]])
            for i in range(16):
                c = (q[r, 4 + 8 * s + i % 8] >> (4 * (i // 8))) & 0xF
                err = np.abs((kv * d).astype(np.float32) - xs[r, s, i]).astype(np.float32)
                assert c == int(np.argmin(err))   # first index among equal errors


def test_int_partials_nvfp4_are_the_sub_block_dots():
    k = 256
    w = o.quantize("nvfp4", o.seeded_normal(42, (1, k), 0.02))
    xq = o.quantize("q8_0", o.seeded_normal(43, (1, k)))
    parts = np.zeros(k // 16, np.int32)
    n = o.lib().wo_int_partials(o.NVFP4, o._ptr(w[0]), o._ptr(xq[0]), k, o._ptr(parts))
    assert n == k // 16
    kv = np.array(GOLDEN["kvalues_mxfp4"], np.int64)
    tab = o.ue4m3_table()
    codes = np.round(o.dequantize("nvfp4", w, k)[0].astype(np.float64) /
                     np.repeat(tab[w[0].reshape(-1, 36)[:, :4].reshape(-1)], 16).astype(np.float64)
                     .clip(min=1e-30))
    xv = xq[0].reshape(-1, 34)[:, 2:].view(np.int8).reshape(-1).astype(np.int64)
    scales = np.repeat(tab[w[0].reshape(-1, 36)[:, :4].reshape(-1)], 16)
    codes = np.where(scales == 0, 0, codes).astype(np.int64)
    assert set(np.unique(codes)) <= set(kv.tolist())
    want = [int((codes[16 * g:16 * g + 16] * xv[16 * g:16 * g + 16]).sum()) for g in range(k // 16)]
    got = [int(p) if tab[w[0].reshape(-1, 36)[g // 4, g % 4]] != 0 else 0 for g, p in enumerate(parts)]
    assert got == want


def test_dequant_iq2_xxs_brute_force():
    # examples/kernels/dequantize/iq2_xxs.py: per 32-group g, word pair
    # q[4g..4g+3]: metadata = q[4g+2] | q[4g+3] << 16; scale = d*(0.5 +
    # meta>>28)*0.25; entry l: grid row = byte l%2 of q[4g + l//2], sign row
    # = (meta >> 7l) & 127.
    grid = np.array([int(x, 16) for x in GOLDEN["iq2xxs_grid"]], np.uint64).view(np.uint8).reshape(256, 8)
    ks = GOLDEN["ksigns_iq2xs"]
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, (300, 66), dtype=np.uint8)
    raw[:, 0:2] = np.array([np.uint16(D16[i % 6]) for i in range(300)], np.uint16).view(np.uint8).reshape(300, 2)
    want = np.zeros((300, 256), np.float32)
    for r in range(300):
        d = float(raw[r, 0:2].view(np.float16)[0])
        q = raw[r, 2:].view(np.uint16)
        for gi in range(8):
            meta = int(q[4 * gi + 2]) | (int(q[4 * gi + 3]) << 16)
            scale = d * (0.5 + (meta >> 28)) * 0.25
            for l in range(4):
                idx = (int(q[4 * gi + l // 2]) >> (8 * (l % 2))) & 0xFF
                sgn = ks[(meta >> (7 * l)) & 127]
                for j in range(8):
                    s = -1 if sgn & (1 << j) else 1
                    want[r, 32 * gi + 8 * l + j] = np.float32(int(grid[idx, j]) * s * scale)
    assert np.array_equal(o.dequantize("iq2_xxs", raw, 256).view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------- Q8 quantizers
def test_q8_0_known_answers():
    x = np.zeros(64, np.float32)
    x[0] = 127.0
    x[1:8] = [0.5, 1.5, 2.5, -0.5, -2.5, 3.5, 126.5]  # d = 1: ties round away from zero
    x[32:64] = np.linspace(-3.0, 1.0, 32, dtype=np.float32)
    y = o.quantize("q8_0", x)
    assert y[0:2].view(np.uint16)[0] == 0x3C00  # fp16(1.0)
    assert list(y[2:10].view(np.int8)) == [127, 1, 2, 3, -1, -3, 4, 127]
    d2 = np.float32(3.0) / np.float32(127)
    assert y[34:36].view(np.uint16)[0] == np.float16(d2).view(np.uint16)
    assert y[36:68].view(np.int8)[0] == -127  # -3.0 is the block maximum
    z = o.quantize("q8_0", np.zeros(32, np.float32))
    assert not z.any()


def test_q8_k_known_answers():
    x = np.zeros(512, np.float32)
    x[0] = 127.0          # iscale = -1: q = rne(-x)
    x[1:7] = [0.5, 1.5, 2.5, -0.5, -1.5, 126.5]
    x[256 + 3] = 5.0      # first index of the largest |x| wins: +5 -> -127
    x[256 + 7] = -5.0
    sentinel = 0x5A
    y = np.full(2 * 292, sentinel, np.uint8)
    o.quantize("q8_k", x, out=y.reshape(2, 292))
    b0, b1 = y[:292], y[292:]
    assert b0[0:4].view(np.float32)[0] == -1.0
    assert list(b0[4:11].view(np.int8)) == [-127, 0, -2, -2, 0, 2, -126]
    bs = b0[260:292].view(np.int16)
    assert bs[0] == int(b0[4:20].view(np.int8).astype(int).sum())
    assert b1[4 + 3].astype(np.int8) == -127 and np.int8(b1[4 + 7]) == 127
    assert b1[0:4].view(np.float32)[0] == np.float32(1.0) / (np.float32(-127.0) / np.float32(5.0))
    # all-zero block: d = 0, qs = 0, bsums left as they were
    z = np.full(292, sentinel, np.uint8)
    o.quantize("q8_k", np.zeros(256, np.float32), out=z.reshape(1, 292))
    assert not z[:260].any() and (z[260:] == sentinel).all()


def test_q8_1_known_answers():
    # quantize_row_q8_1_ref (ggml-quants.c:264-295): Q8_0's d and codes, and
    # s = fp16(sum(q) * d) with the fp32 d
    x = np.zeros(64, np.float32)
    x[0] = 127.0
    x[1:8] = [0.5, 1.5, 2.5, -0.5, -2.5, 3.5, 126.5]
    x[32:64] = np.linspace(-3.0, 1.0, 32, dtype=np.float32)
    y = o.quantize("q8_1", x)
    assert y[0:2].view(np.uint16)[0] == 0x3C00
    q0 = [127, 1, 2, 3, -1, -3, 4, 127]
    assert list(y[4:12].view(np.int8)) == q0
    assert y[2:4].view(np.float16)[0] == np.float16(sum(q0))
    # the second block's codes are Q8_0's, its sum is rounded once to fp16
    q80 = o.quantize("q8_0", x[32:])
    assert np.array_equal(y[40:72], q80[2:34]) and np.array_equal(y[36:38], q80[0:2])
    d2 = np.float32(3.0) / np.float32(127)
    tot = int(y[40:72].view(np.int8).astype(int).sum())
    assert y[38:40].view(np.uint16)[0] == np.float16(np.float32(tot) * d2).view(np.uint16)
    assert not o.quantize("q8_1", np.zeros(32, np.float32)).any()


def test_q4_1_quantizer_known_answer():
    # quantize_row_q4_1_ref (ggml-quants.c:112-146): a block spanning
    # [min, min + 15 d] on the code grid comes back code for code
    d, mn = np.float32(0.25), np.float32(-1.0)
    codes = np.array([(5 * j + 3) % 16 for j in range(32)])
    codes[0], codes[1] = 0, 15
    x = (mn + codes * d).astype(np.float32)
    y = o.quantize("q4_1", x)
    assert y[0:2].view(np.float16)[0] == np.float16(d) and y[2:4].view(np.float16)[0] == np.float16(mn)
    got = np.concatenate([y[4:20] & 0xF, y[4:20] >> 4])
    assert np.array_equal(got, codes)


@pytest.mark.parametrize("act", ["q8_0", "q8_k"])
def test_q8_invariants(act):
    x = o.seeded_normal(21, (64, 1024))
    y = o.quantize(act, x)
    elems, nbytes = o.RECORD[act]
    recs = y.reshape(-1, nbytes)
    xb = x.reshape(-1, elems).astype(np.float64)
    if act == "q8_0":
        d = recs[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        q = recs[:, 2:].view(np.int8).astype(np.float64)
        assert (np.abs(q).max(axis=1) == 127).all()
        # q is rounded against the fp32 d, the record holds fp16(d): up to
        # 127 * 2^-11 * d more
        assert (np.abs(xb - q * d[:, None]) <= (0.5 + 127 * 2.0**-11 + 1e-3) * d[:, None]).all()
    else:
        d = recs[:, 0:4].copy().view(np.float32).astype(np.float64)[:, 0]
        q = recs[:, 4:260].view(np.int8).astype(np.int64)
        bs = recs[:, 260:292].copy().view(np.int16).astype(np.int64)
        assert np.array_equal(bs, q.reshape(-1, 16, 16).sum(axis=2))
        assert (np.abs(q).max(axis=1) == 127).all()
        assert (np.abs(xb - q * d[:, None]) <= 0.5 * np.abs(d)[:, None] * (1 + 1e-5)).all()


# ----------------------------------------------- vec_dot / mul_mat / fp64
def _dequant_act(act, xq, k):
    elems, nbytes = o.RECORD[act]
    recs = xq.reshape(-1, nbytes)
    if act == "q8_0":
        d = recs[:, 0:2].copy().view(np.float16).astype(np.float64)
        q = recs[:, 2:].view(np.int8).astype(np.float64)
    elif act == "q8_1":
        d = recs[:, 0:2].copy().view(np.float16).astype(np.float64)
        q = recs[:, 4:].view(np.int8).astype(np.float64)
    else:
        d = recs[:, 0:4].copy().view(np.float32).astype(np.float64)
        q = recs[:, 4:260].view(np.int8).astype(np.float64)
    return (q * d).reshape(xq.shape[0], k)


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4", "q6_k", "q5_k", "nvfp4", "q4_1", "iq2_xs"])
def test_mul_mat_against_independent_float64_path(fmt):
    n, k, m = 48, 2048, 3
    if fmt == "iq2_xs":
        w = o.random_records(fmt, n, k, seed=31)
    else:
        w = o.quantize(fmt, o.seeded_normal(31, (n, k), 0.02))
    x = o.seeded_normal(32, (m, k))
    xq, y = o.mul_mat(fmt, w, x, n, k, m)
    e, a = o.mul_mat_f64(fmt, w, xq, n, k, m)
    # independent: dequantize both operands (pinned above) and multiply
    ref = _dequant_act(o.ACT_OF[fmt], xq, k) @ o.dequantize(fmt, w, k).astype(np.float64).T
    if fmt == "q4_1":
        # Q4_1's min term uses Q8_1's s (fp16 of sum(q) * fp32 d), not the
        # dequantized activation: replace that part of the reference
        xr = xq.reshape(m, -1, 36)
        s = xr[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
        dx = xr[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        qsum = xr[:, :, 4:].view(np.int8).astype(np.float64).sum(axis=2)
        wm = w.reshape(n, -1, 20)[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
        ref += s @ wm.T - (dx * qsum) @ wm.T
    assert np.allclose(e, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    assert o.within_tolerance(y, e, a).all()
    # a wrong sign or a dropped min term would not be near: check the bound bites
    assert not o.within_tolerance(y * 1.001 + 1e-3, e, a).all()
    # vec_dot of one row pair is the same function
    assert o.vec_dot(fmt, w[5], xq[1], k) == y[1, 5]


@pytest.mark.parametrize("fmt", ["q4_0", "q4_k", "iq2_xxs", "mxfp4"])
@pytest.mark.parametrize("n,m", [(1, 1), (37, 1), (61, 5), (130, 17)])
def test_ggml_scheduled_mul_mat_equals_the_pinned_mul_mat(fmt, n, m):
    """The CPU baseline's MUL_MAT with GGML's thread schedule (wo_mul_mat_ggml,
    ggml-cpu.c:1245-1443) gives the pinned wo_mul_mat's Xq and Y bit for bit,
    at 1, 2 and every thread, on ragged N and M: the schedule only splits the
    work, every output is the same vec_dot."""
    k = 1024
    w = o.quantize(fmt, o.seeded_normal(71, (n, k), 0.02))
    x = o.seeded_normal(72, (m, k))
    xq, y = o.mul_mat(fmt, w, x, n, k, m)
    for threads in (1, 2, o.max_threads()):
        gxq, gy = o.mul_mat_ggml(fmt, w, x, n, k, m, threads=threads)
        assert np.array_equal(gxq, xq)
        assert np.array_equal(gy.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_iq2_caller_table_oracle_is_the_ggml_function_on_ggml_tables(fmt):
    """oracle.iq2_tables_mul_mat_f64 with GGML's grid and sign tables is the
    pinned wo_mul_mat_f64 (GGML's generic vec_dot), E and A exactly."""
    n, k, m = 13, 1024, 3
    w = o.random_records(fmt, n, k, seed=91) if fmt == "iq2_xs" else \
        o.quantize(fmt, o.seeded_normal(91, (n, k), 0.02))
    xq = o.quantize("q8_k", o.seeded_normal(92, (m, k)))
    grid = (o.iq2xs_grid() if fmt == "iq2_xs" else o.iq2xxs_grid()).view(np.int8)
    e, a = o.mul_mat_f64(fmt, w, xq, n, k, m)
    e2, a2 = o.iq2_tables_mul_mat_f64(fmt, w, xq, n, k, m, grid, o.signs_i8x8())
    np.testing.assert_array_equal(e2, e)
    np.testing.assert_array_equal(a2, a)


@pytest.mark.parametrize("fmt", ["iq2_xxs", "iq2_xs"])
def test_iq2_caller_table_oracle_known_answer(fmt):
    """One superblock, worked by hand: grid row 3 = (-56, 1, 0, 127, -128,
    -1, 2, 10) against sign row 5 = (3, -1, 7, 2, -1, 1, 0, -128) in i8
    arithmetic gives bytes (88, -1, 0, -2, -128, -1, 0, 0) (-168, 254, 128
    and -1280 wrap modulo 256); against x = 1..8 that is -568; scale nibble
    2 -> times 5; d = 1, dx = 0.5, times 0.125: -177.5."""
    grid = np.zeros((512 if fmt == "iq2_xs" else 256, 8), np.int8)
    grid[3] = (-56, 1, 0, 127, -128, -1, 2, 10)
    signs = np.zeros((128, 8), np.int8)
    signs[5] = (3, -1, 7, 2, -1, 1, 0, -128)
    rec = np.zeros(74 if fmt == "iq2_xs" else 66, np.uint8)
    rec[0:2] = np.array([1.0], np.float16).view(np.uint8)
    if fmt == "iq2_xs":
        rec[2:4] = np.array([3 | (5 << 9)], np.uint16).view(np.uint8)  # entry 0: grid 3, sign 5
        rec[66] = 2                                                    # elements 0-15: 2 s + 1 = 5
    else:
        rec[2] = 3                                                     # group 0, entry 0: grid 3
        rec[6:10] = np.array([5 | (2 << 28)], np.uint32).view(np.uint8)  # sign row 5, s = 2
    xq = np.zeros(292, np.uint8)
    xq[0:4] = np.array([0.5], np.float32).view(np.uint8)
    xq[4:12] = np.arange(1, 9, dtype=np.int8).view(np.uint8)
    e, a = o.iq2_tables_mul_mat_f64(fmt, rec[None], xq[None], 1, 256, 1, grid, signs)
    assert e[0, 0] == -177.5 and a[0, 0] == 177.5


def test_int_partials_q4_0_are_the_block_dots():
    k = 512
    w = o.quantize("q4_0", o.seeded_normal(41, (1, k), 0.02))
    xq = o.quantize("q8_0", o.seeded_normal(42, (1, k)))
    p = o.int_partials("q4_0", w, xq, k)
    rec = w.reshape(-1, 18)
    qs = rec[:, 2:]
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=1).astype(np.int64) - 8
    xv = xq.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.int64)
    assert np.array_equal(p, (codes * xv).sum(axis=1))


def test_int_partials_q4_k_match_dequantized_integers():
    k = 512
    w = o.quantize("q4_k", o.seeded_normal(43, (1, k), 0.02))
    xq = o.quantize("q8_k", o.seeded_normal(44, (1, k)))
    p = o.int_partials("q4_k", w, xq, k).reshape(-1, 9)
    for b in range(k // 256):
        rec = w[0, 144 * b:144 * (b + 1)]
        qs = rec[16:]
        codes = np.zeros(256, np.int64)
        for e in range(256):
            byte = qs[32 * (e // 64) + e % 32]
            codes[e] = byte & 0xF if e % 64 < 32 else byte >> 4
        xr = xq[0, 292 * b:292 * (b + 1)]
        xv = xr[4:260].view(np.int8).astype(np.int64)
        assert list(p[b, :8]) == [int((codes[32 * s:32 * s + 32] * xv[32 * s:32 * s + 32]).sum())
                                  for s in range(8)]


def test_int_partials_q6_k_are_the_group_dots():
    k = 512
    w = o.quantize("q6_k", o.seeded_normal(45, (1, k), 0.02))
    xq = o.quantize("q8_k", o.seeded_normal(46, (1, k)))
    p = o.int_partials("q6_k", w, xq, k).reshape(-1, 16)
    for b in range(k // 256):
        rec = w[0, 210 * b:210 * (b + 1)]
        codes = np.zeros(256, np.int64)
        for e in range(256):  # the record address of _q6k_record, read back
            h, i = e // 128, e % 128
            lo = (int(rec[64 * h + i % 64]) >> (4 * (i // 64))) & 0xF
            hi = (int(rec[128 + 32 * h + i % 32]) >> (2 * (i // 32))) & 3
            codes[e] = (lo | hi << 4) - 32
        xv = xq[0, 292 * b + 4:292 * b + 260].view(np.int8).astype(np.int64)
        assert list(p[b]) == [int((codes[16 * g:16 * g + 16] * xv[16 * g:16 * g + 16]).sum())
                              for g in range(16)]


# ------------------------------------------------ weight quantizers (inputs)
@pytest.mark.parametrize("fmt,bound", [("q4_0", 0.10), ("q4_k", 0.09), ("mxfp4", 0.13), ("iq2_xxs", 0.45),
                                       ("q6_k", 0.05), ("q5_k", 0.05), ("nvfp4", 0.11)])
def test_weight_quantizer_round_trip(fmt, bound):
    w = o.seeded_normal(51, (32, 4096), 0.02)
    d = o.dequantize(fmt, o.quantize(fmt, w), 4096)
    rel = np.sqrt(((d - w) ** 2).mean()) / np.sqrt((w ** 2).mean())
    assert rel < bound


def _k_scale_min(s: np.ndarray, j: int):
    """get_scale_min_k4 (ggml-quants.c:822-829) over records' 12 scale bytes."""
    if j < 4:
        return s[..., j] & 63, s[..., j + 4] & 63
    return ((s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4),
            (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4))


def _codes_k(fmt: str, rec: np.ndarray) -> np.ndarray:
    """The integer codes of Q4_K / Q5_K / Q6_K records (element order),
    read from the byte layouts of ggml-common.h."""
    e = np.arange(256)
    if fmt in ("q4_k", "q5_k"):
        qs = rec[:, -128:]
        low = qs[:, 32 * (e // 64) + e % 32]
        q = np.where((e % 64) < 32, low & 0xF, low >> 4).astype(np.int32)
        if fmt == "q5_k":
            qh = rec[:, 16:48]
            q += ((qh[:, e % 32] >> (e // 32)) & 1).astype(np.int32) << 4
        return q
    ql, qh = rec[:, :128], rec[:, 128:192]
    h, r = e // 128, e % 128
    lo = ql[:, 64 * h + r % 64]
    q = np.where(r < 64, lo & 0xF, lo >> 4).astype(np.int32)
    q |= ((qh[:, 32 * h + r % 32] >> (2 * (r // 32))) & 3).astype(np.int32) << 4
    return q


def _k_halves(fmt: str, w: np.ndarray, xq: np.ndarray) -> np.ndarray:
    """(m, n, 2): each K = 256 output's two half-superblock terms in fp64,
    from the record bytes (Q4_K / Q5_K: dx (d sum sc P - dmin sum m B),
    B = the group's two Q8_K bsums; Q6_K: dx d sum sc P)."""
    rb = o.RECORD[fmt][1]
    rec = w.reshape(-1, rb)
    codes = _codes_k(fmt, rec).astype(np.int64)                         # (n, 256)
    xv = xq[:, 4:260].view(np.int8).astype(np.int64)                    # (m, 256)
    dx = xq[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    bs = xq[:, 260:292].copy().view(np.int16).astype(np.int64)          # (m, 16)
    f16 = lambda b: b.copy().view(np.float16).astype(np.float64)[..., 0]  # noqa: E731
    out = np.zeros((xq.shape[0], rec.shape[0], 2))
    if fmt == "q6_k":
        d = f16(rec[:, 208:210])
        sc = rec[:, 192:208].view(np.int8).astype(np.int64)
        for j in range(16):
            p = xv[:, 16 * j:16 * j + 16] @ (codes[:, 16 * j:16 * j + 16] - 32).T
            out[:, :, j // 8] += dx[:, None] * d[None, :] * (sc[None, :, j] * p)
        return out
    d, dmin = f16(rec[:, 0:2]), f16(rec[:, 2:4])
    for j in range(8):
        sc, m = _k_scale_min(rec[:, 4:16].astype(np.int64), j)
        p = xv[:, 32 * j:32 * j + 32] @ codes[:, 32 * j:32 * j + 32].T
        b = bs[:, 2 * j] + bs[:, 2 * j + 1]
        out[:, :, j // 4] += dx[:, None] * (d[None, :] * (sc[None, :] * p) - dmin[None, :] * (m[None, :] * b[:, None]))
    return out


def test_mul_mat_f64_magnitude_bounds_half_superblocks():
    """A (the tolerance's magnitude) is summed over scale groups, so it
    bounds every partial sum of whole groups a kernel may round to fp32.
    The case is a Q5_K output of a randomized GPU shape sweep (K = 256):
    its half-superblock terms are +-0.225 and its total 1.2e-5, so a
    per-superblock A (|dx d S| + |dx dmin Mn| ~ 1e-3) was 450x too small
    to cover the fp32 rounding of the halves (1.3e-8)."""
    x = o.seeded_normal(447344297, (285, 256))[40:41]
    w = o.quantize("q5_k", o.seeded_normal(1029995214, (1814, 256), 0.02)[1755:1756])
    xq = o.quantize("q8_k", x)
    e, a = o.mul_mat_f64("q5_k", w, xq, 1, 256, 1)
    halves = _k_halves("q5_k", w, xq)[0, 0]
    assert abs(halves.sum() - e[0, 0]) <= 1e-15 * np.abs(halves).sum()
    assert abs(e[0, 0]) < 2e-5 and np.abs(halves).min() > 0.2
    assert a[0, 0] >= np.abs(halves).sum()
    # fp32 halves summed in fp32 (one rounding each, then the sum) pass the bar
    y = np.float32(np.float32(halves[0]) + np.float32(halves[1]))
    assert o.within_tolerance(np.array([[y]]), e, a).all()
    # and the property on random rows of each K-quant
    for fmt in ("q4_k", "q5_k", "q6_k"):
        w = o.quantize(fmt, o.seeded_normal(61, (64, 256), 0.02))
        xq = o.quantize("q8_k", o.seeded_normal(62, (48, 256)))
        e, a = o.mul_mat_f64(fmt, w, xq, 64, 256, 48)
        halves = _k_halves(fmt, w, xq)
        np.testing.assert_allclose(halves.sum(axis=2), e, rtol=0, atol=1e-12 * a.max())
        assert (a >= np.abs(halves).sum(axis=2) * (1 - 1e-12)).all(), fmt


def _nearest_int(v: np.ndarray) -> np.ndarray:
    return np.rint(v.astype(np.float32)).astype(np.int64)  # RNE, as GGML's 1.5 * 2^23 trick


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
def test_k_quantizer_codes_are_nearest_given_the_record(fmt):
    """What GGML's reference quantizers' last pass fixes, checked on the
    oracle's records: with the record's own fp16 d (and dmin) and 6-bit
    (Q6_K: int8) scales, every code of a sub-block with a non-zero scale is
    nearest_int((x + dmin m) / (d sc)) clamped to the code range
    (quantize_row_q4_K_ref ggml-quants.c:1448-1459, _q5_K_ref :1635-1646,
    _q6_K_ref :1849-1859).  Weights of the tests' generator plus rows with a
    zero sub-block, a constant row and an outlier."""
    x = o.seeded_normal(53, (24, 1024), 0.02)
    x[1, 64:96] = 0.0
    x[2, :] = 0.01
    x[3, 500] = 0.9
    rb = o.RECORD[fmt][1]
    rec = o.quantize(fmt, x).reshape(-1, rb)
    xs = x.reshape(-1, 256).astype(np.float32)
    codes = _codes_k(fmt, rec)
    f16 = lambda b: b.copy().view(np.float16).astype(np.float32)[..., 0]  # noqa: E731
    checked = 0
    if fmt == "q6_k":
        d = f16(rec[:, 208:210])
        sc = rec[:, 192:208].view(np.int8).astype(np.float32)
        for j in range(16):
            dj = (d * sc[:, j]).astype(np.float32)
            live = dj != 0
            v = xs[live, 16 * j:16 * j + 16] / dj[live, None]
            want = np.clip(_nearest_int(v), -32, 31) + 32
            assert (codes[live, 16 * j:16 * j + 16] == want).all(), f"sub-block {j}"
            checked += int(live.sum())
    else:
        d, dmin = f16(rec[:, 0:2]), f16(rec[:, 2:4])
        top = 15 if fmt == "q4_k" else 31
        for j in range(8):
            sc, m = _k_scale_min(rec[:, 4:16], j)
            dj = (d * sc.astype(np.float32)).astype(np.float32)
            dm = (dmin * m.astype(np.float32)).astype(np.float32)
            live = dj != 0
            v = (xs[live, 32 * j:32 * j + 32] + dm[live, None]) / dj[live, None]
            want = np.clip(_nearest_int(v), 0, top)
            assert (codes[live, 32 * j:32 * j + 32] == want).all(), f"sub-block {j}"
            checked += int(live.sum())
    assert checked > 0.9 * xs.shape[0] * (16 if fmt == "q6_k" else 8)


def test_q4_0_quantizer_error_is_half_a_step():
    w = o.seeded_normal(52, (16, 1024), 0.02)
    q = o.quantize("q4_0", w).reshape(-1, 18)
    d = np.abs(q[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0])
    err = np.abs(o.dequantize("q4_0", q, 32).astype(np.float64) - w.reshape(-1, 32))
    # the block maximum maps to -8 exactly; the +7 clamp side may lose up to a full step
    assert (err <= d[:, None] * 1.001 + 1e-7).all()


def _q4_0_codes(rec: np.ndarray) -> np.ndarray:
    qs = rec[:, 2:18].astype(np.int64)
    return np.concatenate([qs & 15, qs >> 4], axis=1)  # element j: low nibble, j + 16: high


def test_q4_0_quantizer_known_answers():
    """quantize_row_q4_0_ref (ggml-quants.c:28-53): d = max / -8 with max
    the signed value of largest |x| (first index on ties), id = 1 / d,
    q = MIN(15, (int8_t)(x id + 8.5)), i.e. round half up and truncation
    toward zero of the biased value, element j in the low nibble of byte j
    and j + 16 in the high one."""
    rng = np.random.default_rng(5)
    # blocks on the grid: x = d (q - 8) with one element at -8 d, d random fp16
    nblk = 64
    q = rng.integers(0, 16, size=(nblk, 32))
    q[np.arange(nblk), rng.integers(0, 32, size=nblk)] = 0
    d = o.fp16_to_fp32(o.fp32_to_fp16(rng.uniform(1e-3, 1.0, size=nblk).astype(np.float32)))
    d[::2] = -d[::2]  # a negative d: the largest magnitude is positive
    x = (d[:, None].astype(np.float64) * (q - 8)).astype(np.float32)
    rec = o.quantize("q4_0", x.reshape(1, -1)).reshape(nblk, 18)
    assert np.array_equal(rec[:, 0:2].copy().view(np.uint16)[:, 0], o.fp32_to_fp16(d))
    assert np.array_equal(_q4_0_codes(rec), q)
    # rounding: with d = 2^-3 (id exact) x id = v gives floor(v + 8.5), clamped to 15
    v = np.array([-8, -1.5, -0.5, 0.5, 1.5, 2.5, -2.5, 6.49, 6.5, 7.0, 7.49, 7.5, 8.0, 0.0,
                  3.25, -3.25, -7.5, 5.5, 4.5, -4.5, 1, 2, 3, 4, 5, 6, 7, -7, -6, -5, -4, -3])
    x = (np.float32(-0.125) * v).astype(np.float32)  # max = x[0] = +1, d = 1 / -8
    rec = o.quantize("q4_0", x.reshape(1, 32))
    want = np.minimum(15, np.floor(v + 8.5)).astype(np.int64)
    assert np.array_equal(_q4_0_codes(rec.reshape(1, 18))[0], want)
    # a tie on |x|: the first index sets the sign of d
    x = np.zeros((1, 32), np.float32)
    x[0, 3], x[0, 9] = -2.0, 2.0
    rec = o.quantize("q4_0", x).reshape(1, 18)
    assert o.fp16_to_fp32(rec[:, 0:2].copy().view(np.uint16))[0] == 0.25  # -2 / -8
    assert _q4_0_codes(rec)[0, 3] == 0 and _q4_0_codes(rec)[0, 9] == 15  # 8 + 8.5 -> 16 -> 15
    # an all-zero block: d = 0 / -8 = -0 (fp16 0x8000), id = 0, every code 8
    rec = o.quantize("q4_0", np.zeros((1, 32), np.float32)).reshape(1, 18)
    assert rec[0, 0:2].copy().view(np.uint16)[0] == 0x8000 and (rec[0, 2:] == 0x88).all()


def test_mxfp4_quantizer_known_answers():
    """quantize_row_mxfp4_ref / best_index_mxfp4 (ggml-quants.c:299-344):
    e = floor(log2(amax)) - 2 + 127, d = 2^(e - 128), and each value takes
    the first kvalues_mxfp4 index at the smallest |kv d - x|: on ties the
    lower index (0 before -0, 4 before 6, -4 before -6)."""
    kv = o.kvalues_mxfp4().astype(np.int64)
    rng = np.random.default_rng(6)
    nblk = 64
    p = rng.integers(-20, 20, size=nblk)                   # amax in [2^p, 2^(p+1))
    d = np.ldexp(1.0, p - 3)                               # 2^(e - 128) with e = p + 125
    c = rng.integers(0, 16, size=(nblk, 32))
    c[c == 8] = 0                                          # kv[8] = -0 encodes as index 0
    top = rng.integers(0, 32, size=nblk)
    c[np.arange(nblk), top] = np.where(rng.integers(0, 2, size=nblk) == 1, 7, 15)  # +-12: amax = 1.5 2^p
    x = (kv[c] * d[:, None]).astype(np.float32)
    rec = o.quantize("mxfp4", x.reshape(1, -1)).reshape(nblk, 17)
    assert np.array_equal(rec[:, 0].astype(np.int64), p + 125)
    codes = np.concatenate([rec[:, 1:17] & 15, rec[:, 1:17] >> 4], axis=1).astype(np.int64)
    assert np.array_equal(codes, c)
    # ties and values between the grid points, in units of d = 2^-3 (amax = 1.5)
    u = np.array([12, 5, -5, 7, -7, 10, -10, 0.5, -0.5, 1.5, 2.5, 3.5, 15, -15, 0, 0.49,
                  5.01, 4.99, 9.99, 10.01, -1.5, -2.5, -3.5, -0.51, 11.9, 6, -12, 8, -8, 3, 2, 1])
    want = [7, 4, 12, 5, 13, 6, 14, 0, 0, 1, 2, 3, 7, 15, 0, 0,
            5, 4, 6, 7, 9, 10, 11, 9, 7, 5, 15, 6, 14, 3, 2, 1]
    x = (u * 0.125).astype(np.float32).reshape(1, 32)
    rec = o.quantize("mxfp4", x).reshape(1, 17)
    assert rec[0, 0] == 125  # amax = 15/8: floor(log2) = 0, e = 0 - 2 + 127
    got = np.concatenate([rec[0, 1:17] & 15, rec[0, 1:17] >> 4])
    assert list(got) == want
    # an all-zero block: e = 0 and every code 0
    assert not o.quantize("mxfp4", np.zeros((1, 32), np.float32)).any()


# ------------------------------------------------ Q4K_I[16] interleave layout
def test_interleave_matches_the_reference_record_address():
    """oracle.interleave_rows against the record pointer the reference's
    emitter generates for a derived interleave (lib/Target/Emission/
    Memory.cpp:984-991: ((row / R) * blocks + block) * (144 * R) + row % R,
    bytes at stride R), evaluated element by element."""
    rows, n, k = 16, 48, 768
    nsb = k // 256
    rng = np.random.default_rng(5)
    w = rng.integers(0, 256, size=n * nsb * 144, dtype=np.uint8)
    packed = o.interleave_rows(w, n, k, rows)
    assert packed.shape == w.shape
    src = w.reshape(n, nsb, 144)
    for row in range(n):
        for block in range(nsb):
            record = ((row // rows) * nsb + block) * (144 * rows) + row % rows
            got = packed[record + rows * np.arange(144)]
            np.testing.assert_array_equal(got, src[row, block])


def test_interleave_known_answer_and_inverse():
    # byte b of row r of superblock j holds (r + 7 j + 13 b) % 256: spot
    # positions, then the permutation is a bijection with a known inverse
    n, k = 32, 512
    r, j, b = np.meshgrid(np.arange(n), np.arange(k // 256), np.arange(144), indexing="ij")
    w = ((r + 7 * j + 13 * b) % 256).astype(np.uint8).reshape(-1)
    p = o.interleave_rows(w, n, k)
    assert p[0] == 0 and p[1] == 1 and p[16] == 13           # rows 0, 1 byte 0; row 0 byte 1
    assert p[2304] == 7                                       # cohort 0, superblock 1, row 0, byte 0
    assert p[2 * 2304 + 16 * 143 + 15] == (16 + 15 + 13 * 143) % 256  # cohort 1, superblock 0
    back = p.reshape(n // 16, k // 256, 144, 16).transpose(0, 3, 1, 2).reshape(-1)
    np.testing.assert_array_equal(back, w)
    with pytest.raises(ValueError):
        o.interleave_rows(w[: 30 * 2 * 144], 30, k)
