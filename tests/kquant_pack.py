"""Test-side packers: build GGUF k-quant blocks from explicit parameters
(scales, mins, integer codes), so tests know every field of a block and can
derive expected values in closed form. Layouts are those the reference
decodes (E:598-853): Q4_K/Q5_K 6-bit scale packing of get_scale_min_k4
(E:743-749), Q5_K high bits in qh, Q6_K ql/qh split with int8 group scales,
Q8_0 fp16 d + int8 codes."""
import numpy as np


def f16(x) -> int:
    return int(np.float16(x).view(np.uint16))


def pack_scales_k4(sc, m) -> bytes:
    """Inverse of get_scale_min_k4: 8 six-bit scales + 8 six-bit mins -> 12 bytes."""
    q = [0] * 12
    for j in range(8):
        s, mm = int(sc[j]), int(m[j])
        assert 0 <= s < 64 and 0 <= mm < 64
        if j < 4:
            q[j] |= s
            q[j + 4] |= mm
        else:
            q[j + 4] |= (s & 0x0F) | ((mm & 0x0F) << 4)
            q[j - 4] |= (s >> 4) << 6
            q[j] |= (mm >> 4) << 6
    return bytes(q)


def pack_q4_k(d, dmin, sc, m, codes) -> np.ndarray:
    """codes: 256 ints in 0..15, value index k = 64j + 32h + l."""
    codes = np.asarray(codes, np.int64)
    out = bytearray(144)
    out[0:2] = f16(d).to_bytes(2, "little")
    out[2:4] = f16(dmin).to_bytes(2, "little")
    out[4:16] = pack_scales_k4(sc, m)
    for j in range(4):
        for l in range(32):
            lo, hi = codes[64 * j + l], codes[64 * j + 32 + l]
            assert 0 <= lo < 16 and 0 <= hi < 16
            out[16 + 32 * j + l] = int(lo) | (int(hi) << 4)
    return np.frombuffer(bytes(out), np.uint8)


def pack_q5_k(d, dmin, sc, m, codes) -> np.ndarray:
    """codes: 256 ints in 0..31."""
    codes = np.asarray(codes, np.int64)
    out = bytearray(176)
    out[0:2] = f16(d).to_bytes(2, "little")
    out[2:4] = f16(dmin).to_bytes(2, "little")
    out[4:16] = pack_scales_k4(sc, m)
    for j in range(4):
        for l in range(32):
            lo, hi = int(codes[64 * j + l]), int(codes[64 * j + 32 + l])
            assert 0 <= lo < 32 and 0 <= hi < 32
            out[48 + 32 * j + l] = (lo & 15) | ((hi & 15) << 4)
            out[16 + l] |= ((lo >> 4) << (2 * j)) | ((hi >> 4) << (2 * j + 1))
    return np.frombuffer(bytes(out), np.uint8)


def pack_q6_k(d, sc, codes) -> np.ndarray:
    """codes: 256 ints in 0..63 (value = code - 32); sc: 16 int8 group scales
    for values [16g, 16g + 16)."""
    codes = np.asarray(codes, np.int64)
    out = bytearray(210)
    for half in range(2):
        for l in range(32):
            q = [int(codes[128 * half + 32 * i + l]) for i in range(4)]
            assert all(0 <= v < 64 for v in q)
            out[64 * half + l] = (q[0] & 15) | ((q[2] & 15) << 4)
            out[64 * half + 32 + l] = (q[1] & 15) | ((q[3] & 15) << 4)
            out[128 + 32 * half + l] = (q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6)
    out[192:208] = np.asarray(sc, np.int8).tobytes()
    out[208:210] = f16(d).to_bytes(2, "little")
    return np.frombuffer(bytes(out), np.uint8)


def q6_group_of_value(k: int) -> int:
    """Scale index of value k in a Q6_K block: sc[8*half + l//16 + 2*i]
    for k = 128*half + 32*i + l (E:712-740)."""
    half, r = divmod(k, 128)
    i, l = divmod(r, 32)
    return 8 * half + l // 16 + 2 * i


def pack_q8_0(d, codes) -> np.ndarray:
    out = bytearray(34)
    out[0:2] = f16(d).to_bytes(2, "little")
    out[2:34] = np.asarray(codes, np.int8).tobytes()
    return np.frombuffer(bytes(out), np.uint8)


def expand_sub(vals8):
    """8 per-sub-block values -> 256 per-value values (sub-block = k // 32)."""
    return np.repeat(np.asarray(vals8, np.int64), 32)
