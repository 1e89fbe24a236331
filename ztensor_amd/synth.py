"""Seeded synthetic weights and activations for the decode-path workloads.

Every generator returns the reference's own serialised format (the bytes
RawBytes()/NewXStorageFromRaw use), so the same arrays feed the oracle and,
after the load-time repack, the GPU.  Distributions follow the benchmark
configurations of this path:

  Q4_0     nibbles U[0,15], fp16 block scale |N(0,1)|*0.02, fp32 x ~ N(0,1)
  Q8_0     int8 U[-127,127], fp32 block scale |N(0,1)|*0.02
  W4A16    uint4 U[0,15], group 128, fp16 scales |N(0,1)|*0.02, zero-point 8,
           fp16 x ~ N(0,1)
  IQ4_NL   nibbles U[0,15], fp16 block scale |N(0,1)|*0.01, fp16 x ~ N(0,1)
  Ternary  w in {-1,0,+1} with p = {.25,.5,.25}, one fp32 weight scale,
           int8 x = clip(round(N(0,1)*32), -127, 127) with an fp32 scale
  Q4_K/Q5_K codes U[0,15] / U[0,31], 6-bit sub-block scales and mins
           U[0,63], fp16 d |N(0,1)|*0.002 and dmin |N(0,1)|*0.001
  Q6_K     codes U[0,63], int8 sub-block scales U[-64,63], fp16 d
           |N(0,1)|*0.0005
  Q5_0     codes U[0,31], fp16 block scale |N(0,1)|*0.02
  (the K-quant and Q5_0 configurations take fp32 x ~ N(0,1))

Seeds are 0x5EED0000 + 16*config + shape (numpy PCG64), so any host
regenerates identical inputs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 0x5EED0000


def seed_for(config: int, shape: int = 0) -> int:
    return SEED_BASE + 16 * config + shape


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> fp16 bits (round to nearest even) as uint16."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


# --------------------------------------------------------------- packers


def pack_q4_0(nib: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Nibbles [nblk,32] (0..15) and fp16 scale bits [nblk] -> 18-byte Q4_0
    blocks (tensor/quantized.go:146-156): low nibble = element j, high
    nibble = element j+16."""
    nib = nib.reshape(-1, 32).astype(np.uint8)
    nblk = nib.shape[0]
    out = np.empty((nblk, 18), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nblk, 1).view(np.uint8)
    out[:, 2:] = nib[:, :16] | (nib[:, 16:] << 4)
    return out.reshape(-1)


def pack_iq4nl(nib: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Nibbles [nblk,32] -> 18-byte IQ4_NL blocks, interleaved order
    (tensor/iq4_storage.go:36-46): byte i = element 2i | element 2i+1 << 4."""
    nib = nib.reshape(-1, 32).astype(np.uint8)
    nblk = nib.shape[0]
    out = np.empty((nblk, 18), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nblk, 1).view(np.uint8)
    out[:, 2:] = nib[:, 0::2] | (nib[:, 1::2] << 4)
    return out.reshape(-1)


def pack_q8_0(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """int8 [nblk,32] and fp32 scales [nblk] -> 36-byte Q8_0 blocks
    (tensor/quantized.go:425-438)."""
    q = q.reshape(-1, 32).astype(np.int8)
    nblk = q.shape[0]
    out = np.empty((nblk, 36), np.uint8)
    out[:, 0:4] = scale.astype("<f4").reshape(nblk, 1).view(np.uint8)
    out[:, 4:] = q.view(np.uint8)
    return out.reshape(-1)


def pack_nibbles_interleaved(q: np.ndarray) -> np.ndarray:
    """uint4 values [.., K] -> bytes [.., K/2], element j at the low nibble
    of byte j/2 when even, high when odd (GPTQ bits=4,
    tensor/quantized_gptq.go:110-116; AWQ words, tensor/quantized_awq.go:97-105)."""
    q = q.astype(np.uint8)
    return q[..., 0::2] | (q[..., 1::2] << 4)


def pack_ternary(w: np.ndarray) -> np.ndarray:
    """{-1,0,1} values (flat, row-major) -> 2-bit codes, 4 per byte, element
    i at bits 2*(i%4) of byte i/4 (tensor/ternary_storage.go:49-62)."""
    codes = (w.reshape(-1).astype(np.int16) + 1).astype(np.uint8)
    pad = (-codes.size) % 4
    # NewTernaryStorage zero-fills its bytes, so unused codes of the last byte are 00.
    codes = np.concatenate([codes, np.zeros(pad, np.uint8)])
    c = codes.reshape(-1, 4)
    out = c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)
    return out.astype(np.uint8)


def pack_kq_scales_mins(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """6-bit scales and mins [nsb, 8] -> the 12 packed bytes [nsb, 12] of a
    Q4_K / Q5_K super-block, written as the reference's test builders write
    them (tensor/quantized_kquant_test.go:87-94): bytes 0-3 hold scales 0-3
    with the top two bits of scales 4-7, bytes 4-7 the same for the mins,
    bytes 8-11 the low nibbles of scales 4-7 and (high nibble) mins 4-7."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((mn[:, 4:8] & 0xF) << 4)
    return out


def pack_q4_k(q: np.ndarray, sc: np.ndarray, mn: np.ndarray, d_bits: np.ndarray, dmin_bits: np.ndarray) -> np.ndarray:
    """Codes [nsb, 256] (0..15) -> 144-byte Q4_K super-blocks
    (tensor/quantized_kquant_test.go:80-128): group g's 32 bytes hold value
    64g+l in the low nibble of byte l and 64g+32+l in the high nibble."""
    q = q.reshape(-1, 256).astype(np.uint8)
    nsb = q.shape[0]
    out = np.empty((nsb, 144), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nsb, 1).view(np.uint8)
    out[:, 2:4] = dmin_bits.astype("<u2").reshape(nsb, 1).view(np.uint8)
    out[:, 4:16] = pack_kq_scales_mins(sc, mn)
    g = q.reshape(nsb, 4, 64)
    out[:, 16:] = (g[:, :, :32] | (g[:, :, 32:] << 4)).reshape(nsb, 128)
    return out.reshape(-1)


def pack_q5_k(q: np.ndarray, sc: np.ndarray, mn: np.ndarray, d_bits: np.ndarray, dmin_bits: np.ndarray) -> np.ndarray:
    """Codes [nsb, 256] (0..31) -> 176-byte Q5_K super-blocks
    (tensor/quantized_kquant_test.go:414-468): the low four bits as Q4_K,
    the fifth bit of value 64g+l at bit 2g of qh byte l and of value
    64g+32+l at bit 2g+1."""
    q = q.reshape(-1, 256).astype(np.uint8)
    nsb = q.shape[0]
    out = np.empty((nsb, 176), np.uint8)
    out[:, 0:144] = pack_q4_k(q & 0xF, sc, mn, d_bits, dmin_bits).reshape(nsb, 144)
    g = (q >> 4).reshape(nsb, 4, 2, 32)  # [sb, group, half, l]
    qh = np.zeros((nsb, 32), np.uint8)
    for grp in range(4):
        for half in range(2):
            qh |= g[:, grp, half, :] << (2 * grp + half)
    out[:, 144:176] = qh
    return out.reshape(-1)


def pack_q6_k(q: np.ndarray, sc: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Codes [nsb, 256] (0..63, value q-32) and int8 scales [nsb, 16] ->
    210-byte Q6_K super-blocks (tensor/quantized_kquant_test.go:263-292):
    half h, l < 32: ql[64h+l] = q1 & 15 | (q3 & 15) << 4,
    ql[64h+32+l] = q2 & 15 | (q4 & 15) << 4, qh[32h+l] = the top two bits of
    q1, q2, q3, q4 at bits 0, 2, 4, 6, with q1..q4 the values 128h + l,
    +32, +64, +96."""
    q = q.reshape(-1, 2, 4, 32).astype(np.uint8)  # [sb, half, quarter, l]
    nsb = q.shape[0]
    out = np.empty((nsb, 210), np.uint8)
    q1, q2, q3, q4 = q[:, :, 0], q[:, :, 1], q[:, :, 2], q[:, :, 3]
    ql = np.empty((nsb, 2, 64), np.uint8)
    ql[:, :, :32] = (q1 & 0xF) | ((q3 & 0xF) << 4)
    ql[:, :, 32:] = (q2 & 0xF) | ((q4 & 0xF) << 4)
    qh = ((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) | (((q3 >> 4) & 3) << 4) | (((q4 >> 4) & 3) << 6)
    out[:, 0:128] = ql.reshape(nsb, 128)
    out[:, 128:192] = qh.reshape(nsb, 64)
    out[:, 192:208] = sc.reshape(nsb, 16).astype(np.int8).view(np.uint8)
    out[:, 208:210] = d_bits.astype("<u2").reshape(nsb, 1).view(np.uint8)
    return out.reshape(-1)


def pack_q5_0(q: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """Codes [nblk, 32] (0..31, value q-16) -> 22-byte Q5_0 blocks
    (tensor/quantized_q5_0.go:14-45): [fp16 d][uint32 qh: bit j = fifth bit
    of value j][16 bytes: value j low nibble | value j+16 low nibble << 4]."""
    q = q.reshape(-1, 32).astype(np.uint32)
    nblk = q.shape[0]
    out = np.empty((nblk, 22), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nblk, 1).view(np.uint8)
    qh = (((q >> 4) & 1) << np.arange(32, dtype=np.uint32)).sum(axis=1).astype("<u4")
    out[:, 2:6] = qh.reshape(nblk, 1).view(np.uint8)
    out[:, 6:22] = ((q[:, :16] & 0xF) | ((q[:, 16:] & 0xF) << 4)).astype(np.uint8)
    return out.reshape(-1)


def pack_gguf_q8_0(q: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    """int8 [nblk, 32] and fp16 scale bits [nblk] -> 34-byte GGUF Q8_0 blocks
    (tensor/mmap_storage.go:94-96, 265-284): [fp16 d LE][32 x int8]."""
    q = q.reshape(-1, 32).astype(np.int8)
    nblk = q.shape[0]
    out = np.empty((nblk, 34), np.uint8)
    out[:, 0:2] = d_bits.astype("<u2").reshape(nblk, 1).view(np.uint8)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def gguf_q8_0(rows: int, K: int, seed: int) -> np.ndarray:
    """GGUF Q8_0 weights [rows, K]: int8 U[-127,127], fp16 d |N(0,1)|*0.02."""
    g = rng(seed)
    nblk = rows * K // 32
    q = g.integers(-127, 128, size=(nblk, 32), dtype=np.int16).astype(np.int8)
    d = f16_bits(np.abs(g.standard_normal(nblk, dtype=np.float32)) * np.float32(0.02))
    return pack_gguf_q8_0(q, d)


# ------------------------------------------------------------ workloads


@dataclass
class Q4Weights:
    rows: int
    K: int
    raw: np.ndarray  # 18-byte blocks


@dataclass
class Q8Weights:
    rows: int
    K: int
    raw: np.ndarray  # 36-byte blocks


@dataclass
class IQ4Weights:
    rows: int
    K: int
    raw: np.ndarray  # 18-byte blocks


@dataclass
class W4Weights:
    rows: int
    K: int
    group: int
    packed: np.ndarray  # uint8 [rows, K/2]
    scales: np.ndarray  # uint16 fp16 bits [rows, K/group]
    zeros: np.ndarray  # uint16 fp16 bits [rows, K/group]


@dataclass
class TernaryWeights:
    rows: int
    K: int
    raw: np.ndarray  # flat 2-bit packing, ceil(rows*K/4) bytes
    w_scale: np.float32 = field(default_factory=lambda: np.float32(1.0))


def q4_0(rows: int, K: int, seed: int) -> Q4Weights:
    g = rng(seed)
    nblk = rows * K // 32
    nib = g.integers(0, 16, size=(nblk, 32), dtype=np.uint8)
    d = f16_bits(np.abs(g.standard_normal(nblk, dtype=np.float32)) * np.float32(0.02))
    return Q4Weights(rows, K, pack_q4_0(nib, d))


def q8_0(rows: int, K: int, seed: int) -> Q8Weights:
    g = rng(seed)
    nblk = rows * K // 32
    q = g.integers(-127, 128, size=(nblk, 32), dtype=np.int16).astype(np.int8)
    s = (np.abs(g.standard_normal(nblk, dtype=np.float32)) * np.float32(0.02)).astype(np.float32)
    return Q8Weights(rows, K, pack_q8_0(q, s))


def iq4nl(rows: int, K: int, seed: int) -> IQ4Weights:
    g = rng(seed)
    nblk = rows * K // 32
    nib = g.integers(0, 16, size=(nblk, 32), dtype=np.uint8)
    d = f16_bits(np.abs(g.standard_normal(nblk, dtype=np.float32)) * np.float32(0.01))
    return IQ4Weights(rows, K, pack_iq4nl(nib, d))


def w4a16(rows: int, K: int, seed: int, group: int = 128, zero_point: float = 8.0) -> W4Weights:
    g = rng(seed)
    q = g.integers(0, 16, size=(rows, K), dtype=np.uint8)
    ng = K // group
    s = f16_bits(np.abs(g.standard_normal((rows, ng), dtype=np.float32)) * np.float32(0.02))
    z = np.full((rows, ng), f16_bits(np.float32(zero_point)), np.uint16)
    return W4Weights(rows, K, group, pack_nibbles_interleaved(q), s, z)


def ternary(rows: int, K: int, seed: int) -> TernaryWeights:
    g = rng(seed)
    w = g.choice(np.array([-1, 0, 1], np.int8), size=rows * K, p=[0.25, 0.5, 0.25])
    w_scale = np.float32(np.abs(g.standard_normal(dtype=np.float32)) * np.float32(0.02) + np.float32(0.01))
    return TernaryWeights(rows, K, pack_ternary(w), w_scale)


@dataclass
class KQWeights:
    fmt: str  # "q4_k", "q5_k", "q6_k" or "q5_0"
    rows: int
    K: int
    raw: np.ndarray  # contiguous super-blocks / blocks as RawBytes() holds them


KQ_BLOCK = {"q4_k": (256, 144), "q5_k": (256, 176), "q6_k": (256, 210), "q5_0": (32, 22)}


def kquant(fmt: str, rows: int, K: int, seed: int) -> KQWeights:
    """Seeded K-quant / Q5_0 weights of shape [rows, K] (blocks along K)."""
    g = rng(seed)
    vals, _ = KQ_BLOCK[fmt]
    nb = rows * K // vals
    if fmt in ("q4_k", "q5_k"):
        q = g.integers(0, 16 if fmt == "q4_k" else 32, size=(nb, 256), dtype=np.uint8)
        sc = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        mn = g.integers(0, 64, size=(nb, 8), dtype=np.uint8)
        d = f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.002))
        dmin = f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.001))
        raw = (pack_q4_k if fmt == "q4_k" else pack_q5_k)(q, sc, mn, d, dmin)
    elif fmt == "q6_k":
        q = g.integers(0, 64, size=(nb, 256), dtype=np.uint8)
        sc = g.integers(-64, 64, size=(nb, 16), dtype=np.int16).astype(np.int8)
        d = f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.0005))
        raw = pack_q6_k(q, sc, d)
    else:
        q = g.integers(0, 32, size=(nb, 32), dtype=np.uint8)
        d = f16_bits(np.abs(g.standard_normal(nb, dtype=np.float32)) * np.float32(0.02))
        raw = pack_q5_0(q, d)
    return KQWeights(fmt, rows, K, raw)


def x_f32(n: int, seed: int) -> np.ndarray:
    return rng(seed ^ 0xA5A5).standard_normal(n, dtype=np.float32)


def x_f16(n: int, seed: int) -> np.ndarray:
    """fp16 activation bits (uint16)."""
    return f16_bits(rng(seed ^ 0xA5A5).standard_normal(n, dtype=np.float32))


def x_i8(n: int, seed: int) -> tuple[np.ndarray, np.float32]:
    g = rng(seed ^ 0xA5A5)
    q = np.clip(np.rint(g.standard_normal(n, dtype=np.float32) * np.float32(32.0)), -127, 127).astype(np.int8)
    x_scale = np.float32(np.float32(1.0) / np.float32(32.0))
    return q, x_scale


# ---------------------------------------------------------- byte counts

def algorithmic_bytes(fmt: str, rows: int, K: int, N: int = 1, group: int = 128, zeros: bool = True) -> int:
    """Bytes one call must move at minimum: weights + scales (+zeros) +
    activations + output, each read or written once."""
    nblk = rows * K // 32
    if fmt == "q4_0":
        return nblk * 18 + 4 * K * N + 4 * rows * N
    if fmt == "q8_0":
        return nblk * 36 + 4 * K * N + 4 * rows * N
    if fmt == "iq4nl":
        return nblk * 18 + 2 * K * N + 4 * rows * N
    if fmt == "q4_0h":  # Q4_0 weights, fp16 activations
        return nblk * 18 + 2 * K * N + 4 * rows * N
    if fmt == "iq4nl32":  # IQ4_NL weights, fp32 activations
        return nblk * 18 + 4 * K * N + 4 * rows * N
    if fmt == "w4a16":
        ng = rows * K // group
        return rows * K // 2 + 2 * ng * (2 if zeros else 1) + 2 * K * N + 4 * rows * N
    if fmt == "q8_0_gguf":
        return nblk * 34 + 4 * K * N + 4 * rows * N
    if fmt in KQ_BLOCK:
        vals, nbytes = KQ_BLOCK[fmt]
        return rows * K // vals * nbytes + 4 * K * N + 4 * rows * N
    if fmt == "ternary_i8":
        return rows * ((K + 3) // 4) + K * N + 4 * rows * N + 8
    if fmt == "ternary_f32":
        return rows * ((K + 3) // 4) + 4 * K * N + 4 * rows * N
    if fmt == "int4":
        ng = rows * (-(-K // group))
        return rows * K // 2 + 5 * ng + 4 * K * N + 4 * rows * N
    if fmt == "int8":
        return rows * K + 4 * K * N + 4 * rows * N
    raise ValueError(fmt)


# ---- the Dequantizer registry's byte formats (tensor/quant_registry.go)


def pack_awq4_wire(q: np.ndarray, scales: np.ndarray, zeros: np.ndarray, group: int) -> np.ndarray:
    """The registry's AWQ_4 bytes (tensor/quantized_awq.go:242-305) for the
    flat codes q (uint4 values, any length) with fp16 scale / zero bits per
    group: header (numElements, groupSize, nGroups as uint32 LE), the
    (scale, zero) pairs, then each group's codes as little-endian uint32
    words of 8 nibbles, every group starting on a fresh word."""
    q = np.asarray(q, np.uint8).reshape(-1)
    n = q.size
    ng = -(-n // group)
    parts = [np.array([n, group, ng], "<u4").view(np.uint8),
             np.stack([np.asarray(scales, "<u2"), np.asarray(zeros, "<u2")], axis=1).reshape(-1).view(np.uint8)]
    for gi in range(ng):
        c = q[gi * group:(gi + 1) * group]
        words = np.zeros(-(-c.size // 8), np.uint64)
        for j in range(8):
            sel = c[j::8].astype(np.uint64)
            words[:sel.size] |= sel << np.uint64(4 * j)
        parts.append(words.astype("<u4").view(np.uint8))
    return np.concatenate(parts)


def awq4_wire(n: int, group: int, seed: int) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """(wire bytes, codes, scale bits, zero bits) of n seeded AWQ weights:
    codes U[0,15], fp16 scales |N(0,1)|*0.02, fp16 zeros U[0,15) (not only
    integers, as QuantizeAWQ's zero = -min/scale is not)."""
    g = rng(seed)
    ng = -(-n // group)
    q = g.integers(0, 16, size=n, dtype=np.uint8)
    s = f16_bits(np.abs(g.standard_normal(ng, dtype=np.float32)) * np.float32(0.02))
    z = f16_bits(g.random(ng, dtype=np.float32) * np.float32(15.0))
    return pack_awq4_wire(q, s, z, group), q, s, z


def fp8_wire(codes: np.ndarray, scale: float) -> np.ndarray:
    """The registry's FP8_E4M3 / FP8_E5M2 bytes: 4-byte LE fp32 scale, then
    one code byte per element (tensor/quant_registry.go:190-229)."""
    return np.concatenate([np.array([scale], "<f4").view(np.uint8), np.asarray(codes, np.uint8)])


def iq3s(nblocks: int, seed: int) -> np.ndarray:
    """Seeded IQ3_S super-blocks (tensor/iq3_storage.go:12-29 layout, 110
    bytes each): fp16 d = |N(0,1)| * 0.01, every qs, qh, sign and scale byte
    uniform."""
    g = rng(seed)
    raw = g.integers(0, 256, size=(nblocks, 110), dtype=np.uint8)
    d = f16_bits(np.abs(g.standard_normal(nblocks, dtype=np.float32)) * np.float32(0.01))
    raw[:, 0:2] = d.reshape(-1, 1).view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def iq3s_values(raw: np.ndarray, n: int) -> np.ndarray:
    """The IQ3_S element definition evaluated field by field in numpy (fp64):
    value 32 i + 8 j + 4 h + k of a block = +-d (1 + 2 sc_i) (1 + 2 f), with
    f the 2-bit field k of qs byte 8 i + 2 j + h, sc_i the low (even i) or
    high (odd i) nibble of scale byte 106 + i / 2, and the sign from bit
    k + 4 h of sign byte 74 + 4 i + j."""
    b = np.asarray(raw, np.uint8).reshape(-1, 110)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1, 1)
    v = np.arange(256)
    i, j, h, k = v >> 5, (v >> 3) & 3, (v >> 2) & 1, v & 3
    sc = np.where(i % 2 == 0, b[:, 106 + i // 2] & 15, b[:, 106 + i // 2] >> 4).astype(np.float64)
    f = (b[:, 2 + 8 * i + 2 * j + h] >> (2 * k)) & 3
    neg = (b[:, 74 + 4 * i + j] >> (k + 4 * h)) & 1
    out = d * (1 + 2 * sc) * (1 + 2 * f.astype(np.float64))
    return np.where(neg == 1, -out, out).reshape(-1)[:n]


# ---- int4 / int8 GEMM operands (gemm_int4.h, gemm_int8.h)


def pack_int4(v: np.ndarray) -> np.ndarray:
    """Signed int4 values [-8, 7], row-major with an even row length, two a
    byte: element 2b in the low nibble of byte b (gemm_int4.cu:20-27)."""
    q = (np.asarray(v, np.int16) & 0xF).astype(np.uint8).reshape(v.shape[0], -1)
    return (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)


@dataclass
class Int4Weights:
    v: np.ndarray  # int8 [rows, cols], values -8..7
    packed: np.ndarray  # uint8 [rows, cols/2]
    scales: np.ndarray  # float32 [rows, ngroups]
    zeros: np.ndarray  # uint8 [rows, ngroups]


def int4(rows: int, cols: int, group: int, seed: int, zero_max: int = 15) -> Int4Weights:
    """Random int4 weights, groups of `group` along each row of `cols`
    values (the K of gemm_int4_f32, the out of gemm_int4_f32_rmul)."""
    g = rng(seed)
    v = g.integers(-8, 8, size=(rows, cols), dtype=np.int8)
    ng = -(-cols // group)
    scales = (np.abs(g.standard_normal((rows, ng), dtype=np.float32)) * np.float32(0.02) + np.float32(1e-3)).astype(
        np.float32)
    zeros = g.integers(0, zero_max + 1, size=(rows, ng), dtype=np.uint8)
    return Int4Weights(v, pack_int4(v), scales, zeros)


def int4_dense(w: Int4Weights, group: int) -> np.ndarray:
    """float64 weights (v - zero) * scale, groups along each row."""
    cols = w.v.shape[1]
    gi = np.arange(cols) // group
    return (w.v.astype(np.float64) - w.zeros[:, gi].astype(np.float64)) * w.scales[:, gi].astype(np.float64)


def int8(rows: int, cols: int, seed: int) -> np.ndarray:
    return rng(seed).integers(-128, 128, size=(rows, cols), dtype=np.int8)
