"""The oracle's GGUF restatements on the CPU.

ggml's block decoders (Q2_K .. Q6_K, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0) reach
the reference through the gguf package (asdsl/io/gguf_loader.py:150-181),
which is absent here, so they are pinned by hand-worked blocks and by the
layouts' invariants: each scale field, code and high bit moves exactly the
weights the layout assigns it, with the value the formula gives.  The
lossless Q4_K -> ASDSL Q4_K rearrangement is checked through the ASDSL GEMV
(oracle_gemv_q4km, pinned against the reference's compiled kernel): a wrong
field or nibble in either the decoder or the rearrangement changes the
product.  The symmetric requantization is pinned by exact groups, ties,
the floors, and the product package's numpy restatement of the reference's
quantize_weights."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2


def _f16(v) -> np.ndarray:
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def _q4k_block(d=1.0, dmin=0.0, scales=(0,) * 8, mins=(0,) * 8, codes=None) -> np.ndarray:
    """A ggml Q4_K block written field by field from the layout: byte j (j <
    4) = scale j low 6 bits | top 2 bits of scale j+4; byte 4+j the same for
    the mins; byte 8+j = low 4 bits of scale j+4 | low 4 bits of min j+4 << 4;
    code l of sub-block j in byte 16 + 32*(j//2) + l, low nibble for even j."""
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(d), _f16(dmin)
    for j in range(4):
        b[4 + j] = (scales[j] & 63) | ((scales[j + 4] >> 4) << 6)
        b[8 + j] = (mins[j] & 63) | ((mins[j + 4] >> 4) << 6)
        b[12 + j] = (scales[j + 4] & 15) | ((mins[j + 4] & 15) << 4)
    codes = np.zeros(256, np.int64) if codes is None else np.asarray(codes)
    for j in range(8):
        for l in range(32):
            b[16 + 32 * (j // 2) + l] |= int(codes[32 * j + l]) << (4 * (j & 1))
    return b


@pytest.mark.parametrize("j", range(8))
def test_q4k_each_scale_field_moves_its_sub_block(j):
    rng = np.random.default_rng(j)
    codes = rng.integers(0, 16, 256)
    sc = [0] * 8
    sc[j] = 37 + j  # exercises the top bits for j >= 4 (37..44 > 15)
    w = oracle.dequant_gguf_q4k(_q4k_block(d=0.5, scales=sc, codes=codes), 1)
    want = np.zeros(256, np.float32)
    want[32 * j:32 * j + 32] = np.float32(0.5 * sc[j]) * codes[32 * j:32 * j + 32]
    assert np.array_equal(w, want)


@pytest.mark.parametrize("j", range(8))
def test_q4k_each_min_field_moves_its_sub_block(j):
    mins = [0] * 8
    mins[j] = 63 - j
    w = oracle.dequant_gguf_q4k(_q4k_block(d=2.0, dmin=0.25, mins=mins, codes=np.full(256, 9)), 1)
    want = np.zeros(256, np.float32)
    want[32 * j:32 * j + 32] = -np.float32(0.25 * mins[j])
    assert np.array_equal(w, want)


def test_q4k_formula_rounding_and_block_order():
    """w = f32(d*sc)*q - f32(dmin*m), two fp32 roundings per weight, block b
    at weights 256b.."""
    rng = np.random.default_rng(7)
    blocks, want = [], []
    for _ in range(3):
        d, dm = np.float16(rng.uniform(0.001, 0.02)), np.float16(rng.uniform(0.001, 0.02))
        sc, mn, codes = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        blocks.append(_q4k_block(float(d), float(dm), sc, mn, codes))
        d1 = (np.float32(d) * sc.astype(np.float32)).repeat(32)
        m1 = (np.float32(dm) * mn.astype(np.float32)).repeat(32)
        want.append(d1 * codes.astype(np.float32) - m1)
    assert np.array_equal(oracle.dequant_gguf_q4k(np.concatenate(blocks), 3), np.concatenate(want))


def _q6k_block(d, scales, codes) -> np.ndarray:
    """ggml Q6_K from the layout: per half h of 128, code 32k+l (k < 4, l <
    32) keeps its low 4 bits in byte 64h + l + 32(k&1) (low nibble for k < 2)
    and its high 2 bits at bits 2k of byte 128 + 32h + l; int8 scale g (per
    16 weights) at byte 192 + g; fp16 d at 208."""
    b = np.zeros(210, np.uint8)
    for h in range(2):
        for k in range(4):
            for l in range(32):
                c = int(codes[128 * h + 32 * k + l])
                b[64 * h + l + 32 * (k & 1)] |= (c & 15) << (0 if k < 2 else 4)
                b[128 + 32 * h + l] |= (c >> 4) << (2 * k)
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    b[208:210] = _f16(d)
    return b


@pytest.mark.parametrize("g", [0, 3, 5, 10, 15])
def test_q6k_each_scale_moves_its_16_weights(g):
    rng = np.random.default_rng(g)
    codes = rng.integers(0, 64, 256)
    scales = [0] * 16
    scales[g] = -77 + g
    w = oracle.dequant_gguf_q6k(_q6k_block(0.125, scales, codes), 1)
    # scale g covers 16 weights: half g // 8, quarter (g % 8) // 2, l in 16*(g % 2)..
    h, k, l0 = g // 8, (g % 8) // 2, 16 * (g % 2)
    idx = 128 * h + 32 * k + l0 + np.arange(16)
    want = np.zeros(256, np.float32)
    want[idx] = np.float32(0.125 * scales[g]) * (codes[idx] - 32).astype(np.float32)
    assert np.array_equal(w, want)


def test_q6k_codes_span_six_bits():
    codes = np.arange(256) % 64
    w = oracle.dequant_gguf_q6k(_q6k_block(1.0, [1] * 16, codes), 1)
    assert np.array_equal(w, (codes - 32).astype(np.float32))


def test_q4k_rearrangement_through_the_asdsl_gemv():
    """ggml Q4_K blocks -> ASDSL Q4_K -> oracle_gemv_q4km equals the ggml
    decode times the same int8 activation: sum over sub-blocks of xs *
    (d1 * sum q*xq - m1 * sum xq)."""
    rng = np.random.default_rng(3)
    M, K = 6, 512
    nb = M * K // 256
    blocks = rng.integers(0, 256, nb * 144).astype(np.uint8)
    for b in range(nb):  # finite, moderate d and dmin
        blocks[144 * b:144 * b + 2] = _f16(rng.uniform(0.001, 0.01))
        blocks[144 * b + 2:144 * b + 4] = _f16(rng.uniform(0.001, 0.01))
    q4km = oracle.repack_gguf_q4k_to_q4km(blocks, nb)
    x = rng.standard_normal(K).astype(np.float32)
    y = oracle.gemv_q4km(q4km, x, M, K)
    xq, xs = oracle.quantize_activation_q4k(x)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    w = oracle.dequant_gguf_q4k(blocks, nb).reshape(M, K).astype(np.float64)
    assert rel_l2(y, w @ xd) < 1e-6
    # the rearrangement is a bijection on the fields: d, dmin kept; every
    # byte of a block changes something the GEMV reads
    assert np.array_equal(q4km.reshape(nb, 144)[:, :4], blocks.reshape(nb, 144)[:, :4])
    y0 = y
    for byte in (4, 9, 15, 16, 79, 143):
        mod = blocks.copy()
        mod[byte] ^= 0x11
        assert not np.array_equal(oracle.gemv_q4km(oracle.repack_gguf_q4k_to_q4km(mod, nb), x, M, K), y0), byte


def test_quantize_q4_symmetric_exact_groups_and_floors():
    s = 0.25  # exact in fp16: amax = 7.5 * s gives scale s
    codes = np.array([0, 15, 7, 8, 3, 12, 1, 14] * 4)
    w = ((codes - 7.5) * s).astype(np.float32)
    packed, scales, biases = oracle.quantize_q4_symmetric(w, 32)
    assert scales[0] == np.float32(0.25) and biases[0] == np.float32(-1.875)
    got = np.stack([packed & 15, packed >> 4], -1).reshape(-1)
    assert np.array_equal(got, codes)
    # zero group: amax floored at 1e-5, scale f16(1e-5 / 7.5), divisor
    # floored at 1e-4, every code rint(7.5) = 8
    p0, s0, _ = oracle.quantize_q4_symmetric(np.zeros(32, np.float32), 32)
    assert np.all(p0 == 0x88) and s0[0] == np.float32(np.float16(np.float32(1e-5) / np.float32(7.5)))
    # ties round half to even: w / s + 7.5 = 5.5 -> 6 and 6.5 -> 6; amax itself -> 15
    t = np.array([(5.5 - 7.5) * s, (6.5 - 7.5) * s, 7.5 * s] + [0.0] * 29, np.float32)
    pt, _, _ = oracle.quantize_q4_symmetric(t, 32)
    q = np.stack([pt & 15, pt >> 4], -1).reshape(-1)
    assert q[0] == 6 and q[1] == 6 and q[2] == 15


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_q4_symmetric_matches_the_numpy_restatement(gs):
    from asdsl.quantization.core import quantize_weights

    rng = np.random.default_rng(gs)
    w = (rng.standard_normal((48, 256)) * rng.uniform(1e-4, 0.1, (48, 1))).astype(np.float32)
    w[3] = 0.0
    packed, scales, biases = oracle.quantize_q4_symmetric(w, gs)
    qt = quantize_weights(w, bits=4, group_size=gs, symmetric=True)
    assert np.array_equal(packed, qt.data)
    assert np.array_equal(scales, qt.scales.astype(np.float32))
    assert np.array_equal(biases, (-7.5 * qt.scales.astype(np.float32)).astype(np.float32))


# ----------------------------------------------------------- known answers
# Blocks written byte by byte from ggml's layouts (block_q4_K, block_q5_K,
# block_q6_K, block_q8_0) with the expected weights worked out by hand, so
# that nothing here comes from the code under test.  The 12-byte scale/min
# field of Q4_K and Q5_K encodes scales (1, 2, 3, 4, 50, 20, 63, 5) and mins
# (0, 1, 0, 0, 33, 0, 7, 60): bytes 0-3 hold scale j's low 6 bits and, in
# bits 6-7, the top 2 bits of scale j+4; bytes 4-7 the same for the mins;
# bytes 8-11 the low 4 bits of scale j+4 (low nibble) and min j+4 (high).
KA_SCALES = bytes([0xC1, 0x42, 0xC3, 0x04, 0x80, 0x01, 0x00, 0xC0, 0x12, 0x04, 0x7F, 0xC5])


def known_q4k() -> tuple[np.ndarray, dict]:
    """d = 1.0, dmin = 0.5; byte 83 = 0x97 puts codes 7 (sub-block 4) and
    9 (sub-block 5) at position 3; byte 143 = 0x1F codes 15 (sub-block 6) and
    1 (sub-block 7) at position 31; every other code 0."""
    b = bytearray(144)
    b[0:2], b[2:4] = b"\x00\x3c", b"\x00\x38"
    b[4:16] = KA_SCALES
    b[83], b[143] = 0x97, 0x1F
    return np.frombuffer(bytes(b), np.uint8), {
        0: 0.0, 32: -0.5, 131: 333.5, 163: 180.0, 223: 941.5, 255: -25.0, 128: -16.5, 224: -30.0}


def known_q5k() -> tuple[np.ndarray, dict]:
    """d = 1.0, dmin = 1.0; high-bit byte 16 = 0x01 (bit 0: sub-block 0,
    position 0), byte 23 = 0x10 (bit 4: sub-block 4, position 7), byte 47 =
    0xC0 (bits 6, 7: sub-blocks 6, 7, position 31); low-nibble byte 119 =
    0xA3 (sub-blocks 4/5, position 7: 3 and 10), byte 175 = 0xFF (sub-blocks
    6/7, position 31: 15 and 15)."""
    b = bytearray(176)
    b[0:2], b[2:4] = b"\x00\x3c", b"\x00\x3c"
    b[4:16] = KA_SCALES
    b[16], b[23], b[47] = 0x01, 0x10, 0xC0
    b[119], b[175] = 0xA3, 0xFF
    return np.frombuffer(bytes(b), np.uint8), {
        0: 16.0, 32: -1.0, 135: 917.0, 167: 200.0, 223: 1946.0, 255: 95.0, 63: -1.0, 31: 0.0, 128: -33.0}


def known_q6k() -> tuple[np.ndarray, dict]:
    """d = 0.5 (bytes 208-209); scales 2, -3, 7, -1 at bytes 192, 194, 196,
    198, every other scale 1; at position 5 of the first half the four
    quarters' codes 63, 0, 33, 20: low-nibble byte 5 = 0x1F (quarters 0 and
    2), byte 37 = 0x40 (quarters 1 and 3), high-bit byte 133 = 0x63 (2-bit
    fields 3, 0, 2, 1); every other code 0, i.e. -32 after the offset."""
    b = bytearray(210)
    b[5], b[37], b[133] = 0x1F, 0x40, 0x63
    b[192:208] = bytes([1] * 16)
    b[192], b[194], b[196], b[198] = 2, 0xFD, 7, 0xFF
    b[208:210] = b"\x00\x38"
    return np.frombuffer(bytes(b), np.uint8), {
        5: 31.0, 37: 48.0, 69: 3.5, 101: 6.0, 0: -32.0, 16: -16.0, 32: 48.0, 128: -16.0, 255: -16.0}


def known_q8_0() -> tuple[np.ndarray, dict]:
    """d = 0.25, codes -128, -1, 0, 1, 127, then zeros."""
    b = bytearray(34)
    b[0:2] = b"\x00\x34"
    b[2:7] = bytes([0x80, 0xFF, 0x00, 0x01, 0x7F])
    return np.frombuffer(bytes(b), np.uint8), {0: -32.0, 1: -0.25, 2: 0.0, 3: 0.25, 4: 31.75, 31: 0.0}


def known_q4_0() -> tuple[np.ndarray, dict]:
    """d = 0.5; nibble byte 0 = 0x3A (weight 0 code 10, weight 16 code 3),
    byte 15 = 0xF0 (weight 15 code 0, weight 31 code 15); every other byte
    0x88 (code 8: zero)."""
    b = bytearray(18)
    b[0:2] = b"\x00\x38"
    b[2:18] = bytes([0x88] * 16)
    b[2], b[17] = 0x3A, 0xF0
    return np.frombuffer(bytes(b), np.uint8), {0: 1.0, 16: -2.5, 15: -4.0, 31: 3.5, 1: 0.0, 30: 0.0}


def known_q4_1() -> tuple[np.ndarray, dict]:
    """d = 0.25, m = -1.0; nibble byte 2 = 0x5C (weight 2 code 12, weight 18
    code 5); every other code 0."""
    b = bytearray(20)
    b[0:2], b[2:4] = b"\x00\x34", b"\x00\xbc"
    b[4 + 2] = 0x5C
    return np.frombuffer(bytes(b), np.uint8), {2: 2.0, 18: 0.25, 0: -1.0, 31: -1.0}


def known_q5_0() -> tuple[np.ndarray, dict]:
    """d = 1.0; high-bit word with bits 0 and 31 set (bytes 01 00 00 80);
    nibble byte 0 = 0x21 (weight 0: 1 | 16, weight 16: 2), byte 15 = 0xF0
    (weight 15: 0, weight 31: 15 | 16); every other code 0, i.e. -16."""
    b = bytearray(22)
    b[0:2] = b"\x00\x3c"
    b[2:6] = bytes([0x01, 0x00, 0x00, 0x80])
    b[6], b[21] = 0x21, 0xF0
    return np.frombuffer(bytes(b), np.uint8), {0: 1.0, 16: -14.0, 15: -16.0, 31: 15.0, 5: -16.0}


def known_q5_1() -> tuple[np.ndarray, dict]:
    """d = 0.5, m = 2.0; high-bit word with bit 16 set (byte 2 = 0x01);
    nibble byte 0 = 0x37 (weight 0: 7, weight 16: 3 | 16); every other code
    0."""
    b = bytearray(24)
    b[0:2], b[2:4] = b"\x00\x38", b"\x00\x40"
    b[4 + 2] = 0x01
    b[8] = 0x37
    return np.frombuffer(bytes(b), np.uint8), {0: 5.5, 16: 11.5, 1: 2.0, 31: 2.0}


def known_q2k() -> tuple[np.ndarray, dict]:
    """d = 1.0, dmin = 0.5 (bytes 80-83).  Code byte 0 (qs at 16) = 0xE4
    holds codes 0, 1, 2, 3 for weights 0, 32, 64, 96 (scales 0, 2, 4, 6:
    bytes 0x21, 0x03, 0x15, 0xF2, low nibble the scale, high the min); code
    byte 51 = 0x02 gives weight 128 + 16 + 3 = 147 code 2 under scale 9
    (0x47).  Scale 1 is zero: weight 16 is 0."""
    b = bytearray(84)
    b[0], b[2], b[4], b[6], b[9] = 0x21, 0x03, 0x15, 0xF2, 0x47
    b[16] = 0xE4
    b[16 + 51] = 0x02
    b[80:82], b[82:84] = b"\x00\x3c", b"\x00\x38"
    return np.frombuffer(bytes(b), np.uint8), {
        0: -1.0, 1: -1.0, 32: 3.0, 64: 9.5, 96: -1.5, 147: 12.0, 16: 0.0}


def known_q3k() -> tuple[np.ndarray, dict]:
    """d = 0.5 (bytes 108-109).  Scale 0 = 5 | 2 << 4 = 37 (byte 96 low
    nibble 5, byte 104 bits 0-1 = 2): dl = 0.5 * 5; scale 15 = 10 | 1 << 4 =
    26 (byte 103 high nibble 10, byte 107 bits 6-7 = 1): dl = -3; every other
    scale 0, i.e. -32: dl = -16.  Weight 0: code byte 32 = 3, mask byte 0
    bit 0 set: 3.  Weight 245 (n 1, j 3, h 1, l 5): code byte 32 + 53 bits
    6-7 = 3, mask byte 21 bit 7 set: 3.  Weights 1, 241 and 16: code 0 with
    the mask bit clear: -4."""
    b = bytearray(110)
    b[96], b[104], b[103], b[107] = 0x05, 0x02, 0xA0, 0x40
    b[32], b[0] = 0x03, 0x01
    b[32 + 53], b[21] = 0xC0, 0x80
    b[108:110] = b"\x00\x38"
    return np.frombuffer(bytes(b), np.uint8), {
        0: 7.5, 1: -10.0, 2: -10.0, 245: -9.0, 241: 12.0, 16: 64.0}


KNOWN = {"q4k": (known_q4k, oracle.dequant_gguf_q4k, 256), "q5k": (known_q5k, oracle.dequant_gguf_q5k, 256),
         "q6k": (known_q6k, oracle.dequant_gguf_q6k, 256), "q8_0": (known_q8_0, oracle.dequant_gguf_q8_0, 32),
         "q2k": (known_q2k, oracle.dequant_gguf_q2k, 256), "q3k": (known_q3k, oracle.dequant_gguf_q3k, 256),
         **{k: (f, lambda blk, n, k=k: oracle.dequant_gguf_legacy(k, blk, n), 32)
            for k, f in (("q4_0", known_q4_0), ("q4_1", known_q4_1), ("q5_0", known_q5_0), ("q5_1", known_q5_1))}}


@pytest.mark.parametrize("kind", sorted(KNOWN))
def test_known_answer_blocks(kind):
    make, decode, n = KNOWN[kind]
    blk, want = make()
    w = decode(blk, 1)
    assert w.shape == (n,)
    for i, v in want.items():
        assert w[i] == np.float32(v), (kind, i, w[i], v)


@pytest.mark.parametrize("j", range(8))
def test_q5k_each_high_bit_moves_its_weight(j):
    """Bit j of high-bit byte l is the fifth bit of weight 32j + l and of no
    other weight (d = 1, scales 1, mins 0, all low nibbles 0)."""
    b = np.zeros(176, np.uint8)
    b[0:2] = _f16(1.0)
    b[4:8] = 1  # scales 0-3 = 1 (and the top bits of scales 4-7 zero)
    b[12:16] = 1  # scales 4-7 = 1, mins 4-7 = 0
    for l in (0, 13, 31):
        blk = b.copy()
        blk[16 + l] = 1 << j
        w = oracle.dequant_gguf_q5k(blk, 1)
        want = np.zeros(256, np.float32)
        want[32 * j + l] = 16.0
        assert np.array_equal(w, want), (j, l)


@pytest.mark.parametrize("kind", ["q4_0", "q4_1", "q5_0", "q5_1"])
def test_legacy_each_code_and_high_bit_moves_one_weight(kind):
    """Nibble byte j moves weight j (low nibble) and weight j + 16 (high)
    only, and bit i of the Q5 high-bit word moves weight i only, by d
    times the code change (d = 1, m = 0)."""
    nb = oracle.LEGACY_BLOCK_BYTES[kind]
    has_m = nb in (20, 24)
    has_h = nb in (22, 24)
    codes_at = (4 if has_m else 2) + (4 if has_h else 0)
    base = np.zeros(nb, np.uint8)
    base[0:2] = _f16(1.0)
    w0 = oracle.dequant_gguf_legacy(kind, base, 1)
    for j in (0, 7, 15):
        for hi in (0, 1):
            blk = base.copy()
            blk[codes_at + j] = 0x0B << (4 * hi)
            diff = oracle.dequant_gguf_legacy(kind, blk, 1) - w0
            want = np.zeros(32, np.float32)
            want[j + 16 * hi] = 11.0
            assert np.array_equal(diff, want), (kind, j, hi)
    if has_h:
        for i in (0, 9, 16, 31):
            blk = base.copy()
            word = np.frombuffer(np.uint32(1 << i).tobytes(), np.uint8)
            at = 4 if has_m else 2
            blk[at:at + 4] = word
            diff = oracle.dequant_gguf_legacy(kind, blk, 1) - w0
            want = np.zeros(32, np.float32)
            want[i] = 16.0
            assert np.array_equal(diff, want), (kind, i)


@pytest.mark.parametrize("q3", [False, True])
def test_q2k_q3k_each_code_field_moves_its_weight(q3):
    """Bits 2j..2j+1 of code byte 32n + 16h + l move weight 128n + 32j + 16h
    + l and no other; for Q3_K bit 4n + j of mask byte 16h + l moves that
    same weight by 4 steps; each 6-bit (Q3_K) or 4-bit (Q2_K) scale moves
    its 16 weights only."""
    nb, dec = (110, oracle.dequant_gguf_q3k) if q3 else (84, oracle.dequant_gguf_q2k)
    qs_at = 32 if q3 else 16
    base = np.zeros(nb, np.uint8)
    if q3:
        base[108:110] = _f16(1.0)
        base[96:104] = 0x11  # every scale's low 4 bits 1, top bits 0: scale 1 - 32 = -31
    else:
        base[80:82] = _f16(1.0)
        base[0:16] = 0x01  # every scale 1, min 0
    w0 = dec(base, 1)
    for n in (0, 1):
        for j in range(4):
            for h in (0, 1):
                for l in (0, 11):
                    wi = 128 * n + 32 * j + 16 * h + l
                    blk = base.copy()
                    blk[qs_at + 32 * n + 16 * h + l] = 2 << (2 * j)
                    diff = dec(blk, 1) - w0
                    assert np.flatnonzero(diff).tolist() == [wi], (q3, wi)
                    if q3:
                        blk = base.copy()
                        blk[16 * h + l] = 1 << (4 * n + j)
                        diff = dec(blk, 1) - w0
                        assert np.flatnonzero(diff).tolist() == [wi], (q3, wi, "mask")
                        assert diff[wi] == np.float32(-31.0 * 4), (q3, wi)
    if not q3:  # every code 1, so that a scale change shows
        base[16:80] = 0x55
        w0 = dec(base, 1)
    for k in range(16):
        blk = base.copy()
        if q3:  # raise scale k's top 2 bits to 1: the scale moves by 16
            blk[104 + k % 4] = 1 << (2 * (k // 4))
        else:
            blk[k] = 0x03
        changed = np.flatnonzero(dec(blk, 1) != w0)
        n, r = divmod(k, 8)
        j, h = divmod(r, 2)
        want = [128 * n + 32 * j + 16 * h + l for l in range(16)]
        assert changed.tolist() == want, (q3, k)
