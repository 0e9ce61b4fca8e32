"""Pins the CPU oracle (oracle/) before it is trusted to check the GPU results.

Each oracle function is checked by at least one of:
  * the reference's own known-answer tests, transcribed verbatim
    (dequant.rs:153-169, dequant_k.rs:118-178, dtype.rs:76-95,
    fp8_weight.rs:105-134, fp8_gemm.rs:198-208, linear_layer.rs:129-160,
    safetensors_load.rs:41-66);
  * closed forms fixed by the format (IEEE half -> single for all 65,536
    inputs, the OCP e4m3 table, torch's float8_e4m3fn conversion);
  * an independent numpy restatement of each block format
    (tests/reference_np.py) on thousands of seeded blocks, bit for bit.
"""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import synth
from tests import reference_np as ref


# ---------------------------------------------------------------- f16 -----

def test_f16_corners():  # dequant.rs:153-160
    def f(h):
        return np.uint32(oracle.f16_to_f32_bits(h)).view(np.float32)

    assert f(0x3C00) == 1.0
    assert f(0xBC00) == -1.0
    assert f(0x0000) == 0.0
    assert np.isinf(f(0x7C00))
    assert abs(f(0x0001) - 2.0 ** -24) < 1e-30


def test_f16_exhaustive_against_ieee():
    # numpy's half widening is the IEEE closed form; it keeps NaN payloads
    # exactly as dequant.rs:28 does (mantissa << 13, no quieting).
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.f16_to_f32_bits(int(v)) for v in h], dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got, want)


# ----------------------------------------------------------- geometry -----

def test_block_geometry():  # dtype.rs:85-95
    assert oracle.geometry(8) == (32, 34)
    assert oracle.geometry(10) == (256, 84)
    assert oracle.geometry(11) == (256, 110)
    assert oracle.geometry(12) == (256, 144)
    assert oracle.geometry(13) == (256, 176)
    assert oracle.geometry(14) == (256, 210)
    assert oracle.geometry(0) == (1, 4)
    assert oracle.geometry(2) == (32, 18)
    assert oracle.geometry(6) == (32, 22)
    assert oracle.geometry(99) is None  # dtype.rs:82 Unknown(99) not decodable
    assert oracle.geometry(3) is None   # Q4_1 has no geometry


# --------------------------------------------------------------- KATs -----

def test_q8_0_scales_ints():  # dequant.rs:162-169
    block = bytes([0x00, 0x3C]) + bytes(range(32))
    out = oracle.dequant_block("q8_0", block)
    assert np.array_equal(out, np.arange(32, dtype=np.float32))


def test_q4_k_nibbles_and_high_bits():  # dequant_k.rs:118-129
    block = bytes([0x00, 0x3C, 0x00, 0x00]) + bytes([65] + [1] * 11) + bytes([0x11] * 128)
    out = oracle.dequant_block("q4_k", block)
    assert out.shape == (256,)
    assert np.all(out[0:32] == 1.0)
    assert np.all(out[32:64] == 1.0)
    assert np.all(out[128:160] == 17.0)


def test_q5_k_high_bit_reuse_across_groups():  # dequant_k.rs:132-152
    block = bytearray([0x00, 0x3C, 0x00, 0x00]) + bytearray([1] * 12) + bytearray(32) + bytearray([0x11] * 128)
    assert np.all(oracle.dequant_block("q5_k", block) == 1.0)
    hi = bytearray(block)
    hi[16:48] = bytes([0xFF] * 32)
    assert np.all(oracle.dequant_block("q5_k", hi) == 17.0)
    one = bytearray(block)
    one[16] = 0x01
    out = oracle.dequant_block("q5_k", one)
    assert out[0] == 17.0 and out[1] == 1.0 and out[32] == 1.0


def test_q6_k_signed_values_and_scales():  # dequant_k.rs:155-177
    block = bytearray(208) + bytearray([0x00, 0x3C])
    block[192:208] = bytes([1] * 16)
    assert np.all(oracle.dequant_block("q6_k", block) == -32.0)
    q = bytearray(block)
    q[0] = 0x11
    q[128] = 0xFF
    q[192:200] = bytes([1, 2, 3, 4, 5, 6, 7, 8])
    out = oracle.dequant_block("q6_k", q)
    assert out[0] == 17.0 and out[32] == 48.0 and out[64] == 85.0 and out[96] == 112.0
    lane = bytearray(block)
    lane[192:200] = bytes([1, 2, 3, 4, 5, 6, 7, 8])
    lane[16] = 0x11
    assert oracle.dequant_block("q6_k", lane)[16] == -62.0


# ------------------------------------------- hand-derived KATs ----------
#
# The reference's own Q4_K KAT (dequant_k.rs:118-129) has dmin = 0 and
# qs = 0x11, so it fixes neither the min term nor which nibble feeds which
# sub-block.  The vectors below were worked out by hand from the block
# layouts (dequant_k.rs:8-80, dequant.rs:50-77) and are written as literal
# numbers, one per 32-element sub-block, so that a dropped or sign-flipped
# min, swapped nibbles, a wrong scale_min_k4 branch or a shifted qh mask
# fails.
#
# Scale bytes: for j < 4 sc_j = s[j] & 63, m_j = s[j + 4] & 63; for j >= 4
# sc_j = (s[j + 4] & 0xF) | (s[j - 4] >> 6) << 4, m_j = (s[j + 4] >> 4) |
# (s[j] >> 6) << 4.  With
#   s = 41 82 C3 04 | 41 82 C3 04 | 51 62 73 88
# sc = [1, 2, 3, 4, 17, 34, 51, 8] and m = [1, 2, 3, 4, 21, 38, 55, 8]:
# sc_4 = 0x1 | (0x41 >> 6) << 4 = 17, m_4 = 0x5 | (0x41 >> 6) << 4 = 21, ...
SCALES_BOTH = bytes([0x41, 0x82, 0xC3, 0x04, 0x41, 0x82, 0xC3, 0x04, 0x51, 0x62, 0x73, 0x88])
SCALES_MINS_ONLY = bytes([0, 0, 0, 0, 0x41, 0x82, 0xC3, 0x04, 0x50, 0x60, 0x70, 0x80])   # sc = 0
SCALES_SC_ONLY = bytes([0x41, 0x82, 0xC3, 0x04, 0, 0, 0, 0, 0x01, 0x02, 0x03, 0x08])      # m = 0
F16_ZERO, F16_QUARTER, F16_HALF, F16_ONE = b"\x00\x00", b"\x00\x34", b"\x00\x38", b"\x00\x3c"


def _per_sub_block(values, width=32):
    return np.repeat(np.array(values, dtype=np.float32), width)


def test_q4_k_min_term_hand_derived():
    # d = 0, dmin = 1: every element is -m_j of its sub-block, whatever qs is
    block = F16_ZERO + F16_ONE + SCALES_MINS_ONLY + bytes((7 * i + 3) & 0xFF for i in range(128))
    out = oracle.dequant_block("q4_k", block)
    assert np.array_equal(out, _per_sub_block([-1, -2, -3, -4, -21, -38, -55, -8]))


def test_q4_k_nibble_order_hand_derived():
    # d = 1, dmin = 0, every qs byte 0x21: sub-block 2c takes the low nibbles
    # (q = 1) of chunk c, sub-block 2c + 1 the high nibbles (q = 2)
    block = F16_ONE + F16_ZERO + SCALES_SC_ONLY + bytes([0x21] * 128)
    out = oracle.dequant_block("q4_k", block)
    assert np.array_equal(out, _per_sub_block([1, 4, 3, 8, 17, 68, 51, 16]))


def test_q4_k_scale_and_min_together_hand_derived():
    # d = 0.5, dmin = 0.25, qs = 0x21: y = 0.5 sc_j q - 0.25 m_j
    block = F16_HALF + F16_QUARTER + SCALES_BOTH + bytes([0x21] * 128)
    out = oracle.dequant_block("q4_k", block)
    assert np.array_equal(out, _per_sub_block([0.25, 1.5, 0.75, 3.0, 3.25, 24.5, 11.75, 6.0]))
    # one chunk whose low and high nibbles differ per byte: chunk 1 (sub-blocks
    # 2 and 3) holds bytes 0xF0 then 0x0F alternately
    qs = bytearray([0x21] * 128)
    qs[32:64] = bytes([0xF0, 0x0F] * 16)
    out = oracle.dequant_block("q4_k", F16_HALF + F16_QUARTER + SCALES_BOTH + bytes(qs))
    # sub-block 2 (low nibbles, sc 3, m 3): q = 0 -> -0.75, q = 15 -> 21.75
    assert np.array_equal(out[64:96], np.array([-0.75, 21.75] * 16, np.float32))
    # sub-block 3 (high nibbles, sc 4, m 4): q = 15 -> 29.0, q = 0 -> -1.0
    assert np.array_equal(out[96:128], np.array([29.0, -1.0] * 16, np.float32))


def test_q5_k_min_term_and_high_bits_hand_derived():
    # d = dmin = 1, qs = 0x21, qh[l] = 1 << (l % 8): sub-block j = 2c + h uses
    # qh bit 2c + h, so exactly the elements l = j, j + 8, j + 16, j + 24 of
    # sub-block j get +16.  Per sub-block: (value without, value with the bit)
    qh = bytes(1 << (l % 8) for l in range(32))
    block = F16_ONE + F16_ONE + SCALES_BOTH + qh + bytes([0x21] * 128)
    out = oracle.dequant_block("q5_k", block)
    pairs = [(0, 16), (2, 34), (0, 48), (4, 68), (-4, 268), (30, 574), (-4, 812), (8, 136)]
    want = np.empty(256, np.float32)
    for j, (plain, high) in enumerate(pairs):
        want[32 * j:32 * j + 32] = plain
        want[32 * j + j:32 * j + 32:8] = high
    assert np.array_equal(out, want)
    # with dmin = 0 the min term vanishes: sc_j (q + hi) alone
    out0 = oracle.dequant_block("q5_k", F16_ONE + F16_ZERO + SCALES_BOTH + qh + bytes([0x21] * 128))
    assert out0[0] == 17.0 and out0[1] == 1.0 and out0[32] == 4.0 and out0[32 + 1] == 36.0 and out0[128 + 4] == 289.0


def test_q4_0_nibble_order_hand_derived():
    # d = 1; byte i = i | (15 - i) << 4: element i = i - 8, element 16 + i = 7 - i
    block = F16_ONE + bytes(i | ((15 - i) << 4) for i in range(16))
    out = oracle.dequant_block("q4_0", block)
    want = [-8, -7, -6, -5, -4, -3, -2, -1, 0, 1, 2, 3, 4, 5, 6, 7,
            7, 6, 5, 4, 3, 2, 1, 0, -1, -2, -3, -4, -5, -6, -7, -8]
    assert np.array_equal(out, np.array(want, np.float32))
    # d = 0.5 halves every value; bytes 0x0F / 0xF0 give 7 / -8 and -8 / 7
    out = oracle.dequant_block("q4_0", F16_HALF + bytes([0x0F, 0xF0] * 8))
    assert np.array_equal(out, np.array([3.5, -4.0] * 8 + [-4.0, 3.5] * 8, np.float32))


def test_q5_0_single_high_bits_hand_derived():
    # d = 1; qh bits 3 and 20 set (little-endian u32 0x00100008): element 3
    # (low nibble of byte 3) and element 20 (high nibble of byte 4) get +16
    block = F16_ONE + bytes([0x08, 0x00, 0x10, 0x00]) + bytes(i | ((15 - i) << 4) for i in range(16))
    out = oracle.dequant_block("q5_0", block)
    want = [-16, -15, -14, 3, -12, -11, -10, -9, -8, -7, -6, -5, -4, -3, -2, -1,
            -1, -2, -3, -4, 11, -6, -7, -8, -9, -10, -11, -12, -13, -14, -15, -16]
    assert np.array_equal(out, np.array(want, np.float32))
    # every qh bit set: q - 16 + 16 = the nibble itself
    out = oracle.dequant_block("q5_0", F16_ONE + b"\xff\xff\xff\xff" + bytes([0x0F, 0xF0] * 8))
    assert np.array_equal(out, np.array([15.0, 0.0] * 8 + [0.0, 15.0] * 8, np.float32))


# The reference's Q6_K KAT (dequant_k.rs:155-177) sets only qh[0] = 0xFF and
# ql[0] = 0x11 in half 0, so it cannot tell which 2-bit qh field feeds which
# of a position's four outputs, which ql nibble feeds y[l] and which y[l+64],
# or where the second half's ql / qh / scales start.  Here every field is
# distinct.  Per half h and position l < 32 (dequant_k.rs:87-111):
#   y[l]      = d sc[2 0 + l/16] ((ql[l] & F)      | (qh[l] & 3) << 4        - 32)
#   y[l + 32] = d sc[2 1 + l/16] ((ql[l + 32] & F) | ((qh[l] >> 2) & 3) << 4 - 32)
#   y[l + 64] = d sc[2 2 + l/16] ((ql[l] >> 4)     | ((qh[l] >> 4) & 3) << 4 - 32)
#   y[l + 96] = d sc[2 3 + l/16] ((ql[l + 32] >> 4)| ((qh[l] >> 6) & 3) << 4 - 32)
# with ql, qh, sc offset by 64, 32, 8 bytes in half 1.  Block: d = 1;
# ql = 0x21 x32, 0x43 x32, 0x65 x32, 0x87 x32; qh = 0xE4 x32 (fields 0, 1, 2, 3
# from the low bits up), 0x1B x32 (fields 3, 2, 1, 0); scales 1, -2, 3, -4, ...
# Half 0 codes: 1 | 0 = 1 -> -31; 3 | 16 = 19 -> -13; 2 | 32 = 34 -> 2;
# 4 | 48 = 52 -> 20.  Half 1: 5 | 48 = 53 -> 21; 7 | 32 = 39 -> 7;
# 6 | 16 = 22 -> -10; 8 | 0 = 8 -> -24.  Each code times its two scales
# (l < 16, l >= 16) gives the 16 runs of 16 equal elements below.
Q6K_FIELDS_BLOCK = (bytes([0x21] * 32 + [0x43] * 32 + [0x65] * 32 + [0x87] * 32) + bytes([0xE4] * 32 + [0x1B] * 32)
                    + bytes((s if s > 0 else 256 + s) for s in (1, -2, 3, -4, 5, -6, 7, -8, 9, -10, 11, -12, 13, -14,
                                                                 15, -16)) + F16_ONE)
Q6K_FIELDS_OUT = np.repeat(np.array([-31, 62, -39, 52, 10, -12, 140, -160,
                                     189, -210, 77, -84, -130, 140, -360, 384], np.float32), 16)


def test_q6_k_bit_fields_hand_derived():
    assert len(Q6K_FIELDS_BLOCK) == 210
    out = oracle.dequant_block("q6_k", Q6K_FIELDS_BLOCK)
    assert np.array_equal(out, Q6K_FIELDS_OUT)
    # d = 0.5 halves every element (exact: the products are small integers)
    half = Q6K_FIELDS_BLOCK[:208] + F16_HALF
    assert np.array_equal(oracle.dequant_block("q6_k", half), Q6K_FIELDS_OUT * 0.5)


def test_q6_k_bit_fields_catch_plausible_mistakes():
    # decoders with one plausible slip each, written here only to show that
    # the vector above tells them apart from the reference layout
    def decode(block, swap_qh=False, swap_nibbles=False, same_half=False):
        ql, qh, sc = block[0:128], block[128:192], np.frombuffer(block[192:208], np.int8)
        out = np.zeros(256, np.float32)
        for h in range(2):
            o = 0 if same_half else h
            for l in range(32):
                a, b, hb = ql[64 * o + l], ql[64 * o + l + 32], qh[32 * o + l]
                lo_a, hi_a = (a >> 4, a & 15) if swap_nibbles else (a & 15, a >> 4)
                lo_b, hi_b = (b >> 4, b & 15) if swap_nibbles else (b & 15, b >> 4)
                f = [(hb >> s) & 3 for s in (0, 2, 4, 6)]
                if swap_qh:
                    f[1], f[2] = f[2], f[1]
                q = [lo_a | f[0] << 4, lo_b | f[1] << 4, hi_a | f[2] << 4, hi_b | f[3] << 4]
                for j in range(4):
                    out[128 * h + l + 32 * j] = float(sc[8 * h + l // 16 + 2 * j]) * (q[j] - 32)
        return out

    assert np.array_equal(decode(Q6K_FIELDS_BLOCK), Q6K_FIELDS_OUT)
    for slip in ({"swap_qh": True}, {"swap_nibbles": True}, {"same_half": True}):
        assert not np.array_equal(decode(Q6K_FIELDS_BLOCK, **slip), Q6K_FIELDS_OUT), slip


def test_q8_0_signed_codes_hand_derived():
    # d = 0.5; codes 0x80, 0xFF, 0x81, 0x7F are -128, -1, -127, 127 as i8
    # (dequant.rs:40-47): -64, -0.5, -63.5, 63.5.  Unsigned codes would give
    # 64, 127.5, 64.5, 63.5.
    block = F16_HALF + bytes([0x80, 0xFF, 0x81, 0x7F] * 8)
    out = oracle.dequant_block("q8_0", block)
    assert np.array_equal(out, np.array([-64.0, -0.5, -63.5, 63.5] * 8, np.float32))


# ------------------------------------- independent restatements ----------

@pytest.mark.parametrize("qtype", [8, 2, 6, 12, 13, 14])
def test_blocks_match_numpy_restatement(qtype):
    elems, bb = synth.GEOMETRY[qtype]
    nb = 3000
    data = synth.weight_blocks(qtype, 1234 + qtype, nb * elems, 1)
    rc, got = oracle.dequant_tensor(qtype, data, nb * elems)
    assert rc == oracle.OK
    want = ref.DECODERS[qtype](data)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", [8, 2, 6, 12, 13, 14])
def test_raw_random_blocks_match_numpy_restatement(qtype):
    # Every byte random: f16 scales hit subnormals, infinities and NaNs.
    elems, bb = synth.GEOMETRY[qtype]
    nb = 4000
    data = synth.random_bytes(99 + qtype, nb * bb)
    rc, got = oracle.dequant_tensor(qtype, data, nb * elems)
    assert rc == oracle.OK
    with np.errstate(all="ignore"):
        want = ref.DECODERS[qtype](data)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_multithreaded_decode_matches_single():
    data = synth.q4_k_blocks(5, 2048)
    rc1, a = oracle.dequant_tensor(12, data, 2048 * 256)
    rc2, b = oracle.dequant_tensor(12, data, 2048 * 256, threads=4)
    assert rc1 == rc2 == 0 and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------- dequant_tensor error rules ---

def test_dequant_tensor_errors():  # dequant.rs:84-95, 143
    data = np.zeros(1000, dtype=np.uint8)
    assert oracle.dequant_tensor(3, data, 32)[0] == oracle.E_UNSUPPORTED    # Q4_1
    assert oracle.dequant_tensor(10, data, 256)[0] == oracle.E_UNSUPPORTED  # Q2K: no decoder
    assert oracle.dequant_tensor(11, data, 256)[0] == oracle.E_UNSUPPORTED  # Q3K
    assert oracle.dequant_tensor(77, data, 256)[0] == oracle.E_UNSUPPORTED
    assert oracle.dequant_tensor(12, data, 100)[0] == oracle.E_OVERFLOW
    assert oracle.dequant_tensor(12, data[:143], 256)[0] == oracle.E_TRUNCATED
    assert oracle.dequant_tensor(12, data[:144], 256)[0] == oracle.OK
    assert oracle.dequant_tensor(14, data[:419], 512)[0] == oracle.E_TRUNCATED


def test_dense_passthrough_types():  # dequant.rs:98-117
    v = np.array([1.5, -2.25, 3e-8, np.inf], dtype=np.float32)
    rc, out = oracle.dequant_tensor(0, v.view(np.uint8), 4)
    assert rc == 0 and np.array_equal(out.view(np.uint32), v.view(np.uint32))
    h = np.array([1.0, -0.5, 65504.0, 6e-8], dtype=np.float16)
    rc, out = oracle.dequant_tensor(1, h.view(np.uint8), 4)
    assert rc == 0 and np.array_equal(out, h.astype(np.float32))
    bf = torch.tensor([1.0, -3.5, 1e30, 2.0 ** -100], dtype=torch.bfloat16)
    rc, out = oracle.dequant_tensor(30, bf.view(torch.int16).numpy().view(np.uint8), 4)
    assert rc == 0 and np.array_equal(out, bf.float().numpy())


# ------------------------------------------------------------------ FP8 ---

def test_e4m3_decode_kats():  # fp8_weight.rs:120, safetensors_load.rs:41-66
    assert oracle.fp8_decode(0x38) == 1.0
    assert oracle.fp8_decode(0x40) == 2.0
    assert oracle.fp8_decode(0x30) == 0.5
    assert oracle.fp8_decode(0x44) == 3.0


def test_e4m3_decode_exhaustive():
    got = np.array([oracle.fp8_decode(b) for b in range(256)], dtype=np.float32)
    via_torch = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    table = ref.e4m3_table()
    for want in (via_torch, table):
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan], want[~nan])
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF]) and got[0x7E] == 448.0


def _encoder_probe_values():
    t = ref.e4m3_table()[:127].astype(np.float64)
    mids = (t[:-1] + t[1:]) / 2.0
    vals = np.concatenate([t, mids, np.nextafter(mids.astype(np.float32), 0),
                           np.nextafter(mids.astype(np.float32), 1000),
                           synth.normal(3, 20000) * 40.0, synth.normal(4, 2000) * 1e-3,
                           [0.0, 447.9, 448.0, 448.5, 464.0, 480.0, 1e9, np.inf, 1e-45]])
    vals = vals.astype(np.float32)
    return np.concatenate([vals, -vals, [np.float32(-0.0), np.float32(np.nan)]]).astype(np.float32)


def test_e4m3_reference_encoder_is_nearest_tie_low():  # load_safetensors.rs:53-69
    x = _encoder_probe_values()
    got = oracle.fp8_encode_array(x)
    want = ref.e4m3_nearest_tie_low(x)
    assert np.array_equal(got, want)
    assert oracle.fp8_encode(-0.0) == 0x80 and oracle.fp8_encode(float("nan")) == 0x7F


def test_e4m3_rne_encoder_matches_torch():
    x = _encoder_probe_values()
    x = x[~np.isnan(x)]
    got = np.array([oracle.fp8_encode_rne(float(v)) for v in x], dtype=np.uint8)
    want = torch.from_numpy(np.clip(x, -448.0, 448.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_cpu_fp8_gemm_matches_reference():  # fp8_gemm.rs:198-208
    x = np.array([[1.0, 2.0], [3.0, 4.0]], dtype=np.float32)
    w = np.array([[0x38, 0x00], [0x00, 0x40]], dtype=np.uint8)  # [[1, 0], [0, 2]]
    s = np.array([2.0, 0.5], dtype=np.float32)
    y = oracle.fp8_gemm_fallback(x, w, s)
    assert y.shape == (2, 2)
    assert y.reshape(-1).tolist() == [2.0, 2.0, 6.0, 4.0]


def test_fp8_weight_forward_matches_dequant():  # fp8_weight.rs:117-133
    w = np.array([[0x38, 0x40], [0x30, 0x44]], dtype=np.uint8)
    s = np.array([2.0, 0.5], dtype=np.float32)
    x = np.array([[1.5, -2.0]], dtype=np.float32)
    out = oracle.fp8_gemm_fallback(x, w, s)
    deq = np.array([[1.0, 2.0], [0.5, 3.0]], dtype=np.float32) * s[:, None]
    assert np.allclose(out, x @ deq.T, atol=1e-3)
    assert out.reshape(-1).tolist() == [-5.0, -2.625]


def test_per_token_quantize_closed_form():
    x = synth.activations(7, 16, 512)
    x[3] = 0.0
    xq, xs = oracle.fp8_quantize_rows(x)
    amax = np.abs(x).max(axis=1)
    assert xs[3] == 0.0 and not xq[3].any()
    live = amax > 0
    assert np.array_equal(xs[live], (amax[live] / np.float32(448.0)).astype(np.float32))
    dec = torch.from_numpy(xq).view(torch.float8_e4m3fn).float().numpy()
    # the largest element maps to +-448 exactly; every code is within half a
    # step (relative 2^-4) of x / s
    assert np.all(np.abs(dec[live]).max(axis=1) == 448.0)
    inv = (np.float32(448.0) / amax[live]).astype(np.float32)
    scaled = (x[live] * inv[:, None]).astype(np.float32)
    want = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(xq[live], want)


def test_quantized_gemm_f64_closed_form():
    xq = synth.random_bytes(8, 4 * 64).reshape(4, 64) & 0x77  # finite codes
    w = synth.random_bytes(9, 6 * 64).reshape(6, 64) & 0xF7
    xs = np.array([1.0, 0.5, 2.0, 0.25], dtype=np.float32)
    ws = np.linspace(0.5, 2.0, 6).astype(np.float32)
    y = oracle.fp8_gemm_quantized_f64(xq, xs, w, ws)
    t = ref.e4m3_table().astype(np.float64)
    want = (t[xq] @ t[w].T) * xs[:, None] * ws[None, :]
    assert np.allclose(y, want, rtol=1e-15, atol=0)


# ------------------------------------------------------------ linear ------

def test_linear_dense_kats():  # linear_layer.rs:129-160
    w = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    y = oracle.linear_f64(np.ones((1, 3), np.float32), w)
    assert y.shape == (1, 2) and y.reshape(-1).tolist() == [6.0, 15.0]
    w2 = np.array([[1, 2, 3, 4], [2, 3, 4, 5]], dtype=np.float32)
    assert oracle.linear_f64(np.ones((1, 4), np.float32), w2).reshape(-1).tolist() == [10.0, 14.0]


def test_linear_matches_numpy():
    x = synth.activations(1, 5, 300)
    w = synth.activations(2, 7, 300)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(oracle.linear_f64(x, w), want, rtol=1e-12, atol=1e-12)
    y32 = oracle.linear_f32(x, w, threads=2)
    assert np.max(np.abs(y32 - want)) / np.max(np.abs(want)) < 1e-5
