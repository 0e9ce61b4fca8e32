"""Device dequant-to-f32 is bit-identical to the oracle's dequant_tensor
(dequant.rs:83-146), through the weight handle (split layouts) and through
the flat-stream entry point (raw GGUF bytes at any alignment)."""
import numpy as np
import pytest
import torch

import oracle
from runtimed_amd import rq, synth

pytestmark = pytest.mark.gpu

ALL = [rq.Q8_0, rq.Q4_0, rq.Q5_0, rq.Q4_K, rq.Q5_K, rq.Q6_K]


def bits_equal(got: np.ndarray, want: np.ndarray):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("qtype", ALL)
@pytest.mark.parametrize("n,k", [(1, 256), (3, 512), (128, 896), (896, 896), (7, 4864)])
def test_handle_dequant_bit_exact(dev, qtype, n, k):
    print(f"dequant qtype={qtype} n={n} k={k}", flush=True)
    data = synth.weight_blocks(qtype, 1000 + n + k, n, k)
    w = rq.QWeight(qtype, data, n, k)
    got = w.dequantize().cpu().numpy().reshape(-1)
    rc, want = oracle.dequant_tensor(qtype, data, n * k)
    assert rc == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype,mbytes", [(q, 5) for q in ALL] + [(rq.Q8_0, 140), (rq.Q4_K, 140), (rq.Q6_K, 140),
                                                                   (rq.Q5_0, 70)])
def test_large_upload_bit_exact(dev, qtype, mbytes):
    # at least 4 MB of blocks take the staged upload (pinned double-buffered
    # DMA, split on the device); more than 64 MB spans several staging chunks
    elems, bb = rq.GEOMETRY[qtype]
    k = 4096
    n = (mbytes << 20) // (k // elems * bb) + 1
    print(f"upload qtype={qtype} n={n} k={k} bytes={n * k // elems * bb}", flush=True)
    data = synth.random_bytes(91 + qtype + mbytes, n * k // elems * bb)
    w = rq.QWeight(qtype, data, n, k)
    got = w.dequantize().cpu().numpy().reshape(-1)
    rc, want = oracle.dequant_tensor(qtype, data, n * k, threads=8)
    assert rc == 0
    bits_equal(got, want)
    assert w.info()["gguf_bytes"] == n * k // elems * bb


@pytest.mark.parametrize("qtype", ALL)
def test_handle_dequant_random_bytes(dev, qtype):
    # every byte random: f16 scales include subnormals, infinities and NaNs
    elems, bb = rq.GEOMETRY[qtype]
    nb = 2048
    data = synth.random_bytes(77 + qtype, nb * bb)
    w = rq.QWeight(qtype, data, nb, elems)
    got = w.dequantize().cpu().numpy().reshape(-1)
    rc, want = oracle.dequant_tensor(qtype, data, nb * elems)
    assert rc == 0
    bits_equal(got, want)


@pytest.mark.parametrize("qtype", ALL)
@pytest.mark.parametrize("offset", [0, 1, 2, 6])
def test_flat_stream_dequant(dev, qtype, offset):
    elems, bb = rq.GEOMETRY[qtype]
    nb = 515
    data = synth.random_bytes(5 + qtype, nb * bb)
    buf = torch.zeros(nb * bb + offset + 16, dtype=torch.uint8, device=dev)
    buf[offset:offset + nb * bb] = torch.from_numpy(data).to(dev)
    got = rq.dequant_tensor(qtype, buf[offset:offset + nb * bb], nb * elems).cpu().numpy()
    rc, want = oracle.dequant_tensor(qtype, data, nb * elems)
    bits_equal(got, want)


def test_flat_stream_errors(dev):
    buf = torch.zeros(1000, dtype=torch.uint8, device=dev)
    with pytest.raises(rq.RqError) as e:
        rq.dequant_tensor(rq.Q4_K, buf, 100)
    assert e.value.kind == "Overflow"
    with pytest.raises(rq.RqError) as e:
        rq.dequant_tensor(rq.Q6_K, buf[:419], 512)
    assert e.value.kind == "Truncated"
    with pytest.raises(rq.RqError) as e:
        rq.dequant_tensor(10, buf, 256)
    assert e.value.kind == "Unsupported"


def test_reference_kats_on_device(dev):
    # dequant.rs:162-169 and dequant_k.rs:118-177 through the device decoder
    q8 = np.frombuffer(bytes([0x00, 0x3C]) + bytes(range(32)), dtype=np.uint8)
    assert np.array_equal(rq.QWeight(rq.Q8_0, q8, 1, 32).dequantize().cpu().numpy()[0],
                          np.arange(32, dtype=np.float32))
    q4 = np.frombuffer(bytes([0, 0x3C, 0, 0]) + bytes([65] + [1] * 11) + bytes([0x11] * 128), dtype=np.uint8)
    out = rq.QWeight(rq.Q4_K, q4, 1, 256).dequantize().cpu().numpy()[0]
    assert np.all(out[:64] == 1.0) and np.all(out[128:160] == 17.0)
    q6 = bytearray(208) + bytearray([0x00, 0x3C])
    q6[192:200] = bytes([1, 2, 3, 4, 5, 6, 7, 8])
    q6[200:208] = bytes([1] * 8)
    q6[0] = 0x11
    q6[128] = 0xFF
    q6[16] = 0x11
    out = rq.QWeight(rq.Q6_K, np.frombuffer(bytes(q6), np.uint8), 1, 256).dequantize().cpu().numpy()[0]
    assert (out[0], out[32], out[64], out[96], out[16]) == (17.0, 48.0, 85.0, 112.0, -62.0)


def test_hand_derived_kats_on_device(dev):
    # the literal Q6_K bit-field and Q8_0 sign vectors, worked out by hand from
    # dequant_k.rs:87-111 and dequant.rs:40-47, through the device layouts
    # (208-byte Q6_K records + d array, Q8_0 codes + scale array); two rows
    # of each so the second row's scale lookup is covered too
    from tests.test_oracle import F16_HALF, Q6K_FIELDS_BLOCK, Q6K_FIELDS_OUT

    q6 = np.frombuffer(Q6K_FIELDS_BLOCK + Q6K_FIELDS_BLOCK[:208] + F16_HALF, np.uint8)
    out = rq.QWeight(rq.Q6_K, q6, 2, 256).dequantize().cpu().numpy()
    assert np.array_equal(out[0], Q6K_FIELDS_OUT) and np.array_equal(out[1], Q6K_FIELDS_OUT * 0.5)
    q8 = np.frombuffer((F16_HALF + bytes([0x80, 0xFF, 0x81, 0x7F] * 8)) * 2, np.uint8)
    out = rq.QWeight(rq.Q8_0, q8, 2, 32).dequantize().cpu().numpy()
    assert np.array_equal(out, np.tile(np.array([-64.0, -0.5, -63.5, 63.5] * 8, np.float32), (2, 1)))


def test_weight_info(dev):
    data = synth.q4_k_blocks(1, 4864 * 896 // 256)
    w = rq.QWeight(rq.Q4_K, data, 4864, 896)
    info = w.info()
    assert info["gguf_bytes"] == 2451456 and info["n"] == 4864 and info["k"] == 896
    q6 = rq.QWeight(rq.Q6_K, synth.q6_k_blocks(1, 64), 64, 256)
    assert q6.info()["gguf_bytes"] == 64 * 210


def test_golden_fixtures_on_device(dev):
    from tests.golden import load_golden

    for case in load_golden()["dequant"]:
        w = rq.QWeight(case["qtype"], case["blocks"], case["n"], case["k"])
        got = w.dequantize().cpu().numpy().reshape(-1)
        assert np.array_equal(got.view(np.uint32), case["out"].view(np.uint32)), case["name"]
