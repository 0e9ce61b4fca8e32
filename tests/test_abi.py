"""The C-ABI library loads and exports every symbol include/rq.h declares, and
its argument checks answer before any device work (CPU-only: no kernel runs)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from runtimed_amd import rq

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "rq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("rq_weight_create", "rq_weight_destroy", "rq_dequant_f32", "rq_dequant_tensor",
              "rq_linear", "rq_fp8_gemm", "rq_fp8_quantize", "rq_last_error", "rq_embedding",
              "rq_marlin_repack", "rq_marlin_dequant", "rq_marlin_linear", "rq_kv_quantize",
              "rq_kv_dequantize", "rq_linear_bias", "rq_linear_multi", "rq_bias_add"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(rq.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (rq_[a-z0-9_]+)$", out, flags=re.M))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    L = rq.lib()
    for s in declared_symbols():
        assert hasattr(L, s)


def test_abi_version():
    assert rq.lib().rq_abi_version() == 2


def _create(qtype, data, n, k):
    h = ctypes.c_void_p()
    buf = np.ascontiguousarray(data, dtype=np.uint8)
    rc = rq.lib().rq_weight_create(qtype, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, n, k, 0,
                                   ctypes.byref(h))
    return rc, rq.lib().rq_last_error().decode()


def test_create_rejects_like_dequant_tensor():  # dequant.rs:84-95
    data = np.zeros(4096, dtype=np.uint8)
    rc, msg = _create(3, data, 1, 32)            # Q4_1: no decoder
    assert rc == -1 and "not implemented" in msg
    rc, msg = _create(10, data, 1, 256)          # Q2K: geometry, no decoder
    assert rc == -1
    rc, msg = _create(12, data, 1, 100)          # 100 % 256 != 0
    assert rc == -2 and "not a multiple" in msg
    rc, msg = _create(12, data[:143], 1, 256)    # one block needs 144 bytes
    assert rc == -3 and "truncated" in msg
    rc, msg = _create(12, data, 0, 256)
    assert rc == -4


def test_null_and_enum_checks():
    L = rq.lib()
    assert L.rq_weight_create(12, None, 0, 1, 256, 0, None) == -5
    assert L.rq_weight_info(None, None) == -5
    assert L.rq_dequant_f32(None, None, None) == -5
    assert L.rq_embedding(None, None, 1, None, None) == -5
    assert L.rq_linear(None, None, 0, 1, 256, None, 0, None) == -5
    assert L.rq_linear_bias(None, None, 0, 1, 256, None, 0, None, 0, None) == -5
    # rq_linear_multi: nothing to do, a negative count, null arrays
    assert L.rq_linear_multi(0, None, None, 0, 1, 256, None, 0, None, 0, None) == 0
    assert L.rq_linear_multi(-1, None, None, 0, 1, 256, None, 0, None, 0, None) == -5
    assert L.rq_linear_multi(2, None, None, 0, 1, 256, None, 0, None, 0, None) == -5
    # rq_bias_add: enum, shape and null checks before any device work
    assert L.rq_bias_add(None, 99, 1, 4, None, 0, None) == -5
    assert L.rq_bias_add(None, 0, 1, 4, None, 77, None) == -5
    assert L.rq_bias_add(None, 0, -1, 4, None, 0, None) == -4
    assert L.rq_bias_add(None, 0, 0, 4, None, 0, None) == 0
    assert L.rq_bias_add(None, 0, 2, 4, None, 0, None) == -5
    assert L.rq_fp8_quantize(None, 0, 1, 16, 7, None, None, None) == -5  # bad mode
    assert L.rq_fp8_gemm(None, 99, 1, None, None, 16, 16, None, 0, 1, None) == -5
    assert L.rq_dequant_tensor(3, None, 0, 32, None, None) == -1
    assert L.rq_dequant_tensor(12, None, 0, 100, None, None) == -2
    assert L.rq_dequant_tensor(12, None, 10, 256, None, None) == -3
    assert L.rq_dequant_tensor(12, None, 0, 0, None, None) == 0  # empty stream is a no-op
    # Marlin INT4 and the KV quantizer: enum, shape and null checks
    assert L.rq_marlin_repack(None, 99, None, 4, 32, None, None) == -5
    assert L.rq_marlin_repack(None, 0, None, 4, 0, None, None) == -4
    assert L.rq_marlin_repack(None, 0, None, 0, 32, None, None) == 0      # no rows: no-op
    assert L.rq_marlin_dequant(None, None, 4, 32, None, None) == -5
    assert L.rq_marlin_linear(None, None, 4, 32, None, 0, 0, None, 0, None) == 0  # m = 0
    assert L.rq_marlin_linear(None, None, 4, 32, None, 0, 1, None, 0, None) == -5
    assert L.rq_marlin_linear(None, None, 4, 32, None, 0, -1, None, 0, None) == -4
    assert L.rq_kv_quantize(None, 0, 1, 2, 16, 9, None, None, None) == -5   # bad mode
    assert L.rq_kv_quantize(None, 0, -1, 2, 16, 1, None, None, None) == -4
    assert L.rq_kv_quantize(None, 0, 1, 2, 16, 1, None, None, None) == -5  # null scales
    assert L.rq_kv_dequantize(None, 1, None, 1, 2, 0, None, 0, None) == 0  # empty
    assert L.rq_kv_dequantize(None, 2, None, 1, 2, 16, None, 0, None) == -5
    L.rq_weight_destroy(None)


def test_error_message_is_thread_local():
    import threading

    rq.lib().rq_dequant_tensor(12, None, 0, 100, None, None)
    main_msg = rq.lib().rq_last_error().decode()
    seen = []
    t = threading.Thread(target=lambda: seen.append(rq.lib().rq_last_error().decode()))
    t.start()
    t.join()
    assert "not a multiple" in main_msg and seen == [""]
