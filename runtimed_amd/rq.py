"""ctypes binding of librq (include/rq.h) with torch tensors for device memory.

torch is only plumbing here: it allocates device buffers and supplies the
current HIP stream; every kernel that runs is librq's.  The library must be
built (``python -m runtimed_amd.build``); a missing library raises, there is no
fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "librq.so"

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 6, 8, 12, 13, 14
QTYPES = {"Q4_0": Q4_0, "Q5_0": Q5_0, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
# (elements, bytes) per block, dtype.rs:49-64
GEOMETRY = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
            Q6_K: (256, 210)}

F32, F16, BF16, F8E4M3 = 0, 1, 30, 128
FP8_UNSCALED, FP8_PER_TOKEN = 0, 1
# rq_kv_mode: CachePrecision (cache/paged/block.rs:23-27)
KV_F16, KV_FP8, KV_INT8 = 0, 1, 2
SINK_TOKENS_COUNT = 16  # quantize.rs:9
_FTYPE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float8_e4m3fn: F8E4M3,
          torch.uint8: F8E4M3}

STATUS = {0: "OK", -1: "Unsupported", -2: "Overflow", -3: "Truncated", -4: "Shape", -5: "Arg",
          -6: "Device", -7: "NoMem"}


class RqError(RuntimeError):
    """A negative rq_status with the library's thread-local message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code
        self.kind = STATUS.get(code, str(code))
        self.message = message


class _Desc(ctypes.Structure):
    _fields_ = [("qtype", ctypes.c_int32), ("device", ctypes.c_int32), ("n", ctypes.c_int64),
                ("k", ctypes.c_int64), ("gguf_bytes", ctypes.c_uint64),
                ("device_bytes", ctypes.c_uint64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m runtimed_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, sz, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
        L.rq_abi_version.restype = i32
        L.rq_last_error.restype = ctypes.c_char_p
        L.rq_weight_create.argtypes = [i32, vp, sz, i64, i64, i32, ctypes.POINTER(vp)]
        L.rq_weight_destroy.argtypes = [vp]
        L.rq_weight_destroy.restype = None
        L.rq_weight_info.argtypes = [vp, ctypes.POINTER(_Desc)]
        L.rq_dequant_f32.argtypes = [vp, vp, vp]
        L.rq_dequant_tensor.argtypes = [i32, vp, sz, sz, vp, vp]
        L.rq_embedding.argtypes = [vp, vp, i64, vp, vp]
        L.rq_linear.argtypes = [vp, vp, i32, i64, i64, vp, i32, vp]
        L.rq_linear_bias.argtypes = [vp, vp, i32, i64, i64, vp, i32, vp, i32, vp]
        L.rq_linear_multi.argtypes = [i32, vp, vp, i32, i64, i64, vp, i32, vp, i32, vp]
        L.rq_bias_add.argtypes = [vp, i32, i64, i64, vp, i32, vp]
        L.rq_fp8_quantize.argtypes = [vp, i32, i64, i64, i32, vp, vp, vp]
        L.rq_fp8_gemm.argtypes = [vp, i32, i64, vp, vp, i64, i64, vp, i32, i32, vp]
        L.rq_fp8_gemm_q.argtypes = [vp, vp, i64, vp, vp, i64, i64, vp, i32, vp]
        L.rq_fp8_gemm_noalloc.argtypes = [vp, i32, i64, vp, vp, i64, i64, vp, i32, i32, vp]
        L.rq_marlin_repack.argtypes = [vp, i32, vp, i64, i64, vp, vp]
        L.rq_marlin_dequant.argtypes = [vp, vp, i64, i64, vp, vp]
        L.rq_marlin_linear.argtypes = [vp, vp, i64, i64, vp, i32, i64, vp, i32, vp]
        L.rq_kv_quantize.argtypes = [vp, i32, i64, i64, i64, i32, vp, vp, vp]
        L.rq_kv_dequantize.argtypes = [vp, i32, vp, i64, i64, i64, vp, i32, vp]
        for f in ("rq_weight_create", "rq_weight_info", "rq_dequant_f32", "rq_dequant_tensor",
                  "rq_linear", "rq_linear_bias", "rq_linear_multi", "rq_bias_add", "rq_fp8_quantize",
                  "rq_fp8_gemm", "rq_fp8_gemm_q", "rq_fp8_gemm_noalloc"):
            getattr(L, f).restype = i32
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RqError(rc, lib().rq_last_error().decode())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def ftype(dtype: torch.dtype) -> int:
    if dtype not in _FTYPE:
        raise TypeError(f"unsupported dtype {dtype}")
    return _FTYPE[dtype]


class QWeight:
    """A device-resident GGUF weight: the value a runtimed `q_map` entry holds.

    `blocks` is the GGUF block stream of an [n, k] tensor (GGUF dims [k, n]).
    """

    def __init__(self, qtype: int, blocks, n: int, k: int, device: int = 0):
        buf = np.ascontiguousarray(np.frombuffer(blocks, dtype=np.uint8)
                                   if not isinstance(blocks, np.ndarray) else blocks.view(np.uint8))
        h = ctypes.c_void_p()
        check(lib().rq_weight_create(qtype, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, n, k,
                                     device, ctypes.byref(h)))
        self._h = h
        self.qtype, self.n, self.k, self.device = qtype, n, k, torch.device("cuda", device)

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().rq_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def info(self) -> dict:
        d = _Desc()
        check(lib().rq_weight_info(self._h, ctypes.byref(d)))
        return {f: getattr(d, f) for f, _ in _Desc._fields_}

    def dequantize(self) -> torch.Tensor:
        out = torch.empty((self.n, self.k), dtype=torch.float32, device=self.device)
        check(lib().rq_dequant_f32(self._h, _ptr(out), _stream(self.device)))
        return out

    def embedding(self, ids) -> torch.Tensor:
        """Rows `ids` decoded exactly, f32 [len(ids), k] (embed_layer.rs:16-84)."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        out = torch.empty((ids.size, self.k), dtype=torch.float32, device=self.device)
        check(lib().rq_embedding(self._h, ids.ctypes.data_as(ctypes.c_void_p), ids.size, _ptr(out),
                                 _stream(self.device)))
        return out

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                out: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """y = x W^T (+ bias) over the last dimension of x (linear_layer.rs:45-52,
        107-118).  A last dimension other than k raises Shape from the library
        (linear_layer.rs:88-96)."""
        k = x.shape[-1] if x.dim() else 0
        if not x.is_contiguous():
            x = x.contiguous()
        rows = x.numel() // k if k else 0
        if out is None:
            out = torch.empty((*x.shape[:-1], self.n), dtype=out_dtype or x.dtype, device=x.device)
        if bias is None:
            check(lib().rq_linear(self._h, _ptr(x), ftype(x.dtype), rows, k, _ptr(out), ftype(out.dtype),
                                  _stream(x.device)))
        else:
            check(lib().rq_linear_bias(self._h, _ptr(x), ftype(x.dtype), rows, k, _ptr(bias), ftype(bias.dtype),
                                       _ptr(out), ftype(out.dtype), _stream(x.device)))
        return out


def linear_multi(weights, x: torch.Tensor, biases=None, out_dtype: Optional[torch.dtype] = None):
    """Several linears on one input (q/k/v, gate/up: qwen2.rs:99-125) through
    rq_linear_multi; returns the outputs in order."""
    x = x.contiguous()
    outs = [torch.empty((*x.shape[:-1], w.n), dtype=out_dtype or x.dtype, device=x.device) for w in weights]
    if outs:
        linear_multi_into(weights, x, outs, biases)
    return outs


def linear_multi_into(weights, x: torch.Tensor, outs, biases=None) -> None:
    """linear_multi into preallocated outputs (x contiguous; outputs of one dtype)."""
    k = x.shape[-1]
    rows = x.numel() // k if k else 0
    count = len(weights)
    hs = (ctypes.c_void_p * count)(*[w.handle.value for w in weights])
    ys = (ctypes.c_void_p * count)(*[o.data_ptr() for o in outs])
    btype = F32
    bs = None
    if biases is not None:
        present = [b for b in biases if b is not None]
        btype = ftype(present[0].dtype) if present else F32
        bs = (ctypes.c_void_p * count)(*[(b.data_ptr() if b is not None else 0) for b in biases])
    check(lib().rq_linear_multi(count, hs, _ptr(x), ftype(x.dtype), rows, k, bs, btype, ys, ftype(outs[0].dtype),
                                _stream(x.device)))


def bias_add(y: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """y += bias over the last dimension, in y's dtype (linear_layer.rs:111-115)."""
    n = y.shape[-1]
    check(lib().rq_bias_add(_ptr(y), ftype(y.dtype), y.numel() // n if n else 0, n, _ptr(bias.contiguous()),
                            ftype(bias.dtype), _stream(y.device)))
    return y


def dequant_tensor(qtype: int, dev_bytes: torch.Tensor, n_elements: int) -> torch.Tensor:
    """dequant_tensor (dequant.rs:83-146) on GGUF bytes in device memory."""
    out = torch.empty(n_elements, dtype=torch.float32, device=dev_bytes.device)
    check(lib().rq_dequant_tensor(qtype, _ptr(dev_bytes), dev_bytes.numel(), n_elements, _ptr(out),
                                  _stream(dev_bytes.device)))
    return out


def fp8_quantize(x: torch.Tensor, mode: int = FP8_PER_TOKEN):
    k = x.shape[-1]
    m = x.numel() // k
    xq = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    xs = torch.empty(m, dtype=torch.float32, device=x.device)
    check(lib().rq_fp8_quantize(_ptr(x.contiguous()), ftype(x.dtype), m, k, mode, _ptr(xq), _ptr(xs),
                                _stream(x.device)))
    return xq, xs


def fp8_gemm(x: torch.Tensor, w: torch.Tensor, w_scale: Optional[torch.Tensor],
             mode: int = FP8_PER_TOKEN, out_dtype: torch.dtype = torch.bfloat16,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x (w * w_scale)^T with e4m3 w codes [n, k] (fp8_gemm.rs:77-191)."""
    n, k = w.shape
    if x.shape[-1] != k:
        raise RqError(-4, f"expected last dim {k}, got {list(x.shape)}")
    x = x.contiguous()
    m = x.numel() // k
    if out is None:
        out = torch.empty((*x.shape[:-1], n), dtype=out_dtype, device=x.device)
    check(lib().rq_fp8_gemm(_ptr(x), ftype(x.dtype), m, _ptr(w), _ptr(w_scale), n, k, _ptr(out),
                            ftype(out.dtype), mode, _stream(x.device)))
    return out


def fp8_gemm_q(xq: torch.Tensor, xs: Optional[torch.Tensor], w: torch.Tensor,
               w_scale: Optional[torch.Tensor], out: torch.Tensor) -> torch.Tensor:
    n, k = w.shape
    m = xq.numel() // k
    check(lib().rq_fp8_gemm_q(_ptr(xq), _ptr(xs), m, _ptr(w), _ptr(w_scale), n, k, _ptr(out),
                              ftype(out.dtype), _stream(xq.device)))
    return out


# ---- Marlin INT4 weights (crates/runtimed-model/src/ops/marlin_gemv.rs) ----

class MarlinWeight:
    """Packed INT4 weights (marlin_gemv.rs:11-63): `packed` holds the u32 words
    [ceil(in_dim/32), out_dim, 4] (as torch.int32 bits), `scales` f32 [out_dim]."""

    def __init__(self, packed: torch.Tensor, scales: torch.Tensor, in_dim: int, out_dim: int):
        if packed.dtype not in (torch.int32, torch.uint32):
            raise RqError(-5, f"marlin packed must be U32, got {packed.dtype}")
        if tuple(scales.shape) not in ((out_dim,), (out_dim, 1)):
            raise RqError(-4, f"marlin_scales: expected [{out_dim}], got {list(scales.shape)}")
        if packed.device != scales.device:
            raise RqError(-5, "packed and scales must be on the same device")
        k_chunks = (in_dim + 31) // 32
        if packed.numel() < k_chunks * out_dim * 4:
            raise RqError(-4, f"marlin_packed: expected [{k_chunks}, {out_dim}, 4], got {list(packed.shape)}")
        self.packed, self.scales, self.in_dim, self.out_dim = packed, scales, in_dim, out_dim

    @property
    def device(self) -> torch.device:
        return self.packed.device

    def resident_bytes(self) -> int:
        return self.packed.numel() * self.packed.element_size() + self.scales.numel() * self.scales.element_size()

    def _scales_f32(self) -> torch.Tensor:
        return self.scales.reshape(-1).to(torch.float32).contiguous()

    def dequantize(self) -> torch.Tensor:
        """f32 [out_dim, in_dim], bit-exact (marlin_gemv.rs:42-61)."""
        out = torch.empty((self.out_dim, self.in_dim), dtype=torch.float32, device=self.device)
        check(lib().rq_marlin_dequant(_ptr(self.packed.contiguous()), _ptr(self._scales_f32()), self.out_dim,
                                      self.in_dim, _ptr(out), _stream(self.device)))
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return marlin_gemv(x, self)


def repack_marlin_tiles(weight: torch.Tensor, scales: torch.Tensor) -> MarlinWeight:
    """repack_marlin_tiles (marlin_gemv.rs:66-97), run on the device."""
    if weight.dim() != 2:
        raise RqError(-5, f"weight must be 2D, got {list(weight.shape)}")
    out_dim, in_dim = weight.shape
    s32 = scales.reshape(-1).to(torch.float32).contiguous()
    if s32.numel() != out_dim:
        raise RqError(-4, f"scales: expected [{out_dim}], got [{s32.numel()}]")
    w = weight.contiguous()
    packed = torch.empty(((in_dim + 31) // 32, out_dim, 4), dtype=torch.int32, device=w.device)
    if weight.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        w = w.to(torch.float32)
    check(lib().rq_marlin_repack(_ptr(w), ftype(w.dtype), _ptr(s32), out_dim, in_dim, _ptr(packed),
                                 _stream(w.device)))
    return MarlinWeight(packed, scales, in_dim, out_dim)


def marlin_gemv(x: torch.Tensor, w: MarlinWeight) -> torch.Tensor:
    """x @ (w * scale)^T over the last dimension of x, result in x's dtype
    (marlin_gemv.rs:119-202)."""
    in_dim = x.shape[-1] if x.dim() else 0
    if in_dim != w.in_dim:
        raise RqError(-4, f"marlin_gemv: expected [{w.in_dim}], got {list(x.shape)}")
    rows = x.numel() // in_dim if in_dim else 0
    out = torch.empty((*x.shape[:-1], w.out_dim), dtype=x.dtype, device=x.device)
    if rows == 0 or w.out_dim == 0:
        return out.zero_()
    xc = x.contiguous()
    if xc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        xc = xc.to(torch.float32)
        out = out.to(torch.float32)
    check(lib().rq_marlin_linear(_ptr(w.packed.contiguous()), _ptr(w._scales_f32()), w.out_dim, w.in_dim,
                                 _ptr(xc), ftype(xc.dtype), rows, _ptr(out), ftype(out.dtype), _stream(x.device)))
    return out.to(x.dtype)


# ---- paged-KV block quantizer (crates/runtimed-model/src/cache/paged/quantize.rs) ----

def _kv_dims(t: torch.Tensor):
    if t.dim() == 4:
        return t.shape[0], t.shape[1], t.shape[2] * t.shape[3]
    return 1, 1, t.numel()


def _kv_input(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.dtype in (torch.float32, torch.float16, torch.bfloat16) else t.to(torch.float32)


def _kv_quantize(t: torch.Tensor, mode: int):
    b, h, sd = _kv_dims(t)
    src = _kv_input(t)
    qdt = {KV_FP8: torch.float8_e4m3fn, KV_INT8: torch.uint8, KV_F16: torch.float16}[mode]
    q = torch.empty(t.shape, dtype=qdt, device=t.device)
    s = torch.empty(h, dtype=torch.float32, device=t.device)
    check(lib().rq_kv_quantize(_ptr(src), ftype(src.dtype), b, h, sd, mode, _ptr(q), _ptr(s),
                               _stream(t.device)))
    return q, s.reshape(1, h, 1, 1)


def quantize_fp8(t: torch.Tensor):
    """quantize_fp8 (quantize.rs:12-46): (e4m3 codes of t's shape, scales [1, h, 1, 1])."""
    return _kv_quantize(t, KV_FP8)


def quantize_int8(t: torch.Tensor):
    """quantize_int8 (quantize.rs:62-96): (int8 codes as uint8 of t's shape, scales [1, h, 1, 1])."""
    return _kv_quantize(t, KV_INT8)


def _kv_dequantize(q: torch.Tensor, scale: Optional[torch.Tensor], mode: int, target_dtype: torch.dtype):
    b, h, sd = _kv_dims(q)
    out = torch.empty(q.shape, dtype=target_dtype, device=q.device)
    s = scale.reshape(-1).to(torch.float32).contiguous() if scale is not None else None
    if s is not None and s.numel() != h:
        raise RqError(-4, f"scale: expected {h} entries, got {s.numel()}")
    check(lib().rq_kv_dequantize(_ptr(q.contiguous()), mode, _ptr(s), b, h, sd, _ptr(out), ftype(target_dtype),
                                 _stream(q.device)))
    return out


def dequantize_fp8(t: torch.Tensor, scale: torch.Tensor, target_dtype: torch.dtype) -> torch.Tensor:
    """dequantize_fp8 (quantize.rs:48-57)."""
    return _kv_dequantize(t, scale, KV_FP8, target_dtype)


def dequantize_int8(t: torch.Tensor, scale: torch.Tensor, target_dtype: torch.dtype) -> torch.Tensor:
    """dequantize_int8 (quantize.rs:98-107)."""
    return _kv_dequantize(t, scale, KV_INT8, target_dtype)


def quantize_block_kv(token_offset: int, k: torch.Tensor, v: torch.Tensor, requested_precision: int):
    """quantize_block_kv (quantize.rs:109-135): the first SINK_TOKENS_COUNT
    tokens, and Fp16 caches, stay f16 with scale 1."""
    if token_offset < SINK_TOKENS_COUNT or requested_precision == KV_F16:
        kf, _ = _kv_quantize(k, KV_F16)
        vf, _ = _kv_quantize(v, KV_F16)
        one_k = torch.ones(1, dtype=torch.float32, device=k.device)
        one_v = torch.ones(1, dtype=torch.float32, device=v.device)
        return kf, vf, one_k, one_v, KV_F16
    mode = KV_INT8 if requested_precision == KV_INT8 else KV_FP8
    kq, ks = _kv_quantize(k, mode)
    vq, vs = _kv_quantize(v, mode)
    return kq, vq, ks, vs, mode


def dequantize_block(q: torch.Tensor, scale: Optional[torch.Tensor], precision: int,
                     target_dtype: torch.dtype) -> torch.Tensor:
    """QuantizedCacheBlock::dequantize_k / dequantize_v (block.rs:85-140)."""
    if precision == KV_F16:
        return _kv_dequantize(q, None, KV_F16, target_dtype)
    return _kv_dequantize(q, scale, precision, target_dtype)
