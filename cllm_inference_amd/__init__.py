"""cllm_inference_amd -- the quantized linear-layer path of cllm_inference on MI355X (gfx950).

Python mirror of the reference's Quant API (include/cllm/core/quant.hpp:90-151 in the
reference) over the C ABI of libcllm_hip.so (include/cllm_hip.h). Same names, argument
meaning and error behaviour: failures raise RuntimeError with the reference's messages.

Host-array functions take and return numpy arrays and are synchronous, like the reference.
The *_dev functions take torch tensors already on the GPU and enqueue on torch's current
stream. There is no CPU fallback: if the HIP library is not built, importing the functions
works but every call raises.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcllm_hip.so")
QUANT_LIB_PATH = os.path.join(_HERE, "libcllm_quant.so")


class GgmlType(enum.IntEnum):
    """GGUF tensor type ids (reference include/cllm/core/quant.hpp:13-27)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14


# Every symbol include/cllm_hip.h declares: (name, restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
SIGNATURES = {
    "cllm_hip_init": (_I, [_I]),
    "cllm_hip_last_error": (ctypes.c_char_p, []),
    "cllm_hip_block_size": (_I, [_U]),
    "cllm_hip_type_size": (_SZ, [_U]),
    "cllm_hip_has_vec_dot": (_I, [_U]),
    "cllm_hip_quantize_row_q8_0": (_I, [_P, _I64, _I, _P, _P, _P]),
    "cllm_hip_vec_dot_rows": (_I, [_P, _U, _I64, _I, _P, _P, _P, _P]),
    "cllm_hip_matmul_quant": (_I, [_P, _P, _U, _P, _I, _I, _P]),
    "cllm_hip_matmul_quant_batch": (_I, [_P, _P, _U, _P, _I, _I, _I, _P]),
    "cllm_hip_dequantize_block": (_I, [_P, _P, _U, _I64]),
    "cllm_hip_dequantize_block_f16": (_I, [_P, _P, _U, _I64]),
    "cllm_hip_register_weights": (_I, [_P, _SZ]),
    "cllm_hip_unregister_weights": (_I, [_P]),
    "cllm_hip_file_mapping_identity": (_I, [_P, _P]),
    "cllm_hip_allocation_count": (ctypes.c_uint64, []),
    "cllm_hip_quantize_q8_0_dev": (_I, [_P, _I64, _I, _P, _P, _P, _P]),
    "cllm_hip_gemv_q8_dev": (_I, [_P, _U, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "cllm_hip_matmul_quant_dev": (_I, [_P, _P, _U, _P, _I, _I, _I, _P, _P]),
    "cllm_hip_matmul_quant_static_dev": (_I, [_P, _P, _U, _P, _I, _I, _I, _P, _P]),
    "cllm_hip_static_scratch_bytes": (_SZ, []),
    "cllm_hip_read_stream_dev": (_I, [_P, ctypes.c_uint64, _P]),
    "cllm_hip_matmul_route": (ctypes.c_char_p, [_U, _I, _I, _I]),
    "cllm_hip_matmul_plan": (ctypes.c_char_p, [_U, _I, _I, _I]),
    "cllm_hip_tune": (_I, [ctypes.c_char_p, _P, _I]),
    "cllm_hip_rmsnorm_q8_0_dev": (_I, [_P, _P, ctypes.c_float, _I, _I, _P, _P, _P, _P, _P]),
    "cllm_hip_swiglu_q8_0_dev": (_I, [_P, _P, _I, _I, _P, _P, _P, _P, _P]),
    "cllm_hip_add_dev": (_I, [_P, _P, _I64, _P]),
    "cllm_hip_mfma_act_bytes": (_SZ, [_I, _I]),
    "cllm_hip_quantize_mfma_dev": (_I, [_P, _I, _I, _P, _P]),
    "cllm_hip_rmsnorm_mfma_dev": (_I, [_P, _P, ctypes.c_float, _I, _I, _P, _P, _P]),
    "cllm_hip_swiglu_mfma_dev": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "cllm_hip_matmul_mfma_dev": (_I, [_U, _I, _I, _P, _P, _P, _P, _I, _P, _P]),
    "cllm_hip_matmul_mfma_plan": (ctypes.c_char_p, [_U, _I, _I, _P, _I]),
    "cllm_hip_gemv_q8_residual_dev": (_I, [_P, _U, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "cllm_hip_gemv_q8_multi_dev": (_I, [_U, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P]),
    "cllm_hip_gemv_q8_swiglu_dev": (_I, [_U, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P]),
    "cllm_hip_rmsnorm_gemv_multi_dev": (_I, [_U, _I, _I, _P, _P, _P, _P, _P, _P, ctypes.c_float,
                                             _P]),
    "cllm_hip_rmsnorm_gemv_swiglu_dev": (_I, [_U, _I, _I, _P, _P, _P, _P, _P, _P, ctypes.c_float,
                                              _P, _P]),
    "cllm_hip_gguf_open": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(_P)]),
    "cllm_hip_gguf_close": (_I, [_P]),
    "cllm_hip_gguf_tensor_count": (_I, [_P]),
    "cllm_hip_gguf_find": (_I, [_P, ctypes.c_char_p]),
    "cllm_hip_gguf_tensor": (_I, [_P, _I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U),
                                  ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_uint64),
                                  ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_P),
                                  ctypes.POINTER(_P)]),
    "cllm_hip_gguf_config": (_I, [_P, _P]),
    "cllm_hip_rope_neox_dev": (_I, [_P, _I, _I, _I, _I, ctypes.c_float, _P]),
    "cllm_hip_rope_neox2_dev": (_I, [_P, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P]),
    "cllm_hip_matmul_quant_residual_dev": (_I, [_P, _P, _U, _P, _I, _I, _I, _P, _P]),
    "cllm_hip_dequantize_rows_dev": (_I, [_P, _U, _I, _P, _I, _P, _P]),
    "cllm_hip_attention_dev": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "cllm_hip_attention_rope_dev": (_I, [_P, _P, _P, _I, _I, _I, _I, ctypes.c_float, _P, _P]),
    "cllm_hip_attention_plan": (ctypes.c_char_p, [_I, _I, _I, _I, _I]),
}


class ModelConfig(ctypes.Structure):
    """cllm_hip_model_config: ModelConfig (reference gguf.hpp:13-34) plus the file layout."""
    _fields_ = [("arch", ctypes.c_char * 64)] + [
        (n, ctypes.c_uint32) for n in ("n_layers", "n_embd", "n_head", "n_head_kv", "n_ctx",
                                        "n_ff", "vocab_size", "head_dim")] + [
        ("rope_theta", ctypes.c_float), ("norm_eps", ctypes.c_float),
        ("version", ctypes.c_uint32), ("data_offset", ctypes.c_uint64),
        ("data_bytes", ctypes.c_uint64)]

_lib_handle = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads libcllm_hip.so (once) and declares every C-ABI signature."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build it with `python -m cllm_inference_amd.build`")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib_handle = lib
    return _lib_handle


def _check(rc: int) -> None:
    if rc != 0:
        msg = load_library().cllm_hip_last_error().decode()
        raise RuntimeError(msg)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def file_mapping_identity(addr: int) -> tuple:
    """What the library compares before reusing the device copy of the read-only private file
    mapping that holds host address addr (cllm_hip_file_mapping_identity): (start, end, file
    offset, inode, device, file size, mtime ns, ctime ns, file reachable by its path)."""
    info = (ctypes.c_uint64 * 9)()
    _check(load_library().cllm_hip_file_mapping_identity(ctypes.c_void_p(addr), info))
    return tuple(int(v) for v in info)


def block_size(t: int) -> int:
    return load_library().cllm_hip_block_size(int(t))


def type_size(t: int) -> int:
    return load_library().cllm_hip_type_size(int(t))


def has_vec_dot(t: int) -> bool:
    return bool(load_library().cllm_hip_has_vec_dot(int(t)))


@dataclass
class QuantizedQ8_0:
    """Q8_0 activation rows (reference quant.hpp:118-124): fp32 scales, int8 qs, int32
    per-block sums of qs."""
    scales: np.ndarray
    qs: np.ndarray
    bsums: np.ndarray
    n: int


def quantize_row_q8_0(x: np.ndarray, n: int | None = None) -> QuantizedQ8_0:
    """fp32 -> Q8_0. x is one row of n floats, or an (m, n) array quantized row by row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    n = rows.shape[1] if n is None else int(n)
    m = rows.shape[0] if x.ndim > 1 else 1
    qs = np.empty((m, n), dtype=np.int8)
    sc = np.empty((m, max(n // 32, 0)), dtype=np.float32)
    bs = np.empty((m, max(n // 32, 0)), dtype=np.int32)
    _check(load_library().cllm_hip_quantize_row_q8_0(_ptr(rows), n, m, _ptr(qs), _ptr(sc),
                                                     _ptr(bs)))
    if x.ndim == 1:
        qs, sc, bs = qs[0], sc[0], bs[0]
    return QuantizedQ8_0(scales=sc, qs=qs, bsums=bs, n=n)


def vec_dot_rows(w: np.ndarray, t: int, qx: QuantizedQ8_0, n: int, n_w_rows: int = 1) -> np.ndarray:
    """vec_dot_row over n_w_rows consecutive weight rows starting at w."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(n_w_rows, dtype=np.float32)
    _check(load_library().cllm_hip_vec_dot_rows(
        _ptr(w), int(t), int(n), int(n_w_rows), _ptr(np.ascontiguousarray(qx.qs)),
        _ptr(np.ascontiguousarray(qx.scales)), _ptr(np.ascontiguousarray(qx.bsums)), _ptr(out)))
    return out


def vec_dot_row(w_row: np.ndarray, t: int, qx: QuantizedQ8_0, n: int) -> float:
    """Reference quant.hpp:135-136."""
    return float(vec_dot_rows(w_row, t, qx, n, 1)[0])


def matmul_quant(x: np.ndarray, w: np.ndarray, t: int, bias: np.ndarray | None, in_dim: int,
                 out_dim: int) -> np.ndarray:
    """y[out_dim] = x . W^T (+ bias) -- reference quant.hpp:143-145."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.empty(out_dim, dtype=np.float32)
    _check(load_library().cllm_hip_matmul_quant(_ptr(x), _ptr(w), int(t), _ptr(b), int(in_dim),
                                                int(out_dim), _ptr(y)))
    return y


def matmul_quant_batch(x: np.ndarray, w: np.ndarray, t: int, bias: np.ndarray | None,
                       in_dim: int, out_dim: int, n_rows: int) -> np.ndarray:
    """y[n_rows, out_dim] = X . W^T (+ bias) -- reference quant.hpp:149-151."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    y = np.zeros((max(n_rows, 0), out_dim), dtype=np.float32)
    _check(load_library().cllm_hip_matmul_quant_batch(_ptr(x), _ptr(w), int(t), _ptr(b),
                                                      int(in_dim), int(out_dim), int(n_rows),
                                                      _ptr(y)))
    return y


def _src_ptr(src):
    """A host array's address, a torch tensor's device address, or an int address as it is."""
    if isinstance(src, np.ndarray):
        return _ptr(src)
    if hasattr(src, "data_ptr"):
        return ctypes.c_void_p(src.data_ptr())
    return ctypes.c_void_p(int(src))


def dequantize_block(src, t: int, n: int) -> np.ndarray:
    """The first n elements of the blocks at src as float32 -- reference quant.hpp:99. src is a
    uint8 host array, a device tensor, or a raw address (host or device)."""
    out = np.empty(max(int(n), 0), np.float32)
    _check(load_library().cllm_hip_dequantize_block(_src_ptr(src), _ptr(out), int(t), int(n)))
    return out


def dequantize_block_f16(src, t: int, n: int) -> np.ndarray:
    """The same values as binary16 bits (uint16) -- reference quant.hpp:105."""
    out = np.empty(max(int(n), 0), np.uint16)
    _check(load_library().cllm_hip_dequantize_block_f16(_src_ptr(src), _ptr(out), int(t), int(n)))
    return out


# ---- device (torch) entry points --------------------------------------------------------

def _tp(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def quantize_q8_0_dev(x, qs=None, scales=None, bsums=None):
    """x: float32 (m, k) CUDA tensor -> (qs int8 (m, k), scales f32 (m, k/32), bsums i32)."""
    import torch
    m, k = x.shape
    if qs is None:
        qs = torch.empty((m, k), dtype=torch.int8, device=x.device)
        scales = torch.empty((m, k // 32), dtype=torch.float32, device=x.device)
        bsums = torch.empty((m, k // 32), dtype=torch.int32, device=x.device)
    _check(load_library().cllm_hip_quantize_q8_0_dev(_tp(x), k, m, _tp(qs), _tp(scales),
                                                     _tp(bsums), _stream()))
    return qs, scales, bsums


def gemv_q8_dev(w, t: int, in_dim: int, out_dim: int, qs, scales, bsums, bias=None, y=None):
    """vec_dot of every weight row against already-quantized activation rows (device)."""
    import torch
    m = qs.shape[0]
    if y is None:
        y = torch.empty((m, out_dim), dtype=torch.float32, device=qs.device)
    _check(load_library().cllm_hip_gemv_q8_dev(_tp(w), int(t), int(in_dim), int(out_dim), int(m),
                                               _tp(qs), _tp(scales), _tp(bsums), _tp(bias),
                                               _tp(y), _stream()))
    return y


def gemv_q8_multi_dev(ws, t: int, in_dim: int, out_dims, qs, scales, bsums, ys=None,
                      biases=None):
    """One launch over up to three matrices sharing the quantized activation rows (q/k/v,
    gate/up). Returns the list of outputs [n_rows, out_dims[i]]."""
    import torch
    m = qs.shape[0]
    n_mats = len(ws)
    if ys is None:
        ys = [torch.empty((m, int(n)), dtype=torch.float32, device=qs.device) for n in out_dims]
    wa = (ctypes.c_void_p * n_mats)(*[w.data_ptr() for w in ws])
    ya = (ctypes.c_void_p * n_mats)(*[y.data_ptr() for y in ys])
    na = (ctypes.c_int * n_mats)(*[int(n) for n in out_dims])
    ba = None
    if biases is not None:
        ba = (ctypes.c_void_p * n_mats)(*[0 if b is None else b.data_ptr() for b in biases])
    _check(load_library().cllm_hip_gemv_q8_multi_dev(
        int(t), int(in_dim), n_mats, wa, na, ba, ya, int(m), _tp(qs), _tp(scales), _tp(bsums),
        _stream()))
    return ys


def gemv_q8_swiglu_dev(w_gate, w_up, t: int, in_dim: int, n_ff: int, qs, scales, bsums,
                       h=None, bias_gate=None, bias_up=None):
    """h = silu(gate . a) * (up . a) for the n_ff rows of the gate and up matrices against the
    quantized rows, in one launch (engine.cpp:509-512). Returns h [n_rows, n_ff]."""
    import torch
    m = qs.shape[0]
    if h is None:
        h = torch.empty((m, int(n_ff)), dtype=torch.float32, device=qs.device)
    _check(load_library().cllm_hip_gemv_q8_swiglu_dev(
        int(t), int(in_dim), int(n_ff), _tp(w_gate), _tp(w_up), _tp(bias_gate), _tp(bias_up),
        int(m), _tp(qs), _tp(scales), _tp(bsums), _tp(h), _stream()))
    return h


def rmsnorm_gemv_multi_dev(x, norm_w, eps: float, ws, t: int, in_dim: int, out_dims, ys=None,
                           biases=None):
    """RMSNorm of the one row x (float32 (1, in_dim), in_dim <= 4096) with weight norm_w, then
    gemv_q8_multi_dev on it, in one launch (engine.cpp:475-478); the bits of rmsnorm_q8_0_dev
    followed by gemv_q8_multi_dev. Returns the list of outputs [1, out_dims[i]]."""
    import torch
    n_mats = len(ws)
    if ys is None:
        ys = [torch.empty((1, int(n)), dtype=torch.float32, device=x.device) for n in out_dims]
    wa = (ctypes.c_void_p * n_mats)(*[w.data_ptr() for w in ws])
    ya = (ctypes.c_void_p * n_mats)(*[y.data_ptr() for y in ys])
    na = (ctypes.c_int * n_mats)(*[int(n) for n in out_dims])
    ba = None
    if biases is not None:
        ba = (ctypes.c_void_p * n_mats)(*[0 if b is None else b.data_ptr() for b in biases])
    _check(load_library().cllm_hip_rmsnorm_gemv_multi_dev(
        int(t), int(in_dim), n_mats, wa, na, ba, ya, _tp(x), _tp(norm_w), float(eps), _stream()))
    return ys


def rmsnorm_gemv_swiglu_dev(x, norm_w, eps: float, w_gate, w_up, t: int, in_dim: int, n_ff: int,
                            h=None, bias_gate=None, bias_up=None):
    """RMSNorm of the one row x, then gemv_q8_swiglu_dev on it, in one launch
    (engine.cpp:508-512); the bits of rmsnorm_q8_0_dev followed by gemv_q8_swiglu_dev.
    Returns h [1, n_ff]."""
    import torch
    if h is None:
        h = torch.empty((1, int(n_ff)), dtype=torch.float32, device=x.device)
    _check(load_library().cllm_hip_rmsnorm_gemv_swiglu_dev(
        int(t), int(in_dim), int(n_ff), _tp(w_gate), _tp(w_up), _tp(bias_gate), _tp(bias_up),
        _tp(x), _tp(norm_w), float(eps), _tp(h), _stream()))
    return h


def gemv_q8_residual_dev(w, t: int, in_dim: int, out_dim: int, qs, scales, bsums, y, bias=None):
    """y += vec_dot of every weight row against the quantized rows (device): a matmul and
    the residual add after it (engine.cpp:505-506, 512-513) in one launch."""
    m = qs.shape[0]
    _check(load_library().cllm_hip_gemv_q8_residual_dev(
        _tp(w), int(t), int(in_dim), int(out_dim), int(m), _tp(qs), _tp(scales), _tp(bsums),
        _tp(bias), _tp(y), _stream()))
    return y


def matmul_quant_dev(x, w, t: int, bias, in_dim: int, out_dim: int, y=None):
    """matmul_quant_batch on device tensors: x float32 (m, in_dim), w uint8 GGUF blocks."""
    import torch
    m = x.shape[0]
    if y is None:
        y = torch.empty((m, out_dim), dtype=torch.float32, device=x.device)
    _check(load_library().cllm_hip_matmul_quant_dev(_tp(x), _tp(w), int(t), _tp(bias),
                                                    int(in_dim), int(out_dim), int(m), _tp(y),
                                                    _stream()))
    return y


def matmul_quant_residual_dev(x, w, t: int, bias, in_dim: int, out_dim: int, y):
    """y += matmul_quant_batch(x, w) (+ bias) on device tensors: a matmul and the residual
    add after it (engine.cpp:505-506, 512-513)."""
    m = x.shape[0]
    _check(load_library().cllm_hip_matmul_quant_residual_dev(_tp(x), _tp(w), int(t), _tp(bias),
                                                             int(in_dim), int(out_dim), int(m),
                                                             _tp(y), _stream()))
    return y


def matmul_route(t: int, in_dim: int, out_dim: int, n_rows: int) -> str:
    return load_library().cllm_hip_matmul_route(int(t), int(in_dim), int(out_dim),
                                                int(n_rows)).decode()


def read_stream_dev(t) -> None:
    """Reads the CUDA tensor t's bytes once and computes nothing (cllm_hip_read_stream_dev): the
    one-launch HBM read ceiling a GEMV over the same bytes is measured against."""
    _check(load_library().cllm_hip_read_stream_dev(_tp(t), t.numel() * t.element_size(),
                                                   _stream()))


def matmul_plan(t: int, in_dim: int, out_dim: int, n_rows: int) -> str:
    """The kernel instantiation and split count the batch would run (or the route name)."""
    return load_library().cllm_hip_matmul_plan(int(t), int(in_dim), int(out_dim),
                                               int(n_rows)).decode()


def attention_plan(n_rows: int, pos0: int, n_head: int, n_head_kv: int, head_dim: int) -> str:
    """The attention kernel attention_dev would run for this shape, with its workgroups or
    sequence splits ("none" for an unsupported shape)."""
    return load_library().cllm_hip_attention_plan(int(n_rows), int(pos0), int(n_head),
                                                  int(n_head_kv), int(head_dim)).decode()


def tune(knob: str, *values: int) -> None:
    """Sets a process-wide kernel-choice override (cllm_hip_tune); no values resets it."""
    arr = (ctypes.c_int * max(len(values), 1))(*[int(v) for v in values])
    _check(load_library().cllm_hip_tune(knob.encode(), ctypes.cast(arr, ctypes.c_void_p),
                                        len(values)))


# ---- producers of a device-resident layer ------------------------------------------------

def _q8_buffers(m, n, device, want):
    import torch
    if not want:
        return None, None, None
    return (torch.empty((m, n), dtype=torch.int8, device=device),
            torch.empty((m, n // 32), dtype=torch.float32, device=device),
            torch.empty((m, n // 32), dtype=torch.int32, device=device))


def rmsnorm_q8_0_dev(x, w, eps: float, h=True, quantize=True):
    """RMSNorm of each row of x (float32 (m, n) CUDA tensor) with weight w (n,), fused with
    Q8_0 quantization -- engine.cpp:23-28 then quant.cpp:420-452. Returns (h, qs, scales,
    bsums); h is None when h=False, the Q8_0 triple None when quantize=False."""
    import torch
    m, n = x.shape
    hb = torch.empty_like(x) if h else None
    qs, sc, bs = _q8_buffers(m, n, x.device, quantize)
    _check(load_library().cllm_hip_rmsnorm_q8_0_dev(_tp(x), _tp(w), float(eps), int(n), int(m),
                                                    _tp(hb), _tp(qs), _tp(sc), _tp(bs),
                                                    _stream()))
    return hb, qs, sc, bs


def swiglu_q8_0_dev(gate, up, h=True, quantize=True):
    """silu(gate) * up (engine.cpp:38, 511, 596) fused with Q8_0 quantization; gate and up
    are float32 (m, n) CUDA tensors. Returns (h, qs, scales, bsums) like rmsnorm_q8_0_dev."""
    import torch
    m, n = gate.shape
    hb = torch.empty_like(gate) if h else None
    qs, sc, bs = _q8_buffers(m, n, gate.device, quantize)
    _check(load_library().cllm_hip_swiglu_q8_0_dev(_tp(gate), _tp(up), int(n), int(m), _tp(hb),
                                                   _tp(qs), _tp(sc), _tp(bs), _stream()))
    return hb, qs, sc, bs


def add_dev(x, d):
    """x += d in place (the residual adds, engine.cpp:506, 513)."""
    _check(load_library().cllm_hip_add_dev(_tp(x), _tp(d), int(x.numel()), _stream()))
    return x


# ---- prefill linear layer on the weight-row format ----------------------------------------

def mfma_act_new(in_dim: int, n_rows: int, device="cuda"):
    """A device buffer for n_rows rows of the weight-row kernels' activation format."""
    import torch
    nbytes = load_library().cllm_hip_mfma_act_bytes(int(in_dim), int(n_rows))
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def quantize_mfma_dev(x, act=None):
    """Q8_0 of the rows of x [n_rows, in_dim] into the weight-row format (a new buffer if act
    is None); returns act."""
    m, k = x.shape
    if act is None:
        act = mfma_act_new(k, m, x.device)
    _check(load_library().cllm_hip_quantize_mfma_dev(_tp(x), int(k), int(m), _tp(act), _stream()))
    return act


def rmsnorm_mfma_dev(x, norm_w, eps: float, h=None, act=None):
    """RMSNorm of the rows of x into h (fp32, when given) and the weight-row format; returns
    act."""
    m, k = x.shape
    if act is None:
        act = mfma_act_new(k, m, x.device)
    _check(load_library().cllm_hip_rmsnorm_mfma_dev(_tp(x), _tp(norm_w), float(eps), int(k),
                                                    int(m), _tp(h), _tp(act), _stream()))
    return act


def swiglu_mfma_dev(gate, up, h=None, act=None):
    """silu(gate) * up into h (fp32, when given) and the weight-row format; returns act."""
    m, n = gate.shape
    if act is None:
        act = mfma_act_new(n, m, gate.device)
    _check(load_library().cllm_hip_swiglu_mfma_dev(_tp(gate), _tp(up), int(n), int(m), _tp(h),
                                                   _tp(act), _stream()))
    return act


def matmul_mfma_dev(ws, t: int, in_dim: int, out_dims, act, n_rows: int, ys=None, biases=None):
    """matmul_quant_batch of the matrices ws (device weights, one type and in_dim) over the
    activation rows in act; returns the outputs [n_rows, out_dims[i]]."""
    import torch
    n_mats = len(ws)
    if ys is None:
        ys = [torch.empty((n_rows, int(n)), dtype=torch.float32, device=act.device)
              for n in out_dims]
    wa = (ctypes.c_void_p * n_mats)(*[w.data_ptr() for w in ws])
    ya = (ctypes.c_void_p * n_mats)(*[y.data_ptr() for y in ys])
    na = (ctypes.c_int * n_mats)(*[int(n) for n in out_dims])
    ba = None
    if biases is not None:
        ba = (ctypes.c_void_p * n_mats)(*[0 if b is None else b.data_ptr() for b in biases])
    _check(load_library().cllm_hip_matmul_mfma_dev(int(t), int(in_dim), n_mats, wa, na, ba, ya,
                                                   int(n_rows), _tp(act), _stream()))
    return ys


def matmul_mfma_plan(t: int, in_dim: int, out_dims, n_rows: int) -> str:
    na = (ctypes.c_int * len(out_dims))(*[int(n) for n in out_dims])
    return load_library().cllm_hip_matmul_mfma_plan(int(t), int(in_dim), len(out_dims), na,
                                                    int(n_rows)).decode()


# ---- GGUF files ---------------------------------------------------------------------------

@dataclass
class GgufTensorInfo:
    name: str
    type: int
    shape: tuple          # rows first
    offset: int           # in the data section
    host: int             # address in the mapping
    dev: int              # device address (0 without upload)


class GgufFile:
    """A GGUF file parsed by the library (reference GgufLoader::load, gguf.cpp:122-275);
    with upload=True its data section lives on the device and host tensor pointers into the
    mapping resolve to it in every matmul call."""

    def __init__(self, path: str, upload: bool = False):
        lib = load_library()
        h = ctypes.c_void_p()
        _check(lib.cllm_hip_gguf_open(str(path).encode(), 1 if upload else 0, ctypes.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            _check(load_library().cllm_hip_gguf_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self):
        return load_library().cllm_hip_gguf_tensor_count(self._h)

    def tensor(self, i: int) -> GgufTensorInfo:
        name = ctypes.c_char_p()
        t = ctypes.c_uint32()
        nd = ctypes.c_int()
        dims = (ctypes.c_uint64 * 4)()
        off = ctypes.c_uint64()
        host = ctypes.c_void_p()
        dev = ctypes.c_void_p()
        _check(load_library().cllm_hip_gguf_tensor(self._h, int(i), ctypes.byref(name),
                                                   ctypes.byref(t), ctypes.byref(nd), dims,
                                                   ctypes.byref(off), ctypes.byref(host),
                                                   ctypes.byref(dev)))
        return GgufTensorInfo(name.value.decode(), t.value, tuple(dims[:min(nd.value, 4)]),
                              off.value, host.value or 0, dev.value or 0)

    def find(self, name: str) -> int:
        return load_library().cllm_hip_gguf_find(self._h, name.encode())

    def config(self) -> ModelConfig:
        c = ModelConfig()
        _check(load_library().cllm_hip_gguf_config(self._h, ctypes.byref(c)))
        return c


# ---- float ops between the linear layers ------------------------------------------------

def rope_neox_dev(x, n_heads: int, head_dim: int, pos0: int, theta_base: float):
    """NEOX RoPE in place on x (float32 CUDA tensor of n_rows x n_heads x head_dim), row t at
    position pos0 + t -- engine.cpp:41-56."""
    n_rows = x.numel() // (n_heads * head_dim)
    _check(load_library().cllm_hip_rope_neox_dev(_tp(x), int(n_rows), int(n_heads),
                                                 int(head_dim), int(pos0), float(theta_base),
                                                 _stream()))
    return x


def rope_neox2_dev(q, n_head: int, k, n_head_kv: int, head_dim: int, pos0: int,
                   theta_base: float):
    """NEOX RoPE on the queries and the keys in one launch (engine.cpp:481-482)."""
    n_rows = q.numel() // (n_head * head_dim)
    _check(load_library().cllm_hip_rope_neox2_dev(_tp(q), int(n_head), _tp(k), int(n_head_kv),
                                                  int(n_rows), int(head_dim), int(pos0),
                                                  float(theta_base), _stream()))


def attention_dev(q, k_cache, v_cache, pos0: int, n_head: int, n_head_kv: int, head_dim: int,
                  out=None):
    """Grouped-query attention of the query rows q (n_rows x n_head x head_dim) over the
    caches (positions x n_head_kv x head_dim); row t sees positions [0, pos0 + t] --
    engine.cpp:114-146."""
    import torch
    n_rows = q.numel() // (n_head * head_dim)
    if out is None:
        out = torch.empty((n_rows, n_head * head_dim), dtype=torch.float32, device=q.device)
    _check(load_library().cllm_hip_attention_dev(_tp(q), _tp(k_cache), _tp(v_cache), int(n_rows),
                                                 int(pos0), int(n_head), int(n_head_kv),
                                                 int(head_dim), _tp(out), _stream()))
    return out


def attention_rope_dev(q, k_cache, v_cache, pos0: int, n_head: int, n_head_kv: int,
                       head_dim: int, theta_base: float, out=None):
    """A decode step's RoPE and attention in one launch (engine.cpp:486-495): q (one row,
    unrotated, left as it is) and the unrotated key row pos0 of k_cache (rotated in place) get
    the NEOX rotation at position pos0, then the attention over positions [0, pos0]."""
    import torch
    if out is None:
        out = torch.empty((1, n_head * head_dim), dtype=torch.float32, device=q.device)
    _check(load_library().cllm_hip_attention_rope_dev(
        _tp(q), _tp(k_cache), _tp(v_cache), int(pos0), int(n_head), int(n_head_kv),
        int(head_dim), float(theta_base), _tp(out), _stream()))
    return out


def dequantize_rows_dev(w, t: int, in_dim: int, ids, out=None):
    """Rows ids (int32 CUDA tensor) of the weight matrix w (uint8 CUDA tensor) as fp32 --
    the embedding lookup, bit for bit like dequantize_block."""
    import torch
    n = ids.numel()
    if out is None:
        out = torch.empty((n, in_dim), dtype=torch.float32, device=ids.device)
    _check(load_library().cllm_hip_dequantize_rows_dev(_tp(w), int(t), int(in_dim), _tp(ids),
                                                       int(n), _tp(out), _stream()))
    return out
