"""ctypes access to the test oracles: the C restatement (liboracle.so) and, where it was built,
the reference compiled from its own sources (_ref/libcllm_ref.so).

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, always as the reference the results are compared with or the timed CPU
baseline, never as the product.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libcllm_ref.so")
DROPIN_SO = os.path.join(HERE, "_ref", "libengine_dropin.so")
REF_ROOT = "/root/reference"

_P = ctypes.c_void_p
_I = ctypes.c_int
_U = ctypes.c_uint32
_I64 = ctypes.c_int64


def build(with_ref: bool = True, dropin: bool = False) -> None:
    """Compiles liboracle.so, and _ref/libcllm_ref.so when the reference tree is present; with
    dropin (after cllm_inference_amd's libraries are built) also _ref/libengine_dropin.so."""
    targets = ["all"]
    if with_ref and os.path.isdir(REF_ROOT):
        targets.append("ref")
        if dropin:
            targets.append("dropin")
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class _Lib:
    """Common calls of both libraries (prefix 'oracle_' or 'ref_')."""

    def __init__(self, path: str, prefix: str):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = ctypes.CDLL(path)
        self.prefix = prefix
        sig = {
            "quantize_row_q8_0": (_I, [_P, _I64, _P, _P, _P]),
            "matmul_quant": (_I, [_P, _P, _U, _P, _I, _I, _P, _I]),
            "matmul_quant_batch": (_I, [_P, _P, _U, _P, _I, _I, _I, _P, _I]),
            "dequantize": (_I, [_P, _P, _U, _I64]),
            "last_error": (ctypes.c_char_p, []),
        }
        optional = {  # present in rebuilt libraries only
            "dequantize_block": (_I, [_P, _P, _U, _I64]),
            "dequantize_block_f16": (_I, [_P, _P, _U, _I64]),
            "dequantize_f16": (_I, [_P, _P, _U, _I64]),
            "float_to_half": (ctypes.c_uint16, [ctypes.c_float]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(self.lib, prefix + name)
            fn.restype, fn.argtypes = res, args
        for name, (res, args) in optional.items():
            fn = getattr(self.lib, prefix + name, None)
            if fn is not None:
                fn.restype, fn.argtypes = res, args

    def _fn(self, name):
        return getattr(self.lib, self.prefix + name)

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self._fn("last_error")().decode())

    def quantize(self, x: np.ndarray):
        """Row-wise Q8_0 of x (m, k) -> (qs int8 (m, k), scales f32 (m, k/32), bsums i32)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        m, k = x2.shape
        qs = np.empty((m, k), np.int8)
        sc = np.empty((m, k // 32), np.float32)
        bs = np.empty((m, k // 32), np.int32)
        for t in range(m):
            self._check(self._fn("quantize_row_q8_0")(_ptr(x2[t]), k, _ptr(qs[t]), _ptr(sc[t]),
                                                      _ptr(bs[t])))
        return qs, sc, bs

    def matmul(self, x, w, qtype, bias, k, n, m, threads=0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        y = np.zeros((max(m, 1), n), np.float32)
        if m == 1:
            rc = self._fn("matmul_quant")(_ptr(x), _ptr(w), int(qtype), _ptr(b), int(k), int(n),
                                          _ptr(y), int(threads))
        else:
            rc = self._fn("matmul_quant_batch")(_ptr(x), _ptr(w), int(qtype), _ptr(b), int(k),
                                                int(n), int(m), _ptr(y), int(threads))
        self._check(rc)
        return y

    def dequantize(self, src, qtype, n):
        out = np.empty(n, np.float32)
        self._check(self._fn("dequantize")(_ptr(np.ascontiguousarray(src, dtype=np.uint8)),
                                           _ptr(out), int(qtype), int(n)))
        return out

    def dequantize_block(self, src, qtype, n):
        """dequantize_block: any n (the reference library's own entry takes any n too)."""
        out = np.empty(n, np.float32)
        name = "dequantize_block" if self.prefix == "oracle_" else "dequantize"
        self._check(self._fn(name)(_ptr(np.ascontiguousarray(src, dtype=np.uint8)), _ptr(out),
                                   int(qtype), int(n)))
        return out

    def dequantize_block_f16(self, src, qtype, n):
        out = np.empty(n, np.uint16)
        name = "dequantize_block_f16" if self.prefix == "oracle_" else "dequantize_f16"
        self._check(self._fn(name)(_ptr(np.ascontiguousarray(src, dtype=np.uint8)), _ptr(out),
                                   int(qtype), int(n)))
        return out

    def float_to_half(self, x):
        f = self._fn("float_to_half")
        return np.array([f(float(v)) for v in np.asarray(x, np.float32)], np.uint16)


class Oracle(_Lib):
    def __init__(self, path: str = ORACLE_SO):
        super().__init__(path, "oracle_")
        f = self.lib.oracle_matmul_quant_f64
        f.restype = _I
        f.argtypes = [_P, _P, _U, _P, _I, _I, _I, _P, _P]

    def rms_norm(self, x, w, eps):
        """rms_norm_ptr of each row of x (m, n) with weight w (n,)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        out = np.empty_like(x2)
        f = self.lib.oracle_rms_norm
        f.restype, f.argtypes = _I, [_P, _P, _I, _I, ctypes.c_float, _P]
        self._check(f(_ptr(x2), _ptr(np.ascontiguousarray(w, dtype=np.float32)), x2.shape[1],
                      x2.shape[0], float(eps), _ptr(out)))
        return out.reshape(x.shape)

    def swiglu(self, gate, up):
        """silu(gate) * up element-wise."""
        g = np.ascontiguousarray(gate, dtype=np.float32)
        u = np.ascontiguousarray(up, dtype=np.float32)
        out = np.empty_like(g)
        f = self.lib.oracle_swiglu
        f.restype, f.argtypes = _I, [_P, _P, _I64, _P]
        self._check(f(_ptr(g), _ptr(u), g.size, _ptr(out)))
        return out

    def matmul_f64(self, x, w, qtype, bias, k, n, m):
        """fp64 evaluation and per-output absolute-term sums (tolerance floors)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        y = np.zeros((m, n), np.float64)
        a = np.zeros((m, n), np.float64)
        self._check(self.lib.oracle_matmul_quant_f64(_ptr(x), _ptr(w), int(qtype), _ptr(b), int(k),
                                                     int(n), int(m), _ptr(y), _ptr(a)))
        return y, a


class Reference(_Lib):
    """The reference's quant.cpp + thread_pool.cpp + gguf.cpp, compiled unmodified
    (oracle/Makefile)."""

    def __init__(self, path: str = REF_SO):
        super().__init__(path, "ref_")

    def engine_logits(self, path: str, tokens, prefill: bool = False, threads: int = 4):
        """The reference engine's logits on the model file: prefill(tokens) -> (1, vocab), or
        forward(t) for each token in turn -> (len(tokens), vocab)."""
        f = self.lib.ref_engine_logits
        f.restype = ctypes.c_long
        f.argtypes = [ctypes.c_char_p, _P, _I, _I, _I, _P, ctypes.c_size_t]
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(1 << 22, np.float32)
        n = f(str(path).encode(), _ptr(toks), len(toks), 1 if prefill else 0, threads, _ptr(out),
              out.size)
        if n < 0:
            raise RuntimeError(self.lib.ref_last_error().decode())
        rows = 1 if prefill else len(toks)
        return out[:n].reshape(rows, n // rows).copy()

    def gguf_dump(self, path: str):
        """GgufLoader::load(path) as (config fields, [(name, type, shape, offset, data_delta)])."""
        f = self.lib.ref_gguf_dump
        f.restype, f.argtypes = ctypes.c_long, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
        buf = ctypes.create_string_buffer(1 << 22)
        n = f(str(path).encode(), buf, len(buf))
        if n < 0:
            raise RuntimeError(self.lib.ref_last_error().decode())
        lines = buf.raw[:n].decode().splitlines()
        head = lines[0].split()
        cfg = dict(arch="" if head[0] == "-" else head[0],
                   **{k: int(v) for k, v in zip(("n_layers", "n_embd", "n_head", "n_head_kv",
                                                 "n_ctx", "n_ff", "vocab_size", "head_dim"),
                                                head[1:9])},
                   rope_theta=float.fromhex(head[9]), norm_eps=float.fromhex(head[10]))
        tensors = []
        for ln in lines[1:]:
            p = ln.split()
            nd = int(p[2])
            tensors.append((p[0], int(p[1]), tuple(int(v) for v in p[3:3 + nd]), int(p[3 + nd]),
                            int(p[4 + nd])))
        return cfg, tensors


class DropIn(Reference):
    """The reference's engine.cpp, gguf.cpp and thread_pool.cpp compiled against this
    repository's headers and linked to libcllm_quant.so (oracle/Makefile, `dropin`): the
    reference engine with every Quant call served by the MI355X kernels. A test harness for
    the drop-in boundary; the code under test is libcllm_quant.so / libcllm_hip.so."""

    def __init__(self, path: str = DROPIN_SO):
        super().__init__(path)


def oracle() -> Oracle:
    return Oracle()


def reference_or_none():
    try:
        return Reference()
    except (FileNotFoundError, OSError):
        return None


def rel_err_floored(got: np.ndarray, ref: np.ndarray, abs_sum: np.ndarray, floor_pow: int = -10):
    """|got - ref| / max(|ref|, 2^floor_pow * abs_sum): the gate used by the parity tests for
    rows whose output nearly cancels. Returns (max floored relative error, rows that used the
    floor, max raw relative error)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    floor = abs_sum * 2.0 ** floor_pow
    denom = np.maximum(np.abs(ref), floor)
    denom = np.where(denom == 0, 1.0, denom)
    err = np.abs(got - ref) / denom
    raw = np.abs(got - ref) / np.where(ref == 0, 1.0, np.abs(ref))
    return float(err.max(initial=0.0)), int((np.abs(ref) < floor).sum()), float(raw.max(initial=0.0))
