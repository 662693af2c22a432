"""Deterministic synthetic GGUF weight blocks and fp32 activations.

The reference ships no weights or fixtures for its quantized linear path, so every workload
here is synthetic: raw GGUF block bytes laid out exactly as the reference reads them
(src/core/quant.cpp:39-336) with field distributions chosen per workload, and fp32
activation rows ~N(0,1). Generation is pure numpy (PCG64), so the same seed gives the same
bytes on any host.
"""
from __future__ import annotations

import numpy as np

# GGML type ids, include/cllm/core/quant.hpp:13-27
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = (
    0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14)

TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
              Q8_0: "Q8_0", Q8_1: "Q8_1", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
              Q5_K: "Q5_K", Q6_K: "Q6_K"}
NAME_TO_TYPE = {v: k for k, v in TYPE_NAMES.items()}

# The six types with a vec_dot kernel (src/core/quant.cpp:1347-1357); the others take the
# reference's dequantize-and-float-dot fallback (1404-1430).
VEC_DOT_TYPES = (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K)
FLOAT_DOT_TYPES = (F32, F16, Q4_1, Q5_1, Q8_1, Q2_K, Q3_K)

# elements per block and bytes per block, src/core/quant.cpp:340-369
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32, Q8_1: 32,
         Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q8_1: 36,
             Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def row_bytes(qtype: int, k: int) -> int:
    return (k // BLOCK[qtype]) * TYPE_SIZE[qtype]


def _f16_bytes(rng: np.random.Generator, n: int, lo: float, hi: float) -> np.ndarray:
    vals = rng.uniform(lo, hi, size=n).astype(np.float16)
    return vals.view(np.uint8).reshape(n, 2)


def make_weight(qtype: int, n: int, k: int, seed: int) -> np.ndarray:
    """Weight matrix n x k of type qtype as a flat uint8 array of n * row_bytes bytes.

    Field distributions:
      Q8_0: d ~ U(0.002, 0.02) fp16, qs int8 ~ U[-127, 127]
      Q4_0: d ~ U(0.002, 0.02), qs random bytes
      Q5_0: d ~ U(0.002, 0.02), qh and qs random bytes
      Q4_K: d ~ U(1e-3, 1e-2), dmin ~ U(1e-4, 1e-3), 12 random scale bytes (every 6-bit
            scale and min then decodes uniform on [0, 63]), qs random bytes
      Q5_K: as Q4_K plus 32 random qh bytes
      Q6_K: ql, qh random bytes, sc int8 ~ U[-32, 31], d ~ U(1e-3, 1e-2)
      F32, F16: values ~ N(0, 0.02)
      Q4_1, Q5_1: d ~ U(0.002, 0.02), m ~ U(-0.15, -0.01), qh and qs random bytes
      Q8_1: d ~ U(0.002, 0.02), s = d * (sum of the block's qs) as fp16, qs ~ U[-127, 127]
      Q2_K: 16 random scale bytes, qs random, d ~ U(1e-3, 1e-2), dmin ~ U(1e-4, 1e-3)
      Q3_K: hmask, qs and the 12 scale bytes random, d ~ U(1e-3, 1e-2)
    """
    if k % BLOCK[qtype]:
        raise ValueError("k must be a multiple of the block size")
    rng = np.random.default_rng([seed, 0xB10C, qtype])
    nblk = n * (k // BLOCK[qtype])
    ts = TYPE_SIZE[qtype]
    raw = np.frombuffer(rng.bytes(nblk * ts), dtype=np.uint8).copy()
    blk = raw.reshape(nblk, ts)
    if qtype == Q8_0:
        blk[:, 0:2] = _f16_bytes(rng, nblk, 0.002, 0.02)
        blk[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    elif qtype in (Q4_0, Q5_0):
        blk[:, 0:2] = _f16_bytes(rng, nblk, 0.002, 0.02)
    elif qtype in (Q4_K, Q5_K):
        blk[:, 0:2] = _f16_bytes(rng, nblk, 1e-3, 1e-2)
        blk[:, 2:4] = _f16_bytes(rng, nblk, 1e-4, 1e-3)
    elif qtype == Q6_K:
        blk[:, 192:208] = rng.integers(-32, 32, size=(nblk, 16), dtype=np.int8).view(np.uint8)
        blk[:, 208:210] = _f16_bytes(rng, nblk, 1e-3, 1e-2)
    elif qtype == F32:
        raw[:] = (rng.standard_normal(nblk, dtype=np.float32) * np.float32(0.02)).view(np.uint8)
    elif qtype == F16:
        raw[:] = (rng.standard_normal(nblk, dtype=np.float32) * np.float32(0.02)).astype(
            np.float16).view(np.uint8)
    elif qtype in (Q4_1, Q5_1):
        blk[:, 0:2] = _f16_bytes(rng, nblk, 0.002, 0.02)
        blk[:, 2:4] = _f16_bytes(rng, nblk, -0.15, -0.01)
    elif qtype == Q8_1:
        d = rng.uniform(0.002, 0.02, size=nblk).astype(np.float16)
        q = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8)
        blk[:, 0:2] = d.view(np.uint8).reshape(nblk, 2)
        blk[:, 2:4] = (d.astype(np.float32) * q.sum(axis=1, dtype=np.int32)).astype(
            np.float16).view(np.uint8).reshape(nblk, 2)
        blk[:, 4:36] = q.view(np.uint8)
    elif qtype == Q2_K:
        blk[:, 80:82] = _f16_bytes(rng, nblk, 1e-3, 1e-2)
        blk[:, 82:84] = _f16_bytes(rng, nblk, 1e-4, 1e-3)
    elif qtype == Q3_K:
        blk[:, 108:110] = _f16_bytes(rng, nblk, 1e-3, 1e-2)
    else:
        raise ValueError(f"unknown ggml type {qtype}")
    return raw


def make_activation(m: int, k: int, seed: int, outliers: bool = False) -> np.ndarray:
    """fp32 activations m x k ~ N(0, 1); with outliers, each element independently (p = 0.01)
    is scaled by 20."""
    rng = np.random.default_rng([seed, 0xAC7])
    x = rng.standard_normal(size=(m, k), dtype=np.float32)
    if outliers:
        mask = rng.random(size=(m, k)) < 0.01
        x[mask] *= np.float32(20.0)
    return x


# The five workloads: (name, [(label, qtype, n_out, k_in)], m_values, outliers, seed)
CONFIGS = {
    "c0_q8_0_gemv": dict(mats=[("w", Q8_0, 4864, 896)], m=[1], outliers=False, seed=20260),
    "c1_q4_k_gemv": dict(mats=[("ffn", Q4_K, 14336, 4096)], m=[1], outliers=False, seed=20261),
    "c2_q6_k_head": dict(mats=[("output", Q6_K, 128256, 4096)], m=[1], outliers=False, seed=20262),
    "c3_q4_k_m_layer": dict(
        mats=[("wq", Q4_K, 4096, 4096), ("wk", Q4_K, 1024, 4096), ("wv", Q4_K, 1024, 4096),
              ("wo", Q4_K, 4096, 4096), ("gate", Q4_K, 14336, 4096), ("up", Q4_K, 14336, 4096),
              ("down", Q6_K, 4096, 14336)],
        m=[512], outliers=False, seed=20263),
    "c4_m_sweep": dict(mats=[("q5_k", Q5_K, 14336, 4096), ("q8_0", Q8_0, 4096, 4096)],
                       m=[1, 4, 16, 64, 256], outliers=True, seed=20264),
}


def config_weight(cfg: str, label: str) -> tuple[int, int, int, np.ndarray]:
    """(qtype, n, k, bytes) of one matrix of a named workload."""
    c = CONFIGS[cfg]
    for i, (lab, qt, n, k) in enumerate(c["mats"]):
        if lab == label:
            return qt, n, k, make_weight(qt, n, k, c["seed"] * 16 + i)
    raise KeyError(label)


def config_activation(cfg: str, m: int, k: int) -> np.ndarray:
    c = CONFIGS[cfg]
    return make_activation(m, k, c["seed"] * 16 + 15 + k, outliers=c["outliers"])


def rounding_boundary_activation(m: int, k: int, seed: int) -> np.ndarray:
    """fp32 activations m x k in which every 32-element block holds one value x whose Q8_0
    product x * id rounds to the tie fl(x * id) = k + 0.5, while the exact product lies on the
    side of k + 0.5 away from the even neighbour -- so rint(fl(x * id)), the reference's quant,
    and the rounding of the exact product (what a fused multiply-add would give) differ by one.
    The block's other elements are uniform in (-a, a), a its largest magnitude."""
    rng = np.random.default_rng([seed, 0xB0D])
    x = rng.uniform(-1.0, 1.0, size=(m, k)).astype(np.float32)
    for t in range(m):
        for b in range(k // 32):
            blk = x[t, 32 * b: 32 * b + 32]
            a = np.float32(rng.uniform(0.5, 4.0))
            blk *= a * np.float32(0.98)
            blk[0] = a  # the block's amax
            d = np.float32(a / np.float32(127.0))
            inv = np.float32(np.float32(1.0) / d)
            for _ in range(10000):
                kk = int(rng.integers(1, 126))
                cand = np.float32((kk + 0.5) / float(inv))
                for c in (cand, np.nextafter(cand, np.float32(0)), np.nextafter(cand, np.float32(1e9))):
                    exact = float(c) * float(inv)  # exact in double: 24 x 24 bits
                    if (abs(c) < a and float(np.float32(exact)) == kk + 0.5 and
                            np.rint(exact) != np.rint(kk + 0.5)):
                        blk[1 + int(rng.integers(0, 31))] = -c if rng.integers(0, 2) else c
                        break
                else:
                    continue
                break
            else:
                raise RuntimeError("no boundary value found")
    return x
