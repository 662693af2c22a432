"""CPU-only checks of the product libraries: they load, export every declared symbol, and
reject bad arguments with the reference's messages before touching a device."""
import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import cllm_inference_amd as C
from cllm_inference_amd import synth as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "cllm_hip.h")).read()
    return sorted(set(re.findall(r"\b(cllm_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = C.load_library()
    declared = header_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(C.SIGNATURES) == declared


def test_quant_api_library_exports_cpp_symbols():
    assert os.path.exists(C.QUANT_LIB_PATH)
    nm = shutil.which("nm")
    out = subprocess.run([nm, "-D", "--defined-only", "-C", C.QUANT_LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    for sym in ["cllm::matmul_quant(", "cllm::matmul_quant_batch(", "cllm::quantize_row_q8_0(",
                "cllm::vec_dot_row(", "cllm::has_vec_dot(", "cllm::block_size(",
                "cllm::type_size("]:
        assert sym in out, sym
    ctypes.CDLL(C.QUANT_LIB_PATH)


def test_sizes_match_reference_tables():
    for t in C.GgmlType:
        assert C.block_size(t) == {0: 1, 1: 1}.get(int(t), 32 if int(t) <= 9 else 256)
    want = {0: 4, 1: 2, 2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 9: 36, 10: 84, 11: 110, 12: 144,
            13: 176, 14: 210}
    for t, sz in want.items():
        assert C.type_size(t) == sz
    assert {int(t) for t in C.GgmlType if C.has_vec_dot(t)} == {2, 6, 8, 12, 13, 14}


def test_argument_errors_before_device_use():
    x = np.zeros(100, np.float32)
    w = np.zeros(4096, np.uint8)
    with pytest.raises(RuntimeError, match=r"^matmul_quant: in_dim not divisible by block size$"):
        C.matmul_quant(x, w, S.Q4_K, None, 100, 4)
    with pytest.raises(RuntimeError, match=r"^matmul_quant_batch: in_dim not divisible by block size$"):
        C.matmul_quant_batch(np.zeros((2, 100), np.float32), w, S.Q8_0, None, 100, 4, 2)
    # an id that is no GGML type fails like the reference's dequantize fallback
    # (quant.cpp:387); Q4_1 and the other types without vec_dot have float-dot kernels
    with pytest.raises(RuntimeError, match=r"^unsupported ggml type for dequantize$"):
        C.matmul_quant(np.zeros(64, np.float32), w, 5, None, 64, 4)
    with pytest.raises(RuntimeError, match=r"^vec_dot_row: no kernel for this type$"):
        qx = C.QuantizedQ8_0(scales=np.zeros(2, np.float32), qs=np.zeros(64, np.int8),
                             bsums=np.zeros(2, np.int32), n=64)
        C.vec_dot_rows(w, int(C.GgmlType.Q4_1), qx, 64, 4)
    with pytest.raises(RuntimeError, match=r"^quantize_row_q8_0: n not divisible by 32$"):
        C.quantize_row_q8_0(np.zeros(48, np.float32))
    # n_rows <= 0 returns without touching y (quant.cpp:1436)
    y = C.matmul_quant_batch(np.zeros((0, 64), np.float32), w, S.Q8_0, None, 64, 4, 0)
    assert y.shape == (0, 4)


def test_no_device_is_reported_not_faked():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    lib = C.load_library()
    assert lib.cllm_hip_init(0) == 5  # CLLM_HIP_E_NODEV
    assert b"device" in lib.cllm_hip_last_error()


def test_decode_plans():
    """One activation row over a weight stream of at least 4 MiB runs the streaming kernel
    (k_gemv_str, one workgroup per CU), shorter streams the register-ring k_gemv; 2 to 8 rows
    run as one streaming launch on the long streams, else in register-ring launches of up to 8.
    The tuning knob forces either kernel."""
    assert C.matmul_plan(S.Q4_K, 4096, 14336, 1) == "k_gemv_str<Q4_K,1> launches=1"
    assert C.matmul_plan(S.Q6_K, 4096, 128256, 1) == "k_gemv_str<Q6_K,1> launches=1"
    assert C.matmul_plan(S.Q6_K, 14336, 4096, 1) == "k_gemv_str<Q6_K,1> launches=1"
    assert C.matmul_plan(S.Q8_0, 896, 4864, 1) == "k_gemv_str<Q8_0,1> launches=1"
    assert C.matmul_plan(S.Q4_K, 4096, 1024, 1) == "k_gemv<Q4_K,1> launches=1"
    assert C.matmul_plan(S.Q4_0, 4096, 4096, 13) == "k_gemm_sm<Q4_0,1> splits=1 kp=16"
    try:
        C.tune("gemm_small", 2)
        assert C.matmul_plan(S.Q4_0, 4096, 4096, 13) == "k_gemv<Q4_0,8> launches=3"
    finally:
        C.tune("gemm_small")
    assert C.matmul_plan(S.Q4_K, 4096, 14336, 3) == "k_gemv_str<Q4_K,3> launches=1"
    assert C.matmul_plan(S.Q4_K, 4096, 14336, 5) == "k_gemv_str<Q4_K,5> launches=1"
    assert C.matmul_plan(S.Q4_K, 4096, 1024, 3) == "k_gemv<Q4_K,2> launches=2"
    try:
        C.tune("gemv_kernel", 1)
        assert C.matmul_plan(S.Q6_K, 4096, 128256, 1) == "k_gemv<Q6_K,1> launches=1"
        C.tune("gemv_kernel", 2)
        assert C.matmul_plan(S.Q6_K, 4096, 128256, 1) == "k_gemv_st<Q6_K,1> launches=1"
        C.tune("gemv_kernel", 3)
        assert C.matmul_plan(S.Q4_K, 4096, 1024, 1) == "k_gemv_str<Q4_K,1> launches=1"
    finally:
        C.tune("gemv_kernel")


def test_mid_batch_routes():
    """Below 16 rows, Q4_0 / Q5_0 keep the GEMV while it streams the batch in one launch (up to
    8 rows), else take the small-batch kernel from 8 rows. Q6_K keeps a streamed batch of up to 5 rows, else takes the
    small-batch kernel from 4 to 16 rows where the GEMV would need two launches or more, or on
    matrices of 32 M weights or more; the weight-row kernel beyond 16 rows. Q4_K keeps the GEMV
    below 8 rows, Q5_K up to 6, Q8_0 up to 8."""
    # (type, in_dim, out_dim, rows that go to the MFMA route among 1..16, to the small route)
    cases = [
        (S.Q6_K, 4096, 14336, set(), set(range(6, 17))),
        (S.Q6_K, 14336, 4096, set(), set(range(5, 17))),
        (S.Q6_K, 4096, 1024, set(), {5, 6, 7} | set(range(9, 17))),
        (S.Q4_0, 4096, 14336, set(), set(range(9, 17))),
        (S.Q5_0, 4096, 4096, set(), set(range(9, 17))),
        (S.Q4_0, 14336, 4096, set(), set(range(8, 17))),
    ]
    for t, k, n, want_mfma, want_small in cases:
        got = {m for m in range(1, 17) if C.matmul_route(t, k, n, m) == "mfma"}
        assert got == want_mfma, (S.TYPE_NAMES[t], k, n, sorted(got))
        got = {m for m in range(1, 17) if C.matmul_route(t, k, n, m) == "small"}
        assert got == want_small, (S.TYPE_NAMES[t], k, n, sorted(got))
    assert C.matmul_plan(S.Q6_K, 4096, 14336, 8) == "k_gemm_sm<Q6_K,1> splits=1 kp=4"
    assert C.matmul_plan(S.Q6_K, 14336, 4096, 8) == "k_gemm_sm<Q6_K,1> splits=4 kp=4"
    assert C.matmul_plan(S.Q6_K, 4096, 14336, 17) == "k_gemmw_q6k<4,1> splits=4"
    assert C.matmul_plan(S.Q6_K, 4096, 1024, 8) == "k_gemv<Q6_K,8> launches=1"
    # Q6_K rows of a multiple of 16 bytes only (k a multiple of 2048)
    assert C.matmul_route(S.Q6_K, 2816, 14336, 8) != "small"
    for m in range(1, 8):
        assert C.matmul_route(S.Q4_K, 4096, 14336, m) == "gemv"
        assert C.matmul_route(S.Q8_0, 4096, 4096, m) == "gemv"
    assert C.matmul_route(S.Q8_0, 4096, 4096, 8) == "gemv"
    assert C.matmul_route(S.Q5_K, 4096, 14336, 6) == "gemv"
    assert C.matmul_route(S.Q5_K, 4096, 14336, 7) == "small"


def test_prefill_plans():
    """Weight-row plans at large batches (256 CUs when no device is present): 256 x 128 tiles
    unsplit when they fill 3/4 of the CUs; on long K (24 stages of 128 elements per split or
    more) also on 2 or 4 splits that do; else 128 x 64 or 128 x 32 tiles, split to about two
    workgroups per CU. The Q4_K_M layer's shapes at 512 rows keep their plans."""
    assert C.matmul_plan(S.Q4_K, 4096, 14336, 512) == "k_gemmw_q4k<8,1,4,Q4_K> splits=1"
    assert C.matmul_plan(S.Q4_K, 4096, 4096, 512) == "k_gemmw_q4k<4,1,2,Q4_K> splits=2"
    assert C.matmul_plan(S.Q4_K, 4096, 1024, 512) == "k_gemmw_q4k<4,1,1,Q4_K> splits=4"
    assert C.matmul_plan(S.Q6_K, 14336, 4096, 512) == "k_gemmw_q6k<4,2> splits=2"
    # long K
    assert C.matmul_plan(S.Q4_K, 14336, 4096, 384) == "k_gemmw_q4k<8,1,4,Q4_K> splits=4"
    assert C.matmul_plan(S.Q4_K, 14336, 4096, 1024) == "k_gemmw_q4k<8,1,4,Q4_K> splits=2"
    assert C.matmul_plan(S.Q5_K, 11008, 4096, 768) == "k_gemmw_q4k<8,1,4,Q5_K> splits=2"
    assert C.matmul_plan(S.Q4_K, 14336, 2048, 768) == "k_gemmw_q4k<8,1,4,Q4_K> splits=4"
    # too few stages per split (K = 11008 on 4 splits), too few tiles (2048 rows at 512)
    assert C.matmul_plan(S.Q4_K, 11008, 4096, 512) == "k_gemmw_q4k<4,1,2,Q4_K> splits=2"
    assert C.matmul_plan(S.Q4_K, 14336, 2048, 512) == "k_gemmw_q4k<4,1,2,Q4_K> splits=4"
    # 32-element block types and Q6_K above 256 rows: splits by stage-rounds while the tiles
    # make fewer than two rounds (1 resident workgroup per CU for b32, 2 for Q6_K)
    assert C.matmul_plan(S.Q8_0, 14336, 4096, 384) == "k_gemmw_b32<Q8_0,4,2> splits=4"
    assert C.matmul_plan(S.Q8_0, 14336, 4096, 512) == "k_gemmw_b32<Q8_0,4,2> splits=1"
    assert C.matmul_plan(S.Q8_0, 14336, 4096, 768) == "k_gemmw_b32<Q8_0,4,2> splits=2"
    assert C.matmul_plan(S.Q8_0, 4096, 14336, 768) == "k_gemmw_b32<Q8_0,4,2> splits=1"
    assert C.matmul_plan(S.Q8_0, 4096, 4096, 256) == "k_gemmw_b32<Q8_0,4,2> splits=4"
    assert C.matmul_plan(S.Q6_K, 4096, 4096, 384) == "k_gemmw_q6k<4,2> splits=4"
    assert C.matmul_plan(S.Q6_K, 4096, 4096, 768) == "k_gemmw_q6k<4,2> splits=4"
    assert C.matmul_plan(S.Q6_K, 4096, 14336, 1024) == "k_gemmw_q6k<4,2> splits=1"
    assert C.matmul_plan(S.Q4_K, 4096, 4096, 768) == "k_gemmw_q4k<4,1,2,Q4_K> splits=4"
    assert C.matmul_plan(S.Q4_K, 4096, 11008, 384) == "k_gemmw_q4k<4,1,2,Q4_K> splits=4"
    assert C.matmul_plan(S.Q5_K, 4096, 14336, 384) == "k_gemmw_q4k<4,1,2,Q5_K> splits=2"
    assert C.matmul_plan(S.Q4_K, 4096, 4096, 1024) == "k_gemmw_q4k<4,1,2,Q4_K> splits=1"


def test_shapes_past_32_bit_offsets_take_the_int8_kernel():
    """The weight-row kernels index with 32-bit byte offsets: a Q8_0 262144 x 16384 output head
    (4.5 GB of weights) and a batch whose fp16 activations reach 4 GiB go to the int8 kernel
    (64-bit offsets); just below the limit the weight-row kernel keeps them."""
    assert C.matmul_route(S.Q8_0, 16384, 262144, 512) == "mfma"
    assert C.matmul_plan(S.Q8_0, 16384, 262144, 512) == "k_gemm_i8"
    # the small-batch kernel (64-bit offsets) keeps its batches; above it, the int8 kernel
    assert C.matmul_route(S.Q8_0, 16384, 262144, 16) == "small"
    assert C.matmul_plan(S.Q8_0, 16384, 262144, 100) == "k_gemm_i8"
    # weights just under 4 GiB: 4 GiB / 34 bytes per block, 512 blocks per row
    n = ((1 << 32) - 1) // (512 * 34)
    assert C.matmul_plan(S.Q8_0, 16384, n, 512).startswith("k_gemmw_b32<Q8_0")
    assert C.matmul_plan(S.Q8_0, 16384, n + 1, 512) == "k_gemm_i8"
    # activations: 2 m k bytes of fp16 reach 4 GiB at m k = 2^31
    assert C.matmul_plan(S.Q4_K, 8192, 4096, (1 << 31) // 8192 - 1).startswith("k_gemmw_q4k")
    assert C.matmul_plan(S.Q4_K, 8192, 4096, (1 << 31) // 8192) == "k_gemm_i8"


def test_small_batch_plans():
    """8 to 32 rows of Q4_K / Q5_K weights and 8 to 64 of Q8_0 take the small-batch kernel on
    a batch quantized once: token tiles of 16, K split over workgroups only where 16 rows per
    tile of it would not fit the 64 KB of activation LDS, K parts per workgroup chosen for one
    workgroup per CU (256 CUs when no device is present)."""
    assert C.matmul_plan(S.Q5_K, 4096, 14336, 16) == "k_gemm_sm<Q5_K,1> splits=1 kp=4"
    # above 16 rows, matrices of 8192 output rows or more take the weight-row kernel
    assert C.matmul_plan(S.Q5_K, 4096, 14336, 32) == "k_gemmw_q4k<4,1,1,Q5_K> splits=4"
    assert C.matmul_plan(S.Q5_K, 4096, 14336, 17) == "k_gemmw_q4k<4,1,1,Q5_K> splits=4"
    assert C.matmul_plan(S.Q5_K, 4096, 4096, 32) == "k_gemm_sm<Q5_K,2> splits=2 kp=8"
    assert C.matmul_plan(S.Q8_0, 4096, 14336, 32) == "k_gemm_sm<Q8_0,2> splits=2 kp=2"
    assert C.matmul_plan(S.Q8_0, 4096, 4096, 16) == "k_gemm_sm<Q8_0,1> splits=1 kp=16"
    assert C.matmul_plan(S.Q8_0, 4096, 4096, 64) == "k_gemm_sm<Q8_0,4> splits=4 kp=4"
    assert C.matmul_plan(S.Q4_K, 14336, 4096, 16) == "k_gemm_sm<Q4_K,1> splits=4 kp=4"
    assert C.matmul_route(S.Q4_K, 4096, 14336, 4) == "gemv"
    assert C.matmul_route(S.Q4_K, 4096, 14336, 8) == "small"
    assert C.matmul_route(S.Q4_K, 4096, 14336, 64) == "mfma"
    assert C.matmul_route(S.Q8_0, 4096, 4096, 64) == "small"
    assert C.matmul_route(S.Q6_K, 4096, 14336, 16) == "small"
    assert C.matmul_route(S.Q6_K, 4096, 14336, 17) == "mfma"
    try:
        C.tune("gemm_small", 1)
        assert C.matmul_route(S.Q4_K, 4096, 14336, 3) == "small"
        C.tune("gemm_small", 2)
        assert C.matmul_route(S.Q4_K, 4096, 14336, 16) == "mfma"
        C.tune("gemm_small")
        C.tune("gemm_kernel", 1)
        assert C.matmul_route(S.Q4_K, 4096, 14336, 16) == "mfma"
    finally:
        C.tune("gemm_small")
        C.tune("gemm_kernel")


def _libc():
    libc = ctypes.CDLL(None, use_errno=True)
    libc.mmap.restype = ctypes.c_void_p
    libc.mmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                          ctypes.c_int, ctypes.c_long]
    libc.munmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    return libc


PROT_READ, PROT_WRITE, MAP_SHARED, MAP_PRIVATE, MAP_FIXED = 1, 2, 1, 2, 0x10


def test_attention_plans():
    """Many query rows take the MFMA kernel (32 or more of its workgroups: n_kv x pairs of
    row blocks of 32 / n_rep rows, 16 / n_rep at head_dim 256); fewer rows, and a decode row,
    the sequence-split kernel; the attention_kernel knob forces either."""
    p = C.attention_plan
    assert p(512, 0, 32, 8, 128) == "k_attention_mfma<128,2,8> workgroups=256"
    assert p(64, 0, 32, 8, 128) == "k_attention_mfma<128,2,8> workgroups=32"
    assert p(49, 1024, 32, 8, 128) == "k_attention_mfma<128,2,8> workgroups=32"
    assert p(48, 1024, 32, 8, 128).startswith("k_attention<128> splits=")
    assert p(1, 4095, 32, 8, 128) == "k_attention<128> splits=64"
    assert p(1, 0, 32, 8, 128) == "k_attention<128> splits=1"
    assert p(2048, 0, 8, 1, 256) == "k_attention_mfma<256,1,4> workgroups=512"
    assert p(200, 3, 32, 4, 64) == "k_attention_mfma<64,2,8> workgroups=100"
    assert p(16, 0, 32, 2, 128) == "none"   # 16 query heads per KV head
    assert p(16, 0, 32, 8, 96) == "none"
    try:
        C.tune("attention_kernel", 1)
        assert p(512, 0, 32, 8, 128).startswith("k_attention<128> splits=")
        C.tune("attention_kernel", 2)
        assert p(1, 300, 32, 8, 128) == "k_attention_mfma<128,2,8> workgroups=8"
    finally:
        C.tune("attention_kernel")
    with pytest.raises(RuntimeError, match="attention_kernel is 0, 1 or 2"):
        C.tune("attention_kernel", 3)


def test_file_mapping_identity_sees_remaps_and_rewrites(tmp_path):
    """The check made before the device copy of a read-only private file mapping (the engine's
    mmap'd GGUF) is reused: a file unmapped and another mapped at the same address, a rewrite
    in place (same inode, O_TRUNC too), and an unlinked file all change what it compares, and
    memory that is not a read-only private file mapping is refused."""
    import time
    libc = _libc()
    size = 4 * 4096
    rng = np.random.default_rng(3)
    paths = []
    for name in ("a.bin", "b.bin"):
        p = tmp_path / name
        p.write_bytes(rng.integers(0, 256, size, dtype=np.uint8).tobytes())
        paths.append(str(p))
    fa = os.open(paths[0], os.O_RDONLY)
    fb = os.open(paths[1], os.O_RDONLY)
    addr = libc.mmap(None, size, PROT_READ, MAP_PRIVATE, fa, 0)
    assert addr not in (None, ctypes.c_void_p(-1).value)
    try:
        id_a = C.file_mapping_identity(addr + 100)
        st = os.stat(paths[0])
        assert id_a[:4] == (addr, addr + size, 0, st.st_ino)
        assert id_a[4] == (os.major(st.st_dev) << 32 | os.minor(st.st_dev))
        assert id_a[5] == size and id_a[6] == st.st_mtime_ns and id_a[7] == st.st_ctime_ns
        assert id_a[8] == 1
        # unmap, then map the other file at the same address
        assert libc.munmap(addr, size) == 0
        assert libc.mmap(addr, size, PROT_READ, MAP_PRIVATE | MAP_FIXED, fb, 0) == addr
        id_b = C.file_mapping_identity(addr)
        assert id_b[:2] == id_a[:2] and id_b[3] == os.stat(paths[1]).st_ino != id_a[3]
        # the same file rewritten in place, same size: same inode, new times
        time.sleep(0.05)
        with open(paths[1], "r+b") as f:
            f.write(rng.integers(0, 256, size, dtype=np.uint8).tobytes())
        id_b2 = C.file_mapping_identity(addr)
        assert id_b2[3] == id_b[3] and id_b2[5] == size
        assert (id_b2[6], id_b2[7]) != (id_b[6], id_b[7])
        time.sleep(0.05)
        with open(paths[1], "wb") as f:  # O_TRUNC, then the same size again
            f.write(rng.integers(0, 256, size, dtype=np.uint8).tobytes())
        id_b3 = C.file_mapping_identity(addr)
        assert id_b3[3] == id_b[3] and (id_b3[6], id_b3[7]) != (id_b2[6], id_b2[7])
        # unlinked: no longer reachable by its path, the mapping alone identifies it
        os.unlink(paths[1])
        id_b4 = C.file_mapping_identity(addr)
        assert id_b4[:5] == id_b[:5] and id_b4[8] == 0
    finally:
        libc.munmap(addr, size)
        os.close(fa)
        os.close(fb)
    # anonymous memory and a shared writable mapping are not read-only private file mappings
    with pytest.raises(RuntimeError, match="read-only private file mapping"):
        C.file_mapping_identity(np.zeros(4096, np.uint8).ctypes.data)
    fa = os.open(paths[0], os.O_RDWR)
    addr = libc.mmap(None, size, PROT_READ | PROT_WRITE, MAP_SHARED, fa, 0)
    try:
        with pytest.raises(RuntimeError, match="read-only private file mapping"):
            C.file_mapping_identity(addr)
    finally:
        libc.munmap(addr, size)
        os.close(fa)
