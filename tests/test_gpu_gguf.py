"""GGUF upload on the GPU: the data section copied once to the device, host tensor
pointers into the mapping resolving to that copy in the Quant API calls, and the device
addresses cllm_hip_gguf_tensor reports holding the file's bytes."""
import ctypes
import os

import numpy as np
import pytest

import cllm_inference_amd as C
from cllm_inference_amd import synth as S
import gguf_writer as G
from test_gpu_parity import bits, _dev

pytestmark = pytest.mark.gpu


def test_upload_and_pointer_translation(gpu, tmp_path):
    import torch
    mats = [("blk.0.ffn_up.weight", S.Q4_K, 1024, 4096), ("output.weight", S.F16, 512, 896),
            ("blk.0.attn_v.weight", S.Q6_K, 256, 4096)]
    tensors = [(name, (n, k), qt, S.make_weight(qt, n, k, 40 + i).tobytes())
               for i, (name, qt, n, k) in enumerate(mats)]
    path = tmp_path / "w.gguf"
    G.write_gguf(path, [("general.architecture", G.STR, "llama")], tensors)
    with C.GgufFile(path, upload=True) as g:
        cfg = g.config()
        assert cfg.data_bytes >= sum(len(t[3]) for t in tensors)
        for (name, qt, n, k), (_, _, _, raw) in zip(mats, tensors):
            t = g.tensor(g.find(name))
            assert t.dev != 0 and t.dev % 16 == 0
            print("gguf tensor", name, S.TYPE_NAMES[qt], n, k, flush=True)
            x = S.make_activation(2, k, 50)
            w_copy = np.frombuffer(raw, dtype=np.uint8)
            y_copy = gpu.matmul_quant_batch(x, w_copy, qt, None, k, n, 2)
            # a numpy view of the mapping: its address lies in the registered data section
            view = np.ctypeslib.as_array((ctypes.c_uint8 * len(raw)).from_address(t.host))
            y_map = gpu.matmul_quant_batch(x, view, qt, None, k, n, 2)
            assert np.array_equal(bits(y_map), bits(y_copy)), name
            # the device address holds the file's bytes
            xd = _dev(x)
            y_dev = torch.empty((2, n), dtype=torch.float32, device="cuda")
            rc = gpu.load_library().cllm_hip_matmul_quant_dev(
                ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(t.dev), qt, None, k, n, 2,
                ctypes.c_void_p(y_dev.data_ptr()), gpu._stream())
            assert rc == 0, gpu.load_library().cllm_hip_last_error()
            assert np.array_equal(bits(y_dev.cpu().numpy()), bits(y_copy)), name


def test_mmap_weights_rewritten_or_remapped_are_copied_again(gpu, orc, tmp_path):
    """The engine's path: host weight pointers into a read-only private file mapping, nothing
    registered. The first call copies the mapping to the device; later calls reuse the copy
    while the mapping and file are unchanged, and copy again when the file is rewritten in
    place (same inode, pages the mapping shows change too) or another file is mapped at the
    same address. Every result against the oracle on the bytes the mapping shows."""
    import time
    from test_gpu_parity import check_close
    from test_capi_cpu import _libc, PROT_READ, MAP_PRIVATE, MAP_FIXED
    libc = _libc()
    qt, n, k = S.Q4_K, 256, 1024
    size = n * S.row_bytes(qt, k)
    assert size % 4096 == 0
    ws = [S.make_weight(qt, n, k, 600 + i) for i in range(3)]
    x = S.make_activation(1, k, 610)
    paths = [tmp_path / "a.bin", tmp_path / "b.bin"]
    paths[0].write_bytes(ws[0].tobytes())
    paths[1].write_bytes(ws[2].tobytes())

    def run_and_check(addr, w, what):
        view = np.ctypeslib.as_array((ctypes.c_uint8 * size).from_address(addr))
        assert np.array_equal(view, w), what  # what the reference would read
        print("mmap weights", what, flush=True)
        y = gpu.matmul_quant(x[0], view, qt, None, k, n)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, 1)
        check_close(y, orc.matmul(x, w, qt, None, k, n, 1), exact, abs_sum, what)
        return y

    fa = os.open(paths[0], os.O_RDONLY)
    fb = os.open(paths[1], os.O_RDONLY)
    addr = libc.mmap(None, size, PROT_READ, MAP_PRIVATE, fa, 0)
    try:
        y0 = run_and_check(addr, ws[0], "first copy")
        y0b = run_and_check(addr, ws[0], "copy reused")
        assert np.array_equal(bits(y0), bits(y0b))
        time.sleep(0.05)  # past the file system's timestamp granularity
        with open(paths[0], "r+b") as f:
            f.write(ws[1].tobytes())
        run_and_check(addr, ws[1], "file rewritten in place")
        assert libc.munmap(addr, size) == 0
        assert libc.mmap(addr, size, PROT_READ, MAP_PRIVATE | MAP_FIXED, fb, 0) == addr
        run_and_check(addr, ws[2], "other file at the same address")
    finally:
        libc.munmap(addr, size)
        os.close(fa)
        os.close(fb)
