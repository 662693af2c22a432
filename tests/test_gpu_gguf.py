"""GGUF upload on the GPU: the data section copied once to the device, host tensor
pointers into the mapping resolving to that copy in the Quant API calls, and the device
addresses cllm_hip_gguf_tensor reports holding the file's bytes."""
import ctypes

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
