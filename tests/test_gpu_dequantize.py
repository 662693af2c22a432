"""dequantize_block and dequantize_block_f16 on an MI355X (cllm_hip_dequantize_block[_f16]),
bit for bit against the compiled reference (tests/golden/deq.npz: src/core/quant.cpp:371-412)
and against the oracle: thirteen types, n at a block boundary and inside the last block, all
65536 binary16 encodings (NaN payloads included), the special values of float_to_half, and
sources in host memory, in device memory, at an address that is not 16-byte aligned, and in
a run long enough to take several passes through the device staging."""
import hashlib

import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S

pytestmark = pytest.mark.gpu

CASES = split_cases(load_golden("deq.npz"))


def _source(tag, c):
    if "meta" in c:
        qt, n, nb, seed = (int(v) for v in c["meta"])
        w = S.make_weight(qt, 1, nb * S.BLOCK[qt], seed)
        assert hashlib.sha256(w.tobytes()).hexdigest() == str(c["w_sha"]), tag
        return w, qt, n
    t = S.F16 if tag.startswith("f16") else S.F32
    return np.ascontiguousarray(c["src"]).view(np.uint8), t, c["src"].size


@pytest.mark.parametrize("tag", sorted(CASES))
def test_dequantize_block_matches_reference(gpu, tag):
    c = CASES[tag]
    src, t, n = _source(tag, c)
    print("dequantize_block", tag, n, flush=True)
    y = gpu.dequantize_block(src, t, n)
    assert np.array_equal(y.view(np.uint32), c["y"].view(np.uint32)), tag
    y16 = gpu.dequantize_block_f16(src, t, n)
    assert np.array_equal(y16, c["y16"]), tag


def test_dequantize_block_device_and_misaligned_sources(gpu, orc):
    import torch
    for qt in sorted(S.TYPE_NAMES):
        bs = S.BLOCK[qt]
        k = 8 * max(bs, 32)
        w = S.make_weight(qt, 3, k, 500 + qt)
        n = 3 * k - (5 if bs > 1 else 3)
        want = orc.dequantize_block(w, qt, n)
        want16 = orc.dequantize_block_f16(w, qt, n)
        print("sources", S.TYPE_NAMES[qt], n, flush=True)
        # device memory, aligned
        wd = torch.from_numpy(w).cuda()
        assert np.array_equal(gpu.dequantize_block(wd, qt, n).view(np.uint32), want.view(np.uint32))
        # host and device memory two bytes into a buffer (the blocks keep their layout)
        pad = np.zeros(w.size + 16, np.uint8)
        pad[2:2 + w.size] = w
        host_addr = pad.ctypes.data + 2
        assert np.array_equal(gpu.dequantize_block(host_addr, qt, n).view(np.uint32), want.view(np.uint32))
        padd = torch.from_numpy(pad).cuda()
        dev_addr = padd.data_ptr() + 2
        torch.cuda.synchronize()
        assert np.array_equal(gpu.dequantize_block(dev_addr, qt, n).view(np.uint32), want.view(np.uint32))
        assert np.array_equal(gpu.dequantize_block_f16(dev_addr, qt, n), want16)


def test_dequantize_block_long_run(gpu, orc):
    """2^26 + 1040 Q4_0 elements: two passes of the device staging, the second one partial."""
    qt = S.Q4_0
    n = (1 << 26) + 1040
    nb = (n + 31) // 32
    w = S.make_weight(qt, 1, nb * 32, 77)
    print("long run", n, flush=True)
    y = gpu.dequantize_block(w, qt, n)
    want = orc.dequantize_block(w, qt, n)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_dequantize_block_errors(gpu):
    with pytest.raises(RuntimeError, match="unsupported ggml type for dequantize"):
        gpu.dequantize_block(np.zeros(64, np.uint8), 4, 32)
    assert gpu.dequantize_block(np.zeros(64, np.uint8), S.Q8_0, 0).size == 0
