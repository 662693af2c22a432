"""cllm_hip_matmul_quant_static_dev, the matmul entry point that allocates nothing: called
through the C ABI right after cllm_hip_init, it must leave the library's allocation count
unchanged, and its output must equal cllm_hip_matmul_quant_dev's bit for bit (the same kernels
on the same plan; only the scratch comes from the fixed per-GPU array), on two calls in a row
of each route, the second with a smaller input, so the second call runs on scratch the first
one left behind. A batch whose scratch exceeds the array is refused with an error, and so is a
call on a second stream while the first stream's call may still be running.
"""
import ctypes

import numpy as np
import pytest

import cllm_inference_amd as C
from cllm_inference_amd import synth as S

pytestmark = pytest.mark.gpu


def _static(lib, x, w, qt, bias, k, n, y):
    import torch
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return lib.cllm_hip_matmul_quant_static_dev(p(x), p(w), int(qt), p(bias), int(k), int(n),
                                                int(x.shape[0]), p(y), stream)


# (type, n, k, [m of the first call, m of the second]): the MFMA route with split K (the
# 4096 x 4096 Q4_K matrix at 512 rows plans two splits), then the small-batch route with split
# K (32 rows: two splits), Q6_K's kernel, a 32-element block type on the MFMA then the
# small-batch route, the small-batch route then the GEMV route with a quantized batch (3
# rows), the fused decode GEMV (1 row), and the streaming GEMV's whole-batch launch on a
# batch quantized first (8 rows) then quantized inside the launch (5 rows)
CASES = [
    (S.Q4_K, 4096, 4096, [512, 32]),
    (S.Q6_K, 1024, 4096, [256, 16]),
    (S.Q8_0, 768, 2048, [96, 32]),
    (S.Q5_K, 600, 1024, [12, 3]),
    (S.Q4_0, 512, 1024, [2, 1]),
    (S.Q8_0, 4096, 4096, [8, 5]),
]


@pytest.mark.parametrize("qt,n,k,ms", CASES, ids=[f"{S.TYPE_NAMES[c[0]]}-{c[1]}x{c[2]}" for c in CASES])
def test_static_scratch_matches_matmul_quant_dev(gpu, qt, n, k, ms):
    import torch
    lib = C.load_library()
    assert lib.cllm_hip_init(0) == 0
    w = torch.from_numpy(S.make_weight(qt, n, k, 300 + qt)).cuda()
    bias = torch.linspace(-1, 1, n, dtype=torch.float32, device="cuda")
    xs = [torch.from_numpy(S.make_activation(m, k, 40 + 7 * call + qt, outliers=True)).cuda()
          for call, m in enumerate(ms)]
    ys = [torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda") for m in ms]
    torch.cuda.synchronize()
    # the static calls first: nothing else has run on this stream in this test
    allocs = lib.cllm_hip_allocation_count()
    for x, y, m in zip(xs, ys, ms):
        print("static scratch", S.TYPE_NAMES[qt], n, k, "m", m, "plan", gpu.matmul_plan(qt, k, n, m),
              flush=True)
        rc = _static(lib, x, w, qt, bias, k, n, y)
        assert rc == 0, lib.cllm_hip_last_error().decode()
    torch.cuda.synchronize()
    assert lib.cllm_hip_allocation_count() == allocs
    for x, y, m in zip(xs, ys, ms):
        want = gpu.matmul_quant_dev(x, w, qt, bias, k, n)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32)), (S.TYPE_NAMES[qt], m)


def test_static_scratch_refuses_a_second_stream_while_in_use(gpu):
    """A call on stream B while stream A's call is still queued (behind a bounded spin kernel)
    fails with CLLM_HIP_E_BUSY and leaves A's result intact; once A is done, B's call runs."""
    import torch
    lib = C.load_library()
    assert lib.cllm_hip_init(0) == 0
    qt, n, k, m = S.Q4_K, 1024, 4096, 64
    w = torch.from_numpy(S.make_weight(qt, n, k, 77)).cuda()
    x = torch.from_numpy(S.make_activation(m, k, 78, outliers=True)).cuda()
    want = gpu.matmul_quant_dev(x, w, qt, None, k, n)
    ya = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    yb = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    # A's call waits behind a bounded spin; B's call must be refused if A's stream is still
    # busy once B's call has returned (then it was busy during B's check). Should the host
    # have been held until A finished (the spin too short), the premise does not hold: the
    # spin is lengthened and the pair tried again.
    for cycles in (50_000_000, 400_000_000, 2_000_000_000):
        with torch.cuda.stream(sa):
            torch.cuda._sleep(cycles)
            assert _static(lib, x, w, qt, None, k, n, ya) == 0, lib.cllm_hip_last_error().decode()
        with torch.cuda.stream(sb):
            rc = _static(lib, x, w, qt, None, k, n, yb)
        a_busy = not sa.query()
        print("busy check: spin", cycles, "rc", rc, "stream A still busy", a_busy, flush=True)
        if a_busy:
            break
        assert rc == 0, (rc, lib.cllm_hip_last_error().decode())
        torch.cuda.synchronize()
    assert a_busy, "stream A's call finished before B's call at every spin length"
    assert rc == 6, (rc, lib.cllm_hip_last_error().decode())  # CLLM_HIP_E_BUSY
    assert "another stream" in lib.cllm_hip_last_error().decode()
    # the same stream is ordered by the stream itself
    with torch.cuda.stream(sa):
        assert _static(lib, x, w, qt, None, k, n, ya) == 0, lib.cllm_hip_last_error().decode()
    sa.synchronize()
    with torch.cuda.stream(sb):
        assert _static(lib, x, w, qt, None, k, n, yb) == 0, lib.cllm_hip_last_error().decode()
    sb.synchronize()
    assert torch.equal(ya.view(torch.int32), want.view(torch.int32))
    assert torch.equal(yb.view(torch.int32), want.view(torch.int32))


def test_static_scratch_refuses_oversized_batches(gpu):
    import torch
    lib = C.load_library()
    cap = lib.cllm_hip_static_scratch_bytes()
    assert cap == 64 << 20
    k, n, m = 14336, 256, 2048  # ~106 MB of activation scratch
    w = torch.zeros(S.row_bytes(S.Q6_K, k) * n, dtype=torch.uint8, device="cuda")
    x = torch.zeros((m, k), dtype=torch.float32, device="cuda")
    y = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    rc = _static(lib, x, w, S.Q6_K, None, k, n, y)
    assert rc != 0
    assert "fixed buffer" in lib.cllm_hip_last_error().decode()
