"""Every point of the M-sweep workload at full size, on the route and kernel plan that the
default library picks (the plan bench.py times and prints), on an MI355X:
Q5_K 14336x4096 and Q8_0 4096x4096 at M = 1, 4, 16, 64, 256.

Bars: check_close (test_gpu_parity.py) of every output of up to three activation rows against
the compiled reference's rows (tests/golden/batch_large.npz) and of every output of eight more
rows against the oracle; the fused entry point (quantization inside the launch) equal bit for
bit to a second call.
"""
import hashlib

import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S
from test_gpu_parity import bits, check_close, _dev

pytestmark = pytest.mark.gpu

# the default plan of each point (cllm_hip_matmul_plan), as bench.py reports it
PLANS = {
    ("q5_k", 1): "k_gemv_str<Q5_K,1> launches=1",
    ("q5_k", 4): "k_gemv_str<Q5_K,4> launches=1",
    ("q5_k", 16): "k_gemm_sm<Q5_K,1> splits=1 kp=4",
    ("q5_k", 64): "k_gemmw_q4k<4,1,2,Q5_K> splits=4",
    ("q5_k", 256): "k_gemmw_q4k<4,1,2,Q5_K> splits=1",
    ("q8_0", 1): "k_gemv_str<Q8_0,1> launches=1",
    ("q8_0", 4): "k_gemv_str<Q8_0,4> launches=1",
    ("q8_0", 16): "k_gemm_sm<Q8_0,1> splits=1 kp=16",
    ("q8_0", 64): "k_gemm_sm<Q8_0,4> splits=4 kp=4",
    ("q8_0", 256): "k_gemmw_b32<Q8_0,4,2> splits=4",
}


@pytest.mark.parametrize("label,m", sorted(PLANS))
def test_m_sweep_point_default_plan_full_size(gpu, orc, label, m):
    import torch
    c = split_cases(load_golden("batch_large.npz"))
    qt, n, k, w = S.config_weight("c4_m_sweep", label)
    assert hashlib.sha256(w.tobytes()).hexdigest() == str(c[label]["w_sha"])
    x = S.config_activation("c4_m_sweep", m, k)
    g = c[f"{label}_m{m}"]
    assert hashlib.sha256(x.tobytes()).hexdigest() == str(g["x_sha"])
    plan = gpu.matmul_plan(qt, k, n, m)
    print("m sweep full size", label, n, k, m, plan, flush=True)
    assert plan == PLANS[(label, m)], plan
    wd, xd = _dev(w), _dev(x)
    y1 = gpu.matmul_quant_dev(xd, wd, qt, None, k, n)
    y2 = gpu.matmul_quant_dev(xd, wd, qt, None, k, n)
    torch.cuda.synchronize()
    y1, y2 = y1.cpu().numpy().reshape(m, n), y2.cpu().numpy().reshape(m, n)
    assert np.array_equal(bits(y1), bits(y2))
    rows = g["rows"]
    exact, abs_sum = orc.matmul_f64(x[rows], w, qt, None, k, n, len(rows))
    check_close(y1[rows], g["y"], exact, abs_sum, f"{label} m{m} golden rows")
    if m > 8:
        sample = np.sort(np.random.default_rng(m + n).choice(m, size=8, replace=False))
        yo = orc.matmul(x[sample], w, qt, None, k, n, 8, threads=8)
        exact, abs_sum = orc.matmul_f64(x[sample], w, qt, None, k, n, 8)
        check_close(y1[sample], yo, exact, abs_sum, f"{label} m{m} oracle rows")
