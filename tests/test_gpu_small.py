"""The small-batch route (k_gemm_sm.hip: by default up to 32 or 64 activation rows of every
vec_dot type, from 5 to 9 rows depending on the type and on whether the GEMV streams the batch
in one launch; on int8 MFMA, the weights streamed once for the batch, the fp32 rows quantized
once first; the kernel takes 1 to 64) on an MI355X, through the C ABI.

Bars: the check_close bars of test_gpu_parity.py against the oracle (the reference's own
quant.cpp restated) and the fp64 evaluation of the same quantized terms; bit-identical results
between the fused-quantization and pre-quantized entry points (the fused staging quantizes
bit for bit as quantize_row_q8_0) and between repeated runs (every sum has a fixed order,
split-K included).
"""
import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S
from test_gpu_parity import bits, check_close, _dev

pytestmark = pytest.mark.gpu

SMALL_TYPES = [S.Q4_K, S.Q5_K, S.Q8_0]


def _run(gpu, w, x, qt, bias, k, n, m):
    """Fused and pre-quantized results of one batch (device entry points)."""
    import torch
    wd, xd = _dev(w), _dev(x)
    bd = None if bias is None else _dev(bias)
    y_fused = gpu.matmul_quant_dev(xd, wd, qt, bd, k, n).cpu().numpy()
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    y_q8 = gpu.gemv_q8_dev(wd, qt, k, n, qs, sc, bs, bd).cpu().numpy()
    torch.cuda.synchronize()
    return y_fused, y_q8


@pytest.fixture
def small_everywhere(gpu):
    """The small-batch kernel for every batch of 3 to 64 rows (its default range is narrower)."""
    gpu.tune("gemm_small", 1)
    yield
    gpu.tune("gemm_small")


@pytest.mark.parametrize("qt", SMALL_TYPES + [S.Q4_0, S.Q5_0])
def test_small_batches_ragged_shapes_vs_oracle(gpu, orc, qt, small_everywhere):
    """Batch sizes that leave token tiles part-empty (5, 17, 33, 63), row counts that leave a
    row group part-empty, K that splits over workgroups (K = 4096 takes four splits; K = 2816
    is 11 super-blocks, an uneven split), with and without a bias."""
    for (n, k, m) in [(100, 256, 5), (130, 1024, 17), (333, 2816, 33), (77, 4096, 63),
                      (512, 4096, 64), (16, 512, 4)]:
        w = S.make_weight(qt, n, k, 900 + n + m)
        x = S.make_activation(m, k, 901 + m, outliers=True)
        bias = np.random.default_rng(n + m).standard_normal(n).astype(np.float32)
        print("small", S.TYPE_NAMES[qt], n, k, m, gpu.matmul_plan(qt, k, n, m), flush=True)
        assert gpu.matmul_route(qt, k, n, m) == "small"
        for b in (None, bias):
            y_fused, y_q8 = _run(gpu, w, x, qt, b, k, n, m)
            assert np.array_equal(bits(y_fused), bits(y_q8)), (S.TYPE_NAMES[qt], n, k, m)
            exact, abs_sum = orc.matmul_f64(x, w, qt, b, k, n, m)
            yo = orc.matmul(x, w, qt, b, k, n, m)
            check_close(y_fused.reshape(m, n), yo.reshape(m, n), exact, abs_sum,
                        f"small {S.TYPE_NAMES[qt]} {n}x{k} m{m}")


@pytest.mark.parametrize("label,m", [("q5_k", 16), ("q5_k", 64), ("q8_0", 16), ("q8_0", 64)])
def test_m_sweep_full_size_vs_reference_golden(gpu, orc, label, m):
    """The c4 workloads at full size (Q5_K 14336x4096, Q8_0 4096x4096) on the small-batch
    kernel (Q5_K at 64 rows forced onto it, past its default range): the golden rows from the
    compiled reference, sampled rows against the oracle, and two runs bit for bit."""
    qt, n, k, w = S.config_weight("c4_m_sweep", label)
    x = S.config_activation("c4_m_sweep", m, k)
    try:
        gpu.tune("gemm_small", 1)
        plan = gpu.matmul_plan(qt, k, n, m)
        print("c4 full", label, m, plan, flush=True)
        assert plan.startswith("k_gemm_sm<")
        _check_full_size(gpu, orc, label, m, qt, n, k, w, x)
    finally:
        gpu.tune("gemm_small")


def _check_full_size(gpu, orc, label, m, qt, n, k, w, x):
    y1, y_q8 = _run(gpu, w, x, qt, None, k, n, m)
    y2, _ = _run(gpu, w, x, qt, None, k, n, m)
    assert np.array_equal(bits(y1), bits(y2))
    assert np.array_equal(bits(y1), bits(y_q8))
    y1 = y1.reshape(m, n)
    c = split_cases(load_golden("batch.npz"))[f"c4_{label}_m{m}"]
    rb = S.row_bytes(qt, k)
    wsub = w[: 512 * rb]
    exact, abs_sum = orc.matmul_f64(x, wsub, qt, None, k, 512, m)
    check_close(y1[:, :512], c["y"], exact, abs_sum, f"c4 {label} m{m} golden")
    rows = np.arange(3, n, 517)
    sub = w.reshape(n, rb)[rows].reshape(-1)
    exact, abs_sum = orc.matmul_f64(x, sub, qt, None, k, len(rows), m)
    yo = orc.matmul(x, sub, qt, None, k, len(rows), m).reshape(m, len(rows))
    check_close(y1[:, rows], yo, exact, abs_sum, f"c4 {label} m{m} oracle rows")


def test_long_k_splits_and_knobs(gpu, orc):
    """K = 14336 (56 super-blocks: fourteen splits), the knob that takes 3-row batches
    onto the small route and the one that turns it off (the GEMV then computes the same
    terms: within the bars of each other)."""
    qt, n, k = S.Q4_K, 272, 14336
    w = S.make_weight(qt, n, k, 4242)
    for m in (3, 32):
        x = S.make_activation(m, k, 4243 + m, outliers=True)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m).reshape(m, n)
        try:
            gpu.tune("gemm_small", 1)
            assert gpu.matmul_route(qt, k, n, m) == "small"
            print("long k", m, gpu.matmul_plan(qt, k, n, m), flush=True)
            y_small = gpu.matmul_quant_batch(x, w, qt, None, k, n, m).reshape(m, n)
            gpu.tune("gemm_small", 2)
            assert gpu.matmul_route(qt, k, n, m) != "small"
            y_other = gpu.matmul_quant_batch(x, w, qt, None, k, n, m).reshape(m, n)
        finally:
            gpu.tune("gemm_small")
        check_close(y_small, yo, exact, abs_sum, f"small m{m}")
        check_close(y_other, yo, exact, abs_sum, f"other m{m}")


def test_residual_add_on_small_route(gpu, orc):
    """matmul_quant_residual_dev on a small batch: y += x W^T (+ bias), as matmul then add."""
    import torch
    qt, n, k, m = S.Q5_K, 200, 1024, 8
    w = S.make_weight(qt, n, k, 77)
    x = S.make_activation(m, k, 78)
    bias = np.random.default_rng(79).standard_normal(n).astype(np.float32)
    base = np.random.default_rng(80).standard_normal((m, n)).astype(np.float32)
    assert gpu.matmul_route(qt, k, n, m) == "small"
    wd, xd, bd = _dev(w), _dev(x), _dev(bias)
    y = _dev(base)
    gpu.matmul_quant_residual_dev(xd, wd, qt, bd, k, n, y)
    ref = gpu.matmul_quant_dev(xd, wd, qt, bd, k, n).cpu().numpy()
    torch.cuda.synchronize()
    assert np.array_equal(bits(y.cpu().numpy()), bits((base + ref).astype(np.float32)))


@pytest.mark.parametrize("qt", SMALL_TYPES)
def test_in_kernel_quantization_equals_quantized_once(gpu, orc, qt):
    """The small-batch kernel's in-kernel quantization form (every workgroup quantizes the fp32
    rows of its K range, bit for bit as quantize_row_q8_0) against the default form (the batch
    quantized once, then the same kernel plan): equal bit for bit, and against the oracle."""
    for (n, k, m, splits) in [(300, 4096, 16, 4), (77, 2816, 33, 3), (130, 1024, 5, 1),
                              (64, 2048, 64, 2)]:
        w = S.make_weight(qt, n, k, 60 + n + m)
        x = S.make_activation(m, k, 61 + m, outliers=True)
        wd, xd = _dev(w), _dev(x)
        ys, plans = [], []
        try:
            gpu.tune("gemm_small", 1)
            gpu.tune("gemm_small_plan", splits, 0)
            for form in (1, 2):
                gpu.tune("gemm_small_q8", form)
                plans.append(gpu.matmul_plan(qt, k, n, m))
                ys.append(gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy())
        finally:
            for knob in ("gemm_small_q8", "gemm_small_plan", "gemm_small"):
                gpu.tune(knob)
        print("in-kernel quantization", S.TYPE_NAMES[qt], n, k, m, plans, flush=True)
        assert plans[0] == plans[1], plans
        assert np.array_equal(bits(ys[0]), bits(ys[1])), (S.TYPE_NAMES[qt], n, k, m)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m)
        check_close(ys[1].reshape(m, n), yo.reshape(m, n), exact, abs_sum,
                    f"in-kernel {S.TYPE_NAMES[qt]} {n}x{k} m{m}")


@pytest.mark.parametrize("k, n, m", [(14336, 4096, 8), (14336, 4096, 5), (4096, 14336, 16),
                                     (4096, 14336, 6), (4096, 1024, 13), (2048, 333, 9)])
def test_q6_k_small_batches_default_route_vs_oracle(gpu, orc, k, n, m):
    """Q6_K on the small-batch kernel (the batch quantized once, int8 MFMA, the two 16-element
    scales of a block on two MFMAs over its halves): the default route of these shapes, every
    output against the oracle with and without a bias, the fused and pre-quantized entry
    points bit for bit, two runs bit for bit."""
    qt = S.Q6_K
    assert gpu.matmul_route(qt, k, n, m) == "small"
    w = S.make_weight(qt, n, k, 40 + m + n)
    x = S.make_activation(m, k, 41 + m, outliers=True)
    bias = np.random.default_rng(n + m).standard_normal(n).astype(np.float32)
    print("q6_k small", n, k, m, gpu.matmul_plan(qt, k, n, m), flush=True)
    for b in (None, bias):
        y_fused, y_q8 = _run(gpu, w, x, qt, b, k, n, m)
        y2, _ = _run(gpu, w, x, qt, b, k, n, m)
        assert np.array_equal(bits(y_fused), bits(y_q8))
        assert np.array_equal(bits(y_fused), bits(y2))
        exact, abs_sum = orc.matmul_f64(x, w, qt, b, k, n, m)
        yo = orc.matmul(x, w, qt, b, k, n, m, threads=8)
        check_close(y_fused.reshape(m, n), yo.reshape(m, n), exact, abs_sum,
                    f"q6_k small {n}x{k} m{m}")


@pytest.mark.parametrize("qt, k, n, m", [(S.Q4_0, 4096, 14336, 12), (S.Q5_0, 4096, 14336, 16),
                                         (S.Q4_0, 4096, 4096, 64), (S.Q5_0, 14336, 4096, 9)])
def test_q4_0_q5_0_small_batches_default_route_vs_oracle(gpu, orc, qt, k, n, m):
    """Q4_0 / Q5_0 on the small-batch kernel (the batch quantized once; q - 8 and q - 16 formed
    per byte as int8, Q5_0's fifth bits spread from its qh word): the default route of these
    full-size shapes, every output against the oracle with and without a bias, the fp32 and
    quantized-batch entry points bit for bit."""
    assert gpu.matmul_route(qt, k, n, m) == "small"
    w = S.make_weight(qt, n, k, 80 + m + n)
    x = S.make_activation(m, k, 81 + m, outliers=True)
    bias = np.random.default_rng(n + m).standard_normal(n).astype(np.float32)
    print("b32 small", S.TYPE_NAMES[qt], n, k, m, gpu.matmul_plan(qt, k, n, m), flush=True)
    for b in (None, bias):
        y_fused, y_q8 = _run(gpu, w, x, qt, b, k, n, m)
        assert np.array_equal(bits(y_fused), bits(y_q8))
        exact, abs_sum = orc.matmul_f64(x, w, qt, b, k, n, m)
        yo = orc.matmul(x, w, qt, b, k, n, m, threads=8)
        check_close(y_fused.reshape(m, n), yo.reshape(m, n), exact, abs_sum,
                    f"{S.TYPE_NAMES[qt]} small {n}x{k} m{m}")


def test_q6_k_small_kernel_tiles_and_splits(gpu, orc):
    """The Q6_K small-batch kernel forced onto ragged batches of 1 to 4 token tiles, and onto
    K splits and K parts the plan does not take, against the oracle."""
    qt, k = S.Q6_K, 4096
    for n, m, plan in [(77, 17, None), (130, 33, None), (64, 64, None), (100, 3, None),
                       (300, 12, (4, 2)), (300, 12, (2, 8)), (300, 40, (8, 1))]:
        w = S.make_weight(qt, n, k, 50 + n + m)
        x = S.make_activation(m, k, 51 + m, outliers=True)
        try:
            gpu.tune("gemm_small", 1)
            if plan:
                gpu.tune("gemm_small_plan", *plan)
            print("q6_k small forced", n, k, m, gpu.matmul_plan(qt, k, n, m), flush=True)
            assert gpu.matmul_route(qt, k, n, m) == "small"
            y_fused, y_q8 = _run(gpu, w, x, qt, None, k, n, m)
        finally:
            gpu.tune("gemm_small_plan")
            gpu.tune("gemm_small")
        assert np.array_equal(bits(y_fused), bits(y_q8))
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m)
        check_close(y_fused.reshape(m, n), yo.reshape(m, n), exact, abs_sum,
                    f"q6_k forced {n} m{m} plan {plan}")
