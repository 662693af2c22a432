"""GPU parity of the float-dot kernels: the weight types without a vec_dot kernel (F32, F16,
Q4_1, Q5_1, Q8_1, Q2_K, Q3_K), which the reference computes by dequantizing each weight row
and dotting it with the unquantized fp32 activations (src/core/quant.cpp:1404-1430, and row
by row in matmul_quant_batch, 1471-1474).

Bars (the same as for the vec_dot types):
  - |gpu - ref| <= 1e-4 * max(|ref|, 2^-8 * A) against the reference's own fp32 output
    (golden vectors from the compiled reference), A = the row's sum of |x_i * w_i|, and
    |gpu - exact| <= max(1e-4 * max(|exact|, 2^-10 * A), 2 * |ref - exact|, R * A) against
    the fp64 sum of the same products, R = the reference's largest |ref - exact| / A over the
    same output;
  - host and device entry points, and a batch row and the same row alone, agree bit for bit.
"""
import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S
from test_gpu_parity import bits, check_close, _dev

pytestmark = pytest.mark.gpu

FD_TYPES = list(S.FLOAT_DOT_TYPES)


def _case(c):
    qt, n, k, m, seed = (int(v) for v in c["meta"])
    w = S.make_weight(qt, n, k, seed)
    x = S.make_activation(m, k, seed + 1, outliers=True)
    bias = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
    return qt, n, k, m, w, x, bias


def test_fdot_vs_reference_golden(gpu, orc):
    cases = split_cases(load_golden("fdot.npz"))
    assert {int(c["meta"][0]) for c in cases.values()} == set(FD_TYPES)
    for tag, c in cases.items():
        qt, n, k, m, w, x, bias = _case(c)
        print("fdot case", tag, "route", gpu.matmul_route(qt, k, n, m), flush=True)
        y = gpu.matmul_quant_batch(x, w, qt, None, k, n, m).reshape(m, n)
        yb = gpu.matmul_quant_batch(x, w, qt, bias, k, n, m).reshape(m, n)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        check_close(y, c["y"].reshape(m, n), exact, abs_sum, tag)
        exact_b, abs_b = orc.matmul_f64(x, w, qt, bias, k, n, m)
        check_close(yb, c["ybias"].reshape(m, n), exact_b, abs_b, tag + "+bias")
        # the device entry point computes the same bits as the host one
        yd = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, _dev(bias), k, n).cpu().numpy()
        assert np.array_equal(bits(yd), bits(yb)), tag


@pytest.mark.parametrize("qt", FD_TYPES)
def test_fdot_batch_rows_equal_single_rows(gpu, qt):
    # k = 4096 stages the activation rows in LDS, k = 18432 reads them from global memory
    for k, m in ((4096, 6), (18432, 3)):
        n = 75
        w = S.make_weight(qt, n, k, 31 + k)
        x = S.make_activation(m, k, 32 + k, outliers=True)
        print("fdot rows", S.TYPE_NAMES[qt], k, m, flush=True)
        yb = gpu.matmul_quant_batch(x, w, qt, None, k, n, m)
        for t in range(m):
            y1 = gpu.matmul_quant(x[t], w, qt, None, k, n)
            assert np.array_equal(bits(y1), bits(yb[t])), (S.TYPE_NAMES[qt], k, t)


@pytest.mark.parametrize("qt", FD_TYPES)
def test_fdot_edge_shapes(gpu, orc, qt):
    bs = S.BLOCK[qt]
    shapes = [(1, max(bs, 32), 1), (3, 256, 2), (9, 512, 7), (65, 768, 5), (200, 256, 64),
              (130, 14336, 1)]
    if bs == 1:  # rows whose length is not a multiple of 32
        shapes += [(5, 1, 1), (7, 31, 3), (64, 129, 2)]
    for (n, k, m) in shapes:
        if k % bs:
            continue
        print("fdot shape", S.TYPE_NAMES[qt], n, k, m, flush=True)
        w = S.make_weight(qt, n, k, n + k)
        x = S.make_activation(m, k, m + k, outliers=True)
        y = gpu.matmul_quant_batch(x, w, qt, None, k, n, m).reshape(m, n)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m).reshape(m, n)
        check_close(y, yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k} m{m}")


@pytest.mark.parametrize("qt", [S.Q4_1, S.Q5_1, S.Q8_1])
def test_fdot_pipelined_equals_per_row_kernel(gpu, orc, qt):
    """One activation row of the types whose dot is regrouped per block (A * sum x q + B *
    sum x): the pipelined kernel (each wave walks rows, the next row's loads in flight; knob
    gemv_fp_wgs 1-8 workgroups per CU) and the per-row kernel (9) make the same per-row
    additions, so they agree bit for bit, on grids from one workgroup per CU (many rows per
    wave) to more than the rows. The shapes cover short rows (lanes with no unit), one and
    two units per lane, rows past the pipelined kernel's reach (K = 8192: three or more units
    per lane, the per-row kernel whatever the knob) and rows past the grid's last wave."""
    import cllm_inference_amd as C
    for n, k in ((75, 256), (1000, 896), (333, 2048), (2500, 4096), (64, 8192)):
        if k % S.BLOCK[qt]:
            continue
        print("fdot pipelined", S.TYPE_NAMES[qt], n, k, flush=True)
        w = S.make_weight(qt, n, k, 5 * n + k)
        x = S.make_activation(1, k, n + 3, outliers=True)
        C.tune("gemv_fp_wgs", 9)
        ref = gpu.matmul_quant(x[0], w, qt, None, k, n)
        for knob in (1, 2, 3, 4, 8, 0):
            C.tune("gemv_fp_wgs", knob)
            y = gpu.matmul_quant(x[0], w, qt, None, k, n)
            assert np.array_equal(bits(y), bits(ref)), (S.TYPE_NAMES[qt], n, k, knob)
        C.tune("gemv_fp_wgs")
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, 1)
        yo = orc.matmul(x, w, qt, None, k, n, 1)
        check_close(ref[None], yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k}")


def test_fdot_output_head_sample_rows(gpu, orc):
    """An F16 output head of Qwen2.5-0.5B's shape (151936 x 896) on the device path; every
    1024th row is checked against the oracle (the rows are independent)."""
    import torch
    qt, n, k = S.F16, 151936, 896
    w = S.make_weight(qt, n, k, 77)
    x = S.make_activation(1, k, 78)
    y = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, None, k, n).cpu().numpy()[0]
    rows = np.arange(0, n, 1024)
    rb = S.row_bytes(qt, k)
    wsub = w.reshape(n, rb)[rows].reshape(-1)
    exact, abs_sum = orc.matmul_f64(x, wsub, qt, None, k, len(rows), 1)
    yo = orc.matmul(x, wsub, qt, None, k, len(rows), 1)
    check_close(y[rows][None], yo, exact, abs_sum, "F16 head")
    torch.cuda.synchronize()


def test_fdot_routes_and_errors(gpu):
    import torch
    for qt in FD_TYPES:
        assert gpu.matmul_route(qt, 4096, 4096, 1) == "fdot"
        assert gpu.matmul_route(qt, 4096, 4096, 512) == "fdot"
        assert not gpu.has_vec_dot(qt)
    w = S.make_weight(S.Q2_K, 4, 256, 1)
    q = gpu.quantize_row_q8_0(S.make_activation(1, 256, 2)[0])
    with pytest.raises(RuntimeError, match="vec_dot_row: no kernel for this type"):
        gpu.vec_dot_rows(w, S.Q2_K, q, 256, 4)
    with pytest.raises(RuntimeError, match="unsupported ggml type for dequantize"):
        gpu.matmul_quant(np.zeros(64, np.float32), np.zeros(4096, np.uint8), 5, None, 64, 4)
    x = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    wd = torch.zeros(4096 + 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="misaligned"):
        gpu.matmul_quant_dev(x, wd[2:], S.F16, None, 256, 4)
    with pytest.raises(RuntimeError, match="in_dim not divisible by block size"):
        gpu.matmul_quant_dev(x[:, :100].contiguous(), wd, S.Q3_K, None, 100, 4)


@pytest.mark.parametrize("qt", sorted(S.TYPE_NAMES))
def test_dequantize_rows_bit_exact(gpu, orc, qt):
    """The embedding lookup: rows dequantized on the device equal the reference's
    dequantize_block (through the oracle, bit-exact with it) bit for bit."""
    import torch
    bs = S.BLOCK[qt]
    for n, k in ((40, 4096 if bs > 1 else 896), (7, 256 if bs > 1 else 33)):
        if k % bs:
            continue
        w = S.make_weight(qt, n, k, 60 + qt)
        ids = np.array([n - 1, 0, 3, 3, n // 2], np.int32)
        got = gpu.dequantize_rows_dev(_dev(w), qt, k, _dev(ids)).cpu().numpy()
        rb = S.row_bytes(qt, k)
        for i, j in enumerate(ids):
            want = orc.dequantize(w[j * rb:(j + 1) * rb], qt, k)
            assert np.array_equal(bits(got[i]), bits(want)), (S.TYPE_NAMES[qt], n, k, j)
    torch.cuda.synchronize()
