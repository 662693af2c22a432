"""Parity of the MFMA prefill path (matmul_quant_batch with n_rows >= 16) on an MI355X, for
both kernels: int8 MFMA with an fp32 per-block epilogue, and fp16 MFMA as an exact integer
engine.

Same bars as the GEMV tests (check_close in test_gpu_parity.py): |gpu - ref| <=
1e-4 * max(|ref|, 2^-8 * A) against the reference's fp32 output, and no further from the fp64
evaluation of the same quantized terms than max(1e-4 * max(|exact|, 2^-10 * A),
2 * |ref - exact|, R * A) (A = sum of absolute per-block terms, R = the reference's largest
|ref - exact| / A over the same output).
"""
import os

import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S
from test_gpu_parity import check_close, _dev, TYPES

pytestmark = pytest.mark.gpu


KERNELS = {"default": 0, "int8": 1, "f16": 2}


@pytest.fixture(params=list(KERNELS), autouse=True)
def gemm_kernel(request, gpu):
    """Every test runs on each MFMA kernel choice: the default (weight-row fp16 kernel
    k_gemmw.hip where it has the type, else int8), int8 (k_gemm.hip) and activation-row fp16
    (k_gemm16.hip), chosen through the library's tuning knob."""
    gpu.tune("gemm_kernel", KERNELS[request.param])
    yield request.param
    gpu.tune("gemm_kernel")


def test_prefill_layer_slices_vs_reference_golden(gpu, orc):
    """Q4_K_M layer (wq wk wv wo gate up: Q4_K, down: Q6_K): first 16 activation rows against
    the first 512 rows of every matrix."""
    cases = split_cases(load_golden("batch.npz"))
    for label, qt, n, k in S.CONFIGS["c3_q4_k_m_layer"]["mats"]:
        c = cases[label]
        rows = int(c["meta"][4])
        _, _, _, w = S.config_weight("c3_q4_k_m_layer", label)
        x = S.config_activation("c3_q4_k_m_layer", 512, k)[:16]
        wsub = w[: rows * S.row_bytes(qt, k)]
        assert gpu.matmul_route(qt, k, rows, 16) in ("mfma", "small")
        print("prefill slice", label, S.TYPE_NAMES[qt], rows, k, flush=True)
        y = gpu.matmul_quant_batch(x, wsub, qt, None, k, rows, 16)
        exact, abs_sum = orc.matmul_f64(x, wsub, qt, None, k, rows, 16)
        check_close(y, c["y"], exact, abs_sum, label)


@pytest.mark.parametrize("label", ["q5_k", "q8_0"])
@pytest.mark.parametrize("m", [16, 64])
def test_m_sweep_batches_vs_reference_golden(gpu, orc, label, m):
    c = split_cases(load_golden("batch.npz"))[f"c4_{label}_m{m}"]
    qt, n, k, w = S.config_weight("c4_m_sweep", label)
    x = S.config_activation("c4_m_sweep", m, k)
    wsub = w[: 512 * S.row_bytes(qt, k)]
    print("m sweep", label, m, flush=True)
    y = gpu.matmul_quant_batch(x, wsub, qt, None, k, 512, m)
    exact, abs_sum = orc.matmul_f64(x, wsub, qt, None, k, 512, m)
    check_close(y, c["y"], exact, abs_sum, f"{label} m{m}")


@pytest.mark.parametrize("qt", TYPES)
def test_mfma_matches_gemv_and_oracle(gpu, orc, qt, gemm_kernel):
    """Same rows through the MFMA kernel (16 rows at once) and the GEMV kernel (8 + 8); with
    the default kernel choice, every type but Q6_K (whose rows here are not a multiple of 2048
    elements) takes the small-batch kernel for both."""
    import torch
    k, n, m = 1024, 300, 16
    w = S.make_weight(qt, n, k, 70 + qt)
    x = S.make_activation(m, k, 71 + qt, outliers=True)
    wd, xd = _dev(w), _dev(x)
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    y_mfma = gpu.gemv_q8_dev(wd, qt, k, n, qs, sc, bs)  # 16 rows -> MFMA route
    y_gemv = torch.cat([gpu.gemv_q8_dev(wd, qt, k, n, qs[i:i + 8], sc[i:i + 8], bs[i:i + 8])
                        for i in (0, 8)])
    small = gemm_kernel == "default" and qt != S.Q6_K
    assert gpu.matmul_route(qt, k, n, 8) == ("small" if small else "gemv")
    assert gpu.matmul_route(qt, k, n, 16) == ("small" if small else "mfma")
    exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
    yo = orc.matmul(x, w, qt, None, k, n, m)
    check_close(y_mfma.cpu().numpy(), yo, exact, abs_sum, "mfma " + S.TYPE_NAMES[qt])
    check_close(y_gemv.cpu().numpy(), yo, exact, abs_sum, "gemv " + S.TYPE_NAMES[qt])


@pytest.mark.parametrize("qt", TYPES)
def test_mfma_partial_tiles_and_bias(gpu, orc, qt):
    for (n, k, m) in [(1, 256, 16), (130, 512, 17), (129, 256, 65), (64, 2048, 100)]:
        w = S.make_weight(qt, n, k, n * 3 + m)
        x = S.make_activation(m, k, n + m, outliers=True)
        bias = np.random.default_rng(n).standard_normal(n).astype(np.float32)
        print("mfma tile case", S.TYPE_NAMES[qt], n, k, m, flush=True)
        y = gpu.matmul_quant_batch(x, w, qt, bias, k, n, m)
        exact, abs_sum = orc.matmul_f64(x, w, qt, bias, k, n, m)
        yo = orc.matmul(x, w, qt, bias, k, n, m)
        check_close(y, yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k} m{m}")


@pytest.mark.parametrize("qt, k, n, m", [(S.Q6_K, 4096, 14336, 7), (S.Q6_K, 4096, 14336, 13),
                                         (S.Q6_K, 14336, 4096, 5), (S.Q4_0, 4096, 14336, 8),
                                         (S.Q5_0, 4096, 4096, 15), (S.Q6_K, 4096, 1024, 15)])
def test_mid_batches_on_weight_row_kernel(gpu, orc, qt, k, n, m, gemm_kernel):
    """Batches below 16 rows on the weight-row kernel (one partly filled 16-row tile) on
    full-size matrices, every output against the oracle: the route Q4_0 / Q5_0 / Q6_K take
    there with the streaming GEMV (which takes up to 8 rows in one launch) and the small-batch
    kernel switched off."""
    if gemm_kernel != "default":
        pytest.skip("the default route only")
    w = S.make_weight(qt, n, k, 11 + m)
    x = S.make_activation(m, k, 12 + m, outliers=True)
    try:
        gpu.tune("gemv_kernel", 1)
        gpu.tune("gemm_small", 2)
        assert gpu.matmul_route(qt, k, n, m) == "mfma"
        print("mid batch", S.TYPE_NAMES[qt], n, k, m, gpu.matmul_plan(qt, k, n, m), flush=True)
        y = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, None, k, n).cpu().numpy()
    finally:
        gpu.tune("gemm_small")
        gpu.tune("gemv_kernel")
    yo = orc.matmul(x, w, qt, None, k, n, m, threads=8)
    exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
    check_close(y, yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k} m{m}")


def _oracle_f64_rows(orc, x, w, qt, k, n):
    """The oracle's fp64 evaluation and absolute-term sums of every row of x, computed in row
    chunks on a thread pool (the oracle's calls release the interpreter lock)."""
    from concurrent.futures import ThreadPoolExecutor
    m = x.shape[0]
    chunks = [(i, min(i + 16, m)) for i in range(0, m, 16)]
    workers = max(1, min(16, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        parts = list(ex.map(lambda ab: orc.matmul_f64(x[ab[0]:ab[1]], w, qt, None, k, n, ab[1] - ab[0]),
                            chunks))
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])


@pytest.mark.parametrize("label", [mat[0] for mat in S.CONFIGS["c3_q4_k_m_layer"]["mats"]])
def test_full_prefill_layer_every_row_vs_oracle(gpu, orc, label):
    """M = 512 through each matrix of the layer at full size on its default plan: every output
    of all 512 activation rows against the oracle, to check_close's bars."""
    import torch
    qt, n, k, w = S.config_weight("c3_q4_k_m_layer", label)
    x = S.config_activation("c3_q4_k_m_layer", 512, k)
    print("full layer", label, n, k, gpu.matmul_plan(qt, k, n, 512), flush=True)
    wd, xd = _dev(w), _dev(x)
    y = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
    torch.cuda.synchronize()
    del wd, xd
    torch.cuda.empty_cache()
    yo = orc.matmul(x, w, qt, None, k, n, 512, threads=max(1, min(16, os.cpu_count() or 1)))
    exact, abs_sum = _oracle_f64_rows(orc, x, w, qt, k, n)
    check_close(y, yo, exact, abs_sum, f"{label} all 512 rows")


@pytest.mark.parametrize("splits", [None, 4])
@pytest.mark.parametrize("qt", TYPES)
def test_mfma_tails_and_split_k(gpu, orc, qt, splits, gemm_kernel):
    """Output rows and activation rows that end inside a tile (n = 520, m = 80), K = 2048, with
    the planned K split and with K forced into 4 splits (partial sums plus the reduction)."""
    k, n, m = 2048, 520, 80
    w = S.make_weight(qt, n, k, 90 + qt)
    x = S.make_activation(m, k, 91 + qt, outliers=True)
    bias = np.linspace(-1.0, 1.0, n).astype(np.float32)
    print("tails", S.TYPE_NAMES[qt], "splits", splits, flush=True)
    try:
        gpu.tune("gemm_splits", splits or 0)
        y = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, _dev(bias), k, n).cpu().numpy()
    finally:
        gpu.tune("gemm_splits")
    exact, abs_sum = orc.matmul_f64(x, w, qt, bias, k, n, m)
    yo = orc.matmul(x, w, qt, bias, k, n, m)
    check_close(y, yo, exact, abs_sum, f"tails {S.TYPE_NAMES[qt]} splits={splits}")


@pytest.mark.parametrize("m", [256, 512])
def test_m_sweep_q5_k_large_batches_vs_reference_golden(gpu, orc, m, gemm_kernel):
    """The M-sweep's Q5_K 14336x4096 matrix at full size with M = 256 (the plan the bench
    times there) and M = 512 (the largest weight-row tile): every output of three activation
    rows against the reference's (tests/golden/batch_large.npz), eight rows against the oracle,
    and the plan the batch ran named."""
    import hashlib
    import torch
    if gemm_kernel != "default":
        pytest.skip("the default plan's large tiles are the point here")
    c = split_cases(load_golden("batch_large.npz"))
    qt, n, k, w = S.config_weight("c4_m_sweep", "q5_k")
    assert hashlib.sha256(w.tobytes()).hexdigest() == str(c["q5_k"]["w_sha"])
    x = S.config_activation("c4_m_sweep", m, k)
    plan = gpu.matmul_plan(qt, k, n, m)
    print("q5_k 14336x4096 m", m, "plan", plan, flush=True)
    assert plan.startswith("k_gemmw_q4k<4,1,2,Q5_K>" if m == 256 else "k_gemmw_q4k<8,1,4,Q5_K>"), plan
    y = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, None, k, n)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    g = c[f"q5_k_m{m}"]
    rows = g["rows"]
    exact, abs_sum = orc.matmul_f64(x[rows], w, qt, None, k, n, len(rows))
    check_close(y[rows], g["y"], exact, abs_sum, f"q5_k m{m} golden rows")
    sample = np.sort(np.random.default_rng(m).choice(m, size=8, replace=False))
    yo = orc.matmul(x[sample], w, qt, None, k, n, 8, threads=8)
    exact, abs_sum = orc.matmul_f64(x[sample], w, qt, None, k, n, 8)
    check_close(y[sample], yo, exact, abs_sum, f"q5_k m{m} oracle rows")


@pytest.mark.parametrize("k, n", [(768, 77), (1280, 130), (3328, 33)])
def test_q6_k_prefill_super_block_alignments(gpu, orc, k, n, gemm_kernel):
    """Q6_K rows of an odd number of 210-byte super-blocks: the super-blocks sit at byte offsets
    0 and 2 mod 4 by row and by position, so the weight-row kernel realigns its dword loads
    both ways, and (n odd) the matrix ends 2 bytes past a dword boundary, where the last
    super-block's loads must stop. Planned split and 4 splits."""
    m = 40
    w = S.make_weight(S.Q6_K, n, k, k + n)
    x = S.make_activation(m, k, k - n, outliers=True)
    exact, abs_sum = orc.matmul_f64(x, w, S.Q6_K, None, k, n, m)
    yo = orc.matmul(x, w, S.Q6_K, None, k, n, m)
    for splits in (0, 4):
        print("q6_k alignments", k, n, "splits", splits, flush=True)
        try:
            gpu.tune("gemm_splits", splits)
            y = gpu.matmul_quant_dev(_dev(x), _dev(w), S.Q6_K, None, k, n).cpu().numpy()
        finally:
            gpu.tune("gemm_splits")
        check_close(y, yo, exact, abs_sum, f"q6_k {n}x{k} splits={splits}")


@pytest.mark.parametrize("shape", [(4, 1, 1), (4, 1, 2), (4, 1, 4), (8, 1, 2)])
def test_q6_k_tile_shapes(gpu, orc, shape, gemm_kernel):
    """Every compiled Q6_K weight-row tile shape (the plan's 128 x 32 and 128 x 64, and the
    tuning override's others) on ragged batches, against the oracle."""
    if gemm_kernel != "default":
        pytest.skip("tile shapes of the default kernel")
    k, n = 1024, 300
    for m in (16, 40, 100):
        w = S.make_weight(S.Q6_K, n, k, 5 + m)
        x = S.make_activation(m, k, 6 + m, outliers=True)
        exact, abs_sum = orc.matmul_f64(x, w, S.Q6_K, None, k, n, m)
        yo = orc.matmul(x, w, S.Q6_K, None, k, n, m)
        try:
            gpu.tune("gemm_tiles", *shape)
            print("q6_k shape", shape, "m", m, gpu.matmul_plan(S.Q6_K, k, n, m), flush=True)
            y = gpu.matmul_quant_dev(_dev(x), _dev(w), S.Q6_K, None, k, n).cpu().numpy()
        finally:
            gpu.tune("gemm_tiles")
        check_close(y, yo, exact, abs_sum, f"q6_k {shape} m{m}")


K_QUANT_SHAPES = [(S.Q4_K, sh) for sh in [(8, 1, 4), (8, 1, 2), (8, 2, 2), (4, 2, 4), (4, 2, 2),
                                          (4, 1, 2), (4, 1, 1)]] + \
                 [(S.Q5_K, sh) for sh in [(8, 1, 4), (8, 1, 2), (4, 1, 2), (4, 1, 1)]]


@pytest.mark.parametrize("qt, shape", K_QUANT_SHAPES)
def test_k_quant_tile_shapes(gpu, orc, qt, shape, gemm_kernel):
    """Every compiled Q4_K / Q5_K weight-row tile shape (the plan's, and the tuning override's
    others), forced through the knob with the small-batch route off, on ragged batches and
    partial row tiles, against the oracle."""
    if gemm_kernel != "default":
        pytest.skip("tile shapes of the default kernel")
    k, n = 1024, 300
    name = S.TYPE_NAMES[qt]
    for m in (16, 40, 100):
        w = S.make_weight(qt, n, k, 31 + m)
        x = S.make_activation(m, k, 32 + m, outliers=True)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m)
        splits = 2 if m == 100 else 1  # the 100-row batch also through split-K completion
        gpu.tune("gemm_small", 2)
        gpu.tune("gemm_tiles", *shape)
        gpu.tune("gemm_splits", splits)
        try:
            plan = gpu.matmul_plan(qt, k, n, m)
            print(name, "shape", shape, "m", m, plan, flush=True)
            assert gpu.matmul_route(qt, k, n, m) == "mfma"
            assert plan == "k_gemmw_q4k<%d,%d,%d,%s> splits=%d" % (*shape, name, splits), plan
            y = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, None, k, n).cpu().numpy()
        finally:
            gpu.tune("gemm_splits")
            gpu.tune("gemm_tiles")
            gpu.tune("gemm_small")
        check_close(y, yo, exact, abs_sum, f"{name} {shape} m{m}")


@pytest.mark.parametrize("qt, n, k, m, plan", [
    (S.Q4_K, 4096, 14336, 384, "k_gemmw_q4k<8,1,4,Q4_K> splits=4"),
    (S.Q5_K, 4096, 11008, 768, "k_gemmw_q4k<8,1,4,Q5_K> splits=2"),
    (S.Q8_0, 4096, 14336, 384, "k_gemmw_b32<Q8_0,4,2> splits=4"),
    (S.Q6_K, 4096, 4096, 768, "k_gemmw_q6k<4,2> splits=4"),
    (S.Q4_K, 11008, 4096, 384, "k_gemmw_q4k<4,1,2,Q4_K> splits=4")])
def test_long_k_large_batches(gpu, orc, qt, n, k, m, plan, gemm_kernel):
    """Large batches on the plans that split K to fill the CUs (Q4_K / Q5_K long K on 256 x
    128 tiles, the 32-element block types and Q6_K by stage-rounds): 8 sampled activation rows
    (all outputs) against the oracle, every row against row-wise GEMV."""
    import torch
    if gemm_kernel != "default":
        pytest.skip("the default plan only")
    assert gpu.matmul_plan(qt, k, n, m) == plan
    w = S.make_weight(qt, n, k, 41)
    x = S.make_activation(m, k, 42, outliers=True)
    print("long K", S.TYPE_NAMES[qt], n, k, m, plan, flush=True)
    wd, xd = _dev(w), _dev(x)
    y = gpu.matmul_quant_dev(xd, wd, qt, None, k, n)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(m).choice(m, size=8, replace=False))
    yo = orc.matmul(x[rows], w, qt, None, k, n, 8, threads=8)
    exact, abs_sum = orc.matmul_f64(x[rows], w, qt, None, k, n, 8)
    check_close(y.cpu().numpy()[rows], yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k} m{m}")
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    yg = torch.cat([gpu.gemv_q8_dev(wd, qt, k, n, qs[i:i + 8], sc[i:i + 8], bs[i:i + 8])
                    for i in range(0, m, 8)])
    d = (y - yg).abs().cpu().numpy().astype(np.float64)
    scale = np.maximum(np.abs(yg.cpu().numpy()), 1e-3 * np.abs(yg.cpu().numpy()).max(axis=1, keepdims=True))
    assert (d / scale).max() < 1e-3, (d / scale).max()
