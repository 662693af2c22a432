"""Parity of the HIP path with the reference, through the C ABI, on an MI355X.

Bars (written into each test):
  - Q8_0 activation bytes (int8 qs, fp32 scales, int32 block sums): bit-exact.
  - Outputs: |gpu - ref| <= 1e-4 * max(|ref|, 2^-8 * A) against the reference's own fp32
    output, where A is the row's sum of absolute per-block terms; and, against the fp64
    evaluation of the same quantized terms,
    |gpu - exact| <= max(1e-4 * max(|exact|, 2^-10 * A), 2 * |ref - exact|, R * A), where
    R = max over the same activation row of |ref - exact| / A: never further from the exact value
    than twice the reference's own rounding error there, or than the reference's worst
    rounding anywhere in that row of outputs relative to A. The reference's sequential fp32 sum is
    itself up to 1.5e-4 away from exact under the 2^-10 floor on outlier inputs, which is
    why neither gate can use that floor alone. The R * A term is there because a different
    fp32 order than the reference's (split-K partials, fma per block) can miss the first two
    at an element where the reference happens to land near the exact value: on Q4_0
    14336 x 4096 at 8 rows (128 blocks a row), a CPU emulation of the weight-row kernel's
    order lands 5.1e-6 from exact at one element against an allowance of 4.5e-6, while its
    worst |gpu - exact| / A over the output is 1.4e-7 against the reference's 2.9e-7.
  - Anything the GEMV computes twice the same way (host vs device entry point, batch row vs
    single row) must agree bit for bit.
"""
import numpy as np
import pytest

from conftest import load_golden, split_cases
from cllm_inference_amd import synth as S
import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4
TYPES = [S.Q4_0, S.Q5_0, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def check_close(got, ref, exact, abs_sum, what):
    """The two bars above. exact has the outputs' (m, n) shape; R is taken per activation
    row (the last axis), so one row's rounding does not loosen another's."""
    exact = np.asarray(exact, np.float64)
    got = np.asarray(got, np.float64).reshape(exact.shape)
    ref = np.asarray(ref, np.float64).reshape(exact.shape)
    abs_sum = np.asarray(abs_sum, np.float64).reshape(exact.shape)
    d_ref = np.abs(got - ref) / np.maximum(np.maximum(np.abs(ref), abs_sum * 2.0 ** -8), 1e-30)
    assert d_ref.max() <= TOL, f"{what}: vs reference {d_ref.max():.3g} at {np.argmax(d_ref)}"
    ref_worst = (np.abs(ref - exact) / np.maximum(abs_sum, 1e-30)).max(axis=-1, keepdims=True)
    allowed = np.maximum(np.maximum(TOL * np.maximum(np.abs(exact), abs_sum * 2.0 ** -10),
                                    2.0 * np.abs(ref - exact)), ref_worst * abs_sum)
    excess = np.abs(got - exact) - allowed
    assert excess.max() <= 0, f"{what}: vs exact exceeds the bound at {np.argmax(excess)}"


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ------------------------------------------------------------------------- quantize

def test_quantize_bit_exact_host_and_device(gpu):
    for name, c in split_cases(load_golden("q8_act.npz")).items():
        print("quantize case", name, c["x"].shape, flush=True)
        q = gpu.quantize_row_q8_0(c["x"])
        assert np.array_equal(q.qs, c["qs"]), name
        assert np.array_equal(bits(q.scales), bits(c["scales"])), name
        assert np.array_equal(q.bsums, c["bsums"]), name
        qs, sc, bs = gpu.quantize_q8_0_dev(_dev(c["x"]))
        assert np.array_equal(qs.cpu().numpy(), c["qs"]), name
        assert np.array_equal(bits(sc.cpu().numpy()), bits(c["scales"])), name
        assert np.array_equal(bs.cpu().numpy(), c["bsums"]), name


def test_quantize_large_random_matches_oracle(gpu, orc):
    x = S.make_activation(512, 4096, 4242, outliers=True)
    x[7, 64:96] = 0.0
    x[9, :32] *= np.float32(1e-38)
    qs, sc, bs = gpu.quantize_q8_0_dev(_dev(x))
    oq, osc, obs = orc.quantize(x)
    assert np.array_equal(qs.cpu().numpy(), oq)
    assert np.array_equal(bits(sc.cpu().numpy()), bits(osc))
    assert np.array_equal(bs.cpu().numpy(), obs)


# ------------------------------------------------------------------------- GEMV parity

@pytest.mark.parametrize("tag", ["c0", "c1", "c4_q5_k_m1", "c4_q5_k_m4", "c4_q8_0_m1", "c4_q8_0_m4"])
def test_workload_vs_reference_golden(gpu, orc, tag):
    c = split_cases(load_golden("gemv.npz"))[tag]
    qt, n, k, m = (int(v) for v in c["meta"])
    cfg = {"c0": ("c0_q8_0_gemv", "w"), "c1": ("c1_q4_k_gemv", "ffn")}.get(
        tag, ("c4_m_sweep", "q5_k" if "q5_k" in tag else "q8_0"))
    _, _, _, w = S.config_weight(*cfg)
    x = S.config_activation(cfg[0], m, k)
    print("workload", tag, S.TYPE_NAMES[qt], n, k, m, flush=True)
    y_host = gpu.matmul_quant_batch(x, w, qt, None, k, n, m)
    y_dev = gpu.matmul_quant_dev(_dev(x), _dev(w), qt, None, k, n).cpu().numpy()
    assert np.array_equal(bits(y_host), bits(y_dev))
    rows = c["rows"]
    rb = S.row_bytes(qt, k)
    exact, abs_sum = orc.matmul_f64(x, w.reshape(n, rb)[rows].reshape(-1), qt, None, k, len(rows), m)
    check_close(y_host[:, rows], c["y"], exact, abs_sum, tag)


def test_q6_k_output_head_full_size(gpu, orc):
    """128256 x 4096 Q6_K (431 MB): every 16th row against the reference, all rows against
    the device entry point, and a second call on the same buffers must repeat every bit."""
    c = split_cases(load_golden("gemv.npz"))["c2"]
    qt, n, k, m = (int(v) for v in c["meta"])
    _, _, _, w = S.config_weight("c2_q6_k_head", "output")
    x = S.config_activation("c2_q6_k_head", 1, k)
    print("workload c2 Q6_K", n, k, flush=True)
    wd, xd = _dev(w), _dev(x)
    y1 = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
    y2 = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
    assert np.array_equal(bits(y1), bits(y2))
    rows = c["rows"]
    rb = S.row_bytes(qt, k)
    exact, abs_sum = orc.matmul_f64(x, w.reshape(n, rb)[rows].reshape(-1), qt, None, k, len(rows), 1)
    check_close(y1[:, rows], c["y"], exact, abs_sum, "c2")
    # rows the golden file does not hold: against the oracle
    others = np.arange(1, n, 997)
    exact, abs_sum = orc.matmul_f64(x, w.reshape(n, rb)[others].reshape(-1), qt, None, k, len(others), 1)
    yo = orc.matmul(x, w.reshape(n, rb)[others].reshape(-1), qt, None, k, len(others), 1)
    check_close(y1[:, others], yo, exact, abs_sum, "c2-oracle")


@pytest.mark.parametrize("qt,k,mb", [(S.Q6_K, 4096, 40), (S.Q6_K, 14336, 40), (S.Q4_K, 4096, 100)])
def test_staged_stream_equals_register_ring(gpu, orc, qt, k, mb):
    """Long decode streams (Q6_K from 32 MB, Q4_K from 96 MB) take the LDS-staged kernel and
    shorter ones the register-ring kernel; both compute the same per-unit terms in the same
    order, so rows of a long matrix (ragged row count; k = 14336 ends every Q6_K row with a half
    item) must equal bit for bit the same rows run as a small matrix -- with a bias, with the
    residual add, and in the three-matrix launch -- and match the oracle."""
    import torch
    rb = S.row_bytes(qt, k)
    n = (mb << 20) // rb + 3
    print("staged", S.TYPE_NAMES[qt], n, k, flush=True)
    w = S.make_weight(qt, n, k, 9100 + k)
    x = S.make_activation(1, k, 9200 + k, outliers=True)
    bias = np.random.default_rng(k).standard_normal(n).astype(np.float32)
    rows = np.r_[0:96, n // 2:n // 2 + 64, n - 96:n]
    sub = w.reshape(n, rb)[rows].reshape(-1)
    wd, xd, bd = _dev(w), _dev(x), _dev(bias)
    sd, sbd = _dev(sub), _dev(bias[rows])

    y = gpu.matmul_quant_dev(xd, wd, qt, bd, k, n).cpu().numpy()
    y_small = gpu.matmul_quant_dev(xd, sd, qt, sbd, k, len(rows)).cpu().numpy()
    assert np.array_equal(bits(y[:, rows]), bits(y_small))
    exact, abs_sum = orc.matmul_f64(x, sub, qt, bias[rows], k, len(rows), 1)
    yo = orc.matmul(x, sub, qt, bias[rows], k, len(rows), 1)
    check_close(y[:, rows], yo, exact, abs_sum, "staged")

    base = np.random.default_rng(k + 1).standard_normal((1, n)).astype(np.float32)
    r = _dev(base)
    gpu.matmul_quant_residual_dev(xd, wd, qt, bd, k, n, r)
    r_small = _dev(base[:, rows])
    gpu.matmul_quant_residual_dev(xd, sd, qt, sbd, k, len(rows), r_small)
    assert np.array_equal(bits(r.cpu().numpy()[:, rows]), bits(r_small.cpu().numpy()))

    # three matrices in one launch (40 MB in all): the segment of every row resolves as in
    # separate launches
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    cuts = [0, n // 3, n // 3 + 1000, n]
    mats = [_dev(w.reshape(n, rb)[a:b].reshape(-1)) for a, b in zip(cuts, cuts[1:])]
    outs = gpu.gemv_q8_multi_dev(mats, qt, k, [b - a for a, b in zip(cuts, cuts[1:])], qs, sc, bs)
    y_nb = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
    assert np.array_equal(bits(np.concatenate([o.cpu().numpy() for o in outs], axis=1)), bits(y_nb))
    torch.cuda.synchronize()


@pytest.mark.parametrize("qt,n,k", [(S.Q8_0, 4096, 4096), (S.Q4_K, 1024, 4096),
                                    (S.Q6_K, 1000, 14336), (S.Q5_K, 333, 4096)])
def test_streaming_decode_row_handout(gpu, orc, qt, n, k):
    """The one-workgroup-per-CU decode kernel hands a workgroup's rows to its 16 waves from an
    LDS counter. Grids that leave workgroups with fewer rows than waves (a wave with no row
    still stages its share of the activation), and grids whose workgroups hand out several rows
    per wave, must give bit for bit the register-ring kernel's result -- fused quantization,
    a prequantized batch, and the RMSNorm staging -- and match the oracle."""
    import torch
    w = S.make_weight(qt, n, k, 31 + n)
    x = S.make_activation(1, k, 32 + n, outliers=True)
    nw = (1.0 + 0.1 * np.random.default_rng(n).standard_normal(k)).astype(np.float32)
    wd, xd, nwd = _dev(w), _dev(x), _dev(nw)
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    norm = k <= 4096

    def run():
        y = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
        yq = gpu.gemv_q8_dev(wd, qt, k, n, qs, sc, bs).cpu().numpy()
        yn = gpu.rmsnorm_gemv_multi_dev(xd, nwd, 1e-5, [wd], qt, k, [n])[0].cpu().numpy() if norm else None
        torch.cuda.synchronize()
        return y, yq, yn

    try:
        gpu.tune("gemv_kernel", 1)
        ring = run()
        for grid in (0, 7, 61, 192, 224, 300):
            print("row handout", S.TYPE_NAMES[qt], n, k, "grid", grid, flush=True)
            gpu.tune("gemv_kernel", 3)
            gpu.tune("gemv_str_grid", grid)
            got = run()
            for a, b, what in zip(got, ring, ("fused", "prequantized", "rmsnorm")):
                if a is not None:
                    assert np.array_equal(bits(a), bits(b)), (what, grid, np.flatnonzero(bits(a) != bits(b))[:8])
    finally:
        gpu.tune("gemv_kernel")
        gpu.tune("gemv_str_grid")
    exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, 1)
    check_close(ring[0], orc.matmul(x, w, qt, None, k, n, 1), exact, abs_sum, "row handout")


@pytest.mark.parametrize("qt", TYPES)
def test_streaming_batch_equals_register_ring(gpu, orc, qt):
    """2 to 8 activation rows in one launch of the streaming kernel (each lane keeping one sum
    per row) against the register-ring kernel's launches of 1, 2, 4 or 8 rows: bit for bit,
    through the fp32 and quantized-batch entries, with a bias, over two matrices in one launch,
    and on grids that leave workgroups short of rows; and against the oracle."""
    import torch
    k = 1024 if S.BLOCK[qt] == 32 else 2048
    n, n2 = 333, 130
    w, w2 = S.make_weight(qt, n, k, 71), S.make_weight(qt, n2, k, 72)
    bias = np.random.default_rng(73).standard_normal(n).astype(np.float32)
    wd, w2d, bd = _dev(w), _dev(w2), _dev(bias)
    for m in (2, 3, 5, 8):
        x = S.make_activation(m, k, 74 + m, outliers=True)
        xd = _dev(x)
        qs, sc, bs = gpu.quantize_q8_0_dev(xd)

        def run():
            y = gpu.matmul_quant_dev(xd, wd, qt, bd, k, n).cpu().numpy()
            yq = gpu.gemv_q8_dev(wd, qt, k, n, qs, sc, bs, bd).cpu().numpy()
            ym = [t.cpu().numpy() for t in gpu.gemv_q8_multi_dev([wd, w2d], qt, k, [n, n2], qs, sc, bs)]
            torch.cuda.synchronize()
            return [y, yq] + ym

        try:
            gpu.tune("gemm_small", 2)
            gpu.tune("gemv_kernel", 1)
            assert gpu.matmul_route(qt, k, n, m) == "gemv"
            ring = run()
            gpu.tune("gemv_kernel", 3)
            plan = gpu.matmul_plan(qt, k, n, m)
            assert plan == f"k_gemv_str<{S.TYPE_NAMES[qt]},{m}> launches=1", plan
            for grid in (0, 7, 61):
                print("streaming batch", S.TYPE_NAMES[qt], n, k, "m", m, "grid", grid, flush=True)
                gpu.tune("gemv_str_grid", grid)
                got = run()
                for a, b, what in zip(got, ring, ("fused", "quantized", "multi 0", "multi 1")):
                    assert np.array_equal(bits(a), bits(b)), (what, m, grid, np.flatnonzero(bits(a) != bits(b))[:8])
        finally:
            for knob in ("gemv_str_grid", "gemv_kernel", "gemm_small"):
                gpu.tune(knob)
        exact, abs_sum = orc.matmul_f64(x, w, qt, bias, k, n, m)
        check_close(got[0].reshape(m, n), orc.matmul(x, w, qt, bias, k, n, m).reshape(m, n), exact,
                    abs_sum, f"streaming batch {S.TYPE_NAMES[qt]} m{m}")


@pytest.mark.parametrize("m", [1, 2, 16])
def test_fused_quantization_at_rounding_boundaries(gpu, orc, m):
    """Every quantized block of the input holds a value whose rounding a contracted
    x * id + 1.5 * 2^23 would move by one (synth.rounding_boundary_activation): the kernels that
    quantize inside (the one-row streaming GEMV, the two-row register ring, the small-batch
    kernel) must give the pre-quantized path's results bit for bit, and the quantizer the
    oracle's bytes."""
    import torch
    k = 4096
    x = S.rounding_boundary_activation(m, k, 17 + m)
    xd = _dev(x)
    qs, sc, bs = gpu.quantize_q8_0_dev(xd)
    oq, osc, obs = orc.quantize(x)
    assert np.array_equal(qs.cpu().numpy(), oq)
    assert np.array_equal(bits(sc.cpu().numpy()), bits(osc))
    for qt in (S.Q4_K, S.Q8_0):
        n = 2048
        w = S.make_weight(qt, n, k, 600 + qt)
        wd = _dev(w)
        print("boundary", S.TYPE_NAMES[qt], "m", m, gpu.matmul_plan(qt, k, n, m), flush=True)
        y_fused = gpu.matmul_quant_dev(xd, wd, qt, None, k, n).cpu().numpy()
        y_q8 = gpu.gemv_q8_dev(wd, qt, k, n, qs, sc, bs).cpu().numpy()
        torch.cuda.synchronize()
        assert np.array_equal(bits(y_fused), bits(y_q8)), (S.TYPE_NAMES[qt], m)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m)
        check_close(y_fused.reshape(m, n), yo.reshape(m, n), exact, abs_sum, f"boundary m{m}")


def test_all_types_shapes_bias_vs_reference_golden(gpu, orc):
    cases = split_cases(load_golden("types.npz"))
    for tag, c in cases.items():
        qt, n, k, m, seed = (int(v) for v in c["meta"])
        print("types case", tag, flush=True)
        w = S.make_weight(qt, n, k, seed)
        x = S.make_activation(m, k, seed + 1, outliers=True)
        bias = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        y = gpu.matmul_quant_batch(x, w, qt, None, k, n, m)
        yb = gpu.matmul_quant_batch(x, w, qt, bias, k, n, m)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        check_close(y, c["y"], exact, abs_sum, tag)
        exact_b, abs_b = orc.matmul_f64(x, w, qt, bias, k, n, m)
        check_close(yb, c["ybias"], exact_b, abs_b, tag + "+bias")
        # bias is added after the row's accumulation, like the reference
        assert np.array_equal(bits(yb), bits((y + bias).astype(np.float32))), tag


def test_reference_test_inputs(gpu, orc):
    """The inputs the reference's own quant_test builds (quant_test.cpp:237-361)."""
    for name, c in split_cases(load_golden("refkat.npz")).items():
        qt = S.NAME_TO_TYPE[name]
        k = 64 if S.BLOCK[qt] <= 32 else 256
        for xk, yk, m in (("x1", "y1", 1), ("x3", "y3", 3)):
            y = gpu.matmul_quant_batch(c[xk], c["w"], qt, None, k, 40, m)
            exact, abs_sum = orc.matmul_f64(c[xk], c["w"], qt, None, k, 40, m)
            check_close(y.reshape(m, 40), c[yk].reshape(m, 40), exact, abs_sum, name + xk)


@pytest.mark.parametrize("qt", TYPES)
def test_batch_rows_equal_single_rows(gpu, qt):
    """A 13-row batch on the GEMV (the small-batch kernel turned off) equals its rows run one
    at a time, bit for bit."""
    k = 1024
    n = 333
    w = S.make_weight(qt, n, k, 55)
    x = S.make_activation(13, k, 56, outliers=True)
    try:
        gpu.tune("gemm_small", 2)
        yb = gpu.matmul_quant_batch(x, w, qt, None, k, n, 13)
    finally:
        gpu.tune("gemm_small")
    for t in (0, 5, 12):
        y1 = gpu.matmul_quant(x[t], w, qt, None, k, n)
        assert np.array_equal(bits(y1), bits(yb[t])), (S.TYPE_NAMES[qt], t)


@pytest.mark.parametrize("qt", TYPES)
def test_edge_shapes(gpu, orc, qt):
    bs = S.BLOCK[qt]
    for (n, k, m) in [(1, bs, 1), (3, bs, 2), (9, 2 * bs, 7), (65, 3 * bs, 5), (130, 14336 if bs == 256 else 96, 1)]:
        w = S.make_weight(qt, n, k, n + k)
        x = S.make_activation(m, k, m + k, outliers=True)
        y = gpu.matmul_quant_batch(x, w, qt, None, k, n, m).reshape(m, n)
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
        yo = orc.matmul(x, w, qt, None, k, n, m).reshape(m, n)
        check_close(y, yo, exact, abs_sum, f"{S.TYPE_NAMES[qt]} {n}x{k} m{m}")


def test_vec_dot_rows(gpu, orc):
    for qt in TYPES:
        k = 2048
        w = S.make_weight(qt, 10, k, 4)
        x = S.make_activation(1, k, 5)[0]
        q = gpu.quantize_row_q8_0(x)
        got = gpu.vec_dot_rows(w, qt, q, k, 10)
        want = orc.matmul(x, w, qt, None, k, 10, 1)[0]
        exact, abs_sum = orc.matmul_f64(x, w, qt, None, k, 10, 1)
        check_close(got, want, exact[0], abs_sum[0], S.TYPE_NAMES[qt])
        assert abs(gpu.vec_dot_row(w, qt, q, k) - got[0]) == 0.0


def test_registered_weights_resolve_by_offset(gpu):
    import ctypes
    qt, k, n = S.Q4_K, 1024, 64
    region = np.zeros(4096 + 3 * S.row_bytes(qt, k) * n, np.uint8)
    w = S.make_weight(qt, n, k, 8)
    off = 4096 + S.row_bytes(qt, k) * n  # 16-aligned offset inside the region
    region[off: off + w.size] = w
    x = S.make_activation(1, k, 9)[0]
    y_plain = gpu.matmul_quant(x, w, qt, None, k, n)
    lib = gpu.load_library()
    base = region.ctypes.data
    assert lib.cllm_hip_register_weights(ctypes.c_void_p(base), region.size) == 0
    try:
        view = region[off: off + w.size]
        assert view.ctypes.data == base + off
        y_reg = gpu.matmul_quant(x, view, qt, None, k, n)
        assert np.array_equal(bits(y_plain), bits(y_reg))
    finally:
        assert lib.cllm_hip_unregister_weights(ctypes.c_void_p(base)) == 0


def test_device_argument_errors(gpu):
    import torch
    w = torch.zeros(4096 + 16, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="misaligned"):
        gpu.matmul_quant_dev(x, w[1:], S.Q4_K, None, 256, 4)
    with pytest.raises(RuntimeError, match="in_dim not divisible by block size"):
        gpu.matmul_quant_dev(x[:, :100].contiguous(), w, S.Q4_K, None, 100, 4)
    assert gpu.matmul_route(S.Q4_K, 4096, 4096, 1) == "gemv"
