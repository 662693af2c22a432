"""Pins the CPU oracle (oracle/cllm_oracle.c) before it is trusted as the GPU's checker.

Each check is independent of the oracle's own formulas:
  - golden vectors produced by the reference compiled from its own sources (bit-exact);
  - known-answer blocks restated from the reference's tests (tests/quant_test.cpp:58-218);
  - an independent numpy decode of the byte layouts (tests/np_decode.py);
  - closed forms: exact integer dots when every scale is 1, ties-to-even at d = 1;
  - invariants: batch == per-row, y(bias) == y + bias.
A planted mistake (a swapped nibble order) is shown to fail the integer check, and a sum
without the reference's fma contraction is shown to miss the float-dot golden vectors.
"""
import numpy as np
import pytest

from conftest import load_golden, split_cases
import np_decode as D
from cllm_inference_amd import synth as S
import oracle as O

TYPES = [S.Q4_0, S.Q5_0, S.Q8_0, S.Q4_K, S.Q5_K, S.Q6_K]
FD_TYPES = list(S.FLOAT_DOT_TYPES)
ALL_TYPES = TYPES + FD_TYPES


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype.itemsize == 4 else np.uint8)


# ------------------------------------------------------------------ quantize_row_q8_0

def test_quantize_matches_reference_golden(orc):
    cases = split_cases(load_golden("q8_act.npz"))
    assert set(cases) >= {"special", "c0", "c1", "c4", "c3_down"}
    for name, c in cases.items():
        qs, sc, bs = orc.quantize(c["x"])
        assert np.array_equal(qs, c["qs"]), name
        assert np.array_equal(bits(sc), bits(c["scales"])), name
        assert np.array_equal(bs, c["bsums"]), name


def test_quantize_closed_forms(orc):
    # amax = 127 -> d = 1 exactly, id = 1, q = rint(x): ties to even
    x = np.zeros(64, np.float32)
    x[:10] = [127, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5, -127]
    qs, sc, bs = orc.quantize(x)
    assert sc[0, 0] == np.float32(1.0)
    assert list(qs[0, :10]) == [127, 2, 4, -2, -4, 0, 2, 0, 126, -127]
    assert bs[0, 0] == int(qs[0, :32].astype(np.int64).sum())
    # all-zero block
    assert sc[0, 1] == 0.0 and not qs[0, 32:].any() and bs[0, 1] == 0
    # the block maximum always maps to +-127 and nothing reaches -128
    rng = np.random.default_rng(3)
    x = rng.standard_normal((8, 256)).astype(np.float32) * 5
    qs, sc, bs = orc.quantize(x)
    blk = qs.reshape(-1, 32).astype(np.int64)
    assert (np.abs(blk).max(axis=1) == 127).all()
    assert blk.min() >= -127
    assert np.array_equal(blk.sum(axis=1), bs.reshape(-1))
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(bits(sc.reshape(-1)), bits((amax / np.float32(127.0)).astype(np.float32)))


def test_quantize_rejects_ragged(orc):
    with pytest.raises(RuntimeError, match="quantize_row_q8_0: n not divisible by 32"):
        orc.quantize(np.zeros((1, 48), np.float32))


# ------------------------------------------------------------------ block layouts

def _blk(n):
    return np.zeros(n, np.uint8)


def _put_one(b, off):
    b[off], b[off + 1] = 0x00, 0x3C  # fp16 1.0


def test_dequant_known_answers(orc):
    """The reference's own hand-built blocks (quant_test.cpp:58-218), restated."""
    b = _blk(18); _put_one(b, 0); b[2] = 0x9A
    y = orc.dequantize(b, S.Q4_0, 32)
    assert (y[0], y[16], y[1]) == (2.0, 1.0, -8.0)
    b = _blk(22); _put_one(b, 0); b[2] = 0x01; b[6] = 0x21
    y = orc.dequantize(b, S.Q5_0, 32)
    assert (y[0], y[16]) == (1.0, -14.0)
    b = _blk(34); _put_one(b, 0); b[2] = 0xFF; b[3] = 0x02
    y = orc.dequantize(b, S.Q8_0, 32)
    assert (y[0], y[1]) == (-1.0, 2.0)
    b = _blk(144); b[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]; b[16] = 0x21; _put_one(b, 0)
    y = orc.dequantize(b, S.Q4_K, 256)
    assert (y[0], y[32], y[1]) == (1.0, 2.0, 0.0)
    b = _blk(176); b[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]; b[48] = 0x21; _put_one(b, 0)
    y = orc.dequantize(b, S.Q5_K, 256)
    assert (y[0], y[32]) == (1.0, 2.0)
    b[16] = 0x01
    assert orc.dequantize(b, S.Q5_K, 256)[0] == 17.0
    b = _blk(210); b[192:208] = 1; b[0] = 0x21; _put_one(b, 208)
    y = orc.dequantize(b, S.Q6_K, 256)
    assert (y[0], y[64]) == (-31.0, -30.0)


def _put_f16(b, off, v):
    b[off:off + 2] = np.array([v], np.float16).view(np.uint8)


def test_dequant_known_answers_float_dot_types(orc):
    """The reference's hand-built blocks for the types without vec_dot
    (quant_test.cpp:42-55, 70-80, 95-105, 120-130, 133-149, 152-170), restated."""
    f = np.array([1.5, -2.25, 0.0, 3.0], np.float32)
    y = orc.dequantize(f.view(np.uint8), S.F32, 4)
    assert (y[0], y[1]) == (1.5, -2.25)
    b = np.array([0x00, 0x3C, 0x00, 0x38, 0x00, 0x00, 0x00, 0xC0], np.uint8)  # 1, .5, 0, -2
    assert tuple(orc.dequantize(b, S.F16, 4)) == (1.0, 0.5, 0.0, -2.0)
    b = _blk(20); _put_one(b, 0); _put_f16(b, 2, 0.5); b[4] = 0x21
    y = orc.dequantize(b, S.Q4_1, 32)
    assert (y[0], y[16], y[1]) == (1.5, 2.5, 0.5)
    b = _blk(24); _put_one(b, 0); b[4] = 0x01; b[8] = 0x21
    y = orc.dequantize(b, S.Q5_1, 32)
    assert (y[0], y[16]) == (17.0, 2.0)
    b = _blk(36); _put_one(b, 0); b[4] = 0xFF; b[5] = 0x02
    y = orc.dequantize(b, S.Q8_1, 32)
    assert (y[0], y[1]) == (-1.0, 2.0)
    b = _blk(84); b[0:16] = 0x01; b[16] = 0x03; b[32] = 0x03; _put_one(b, 80)
    y = orc.dequantize(b, S.Q2_K, 256)
    assert (y[0], y[16], y[32], y[128]) == (3.0, 3.0, 0.0, 0.0)
    b = _blk(110); b[96:104] = 0x11; b[104:108] = 0xAA; _put_one(b, 108)
    y = orc.dequantize(b, S.Q3_K, 256)
    assert (y[0], y[255]) == (-4.0, -4.0)
    b[0:32] = 0xFF
    y = orc.dequantize(b, S.Q3_K, 256)
    assert (y[0], y[255]) == (0.0, 0.0)


def test_dequant_unknown_type_fails(orc):
    with pytest.raises(RuntimeError, match="unsupported ggml type for dequantize"):
        orc.dequantize(_blk(64), 999, 32)


@pytest.mark.parametrize("qt", ALL_TYPES)
def test_dequant_matches_numpy_layout_decode(orc, qt):
    k = 512
    w = S.make_weight(qt, 3, k, 11)
    q, scale, wmin = D.decode(w, qt, 3, k)
    want = (scale * q - wmin).astype(np.float32)
    for j in range(3):
        got = orc.dequantize(w[j * S.row_bytes(qt, k):], qt, k)
        # fp32 evaluation order of d*sc*q - dmin*m may differ from the float64 one by 1 ulp
        np.testing.assert_allclose(got, want[j], rtol=2e-7, atol=1e-12)


# ------------------------------------------------------------------ vec_dot / matmul

def _int_special_weight(qt, n, k, rng):
    """Every effective per-element scale is 1 and every min 0: d = 1 (Q6_K sc = 1; K-quants
    sc = 1, m = 0, dmin = 0), random quant bits. y is then an exact integer dot."""
    w = S.make_weight(qt, n, k, int(rng.integers(1 << 30)))
    blk = w.reshape(-1, S.TYPE_SIZE[qt])
    if qt in (S.Q8_0, S.Q4_0, S.Q5_0):
        blk[:, 0:2] = [0x00, 0x3C]
    elif qt in (S.Q4_K, S.Q5_K):
        blk[:, 0:2] = [0x00, 0x3C]
        blk[:, 2:4] = 0
        blk[:, 4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    else:
        blk[:, 192:208] = 1
        blk[:, 208:210] = [0x00, 0x3C]
    return w


def _int_special_x(m, k, rng):
    """Activation blocks with amax = 127 so that d = 1 and q = rint(x)."""
    x = rng.integers(-127, 128, size=(m, k)).astype(np.float32)
    x[:, ::32] = 127.0
    return x


@pytest.mark.parametrize("qt", TYPES)
def test_matmul_exact_integer_case(orc, qt):
    rng = np.random.default_rng(qt)
    n, k, m = 37, 512, 2
    w = _int_special_weight(qt, n, k, rng)
    x = _int_special_x(m, k, rng)
    q, scale, wmin = D.decode(w, qt, n, k)
    assert (scale == 1).all() and (wmin == 0).all()
    want = x.astype(np.int64) @ q.T
    got = orc.matmul(x, w, qt, None, k, n, m)
    assert np.array_equal(got.astype(np.int64), want)


def test_planted_nibble_swap_is_caught():
    """A decoder that swaps the Q4_K nibble order must fail the integer check."""
    rng = np.random.default_rng(5)
    n, k = 8, 256
    w = _int_special_weight(S.Q4_K, n, k, rng)
    x = _int_special_x(1, k, rng)
    q, _, _ = D.decode(w, S.Q4_K, n, k)
    wrong = q.reshape(n, 4, 2, 32)[:, :, ::-1, :].reshape(n, k)  # high/low nibble swapped
    good = x.astype(np.int64) @ q.T
    bad = x.astype(np.int64) @ wrong.T
    assert not np.array_equal(good, bad)


@pytest.mark.parametrize("qt", TYPES)
def test_f64_matches_bruteforce(orc, qt):
    n, k, m = 19, 512, 3
    w = S.make_weight(qt, n, k, 123)
    x = S.make_activation(m, k, 321, outliers=True)
    qs, sc, _ = orc.quantize(x)
    xv = qs.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=1)
    q, scale, wmin = D.decode(w, qt, n, k)
    wv = scale * q - wmin
    want = xv @ wv.T
    got, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12 * abs_sum.max())
    # and the fp32 oracle is within the gate of its own fp64 evaluation
    y32 = orc.matmul(x, w, qt, None, k, n, m)
    err, _, _ = O.rel_err_floored(y32, got, abs_sum)
    assert err < 1e-4


def test_oracle_matches_reference_golden_types(orc):
    cases = split_cases(load_golden("types.npz"))
    assert len(cases) >= 20
    for tag, c in cases.items():
        qt, n, k, m, seed = (int(v) for v in c["meta"])
        w = S.make_weight(qt, n, k, seed)
        assert O_sha(w) == str(c["w_sha"]), f"generator drift for {tag}"
        x = S.make_activation(m, k, seed + 1, outliers=True)
        bias = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
        y = orc.matmul(x, w, qt, None, k, n, m)
        yb = orc.matmul(x, w, qt, bias, k, n, m)
        assert np.array_equal(bits(y), bits(c["y"])), tag
        assert np.array_equal(bits(yb), bits(c["ybias"])), tag
        # reference semantics: bias is added after the row's accumulation
        assert np.array_equal(bits(yb), bits((y + bias).astype(np.float32))), tag


def O_sha(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("tag", ["c0", "c1", "c4_q5_k_m1", "c4_q5_k_m4", "c4_q8_0_m1", "c4_q8_0_m4"])
def test_oracle_matches_reference_golden_workloads(orc, tag):
    c = split_cases(load_golden("gemv.npz"))[tag]
    qt, n, k, m = (int(v) for v in c["meta"])
    cfg = {"c0": ("c0_q8_0_gemv", "w"), "c1": ("c1_q4_k_gemv", "ffn")}.get(
        tag, ("c4_m_sweep", "q5_k" if "q5_k" in tag else "q8_0"))
    _, _, _, w = S.config_weight(*cfg)
    x = S.config_activation(cfg[0], m, k)
    assert O_sha(w) == str(c["w_sha"]) and O_sha(x) == str(c["x_sha"])
    rows = c["rows"]
    rb = S.row_bytes(qt, k)
    wsub = w.reshape(n, rb)[rows].reshape(-1)
    y = orc.matmul(x, wsub, qt, None, k, len(rows), m)
    assert np.array_equal(bits(y), bits(c["y"]))


def test_oracle_matches_reference_golden_m_sweep_full_size(orc):
    """Every point of the M-sweep at full size (Q5_K 14336x4096, Q8_0 4096x4096): the oracle's
    rows bit-identical to the compiled reference's (tests/golden/batch_large.npz)."""
    c = split_cases(load_golden("batch_large.npz"))
    seen = 0
    for label in ("q5_k", "q8_0"):
        qt, n, k, w = S.config_weight("c4_m_sweep", label)
        assert O_sha(w) == str(c[label]["w_sha"]), f"generator drift for {label}"
        for m in S.CONFIGS["c4_m_sweep"]["m"] + ([512] if label == "q5_k" else []):
            g = c[f"{label}_m{m}"]
            x = S.config_activation("c4_m_sweep", m, k)
            assert O_sha(x) == str(g["x_sha"]), f"generator drift for {label} m{m}"
            rows = g["rows"]
            y = orc.matmul(x[rows], w, qt, None, k, n, len(rows), threads=8)
            assert np.array_equal(bits(y), bits(g["y"])), f"{label} m{m}"
            seen += 1
    assert seen == 11


def test_oracle_matches_reference_golden_refkat(orc):
    cases = split_cases(load_golden("refkat.npz"))
    assert len(cases) == 13
    for name, c in cases.items():
        qt = S.NAME_TO_TYPE[name]
        k = 64 if S.BLOCK[qt] <= 32 else 256
        assert np.array_equal(bits(orc.matmul(c["x1"], c["w"], qt, None, k, 40, 1)), bits(c["y1"]))
        assert np.array_equal(bits(orc.matmul(c["x3"], c["w"], qt, None, k, 40, 3)), bits(c["y3"]))


def test_batch_equals_rows_and_bias(orc):
    qt, n, k, m = S.Q4_K, 300, 1024, 5
    w = S.make_weight(qt, n, k, 1)
    x = S.make_activation(m, k, 2, outliers=True)
    yb = orc.matmul(x, w, qt, None, k, n, m)
    for t in range(m):
        assert np.array_equal(bits(orc.matmul(x[t], w, qt, None, k, n, 1)[0]), bits(yb[t]))
    # threaded row split (ThreadPool chunking) does not change a bit
    assert np.array_equal(bits(orc.matmul(x, w, qt, None, k, n, m, threads=7)), bits(yb))


def test_matmul_shape_error(orc):
    with pytest.raises(RuntimeError, match="matmul_quant: in_dim not divisible by block size"):
        orc.matmul(np.zeros(100, np.float32), np.zeros(1000, np.uint8), S.Q4_K, None, 100, 2, 1)
    with pytest.raises(RuntimeError, match="matmul_quant_batch: in_dim not divisible by block size"):
        orc.matmul(np.zeros((2, 100), np.float32), np.zeros(1000, np.uint8), S.Q8_0, None, 100, 2, 2)


def test_compiled_reference_agrees_when_present(orc):
    ref = O.reference_or_none()
    if ref is None:
        pytest.skip("oracle/_ref/libcllm_ref.so not built (reference tree absent)")
    for qt in TYPES:
        k = 512
        w = S.make_weight(qt, 50, k, 99)
        x = S.make_activation(3, k, 98, outliers=True)
        assert np.array_equal(bits(ref.matmul(x, w, qt, None, k, 50, 3)),
                              bits(orc.matmul(x, w, qt, None, k, 50, 3)))


# ------------------------------------------------------------ types without vec_dot

def _fdot_case(c):
    qt, n, k, m, seed = (int(v) for v in c["meta"])
    w = S.make_weight(qt, n, k, seed)
    x = S.make_activation(m, k, seed + 1, outliers=True)
    bias = np.random.default_rng(seed).standard_normal(n).astype(np.float32)
    return qt, n, k, m, w, x, bias


def test_fdot_oracle_matches_reference_golden(orc):
    cases = split_cases(load_golden("fdot.npz"))
    assert {int(c["meta"][0]) for c in cases.values()} == set(FD_TYPES)
    for tag, c in cases.items():
        qt, n, k, m, w, x, bias = _fdot_case(c)
        assert O_sha(w) == str(c["w_sha"]), f"generator drift for {tag}"
        assert np.array_equal(bits(orc.matmul(x, w, qt, None, k, n, m)), bits(c["y"])), tag
        assert np.array_equal(bits(orc.matmul(x, w, qt, bias, k, n, m, threads=5)),
                              bits(c["ybias"])), tag


def test_fdot_golden_pins_fma_contraction():
    """The reference accumulates acc = fma(x, w, acc) from acc = bias; the same sum with a
    separately rounded product misses the golden bits."""
    c = split_cases(load_golden("fdot.npz"))["F16_64x4096_m1"]
    qt, n, k, m, w, x, bias = _fdot_case(c)
    q, scale, wmin = D.decode(w, qt, n, k)
    wv = (scale * q - wmin).astype(np.float32)
    y = np.zeros(n, np.float32)
    for i in range(k):
        y = (y + x[0, i] * wv[:, i]).astype(np.float32)
    assert not np.array_equal(bits(y), bits(c["y"][0]))
    np.testing.assert_allclose(y, c["y"][0], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("qt", FD_TYPES)
def test_fdot_f64_matches_bruteforce(orc, qt):
    n, k, m = 19, 512, 3
    w = S.make_weight(qt, n, k, 123)
    x = S.make_activation(m, k, 321, outliers=True)
    q, scale, wmin = D.decode(w, qt, n, k)
    want = x.astype(np.float64) @ (scale * q - wmin).T
    got, abs_sum = orc.matmul_f64(x, w, qt, None, k, n, m)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12 * abs_sum.max())
    y32 = orc.matmul(x, w, qt, None, k, n, m)
    err, _, _ = O.rel_err_floored(y32, got, abs_sum)
    assert err < 1e-4


@pytest.mark.parametrize("qt", FD_TYPES)
def test_fdot_batch_equals_rows_and_exact_cases(orc, qt):
    n, k, m = 33, 512, 4
    w = S.make_weight(qt, n, k, 7)
    x = S.make_activation(m, k, 8, outliers=True)
    yb = orc.matmul(x, w, qt, None, k, n, m)
    for t in range(m):
        assert np.array_equal(bits(orc.matmul(x[t], w, qt, None, k, n, 1)[0]), bits(yb[t]))
    # integer activations against integer-valued weights: every product and partial sum is
    # exact, so any order of summation gives the exact integer dot
    q, scale, wmin = D.decode(w, qt, n, k)
    wv = scale * q - wmin
    xi = np.random.default_rng(qt).integers(-3, 4, size=(2, k)).astype(np.float32)
    if qt in (S.F32, S.F16):
        wi = np.round(wv * 64)
        wb = (wi.astype(np.float32) if qt == S.F32 else wi.astype(np.float16)).view(np.uint8).copy()
        want = xi.astype(np.float64) @ wi.T
        assert np.array_equal(orc.matmul(xi, wb.reshape(-1), qt, None, k, n, 2).astype(np.float64),
                              want)


def test_fdot_unknown_type_fails(orc):
    with pytest.raises(RuntimeError, match="unsupported ggml type for dequantize"):
        orc.matmul(np.zeros(64, np.float32), np.zeros(1000, np.uint8), 5, None, 64, 3, 1)


# ------------------------------------------------- producers of the linear layers' inputs

def test_rms_norm_closed_form(orc):
    """Inputs whose squares and running sums are exact in fp32 (multiples of 1/2 up to 8),
    so the sequential sum equals the exact one whatever the contraction; rms and the output
    then follow from single IEEE operations, restated in numpy float32."""
    rng = np.random.default_rng(3)
    n, rows, eps = 896, 3, np.float32(1e-6)
    x = (rng.integers(-16, 17, size=(rows, n)) * 0.5).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    got = orc.rms_norm(x, w, eps)
    for r in range(rows):
        s = np.float32(np.sum(x[r].astype(np.float64) ** 2))      # exact
        rms = np.float32(1.0) / np.sqrt(np.float32(s / np.float32(n)) + eps)
        want = (x[r] * rms).astype(np.float32) * w
        assert np.array_equal(bits(got[r]), bits(want.astype(np.float32)))
    # a plausible slip (mean over n - 1, or eps dropped) changes the bits
    s = np.float32(np.sum(x[0].astype(np.float64) ** 2))
    bad = np.float32(1.0) / np.sqrt(np.float32(s / np.float32(n - 1)) + eps)
    assert not np.array_equal(bits(got[0]), bits((x[0] * bad).astype(np.float32) * w))


def test_rms_norm_general_inputs_close_to_f64(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 4096)).astype(np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(got, want, rtol=2e-6)


def test_swiglu_closed_forms_and_f64(orc):
    g = np.array([0.0, -0.0, 100.0, -100.0, 1.0, -1.0, 20.0, -20.0], np.float32)
    u = np.array([3.0, 3.0, 0.5, 2.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    h = orc.swiglu(g, u)
    assert h[0] == 0.0 and h[2] == 50.0           # silu(0) = 0; exp(-100) is lost in 1 + e
    assert h[3] == 0.0 and np.signbit(h[3])       # -100 / (1 + inf) = -0
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(10000) * 4).astype(np.float32)
    u = rng.standard_normal(10000).astype(np.float32)
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u
    np.testing.assert_allclose(orc.swiglu(g, u), want, rtol=1e-6, atol=1e-30)


# ------------------------------------------------ dequantize_block / dequantize_block_f16

def _deq_cases():
    return split_cases(load_golden("deq.npz"))


def test_dequantize_block_oracle_matches_reference_golden(orc):
    """oracle_dequantize_block / _f16 against the compiled reference's dequantize_block and
    dequantize_block_f16 (src/core/quant.cpp:371-412), bit for bit: thirteen types, n at a
    block boundary and inside the last block, all 65536 binary16 encodings, and fp32 values
    at every case of float_to_half."""
    import hashlib
    for tag, c in _deq_cases().items():
        if "meta" in c:
            qt, n, nb, seed = (int(v) for v in c["meta"])
            w = S.make_weight(qt, 1, nb * S.BLOCK[qt], seed)
            assert hashlib.sha256(w.tobytes()).hexdigest() == str(c["w_sha"]), tag
            src, t = w, qt
        else:
            src = c["src"].view(np.uint8)
            t = S.F16 if tag.startswith("f16") else S.F32
            n = c["src"].size
        y = orc.dequantize_block(src, t, n)
        assert np.array_equal(y.view(np.uint32), c["y"].view(np.uint32)), tag
        assert np.array_equal(orc.dequantize_block_f16(src, t, n), c["y16"]), tag


def test_float_to_half_closed_forms(orc):
    """Pins oracle_float_to_half by what the rule fixes: every binary16 value converts back
    to itself; normal results truncate (the next float below 2^k(1 + 2^-10) keeps 2^k);
    subnormal results round to nearest with ties to even; overflow and NaN; and, for
    the quantized blocks, the f16 output is float_to_half of the fp32 output."""
    h = np.arange(65536, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(f)
    assert np.array_equal(orc.float_to_half(f[finite]), h[finite])
    one_minus = np.nextafter(np.float32(1.0 + 2 ** -10), np.float32(0))
    assert orc.float_to_half(np.array([one_minus], np.float32))[0] == 0x3C00  # truncated
    tiny = np.float32(2.0 ** -24)  # binary16's smallest subnormal
    got = orc.float_to_half(np.array([tiny * 0.5, tiny * 1.5, tiny * 2.5, tiny * 0.75], np.float32))
    assert list(got) == [0x0000, 0x0002, 0x0002, 0x0001]  # ties to even, 0.75 rounds up
    big = orc.float_to_half(np.array([65520.0, 1e30, -np.inf, np.nan], np.float32))
    assert list(big) == [0x7BFF, 0x7C00, 0xFC00, 0x7E00]
    for tag, c in _deq_cases().items():
        if "meta" in c:
            assert np.array_equal(orc.float_to_half(c["y"]), c["y16"]), tag


def test_dequantize_block_partial_equals_prefix(orc):
    """A partial last block yields the prefix of the whole block's values (the reference
    guards its stores with < n and reads the block whole)."""
    for qt in ALL_TYPES:
        bs = S.BLOCK[qt]
        w = S.make_weight(qt, 1, 2 * max(bs, 32), 31 + qt)
        full = orc.dequantize_block(w, qt, 2 * max(bs, 32))
        for n in (1, max(bs, 32) + 5, 2 * max(bs, 32) - 1):
            assert np.array_equal(orc.dequantize_block(w, qt, n).view(np.uint32),
                                  full[:n].view(np.uint32)), (qt, n)


def test_quantization_rounds_the_product_before_the_magic_add():
    """Inputs whose every 32-element block holds a value with fl(x * id) on a tie that the
    exact product x * id does not sit on: the oracle's quants are rint(fl(x * id)) (the
    reference's (int)nearbyint(x[i] * id), quant.cpp:444) and differ from the rounding of the
    exact product -- what a fused multiply-add computes -- in every block, so the device tests
    on this input catch a contracted rounding."""
    x = S.rounding_boundary_activation(4, 1024, 3)
    qs, sc, _ = O.oracle().quantize(x)
    f32 = np.float32
    for t in range(4):
        for b in range(1024 // 32):
            e = x[t, 32 * b: 32 * b + 32]
            inv = f32(f32(1.0) / sc[t, b])
            sep = np.rint((e * inv).astype(np.float32).astype(np.float64)).astype(np.int64)
            fused = np.rint(e.astype(np.float64) * np.float64(inv)).astype(np.int64)
            assert np.array_equal(qs[t, 32 * b: 32 * b + 32], sep)
            assert (sep != fused).sum() == 1, (t, b)
