"""GPU parity of the fused producers of a device-resident layer: RMSNorm and SwiGLU, each
fused with the Q8_0 quantization matmul_quant applies to its input, and the residual add.

Bars (written into each test):
  - h (fp32) against the reference's arithmetic (the oracle's restatement of
    rms_norm_ptr / silu, src/core/engine.cpp:23-28, 38): within 2e-6 relative, and never
    further from the fp64 value than the reference's own h is, plus 4 ulp (the sum of
    squares is reduced in parallel rather than sequentially; silu uses the device's expf);
  - the Q8_0 blocks equal quantize_row_q8_0 of the GPU's own h, bit for bit;
  - against quantize_row_q8_0 of the reference's h, codes differ only at rounding
    boundaries: by at most 1, in under 0.1 % of the elements;
  - a whole decode sub-layer (RMSNorm -> Q8_0 -> GEMV) meets the GEMV's own 1e-4 bar
    against the reference's matmul_quant of the reference's h.
"""
import numpy as np
import pytest

from cllm_inference_amd import synth as S
from test_gpu_parity import bits, check_close, _dev

pytestmark = pytest.mark.gpu


def _check_h(got, ref, exact, what):
    got = np.asarray(got, np.float64)
    ref32 = np.asarray(ref, np.float32)
    ref = ref32.astype(np.float64)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 2e-6, f"{what}: {rel.max():.3g} relative to the reference"
    ulp = np.spacing(np.abs(ref32)).astype(np.float64)
    excess = np.abs(got - exact) - (np.abs(ref - exact) + 4 * ulp)
    assert excess.max() <= 0, f"{what}: further from fp64 than the reference + 4 ulp"


def _check_q8(gpu, orc, h_gpu, h_ref, qs, sc, bs, what):
    n = h_gpu.shape[1]
    q_own, s_own, b_own = orc.quantize(h_gpu)
    assert np.array_equal(qs, q_own), what
    assert np.array_equal(bits(sc), bits(s_own)), what
    assert np.array_equal(bs, b_own), what
    q_ref, _, _ = orc.quantize(h_ref)
    diff = qs.astype(np.int32) - q_ref.astype(np.int32)
    assert np.abs(diff).max() <= 1, what
    assert np.count_nonzero(diff) <= max(1, int(1e-3 * diff.size)), what


@pytest.mark.parametrize("n,m", [(896, 1), (4096, 1), (4096, 5), (14336, 2), (5120, 3)])
def test_rmsnorm_q8_0(gpu, orc, n, m):
    rng = np.random.default_rng(n + m)
    x = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    w = (1 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    eps = 1e-5
    print("rmsnorm", n, m, flush=True)
    h, qs, sc, bs = gpu.rmsnorm_q8_0_dev(_dev(x), _dev(w), eps)
    h = h.cpu().numpy()
    h_ref = orc.rms_norm(x, w, eps)
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt((x64 ** 2).sum(axis=1, keepdims=True) / n + eps) * w
    _check_h(h, h_ref, exact, f"rmsnorm {n}x{m}")
    _check_q8(gpu, orc, h, h_ref, qs.cpu().numpy(), sc.cpu().numpy(), bs.cpu().numpy(),
              f"rmsnorm {n}x{m}")
    # h alone, and the Q8_0 blocks alone, are the same values
    h2, _, _, _ = gpu.rmsnorm_q8_0_dev(_dev(x), _dev(w), eps, quantize=False)
    _, qs2, _, _ = gpu.rmsnorm_q8_0_dev(_dev(x), _dev(w), eps, h=False)
    assert np.array_equal(bits(h2.cpu().numpy()), bits(h))
    assert np.array_equal(qs2.cpu().numpy(), qs.cpu().numpy())


@pytest.mark.parametrize("n,m", [(14336, 1), (14336, 3), (4864, 2), (96, 7)])
def test_swiglu_q8_0(gpu, orc, n, m):
    rng = np.random.default_rng(7 * n + m)
    g = (rng.standard_normal((m, n)) * 3).astype(np.float32)
    u = rng.standard_normal((m, n)).astype(np.float32)
    g[0, :4] = [0.0, 100.0, -100.0, -0.0]
    print("swiglu", n, m, flush=True)
    h, qs, sc, bs = gpu.swiglu_q8_0_dev(_dev(g), _dev(u))
    h = h.cpu().numpy()
    h_ref = orc.swiglu(g, u)
    g64 = g.astype(np.float64)
    with np.errstate(over="ignore"):
        exact = g64 / (1 + np.exp(-g64)) * u
    _check_h(h, h_ref, exact, f"swiglu {n}x{m}")
    assert h[0, 1] == h_ref[0, 1] and np.signbit(h[0, 2]) == np.signbit(h_ref[0, 2])
    _check_q8(gpu, orc, h, h_ref, qs.cpu().numpy(), sc.cpu().numpy(), bs.cpu().numpy(),
              f"swiglu {n}x{m}")


def test_add(gpu):
    rng = np.random.default_rng(9)
    for n in (4096, 4099, 3):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        ad = _dev(a)
        gpu.add_dev(ad, _dev(b))
        assert np.array_equal(bits(ad.cpu().numpy()), bits((a + b).astype(np.float32)))


@pytest.mark.parametrize("qt", [S.Q4_K, S.Q6_K, S.Q8_0])
def test_rmsnorm_then_gemv_meets_the_gemv_bar(gpu, orc, qt):
    """RMSNorm -> Q8_0 -> GEMV on device against the reference's rms_norm then matmul_quant."""
    n_out, k = 1024, 4096
    rng = np.random.default_rng(qt)
    x = (rng.standard_normal((1, k)) * 2).astype(np.float32)
    wn = (1 + 0.2 * rng.standard_normal(k)).astype(np.float32)
    w = S.make_weight(qt, n_out, k, 11)
    _, qs, sc, bs = gpu.rmsnorm_q8_0_dev(_dev(x), _dev(wn), 1e-5, h=False)
    y = gpu.gemv_q8_dev(_dev(w), qt, k, n_out, qs, sc, bs).cpu().numpy()
    h_ref = orc.rms_norm(x, wn, 1e-5)
    yo = orc.matmul(h_ref, w, qt, None, k, n_out, 1).reshape(1, n_out)
    exact, abs_sum = orc.matmul_f64(h_ref, w, qt, None, k, n_out, 1)
    check_close(y, yo, exact, abs_sum, f"rmsnorm+gemv {S.TYPE_NAMES[qt]}")


def test_producer_argument_errors(gpu):
    import torch
    x = torch.zeros((1, 48), dtype=torch.float32, device="cuda")
    w = torch.zeros(48, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="quantize_row_q8_0: n not divisible by 32"):
        gpu.rmsnorm_q8_0_dev(x, w, 1e-5)
    h, _, _, _ = gpu.rmsnorm_q8_0_dev(x, w, 1e-5, quantize=False)  # fp32 output is fine
    assert h.shape == (1, 48)
    with pytest.raises(RuntimeError, match="misaligned"):
        gpu.add_dev(torch.zeros(9, device="cuda")[1:], torch.zeros(8, device="cuda"))


@pytest.mark.parametrize("qt", [S.Q4_K, S.Q6_K, S.Q5_0])
def test_gemv_residual_equals_gemv_then_add(gpu, qt):
    """y += W a (+ b) in one launch gives the bits of the separate matmul and add."""
    import torch
    n_out, k, m = 4096, 4096, 3
    rng = np.random.default_rng(qt + 100)
    w = _dev(S.make_weight(qt, n_out, k, 12))
    a = _dev(S.make_activation(m, k, 13))
    bias = _dev(rng.standard_normal(n_out).astype(np.float32))
    resid = rng.standard_normal((m, n_out)).astype(np.float32)
    qs, sc, bs = gpu.quantize_q8_0_dev(a)
    mm = gpu.gemv_q8_dev(w, qt, k, n_out, qs, sc, bs, bias=bias).cpu().numpy()
    y = _dev(resid)
    gpu.gemv_q8_residual_dev(w, qt, k, n_out, qs, sc, bs, y, bias=bias)
    assert np.array_equal(bits(y.cpu().numpy()), bits((resid + mm).astype(np.float32)))
    torch.cuda.synchronize()


@pytest.mark.parametrize("qt", [S.Q4_K, S.Q6_K, S.Q8_0])
def test_gemv_multi_equals_separate_launches(gpu, qt):
    """q/k/v (and gate/up) in one launch give the bits of one launch per matrix."""
    rng = np.random.default_rng(qt + 200)
    k, m = 4096, 2
    dims = [4096, 1024, 1000]
    ws = [_dev(S.make_weight(qt, n, k, 20 + i)) for i, n in enumerate(dims)]
    biases = [_dev(rng.standard_normal(dims[0]).astype(np.float32)), None,
              _dev(rng.standard_normal(dims[2]).astype(np.float32))]
    qs, sc, bs = gpu.quantize_q8_0_dev(_dev(S.make_activation(m, k, 21)))
    for n_mats in (3, 2):
        ys = gpu.gemv_q8_multi_dev(ws[:n_mats], qt, k, dims[:n_mats], qs, sc, bs,
                                   biases=biases[:n_mats])
        for i in range(n_mats):
            one = gpu.gemv_q8_dev(ws[i], qt, k, dims[i], qs, sc, bs, bias=biases[i])
            assert np.array_equal(bits(ys[i].cpu().numpy()), bits(one.cpu().numpy())), (n_mats, i)


@pytest.mark.parametrize("qt,m,n_ff,k", [(S.Q4_K, 1, 14336, 4096), (S.Q4_K, 2, 1000, 4096),
                                         (S.Q6_K, 1, 4096, 4096), (S.Q8_0, 5, 2048, 4096),
                                         (S.Q5_K, 8, 777, 4096), (S.Q4_K, 8, 4200, 14336)])
def test_gemv_swiglu_equals_projections_then_swiglu(gpu, qt, m, n_ff, k):
    """gate, up and silu(gate) * up in one launch give the bits of the two projections in one
    launch followed by the SwiGLU producer (ragged row counts, several activation rows, and
    rows of several 64-unit items streamed through the two-deep ring included), with and
    without biases."""
    rng = np.random.default_rng(qt + 400 + m)
    wg = _dev(S.make_weight(qt, n_ff, k, 40))
    wu = _dev(S.make_weight(qt, n_ff, k, 41))
    qs, sc, bs = gpu.quantize_q8_0_dev(_dev(S.make_activation(m, k, 42)))
    for with_bias in (False, True):
        bg = _dev(rng.standard_normal(n_ff).astype(np.float32)) if with_bias else None
        bu = _dev(rng.standard_normal(n_ff).astype(np.float32)) if with_bias else None
        print("swiglu gemv", S.TYPE_NAMES[qt], m, n_ff, with_bias, flush=True)
        g, u = gpu.gemv_q8_multi_dev([wg, wu], qt, k, [n_ff, n_ff], qs, sc, bs,
                                     biases=[bg, bu] if with_bias else None)
        h_ref = gpu.swiglu_q8_0_dev(g, u, quantize=False)[0]
        h = gpu.gemv_q8_swiglu_dev(wg, wu, qt, k, n_ff, qs, sc, bs, bias_gate=bg, bias_up=bu)
        assert np.array_equal(bits(h.cpu().numpy()), bits(h_ref.cpu().numpy())), with_bias


@pytest.mark.parametrize("qt,k,dims,with_bias", [
    (S.Q4_K, 4096, (4096, 1024, 1024), False), (S.Q6_K, 2048, (512, 256), False),
    (S.Q8_0, 896, (896, 128, 128), True), (S.Q5_0, 4096, (300,), True),
    (S.Q4_0, 1024, (1000, 24), False), (S.Q5_K, 3072, (3072, 1024, 1024), True),
    # streams long enough for the LDS-staged kernel (40 MB of Q6_K, 99 MB of Q4_K)
    (S.Q6_K, 4096, (12000,), False), (S.Q4_K, 4096, (43000,), True)])
def test_rmsnorm_gemv_equals_rmsnorm_then_gemv(gpu, qt, k, dims, with_bias):
    """The RMSNorm inside the GEMV's staging (q/k/v after attn_norm) gives the bits of the
    RMSNorm producer followed by the GEMV on its Q8_0 rows: the staging reduces the sum of
    squares in the producer's order. Row lengths below 4096 and not a multiple of 256 (the
    producer's idle threads) included, and streams that take the LDS-staged kernel."""
    rng = np.random.default_rng(qt + 500 + k)
    ws = [_dev(S.make_weight(qt, n, k, 50 + i)) for i, n in enumerate(dims)]
    x = _dev((3.0 * rng.standard_normal((1, k))).astype(np.float32))
    nw = _dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    biases = [_dev(rng.standard_normal(n).astype(np.float32)) for n in dims] if with_bias else None
    print("rmsnorm gemv", S.TYPE_NAMES[qt], k, dims, with_bias, flush=True)
    _, qs, sc, bs = gpu.rmsnorm_q8_0_dev(x, nw, 1e-5, h=False)
    ref = gpu.gemv_q8_multi_dev(ws, qt, k, dims, qs, sc, bs, biases=biases)
    got = gpu.rmsnorm_gemv_multi_dev(x, nw, 1e-5, ws, qt, k, dims, biases=biases)
    for g, r in zip(got, ref):
        assert np.array_equal(bits(g.cpu().numpy()), bits(r.cpu().numpy()))


@pytest.mark.parametrize("qt,k,n_ff", [(S.Q4_K, 4096, 14336), (S.Q8_0, 896, 4864),
                                       (S.Q6_K, 1024, 3000)])
def test_rmsnorm_gemv_swiglu_equals_rmsnorm_then_swiglu_gemv(gpu, qt, k, n_ff):
    """ffn_norm, gate, up and their SwiGLU in one launch give the bits of the RMSNorm producer
    followed by the SwiGLU GEMV."""
    rng = np.random.default_rng(qt + 600 + k)
    wg = _dev(S.make_weight(qt, n_ff, k, 60))
    wu = _dev(S.make_weight(qt, n_ff, k, 61))
    x = _dev((0.02 * rng.standard_normal((1, k))).astype(np.float32))
    nw = _dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    print("rmsnorm swiglu gemv", S.TYPE_NAMES[qt], k, n_ff, flush=True)
    _, qs, sc, bs = gpu.rmsnorm_q8_0_dev(x, nw, 1e-6, h=False)
    ref = gpu.gemv_q8_swiglu_dev(wg, wu, qt, k, n_ff, qs, sc, bs)
    got = gpu.rmsnorm_gemv_swiglu_dev(x, nw, 1e-6, wg, wu, qt, k, n_ff)
    assert np.array_equal(bits(got.cpu().numpy()), bits(ref.cpu().numpy()))


def test_rmsnorm_gemv_argument_errors(gpu):
    """Rows longer than 4096, or not a multiple of 32, are refused before any launch."""
    k = 8192
    w = _dev(S.make_weight(S.Q8_0, 64, k, 62))
    x = _dev(np.ones((1, k), np.float32))
    nw = _dev(np.ones(k, np.float32))
    with pytest.raises(Exception, match="rms_norm"):
        gpu.rmsnorm_gemv_multi_dev(x, nw, 1e-5, [w], S.Q8_0, k, [64])
    with pytest.raises(Exception, match="rms_norm"):
        gpu.rmsnorm_gemv_swiglu_dev(x, nw, 1e-5, w, w, S.Q8_0, k, 64)


@pytest.mark.parametrize("qt,m", [(S.Q4_K, 1), (S.Q6_K, 2), (S.Q8_0, 5), (S.Q4_K, 20), (S.F16, 1),
                                  (S.Q3_K, 3)])
def test_matmul_residual_equals_matmul_then_add(gpu, qt, m):
    """y += matmul(x) in the fused GEMV (small batches of vec_dot types) or with a separate
    add (float-dot types, MFMA batches) gives the bits of the matmul and the add."""
    n_out, k = 1024, 4096
    rng = np.random.default_rng(qt + 300 + m)
    w = _dev(S.make_weight(qt, n_out, k, 14))
    x = _dev(S.make_activation(m, k, 15))
    bias = _dev(rng.standard_normal(n_out).astype(np.float32))
    resid = rng.standard_normal((m, n_out)).astype(np.float32)
    mm = gpu.matmul_quant_dev(x, w, qt, bias, k, n_out).cpu().numpy()
    y = _dev(resid)
    gpu.matmul_quant_residual_dev(x, w, qt, bias, k, n_out, y)
    assert np.array_equal(bits(y.cpu().numpy()), bits((resid + mm).astype(np.float32)))
