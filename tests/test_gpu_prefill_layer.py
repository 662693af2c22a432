"""The prefill linear layer on the device (the prefill half of the device-resident path):
producers that write the weight-row MFMA kernels' activation format once per input, and the
q/k/v and gate/up projections each in one weight-row launch on it (src/core/engine.cpp:556-597,
where every mm_batch quantizes its input again).

Bars: the producers' format equal bit for bit to quantizing their own fp32 output (the same
Q8_0 arithmetic, quantize_row_q8_0); the matmuls within check_close (test_gpu_parity.py) of
the oracle on sampled activation rows at the Llama-3-8B Q4_K_M layer's full sizes, M = 512;
and the whole linear layer (RMSNorm, q/k/v, wo and its residual add, RMSNorm, gate/up, SwiGLU,
down and its residual add) step by step against the oracle on sampled rows.
"""
import numpy as np
import pytest

from cllm_inference_amd import synth as S
from test_gpu_parity import bits, check_close, _dev

pytestmark = pytest.mark.gpu

CFG = "c3_q4_k_m_layer"
M = 512
EPS = 1e-5


def _mat(label):
    qt, n, k, w = S.config_weight(CFG, label)
    return qt, n, k, w


def _norm_weight(k, seed):
    return np.random.default_rng(seed).uniform(0.5, 1.5, k).astype(np.float32)


def test_producers_write_the_format_of_their_own_output(gpu):
    """RMSNorm and SwiGLU into the format equal, bit for bit, their fp32 output (as the Q8_0
    producers write it) quantized into the format by the plain quantizer."""
    import torch
    k, n_ff, m = 4096, 14336, 64
    x = _dev(S.make_activation(m, k, 5, outliers=True))
    nw = _dev(_norm_weight(k, 6))
    h = torch.empty_like(x)
    act = gpu.rmsnorm_mfma_dev(x, nw, EPS, h=h)
    h_ref, _, _, _ = gpu.rmsnorm_q8_0_dev(x, nw, EPS)
    act_ref = gpu.quantize_mfma_dev(h_ref)
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32))
    assert torch.equal(act, act_ref)
    g = _dev(S.make_activation(m, n_ff, 7, outliers=True))
    u = _dev(S.make_activation(m, n_ff, 8, outliers=True))
    hs = torch.empty_like(g)
    act2 = gpu.swiglu_mfma_dev(g, u, h=hs)
    hs_ref, _, _, _ = gpu.swiglu_q8_0_dev(g, u)
    act2_ref = gpu.quantize_mfma_dev(hs_ref)
    torch.cuda.synchronize()
    assert torch.equal(hs.view(torch.int32), hs_ref.view(torch.int32))
    assert torch.equal(act2, act2_ref)
    # and the format's codes and scales are the Q8_0 batch's
    qs, sc, _ = gpu.quantize_q8_0_dev(h_ref)
    n = m * k
    xs = act_ref[: n // 32 * 4].view(torch.float32)
    off = -(-(n // 32 * 4) // 256) * 256
    qh = act_ref[off: off + 2 * n].view(torch.float16)
    assert torch.equal(xs.view(torch.int32), sc.reshape(-1).view(torch.int32))
    assert torch.equal(qh.float(), qs.reshape(-1).float())


@pytest.mark.parametrize("labels", [("wq", "wk", "wv"), ("gate", "up"), ("down",)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_projections_in_one_launch_vs_oracle(gpu, orc, labels, with_bias):
    """q/k/v and gate/up (Q4_K) each in one weight-row launch, down (Q6_K) in its own, at
    M = 512 from one activation format: 8 sampled rows of every output against the oracle."""
    import torch
    mats = [_mat(lb) for lb in labels]
    qt, k = mats[0][0], mats[0][2]
    x = S.config_activation(CFG, M, k)
    ns = [n for _, n, _, _ in mats]
    rng = np.random.default_rng(len(labels))
    biases = [rng.standard_normal(n).astype(np.float32) for n in ns] if with_bias else None
    plan = gpu.matmul_mfma_plan(qt, k, ns, M)
    print("prefill projections", labels, "bias", with_bias, plan, flush=True)
    if len(labels) > 1:
        assert plan.endswith(f"matrices={len(labels)} launches=1"), plan
    act = gpu.quantize_mfma_dev(_dev(x))
    ys = gpu.matmul_mfma_dev([_dev(w) for _, _, _, w in mats], qt, k, ns, act, M,
                             biases=None if biases is None else [_dev(b) for b in biases])
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(11).choice(M, size=8, replace=False))
    for i, (lb, (_, n, _, w)) in enumerate(zip(labels, mats)):
        b = None if biases is None else biases[i]
        yo = orc.matmul(x[rows], w, qt, b, k, n, 8, threads=8)
        exact, abs_sum = orc.matmul_f64(x[rows], w, qt, b, k, n, 8)
        check_close(ys[i].cpu().numpy()[rows], yo, exact, abs_sum, f"{lb} bias={with_bias}")


def test_prefill_linear_layer_vs_oracle_chain(gpu, orc):
    """The layer's linear path at M = 512 with the device producers and fused launches (the
    attention output a given input: the linear path only). On 4 sampled rows every step is
    checked against the oracle fed with the device's own fp32 input to that step: the
    RMSNorms and SwiGLU to the producers' bar (a relative 2e-6: a parallel sum of squares,
    the device's expf), each matmul to check_close, the residual adds exactly."""
    import torch
    k = 4096
    x0 = S.config_activation(CFG, M, k)
    attn = S.make_activation(M, k, 99)
    nw1, nw2 = _norm_weight(k, 1), _norm_weight(k, 2)
    w = {lb: _mat(lb) for lb in ("wq", "wk", "wv", "wo", "gate", "up", "down")}
    wd = {lb: _dev(v[3]) for lb, v in w.items()}
    x = _dev(x0)
    q_dim, kv_dim, n_ff = w["wq"][1], w["wk"][1], w["gate"][1]
    print("prefill layer M", M, flush=True)
    h, h2 = torch.empty_like(x), torch.empty_like(x)
    hs = torch.empty((M, n_ff), dtype=torch.float32, device="cuda")
    # attention half: RMSNorm -> q/k/v (one launch); wo on the attention output, residual add
    act = gpu.rmsnorm_mfma_dev(x, _dev(nw1), EPS, h=h)
    q, kk, v = gpu.matmul_mfma_dev([wd["wq"], wd["wk"], wd["wv"]], S.Q4_K, k,
                                   [q_dim, kv_dim, kv_dim], act, M)
    act_attn = gpu.quantize_mfma_dev(_dev(attn))
    (o,) = gpu.matmul_mfma_dev([wd["wo"]], S.Q4_K, k, [k], act_attn, M)
    gpu.add_dev(x, o)
    x1 = x.clone()
    # feed-forward half: RMSNorm -> gate/up (one launch) -> SwiGLU -> down, residual add
    act2 = gpu.rmsnorm_mfma_dev(x, _dev(nw2), EPS, h=h2)
    g, u = gpu.matmul_mfma_dev([wd["gate"], wd["up"]], S.Q4_K, k, [n_ff, n_ff], act2, M)
    act3 = gpu.swiglu_mfma_dev(g, u, h=hs)
    (d,) = gpu.matmul_mfma_dev([wd["down"]], S.Q6_K, n_ff, [k], act3, M)
    gpu.add_dev(x, d)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(3).choice(M, size=4, replace=False))
    r = len(rows)
    cpu = lambda t: t.cpu().numpy()[rows]  # noqa: E731

    def near(got, ref, what, tol=2e-6):
        ref = ref.astype(np.float64)
        scale = np.maximum(np.abs(ref), tol * np.abs(ref).max())
        err = (np.abs(got.astype(np.float64) - ref) / scale).max()
        assert err <= tol, f"{what}: {err:.3g}"

    def mm(inp, lb, out):
        qt, n, kk_, wb = w[lb]
        yo = orc.matmul(inp, wb, qt, None, kk_, n, r, threads=8)
        exact, abs_sum = orc.matmul_f64(inp, wb, qt, None, kk_, n, r)
        check_close(out, yo, exact, abs_sum, f"layer {lb}")

    near(cpu(h), orc.rms_norm(x0[rows], nw1, EPS), "attn_norm")
    for lb, out in (("wq", q), ("wk", kk), ("wv", v)):
        mm(cpu(h), lb, cpu(out))
    mm(attn[rows], "wo", cpu(o))
    assert np.array_equal(bits(cpu(x1)), bits((x0[rows] + cpu(o)).astype(np.float32)))
    near(cpu(h2), orc.rms_norm(cpu(x1), nw2, EPS), "ffn_norm")
    mm(cpu(h2), "gate", cpu(g))
    mm(cpu(h2), "up", cpu(u))
    near(cpu(hs), orc.swiglu(cpu(g), cpu(u)), "swiglu")
    mm(cpu(hs), "down", cpu(d))
    assert np.array_equal(bits(x.cpu().numpy()[rows]), bits((cpu(x1) + cpu(d)).astype(np.float32)))
