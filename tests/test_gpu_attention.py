"""GPU checks of the float ops between the linear layers: NEOX RoPE and grouped-query
attention over a KV cache (src/core/engine.cpp:41-56, 114-146).

Bars: RoPE within 4 ulp of the reference's formula evaluated in float64 from the same
fp32 inputs (the device's powf / cosf / sinf are within an ulp or two); attention within
2e-6 of |out|_max per head against float64 softmax attention (the summation order differs:
chunked online softmax, sequence splits, the fp32 MFMA kernel's 16-position steps and
position quarters); closed forms: one position gives v_0 exactly, equal keys give the mean
of the values. Both attention kernels (the split kernel, the many-row MFMA kernel) run every
prefill case, forced through the attention_kernel knob.
"""
import numpy as np
import pytest

from test_gpu_parity import _dev

pytestmark = pytest.mark.gpu


def _rope_ref(x, n_heads, hd, pos0, base):
    x = x.astype(np.float64).reshape(x.shape[0], n_heads, hd)
    half = hd // 2
    i = np.arange(half)
    out = x.copy()
    for t in range(x.shape[0]):
        inv = np.float32(base) ** (np.float32(i) / np.float32(half)).astype(np.float64)
        theta = (pos0 + t) / inv
        c, s = np.cos(theta), np.sin(theta)
        x0, x1 = x[t, :, :half], x[t, :, half:]
        out[t, :, :half] = x0 * c - x1 * s
        out[t, :, half:] = x0 * s + x1 * c
    return out.reshape(x.shape[0], -1)


@pytest.mark.parametrize("hd,heads,rows,pos0,base", [(128, 32, 1, 0, 500000.0),
                                                     (128, 8, 3, 4093, 500000.0),
                                                     (64, 14, 5, 17, 1000000.0),
                                                     (256, 4, 2, 100000, 10000.0)])
def test_rope(gpu, hd, heads, rows, pos0, base):
    rng = np.random.default_rng(hd + rows)
    x = rng.standard_normal((rows, heads * hd)).astype(np.float32)
    xd = _dev(x)
    gpu.rope_neox_dev(xd, heads, hd, pos0, base)
    got = xd.cpu().numpy().astype(np.float64)
    want = _rope_ref(x, heads, hd, pos0, base)
    # the angle (pos / base^(i/half) in fp32) carries a relative error of a few ulp, which
    # at large positions moves cos/sin by |theta| * 2^-23; allow that plus 4 ulp of |x|
    theta_max = (pos0 + rows) * 1.0
    tol = (4 * 2.0 ** -24 + 3 * theta_max * 2.0 ** -24) * np.abs(x).max() * 2
    assert np.abs(got - want).max() <= tol


def _attn_ref(q, kc, vc, pos0, n_head, n_kv, hd):
    rows = q.shape[0]
    q = q.astype(np.float64).reshape(rows, n_head, hd)
    kc = kc.astype(np.float64).reshape(-1, n_kv, hd)
    vc = vc.astype(np.float64).reshape(-1, n_kv, hd)
    rep = n_head // n_kv
    out = np.zeros((rows, n_head, hd))
    for t in range(rows):
        L = pos0 + t + 1
        for h in range(n_head):
            s = kc[:L, h // rep] @ q[t, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ vc[:L, h // rep]
    return out.reshape(rows, -1)


@pytest.mark.parametrize("hd,n_head,n_kv,rows,pos0", [(128, 32, 8, 1, 0), (128, 32, 8, 1, 4095),
                                                      (128, 32, 8, 1, 1500),
                                                      (128, 32, 8, 7, 300), (64, 14, 2, 1, 1000),
                                                      (64, 16, 16, 33, 0), (256, 8, 1, 2, 129),
                                                      (128, 40, 8, 64, 64)])
def test_attention(gpu, hd, n_head, n_kv, rows, pos0):
    rng = np.random.default_rng(hd * 7 + rows + pos0)
    L = pos0 + rows
    q = rng.standard_normal((rows, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    vc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    print("attention", hd, n_head, n_kv, rows, pos0, flush=True)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), pos0, n_head, n_kv, hd).cpu().numpy()
    want = _attn_ref(q, kc, vc, pos0, n_head, n_kv, hd)
    err = np.abs(got - want).reshape(rows, n_head, hd).max(axis=2)
    scale = np.abs(want).reshape(rows, n_head, hd).max(axis=2)
    assert (err <= 2e-6 * np.maximum(scale, 1e-3)).all(), err.max()


# prefill shapes: Llama-3-8B heads at 512 rows, ragged row counts (blocks of 4 / 8 / 16 / 32
# rows per workgroup half), a cache ahead of the batch, every GQA ratio 1..8 (3, 5, 6, 7 leave
# columns of a block unused), one row and a few rows
PREFILL_CASES = [(128, 32, 8, 512, 0), (128, 32, 8, 100, 37), (64, 16, 16, 33, 0),
                 (256, 8, 1, 70, 129), (128, 40, 8, 64, 64), (64, 14, 2, 45, 1000),
                 (128, 24, 8, 19, 5), (128, 12, 2, 130, 0), (128, 32, 8, 1, 300),
                 (128, 32, 8, 7, 300), (128, 64, 8, 48, 2000), (256, 16, 2, 9, 0),
                 (64, 32, 4, 200, 3)]


@pytest.mark.parametrize("kernel", [1, 2], ids=["split", "mfma"])
@pytest.mark.parametrize("hd,n_head,n_kv,rows,pos0", PREFILL_CASES)
def test_attention_prefill_both_kernels(gpu, kernel, hd, n_head, n_kv, rows, pos0):
    rng = np.random.default_rng(hd * 11 + n_head + rows + pos0)
    L = pos0 + rows
    q = rng.standard_normal((rows, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    vc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    print("attention kernel", kernel, hd, n_head, n_kv, rows, pos0, flush=True)
    gpu.tune("attention_kernel", kernel)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), pos0, n_head, n_kv, hd).cpu().numpy()
    want = _attn_ref(q, kc, vc, pos0, n_head, n_kv, hd)
    err = np.abs(got - want).reshape(rows, n_head, hd).max(axis=2)
    scale = np.abs(want).reshape(rows, n_head, hd).max(axis=2)
    assert (err <= 2e-6 * np.maximum(scale, 1e-3)).all(), err.max()


def test_attention_mfma_closed_forms(gpu):
    """The MFMA kernel: one position returns v_0 bit for bit (one probability of exactly 1,
    one sum of 1); equal keys over a long causal batch give each row the mean of the values it
    sees."""
    rng = np.random.default_rng(5)
    hd, n_head, n_kv = 128, 8, 2
    gpu.tune("attention_kernel", 2)
    q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((1, n_kv * hd)).astype(np.float32)
    vc = rng.standard_normal((1, n_kv * hd)).astype(np.float32)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), 0, n_head, n_kv, hd).cpu().numpy()
    want = np.repeat(vc.reshape(n_kv, hd), n_head // n_kv, axis=0).reshape(1, -1)
    assert np.array_equal(got, want)
    rows, pos0 = 96, 300
    L = pos0 + rows
    q = rng.standard_normal((rows, n_head * hd)).astype(np.float32)
    kc = np.tile(rng.standard_normal((1, n_kv * hd)).astype(np.float32), (L, 1))
    vc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), pos0, n_head, n_kv, hd).cpu().numpy()
    csum = np.cumsum(vc.astype(np.float64).reshape(L, n_kv, hd), axis=0)
    for t in range(rows):
        mean = csum[pos0 + t] / (pos0 + t + 1)
        want = np.repeat(mean, n_head // n_kv, axis=0).reshape(-1)
        assert np.abs(got[t] - want).max() <= 1e-6, t


@pytest.mark.parametrize("hd,n_head,n_kv,pos0,base", [(128, 32, 8, 1024, 500000.0),
                                                      (128, 32, 8, 0, 500000.0),
                                                      (64, 14, 2, 63, 1000000.0),
                                                      (256, 8, 1, 200, 10000.0),
                                                      (128, 40, 8, 4095, 1000000.0)])
def test_attention_rope_equals_rope_then_attention(gpu, hd, n_head, n_kv, pos0, base):
    """RoPE fused into the decode attention: the output and the rotated key row equal, bit for
    bit, the rotation of the queries and the key row followed by the attention; q stays as it
    was and no other cache row changes."""
    rng = np.random.default_rng(hd + n_head + pos0)
    L = pos0 + 1
    q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((L + 3, n_kv * hd)).astype(np.float32)
    vc = rng.standard_normal((L + 3, n_kv * hd)).astype(np.float32)
    print("attention+rope", hd, n_head, n_kv, pos0, flush=True)
    qa, ka = _dev(q), _dev(kc)
    gpu.rope_neox2_dev(qa, n_head, ka[pos0:pos0 + 1], n_kv, hd, pos0, base)
    want = gpu.attention_dev(qa, ka, _dev(vc), pos0, n_head, n_kv, hd).cpu().numpy()
    qb, kb = _dev(q), _dev(kc)
    got = gpu.attention_rope_dev(qb, kb, _dev(vc), pos0, n_head, n_kv, hd, base).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    kb_h, ka_h = kb.cpu().numpy(), ka.cpu().numpy()
    assert np.array_equal(kb_h.view(np.uint32), ka_h.view(np.uint32))
    assert np.array_equal(qb.cpu().numpy().view(np.uint32), q.view(np.uint32))


def test_attention_closed_forms(gpu):
    rng = np.random.default_rng(1)
    hd, n_head, n_kv = 128, 8, 2
    # one position: every head returns its KV head's v_0, bit for bit
    q = rng.standard_normal((1, n_head * hd)).astype(np.float32)
    kc = rng.standard_normal((1, n_kv * hd)).astype(np.float32)
    vc = rng.standard_normal((1, n_kv * hd)).astype(np.float32)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), 0, n_head, n_kv, hd).cpu().numpy()
    want = np.repeat(vc.reshape(n_kv, hd), n_head // n_kv, axis=0).reshape(1, -1)
    assert np.array_equal(got, want)
    # equal keys: uniform weights, the mean of the values
    L = 1000
    kc = np.tile(rng.standard_normal((1, n_kv * hd)).astype(np.float32), (L, 1))
    vc = rng.standard_normal((L, n_kv * hd)).astype(np.float32)
    got = gpu.attention_dev(_dev(q), _dev(kc), _dev(vc), L - 1, n_head, n_kv, hd).cpu().numpy()
    mean = vc.astype(np.float64).reshape(L, n_kv, hd).mean(axis=0)
    want = np.repeat(mean, n_head // n_kv, axis=0).reshape(1, -1)
    assert np.abs(got - want).max() <= 1e-6


def test_attention_argument_errors(gpu):
    import torch
    q = torch.zeros((1, 8 * 96), device="cuda")
    with pytest.raises(RuntimeError, match="head_dim must be 64, 128 or 256"):
        gpu.attention_dev(q, q, q, 0, 8, 2, 96)
    q = torch.zeros((1, 32 * 128), device="cuda")
    with pytest.raises(RuntimeError, match="at most 8 query heads"):
        gpu.attention_dev(q, q, q, 0, 32, 2, 128)
    q = torch.zeros((1, 32 * 128), device="cuda")
    kv = torch.zeros((4, 8 * 128), device="cuda")
    for bad in (0.0, -10000.0, float("nan")):
        with pytest.raises(RuntimeError, match="theta_base must be positive"):
            gpu.attention_rope_dev(q, kv, kv, 3, 32, 8, 128, bad)
    with pytest.raises(RuntimeError, match="head_dim must be 64, 128 or 256"):
        gpu.attention_rope_dev(q, kv, kv, 3, 32, 8, 96, 10000.0)
