"""Throughput of the quantized linear-layer path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-extra]

Headline workload: Q4_K decode GEMV, Llama-3-8B FFN shape (14336 x 4096, M = 1). A step is
one matmul_quant call on device-resident buffers: fp32 -> Q8_0 activation quantization plus
the GEMV over all 14336 weight rows, fused into one kernel launch. The 33 MB weight fits the 256 MB Infinity Cache, so
steps rotate over enough weight copies (>= 512 MB) that every step reads its weights from
HBM. value = algorithmic bytes per step / step time, with algorithmic bytes =
N*(K/256)*144 + 4*K*M + 4*N*M (weights + fp32 x + fp32 y).

roofline: a step is a single kernel (the GEMV quantizes its activation row in LDS), so its
HIP-event time on the stream it runs on is the kernel's average duration; against 8 TB/s. cpu_baseline: the reference's own quant.cpp +
ThreadPool (compiled from its sources into oracle/_ref) running matmul_quant on the same
workload on this host's cores.

Prints exactly one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5033.0  # 256 CU x 2.4 GHz x 8192 int8 ops / clk / CU (dense)
FP16_PEAK_TFLOPS = 2516.0  # dense fp16 MFMA, the unit the prefill GEMM computes on
FP32_MFMA_PEAK_TFLOPS = 157.3  # dense fp32 MFMA, the unit the many-row attention kernel computes on
ROTATE_BYTES = 512 << 20


def algo_bytes(qt, n, k, m):
    from cllm_inference_amd import synth as S
    return n * S.row_bytes(qt, k) + 4 * k * m + 4 * n * m


def _events():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


WARM_MS = 30.0  # untimed graph replays before timing (--warm-ms)


def time_loop(fn, steps, warmup):
    """Average ms per call of fn(i), i < steps, with launch overhead taken out.

    The `steps` calls are captured once into a HIP graph on a dedicated stream (after
    `warmup` eager calls on that stream, so every per-stream workspace already exists and
    nothing allocates during capture); untimed replays run for at least 30 ms of GPU time,
    then three replays are timed with HIP events, each bracketed by device synchronisation,
    and the median is kept. The 30 ms: after the host-side setup of a workload the first
    ~10 ms of replays ran slower on MI355X (the Q6_K 128256x4096 head: 74.6 us per call in
    the first 50-call replay after one warm replay, 66.6 us after 30 ms, for either kernel).
    """
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(warmup, 1)):
            fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            fn(i)
    a, b = _events()
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    for _ in range(min(200, int(WARM_MS / max(a.elapsed_time(b), 1e-3)))):
        g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(3):
        a, b = _events()
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / steps)
    del g
    return sorted(times)[1]


def rotated_weights(w_np, copies):
    import torch
    base = torch.from_numpy(w_np).cuda()
    return [base] + [base.clone() for _ in range(copies - 1)]


def decode_point(C, S, cfg, label, m, steps, warmup, cold=True, ceiling=False):
    """One decode workload: returns dict with step and GEMV-kernel timings. With ceiling, also
    the one-launch read ceiling of the same weight copies (cllm_hip_read_stream_dev: the
    stream read once, nothing computed)."""
    import torch
    qt, n, k, w = S.config_weight(cfg, label)
    x = torch.from_numpy(S.config_activation(cfg, m, k)).cuda()
    copies = max(2, -(-ROTATE_BYTES // w.size)) if cold else 1
    ws = rotated_weights(w, copies)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    qs, sc, bs = C.quantize_q8_0_dev(x)

    def step(i):
        C.matmul_quant_dev(x, ws[i % copies], qt, None, k, n, y=y)

    def gemv(i):
        C.gemv_q8_dev(ws[i % copies], qt, k, n, qs, sc, bs, None, y=y)

    ms_step = time_loop(step, steps, warmup)
    ms_gemv = time_loop(gemv, steps, warmup)
    ms_read = time_loop(lambda i: C.read_stream_dev(ws[i % copies]), steps, warmup) if ceiling else None
    nbytes = algo_bytes(qt, n, k, m)
    del ws
    torch.cuda.empty_cache()
    print(f"[bench] {S.TYPE_NAMES[qt]} {n}x{k} m={m} copies={copies}: step {ms_step * 1e3:.2f} us, "
          f"gemv {ms_gemv * 1e3:.2f} us, {nbytes / ms_gemv / 1e6:.1f} GB/s", file=sys.stderr, flush=True)
    if ceiling:
        print(f"[bench] one-launch read of the same {w.size} weight bytes: {ms_read * 1e3:.2f} us, "
              f"{w.size / ms_read / 1e6:.1f} GB/s", file=sys.stderr, flush=True)
    return dict(type=S.TYPE_NAMES[qt], n=n, k=k, m=m, copies=copies, bytes=nbytes,
                weight_bytes=int(w.size), ms_step=ms_step, ms_gemv=ms_gemv, ms_read=ms_read,
                gbs_step=nbytes / ms_step / 1e6, gbs_gemv=nbytes / ms_gemv / 1e6,
                route=C.matmul_route(qt, k, n, m), plan=C.matmul_plan(qt, k, n, m))


def host_api_point(C, S, calls=50):
    """c1 through the host-pointer matmul_quant the engine calls (engine.cpp:237-238): x and y in
    host memory, so each call copies x in and y out over PCIe and synchronizes. With the
    weights registered once (cllm_hip_register_weights) they stay in HBM, and so do weights in
    a read-only private file mapping (the engine's mmap'd model) after the first call;
    unregistered anonymous host weights are copied in on every call. Wall-clock medians."""
    import ctypes
    qt, n, k, w = S.config_weight("c1_q4_k_gemv", "ffn")
    x = S.config_activation("c1_q4_k_gemv", 1, k)[0]
    lib = C.load_library()

    def med():
        C.matmul_quant(x, w, qt, None, k, n)
        ts = []
        for _ in range(calls):
            t0 = time.perf_counter()
            C.matmul_quant(x, w, qt, None, k, n)
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    unreg = med()
    assert lib.cllm_hip_register_weights(ctypes.c_void_p(w.ctypes.data), w.size) == 0
    try:
        reg = med()
    finally:
        lib.cllm_hip_unregister_weights(ctypes.c_void_p(w.ctypes.data))
    # the engine's own path (gguf.cpp:178, engine.cpp:237-238): weights inside a PROT_READ /
    # MAP_PRIVATE mapping of the model file, nothing registered. The library copies the
    # mapping to the device on the first call and checks per call that mapping and file are
    # unchanged.
    import mmap
    import tempfile
    fd, path = tempfile.mkstemp(suffix=".bin")
    try:
        os.write(fd, w.tobytes())
        mm = mmap.mmap(fd, w.size, flags=mmap.MAP_PRIVATE, prot=mmap.PROT_READ)
        try:
            w_map = np.frombuffer(mm, dtype=np.uint8)
            auto = med_of(lambda: C.matmul_quant(x, w_map, qt, None, k, n), calls)
            del w_map
        finally:
            mm.close()
    finally:
        os.close(fd)
        os.unlink(path)
    nbytes = algo_bytes(qt, n, k, 1)
    print(f"[bench] host-pointer matmul_quant c1: registered {reg * 1e6:.1f} us, read-only file "
          f"mapping {auto * 1e6:.1f} us, unregistered {unreg * 1e6:.1f} us", file=sys.stderr,
          flush=True)
    return {"registered_us": round(reg * 1e6, 1), "registered_gbs": round(nbytes / reg / 1e9, 1),
            "file_mapping_us": round(auto * 1e6, 1),
            "file_mapping_gbs": round(nbytes / auto / 1e9, 1),
            "file_mapping_over_registered_us": round((auto - reg) * 1e6, 1),
            "unregistered_us": round(unreg * 1e6, 1),
            "unregistered_gbs": round(nbytes / unreg / 1e9, 1), "calls": calls}


def med_of(fn, calls):
    """Median wall-clock seconds of calls calls of fn, after one untimed call."""
    fn()
    ts = []
    for _ in range(calls):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def read_ceiling(p):
    """The one-launch read of a decode point's weight copies, and the fused step against it."""
    wb = p["weight_bytes"]
    return {"us": round(p["ms_read"] * 1e3, 3), "gbs": round(wb / p["ms_read"] / 1e6, 1),
            "frac_hbm": round(wb / p["ms_read"] / 1e6 / HBM_PEAK_GBS, 4),
            "step_over_read": round(p["ms_step"] / p["ms_read"], 3),
            "kernel": "k_read_stream (16-byte nontemporal grid-stride loop, 4 x 512 threads per CU)"}


def m_sweep(C, S, steps, warmup):
    """c4: Q5_K 14336x4096 and Q8_0 4096x4096 at M = 1, 4, 16, 64, 256, cold weights; the
    M = 1 points with the one-launch read ceiling of their weight copies."""
    sweep = {}
    for label in ("q5_k", "q8_0"):
        for m in (1, 4, 16, 64, 256):
            p = decode_point(C, S, "c4_m_sweep", label, m, steps, warmup, cold=True,
                             ceiling=m == 1)
            ops = 2.0 * m * p["n"] * p["k"]
            sweep[f"{label}_m{m}"] = {
                "route": p["route"], "plan": p["plan"], "us": round(p["ms_step"] * 1e3, 2),
                "gbs": round(p["gbs_step"], 1),
                "frac_hbm": round(p["gbs_step"] / HBM_PEAK_GBS, 4),
                "tops": round(ops / p["ms_step"] / 1e9, 2),
                "frac_int8": round(ops / p["ms_step"] / 1e9 / INT8_PEAK_TOPS, 4)}
            if m == 1:
                sweep[f"{label}_m{m}"]["read_ceiling"] = read_ceiling(p)
    return sweep


def float_dot_points(C, S, steps, warmup):
    """The types without vec_dot (float-dot kernels): decode GEMV at the Llama-3-8B FFN shape
    14336 x 4096 for each type, M = 1 and 4, plus an F16 output head of Qwen2.5-0.5B's shape
    (151936 x 896), all with rotating cold weight copies."""
    import torch
    out = {}
    shapes = [(qt, 14336, 4096) for qt in S.FLOAT_DOT_TYPES] + [(S.F16, 151936, 896)]
    for qt, n, k in shapes:
        w = S.make_weight(qt, n, k, 5150 + qt)
        copies = max(2, -(-ROTATE_BYTES // w.size))
        ws = rotated_weights(w, copies)
        for m in (1, 4):
            x = torch.from_numpy(S.make_activation(m, k, 5151)).cuda()
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")

            def step(i):
                C.matmul_quant_dev(x, ws[i % copies], qt, None, k, n, y=y)

            ms = time_loop(step, steps, warmup)
            nbytes = algo_bytes(qt, n, k, m)
            tag = f"{S.TYPE_NAMES[qt]}_{n}x{k}_m{m}"
            out[tag] = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / ms / 1e6, 1),
                        "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                        "route": C.matmul_route(qt, k, n, m)}
            if m == 1:  # the one-launch read of the same weight copies: the step's floor
                ms_read = time_loop(lambda i: C.read_stream_dev(ws[i % copies]), steps, warmup)
                out[tag]["read_ceiling"] = read_ceiling(
                    {"weight_bytes": int(w.size), "ms_read": ms_read, "ms_step": ms})
            print(f"[bench] float-dot {tag}: {ms * 1e3:.2f} us, {nbytes / ms / 1e6:.1f} GB/s",
                  file=sys.stderr, flush=True)
        del ws
        torch.cuda.empty_cache()
    return out


def decode_layer_device(C, S, steps, warmup, copies=4):
    """The linear path of one Llama-3-8B decode layer in the Q4_K_M mix, device-resident:
    RMSNorm+Q8_0 -> one GEMV launch for q/k/v; the wo GEMV quantizing the attention output
    (a fixed synthetic vector: attention itself is measured with the whole model) and adding
    the residual;
    RMSNorm+Q8_0 -> one launch for gate, up and silu(gate) * up -> the down GEMV quantizing h
    and adding the residual (engine.cpp:475-513). Six launches per layer (the residual adds
    ride in the wo and down GEMVs, the SwiGLU in the gate/up GEMV). `copies` distinct
    copies of the layer's weights rotate so that each step streams its weights from HBM, as
    the 32 different layers of a model would."""
    import torch
    cfg = "c3_q4_k_m_layer"
    mats = {label: (qt, n, k) for label, qt, n, k in S.CONFIGS[cfg]["mats"]}
    layers = []
    for c in range(copies):
        layer = {}
        for label in mats:
            _, _, _, w = S.config_weight(cfg, label)
            t = torch.from_numpy(w).cuda()
            layer[label] = t if c == 0 else t.clone()
        layers.append(layer)
    wbytes = sum(layers[0][l].numel() for l in mats)
    n_embd, n_ff = 4096, 14336
    rng = np.random.default_rng(20265)
    x0 = torch.from_numpy(rng.standard_normal((1, n_embd)).astype(np.float32)).cuda()
    x = x0.clone()
    wn1 = torch.from_numpy((1 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)).cuda()
    wn2 = torch.from_numpy((1 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)).cuda()
    attn = torch.from_numpy(rng.standard_normal((1, n_embd)).astype(np.float32)).cuda()
    outs = {l: torch.empty((1, n), dtype=torch.float32, device="cuda")
            for l, (_, n, _) in mats.items()}

    hbuf = torch.empty((1, n_ff), dtype=torch.float32, device="cuda")
    qkv, gu = ("wq", "wk", "wv"), ("gate", "up")
    assert len({mats[l][0] for l in qkv}) == 1 and len({mats[l][0] for l in gu}) == 1

    def step(i):
        L = layers[i % copies]
        qt, _, k = mats["wq"]
        C.rmsnorm_gemv_multi_dev(x, wn1, 1e-5, [L[l] for l in qkv], qt, k,
                                 [mats[l][1] for l in qkv], ys=[outs[l] for l in qkv])
        qt, n, k = mats["wo"]
        C.matmul_quant_residual_dev(attn, L["wo"], qt, None, k, n, x)
        qt, n_g, k = mats["gate"]
        C.rmsnorm_gemv_swiglu_dev(x, wn2, 1e-5, L["gate"], L["up"], qt, k, n_g, h=hbuf)
        qt, n, k = mats["down"]
        C.matmul_quant_residual_dev(hbuf, L["down"], qt, None, k, n, x)

    ms = time_loop(step, steps, warmup)
    x.copy_(x0)
    per = {"layer_us": round(ms * 1e3, 2), "weight_bytes": int(wbytes), "launches": 4,
           "gbs": round(wbytes / ms / 1e6, 1),
           "frac_hbm": round(wbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
           "projected_tokens_per_s_32_layers_linear_only": round(1e3 / (32 * ms), 1),
           "weight_copies_rotated": copies}
    print(f"[bench] device-resident decode layer (linear path): {ms * 1e3:.2f} us, "
          f"{wbytes / ms / 1e6:.1f} GB/s", file=sys.stderr, flush=True)
    del layers
    torch.cuda.empty_cache()
    return per


def decode_model(C, S, steps, warmup, n_layers=4, pos=1024):
    """A whole decode step on the device (embedding lookup, n_layers Llama-3-8B layers in the
    Q4_K_M mix with attention over `pos` cached positions, final norm, Q6_K head of 128256
    rows), from a GGUF file uploaded once; the per-layer figure gives a 32-layer projection.
    Random weights, synthetic cache contents."""
    import tempfile
    import torch
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import device_model as DM
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "llama3_8b_slice.gguf")
        DM.write_model(path, arch="llama", n_layers=n_layers, n_embd=4096, n_head=32, n_kv=8,
                       n_ff=14336, vocab=128256, n_ctx=pos + 8, wtype=S.Q4_K,
                       wtype_down=S.Q6_K, emb_type=S.Q4_K, out_type=S.Q6_K, seed=11)
        m = DM.DeviceModel(path)
    for kc, vc in zip(m.k_cache, m.v_cache):
        kc.normal_()
        vc.normal_()
    ids = torch.tensor([1234], dtype=torch.int32, device="cuda")
    ms = time_loop(lambda i: m.step_ids(ids, pos), steps, warmup)
    head_w = m.t["output.weight"]
    head_bytes = S.row_bytes(head_w.type, 4096) * 128256
    layer_bytes = sum(S.row_bytes(qt, k) * n for _, qt, n, k in S.CONFIGS["c3_q4_k_m_layer"]["mats"])
    kv_bytes = 2 * (pos + 1) * 8 * 128 * 4
    m.close()
    # per layer: the step minus the head GEMV's share (its bytes at the step's mean rate)
    total = n_layers * (layer_bytes + kv_bytes) + head_bytes
    layer_ms = ms * (layer_bytes + kv_bytes) / total
    proj = 32 * layer_ms + ms * head_bytes / total
    out = {"n_layers": n_layers, "kv_positions": pos, "step_us": round(ms * 1e3, 1),
           "gbs": round(total / ms / 1e6, 1), "frac_hbm": round(total / ms / 1e6 / HBM_PEAK_GBS, 4),
           "projected_llama3_8b_32_layer_tokens_per_s": round(1e3 / proj, 1)}
    print(f"[bench] device decode step, {n_layers} layers at position {pos}: {ms * 1e3:.1f} us "
          f"({total / ms / 1e6:.1f} GB/s); 32-layer projection {1e3 / proj:.1f} tokens/s",
          file=sys.stderr, flush=True)
    return out


def prefill_attention(C, steps, warmup, m=512, pos0=0, n_head=32, n_kv=8, head_dim=128):
    """f4 at prefill: a prompt of m rows at positions pos0 .. pos0 + m - 1 in one Llama-3-8B
    layer (32 query heads over 8 KV heads of 128): RoPE of q and of the new key rows, then
    causal grouped-query attention over the cache (engine.cpp:581-586). Synthetic q/k/v.
    Algorithmic work: 2 x 2 x head_dim multiply-adds per (query, head, visible position), for
    q.k and for p.v."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn((m, n_head * head_dim), device="cuda", generator=g)
    kc = torch.randn((pos0 + m, n_kv * head_dim), device="cuda", generator=g)
    vc = torch.randn((pos0 + m, n_kv * head_dim), device="cuda", generator=g)
    out = torch.empty_like(q)
    q0, k0 = q.clone(), kc.clone()

    def step(i):
        q.copy_(q0)
        kc[pos0:].copy_(k0[pos0:])
        C.rope_neox2_dev(q, n_head, kc[pos0:], n_kv, head_dim, pos0, 500000.0)
        C.attention_dev(q, kc, vc, pos0, n_head, n_kv, head_dim, out=out)

    ms_all = time_loop(step, steps, warmup)
    att = lambda i: C.attention_dev(q, kc, vc, pos0, n_head, n_kv, head_dim, out=out)
    ms_att = time_loop(att, steps, warmup)
    C.tune("attention_kernel", 1)  # the sequence-split kernel on the same rows, for comparison
    try:
        ms_split = time_loop(att, steps, warmup)
    finally:
        C.tune("attention_kernel")
    visible = sum(pos0 + t + 1 for t in range(m))
    flop = 2 * 2 * head_dim * visible * n_head
    out_d = {"rows": m, "pos0": pos0, "n_head": n_head, "n_head_kv": n_kv, "head_dim": head_dim,
             "plan": C.attention_plan(m, pos0, n_head, n_kv, head_dim),
             "attention_us": round(ms_att * 1e3, 1), "rope_and_attention_us": round(ms_all * 1e3, 1),
             "split_kernel_us": round(ms_split * 1e3, 1),
             "gflops": round(flop / ms_att / 1e6, 1),
             "frac_fp32_mfma": round(flop / ms_att / 1e9 / FP32_MFMA_PEAK_TFLOPS, 4)}
    print(f"[bench] prefill attention m={m} pos0={pos0} ({out_d['plan']}): {ms_att * 1e3:.1f} us "
          f"({flop / ms_att / 1e6:.1f} GFLOP/s; the split kernel {ms_split * 1e3:.1f} us), with the RoPE "
          f"launch and input copies {ms_all * 1e3:.1f} us", file=sys.stderr, flush=True)
    return out_d


def gguf_upload(C, S, gib=1.0):
    """f2: the GGUF data section's one-time upload (parse, map, pinned double-buffered H2D,
    registration) for a synthetic file of `gib` GiB written to local temporary storage."""
    import tempfile
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_writer as G
    n, k = int(gib * (1 << 30)) // S.row_bytes(S.Q4_K, 4096), 4096
    raw = np.random.default_rng(5).integers(0, 256, size=n * S.row_bytes(S.Q4_K, k),
                                            dtype=np.uint8).tobytes()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "upload.gguf")
        G.write_gguf(path, [("general.architecture", G.STR, "llama")],
                     [("blob.weight", (n, k), S.Q4_K, raw)])
        del raw
        with open(path, "rb") as f:  # page cache warm, as after the engine's own load
            while f.read(64 << 20):
                pass
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            g = C.GgufFile(path, upload=True)
            times.append(time.perf_counter() - t0)
            nbytes = g.config().data_bytes
            g.close()
    t = sorted(times)[1]
    out = {"bytes": int(nbytes), "seconds": round(t, 4), "gbs": round(nbytes / t / 1e9, 2)}
    print(f"[bench] GGUF upload {nbytes / 2**30:.2f} GiB: {t * 1e3:.1f} ms, "
          f"{nbytes / t / 1e9:.2f} GB/s", file=sys.stderr, flush=True)
    return out


def prefill_layer(C, S, steps, warmup):
    """The Llama-3-8B layer in the Q4_K_M mix at M = 512: every matrix timed on its own
    (graph-timed, device-resident inputs), then summed."""
    import torch
    cfg = "c3_q4_k_m_layer"
    per = {}
    total_ms = 0.0
    total_ops = 0.0
    for label, qt, n, k in S.CONFIGS[cfg]["mats"]:
        _, _, _, w = S.config_weight(cfg, label)
        x = torch.from_numpy(S.config_activation(cfg, 512, k)).cuda()
        wd = torch.from_numpy(w).cuda()
        y = torch.empty((512, n), dtype=torch.float32, device="cuda")
        ms = time_loop(lambda i: C.matmul_quant_dev(x, wd, qt, None, k, n, y=y), steps, warmup)
        ops = 2.0 * 512 * n * k
        per[label] = {"type": S.TYPE_NAMES[qt], "n": n, "k": k, "us": round(ms * 1e3, 1),
                      "tops": round(ops / ms / 1e9, 1),
                      "frac_int8": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4),
                      "route": C.matmul_route(qt, k, n, 512), "plan": C.matmul_plan(qt, k, n, 512)}
        print(f"[bench] prefill {label} {S.TYPE_NAMES[qt]} {n}x{k} m=512: {ms * 1e3:.1f} us, "
              f"{ops / ms / 1e9:.1f} TOPS", file=sys.stderr, flush=True)
        total_ms += ms
        total_ops += ops
        del wd, x, y
        torch.cuda.empty_cache()
    return {"layer_us": round(total_ms * 1e3, 1), "tops": round(total_ops / total_ms / 1e9, 1),
            "frac_int8": round(total_ops / total_ms / 1e9 / INT8_PEAK_TOPS, 4),
            "frac_fp16_mfma": round(total_ops / total_ms / 1e9 / FP16_PEAK_TFLOPS, 4),
            "tokens_per_s_per_layer": round(512 / (total_ms * 1e-3), 0),
            "llama3_8b_32_layer_projection_tokens_per_s": round(512 / (32 * total_ms * 1e-3), 0),
            "matrices": per}


def prefill_layer_device(C, S, steps, warmup, c3=None):
    """The linear path of the same layer at M = 512 on the device, as one step: RMSNorm into
    the weight-row activation format -> q/k/v in one launch; the attention output (a fixed
    synthetic input: attention is not on the linear path) quantized into the format -> wo ->
    residual add; RMSNorm into the format -> gate/up in one launch -> SwiGLU into the format
    -> down -> residual add (engine.cpp:556-597): 10 launches, 4 quantizations, against the
    14 launches and 7 quantizations of the matrices one by one (c3). Graph-timed."""
    import torch
    cfg = "c3_q4_k_m_layer"
    m = 512
    mats = {label: (qt, n, k) for label, qt, n, k in S.CONFIGS[cfg]["mats"]}
    wd = {label: torch.from_numpy(S.config_weight(cfg, label)[3]).cuda() for label in mats}
    n_embd, n_ff = 4096, 14336
    rng = np.random.default_rng(20266)
    x = torch.from_numpy(S.config_activation(cfg, m, n_embd)).cuda()
    attn = torch.from_numpy(rng.standard_normal((m, n_embd)).astype(np.float32)).cuda()
    wn1 = torch.from_numpy((1 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)).cuda()
    wn2 = torch.from_numpy((1 + 0.1 * rng.standard_normal(n_embd)).astype(np.float32)).cuda()
    out = {l: torch.empty((m, n), dtype=torch.float32, device="cuda") for l, (_, n, _) in mats.items()}
    act1, act2 = C.mfma_act_new(n_embd, m), C.mfma_act_new(n_embd, m)
    act3, act4 = C.mfma_act_new(n_embd, m), C.mfma_act_new(n_ff, m)
    qkv, gu = ("wq", "wk", "wv"), ("gate", "up")
    qt = mats["wq"][0]
    assert {mats[l][0] for l in qkv + gu + ("wo",)} == {qt}

    def run_qkv():
        C.matmul_mfma_dev([wd[l] for l in qkv], qt, n_embd, [mats[l][1] for l in qkv], act1, m,
                          ys=[out[l] for l in qkv])

    def run_gu():
        C.matmul_mfma_dev([wd[l] for l in gu], qt, n_embd, [n_ff, n_ff], act3, m,
                          ys=[out[l] for l in gu])

    def step(i):
        C.rmsnorm_mfma_dev(x, wn1, 1e-5, act=act1)
        run_qkv()
        C.quantize_mfma_dev(attn, act=act2)
        C.matmul_mfma_dev([wd["wo"]], qt, n_embd, [n_embd], act2, m, ys=[out["wo"]])
        C.add_dev(x, out["wo"])
        C.rmsnorm_mfma_dev(x, wn2, 1e-5, act=act3)
        run_gu()
        C.swiglu_mfma_dev(out["gate"], out["up"], act=act4)
        C.matmul_mfma_dev([wd["down"]], mats["down"][0], n_ff, [n_embd], act4, m, ys=[out["down"]])
        C.add_dev(x, out["down"])

    ms = time_loop(step, steps, warmup)
    ms_qkv = time_loop(lambda i: run_qkv(), steps, warmup)
    ms_gu = time_loop(lambda i: run_gu(), steps, warmup)
    ops = sum(2.0 * m * n * k for (_, n, k) in mats.values())
    res = {"layer_us": round(ms * 1e3, 1), "tops": round(ops / ms / 1e9, 1),
           "frac_int8": round(ops / ms / 1e9 / INT8_PEAK_TOPS, 4),
           "frac_fp16_mfma": round(ops / ms / 1e9 / FP16_PEAK_TFLOPS, 4),
           "launches": 10, "activation_quantizations": 4,
           "qkv_one_launch_us": round(ms_qkv * 1e3, 1),
           "qkv_plan": C.matmul_mfma_plan(qt, n_embd, [mats[l][1] for l in qkv], m),
           "gate_up_one_launch_us": round(ms_gu * 1e3, 1),
           "gate_up_plan": C.matmul_mfma_plan(qt, n_embd, [n_ff, n_ff], m),
           "tokens_per_s_per_layer": round(m / (ms * 1e-3), 0)}
    if c3 is not None:
        mt = c3["matrices"]
        res["c3_layer_us"] = c3["layer_us"]
        res["c3_qkv_us"] = round(sum(mt[l]["us"] for l in qkv), 1)
        res["c3_gate_up_us"] = round(sum(mt[l]["us"] for l in gu), 1)
    print(f"[bench] device prefill layer m=512: {ms * 1e3:.1f} us ({ops / ms / 1e9:.1f} TOPS); "
          f"q/k/v in one launch {ms_qkv * 1e3:.1f} us, gate/up {ms_gu * 1e3:.1f} us",
          file=sys.stderr, flush=True)
    del wd, x, attn, out
    torch.cuda.empty_cache()
    return res


def cpu_share():
    """CPUs this process may run on: its affinity set, capped by a cgroup v2 CPU quota."""
    n = len(os.sched_getaffinity(0))
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()
        if quota != "max":
            n = min(n, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    return n


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_call(fn, cap_s, least=3):
    """Median seconds of fn(): 3 warm-up calls (1 if a call is long), then timed calls until 10
    have run or cap_s has passed (at least `least`)."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    for _ in range(2 if first * 4 < cap_s else 0):
        fn()
    times = []
    t_end = time.perf_counter() + cap_s
    while len(times) < least or (len(times) < 10 and time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(S, seconds=30.0):
    """The reference's matmul_quant / matmul_quant_batch (AVX2 + its ThreadPool, compiled from
    its sources into oracle/_ref; the oracle's C restatement if that is absent) on this host,
    on the same seeded workloads as the GPU figures, activation quantization included. Threads
    = the CPUs this job may use (the reference's ThreadPool(0) takes hardware_concurrency();
    on a host whose job share is smaller, more threads than the share only time-slice). Each
    point is bounded to a share of `seconds`; c1 also runs on one thread."""
    import oracle
    lib, kind = oracle.reference_or_none(), "reference"
    if lib is None:
        lib, kind = oracle.Oracle(), "port"
    threads = cpu_share()
    points = [("c1_q4_k_gemv", "ffn", 1), ("c0_q8_0_gemv", "w", 1), ("c2_q6_k_head", "output", 1)]
    points += [("c4_m_sweep", lab, m) for lab in ("q5_k", "q8_0") for m in (1, 4, 16, 64, 256)]
    cap = seconds / (len(points) + 4)
    out, head, samples = {}, None, 0
    for cfg, label, m in points:
        qt, n, k, w = S.config_weight(cfg, label)
        x = S.config_activation(cfg, m, k)
        sec, calls = _median_call(lambda: lib.matmul(x, w, qt, None, k, n, m, threads=threads), cap)
        samples += calls
        nbytes = algo_bytes(qt, n, k, m)
        tag = f"{cfg}_{label}_m{m}" if cfg == "c4_m_sweep" else cfg
        rec = {"type": S.TYPE_NAMES[qt], "n": n, "k": k, "m": m, "ms": round(sec * 1e3, 3),
               "calls": calls}
        if m <= 64:
            rec["gbs"] = round(nbytes / sec / 1e9, 3)
        if m >= 64:
            rec["gops"] = round(2.0 * m * n * k / sec / 1e9, 2)
        out[tag] = rec
        if cfg == "c1_q4_k_gemv":
            head = (nbytes, sec, calls)
            sec1, calls1 = _median_call(lambda: lib.matmul(x, w, qt, None, k, n, m, threads=1), cap)
            samples += calls1
            out["c1_q4_k_gemv_1_thread"] = {"ms": round(sec1 * 1e3, 3), "calls": calls1,
                                            "gbs": round(nbytes / sec1 / 1e9, 3)}
        del w
    # c3: the Q4_K_M layer at M = 512, each matrix once per call
    cfg = "c3_q4_k_m_layer"
    mats = [(S.config_weight(cfg, label), label) for label, _, _, _ in S.CONFIGS[cfg]["mats"]]
    xs = {k: S.config_activation(cfg, 512, k) for k in {mk for (_, _, mk, _), _ in mats}}

    def layer():
        for (qt, n, k, w), _ in mats:
            lib.matmul(xs[k], w, qt, None, k, n, 512, threads=threads)

    sec, calls = _median_call(layer, 2 * cap, least=2)
    samples += calls
    ops = sum(2.0 * 512 * n * k for (_, n, k, _), _ in mats)
    out["c3_q4_k_m_layer_m512"] = {"ms": round(sec * 1e3, 1), "calls": calls,
                                   "gops": round(ops / sec / 1e9, 2)}
    nbytes, sec, calls = head
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": kind, "nproc": os.cpu_count(), "cpu_share": threads, "cpu_model": cpu_model(),
            "sample": f"median of {calls} matmul_quant calls on the same Q4_K 14336x4096 M=1 "
                      f"workload (activation quantization included) after warm-up, {threads} "
                      f"ThreadPool workers; {samples} timed calls over all points, each point "
                      f"bounded to ~{cap:.1f} s",
            "configs": out}


def main():
    global WARM_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=30.0)
    ap.add_argument("--warm-ms", type=float, default=WARM_MS,
                    help="GPU time of untimed graph replays before each timed loop (0 for "
                         "counter runs, which profile every dispatch)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the M=512 Q4_K_M layer (for counter profiles of the GEMM) and "
                         "print its figures as one JSON line")
    ap.add_argument("--model-only", action="store_true",
                    help="run only the whole-model decode step and print it as one JSON line")
    ap.add_argument("--upload-only", action="store_true",
                    help="run only the GGUF upload measurement and print it as one JSON line")
    ap.add_argument("--layer-only", action="store_true",
                    help="run only the device-resident decode layer and print it as one JSON "
                         "line")
    ap.add_argument("--float-dot-only", action="store_true",
                    help="run only the float-dot types' decode GEMVs and print them as one "
                         "JSON line")
    ap.add_argument("--c0-only", action="store_true",
                    help="run only the L2-resident Q8_0 4864x896 GEMV (c0) and print it as one "
                         "JSON line")
    ap.add_argument("--sweep-only", action="store_true",
                    help="run only the c4 M-sweep and print it as one JSON line")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the M=512 prefill attention (f4) and print it as one JSON line")
    ap.add_argument("--head-only", action="store_true",
                    help="run only the Q6_K 128256x4096 output-head GEMV and print it as one JSON "
                         "line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 10 device copies of 64 MiB (a kernel of known traffic, for "
                         "scaling FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    WARM_MS = args.warm_ms
    if args.gpus != 1:
        print("bench.py measures one GPU: the path is not sharded across GPUs; run with "
              "--gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import cllm_inference_amd as C
    from cllm_inference_amd import synth as S

    lib = C.load_library()
    assert lib.cllm_hip_init(0) == 0, lib.cllm_hip_last_error().decode()

    if args.copy_calibration:
        src = torch.ones(64 << 18, dtype=torch.float32, device="cuda")  # 64 MiB
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.model_only:
        print(json.dumps({"f4_device_decode_step": decode_model(C, S, max(10, args.steps // 10),
                                                                 max(2, args.warmup // 10))}))
        return

    if args.upload_only:
        print(json.dumps({"f2_gguf_upload": gguf_upload(C, S)}))
        return

    if args.layer_only:
        print(json.dumps({"f1_decode_layer_device": decode_layer_device(
            C, S, max(20, args.steps // 4), max(3, args.warmup // 4))}))
        return

    if args.float_dot_only:
        print(json.dumps({"f3_float_dot_types": float_dot_points(C, S, max(20, args.steps // 4),
                                                                 max(3, args.warmup // 4))}))
        return

    if args.c0_only:
        c0 = decode_point(C, S, "c0_q8_0_gemv", "w", 1, args.steps, args.warmup, cold=False)
        print(json.dumps({"c0_q8_0_l2_resident": {"kernel": c0["plan"],
                                                  "step_us": round(c0["ms_step"] * 1e3, 2),
                                                  "gemv_us": round(c0["ms_gemv"] * 1e3, 2)}}))
        return

    if args.sweep_only:
        print(json.dumps({"c4_m_sweep": m_sweep(C, S, max(20, args.steps // 4),
                                                max(3, args.warmup // 4))}))
        return

    if args.head_only:
        c2 = decode_point(C, S, "c2_q6_k_head", "output", 1, max(20, args.steps // 4),
                          max(3, args.warmup // 4), cold=True, ceiling=True)
        print(json.dumps({"c2_q6_k_head": {"step_us": round(c2["ms_step"] * 1e3, 2),
                                           "gemv_gbs": round(c2["gbs_gemv"], 1),
                                           "gemv_frac_hbm": round(c2["gbs_gemv"] / HBM_PEAK_GBS, 4),
                                           "gemv_us": round(c2["ms_gemv"] * 1e3, 2),
                                           "read_ceiling": read_ceiling(c2)}}))
        return

    if args.attention_only:
        print(json.dumps({"f4_prefill_attention_m512": prefill_attention(
            C, max(5, args.steps // 20), max(2, args.warmup // 10))}))
        return

    if args.prefill_only:
        layer = prefill_layer(C, S, max(5, args.steps // 20), max(2, args.warmup // 10))
        dev = prefill_layer_device(C, S, max(5, args.steps // 20), max(2, args.warmup // 10),
                                   c3=layer)
        print(json.dumps({"c3_prefill_layer_m512": layer, "f1_prefill_layer_device": dev}))
        return

    head = decode_point(C, S, "c1_q4_k_gemv", "ffn", 1, args.steps, args.warmup, cold=True,
                        ceiling=True)
    extra = {}
    if not args.no_extra:
        warm = decode_point(C, S, "c1_q4_k_gemv", "ffn", 1, args.steps, args.warmup, cold=False)
        extra["c1_q4_k_warm_mall_gbs"] = round(warm["gbs_gemv"], 1)
        c2 = decode_point(C, S, "c2_q6_k_head", "output", 1, max(20, args.steps // 4),
                          max(3, args.warmup // 4), cold=True, ceiling=True)
        extra["c2_q6_k_head"] = {"kernel": c2["plan"],
                                 "step_us": round(c2["ms_step"] * 1e3, 2),
                                 "step_gbs": round(c2["gbs_step"], 1),
                                 "step_frac_hbm": round(c2["gbs_step"] / HBM_PEAK_GBS, 4),
                                 "gemv_us": round(c2["ms_gemv"] * 1e3, 2),
                                 "gemv_gbs": round(c2["gbs_gemv"], 1),
                                 "gemv_frac_hbm": round(c2["gbs_gemv"] / HBM_PEAK_GBS, 4),
                                 "read_ceiling": read_ceiling(c2),
                                 "tokens_per_s": round(1e3 / c2["ms_step"], 1)}
        c0 = decode_point(C, S, "c0_q8_0_gemv", "w", 1, args.steps, args.warmup, cold=False)
        extra["c0_q8_0_l2_resident"] = {"kernel": c0["plan"], "gemv_gbs": round(c0["gbs_gemv"], 1),
                                        "gemv_us": round(c0["ms_gemv"] * 1e3, 2),
                                        "step_us": round(c0["ms_step"] * 1e3, 2)}
        extra["c4_m_sweep"] = m_sweep(C, S, max(20, args.steps // 4), max(3, args.warmup // 4))
        extra["c3_prefill_layer_m512"] = prefill_layer(C, S, max(5, args.steps // 20),
                                                        max(2, args.warmup // 10))
        C.tune("gemm_kernel", 1)  # the int8 MFMA kernel on the same layer
        try:
            l8 = prefill_layer(C, S, max(5, args.steps // 20), max(2, args.warmup // 10))
        finally:
            C.tune("gemm_kernel")
        extra["c3_prefill_layer_m512_int8_kernel"] = {
            "layer_us": l8["layer_us"], "tops": l8["tops"], "frac_int8": l8["frac_int8"],
            "matrices_us": {lab: r["us"] for lab, r in l8["matrices"].items()}}
        extra["c1_host_pointer_api"] = host_api_point(C, S)
        extra["f3_float_dot_types"] = float_dot_points(C, S, max(20, args.steps // 4),
                                                       max(3, args.warmup // 4))
        extra["f1_decode_layer_device"] = decode_layer_device(C, S, max(20, args.steps // 4),
                                                              max(3, args.warmup // 4))
        extra["f1_prefill_layer_device"] = prefill_layer_device(
            C, S, max(5, args.steps // 20), max(2, args.warmup // 10),
            c3=extra["c3_prefill_layer_m512"])
        extra["f2_gguf_upload"] = gguf_upload(C, S)
        extra["f4_device_decode_step"] = decode_model(C, S, max(10, args.steps // 10),
                                                      max(2, args.warmup // 10))
        extra["f4_prefill_attention_m512"] = prefill_attention(C, max(5, args.steps // 20),
                                                               max(2, args.warmup // 10))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(S, seconds=args.cpu_seconds)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_c1_q4_k_gemv.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")

    out = {
        "metric": "Q4_K decode GEMV HBM throughput (14336x4096, M=1)",
        "value": round(head["gbs_step"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded GGUF Q4_K blocks, N(0,1) fp32 activations)",
        "config": {"workload": "Q4_K decode GEMV 14336x4096 M=1, Llama-3-8B FFN shape; "
                               f"{head['copies']} rotating weight copies so each step reads HBM",
                   "type": "Q4_K", "out_dim": 14336, "in_dim": 4096, "n_rows": 1,
                   "algorithmic_bytes_per_step": head["bytes"]},
        "frac_of_hbm_peak": round(head["gbs_step"] / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(1e3 / head["ms_step"], 1),
        # A decode step is one kernel launch (the GEMV quantizing its activation in LDS), so
        # the step's HIP-event time is that kernel's average duration.
        "roofline": {"bound": "hbm", "achieved": round(head["gbs_step"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs_step"] / HBM_PEAK_GBS, 4),
                     "kernel": head["plan"] + " (fused Q8_0 activation quantization)",
                     "kernel_us": round(head["ms_step"] * 1e3, 3),
                     "traffic": traffic,
                     "one_launch_read_ceiling": read_ceiling(head)},
        "gemv_prequantized": {"kernel_us": round(head["ms_gemv"] * 1e3, 3),
                              "gbs": round(head["gbs_gemv"], 1)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
