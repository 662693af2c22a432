"""A device-resident Llama-family forward composed from the library's kernels, and the
synthetic GGUF models it runs on -- the end-to-end check of the device linear path (RMSNorm
and SwiGLU producers fused with Q8_0, q/k/v and gate/up in one launch, residual adds in the
GEMV) together with the float ops (RoPE, QK norms, attention, embedding lookup) against the
reference engine's own logits (oracle/_ref, TransformerEngine::forward / prefill,
src/core/engine.cpp:466-610).

This mirrors the reference's forward step by step; it is test and benchmark code, not an
engine (no sampling, no tokenizer, no context management beyond the KV cache).
"""
from __future__ import annotations

import numpy as np

from cllm_inference_amd import synth as S
import gguf_writer as G


class DevPtr:
    """A raw device address where the bindings expect a tensor (they only use data_ptr)."""

    def __init__(self, p: int):
        self.p = int(p)

    def data_ptr(self) -> int:
        return self.p


def write_model(path, arch="llama", n_layers=2, n_embd=256, n_head=4, n_kv=2, n_ff=512,
                vocab=320, n_ctx=256, head_dim=None, wtype=S.Q4_K, wtype_v=None,
                wtype_down=S.Q6_K, emb_type=S.Q8_0, out_type=S.Q6_K, seed=7):
    """A random model of the reference's layout (engine.cpp:350-416): token_embd, output_norm,
    output (omitted for out_type None: tied to the embedding), and per layer the norms and
    the seven projections; qwen2 adds q/k/v biases, qwen3 q/k norms and an explicit
    head_dim."""
    rng = np.random.default_rng(seed)
    hd = head_dim or n_embd // n_head
    q_dim, kv_dim = n_head * hd, n_kv * hd
    kv = [("general.architecture", G.STR, arch),
          (f"{arch}.block_count", G.U32, n_layers), (f"{arch}.embedding_length", G.U32, n_embd),
          (f"{arch}.attention.head_count", G.U32, n_head),
          (f"{arch}.attention.head_count_kv", G.U32, n_kv),
          (f"{arch}.context_length", G.U32, n_ctx), (f"{arch}.feed_forward_length", G.U32, n_ff),
          (f"{arch}.rope.freq_base", G.F32, 10000.0 if arch == "llama" else 1000000.0),
          (f"{arch}.attention.layer_norm_rms_epsilon", G.F32, 1e-5),
          (f"{arch}.vocab_size", G.U32, vocab)]
    if head_dim:
        kv.append((f"{arch}.attention.key_length", G.U32, hd))
    tensors = []
    counter = [seed * 1000]

    def mat(name, qt, n, k):
        counter[0] += 1
        tensors.append((name, (n, k), qt, S.make_weight(qt, n, k, counter[0]).tobytes()))

    def vec(name, n, mean=1.0, sd=0.1):
        tensors.append((name, (n,), S.F32,
                        (mean + sd * rng.standard_normal(n)).astype(np.float32).tobytes()))

    mat("token_embd.weight", emb_type, vocab, n_embd)
    vec("output_norm.weight", n_embd)
    if out_type is not None:
        mat("output.weight", out_type, vocab, n_embd)
    for l in range(n_layers):
        p = f"blk.{l}."
        vec(p + "attn_norm.weight", n_embd)
        mat(p + "attn_q.weight", wtype, q_dim, n_embd)
        mat(p + "attn_k.weight", wtype, kv_dim, n_embd)
        mat(p + "attn_v.weight", wtype_v or wtype, kv_dim, n_embd)
        if arch == "qwen2":
            for nm, n in (("attn_q.bias", q_dim), ("attn_k.bias", kv_dim), ("attn_v.bias", kv_dim)):
                vec(p + nm, n, 0.0, 0.5)
        if arch == "qwen3":
            vec(p + "attn_q_norm.weight", hd)
            vec(p + "attn_k_norm.weight", hd)
        mat(p + "attn_output.weight", wtype, n_embd, q_dim)
        vec(p + "ffn_norm.weight", n_embd)
        mat(p + "ffn_gate.weight", wtype, n_ff, n_embd)
        mat(p + "ffn_up.weight", wtype, n_ff, n_embd)
        mat(p + "ffn_down.weight", wtype_down, n_embd, n_ff)
    G.write_gguf(path, kv, tensors)


class DeviceModel:
    """The reference engine's forward (engine.cpp:466-528) and prefill (520-610) on the
    device, from a GGUF file uploaded once."""

    def __init__(self, path):
        import torch
        import cllm_inference_amd as C
        self.C = C
        self.g = C.GgufFile(path, upload=True)
        c = self.g.config()
        self.n_layers, self.n_embd = c.n_layers, c.n_embd
        self.n_head, self.n_kv, self.hd = c.n_head, c.n_head_kv, c.head_dim
        self.n_ff, self.vocab, self.eps, self.theta = c.n_ff, c.vocab_size, c.norm_eps, c.rope_theta
        self.q_dim, self.kv_dim = self.n_head * self.hd, self.n_kv * self.hd
        self.n_ctx = c.n_ctx
        self.t = {}
        for i in range(len(self.g)):
            info = self.g.tensor(i)
            self.t[info.name] = info
        if "output.weight" not in self.t:
            self.t["output.weight"] = self.t["token_embd.weight"]
        dev = lambda name: DevPtr(self.t[name].dev)  # noqa: E731
        self.w = {name: dev(name) for name in self.t}
        self.k_cache = [torch.zeros((self.n_ctx, self.kv_dim), device="cuda") for _ in range(self.n_layers)]
        self.v_cache = [torch.zeros((self.n_ctx, self.kv_dim), device="cuda") for _ in range(self.n_layers)]
        self.pos = 0

    def close(self):
        self.g.close()

    def _type(self, name):
        return self.t[name].type

    def _linear(self, names, outs, h, q8, biases=None, residual=False):
        """y_i = W_i h (+ b_i) for the matrices `names` sharing the input rows h (fp32) and
        their Q8_0 blocks q8; one launch when the types allow, the residual add fused."""
        C = self.C
        types = {self._type(n) for n in names}
        rows = h.shape[0]
        if len(types) == 1 and C.has_vec_dot(next(iter(types))) and rows < 16:
            qt = next(iter(types))
            qs, sc, bs = q8
            k = h.shape[1]
            if residual:
                assert len(names) == 1 and biases is None
                C.gemv_q8_residual_dev(self.w[names[0]], qt, k, outs[0].shape[1], qs, sc, bs, outs[0])
            else:
                C.gemv_q8_multi_dev([self.w[n] for n in names], qt, k,
                                    [o.shape[1] for o in outs], qs, sc, bs, ys=outs, biases=biases)
            return
        import torch
        for i, n in enumerate(names):
            b = None if biases is None else biases[i]
            k = h.shape[1]
            if residual:
                tmp = torch.empty_like(outs[i])
                C.matmul_quant_dev(h, self.w[n], self._type(n), b, k, outs[i].shape[1], y=tmp)
                C.add_dev(outs[i], tmp)
            else:
                C.matmul_quant_dev(h, self.w[n], self._type(n), b, k, outs[i].shape[1], y=outs[i])

    def step(self, tokens, logits=True):
        """Runs the tokens (a list) at positions pos .. pos + len - 1, appending to the KV
        caches; returns the last token's logits (1, vocab) when asked."""
        import torch
        ids = torch.tensor(tokens, dtype=torch.int32, device="cuda")
        out = self.step_ids(ids, self.pos, logits)
        self.pos += len(tokens)
        return out

    def step_ids(self, ids, pos0, logits=True):
        """step() on token ids already on the device, at positions pos0 ..; allocates only
        through torch, so a HIP graph can capture it once every workspace exists."""
        import torch
        C = self.C
        T = ids.numel()
        emb = self.t["token_embd.weight"]
        x = C.dequantize_rows_dev(DevPtr(emb.dev), emb.type, self.n_embd, ids)
        q = torch.empty((T, self.q_dim), device="cuda")
        attn = torch.empty((T, self.q_dim), device="cuda")
        gate = torch.empty((T, self.n_ff), device="cuda")
        up = torch.empty((T, self.n_ff), device="cuda")
        for l in range(self.n_layers):
            p = f"blk.{l}."
            kc = self.k_cache[l][pos0:pos0 + T]
            vc = self.v_cache[l][pos0:pos0 + T]
            biases = None
            if p + "attn_q.bias" in self.w:
                biases = [self.w[p + "attn_q.bias"], self.w[p + "attn_k.bias"], self.w[p + "attn_v.bias"]]
            qkv = [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"]
            if self._norm_fusable(T, qkv):  # attn_norm rides in the q/k/v launch
                C.rmsnorm_gemv_multi_dev(x, self.w[p + "attn_norm.weight"], self.eps,
                                         [self.w[n] for n in qkv], self._type(qkv[0]), self.n_embd,
                                         [self.q_dim, self.kv_dim, self.kv_dim], ys=[q, kc, vc],
                                         biases=biases)
            else:
                h, qs, sc, bs = C.rmsnorm_q8_0_dev(x, self.w[p + "attn_norm.weight"], self.eps)
                self._linear(qkv, [q, kc, vc], h, (qs, sc, bs), biases)
            if p + "attn_q_norm.weight" in self.w:  # Qwen3 per-head norms, in place
                qv = q.view(T * self.n_head, self.hd)
                self._norm_inplace(qv, self.w[p + "attn_q_norm.weight"])
                self._norm_inplace(kc.view(T * self.n_kv, self.hd), self.w[p + "attn_k_norm.weight"])
            if T == 1:  # decode: the rotation rides in the attention launch
                C.attention_rope_dev(q, self.k_cache[l], self.v_cache[l], pos0, self.n_head,
                                     self.n_kv, self.hd, self.theta, out=attn)
            else:
                C.rope_neox2_dev(q, self.n_head, kc, self.n_kv, self.hd, pos0, self.theta)
                C.attention_dev(q, self.k_cache[l], self.v_cache[l], pos0, self.n_head, self.n_kv,
                                self.hd, out=attn)
            # the GEMV quantizes the attention output itself and adds into x
            wo = p + "attn_output.weight"
            C.matmul_quant_residual_dev(attn, self.w[wo], self._type(wo), None, self.q_dim,
                                        self.n_embd, x)
            wg, wu, wd = p + "ffn_gate.weight", p + "ffn_up.weight", p + "ffn_down.weight"
            tg = self._type(wg)
            if self._norm_fusable(T, [wg, wu]) and C.has_vec_dot(self._type(wd)):
                # ffn_norm, gate, up and the SwiGLU in one launch
                C.rmsnorm_gemv_swiglu_dev(x, self.w[p + "ffn_norm.weight"], self.eps, self.w[wg],
                                          self.w[wu], tg, self.n_embd, self.n_ff, h=gate)
                C.matmul_quant_residual_dev(gate, self.w[wd], self._type(wd), None, self.n_ff,
                                            self.n_embd, x)
                continue
            h, qs, sc, bs = C.rmsnorm_q8_0_dev(x, self.w[p + "ffn_norm.weight"], self.eps)
            if T < 16 and tg == self._type(wu) and C.has_vec_dot(tg) and C.has_vec_dot(self._type(wd)):
                # gate, up and the SwiGLU in one launch; the down GEMV quantizes h itself and
                # adds the residual
                C.gemv_q8_swiglu_dev(self.w[wg], self.w[wu], tg, self.n_embd, self.n_ff, qs, sc, bs,
                                     h=gate)
                C.matmul_quant_residual_dev(gate, self.w[wd], self._type(wd), None, self.n_ff,
                                            self.n_embd, x)
            else:
                self._linear([wg, wu], [gate, up], h, (qs, sc, bs))
                hs, qs, sc, bs = C.swiglu_q8_0_dev(gate, up)
                self._linear([wd], [x], hs, (qs, sc, bs), residual=True)
        if not logits:
            return None
        xl = x[T - 1:T].contiguous()
        out = torch.empty((1, self.vocab), device="cuda")
        if self._norm_fusable(1, ["output.weight"]):  # output_norm rides in the head GEMV
            C.rmsnorm_gemv_multi_dev(xl, self.w["output_norm.weight"], self.eps,
                                     [self.w["output.weight"]], self._type("output.weight"),
                                     self.n_embd, [self.vocab], ys=[out])
            return out
        h, qs, sc, bs = C.rmsnorm_q8_0_dev(xl, self.w["output_norm.weight"], self.eps)
        self._linear(["output.weight"], [out], h, (qs, sc, bs))
        return out

    def _norm_fusable(self, T, names):
        """One decode row, matrices of one vec_dot type, and a row the fused RMSNorm staging
        takes (a multiple of 32 up to 4096 elements)."""
        types = {self._type(n) for n in names}
        return (T == 1 and len(types) == 1 and self.C.has_vec_dot(next(iter(types)))
                and self.n_embd <= 4096 and self.n_embd % 32 == 0)

    def _norm_inplace(self, rows, w):
        lib = self.C.load_library()
        m, n = rows.shape
        self.C._check(lib.cllm_hip_rmsnorm_q8_0_dev(self.C._tp(rows), self.C._tp(w),
                                                    float(self.eps), int(n), int(m),
                                                    self.C._tp(rows), None, None, None,
                                                    self.C._stream()))
