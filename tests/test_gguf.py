"""The GGUF reader (cllm_hip_gguf_*): tensor table, data section and hyper-parameters of
files written by tests/gguf_writer.py, checked against what the writer put there and, where
oracle/_ref is built, against the reference's own GgufLoader::load (gguf.cpp:122-275) on the
same files. Parsing needs no GPU (upload = 0)."""
import ctypes

import numpy as np
import pytest

import cllm_inference_amd as C
from cllm_inference_amd import synth as S
import gguf_writer as G
import oracle as O


def _llama_file(path, version=3, extra_kv=()):
    rng = np.random.default_rng(1)
    tensors = [
        ("token_embd.weight", (3, 256), S.Q4_K, S.make_weight(S.Q4_K, 3, 256, 1).tobytes()),
        ("blk.0.attn_norm.weight", (256,), S.F32, rng.standard_normal(256).astype(np.float32).tobytes()),
        ("blk.0.attn_q.weight", (256, 256), S.Q8_0, S.make_weight(S.Q8_0, 256, 256, 2).tobytes()),
        ("blk.0.ffn_down.weight", (256, 512), S.Q6_K, S.make_weight(S.Q6_K, 256, 512, 3).tobytes()),
        ("output.weight", (3, 256), S.F16, S.make_weight(S.F16, 3, 256, 4).tobytes()),
        ("odd.weight", (5, 7, 2), S.F32, rng.standard_normal(70).astype(np.float32).tobytes()),
    ]
    kv = [
        ("general.architecture", G.STR, "llama"),
        ("general.noise_u8", G.U8, 7), ("general.noise_i8", G.I8, -7),
        ("general.noise_u16", G.U16, 700), ("general.noise_i16", G.I16, -700),
        ("general.noise_u64", G.U64, 1 << 40), ("general.noise_i64", G.I64, -(1 << 40)),
        ("general.noise_f64", G.F64, 2.5), ("general.noise_bool", G.BOOL, 1),
        ("general.noise_arr_u16", G.ARR, (G.U16, [1, 2, 3])),
        ("general.noise_nested", G.ARR, (G.ARR, [(G.U8, [1, 2]), (G.STR, ["x", "yz"])])),
        ("llama.block_count", G.U32, 1), ("llama.embedding_length", G.U32, 256),
        ("llama.attention.head_count", G.U32, 4), ("llama.attention.head_count_kv", G.U32, 2),
        ("llama.context_length", G.U32, 2048), ("llama.feed_forward_length", G.U32, 512),
        ("llama.rope.freq_base", G.F32, 500000.0),
        ("llama.attention.layer_norm_rms_epsilon", G.F32, 1e-5),
        ("tokenizer.ggml.tokens", G.ARR, (G.STR, ["<s>", "</s>", "a"])),
        ("tokenizer.ggml.scores", G.ARR, (G.F32, [0.0, 0.0, -1.0])),
        ("tokenizer.ggml.token_type", G.ARR, (G.I32, [3, 3, 1])),
        *extra_kv,
    ]
    offsets, data_at = G.write_gguf(path, kv, tensors, version=version)
    return tensors, dict(offsets), data_at


def _ours(path):
    with C.GgufFile(path) as g:
        cfg = g.config()
        tensors = [g.tensor(i) for i in range(len(g))]
        found = {t.name: g.find(t.name) for t in tensors}
        assert g.find("no.such.tensor") == -1
        raw = {t.name: ctypes.string_at(t.host, 16) for t in tensors}
    return cfg, tensors, found, raw


@pytest.mark.parametrize("version", [2, 3])
def test_table_config_and_data_pointers(tmp_path, version):
    path = tmp_path / "m.gguf"
    tensors, offsets, data_at = _llama_file(path, version)
    cfg, got, found, raw = _ours(path)
    assert cfg.version == version and cfg.data_offset == data_at and data_at % 32 == 0
    assert [t.name for t in got] == [t[0] for t in tensors]
    for i, ((name, shape, gtype, data), t) in enumerate(zip(tensors, got)):
        assert found[name] == i
        assert t.type == gtype and t.shape == tuple(shape) and t.offset == offsets[name]
        assert raw[name] == data[:16]  # the host pointer addresses the tensor's bytes
        assert t.dev == 0              # nothing uploaded
    assert cfg.arch == b"llama" and cfg.n_layers == 1 and cfg.n_embd == 256
    assert (cfg.n_head, cfg.n_head_kv, cfg.head_dim) == (4, 2, 64)
    assert (cfg.n_ctx, cfg.n_ff, cfg.vocab_size) == (2048, 512, 3)
    assert cfg.rope_theta == np.float32(500000.0) and cfg.norm_eps == np.float32(1e-5)


def test_arch_prefix_fallbacks_and_kinds(tmp_path):
    """Fields under "<arch>." win, "llama." is the fallback; a field stored with another
    value type is ignored; n_head_kv defaults to n_head, vocab_size to the token count,
    head_dim to attention.key_length when given (gguf.cpp:213-272)."""
    path = tmp_path / "q.gguf"
    kv = [("general.architecture", G.STR, "qwen3"),
          ("qwen3.block_count", G.U32, 28), ("llama.block_count", G.U32, 99),
          ("llama.embedding_length", G.U32, 1024),
          ("qwen3.attention.head_count", G.U32, 16),
          ("qwen3.attention.key_length", G.U32, 128),
          ("qwen3.context_length", G.U64, 40960),          # wrong kind: ignored
          ("qwen3.rope.freq_base", G.F32, 1e6),
          ("tokenizer.ggml.tokens", G.ARR, (G.STR, [str(i) for i in range(10)]))]
    G.write_gguf(path, kv, [("w", (2, 32), S.Q8_0, S.make_weight(S.Q8_0, 2, 32, 5).tobytes())])
    cfg, _, _, _ = _ours(path)
    assert cfg.arch == b"qwen3" and cfg.n_layers == 28 and cfg.n_embd == 1024
    assert cfg.n_head == 16 and cfg.n_head_kv == 16 and cfg.head_dim == 128
    assert cfg.n_ctx == 0 and cfg.vocab_size == 10 and cfg.rope_theta == 1e6
    assert cfg.norm_eps == np.float32(1e-5)


def test_errors(tmp_path):
    ok = tmp_path / "ok.gguf"
    _llama_file(ok)
    data = ok.read_bytes()
    cases = {
        "missing": (None, r"cannot open model file: "),
        "magic": (b"GGUX" + data[4:], r"^invalid GGUF magic$"),
        "version": (data[:4] + (4).to_bytes(4, "little") + data[8:], r"^unsupported GGUF version: 4$"),
        "short": (data[:3], r"^invalid GGUF magic$"),
        "truncated": (data[:60], r"^read_(u32|u64|string)$"),
        "badtype": (None, r"^unknown value type$"),
    }
    for name, (content, msg) in cases.items():
        path = tmp_path / f"{name}.gguf"
        if name == "badtype":
            G.write_gguf(path, [("general.architecture", G.STR, "llama")], [])
            b = bytearray(path.read_bytes())
            # the value type of the only key sits after magic, version, counts and the key
            at = 4 + 4 + 8 + 8 + 8 + len("general.architecture")
            b[at:at + 4] = (99).to_bytes(4, "little")
            path.write_bytes(bytes(b))
        elif content is not None:
            path.write_bytes(content)
        with pytest.raises(RuntimeError, match=msg):
            C.GgufFile(path)
        ref = O.reference_or_none()
        if ref is not None:
            with pytest.raises(RuntimeError, match=msg):
                ref.gguf_dump(path)


def test_matches_compiled_reference_loader(tmp_path):
    ref = O.reference_or_none()
    if ref is None:
        pytest.skip("oracle/_ref/libcllm_ref.so not built (reference tree absent)")
    files = []
    for v in (2, 3):
        p = tmp_path / f"l{v}.gguf"
        _llama_file(p, v)
        files.append(p)
    p = tmp_path / "q.gguf"
    G.write_gguf(p, [("general.architecture", G.STR, "qwen2"), ("llama.block_count", G.U32, 3),
                     ("qwen2.embedding_length", G.U32, 896),
                     ("qwen2.attention.head_count", G.U32, 14),
                     ("qwen2.attention.head_count_kv", G.U32, 2)],
                 [("a", (4, 64), S.Q4_0, S.make_weight(S.Q4_0, 4, 64, 9).tobytes()),
                  ("b", (64,), S.F16, S.make_weight(S.F16, 1, 64, 10).tobytes())])
    files.append(p)
    for path in files:
        rcfg, rtensors = ref.gguf_dump(path)
        cfg, got, _, _ = _ours(path)
        assert rcfg["arch"] == cfg.arch.decode()
        for k in ("n_layers", "n_embd", "n_head", "n_head_kv", "n_ctx", "n_ff", "vocab_size",
                  "head_dim"):
            assert rcfg[k] == getattr(cfg, k), k
        assert np.float32(rcfg["rope_theta"]) == cfg.rope_theta
        assert np.float32(rcfg["norm_eps"]) == cfg.norm_eps
        assert len(rtensors) == len(got)
        for (name, gtype, shape, off, delta), t in zip(rtensors, got):
            assert (name, gtype, shape, off) == (t.name, t.type, t.shape, t.offset)
            assert delta == cfg.data_offset + t.offset


def test_truncated_file_is_rejected(tmp_path):
    """A tensor whose bytes run past the end of the file fails at open (the device copy is the
    data section, so such a pointer would send kernels out of bounds)."""
    path = tmp_path / "m.gguf"
    _llama_file(path)
    raw = path.read_bytes()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(raw[:-100])  # odd.weight (280 bytes, the last tensor) loses its tail
    with pytest.raises(RuntimeError, match="odd.weight extends past the end of the file"):
        C.GgufFile(cut)
    cut.write_bytes(raw)  # the whole file opens
    with C.GgufFile(cut) as g:
        assert len(g) == 6


def test_too_many_dimensions_is_rejected(tmp_path):
    path = tmp_path / "m.gguf"
    data = np.zeros(32, np.float32).tobytes()
    G.write_gguf(path, [("general.architecture", G.STR, "llama")],
                 [("t5.weight", (1, 1, 2, 2, 8), S.F32, data)])
    with pytest.raises(RuntimeError, match="t5.weight: 5 dimensions"):
        C.GgufFile(path)
