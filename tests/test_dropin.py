"""The drop-in boundary: the reference's own TransformerEngine (src/core/engine.cpp), unmodified,
built against this repository's include/ and linked to libcllm_quant.so.

- CPU: engine.cpp, gguf.cpp and thread_pool.cpp of the reference compile against include/
  (whose quant.hpp and tensor.hpp take the place of the reference's) and link into a shared
  object with --no-undefined against libcllm_quant.so: every Quant symbol the engine uses
  (matmul_quant, matmul_quant_batch, dequantize_block, Tensor::dequantize, ...) is defined by
  this library. Needs the reference tree (skipped without it); only the build is checked.
- GPU: that engine (oracle/_ref/libengine_dropin.so, built by __graft_entry__.build()) runs
  the synthetic Llama / Qwen2 / Qwen3 models of tests/golden/model.npz with every matmul and
  the embedding lookup on the MI355X path, through host pointers into its mmap'd GGUF file.
  Its logits must match the reference engine's own (the same engine over the reference's
  quant.cpp) within 2e-5 of the largest |logit| of each step, with the same argmax.
"""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, load_golden, split_cases
import oracle

REF = oracle.REF_ROOT
PKG = os.path.join(ROOT, "cllm_inference_amd")
QUANT_SO = os.path.join(PKG, "libcllm_quant.so")

# the reference's engine and the two files it needs besides the Quant API
ENGINE_SOURCES = ["src/core/engine.cpp", "src/core/gguf.cpp", "src/core/thread_pool.cpp"]


def _cxx() -> str:
    for c in ("clang++", "g++"):
        if subprocess.run(["which", c], capture_output=True).returncode == 0:
            return c
    pytest.skip("no C++ compiler")


@pytest.mark.skipif(not os.path.isdir(REF), reason="needs the reference tree")
def test_reference_engine_links_against_libcllm_quant(tmp_path):
    assert os.path.exists(QUANT_SO), "build libcllm_quant.so first (__graft_entry__.build())"
    cxx = _cxx()
    objs = []
    for src in ENGINE_SOURCES:
        obj = str(tmp_path / (os.path.basename(src) + ".o"))
        subprocess.run([cxx, "-std=c++20", "-O1", "-fPIC", "-w", "-I" + os.path.join(ROOT, "include"),
                        "-I" + os.path.join(REF, "include"), "-c", os.path.join(REF, src), "-o", obj],
                       check=True)
        objs.append(obj)
    # the engine's Quant references must be exactly those libcllm_quant.so defines
    undef = subprocess.run(["nm", "-C", "--undefined-only", objs[0]], capture_output=True,
                           text=True, check=True).stdout
    wanted = sorted({ln.split(" U ", 1)[1].strip() for ln in undef.splitlines()
                     if " U cllm::" in ln and " U cllm::ThreadPool::" not in ln})
    print("engine.cpp needs:", *wanted, sep="\n  ")
    for sym in ("cllm::matmul_quant(", "cllm::matmul_quant_batch(", "cllm::dequantize_block(",
                "cllm::Tensor::dequantize() const", "cllm::Tensor::dequantize_f16() const"):
        assert any(w.startswith(sym) for w in wanted), sym
    defined = subprocess.run(["nm", "-C", "-D", "--defined-only", QUANT_SO], capture_output=True,
                             text=True, check=True).stdout
    for w in wanted:
        assert w in defined, f"libcllm_quant.so does not define {w}"
    out = str(tmp_path / "libengine_check.so")
    subprocess.run([cxx, "-shared", "-fPIC", "-o", out, *objs, "-L" + PKG, "-lcllm_quant",
                    "-Wl,--no-undefined", "-Wl,-rpath," + PKG, "-pthread"], check=True)
    assert os.path.getsize(out) > 0


CASES = split_cases(load_golden("model.npz"))


def _check(got, want, what):
    got = np.asarray(got, np.float64).reshape(want.shape)
    for r in range(want.shape[0]):
        scale = np.abs(want[r]).max()
        err = np.abs(got[r] - want[r]).max()
        print(what, r, "max err / max |logit| = %.3g" % (err / scale), flush=True)
        assert err <= 2e-5 * scale, (what, r, err / scale)
        assert np.argmax(got[r]) == np.argmax(want[r]), (what, r)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_engine_runs_on_the_gpu_path(gpu, tmp_path, name):
    import device_model as DM
    if not os.path.exists(oracle.DROPIN_SO):
        pytest.skip("oracle/_ref/libengine_dropin.so was not built (needs the reference tree)")
    c = CASES[name]
    path = tmp_path / f"{name}.gguf"
    DM.write_model(path, **json.loads(str(c["kwargs"])))
    assert hashlib.sha256(path.read_bytes()).hexdigest() == str(c["file_sha"]), "generator drift"
    eng = oracle.DropIn()
    toks = [int(t) for t in c["tokens"]]
    print("drop-in engine", name, flush=True)
    _check(eng.engine_logits(path, toks[:6]), c["decode6"], f"{name} decode")
    _check(eng.engine_logits(path, toks[:6], prefill=True), c["prefill6"], f"{name} prefill6")
    _check(eng.engine_logits(path, toks, prefill=True), c["prefill20"], f"{name} prefill20")
