"""The C++ Quant API (include/cllm/core/quant.hpp over libcllm_quant.so) driven from C++, the
way the reference's own tests/quant_test.cpp drives its API. The program is
tests/cpp/quant_api_test.cpp; its expected values come from the C oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "quant_api_test")


def _binary() -> str:
    if not os.path.exists(BIN):
        # cheap host-only build; the libraries it links are built by __graft_entry__.build()
        subprocess.run(["make", "-s", "-C", os.path.dirname(BIN)], check=True)
    return BIN


def _run(args):
    proc = subprocess.run([_binary()] + args, capture_output=True, text=True, timeout=300)
    print(proc.stdout[-4000:], proc.stderr[-2000:])
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert ", 0 failed" in proc.stdout


def test_cpp_quant_api_without_device():
    """Size tables, has_vec_dot, fp16 conversions over all 65536 encodings, and every
    argument error with the reference's message text."""
    _run(["--cpu"])


@pytest.mark.gpu
def test_cpp_quant_api_on_gpu():
    """Everything above, then quantize_row_q8_0 bit-exact, vec_dot_row, matmul_quant on the
    reference test's weight patterns, the bias difference, and matmul_quant_batch against
    row-by-row and against the exact quantized result (GEMV and MFMA batch sizes)."""
    _run([])
