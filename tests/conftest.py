import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def split_cases(data: dict) -> dict:
    """{'tag__field': arr} -> {tag: {field: arr}}"""
    out: dict = {}
    for key, val in data.items():
        tag, field = key.split("__", 1)
        out.setdefault(tag, {})[field] = val
    return out


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not os.path.exists(oracle.ORACLE_SO):
        oracle.build(with_ref=False)
    return oracle.Oracle()


# every process-wide kernel-choice override of cllm_hip_tune
TUNING_KNOBS = ("gemm_kernel", "gemm_tiles", "gemm_splits", "gemv_kernel", "gemv_str_grid",
                "gemm_small", "gemm_small_plan", "gemm_small_q8", "gemv_fused_rows", "gemv_waves",
                "attention_kernel", "gemv_fp_wgs")


@pytest.fixture(autouse=True)
def _reset_tuning_knobs():
    """A test that forces a kernel plan and then fails leaves no override behind for the tests
    after it: every knob is reset after each test that loaded the library."""
    yield
    import cllm_inference_amd as C
    if C._lib_handle is not None:
        for knob in TUNING_KNOBS:
            C.tune(knob)


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on device 0; the test fails (never falls back) if it cannot run."""
    import torch
    import cllm_inference_amd as C
    assert torch.cuda.is_available(), "no GPU visible to torch"
    lib = C.load_library()
    rc = lib.cllm_hip_init(0)
    assert rc == 0, lib.cllm_hip_last_error().decode()
    return C
