"""The C ABI without a GPU: the library loads, exports every function
include/nnc_hip.h declares, and refuses bad arguments with nnc's statuses
before touching a device. Plus the host-side rules it mirrors and the
synthetic-input generator."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import nnc_hip, synth

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nnc_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nnc_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return nh.load_library()


def test_header_declares_the_bound_functions():
    assert declared_functions() == sorted(nnc_hip.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = C.CDLL(str(nnc_hip.LIB_PATH))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_status_values_and_strings_match_nnc(lib):
    # reference nnc.h:50-61 and baseline.cpp:169-184
    want = {0: "ok", 1: "invalid argument", 2: "unsupported CPU", 3: "I/O error", 4: "bad file format",
            5: "unsupported model", 6: "out of memory", 7: "context full", 8: "cancelled"}
    for code, text in want.items():
        assert lib.nnc_hip_status_string(code).decode() == text
        assert nh.NncStatus(code).value == code
    assert lib.nnc_hip_status_string(99).decode() == "unknown status"
    assert "NNC_ERR_CONTEXT_FULL = 7" in HEADER.read_text()


def _create(lib, rows, kv_dim, bf16=True):
    n = len(rows)
    h = C.c_void_p()
    st = lib.nnc_hip_kv_create(n, (C.c_int32 * max(n, 1))(*rows), (C.c_int32 * max(n, 1))(*kv_dim), bf16,
                               C.byref(h))
    return st, h


def test_create_refuses_bad_arguments(lib):
    for rows, kv_dim in (([], []), ([0], [1024]), ([16], [0]), ([16], [12]), ([16, -1], [64, 64])):
        st, h = _create(lib, rows, kv_dim)
        assert st == nh.NncStatus.INVALID_ARGUMENT, (rows, kv_dim)
        assert not h.value
        assert lib.nnc_hip_last_error()
    st = lib.nnc_hip_kv_create(1, (C.c_int32 * 1)(16), (C.c_int32 * 1)(64), True, None)
    assert st == nh.NncStatus.INVALID_ARGUMENT


def test_create_without_a_device_reports_it(lib):
    hip = C.CDLL("libamdhip64.so")
    n = C.c_int(0)
    have_gpu = hip.hipGetDeviceCount(C.byref(n)) == 0 and n.value > 0
    st, h = _create(lib, [256], [64])
    if have_gpu:
        assert st == nh.NncStatus.OK
        lib.nnc_hip_kv_free(h)
    else:
        assert st == nh.NncStatus.UNSUPPORTED_CPU
        assert b"no HIP device" in lib.nnc_hip_last_error()


def test_calls_on_a_null_cache_are_refused(lib):
    q = np.zeros(64, dtype=np.float32)
    st = lib.nnc_hip_attend(None, 0, q.ctypes.data, q.ctypes.data, 1, 0, 1, 0, True, 1, 1, 64, 0.125)
    assert st == nh.NncStatus.INVALID_ARGUMENT
    st = lib.nnc_hip_kv_append(None, 0, 0, 1, q.ctypes.data, q.ctypes.data)
    assert st == nh.NncStatus.INVALID_ARGUMENT
    assert lib.nnc_hip_kv_sync(None) == nh.NncStatus.INVALID_ARGUMENT
    assert lib.nnc_hip_kv_bytes(None) == 0
    assert lib.nnc_hip_kv_stream(None) is None
    assert lib.nnc_hip_kv_set_exact_batches(None, True) == nh.NncStatus.INVALID_ARGUMENT
    lib.nnc_hip_kv_free(None)  # a no-op
    assert lib.nnc_hip_fill_normal(None, 10, 1, 0, False, None) == nh.NncStatus.INVALID_ARGUMENT
    assert lib.nnc_hip_fill_normal(q.ctypes.data, 10, 1, 3, False, None) == nh.NncStatus.INVALID_ARGUMENT
    # The gemvs and argmaxes check their arguments before touching a device.
    idx = C.c_int32(-7)
    st = lib.nnc_hip_gemv_bf16(None, q.ctypes.data, q.ctypes.data, 32, q.ctypes.data, 2, 2, 32, 1)
    assert st == nh.NncStatus.INVALID_ARGUMENT
    st = lib.nnc_hip_gemv_bf16_argmax(None, q.ctypes.data, q.ctypes.data, 2, 32, C.byref(idx))
    assert st == nh.NncStatus.INVALID_ARGUMENT and idx.value == -7
    st = lib.nnc_hip_argmax_f32(None, q.ctypes.data, 64, C.byref(idx))
    assert st == nh.NncStatus.INVALID_ARGUMENT and idx.value == -7


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(FileNotFoundError):
        nnc_hip.load_library(tmp_path / "libnnc_hip.so")


def test_kv_rows_rule():
    # reference tests.cpp:2606-2609 and model.cpp:1936-1957
    assert nh.kv_rows(1200, 40, 16) == 256 and nh.max_rewind(256, 40) == 216
    assert nh.kv_rows(1200, 0, 16) == 1200
    assert nh.kv_rows(8192, 512, 2048) == 2560  # Gemma-3-1B local layers at 2048-token chunks
    assert nh.kv_rows(16640, 1024, 1024) == 2048  # Gemma-3-4B local layers at 1024-token chunks
    assert nh.kv_rows(300, 512, 16) == 300  # a ring only when it is smaller than the context


def test_generator_is_deterministic_and_offsettable():
    a = synth.normal(99, 100001)
    assert np.array_equal(a, synth.normal(99, 100001))
    assert np.array_equal(a[12345:12400], synth.normal(99, 55, 12345))
    assert np.array_equal(a[1:2], synth.normal(99, 1, 1))
    assert not np.array_equal(a[:1000], synth.normal(100, 1000))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    # splitmix64 known answer: seed 0, first draw (the widely published first output)
    z = synth._splitmix64(0, np.array([0], dtype=np.uint64))[0]
    assert int(z) == 0xE220A8397B1DCDAF


def test_configs_follow_the_benchmark_shapes():
    c = synth.CONFIGS
    assert (c["D"].n_head, c["D"].n_kv, c["D"].head_dim, c["D"].n_layer) == (32, 8, 128, 36)
    assert [li for li in range(26) if not c["C"].sliding(li)] == [5, 11, 17, 23]
    assert sum(c["E"].sliding(li) for li in range(34)) == 29
    assert not c["A"].kv_bf16 and c["A"].tol == 1e-3
    assert c["B"].attn_scale == 0.125 and c["A"].attn_scale == 1.0 / 16
