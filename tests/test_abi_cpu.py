"""CPU-only checks of the C-ABI library: it loads, exports every symbol include/*.h declares, and
its GPU-free paths (version, capabilities, status names, null-pointer rejection) behave. No call
here touches the HIP runtime."""

import ctypes
import glob
import os
import re

import pytest

from models_amd import attention as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"JMODELS_ATTN_API\s+[\w\s\*]*?\b(jmodels_attn_\w+)\s*\(", text))
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(A.DEFAULT_LIBRARY):
        from models_amd import build
        build.build()
    return A.load_library()


def test_library_exports_every_declared_symbol(lib):
    declared = _declared_functions()
    assert len(declared) >= 30
    assert declared == set(A.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_library_only_exports_the_abi():
    out = os.popen(f"nm -D --defined-only {A.DEFAULT_LIBRARY}").read()
    funcs = [ln.split()[-1] for ln in out.splitlines() if " T " in ln]
    assert funcs and all(f.startswith("jmodels_attn_") for f in funcs), funcs


def test_abi_version_and_capabilities(lib):
    assert lib.jmodels_attn_abi_version() == A.ABI_VERSION == 2
    caps = lib.jmodels_attn_capabilities()
    for bit in (A.CAP_DECODE_F32, A.CAP_DECODE_F16, A.CAP_PREFILL_MFMA, A.CAP_RAGGED_DECODE,
                A.CAP_SLIDING_WINDOW, A.CAP_RING_LAYERS, A.CAP_DEVICE_POINTERS, A.CAP_QK_NORM,
                A.CAP_VALUE_NORM):
        assert caps & bit


def test_status_names(lib):
    # NativeKernelLibrary.statusName analogue: codes 0-4 keep backend-native's meaning.
    names = {0: "OK", 1: "NULL_POINTER", 2: "INVALID_SHAPE", 3: "BUFFER_TOO_SMALL", 4: "PANIC",
             5: "DEVICE_ERROR", 6: "OUT_OF_RANGE", 7: "UNAVAILABLE", 8: "NON_FINITE", 9: "NOT_CAPTURABLE",
             99: "UNKNOWN"}
    for code, name in names.items():
        assert lib.jmodels_attn_status_name(code).decode() == name


def test_null_handles_are_rejected_without_a_gpu(lib):
    assert lib.jmodels_attn_context_destroy(None) == A.NULL_POINTER
    assert lib.jmodels_attn_rope_destroy(None) == A.NULL_POINTER
    assert lib.jmodels_attn_kv_destroy(None) == A.NULL_POINTER
    assert lib.jmodels_attn_norm_destroy(None) == A.NULL_POINTER
    h = ctypes.c_void_p()
    assert lib.jmodels_attn_norm_create_ex(None, 64, None, None, 1e-6, A.NORM_VALUE_RMS,
                                           ctypes.byref(h)) == A.NULL_POINTER
    out_h = ctypes.c_void_p()
    assert lib.jmodels_attn_norm_create(None, 128, None, None, 1e-6, ctypes.byref(out_h)) == \
        A.NULL_POINTER
    assert lib.jmodels_attn_kv_clear(None, -1) == A.NULL_POINTER
    assert lib.jmodels_attn_kv_discard_from(None, 0, 0) == A.NULL_POINTER
    out = ctypes.c_int32()
    assert lib.jmodels_attn_kv_contains(None, 0, 0, 0, ctypes.byref(out)) == A.NULL_POINTER
    assert lib.jmodels_attn_context_synchronize(None) == A.NULL_POINTER
    assert "null" in lib.jmodels_attn_last_error().decode()
    layer = A._Layer(0, 8, 0, 0, 0.0, 0, None, None)
    rows = (ctypes.c_uint32 * 1)(0)
    assert lib.jmodels_attn_decode(None, None, ctypes.byref(layer), 1, rows, rows, None, 0, None,
                                   0, None, 0, None, 0) == A.NULL_POINTER
    assert lib.jmodels_attn_prefill(None, None, ctypes.byref(layer), 0, 0, 1, None, 0, None, 0,
                                    None, 0, None, 0) == A.NULL_POINTER


def test_layer_struct_matches_header_layout():
    # jmodels_attn_layer: 6 x 4-byte fields, then the rope and qk_norm pointers = 40 bytes.
    assert ctypes.sizeof(A._Layer) == 40
    assert A._Layer.rope.offset == 24
    assert A._Layer.qk_norm.offset == 32


def test_window_helpers_follow_llama_config():
    assert A.attention_start_position(700, 512) == 189
    assert A.attention_start_position(10, 512) == 0
    assert A.attention_start_position(700, 0) == 0
    assert [A.uses_sliding_window(l, 6, 512) for l in range(6)] == [True] * 5 + [False]
    assert not A.uses_sliding_window(0, 6, 0)
    assert A.default_scale(128) == pytest.approx(0.08838834764831845, rel=1e-7)
