"""ctypes wrapper over the CPU oracle (``libjmattn_oracle.so``).

TEST INFRASTRUCTURE ONLY. This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it. The product
package ``models_amd`` never imports, loads or calls anything under ``oracle/``.

The C file restates backend-java's GQA + KV-cache path (paths relative to
``backend-java/src/main/java/com/integrallis/models/backend/purejava/``). What pins each part:

==========================  =====================================================================
oracle function             pinned by
==========================  =====================================================================
f16 round (KvCache :94)     IEEE RNE definition: numpy float16 casts over ~1M bit patterns incl.
                            subnormals/overflow/ties; KvCacheTest :281-299 (1/3, exact values)
rotary frequencies/factors  RotaryTableTest golden -4.9626341/-1.1714368 (:80-91); table == direct
                            rope (:43-78); TensorOpsTest NeoX and frequency-scale closed forms
                            (:1527-1562); identity at position 0; norm preservation
rope / ropeNeox             same as above, plus hand-computed pair rotations
softmax                     TensorOpsTest :1368-1454 (uniform, sum-to-1, large, offset, -inf mask,
                            rejections); float64 softmax on random rows
KvCache                     KvCacheTest offsets/buffers/growth/discard/clear/bounds (:42-300)
LayeredKvCache              LayeredKvCacheTest spans (2,2,4,2),(4,2,0,0), buffers, bytes (:28-160)
rms_norm / qk_norm_heads    TensorOpsTest.RmsNorm known answers (:42-67); float64 rms on random
                            heads; in place == out of place; zero head -> 0 (rms = sqrt(eps))
q8_0 activation quantize    ggmlNearestInt == IEEE round-half-even (numpy rint) over the int8
                            range and ties; scales == numpy float16 of absmax/127; zero and NaN
                            blocks; every |q| <= 127 and q * scale within half a step of x
q8_k activation quantize    numpy: sign-aware block maximum (first index on ties), rint,
                            clamp at 127, 16-element sums, scale 1 / inverse
quantized matmul Q4_K/Q5_K/ NativeKernelLibraryTest's block builders (q4KBlock, q5KBlock,
  Q6_K                      q6KBlock) whose logical scales, mins and quants numpy's dequantization
                            must recover; float64 product of the dequantized blocks (one rounding
                            per term of the fma chains); Q5_K with its fifth bits cleared == Q4_K
quantized matmul Q4_0/Q8_0/ float64 dot of the dequantized weights with the dequantized Q8_0
  Q5_0                      activations (rounding of the per-block fma chain only); hand-computed
                            one-block cases (nibble order, the -8 / -16 offsets, the fifth bits,
                            scale product); the fixtures of NativeKernelLibraryTest (inputs /
                            fillWeights / fillQ8_0Weights / fillQ5_0Weights, :660-722)
                            regenerated as data, fillQ5_0Weights with its logical quants
attention start (window)    EncoderAttentionWindowTest causal bounds (:76-145); brute force
gqa / decode / prefill      float64 dense softmax(QK^T s)V on small shapes (brute force); L=1 -> V;
                            uniform scores -> mean of V rows; one-hot key; equal Q within a GQA
                            group -> equal outputs; prefill == token-at-a-time (LlamaForwardPassTest
                            :462); batched-vs-unbatched equivalence (:1071-1130)
==========================  =====================================================================

Parity unpinned: the lane order of vectors-core's ``VectorUtil.dotProduct`` /
``addScaledInPlace`` (com.integrallis:vectors-core:0.1.9 is not vendored and cannot be fetched);
the oracle uses sequential float sums. Golden attention vectors do not exist in the reference.
Bit-level equality of scores and outputs is therefore unpinned; the checks above bound the
oracle's error far below the path's 1e-3 / 2e-2 tolerances.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libjmattn_oracle.so")
_lib: Optional[ctypes.CDLL] = None

OK = 0
ILLEGAL_ARGUMENT = 1
ILLEGAL_STATE = 2

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)


def build() -> str:
    """Compiles the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    c_int, c_float, c_void = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    sig = {
        "jmo_float_to_f16": (ctypes.c_uint16, [c_float]),
        "jmo_f16_to_float": (c_float, [ctypes.c_uint16]),
        "jmo_f16_round_array": (None, [_f32p, _f32p, ctypes.c_size_t]),
        "jmo_rotary_frequencies": (c_int, [c_int, c_float, _f32p]),
        "jmo_rotary_factors": (c_int, [c_int, c_float, c_float, _f32p, c_int, _f32p, _f32p]),
        "jmo_rope_apply": (None, [_f32p, _f32p, _f32p, c_int, c_int]),
        "jmo_rope_direct": (None, [_f32p, c_int, c_int, c_float, c_float, c_int]),
        "jmo_softmax": (c_int, [_f32p, c_int]),
        "jmo_rms_norm": (None, [_f32p, _f32p, _f32p, c_int, c_float]),
        "jmo_qk_norm_heads": (None, [_f32p, c_int, c_int, _f32p, c_float]),
        "jmo_dot": (c_float, [_f32p, _f32p, c_int]),
        "jmo_value_rms_norm": (c_int, [_f32p, _f32p, c_int, c_float]),
        "jmo_kv_create": (c_void, [c_int, c_int, c_int, c_int, c_int]),
        "jmo_kv_destroy": (None, [c_void]),
        "jmo_kv_store": (c_int, [c_void, c_int, c_int, _f32p, _f32p]),
        "jmo_kv_key_offset": (ctypes.c_int64, [c_void, c_int, c_int]),
        "jmo_kv_value_offset": (ctypes.c_int64, [c_void, c_int, c_int]),
        "jmo_kv_key_slice": (c_int, [c_void, c_int, c_int, c_int, _f32p]),
        "jmo_kv_value_slice": (c_int, [c_void, c_int, c_int, c_int, _f32p]),
        "jmo_kv_key": (c_int, [c_void, c_int, c_int, _f32p]),
        "jmo_kv_value": (c_int, [c_void, c_int, c_int, _f32p]),
        "jmo_kv_clear": (None, [c_void]),
        "jmo_kv_discard_from": (c_int, [c_void, c_int]),
        "jmo_kv_reserve": (c_int, [c_void, c_int]),
        "jmo_kv_allocated_capacity": (c_int, [c_void]),
        "jmo_kv_key_buffer": (_f32p, [c_void]),
        "jmo_kv_value_buffer": (_f32p, [c_void]),
        "jmo_kv_buffer_length": (ctypes.c_int64, [c_void, c_int]),
        "jmo_lkv_create": (c_void, [c_int, c_int, _i32p, _i32p, _i32p]),
        "jmo_lkv_destroy": (None, [c_void]),
        "jmo_lkv_store": (c_int, [c_void, c_int, c_int, _f32p, _f32p]),
        "jmo_lkv_contains": (c_int, [c_void, c_int, c_int]),
        "jmo_lkv_attention_view": (c_int, [c_void, c_int, c_int, c_int, _i32p, _i32p]),
        "jmo_lkv_discard_from": (c_int, [c_void, c_int]),
        "jmo_lkv_clear": (None, [c_void]),
        "jmo_lkv_oldest": (c_int, [c_void, c_int]),
        "jmo_lkv_newest": (c_int, [c_void, c_int]),
        "jmo_lkv_allocated_capacity": (c_int, [c_void, c_int]),
        "jmo_lkv_physical_capacity": (c_int, [c_void, c_int]),
        "jmo_lkv_allocated_bytes": (ctypes.c_int64, [c_void]),
        "jmo_lkv_maximum_bytes": (ctypes.c_int64, [c_void]),
        "jmo_lkv_key_offset": (ctypes.c_int64, [c_void, c_int, c_int]),
        "jmo_lkv_key_buffer": (_f32p, [c_void, c_int]),
        "jmo_lkv_value_buffer": (_f32p, [c_void, c_int]),
        "jmo_lkv_buffer_length": (ctypes.c_int64, [c_void, c_int, c_int]),
        "jmo_attention_start": (c_int, [c_int, c_int]),
        "jmo_gqa": (c_int, [c_void, c_int, c_int, c_int, _f32p, c_int, c_int, c_int, c_int,
                            c_float, _f32p, _f32p]),
        "jmo_gqa_rows": (c_int, [_f32p, _f32p, _f32p, c_int, c_int, c_int, c_int, c_int, c_int,
                                 c_int, c_float, _f32p, _f32p]),
        "jmo_gqa_layered": (c_int, [c_void, c_int, c_int, c_int, _f32p, c_int, c_int, c_int,
                                    c_float, _f32p, _f32p]),
        "jmo_decode_layer": (c_int, [c_void, c_int, c_int, c_int, _f32p, _f32p, _f32p, c_int,
                                     c_int, c_int, c_int, c_float, c_float, c_int, c_float,
                                     _f32p, _f32p]),
        "jmo_prefill_layer": (c_int, [c_void, c_int, c_int, c_int, c_int, _f32p, _f32p, _f32p,
                                      c_int, c_int, c_int, c_int, c_float, c_float, c_int,
                                      c_float, _f32p, _f32p]),
        "jmo_gqa_rows_batch": (c_int, [c_int, ctypes.POINTER(_f32p), ctypes.POINTER(_f32p),
                                       ctypes.POINTER(_f32p), _i32p, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_float, ctypes.POINTER(_f32p), c_int]),
        "jmo_gqa_rows_batch8": (c_int, [c_int, ctypes.POINTER(_f32p), ctypes.POINTER(_f32p),
                                       ctypes.POINTER(_f32p), _i32p, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_float, ctypes.POINTER(_f32p), c_int]),
        "jmo_q8_0_quantize": (None, [_f32p, c_int, c_int, c_void, _f32p]),
        "jmo_q8_k_quantize": (None, [_f32p, c_int, c_int, c_void, _f32p, c_void]),
        "jmo_quantized_matmul": (c_int, [c_int, c_void, _f32p, c_int, c_int, c_int, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        kind = {ILLEGAL_ARGUMENT: "IllegalArgumentException",
                ILLEGAL_STATE: "IllegalStateException"}.get(status, f"status {status}")
        super().__init__(f"{what}: {kind}")
        self.status = status


def _check(status: int, what: str) -> None:
    if status != OK:
        raise OracleError(status, what)


# ------------------------------------------------------------------ elementwise helpers

def f16_round(x) -> np.ndarray:
    """float16ToFloat(floatToFloat16(x)) element-wise (KvCache.storeHalfPrecision)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().jmo_f16_round_array(_ptr(x), _ptr(out), x.size)
    return out


def float_to_f16_bits(x: float) -> int:
    return int(lib().jmo_float_to_f16(ctypes.c_float(x)))


def rotary_frequencies(rotary_dim: int, theta: float) -> np.ndarray:
    out = np.empty(rotary_dim // 2, np.float32)
    _check(lib().jmo_rotary_frequencies(rotary_dim, theta, _ptr(out)), "rotary_frequencies")
    return out


def rotary_factors(rotary_dim: int, theta: float, frequency_scale: float, position: int,
                   factors=None):
    pairs = rotary_dim // 2
    c = np.empty(pairs, np.float32)
    s = np.empty(pairs, np.float32)
    fp = None
    if factors is not None:
        factors = _f32(factors)
        fp = _ptr(factors)
    _check(lib().jmo_rotary_factors(rotary_dim, theta, frequency_scale, fp, position, _ptr(c),
                                    _ptr(s)), "rotary_factors")
    return c, s


def rope_apply(vec, cos_f, sin_f, neox: bool) -> np.ndarray:
    v = _f32(vec).copy()
    cos_f, sin_f = _f32(cos_f), _f32(sin_f)
    lib().jmo_rope_apply(_ptr(v), _ptr(cos_f), _ptr(sin_f), cos_f.size, int(neox))
    return v


def rope_direct(vec, position: int, head_dim: int, theta: float, frequency_scale: float,
                neox: bool) -> np.ndarray:
    v = _f32(vec).copy()
    lib().jmo_rope_direct(_ptr(v), position, head_dim, theta, frequency_scale, int(neox))
    return v


def softmax(x) -> np.ndarray:
    v = _f32(x).copy()
    _check(lib().jmo_softmax(_ptr(v), v.size), "softmax")
    return v


def rms_norm(x, weight, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(weight)
    out = np.empty_like(x)
    lib().jmo_rms_norm(_ptr(out), _ptr(x), _ptr(w), x.size, eps)
    return out


def qk_norm_heads(x, heads: int, head_dim: int, weight, eps: float) -> np.ndarray:
    """normalizeHead applied to each of ``heads`` consecutive heads (a copy of x)."""
    v = _f32(x).copy()
    w = _f32(weight)
    assert v.size == heads * head_dim and w.size == head_dim
    lib().jmo_qk_norm_heads(_ptr(v), heads, head_dim, _ptr(w), eps)
    return v


def value_rms_norm(x, eps: float, offset: int = 0, length: int = None) -> np.ndarray:
    """Gemma4Math.normalizeWithoutWeight over x[offset:offset+length] (a copy of x; the rest
    unchanged)."""
    v = _f32(x).copy()
    length = v.size - offset if length is None else length
    seg = v[offset:offset + length].copy()
    _check(lib().jmo_value_rms_norm(_ptr(seg), _ptr(seg), length, eps), "value_rms_norm")
    v[offset:offset + length] = seg
    return v


def value_rms_heads(x, heads: int, head_dim: int, eps: float) -> np.ndarray:
    """normalizeWithoutWeight applied to each of ``heads`` consecutive heads (a copy of x), as
    Gemma4ForwardPass does to every value head (gemma4/Gemma4ForwardPass.java:990-996)."""
    v = _f32(x).reshape(-1)
    assert v.size == heads * head_dim
    return np.concatenate([value_rms_norm(v[h * head_dim:(h + 1) * head_dim], eps)
                           for h in range(heads)])


def attention_start(position: int, window: int) -> int:
    return int(lib().jmo_attention_start(position, window))


# ------------------------------------------------------------------ KvCache

class KvCache:
    """Restated ``KvCache`` (cache/KvCache.java) with the reference's method names."""

    def __init__(self, num_layers: int, max_seq_len: int, key_dim: int, value_dim: int,
                 half_precision: bool = False):
        self._h = lib().jmo_kv_create(num_layers, max_seq_len, key_dim, value_dim,
                                      int(half_precision))
        if not self._h:
            raise OracleError(ILLEGAL_ARGUMENT, "KvCache")
        self.num_layers, self.max_seq_len = num_layers, max_seq_len
        self.key_dim, self.value_dim = key_dim, value_dim

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().jmo_kv_destroy(h)
            self._h = None

    def store(self, layer: int, position: int, key, value) -> None:
        k, v = _f32(key), _f32(value)
        if k.size != self.key_dim or v.size != self.value_dim:
            raise OracleError(ILLEGAL_ARGUMENT, "store: vector length")
        _check(lib().jmo_kv_store(self._h, layer, position, _ptr(k), _ptr(v)), "store")

    def key_offset(self, layer: int, position: int) -> int:
        off = lib().jmo_kv_key_offset(self._h, layer, position)
        if off < 0:
            raise OracleError(ILLEGAL_ARGUMENT, "keyOffset")
        return int(off)

    def value_offset(self, layer: int, position: int) -> int:
        off = lib().jmo_kv_value_offset(self._h, layer, position)
        if off < 0:
            raise OracleError(ILLEGAL_ARGUMENT, "valueOffset")
        return int(off)

    def _slice(self, fn, dim, layer, frm, to):
        out = np.empty(max(to - frm, 0) * dim, np.float32)
        _check(fn(self._h, layer, frm, to, _ptr(out)), "slice")
        return out

    def key_slice(self, layer: int, frm: int, to: int) -> np.ndarray:
        return self._slice(lib().jmo_kv_key_slice, self.key_dim, layer, frm, to)

    def value_slice(self, layer: int, frm: int, to: int) -> np.ndarray:
        return self._slice(lib().jmo_kv_value_slice, self.value_dim, layer, frm, to)

    def key(self, layer: int, position: int):
        out = np.empty(self.key_dim, np.float32)
        r = lib().jmo_kv_key(self._h, layer, position, _ptr(out))
        if r < 0:
            raise OracleError(-r, "key")
        return out if r == 1 else None

    def value(self, layer: int, position: int):
        out = np.empty(self.value_dim, np.float32)
        r = lib().jmo_kv_value(self._h, layer, position, _ptr(out))
        if r < 0:
            raise OracleError(-r, "value")
        return out if r == 1 else None

    def clear(self) -> None:
        lib().jmo_kv_clear(self._h)

    def discard_from(self, position: int) -> None:
        _check(lib().jmo_kv_discard_from(self._h, position), "discardFrom")

    def reserve_sequence_capacity(self, n: int) -> None:
        _check(lib().jmo_kv_reserve(self._h, n), "reserveSequenceCapacity")

    def allocated_sequence_capacity(self) -> int:
        return int(lib().jmo_kv_allocated_capacity(self._h))

    def key_buffer(self) -> np.ndarray:
        n = lib().jmo_kv_buffer_length(self._h, 0)
        return np.ctypeslib.as_array(lib().jmo_kv_key_buffer(self._h), shape=(n,)).copy()

    def value_buffer(self) -> np.ndarray:
        n = lib().jmo_kv_buffer_length(self._h, 1)
        return np.ctypeslib.as_array(lib().jmo_kv_value_buffer(self._h), shape=(n,)).copy()

    # ---- attention over this cache

    def gqa(self, layer: int, position: int, q, num_heads: int, num_kv_heads: int,
            key_length: int, value_length: int, scale: float, window: int = 0) -> np.ndarray:
        q = _f32(q)
        out = np.empty(num_heads * value_length, np.float32)
        scores = np.empty(self.max_seq_len, np.float32)
        _check(lib().jmo_gqa(self._h, layer, position, window, _ptr(q), num_heads, num_kv_heads,
                             key_length, value_length, scale, _ptr(out), _ptr(scores)), "gqa")
        return out

    def decode_layer(self, layer: int, position: int, q, k, v, num_heads: int,
                     num_kv_heads: int, key_length: int, value_length: int, rope_theta: float,
                     rope_scale: float, neox: bool, scale: float, window: int = 0):
        """One decode token through one layer; returns (out, rotated q, rotated k)."""
        q, k, v = _f32(q).copy(), _f32(k).copy(), _f32(v)
        out = np.empty(num_heads * value_length, np.float32)
        scores = np.empty(self.max_seq_len, np.float32)
        _check(lib().jmo_decode_layer(self._h, layer, position, window, _ptr(q), _ptr(k), _ptr(v),
                                      num_heads, num_kv_heads, key_length, value_length,
                                      rope_theta, rope_scale, int(neox), scale, _ptr(out),
                                      _ptr(scores)), "decode_layer")
        return out, q, k

    def prefill_layer(self, layer: int, start: int, q, k, v, num_heads: int, num_kv_heads: int,
                      key_length: int, value_length: int, rope_theta: float, rope_scale: float,
                      neox: bool, scale: float, window: int = 0):
        q, k, v = _f32(q).copy(), _f32(k).copy(), _f32(v)
        n = q.size // (num_heads * key_length)
        out = np.empty(n * num_heads * value_length, np.float32)
        scores = np.empty(self.max_seq_len, np.float32)
        _check(lib().jmo_prefill_layer(self._h, layer, start, n, window, _ptr(q), _ptr(k),
                                       _ptr(v), num_heads, num_kv_heads, key_length, value_length,
                                       rope_theta, rope_scale, int(neox), scale, _ptr(out),
                                       _ptr(scores)), "prefill_layer")
        return out, q, k


# ------------------------------------------------------------------ LayeredKvCache

class LayeredKvCache:
    """Restated ``LayeredKvCache`` (cache/LayeredKvCache.java); ring capacity 0 means LINEAR."""

    def __init__(self, max_seq_len: int, specs):
        kd = (ctypes.c_int * len(specs))(*[s[0] for s in specs])
        vd = (ctypes.c_int * len(specs))(*[s[1] for s in specs])
        rc = (ctypes.c_int * len(specs))(*[s[2] for s in specs])
        self._h = lib().jmo_lkv_create(max_seq_len, len(specs), kd, vd, rc)
        if not self._h:
            raise OracleError(ILLEGAL_ARGUMENT, "LayeredKvCache")
        self.specs = list(specs)
        self.max_seq_len = max_seq_len

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().jmo_lkv_destroy(h)
            self._h = None

    def store(self, layer, position, key, value):
        k, v = _f32(key), _f32(value)
        if not (0 <= layer < len(self.specs)):
            raise OracleError(ILLEGAL_ARGUMENT, "layer out of range")
        if k.size < self.specs[layer][0] or v.size < self.specs[layer][1]:
            raise OracleError(ILLEGAL_ARGUMENT, "key range")
        _check(lib().jmo_lkv_store(self._h, layer, position, _ptr(k), _ptr(v)), "store")

    def contains(self, layer, position) -> bool:
        r = lib().jmo_lkv_contains(self._h, layer, position)
        if r < 0:
            raise OracleError(-r, "contains")
        return bool(r)

    def attention_view(self, layer, frm, to):
        count = ctypes.c_int(0)
        spans = (ctypes.c_int * 8)()
        _check(lib().jmo_lkv_attention_view(self._h, layer, frm, to, ctypes.byref(count), spans),
               "attentionView")
        return [tuple(spans[4 * i:4 * i + 4]) for i in range(count.value)]

    def discard_from(self, position):
        _check(lib().jmo_lkv_discard_from(self._h, position), "discardFrom")

    def clear(self):
        lib().jmo_lkv_clear(self._h)

    def oldest_retained_position(self, layer):
        r = lib().jmo_lkv_oldest(self._h, layer)
        return None if r < 0 else r

    def newest_retained_position(self, layer):
        r = lib().jmo_lkv_newest(self._h, layer)
        return None if r < 0 else r

    def allocated_sequence_capacity(self, layer):
        return int(lib().jmo_lkv_allocated_capacity(self._h, layer))

    def physical_sequence_capacity(self, layer):
        return int(lib().jmo_lkv_physical_capacity(self._h, layer))

    def allocated_bytes(self):
        return int(lib().jmo_lkv_allocated_bytes(self._h))

    def maximum_bytes(self):
        return int(lib().jmo_lkv_maximum_bytes(self._h))

    def key_offset(self, layer, position):
        r = lib().jmo_lkv_key_offset(self._h, layer, position)
        if r < 0:
            raise OracleError(ILLEGAL_STATE, "keyOffset")
        return int(r)

    def key_buffer(self, layer):
        n = lib().jmo_lkv_buffer_length(self._h, layer, 0)
        if n == 0:
            return np.empty(0, np.float32)
        return np.ctypeslib.as_array(lib().jmo_lkv_key_buffer(self._h, layer), shape=(n,)).copy()

    def value_buffer(self, layer):
        n = lib().jmo_lkv_buffer_length(self._h, layer, 1)
        if n == 0:
            return np.empty(0, np.float32)
        return np.ctypeslib.as_array(lib().jmo_lkv_value_buffer(self._h, layer),
                                     shape=(n,)).copy()

    def gqa(self, layer, position, q, num_heads, num_kv_heads, head_dim, scale, window=0):
        q = _f32(q)
        out = np.empty(num_heads * head_dim, np.float32)
        scores = np.empty(self.max_seq_len, np.float32)
        _check(lib().jmo_gqa_layered(self._h, layer, position, window, _ptr(q), num_heads,
                                     num_kv_heads, head_dim, scale, _ptr(out), _ptr(scores)),
               "computeAttention")
        return out


# ------------------------------------------------------------------ attention over arrays

def gqa_rows(q, keys, values, num_heads: int, num_kv_heads: int, key_length: int,
             value_length: int, scale: float) -> np.ndarray:
    """GQA for one query token over contiguous rows keys[rows, Hkv*dk], values[rows, Hkv*dv]."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    rows = keys.size // (num_kv_heads * key_length)
    out = np.empty(num_heads * value_length, np.float32)
    scores = np.empty(max(rows, 1), np.float32)
    _check(lib().jmo_gqa_rows(_ptr(q), _ptr(keys), _ptr(values), rows, num_kv_heads * key_length,
                              num_kv_heads * value_length, num_heads, num_kv_heads, key_length,
                              value_length, scale, _ptr(out), _ptr(scores)), "gqa_rows")
    return out


def gqa_rows_batch(qs, keys_list, values_list, num_heads, num_kv_heads, key_length,
                   value_length, scale, threads=1, lanes8=False):
    """Independent sequences, work split over (sequence, kv head) units on ``threads`` threads.
    lanes8: dot products in eight partial sums (vectorised; timing only, not the parity oracle)."""
    n = len(qs)
    qs = [_f32(q) for q in qs]
    ks = [_f32(k) for k in keys_list]
    vs = [_f32(v) for v in values_list]
    outs = [np.empty(num_heads * value_length, np.float32) for _ in range(n)]
    rows = (ctypes.c_int * n)(*[k.size // (num_kv_heads * key_length) for k in ks])
    P = _f32p * n
    fn = lib().jmo_gqa_rows_batch8 if lanes8 else lib().jmo_gqa_rows_batch
    _check(fn(n, P(*[_ptr(a) for a in qs]), P(*[_ptr(a) for a in ks]),
                                    P(*[_ptr(a) for a in vs]), rows, num_kv_heads * key_length,
                                    num_kv_heads * value_length, num_heads, num_kv_heads,
                                    key_length, value_length, scale,
                                    P(*[_ptr(a) for a in outs]), threads), "gqa_rows_batch")
    return outs


# ------------------------------------------------------------------ GGUF block-quantized projection

FMT_Q4_0 = 0
FMT_Q8_0 = 1
FMT_Q4_K = 2
FMT_Q6_K = 3
FMT_Q5_K = 4
FMT_Q5_0 = 5
BLOCK_BYTES = {FMT_Q4_0: 18, FMT_Q8_0: 34, FMT_Q4_K: 144, FMT_Q6_K: 210, FMT_Q5_K: 176,
               FMT_Q5_0: 22}
BLOCK_ELEMS = {FMT_Q4_0: 32, FMT_Q8_0: 32, FMT_Q4_K: 256, FMT_Q6_K: 256, FMT_Q5_K: 256,
               FMT_Q5_0: 32}


def q8_k_quantize(x, batch: int, cols: int):
    """quantize_q8_k_batch (RS:3906-3952): (int8 [batch*cols], scales [batch*cols/256],
    int16 sums [batch*cols/16])."""
    x = _f32(x)
    if x.size != batch * cols or cols % 256:
        raise OracleError(ILLEGAL_ARGUMENT, "q8_k_quantize shape")
    q = np.empty(batch * cols, np.int8)
    scales = np.empty(batch * cols // 256, np.float32)
    sums = np.empty(batch * cols // 16, np.int16)
    lib().jmo_q8_k_quantize(_ptr(x), batch, cols, q.ctypes.data, _ptr(scales), sums.ctypes.data)
    return q, scales, sums


def q8_0_quantize(x, batch: int, cols: int):
    """quantizeInputs (NativeKernelLibraryTest.java:998-1017): (int8 [batch*cols], scales)."""
    x = _f32(x)
    if x.size != batch * cols or cols % 32:
        raise OracleError(ILLEGAL_ARGUMENT, "q8_0_quantize shape")
    q = np.empty(batch * cols, np.int8)
    scales = np.empty(batch * cols // 32, np.float32)
    lib().jmo_q8_0_quantize(_ptr(x), batch, cols, q.ctypes.data, _ptr(scales))
    return q, scales


def quantized_matmul(fmt: int, weights, x, batch: int, rows: int, cols: int) -> np.ndarray:
    """referenceQ4_0F32BatchedMatmul / referenceQ8_0F32BatchedMatmul /
    referenceQ5_0F32BatchedMatmul (NativeKernelLibraryTest.java:909-993) and backend-native's
    scalar K-quant row kernels (RS:3410-3577): out [batch, rows]."""
    if isinstance(weights, (bytes, bytearray)):
        weights = np.frombuffer(bytes(weights), np.uint8)
    w = np.ascontiguousarray(weights, dtype=np.uint8).reshape(-1)
    x = _f32(x)
    if fmt not in BLOCK_BYTES or cols % BLOCK_ELEMS[fmt] \
            or w.size < rows * cols // BLOCK_ELEMS[fmt] * BLOCK_BYTES[fmt] or x.size != batch * cols:
        raise OracleError(ILLEGAL_ARGUMENT, "quantized_matmul shape")
    out = np.empty(batch * rows, np.float32)
    _check(lib().jmo_quantized_matmul(fmt, w.ctypes.data, _ptr(x), batch, rows, cols, _ptr(out)),
           "quantized_matmul")
    return out.reshape(batch, rows)
