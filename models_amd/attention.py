"""Python mirror of backend-java's attention/KV-cache contract over ``libjmodels_attn.so``.

This is the host side above the C ABI (``include/jmodels_attn.h``). Names follow the reference
(paths relative to ``backend-java/src/main/java/com/integrallis/models/backend/purejava/``):

* :class:`HipAttentionLibrary` — ``NativeKernelLibrary.open`` (backend-native
  ``NativeKernelLibrary.java:126-191``): load the library, check the ABI version and the
  required capabilities, create a context; ``close`` is idempotent.
* :class:`HipRotaryTable` — ``ops/RotaryTable.java`` (factors resident in HBM).
* :class:`HipKvCache` — ``cache/KvCache.java`` / ``cache/LayeredKvCache.java`` resident in HBM:
  ``store``, ``key_slice``/``value_slice``, ``contains``, ``discard_from``, ``clear``.
* :class:`HipQkNorm` — a layer's QK-norm weights (``LlamaForwardPass.normalizeHead``).
* :class:`AttentionLayer` — the per-layer flags ``LlamaConfig`` supplies (heads, window, NeoX,
  scale, RoPE table, QK-norm).
* ``decode`` / ``attend`` / ``append`` / ``prefill`` — the attention block of
  ``llama/LlamaForwardPass.java`` (:1069-1128, :1479-1541, :793-839).

Shape errors raise ``ValueError`` before crossing the boundary (as the reference validates before
the downcall, ``NativeKernelLibrary.java:552-578``); a non-zero native status raises
:class:`AttentionStatusError` (the reference's ``IllegalStateException`` mapping, :771-779).
There is no CPU fallback: without the HIP library and a gfx950 GPU every call fails loudly.
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

ABI_VERSION = 2

OK = 0
NULL_POINTER = 1
INVALID_SHAPE = 2
BUFFER_TOO_SMALL = 3
PANIC = 4
DEVICE_ERROR = 5
OUT_OF_RANGE = 6
UNAVAILABLE = 7
NON_FINITE = 8
NOT_CAPTURABLE = 9

CAP_DECODE_F32 = 1 << 0
CAP_DECODE_F16 = 1 << 1
CAP_PREFILL_MFMA = 1 << 2
CAP_RAGGED_DECODE = 1 << 3
CAP_SLIDING_WINDOW = 1 << 4
CAP_RING_LAYERS = 1 << 5
CAP_DEVICE_POINTERS = 1 << 6
CAP_QK_NORM = 1 << 7
CAP_VALUE_NORM = 1 << 8

NORM_VALUE_RMS = 1

KV_F32 = 0
KV_F16 = 1
WEIGHTS_Q4_0 = 0
WEIGHTS_Q8_0 = 1
WEIGHTS_Q4_K = 2
WEIGHTS_Q6_K = 3
WEIGHTS_Q5_K = 4
WEIGHTS_Q5_0 = 5
ADDEND_NONE = 0
ADDEND_BIAS = 1
ADDEND_RESIDUAL = 2

EXPORTS = (
    "jmodels_attn_abi_version", "jmodels_attn_capabilities", "jmodels_attn_status_name",
    "jmodels_attn_last_error", "jmodels_attn_context_create", "jmodels_attn_context_destroy",
    "jmodels_attn_context_synchronize", "jmodels_attn_context_stream", "jmodels_attn_rope_create",
    "jmodels_attn_rope_destroy", "jmodels_attn_kv_create", "jmodels_attn_kv_destroy",
    "jmodels_attn_kv_clear", "jmodels_attn_kv_discard_from", "jmodels_attn_kv_contains",
    "jmodels_attn_kv_store", "jmodels_attn_kv_read", "jmodels_attn_kv_bytes",
    "jmodels_attn_append", "jmodels_attn_attend", "jmodels_attn_decode", "jmodels_attn_prefill",
    "jmodels_attn_append_device", "jmodels_attn_attend_device", "jmodels_attn_decode_device",
    "jmodels_attn_prefill_device", "jmodels_attn_attend_causal",
    "jmodels_attn_attend_causal_device", "jmodels_attn_norm_create", "jmodels_attn_norm_create_ex",
    "jmodels_attn_norm_destroy", "jmodels_attn_decode_device_noalloc",
    "jmodels_attn_kv_create_layered", "jmodels_attn_quantized_matmul_device",
    "jmodels_attn_quantized_grouped_matmul_device",
)

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIBRARY = os.path.join(_HERE, "libjmodels_attn.so")
LIBRARY_PROPERTY = "MODELS_HIP_ATTENTION_LIBRARY"


class AttentionStatusError(RuntimeError):
    """A native call returned a non-zero status."""

    def __init__(self, status: int, name: str, detail: str, call: str):
        super().__init__(f"{call} failed with {name} ({status}): {detail}")
        self.status = status
        self.status_name = name
        self.detail = detail


class _Layer(ctypes.Structure):
    _fields_ = [
        ("layer", ctypes.c_uint32),
        ("num_heads", ctypes.c_uint32),
        ("sliding_window", ctypes.c_uint32),
        ("neox", ctypes.c_uint32),
        ("scale", ctypes.c_float),
        ("reserved", ctypes.c_uint32),
        ("rope", ctypes.c_void_p),
        ("qk_norm", ctypes.c_void_p),
    ]


_u32, _u64, _i32, _cf = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_float
_vp = ctypes.c_void_p
_u32p = ctypes.POINTER(ctypes.c_uint32)
_LP = ctypes.POINTER(_Layer)


def _declare(lib: ctypes.CDLL) -> None:
    sig = {
        "jmodels_attn_abi_version": (_u32, []),
        "jmodels_attn_capabilities": (_u64, []),
        "jmodels_attn_status_name": (ctypes.c_char_p, [_i32]),
        "jmodels_attn_last_error": (ctypes.c_char_p, []),
        "jmodels_attn_context_create": (_vp, [_i32]),
        "jmodels_attn_context_destroy": (_i32, [_vp]),
        "jmodels_attn_context_synchronize": (_i32, [_vp]),
        "jmodels_attn_context_stream": (_i32, [_vp, ctypes.POINTER(_vp)]),
        "jmodels_attn_rope_create": (_i32, [_vp, _u32, _cf, _cf, _vp, _u32, _u32,
                                            ctypes.POINTER(_vp)]),
        "jmodels_attn_rope_destroy": (_i32, [_vp]),
        "jmodels_attn_norm_create": (_i32, [_vp, _u32, _vp, _vp, _cf, ctypes.POINTER(_vp)]),
        "jmodels_attn_norm_create_ex": (_i32, [_vp, _u32, _vp, _vp, _cf, _u32, ctypes.POINTER(_vp)]),
        "jmodels_attn_norm_destroy": (_i32, [_vp]),
        "jmodels_attn_kv_create": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _vp,
                                          ctypes.POINTER(_vp)]),
        "jmodels_attn_kv_create_layered": (_i32, [_vp, _u32, _u32, _u32, _vp, _u32, ctypes.POINTER(_vp)]),
        "jmodels_attn_kv_destroy": (_i32, [_vp]),
        "jmodels_attn_quantized_matmul_device": (_i32, [_vp, _u32, _vp, _u64, _vp, _u64, _vp, _u64,
                                                        _u32, _u32, _u32, _vp, _u32]),
        "jmodels_attn_quantized_grouped_matmul_device": (_i32, [_vp, _vp, _vp, _vp, _vp, _u32, _vp,
                                                                _u64, _vp, _u64, _u32, _u32, _vp,
                                                                _u32]),
        "jmodels_attn_kv_clear": (_i32, [_vp, _i32]),
        "jmodels_attn_kv_discard_from": (_i32, [_vp, _u32, _u32]),
        "jmodels_attn_kv_contains": (_i32, [_vp, _u32, _u32, _u32, ctypes.POINTER(_i32)]),
        "jmodels_attn_kv_store": (_i32, [_vp, _vp, _u32, _u32, _u32, _vp, _u64, _vp, _u64]),
        "jmodels_attn_kv_read": (_i32, [_vp, _vp, _u32, _u32, _u32, _u32, _vp, _u64, _vp, _u64]),
        "jmodels_attn_kv_bytes": (_i32, [_vp, ctypes.POINTER(_u64)]),
    }
    rows = [_vp, _vp, _LP, _u32, _u32p, _u32p]
    for name in ("jmodels_attn_append", "jmodels_attn_append_device"):
        sig[name] = (_i32, rows + [_vp, _u64, _vp, _u64, _vp, _u64, _vp, _u64])
    for name in ("jmodels_attn_attend", "jmodels_attn_attend_device"):
        sig[name] = (_i32, rows + [_vp, _u64, _vp, _u64])
    for name in ("jmodels_attn_decode", "jmodels_attn_decode_device",
                 "jmodels_attn_decode_device_noalloc"):
        sig[name] = (_i32, rows + [_vp, _u64, _vp, _u64, _vp, _u64, _vp, _u64])
    for name in ("jmodels_attn_attend_causal", "jmodels_attn_attend_causal_device"):
        sig[name] = (_i32, [_vp, _vp, _LP, _u32, _u32, _u32, _vp, _u64, _vp, _u64])
    for name in ("jmodels_attn_prefill", "jmodels_attn_prefill_device"):
        sig[name] = (_i32, [_vp, _vp, _LP, _u32, _u32, _u32, _vp, _u64, _vp, _u64, _vp, _u64,
                            _vp, _u64])
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


_LIBS: dict = {}


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """dlopen the HIP library (``MODELS_HIP_ATTENTION_LIBRARY`` overrides the in-tree path) and
    verify every export of ``include/jmodels_attn.h`` and the ABI version; no GPU is touched."""
    path = path or os.environ.get(LIBRARY_PROPERTY) or DEFAULT_LIBRARY
    path = os.path.abspath(path)
    if path in _LIBS:
        return _LIBS[path]
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"HIP attention library not found at {path}; build it with `python -m models_amd.build`")
    lib = ctypes.CDLL(path)
    missing = [name for name in EXPORTS if not hasattr(lib, name)]
    if missing:
        raise RuntimeError(f"{path} lacks exports: {missing}")
    _declare(lib)
    version = lib.jmodels_attn_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"ABI version mismatch: library {version}, binding {ABI_VERSION}")
    _LIBS[path] = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def uses_sliding_window(layer: int, pattern: int, sliding_window: int) -> bool:
    """LlamaConfig.usesSlidingWindow for the Gemma family (llama/LlamaConfig.java:157-162)."""
    return sliding_window > 0 and layer % pattern < pattern - 1


def attention_start_position(position: int, sliding_window: int) -> int:
    """LlamaConfig.attentionStartPosition, causal branch (llama/LlamaConfig.java:184-195)."""
    if position < 0:
        raise ValueError("position must be >= 0")
    if sliding_window <= 0:
        return 0
    return max(0, position - sliding_window + 1)


class HipAttentionLibrary:
    """Loaded library + one context on one GPU (NativeKernelLibrary analogue)."""

    def __init__(self, device: int = 0, path: Optional[str] = None,
                 required_capabilities: int = 0):
        self.lib = load_library(path)
        caps = self.lib.jmodels_attn_capabilities()
        if caps & required_capabilities != required_capabilities:
            raise RuntimeError(f"library lacks capabilities {required_capabilities & ~caps:#x}")
        self.capabilities = caps
        ctx = self.lib.jmodels_attn_context_create(device)
        if not ctx:
            raise AttentionStatusError(
                -1, "CONTEXT_CREATE_FAILED",
                self.lib.jmodels_attn_last_error().decode(), "jmodels_attn_context_create")
        self.ctx = ctx
        self.device = device

    # ---- plumbing

    def check(self, status: int, call: str) -> None:
        if status != OK:
            name = self.lib.jmodels_attn_status_name(status).decode()
            detail = self.lib.jmodels_attn_last_error().decode()
            raise AttentionStatusError(status, name, detail, call)

    def synchronize(self) -> None:
        self.check(self.lib.jmodels_attn_context_synchronize(self.ctx), "synchronize")

    def stream(self) -> int:
        out = _vp()
        self.check(self.lib.jmodels_attn_context_stream(self.ctx, ctypes.byref(out)), "stream")
        return out.value or 0

    def close(self) -> None:
        if getattr(self, "ctx", None):
            self.check(self.lib.jmodels_attn_context_destroy(self.ctx), "context_destroy")
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- factories

    def rotary_table(self, rotary_dim: int, theta: float, frequency_scale: float = 1.0,
                     max_positions: int = 4096, frequency_factors=None) -> "HipRotaryTable":
        return HipRotaryTable(self, rotary_dim, theta, frequency_scale, max_positions,
                              frequency_factors)

    def qk_norm(self, head_dim: int, q_weight=None, k_weight=None,
                eps: float = 1e-6, value_rms: bool = False) -> "HipQkNorm":
        return HipQkNorm(self, head_dim, q_weight, k_weight, eps, value_rms)

    def kv_cache(self, num_layers: int, max_seq_len: int, num_kv_heads: int, key_length: int,
                 value_length: int, half_precision: bool = True, sequences: int = 1,
                 ring_capacity: Optional[Sequence[int]] = None) -> "HipKvCache":
        """One shape for every layer (KvCache, or LayeredKvCache with ring_capacity)."""
        rings = list(ring_capacity) if ring_capacity is not None else [0] * num_layers
        if len(rings) != num_layers:
            raise ValueError("ring_capacity needs one entry per layer")
        specs = [LayerSpec(num_kv_heads, key_length, value_length, r) for r in rings]
        return HipKvCache(self, specs, max_seq_len, half_precision, sequences, uniform=True)

    def layered_kv_cache(self, specs: Sequence["LayerSpec"], max_seq_len: int,
                         half_precision: bool = True, sequences: int = 1) -> "HipKvCache":
        """LayeredKvCache(maxSeqLen, LayerSpec[]) (cache/LayeredKvCache.java:124-156): per-layer kv
        heads, head lengths and retention, as Gemma4KvCache builds them
        (gemma4/Gemma4KvCache.java:39-47)."""
        return HipKvCache(self, list(specs), max_seq_len, half_precision, sequences, uniform=False)


    # ---- quantized projections (device pointers, asynchronous on the context stream)

    def quantized_matmul_device(self, fmt: int, weights_ptr: int, weight_bytes: int, x_ptr: int,
                                x_elems: int, out_ptr: int, out_elems: int, batch: int, rows: int,
                                cols: int, addend_ptr: Optional[int] = None,
                                addend_mode: int = ADDEND_NONE) -> None:
        """jmodels_quantized_f32_batched_matmul_with_context on device memory (Q4_0, Q8_0, Q5_0,
        Q4_K, Q5_K, Q6_K)."""
        self.check(self.lib.jmodels_attn_quantized_matmul_device(
            self.ctx, fmt, weights_ptr, weight_bytes, x_ptr, x_elems, out_ptr, out_elems, batch,
            rows, cols, addend_ptr, addend_mode), "quantized_matmul_device")

    def quantized_grouped_matmul_device(self, formats, weight_ptrs, weight_bytes, rows, x_ptr: int,
                                        x_elems: int, out_ptr: int, out_elems: int, batch: int,
                                        cols: int, addend_ptrs=None,
                                        addend_mode: int = ADDEND_NONE) -> None:
        """Q/K/V (or any up to 16 matrices) over one activation batch; outputs matrix after
        matrix, each [batch][rows]."""
        n = len(formats)
        fm = (ctypes.c_uint32 * n)(*formats)
        wp = (ctypes.c_void_p * n)(*weight_ptrs)
        wb = (ctypes.c_uint64 * n)(*weight_bytes)
        rw = (ctypes.c_uint32 * n)(*rows)
        ad = (ctypes.c_void_p * n)(*addend_ptrs) if addend_ptrs is not None else None
        self.check(self.lib.jmodels_attn_quantized_grouped_matmul_device(
            self.ctx, fm, wp, wb, rw, n, x_ptr, x_elems, out_ptr, out_elems, batch, cols, ad,
            addend_mode), "quantized_grouped_matmul_device")

    def quantized_matmul(self, fmt: int, weights, x, batch: int, rows: int, cols: int,
                         addend=None, addend_mode: int = ADDEND_NONE) -> np.ndarray:
        """Host-buffer convenience over quantized_matmul_device: uploads the GGUF weight bytes,
        the activations [batch][cols] and the addend, runs, returns out [batch, rows]."""
        from models_amd import hip_runtime as rt
        wb = np.frombuffer(bytes(weights), np.uint8) if isinstance(weights, (bytes, bytearray)) \
            else np.ascontiguousarray(weights, np.uint8).reshape(-1)
        xs = _f32(x)
        dw, dx = rt.DeviceArray.from_host(wb), rt.DeviceArray.from_host(xs)
        dout = rt.DeviceArray(batch * rows)
        dadd = rt.DeviceArray.from_host(_f32(addend)) if addend is not None else None
        try:
            self.quantized_matmul_device(fmt, dw.ptr, wb.size, dx.ptr, xs.size, dout.ptr,
                                         batch * rows, batch, rows, cols,
                                         dadd.ptr if dadd is not None else None, addend_mode)
            self.synchronize()
            return dout.download().reshape(batch, rows)
        finally:
            for d in (dw, dx, dout, dadd):
                if d is not None:
                    d.free()


class HipRotaryTable:
    """RotaryTable (ops/RotaryTable.java:48-186) with factors for [0, max_positions) in HBM."""

    def __init__(self, owner: HipAttentionLibrary, rotary_dim: int, theta: float,
                 frequency_scale: float, max_positions: int, frequency_factors=None):
        self.owner = owner
        if rotary_dim <= 0 or rotary_dim % 2:
            raise ValueError(f"rotaryDim must be positive and even: {rotary_dim}")
        factors = None
        fp, fc = None, 0
        if frequency_factors is not None:
            factors = _f32(frequency_factors)
            fp, fc = _ptr(factors), factors.size
        out = _vp()
        owner.check(owner.lib.jmodels_attn_rope_create(owner.ctx, rotary_dim, theta,
                                                       frequency_scale, fp, fc, max_positions,
                                                       ctypes.byref(out)), "rope_create")
        self.handle = out.value
        self.rotary_dim = rotary_dim
        self.max_positions = max_positions

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.owner.check(self.owner.lib.jmodels_attn_rope_destroy(self.handle), "rope_destroy")
            self.handle = None


class HipQkNorm:
    """A layer's attn_q_norm / attn_k_norm weights (llama/LlamaWeights.java:99-101) in HBM; each q
    and k head is RMS-normalised with them before RoPE (LlamaForwardPass.normalizeHead, :1672-1676).
    A missing weight (None) leaves that side unnormalised, as an empty weight array does. With
    value_rms, each value head is also RMS-normalised without a weight before it is stored
    (Gemma4ForwardPass, gemma4/Gemma4ForwardPass.java:990-996; Gemma4Math.normalizeWithoutWeight)."""

    def __init__(self, owner: HipAttentionLibrary, head_dim: int, q_weight, k_weight, eps: float,
                 value_rms: bool = False):
        self.owner = owner
        qw = None if q_weight is None else _f32(q_weight)
        kw = None if k_weight is None else _f32(k_weight)
        for w in (qw, kw):
            if w is not None and w.size != head_dim:
                raise ValueError(f"norm weight has {w.size} elements, head_dim is {head_dim}")
        out = _vp()
        owner.check(owner.lib.jmodels_attn_norm_create_ex(
            owner.ctx, head_dim, None if qw is None else _ptr(qw), None if kw is None else _ptr(kw),
            eps, NORM_VALUE_RMS if value_rms else 0, ctypes.byref(out)), "norm_create")
        self.handle = out.value
        self.head_dim, self.eps, self.value_rms = head_dim, eps, value_rms

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.owner.check(self.owner.lib.jmodels_attn_norm_destroy(self.handle), "norm_destroy")
            self.handle = None


@dataclass
class AttentionLayer:
    """Per-layer attention parameters (LlamaConfig flags for one layer)."""

    layer: int
    num_heads: int
    sliding_window: int = 0
    neox: bool = False
    scale: float = 0.0  # 0 -> (float)(1/sqrt(key_length))
    rope: Optional[HipRotaryTable] = None
    qk_norm: Optional[HipQkNorm] = None

    def struct(self) -> _Layer:
        return _Layer(self.layer, self.num_heads, self.sliding_window, int(bool(self.neox)),
                      self.scale, 0, self.rope.handle if self.rope is not None else None,
                      self.qk_norm.handle if self.qk_norm is not None else None)


@dataclass(frozen=True)
class LayerSpec:
    """LayeredKvCache.LayerSpec (cache/LayeredKvCache.java:41-64) with keyDim = num_kv_heads *
    key_length and valueDim = num_kv_heads * value_length; ring_capacity 0 = LINEAR."""

    num_kv_heads: int
    key_length: int
    value_length: int
    ring_capacity: int = 0

    @property
    def key_dim(self) -> int:
        return self.num_kv_heads * self.key_length

    @property
    def value_dim(self) -> int:
        return self.num_kv_heads * self.value_length


class _LayerSpecC(ctypes.Structure):
    _fields_ = [("num_kv_heads", ctypes.c_uint32), ("key_length", ctypes.c_uint32),
                ("value_length", ctypes.c_uint32), ("ring_capacity", ctypes.c_uint32)]


class HipKvCache:
    """Device-resident KV cache for ``sequences`` independent sessions (KvCache / LayeredKvCache).
    Shapes are per layer (``specs``); num_kv_heads, key_length, value_length, key_dim and
    value_dim name layer 0's for caches of one shape."""

    def __init__(self, owner: HipAttentionLibrary, specs: Sequence[LayerSpec], max_seq_len: int,
                 half_precision: bool, sequences: int, uniform: bool):
        self.owner = owner
        self.specs = list(specs)
        self.num_layers, self.max_seq_len = len(self.specs), max_seq_len
        first = self.specs[0]
        self.num_kv_heads, self.key_length, self.value_length = (first.num_kv_heads, first.key_length,
                                                                 first.value_length)
        self.key_dim, self.value_dim = first.key_dim, first.value_dim
        self.sequences = sequences
        self.half_precision = half_precision
        out = _vp()
        dtype = KV_F16 if half_precision else KV_F32
        if uniform:
            ring = (ctypes.c_uint32 * self.num_layers)(*[sp.ring_capacity for sp in self.specs])
            owner.check(owner.lib.jmodels_attn_kv_create(
                owner.ctx, sequences, self.num_layers, max_seq_len, first.num_kv_heads,
                first.key_length, first.value_length, dtype, ring, ctypes.byref(out)), "kv_create")
        else:
            arr = (_LayerSpecC * self.num_layers)(
                *[_LayerSpecC(sp.num_kv_heads, sp.key_length, sp.value_length, sp.ring_capacity)
                  for sp in self.specs])
            owner.check(owner.lib.jmodels_attn_kv_create_layered(
                owner.ctx, sequences, self.num_layers, max_seq_len, arr, dtype, ctypes.byref(out)),
                "kv_create_layered")
        self.handle = out.value

    def spec(self, layer: int) -> LayerSpec:
        """Layer ``layer``'s shape; for a layer outside the cache, layer 0's, so that the call
        reaches the library and fails there with its OUT_OF_RANGE status."""
        return self.specs[layer] if 0 <= layer < self.num_layers else self.specs[0]

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.owner.check(self.owner.lib.jmodels_attn_kv_destroy(self.handle), "kv_destroy")
            self.handle = None

    # ---- KvCache API

    def store(self, layer: int, position: int, key, value, sequence: int = 0) -> None:
        k = _f32(key)
        v = _f32(value)
        sp = self.spec(layer)
        if k.size != sp.key_dim:
            raise ValueError(f"key.length must equal {sp.key_dim}: {k.size}")
        if v.size != sp.value_dim:
            raise ValueError(f"value.length must equal {sp.value_dim}: {v.size}")
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_store(o.ctx, self.handle, sequence, layer, position,
                                            _ptr(k), k.size, _ptr(v), v.size), "kv_store")

    def read(self, layer: int, frm: int, to: int, sequence: int = 0):
        n = max(to - frm, 0)
        sp = self.spec(layer)
        keys = np.empty(n * sp.key_dim, np.float32)
        values = np.empty(n * sp.value_dim, np.float32)
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_read(o.ctx, self.handle, sequence, layer, frm, to,
                                           _ptr(keys), keys.size, _ptr(values), values.size),
                "kv_read")
        return keys, values

    def key_slice(self, layer: int, frm: int, to: int, sequence: int = 0) -> np.ndarray:
        return self.read(layer, frm, to, sequence)[0]

    def value_slice(self, layer: int, frm: int, to: int, sequence: int = 0) -> np.ndarray:
        return self.read(layer, frm, to, sequence)[1]

    def contains(self, layer: int, position: int, sequence: int = 0) -> bool:
        out = ctypes.c_int32()
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_contains(self.handle, sequence, layer, position,
                                               ctypes.byref(out)), "kv_contains")
        return bool(out.value)

    def discard_from(self, position: int, sequence: int = 0) -> None:
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_discard_from(self.handle, sequence, position),
                "kv_discard_from")

    def clear(self, sequence: int = -1) -> None:
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_clear(self.handle, sequence), "kv_clear")

    def device_bytes(self) -> int:
        out = ctypes.c_uint64()
        o = self.owner
        o.check(o.lib.jmodels_attn_kv_bytes(self.handle, ctypes.byref(out)), "kv_bytes")
        return out.value

    # ---- attention (host buffers, synchronous)

    def _rows(self, sequences, positions):
        seq = np.ascontiguousarray(sequences, dtype=np.uint32).reshape(-1)
        pos = np.ascontiguousarray(positions, dtype=np.uint32).reshape(-1)
        if seq.size != pos.size or seq.size == 0:
            raise ValueError("sequences and positions must be non-empty and of equal length")
        return seq, pos

    def _check_heads(self, layer: AttentionLayer):
        if layer.num_heads <= 0 or layer.num_heads % self.spec(layer.layer).num_kv_heads:
            raise ValueError("numHeads must be divisible by numKvHeads")

    def append(self, layer: AttentionLayer, positions, q, k, v, sequences=None):
        """RoPE + store; returns the rotated queries."""
        self._check_heads(layer)
        seq, pos = self._rows(np.zeros(np.size(positions)) if sequences is None else sequences,
                              positions)
        q, k, v = _f32(q), _f32(k), _f32(v)
        qr = np.empty_like(q)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_append(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size,
            _ptr(qr), qr.size), "append")
        return qr

    def attend(self, layer: AttentionLayer, positions, q, sequences=None) -> np.ndarray:
        """groupedQueryAttention for already-rotated queries."""
        self._check_heads(layer)
        seq, pos = self._rows(np.zeros(np.size(positions)) if sequences is None else sequences,
                              positions)
        q = _f32(q)
        out = np.empty(seq.size * layer.num_heads * self.spec(layer.layer).value_length, np.float32)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_attend(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), _ptr(q), q.size, _ptr(out), out.size), "attend")
        return out

    def decode(self, layer: AttentionLayer, positions, q, k, v, sequences=None) -> np.ndarray:
        """One token per session: RoPE, append, attend."""
        self._check_heads(layer)
        seq, pos = self._rows(np.zeros(np.size(positions)) if sequences is None else sequences,
                              positions)
        q, k, v = _f32(q), _f32(k), _f32(v)
        out = np.empty(seq.size * layer.num_heads * self.spec(layer.layer).value_length, np.float32)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_decode(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size,
            _ptr(out), out.size), "decode")
        return out

    def prefill(self, layer: AttentionLayer, start: int, q, k, v, sequence: int = 0) -> np.ndarray:
        """Causal prefill of consecutive rows start .. start+n-1."""
        self._check_heads(layer)
        q, k, v = _f32(q), _f32(k), _f32(v)
        sp = self.spec(layer.layer)
        n = q.size // (layer.num_heads * sp.key_length)
        out = np.empty(n * layer.num_heads * sp.value_length, np.float32)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_prefill(
            o.ctx, self.handle, ctypes.byref(st), sequence, start, n, _ptr(q), q.size, _ptr(k),
            k.size, _ptr(v), v.size, _ptr(out), out.size), "prefill")
        return out

    def attend_causal(self, layer: AttentionLayer, start: int, q, sequence: int = 0) -> np.ndarray:
        """computeBatchedAttention: causal attention of cached rows start .. start+n-1."""
        self._check_heads(layer)
        q = _f32(q)
        sp = self.spec(layer.layer)
        n = q.size // (layer.num_heads * sp.key_length)
        out = np.empty(n * layer.num_heads * sp.value_length, np.float32)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_attend_causal(
            o.ctx, self.handle, ctypes.byref(st), sequence, start, n, _ptr(q), q.size, _ptr(out),
            out.size), "attend_causal")
        return out

    # ---- attention (device pointers, asynchronous on the context stream)

    def attend_causal_device(self, layer: AttentionLayer, sequence: int, start: int, n: int,
                             q_ptr: int, q_elems: int, out_ptr: int, out_elems: int) -> None:
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_attend_causal_device(
            o.ctx, self.handle, ctypes.byref(st), sequence, start, n, q_ptr, q_elems, out_ptr,
            out_elems), "attend_causal_device")


    def decode_device(self, layer: AttentionLayer, sequences, positions, q_ptr: int, q_elems: int,
                      k_ptr: int, k_elems: int, v_ptr: int, v_elems: int, out_ptr: int,
                      out_elems: int) -> None:
        seq, pos = self._rows(sequences, positions)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_decode_device(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), q_ptr, q_elems, k_ptr, k_elems, v_ptr, v_elems, out_ptr,
            out_elems), "decode_device")

    def decode_device_noalloc(self, layer: AttentionLayer, sequences, positions, q_ptr: int,
                              q_elems: int, k_ptr: int, k_elems: int, v_ptr: int, v_elems: int,
                              out_ptr: int, out_elems: int) -> None:
        """decode_device on the GPU's fixed scratch: allocates no device memory."""
        seq, pos = self._rows(sequences, positions)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_decode_device_noalloc(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), q_ptr, q_elems, k_ptr, k_elems, v_ptr, v_elems, out_ptr,
            out_elems), "decode_device_noalloc")

    def attend_device(self, layer: AttentionLayer, sequences, positions, q_ptr: int,
                      q_elems: int, out_ptr: int, out_elems: int) -> None:
        seq, pos = self._rows(sequences, positions)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_attend_device(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), q_ptr, q_elems, out_ptr, out_elems), "attend_device")

    def append_device(self, layer: AttentionLayer, sequences, positions, q_ptr: int,
                      q_elems: int, k_ptr: int, k_elems: int, v_ptr: int, v_elems: int,
                      qrot_ptr: int = 0, qrot_elems: int = 0) -> None:
        seq, pos = self._rows(sequences, positions)
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_append_device(
            o.ctx, self.handle, ctypes.byref(st), seq.size, seq.ctypes.data_as(_u32p),
            pos.ctypes.data_as(_u32p), q_ptr, q_elems, k_ptr, k_elems, v_ptr, v_elems,
            qrot_ptr or None, qrot_elems), "append_device")

    def prefill_device(self, layer: AttentionLayer, sequence: int, start: int, n: int,
                       q_ptr: int, q_elems: int, k_ptr: int, k_elems: int, v_ptr: int,
                       v_elems: int, out_ptr: int, out_elems: int) -> None:
        st = layer.struct()
        o = self.owner
        o.check(o.lib.jmodels_attn_prefill_device(
            o.ctx, self.handle, ctypes.byref(st), sequence, start, n, q_ptr, q_elems, k_ptr,
            k_elems, v_ptr, v_elems, out_ptr, out_elems), "prefill_device")


def default_scale(key_length: int) -> float:
    """(float)(1.0 / Math.sqrt(keyLength)) (llama/LlamaForwardPass.java:1559)."""
    return float(np.float32(1.0 / math.sqrt(key_length)))
