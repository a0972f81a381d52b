/*
 * FFM binding of libjmodels_attn (include/jmodels_attn.h, ABI 2): grouped-query attention, KV
 * cache and the quantized projections around them on an MI355X, for backend-java. It follows
 * backend-native's NativeKernelLibrary (backend-native/src/main/java/com/integrallis/models/
 * backend/nativekernel/NativeKernelLibrary.java:126-191 open, 601-642 calls, 689-713 close,
 * 771-779 status names): the ABI version and the capability mask are checked when the library is
 * opened, every call checks its status and turns a failure into an exception naming the status,
 * and close is synchronized and idempotent.
 *
 * Not compiled in this repository (no JDK is installed where it was written). Every downcall's
 * FunctionDescriptor is in DOWNCALLS below, one entry per export of the header, in the header's
 * order; tests/test_java_binding_cpu.py checks that table against include/jmodels_attn.h.
 */
package com.integrallis.models.backend.hip;

import static java.lang.foreign.ValueLayout.ADDRESS;
import static java.lang.foreign.ValueLayout.JAVA_FLOAT;
import static java.lang.foreign.ValueLayout.JAVA_INT;
import static java.lang.foreign.ValueLayout.JAVA_LONG;
import static java.util.Map.entry;

import java.lang.foreign.Arena;
import java.lang.foreign.FunctionDescriptor;
import java.lang.foreign.Linker;
import java.lang.foreign.MemoryLayout;
import java.lang.foreign.MemorySegment;
import java.lang.foreign.StructLayout;
import java.lang.foreign.SymbolLookup;
import java.lang.invoke.MethodHandle;
import java.nio.file.Files;
import java.nio.file.Path;
import java.util.HashMap;
import java.util.Map;
import java.util.Objects;

/** One HIP attention context on one GPU; one caller at a time (the methods are synchronized). */
public final class HipAttentionLibrary implements AutoCloseable {

  /** The ABI this binding was written against (JMODELS_ATTN_ABI_VERSION). */
  public static final int ABI_VERSION = 2;

  /** System property and environment variable naming the library file. */
  public static final String LIBRARY_PROPERTY = "models.hip.attention.library";

  public static final String LIBRARY_ENVIRONMENT = "MODELS_HIP_ATTENTION_LIBRARY";

  // Capability bits (JMODELS_ATTN_CAP_*).
  public static final long CAP_DECODE_F32 = 1L << 0;
  public static final long CAP_DECODE_F16 = 1L << 1;
  public static final long CAP_PREFILL_MFMA = 1L << 2;
  public static final long CAP_RAGGED_DECODE = 1L << 3;
  public static final long CAP_SLIDING_WINDOW = 1L << 4;
  public static final long CAP_RING_LAYERS = 1L << 5;
  public static final long CAP_DEVICE_POINTERS = 1L << 6;
  public static final long CAP_QK_NORM = 1L << 7;
  public static final long CAP_VALUE_NORM = 1L << 8;
  public static final long CAP_QUANT_MATMUL = 1L << 9;

  // Status codes: 0-4 keep backend-native's meaning (RS:78-82), 5-9 are this library's.
  public static final int OK = 0;
  public static final int NULL_POINTER = 1;
  public static final int INVALID_SHAPE = 2;
  public static final int BUFFER_TOO_SMALL = 3;
  public static final int PANIC = 4;
  public static final int DEVICE_ERROR = 5;
  public static final int OUT_OF_RANGE = 6;
  public static final int UNAVAILABLE = 7;
  public static final int NON_FINITE = 8;
  public static final int NOT_CAPTURABLE = 9;

  public static final int KV_F32 = 0;
  public static final int KV_F16 = 1;
  public static final int NORM_VALUE_RMS = 1;
  public static final int ADDEND_NONE = 0;
  public static final int ADDEND_BIAS = 1;
  public static final int ADDEND_RESIDUAL = 2;

  /** jmodels_attn_layer: one layer's parameters for a call (40 bytes). */
  public static final StructLayout LAYER =
      MemoryLayout.structLayout(
          JAVA_INT.withName("layer"),
          JAVA_INT.withName("num_heads"),
          JAVA_INT.withName("sliding_window"),
          JAVA_INT.withName("neox"),
          JAVA_FLOAT.withName("scale"),
          JAVA_INT.withName("reserved"),
          ADDRESS.withName("rope"),
          ADDRESS.withName("qk_norm"));

  /** jmodels_attn_layer_spec: one layer of a layered cache (16 bytes). */
  public static final StructLayout LAYER_SPEC =
      MemoryLayout.structLayout(
          JAVA_INT.withName("num_kv_heads"),
          JAVA_INT.withName("key_length"),
          JAVA_INT.withName("value_length"),
          JAVA_INT.withName("ring_capacity"));

  // Parameter shapes shared by several entry points (uint32_t and int32_t are JAVA_INT, uint64_t
  // JAVA_LONG, float JAVA_FLOAT, every pointer ADDRESS).
  private static final FunctionDescriptor STATUS_OF_HANDLE = FunctionDescriptor.of(JAVA_INT, ADDRESS);
  private static final FunctionDescriptor ROWS_APPEND =
      FunctionDescriptor.of(
          JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, ADDRESS, ADDRESS,
          ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG);
  private static final FunctionDescriptor ROWS_ATTEND =
      FunctionDescriptor.of(
          JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, ADDRESS, ADDRESS,
          ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG);
  private static final FunctionDescriptor ROWS_DECODE = ROWS_APPEND;
  private static final FunctionDescriptor CAUSAL =
      FunctionDescriptor.of(
          JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT,
          ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG);
  private static final FunctionDescriptor PREFILL =
      FunctionDescriptor.of(
          JAVA_INT, ADDRESS, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT,
          ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG);

  /** Every export of include/jmodels_attn.h with its descriptor, in the header's order. */
  static final Map<String, FunctionDescriptor> DOWNCALLS =
      Map.ofEntries(
          entry("jmodels_attn_abi_version", FunctionDescriptor.of(JAVA_INT)),
          entry("jmodels_attn_capabilities", FunctionDescriptor.of(JAVA_LONG)),
          entry("jmodels_attn_status_name", FunctionDescriptor.of(ADDRESS, JAVA_INT)),
          entry("jmodels_attn_last_error", FunctionDescriptor.of(ADDRESS)),
          entry("jmodels_attn_context_create", FunctionDescriptor.of(ADDRESS, JAVA_INT)),
          entry("jmodels_attn_context_destroy", STATUS_OF_HANDLE),
          entry("jmodels_attn_context_synchronize", STATUS_OF_HANDLE),
          entry("jmodels_attn_context_stream", FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS)),
          entry("jmodels_attn_rope_create",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_FLOAT, JAVA_FLOAT, ADDRESS,
                  JAVA_INT, JAVA_INT, ADDRESS)),
          entry("jmodels_attn_rope_destroy", STATUS_OF_HANDLE),
          entry("jmodels_attn_norm_create",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS, ADDRESS, JAVA_FLOAT,
                  ADDRESS)),
          entry("jmodels_attn_norm_create_ex",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS, ADDRESS, JAVA_FLOAT,
                  JAVA_INT, ADDRESS)),
          entry("jmodels_attn_norm_destroy", STATUS_OF_HANDLE),
          entry("jmodels_attn_kv_create",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, JAVA_INT,
                  JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS, ADDRESS)),
          entry("jmodels_attn_kv_create_layered",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS,
                  JAVA_INT, ADDRESS)),
          entry("jmodels_attn_kv_destroy", STATUS_OF_HANDLE),
          entry("jmodels_attn_kv_clear", FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT)),
          entry("jmodels_attn_kv_discard_from",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT)),
          entry("jmodels_attn_kv_contains",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS)),
          entry("jmodels_attn_kv_store",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT,
                  ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG)),
          entry("jmodels_attn_kv_read",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, JAVA_INT, JAVA_INT, JAVA_INT,
                  JAVA_INT, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG)),
          entry("jmodels_attn_kv_bytes", FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS)),
          entry("jmodels_attn_append", ROWS_APPEND),
          entry("jmodels_attn_attend", ROWS_ATTEND),
          entry("jmodels_attn_decode", ROWS_DECODE),
          entry("jmodels_attn_prefill", PREFILL),
          entry("jmodels_attn_attend_causal", CAUSAL),
          entry("jmodels_attn_append_device", ROWS_APPEND),
          entry("jmodels_attn_attend_device", ROWS_ATTEND),
          entry("jmodels_attn_decode_device", ROWS_DECODE),
          entry("jmodels_attn_decode_device_noalloc", ROWS_DECODE),
          entry("jmodels_attn_attend_causal_device", CAUSAL),
          entry("jmodels_attn_prefill_device", PREFILL),
          entry("jmodels_attn_quantized_matmul_device",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, JAVA_INT, ADDRESS, JAVA_LONG, ADDRESS,
                  JAVA_LONG, ADDRESS, JAVA_LONG, JAVA_INT, JAVA_INT, JAVA_INT, ADDRESS, JAVA_INT)),
          entry("jmodels_attn_quantized_grouped_matmul_device",
              FunctionDescriptor.of(JAVA_INT, ADDRESS, ADDRESS, ADDRESS, ADDRESS, ADDRESS,
                  JAVA_INT, ADDRESS, JAVA_LONG, ADDRESS, JAVA_LONG, JAVA_INT, JAVA_INT, ADDRESS,
                  JAVA_INT)));

  private final Arena arena;
  private final long capabilities;
  private final Map<String, MethodHandle> handles;
  private final MemorySegment context;
  private boolean closed;

  private HipAttentionLibrary(
      Arena arena, long capabilities, Map<String, MethodHandle> handles, MemorySegment context) {
    this.arena = arena;
    this.capabilities = capabilities;
    this.handles = handles;
    this.context = context;
  }

  /**
   * The library named by {@value #LIBRARY_PROPERTY} or {@value #LIBRARY_ENVIRONMENT}, opened on
   * GPU {@code device}.
   */
  public static HipAttentionLibrary openConfigured(int device) {
    String path = System.getProperty(LIBRARY_PROPERTY);
    if (path == null || path.isBlank()) path = System.getenv(LIBRARY_ENVIRONMENT);
    if (path == null || path.isBlank()) {
      throw new IllegalArgumentException(
          "set -D" + LIBRARY_PROPERTY + " or " + LIBRARY_ENVIRONMENT + " to libjmodels_attn.so");
    }
    return open(Path.of(path), device);
  }

  /**
   * Opens the library, rejects another ABI version or a library without f16 decode, and creates
   * a context on GPU {@code device}.
   */
  public static HipAttentionLibrary open(Path libraryPath, int device) {
    Objects.requireNonNull(libraryPath, "libraryPath");
    Path normalized = libraryPath.toAbsolutePath().normalize();
    if (!Files.isRegularFile(normalized)) {
      throw new IllegalArgumentException("HIP attention library does not exist: " + normalized);
    }
    Arena arena = Arena.ofShared();
    try {
      SymbolLookup lookup = SymbolLookup.libraryLookup(normalized, arena);
      Linker linker = Linker.nativeLinker();
      Map<String, MethodHandle> handles = new HashMap<>();
      for (Map.Entry<String, FunctionDescriptor> e : DOWNCALLS.entrySet()) {
        MemorySegment symbol =
            lookup
                .find(e.getKey())
                .orElseThrow(() -> new IllegalArgumentException("missing export " + e.getKey()));
        handles.put(e.getKey(), linker.downcallHandle(symbol, e.getValue()));
      }
      int abi = (int) handles.get("jmodels_attn_abi_version").invokeExact();
      if (abi != ABI_VERSION) {
        throw new IllegalArgumentException(
            "unsupported HIP attention ABI " + abi + "; expected " + ABI_VERSION);
      }
      long caps = (long) handles.get("jmodels_attn_capabilities").invokeExact();
      if ((caps & CAP_DECODE_F16) == 0) {
        throw new IllegalArgumentException("HIP attention library has no f16 decode kernel");
      }
      MemorySegment ctx =
          (MemorySegment) handles.get("jmodels_attn_context_create").invokeExact(device);
      if (ctx.address() == 0) {
        throw new IllegalStateException(
            "HIP attention context creation failed on device " + device + ": " + lastError(handles));
      }
      return new HipAttentionLibrary(arena, caps, Map.copyOf(handles), ctx);
    } catch (RuntimeException | LinkageError failure) {
      arena.close();
      throw failure;
    } catch (Throwable t) {
      arena.close();
      throw new IllegalStateException("HIP attention library could not be opened", t);
    }
  }

  public int abiVersion() {
    return ABI_VERSION;
  }

  public long capabilities() {
    return capabilities;
  }

  public boolean supports(long capability) {
    return (capabilities & capability) == capability;
  }

  // ---------------------------------------------------------------- handles and status

  private MethodHandle h(String name) {
    return handles.get(name);
  }

  private void ensureOpen() {
    if (closed) throw new IllegalStateException("HIP attention library is closed");
  }

  private static String lastError(Map<String, MethodHandle> handles) throws Throwable {
    MemorySegment s = (MemorySegment) handles.get("jmodels_attn_last_error").invokeExact();
    return s.address() == 0 ? "" : s.reinterpret(4096).getString(0);
  }

  /** The status name, as NativeKernelLibrary.statusName (NativeKernelLibrary.java:771-779). */
  public String statusName(int status) {
    try {
      MemorySegment s = (MemorySegment) h("jmodels_attn_status_name").invokeExact(status);
      return s.reinterpret(64).getString(0);
    } catch (Throwable t) {
      return "STATUS_" + status;
    }
  }

  /**
   * A non-zero status becomes the exception backend-java throws for the same condition: shapes,
   * sizes and ranges IllegalArgumentException (KvCache's bounds checks, cache/KvCache.java:
   * 237-244), unavailable positions and non-finite scores IllegalStateException (:232-235;
   * ops/TensorOps.java:1256-1269), everything else IllegalStateException naming the status.
   */
  private void check(int status, String operation) throws Throwable {
    if (status == OK) return;
    String detail = lastError(handles);
    String message = operation + " failed: " + statusName(status) + (detail.isEmpty() ? "" : ": " + detail);
    switch (status) {
      case NULL_POINTER, INVALID_SHAPE, BUFFER_TOO_SMALL, OUT_OF_RANGE ->
          throw new IllegalArgumentException(message);
      default -> throw new IllegalStateException(message);
    }
  }

  private static RuntimeException bridge(String operation, Throwable t) {
    if (t instanceof RuntimeException r) return r;
    if (t instanceof Error e) throw e;
    return new IllegalStateException("HIP attention bridge failed during " + operation, t);
  }

  private static MemorySegment out(Arena call) {
    return call.allocate(ADDRESS);
  }

  // ---------------------------------------------------------------- context

  /** Waits for the context stream; reports errors kernels recorded since the last call. */
  public synchronized void synchronize() {
    ensureOpen();
    try {
      check((int) h("jmodels_attn_context_synchronize").invokeExact(context), "synchronize");
    } catch (Throwable t) {
      throw bridge("synchronize", t);
    }
  }

  // ---------------------------------------------------------------- RoPE tables and norms

  /**
   * RotaryTable factors for positions [0, maxPositions) in device memory
   * (ops/RotaryTable.java:48-186); frequencyFactors may be null.
   */
  public synchronized MemorySegment ropeCreate(
      int rotaryDim, float theta, float frequencyScale, float[] frequencyFactors, int maxPositions) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment factors =
          frequencyFactors == null ? MemorySegment.NULL : call.allocateFrom(JAVA_FLOAT, frequencyFactors);
      int count = frequencyFactors == null ? 0 : frequencyFactors.length;
      MemorySegment result = out(call);
      check((int) h("jmodels_attn_rope_create")
              .invokeExact(context, rotaryDim, theta, frequencyScale, factors, count, maxPositions,
                  result),
          "rope_create");
      return result.get(ADDRESS, 0);
    } catch (Throwable t) {
      throw bridge("rope_create", t);
    }
  }

  /** Per-head RMS-norm weights of q and k (either may be null); flags NORM_VALUE_RMS for Gemma 4. */
  public synchronized MemorySegment normCreate(
      int headDim, float[] qWeight, float[] kWeight, float eps, int flags) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment q = qWeight == null ? MemorySegment.NULL : call.allocateFrom(JAVA_FLOAT, qWeight);
      MemorySegment k = kWeight == null ? MemorySegment.NULL : call.allocateFrom(JAVA_FLOAT, kWeight);
      MemorySegment result = out(call);
      check((int) h("jmodels_attn_norm_create_ex")
              .invokeExact(context, headDim, q, k, eps, flags, result),
          "norm_create_ex");
      return result.get(ADDRESS, 0);
    } catch (Throwable t) {
      throw bridge("norm_create_ex", t);
    }
  }

  public synchronized void ropeDestroy(MemorySegment rope) {
    destroy("jmodels_attn_rope_destroy", rope);
  }

  public synchronized void normDestroy(MemorySegment norm) {
    destroy("jmodels_attn_norm_destroy", norm);
  }

  private void destroy(String name, MemorySegment handle) {
    if (handle == null || handle.address() == 0) return;
    try {
      check((int) h(name).invokeExact(handle), name);
    } catch (Throwable t) {
      throw bridge(name, t);
    }
  }

  // ---------------------------------------------------------------- KV cache

  /**
   * A device KV cache for `sequences` sessions (KvCache, cache/KvCache.java:35-48), f16 or f32;
   * ringCapacity[l] = 0 keeps layer l LINEAR, else RING of that many slots
   * (cache/LayeredKvCache.java:354-356). ringCapacity may be null (all LINEAR).
   */
  public synchronized MemorySegment kvCreate(
      int sequences, int numLayers, int maxSeqLen, int numKvHeads, int keyLength, int valueLength,
      boolean halfPrecision, int[] ringCapacity) {
    ensureOpen();
    if (ringCapacity != null && ringCapacity.length != numLayers) {
      throw new IllegalArgumentException("ringCapacity needs one entry per layer");
    }
    try (Arena call = Arena.ofConfined()) {
      MemorySegment rings = ringCapacity == null ? MemorySegment.NULL : call.allocateFrom(JAVA_INT, ringCapacity);
      MemorySegment result = out(call);
      check((int) h("jmodels_attn_kv_create")
              .invokeExact(context, sequences, numLayers, maxSeqLen, numKvHeads, keyLength,
                  valueLength, halfPrecision ? KV_F16 : KV_F32, rings, result),
          "kv_create");
      return result.get(ADDRESS, 0);
    } catch (Throwable t) {
      throw bridge("kv_create", t);
    }
  }

  /**
   * A layered cache (LayeredKvCache, cache/LayeredKvCache.java:124-156): spec[l] = {numKvHeads,
   * keyLength, valueLength, ringCapacity} of layer l.
   */
  public synchronized MemorySegment kvCreateLayered(
      int sequences, int maxSeqLen, int[][] specs, boolean halfPrecision) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment s = call.allocate(LAYER_SPEC, specs.length);
      for (int l = 0; l < specs.length; l++) {
        if (specs[l].length != 4) throw new IllegalArgumentException("layer spec " + l + " needs 4 values");
        for (int j = 0; j < 4; j++) s.setAtIndex(JAVA_INT, 4L * l + j, specs[l][j]);
      }
      MemorySegment result = out(call);
      check((int) h("jmodels_attn_kv_create_layered")
              .invokeExact(context, sequences, specs.length, maxSeqLen, s,
                  halfPrecision ? KV_F16 : KV_F32, result),
          "kv_create_layered");
      return result.get(ADDRESS, 0);
    } catch (Throwable t) {
      throw bridge("kv_create_layered", t);
    }
  }

  public synchronized void kvDestroy(MemorySegment kv) {
    destroy("jmodels_attn_kv_destroy", kv);
  }

  public synchronized void kvClear(MemorySegment kv, int sequence) {
    ensureOpen();
    try {
      check((int) h("jmodels_attn_kv_clear").invokeExact(kv, sequence), "kv_clear");
    } catch (Throwable t) {
      throw bridge("kv_clear", t);
    }
  }

  public synchronized void kvDiscardFrom(MemorySegment kv, int sequence, int position) {
    ensureOpen();
    try {
      check((int) h("jmodels_attn_kv_discard_from").invokeExact(kv, sequence, position),
          "kv_discard_from");
    } catch (Throwable t) {
      throw bridge("kv_discard_from", t);
    }
  }

  public synchronized boolean kvContains(MemorySegment kv, int sequence, int layer, int position) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment result = call.allocate(JAVA_INT);
      check((int) h("jmodels_attn_kv_contains").invokeExact(kv, sequence, layer, position, result),
          "kv_contains");
      return result.get(JAVA_INT, 0) != 0;
    } catch (Throwable t) {
      throw bridge("kv_contains", t);
    }
  }

  /** KvCache.keySlice / valueSlice (cache/KvCache.java:105-115) of positions [from, to). */
  public synchronized void kvRead(
      MemorySegment kv, int sequence, int layer, int from, int to, float[] keys, float[] values) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment ks = call.allocate(JAVA_FLOAT, keys.length);
      MemorySegment vs = call.allocate(JAVA_FLOAT, values.length);
      check((int) h("jmodels_attn_kv_read")
              .invokeExact(context, kv, sequence, layer, from, to, ks, (long) keys.length, vs,
                  (long) values.length),
          "kv_read");
      MemorySegment.copy(ks, JAVA_FLOAT, 0, keys, 0, keys.length);
      MemorySegment.copy(vs, JAVA_FLOAT, 0, values, 0, values.length);
    } catch (Throwable t) {
      throw bridge("kv_read", t);
    }
  }

  // ---------------------------------------------------------------- attention

  /** Fills a jmodels_attn_layer struct in `call`. */
  public static MemorySegment layer(
      Arena call, int layer, int numHeads, int slidingWindow, boolean neox, float scale,
      MemorySegment rope, MemorySegment qkNorm) {
    MemorySegment l = call.allocate(LAYER);
    l.set(JAVA_INT, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("layer")), layer);
    l.set(JAVA_INT, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("num_heads")), numHeads);
    l.set(JAVA_INT, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("sliding_window")), slidingWindow);
    l.set(JAVA_INT, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("neox")), neox ? 1 : 0);
    l.set(JAVA_FLOAT, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("scale")), scale);
    l.set(ADDRESS, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("rope")),
        rope == null ? MemorySegment.NULL : rope);
    l.set(ADDRESS, LAYER.byteOffset(MemoryLayout.PathElement.groupElement("qk_norm")),
        qkNorm == null ? MemorySegment.NULL : qkNorm);
    return l;
  }

  /**
   * One decode token per listed session on host buffers (copied in and out by the library):
   * QK-norm, RoPE, append and attention, as forwardSequenceInternal's attention block
   * (llama/LlamaForwardPass.java:1069-1128) and attendIndependentSessions (:793-839).
   */
  public synchronized void decode(
      MemorySegment kv, MemorySegment layer, int[] sequences, int[] positions, float[] q,
      float[] k, float[] v, float[] out) {
    ensureOpen();
    if (sequences.length != positions.length) {
      throw new IllegalArgumentException("sequences and positions differ in length");
    }
    try (Arena call = Arena.ofConfined()) {
      MemorySegment os = call.allocate(JAVA_FLOAT, out.length);
      check((int) h("jmodels_attn_decode")
              .invokeExact(context, kv, layer, sequences.length, call.allocateFrom(JAVA_INT, sequences),
                  call.allocateFrom(JAVA_INT, positions), call.allocateFrom(JAVA_FLOAT, q),
                  (long) q.length, call.allocateFrom(JAVA_FLOAT, k), (long) k.length,
                  call.allocateFrom(JAVA_FLOAT, v), (long) v.length, os, (long) out.length),
          "decode");
      MemorySegment.copy(os, JAVA_FLOAT, 0, out, 0, out.length);
    } catch (Throwable t) {
      throw bridge("decode", t);
    }
  }

  /**
   * Causal prefill of rows start .. start + n - 1 of one session on host buffers
   * (prepareBatchedAttention + computeBatchedAttention, llama/LlamaForwardPass.java:1479-1541).
   */
  public synchronized void prefill(
      MemorySegment kv, MemorySegment layer, int sequence, int start, int n, float[] q, float[] k,
      float[] v, float[] out) {
    ensureOpen();
    try (Arena call = Arena.ofConfined()) {
      MemorySegment os = call.allocate(JAVA_FLOAT, out.length);
      check((int) h("jmodels_attn_prefill")
              .invokeExact(context, kv, layer, sequence, start, n, call.allocateFrom(JAVA_FLOAT, q),
                  (long) q.length, call.allocateFrom(JAVA_FLOAT, k), (long) k.length,
                  call.allocateFrom(JAVA_FLOAT, v), (long) v.length, os, (long) out.length),
          "prefill");
      MemorySegment.copy(os, JAVA_FLOAT, 0, out, 0, out.length);
    } catch (Throwable t) {
      throw bridge("prefill", t);
    }
  }

  /**
   * The device-pointer decode for callers that keep q/k/v and the output resident (the Q/K/V
   * projection below writes them there); asynchronous on the context stream.
   */
  public synchronized void decodeDevice(
      MemorySegment kv, MemorySegment layer, MemorySegment sequences, MemorySegment positions,
      int count, MemorySegment q, long qElements, MemorySegment k, long kElements, MemorySegment v,
      long vElements, MemorySegment out, long outElements) {
    ensureOpen();
    try {
      check((int) h("jmodels_attn_decode_device")
              .invokeExact(context, kv, layer, count, sequences, positions, q, qElements, k,
                  kElements, v, vElements, out, outElements),
          "decode_device");
    } catch (Throwable t) {
      throw bridge("decode_device", t);
    }
  }

  // ---------------------------------------------------------------- quantized projections

  /**
   * Grouped Q/K/V projection on device memory (backend-native's
   * jmodels_quantized_f32_grouped_batched_matmul_with_context, RS:582-637, plus the bias):
   * formats are backend-native's codes (RS:150-161), outputs matrix after matrix.
   */
  public synchronized void quantizedGroupedMatmulDevice(
      int[] formats, MemorySegment[] weights, long[] weightBytes, int[] rows, MemorySegment input,
      long inputElements, MemorySegment output, long outputElements, int batch, int cols,
      MemorySegment[] addends, int addendMode) {
    ensureOpen();
    int n = formats.length;
    if (weights.length != n || weightBytes.length != n || rows.length != n
        || (addends != null && addends.length != n)) {
      throw new IllegalArgumentException("grouped projection arrays differ in length");
    }
    try (Arena call = Arena.ofConfined()) {
      MemorySegment w = call.allocate(ADDRESS, n);
      MemorySegment a = addends == null ? MemorySegment.NULL : call.allocate(ADDRESS, n);
      for (int i = 0; i < n; i++) {
        w.setAtIndex(ADDRESS, i, weights[i]);
        if (addends != null) a.setAtIndex(ADDRESS, i, addends[i]);
      }
      check((int) h("jmodels_attn_quantized_grouped_matmul_device")
              .invokeExact(context, call.allocateFrom(JAVA_INT, formats), w,
                  call.allocateFrom(JAVA_LONG, weightBytes), call.allocateFrom(JAVA_INT, rows), n,
                  input, inputElements, output, outputElements, batch, cols, a, addendMode),
          "quantized_grouped_matmul_device");
    } catch (Throwable t) {
      throw bridge("quantized_grouped_matmul_device", t);
    }
  }

  /** One projection on device memory; ADDEND_RESIDUAL adds x in place (x += wo . attn). */
  public synchronized void quantizedMatmulDevice(
      int format, MemorySegment weights, long weightBytes, MemorySegment input, long inputElements,
      MemorySegment output, long outputElements, int batch, int rows, int cols,
      MemorySegment addend, int addendMode) {
    ensureOpen();
    try {
      check((int) h("jmodels_attn_quantized_matmul_device")
              .invokeExact(context, format, weights, weightBytes, input, inputElements, output,
                  outputElements, batch, rows, cols,
                  addend == null ? MemorySegment.NULL : addend, addendMode),
          "quantized_matmul_device");
    } catch (Throwable t) {
      throw bridge("quantized_matmul_device", t);
    }
  }

  // ---------------------------------------------------------------- close

  /** Destroys the context once and releases the library; later calls throw. */
  @Override
  public synchronized void close() {
    if (closed) return;
    closed = true;
    try {
      int status = (int) h("jmodels_attn_context_destroy").invokeExact(context);
      if (status != OK) {
        throw new IllegalStateException("context_destroy failed: " + statusName(status));
      }
    } catch (RuntimeException e) {
      throw e;
    } catch (Throwable t) {
      throw new IllegalStateException("HIP attention bridge failed during close", t);
    } finally {
      arena.close();
    }
  }
}
