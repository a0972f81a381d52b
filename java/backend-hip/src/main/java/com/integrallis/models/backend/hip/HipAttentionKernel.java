/*
 * backend-java's AttentionKernel on an MI355X through libjmodels_attn: the KV cache of every
 * session lives in HBM (allocated at maxSequenceLength, appended in place each step), RoPE
 * tables and QK-norm weights are built once per layer shape, and each call is one downcall
 * (HipAttentionLibrary). It plays the part RustGgufBatchedMatrixKernel plays for the quantized
 * matmuls (backend-native/src/main/java/com/integrallis/models/backend/nativekernel/
 * RustGgufBatchedMatrixKernel.java): reusable native state, synchronized methods, shapes checked
 * in Java before the downcall and again in C.
 *
 * Not compiled in this repository (no JDK is installed where it was written).
 */
package com.integrallis.models.backend.hip;

import com.integrallis.models.backend.purejava.spi.AttentionKernel;
import java.lang.foreign.Arena;
import java.lang.foreign.MemorySegment;
import java.util.HashMap;
import java.util.Map;
import java.util.Objects;

/** One model's attention and KV cache on one GPU. */
public final class HipAttentionKernel implements AttentionKernel {

  private final HipAttentionLibrary library;
  private final Shape shape;
  private final MemorySegment kv;
  private final Map<RopeKey, MemorySegment> ropes = new HashMap<>();
  private final Map<Integer, MemorySegment> norms = new HashMap<>();
  private boolean closed;

  private record RopeKey(int rotaryDim, double theta, float frequencyScale) {}

  private HipAttentionKernel(HipAttentionLibrary library, Shape shape, MemorySegment kv) {
    this.library = library;
    this.shape = shape;
    this.kv = kv;
  }

  /**
   * Opens the configured library on GPU {@code device} and allocates the cache for {@code shape};
   * ringCapacity[l] &gt; 0 keeps layer l as a ring of that many slots (null: every layer linear).
   */
  public static HipAttentionKernel open(Shape shape, int[] ringCapacity, int device) {
    Objects.requireNonNull(shape, "shape");
    HipAttentionLibrary library = HipAttentionLibrary.openConfigured(device);
    try {
      if (!supported(library, shape)) {
        throw new IllegalArgumentException("HIP attention does not support " + shape);
      }
      MemorySegment kv =
          library.kvCreate(
              shape.sessions(), shape.numLayers(), shape.maxSequenceLength(), shape.numKvHeads(),
              shape.keyLength(), shape.valueLength(), shape.halfPrecisionKv(), ringCapacity);
      return new HipAttentionKernel(library, shape, kv);
    } catch (RuntimeException e) {
      library.close();
      throw e;
    }
  }

  private static boolean supported(HipAttentionLibrary library, Shape s) {
    int d = s.keyLength();
    boolean dims =
        s.keyLength() == s.valueLength()
            && (s.halfPrecisionKv()
                ? (d == 32 || d == 64 || d == 128 || d == 256 || d == 512)
                : (d >= 16 && d <= 512 && d % 16 == 0));
    long need = s.halfPrecisionKv() ? HipAttentionLibrary.CAP_DECODE_F16 : HipAttentionLibrary.CAP_DECODE_F32;
    return dims && library.supports(need);
  }

  @Override
  public String implementation() {
    return "hip-gfx950";
  }

  @Override
  public boolean supports(Shape other) {
    return shape.equals(other) && supported(library, other);
  }

  @Override
  public synchronized boolean isEligible(Shape other, int rows, int contextLength) {
    return supports(other) && contextLength <= shape.maxSequenceLength();
  }

  private void ensureOpen() {
    if (closed) throw new IllegalStateException("HIP attention kernel is closed");
  }

  private MemorySegment rope(Layer layer) {
    if (!layer.rope()) return MemorySegment.NULL;
    RopeKey key = new RopeKey(shape.keyLength(), layer.ropeTheta(), layer.ropeFrequencyScale());
    return ropes.computeIfAbsent(
        key,
        k -> library.ropeCreate(k.rotaryDim(), (float) k.theta(), k.frequencyScale(), null,
            shape.maxSequenceLength()));
  }

  private MemorySegment norm(Layer layer) {
    if (layer.qNorm() == null && layer.kNorm() == null) return MemorySegment.NULL;
    return norms.computeIfAbsent(
        layer.layer(),
        l -> library.normCreate(shape.keyLength(), layer.qNorm(), layer.kNorm(), layer.normEpsilon(), 0));
  }

  private void checkRows(int count, float[] q, float[] k, float[] v, float[] out) {
    // The reference checks buffer extents before its loops; so does this binding, before the
    // downcall (which checks again).
    long qn = (long) count * shape.numHeads() * shape.keyLength();
    long kn = (long) count * shape.numKvHeads() * shape.keyLength();
    long vn = (long) count * shape.numKvHeads() * shape.valueLength();
    long on = (long) count * shape.numHeads() * shape.valueLength();
    if (q.length < qn || k.length < kn || v.length < vn || out.length < on) {
      throw new IllegalArgumentException("attention buffers are smaller than " + count + " rows");
    }
  }

  @Override
  public synchronized void decode(
      Layer layer, int[] sessions, int[] positions, float[] q, float[] k, float[] v, float[] out) {
    ensureOpen();
    if (sessions.length != positions.length || sessions.length == 0) {
      throw new IllegalArgumentException("one position per session is required");
    }
    checkRows(sessions.length, q, k, v, out);
    try (Arena call = Arena.ofConfined()) {
      MemorySegment l =
          HipAttentionLibrary.layer(call, layer.layer(), shape.numHeads(), layer.slidingWindow(),
              layer.neox(), layer.scale(), rope(layer), norm(layer));
      library.decode(kv, l, sessions, positions, q, k, v, out);
    }
  }

  @Override
  public synchronized void prefill(
      Layer layer, int session, int start, int n, float[] q, float[] k, float[] v, float[] out) {
    ensureOpen();
    if (n <= 0) throw new IllegalArgumentException("prefill needs at least one row");
    checkRows(n, q, k, v, out);
    try (Arena call = Arena.ofConfined()) {
      MemorySegment l =
          HipAttentionLibrary.layer(call, layer.layer(), shape.numHeads(), layer.slidingWindow(),
              layer.neox(), layer.scale(), rope(layer), norm(layer));
      library.prefill(kv, l, session, start, n, q, k, v, out);
    }
  }

  @Override
  public synchronized void discardFrom(int session, int position) {
    ensureOpen();
    library.kvDiscardFrom(kv, session, position);
  }

  @Override
  public synchronized void clear(int session) {
    ensureOpen();
    library.kvClear(kv, session);
  }

  @Override
  public synchronized boolean contains(int session, int layer, int position) {
    ensureOpen();
    return library.kvContains(kv, session, layer, position);
  }

  @Override
  public synchronized void read(int session, int layer, int from, int to, float[] keys, float[] values) {
    ensureOpen();
    library.kvRead(kv, session, layer, from, to, keys, values);
  }

  /** Releases the cache, the RoPE tables and norms, then the context; idempotent. */
  @Override
  public synchronized void close() {
    if (closed) return;
    closed = true;
    try {
      library.kvDestroy(kv);
      for (MemorySegment r : ropes.values()) library.ropeDestroy(r);
      for (MemorySegment n : norms.values()) library.normDestroy(n);
    } finally {
      library.close();
    }
  }
}
