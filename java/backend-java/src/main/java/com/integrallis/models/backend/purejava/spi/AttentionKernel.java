/*
 * Addition to backend-java: the service interface through which LlamaForwardPass hands its
 * grouped-query attention and KV cache to an accelerator. backend-java keeps attention private to
 * LlamaForwardPass (llama/LlamaForwardPass.java:1069-1128, 1479-1541, 1543-1670, 793-839) with the
 * cache in its own KvCache (cache/KvCache.java); this interface names those steps so that an
 * implementation can own the cache in device memory. It follows the shape of
 * GgufBatchedMatrixKernel (spi/GgufBatchedMatrixKernel.java:23-221): an implementation id,
 * capability and eligibility queries asked before any call, AutoCloseable.
 *
 * Not compiled in this repository (no JDK is installed where it was written); the C ABI it binds
 * is include/jmodels_attn.h.
 */
package com.integrallis.models.backend.purejava.spi;

/**
 * Grouped-query attention over a KV cache the implementation owns.
 *
 * <p>One instance serves one model and is used by one caller at a time, as a backend-java
 * instance is (api/InferenceBackend.java:22-27). Positions, layers and sessions follow KvCache:
 * {@link #decode} stores the new row of every listed session at its position and attends over
 * {@code [attentionStartPosition(p), p]} of that session; an unpopulated visible position is an
 * {@link IllegalStateException}, a position or layer out of range an {@link
 * IllegalArgumentException}, as KvCache throws them (cache/KvCache.java:232-244).
 */
public interface AttentionKernel extends AutoCloseable {

  /** Shape of one model's attention, as LlamaConfig describes it (llama/LlamaConfig.java:78-95). */
  record Shape(
      int numLayers,
      int numHeads,
      int numKvHeads,
      int keyLength,
      int valueLength,
      int maxSequenceLength,
      int sessions,
      boolean halfPrecisionKv) {
    public Shape {
      if (numLayers <= 0 || numHeads <= 0 || numKvHeads <= 0 || keyLength <= 0 || valueLength <= 0
          || maxSequenceLength <= 0 || sessions <= 0) {
        throw new IllegalArgumentException("attention shape dimensions must be positive");
      }
      if (numHeads % numKvHeads != 0) {
        throw new IllegalArgumentException(
            "numHeads must be a multiple of numKvHeads (llama/LlamaConfig.java:46-48)");
      }
    }
  }

  /**
   * One layer's attention parameters for a call: its sliding window (0 = global; first visible
   * position max(0, p - w + 1), llama/LlamaConfig.java:184-195), the RoPE pair layout (NeoX
   * split-half or interleaved, llama/LlamaConfig.java:122-126), whether RoPE applies
   * (usesRope), the score scale (0 = (float) (1 / sqrt(keyLength))) and the layer's QK-norm
   * weights (null when the layer has none, llama/LlamaWeights.java:99-101).
   */
  record Layer(
      int layer,
      int slidingWindow,
      boolean neox,
      boolean rope,
      double ropeTheta,
      float ropeFrequencyScale,
      float scale,
      float[] qNorm,
      float[] kNorm,
      float normEpsilon) {}

  /** Stable implementation identifier used in diagnostics. */
  default String implementation() {
    return "custom";
  }

  /** Whether this implementation can hold and attend a model of this shape. */
  boolean supports(Shape shape);

  /**
   * Whether this implementation should run a call of {@code rows} query rows at the given context
   * length; implementations may decline shapes where boundary overhead would make it slower than
   * the Java loops.
   */
  default boolean isEligible(Shape shape, int rows, int contextLength) {
    return supports(shape);
  }

  /**
   * One decode token for each listed session: QK-norm and RoPE on q and the new k, the new k and v
   * stored at {@code positions[i]} of {@code sessions[i]}, then attention over the session's
   * visible positions (forwardSequenceInternal's attention block, llama/LlamaForwardPass.java:
   * 1069-1128, and attendIndependentSessions, :793-839). q is {@code [count][numHeads *
   * keyLength]}, k {@code [count][numKvHeads * keyLength]}, v {@code [count][numKvHeads *
   * valueLength]}, out {@code [count][numHeads * valueLength]}. Sessions must be distinct
   * (:933-960).
   */
  void decode(Layer layer, int[] sessions, int[] positions, float[] q, float[] k, float[] v,
      float[] out);

  /**
   * Causal prefill of rows {@code start .. start + n - 1} of one session
   * (prepareBatchedAttention + computeBatchedAttention, llama/LlamaForwardPass.java:1479-1541):
   * every row stored, then row b attends {@code [attentionStartPosition(start + b), start + b]}.
   */
  void prefill(Layer layer, int session, int start, int n, float[] q, float[] k, float[] v,
      float[] out);

  /** KvCache.discardFrom (cache/KvCache.java:161-173) for one session. */
  void discardFrom(int session, int position);

  /** KvCache.clear (cache/KvCache.java:156-158); session &lt; 0 clears every session. */
  void clear(int session);

  /** Whether (session, layer, position) holds a stored row (cache/KvCache.java:72). */
  boolean contains(int session, int layer, int position);

  /**
   * Reads rows {@code from .. to - 1} of one session's layer back in KvCache's flat layout
   * ({@code [position][numKvHeads * length]}, cache/KvCache.java:105-115), for tests.
   */
  void read(int session, int layer, int from, int to, float[] keys, float[] values);

  /** No attention kernel: LlamaForwardPass keeps its own loops. */
  static AttentionKernel none() {
    return NoAttentionKernel.INSTANCE;
  }

  @Override
  void close();

  /** The absent kernel: supports nothing, so no call reaches it. */
  final class NoAttentionKernel implements AttentionKernel {
    static final NoAttentionKernel INSTANCE = new NoAttentionKernel();

    private NoAttentionKernel() {}

    @Override
    public String implementation() {
      return "none";
    }

    @Override
    public boolean supports(Shape shape) {
      return false;
    }

    private static UnsupportedOperationException absent() {
      return new UnsupportedOperationException("no attention kernel is installed");
    }

    @Override
    public void decode(Layer layer, int[] sessions, int[] positions, float[] q, float[] k,
        float[] v, float[] out) {
      throw absent();
    }

    @Override
    public void prefill(Layer layer, int session, int start, int n, float[] q, float[] k,
        float[] v, float[] out) {
      throw absent();
    }

    @Override
    public void discardFrom(int session, int position) {
      throw absent();
    }

    @Override
    public void clear(int session) {
      throw absent();
    }

    @Override
    public boolean contains(int session, int layer, int position) {
      throw absent();
    }

    @Override
    public void read(int session, int layer, int from, int to, float[] keys, float[] values) {
      throw absent();
    }

    @Override
    public void close() {}
  }
}
