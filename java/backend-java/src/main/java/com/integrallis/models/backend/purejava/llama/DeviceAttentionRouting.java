/*
 * Addition to backend-java: how LlamaForwardPass hands its attention to an AttentionKernel.
 * LlamaForwardPass (llama/LlamaForwardPass.java:178-225) would take the kernel next to its
 * GgufBatchedMatrixKernel, ask plan(...) once, and, when the decision is ENABLED, call
 *
 *   decodeLayer   in forwardSequenceInternal instead of QK-norm, applyRope, KvCache.store and
 *                 the grouped-query loop of :1069-1128;
 *   prefillChunk  in prefillBatch instead of prepareBatchedAttention + computeBatchedAttention
 *                 (:603-604 over :1479-1541);
 *   attendSessions in attendIndependentSessions instead of its per-session loop (:793-839);
 *   rewind/reset  where the pass calls KvCache.discardFrom / clear.
 *
 * The decision is recorded like the planner's other attention choices
 * (plan/ExecutionPlanner.java:488-536) and is behind the flag models.hip.attention.
 *
 * Not compiled in this repository (no JDK is installed where it was written).
 */
package com.integrallis.models.backend.purejava.llama;

import com.integrallis.models.api.OptimizationDecision;
import com.integrallis.models.api.OptimizationStatus;
import com.integrallis.models.backend.purejava.spi.AttentionKernel;
import java.util.List;
import java.util.Map;

/** The per-layer parameters and calls of one model's device attention. */
public final class DeviceAttentionRouting {

  /** System property that enables device attention when a kernel is installed. */
  public static final String FLAG = "models.hip.attention";

  private final AttentionKernel kernel;
  private final AttentionKernel.Layer[] layers;

  private DeviceAttentionRouting(AttentionKernel kernel, AttentionKernel.Layer[] layers) {
    this.kernel = kernel;
    this.layers = layers;
  }

  /**
   * Decides whether this model's attention runs on the kernel, appends the decision to
   * `decisions`, and returns the routing when it does (null otherwise). qNorms / kNorms hold each
   * layer's attn_q_norm / attn_k_norm weights (llama/LlamaWeights.java:99-101), null entries for
   * layers without them.
   */
  public static DeviceAttentionRouting plan(
      LlamaConfig config,
      AttentionKernel kernel,
      int maxSequenceLength,
      int sessions,
      boolean halfPrecisionKv,
      float[][] qNorms,
      float[][] kNorms,
      List<OptimizationDecision> decisions) {
    String id = "device-attention";
    if (kernel == null || "none".equals(kernel.implementation())) {
      decisions.add(new OptimizationDecision(id, OptimizationStatus.UNSUPPORTED,
          "no attention kernel is installed", Map.of()));
      return null;
    }
    if (config.usesBidirectionalAttention()) {
      decisions.add(new OptimizationDecision(id, OptimizationStatus.UNSUPPORTED,
          "the encoder's bidirectional window is not offloaded", Map.of()));
      return null;
    }
    AttentionKernel.Shape shape =
        new AttentionKernel.Shape(config.numLayers(), config.numHeads(), config.numKvHeads(),
            config.keyLength(), config.valueLength(), maxSequenceLength, sessions, halfPrecisionKv);
    if (!kernel.supports(shape)) {
      decisions.add(new OptimizationDecision(id, OptimizationStatus.UNSUPPORTED,
          kernel.implementation() + " does not support this attention shape",
          Map.of("head-dim", Integer.toString(config.keyLength()))));
      return null;
    }
    if (!Boolean.parseBoolean(System.getProperty(FLAG, "false"))) {
      decisions.add(new OptimizationDecision(id, OptimizationStatus.DISABLED,
          "disabled by " + FLAG, Map.of("implementation", kernel.implementation())));
      return null;
    }
    AttentionKernel.Layer[] layers = new AttentionKernel.Layer[config.numLayers()];
    for (int l = 0; l < layers.length; l++) {
      layers[l] =
          new AttentionKernel.Layer(
              l,
              config.usesSlidingWindow(l) ? config.slidingWindow() : 0,
              config.usesNeoxRope(),
              config.usesRope(l),
              config.ropeTheta(l),
              config.ropeFrequencyScale(l),
              0.0f,  // the library's default, (float) (1 / sqrt(keyLength))
              qNorms == null ? null : qNorms[l],
              kNorms == null ? null : kNorms[l],
              config.rmsNormEps());
    }
    decisions.add(new OptimizationDecision(id, OptimizationStatus.ENABLED,
        "attention and KV cache on " + kernel.implementation(),
        Map.of("implementation", kernel.implementation(),
            "kv", halfPrecisionKv ? "f16" : "f32",
            "sessions", Integer.toString(sessions))));
    return new DeviceAttentionRouting(kernel, layers);
  }

  /**
   * One token of one session through layer `layer`: raw q, k, v from the projections in, the
   * attention output out (the pass then applies wo and the residual, :1131-1138).
   */
  public void decodeLayer(int layer, int session, int position, float[] q, float[] k, float[] v,
      float[] out) {
    kernel.decode(layers[layer], new int[] {session}, new int[] {position}, q, k, v, out);
  }

  /** One prefill chunk of n rows starting at `start` (the rows of prefillBatch's batch). */
  public void prefillChunk(int layer, int session, int start, int n, float[] q, float[] k,
      float[] v, float[] out) {
    kernel.prefill(layers[layer], session, start, n, q, k, v, out);
  }

  /** attendIndependentSessions: one token for each listed (distinct) session. */
  public void attendSessions(int layer, int[] sessions, int[] positions, float[] q, float[] k,
      float[] v, float[] out) {
    kernel.decode(layers[layer], sessions, positions, q, k, v, out);
  }

  /** KvCache.discardFrom for a session's rewind. */
  public void rewind(int session, int position) {
    kernel.discardFrom(session, position);
  }

  /** KvCache.clear for a session's reset. */
  public void reset(int session) {
    kernel.clear(session);
  }
}
