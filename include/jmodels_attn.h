/*
 * jmodels_attn — MI355X (gfx950) grouped-query attention and KV-cache library, C ABI.
 *
 * Drop-in for backend-java's attention/KV-cache path of integrallis/models. Reference paths
 * (relative to /root/reference):
 *   BJ/ = backend-java/src/main/java/com/integrallis/models/backend/purejava/
 *   RS  = backend-native/src/main/rust/model-kernels/src/lib.rs   (C-ABI conventions followed)
 *   BN/ = backend-native/src/main/java/com/integrallis/models/backend/nativekernel/
 *
 * Conventions (after RS:58-82, 469-584):
 *   - every export is extern "C", takes plain pointers, u32 dims and u64 element counts, and
 *     returns an int32 status (0 = OK); nothing unwinds across the boundary (C++ try/catch at
 *     every export, like the Rust catch_unwind wrappers at RS:497-537);
 *   - a context is created per GPU and used by one caller at a time (the single-caller contract
 *     of API/InferenceBackend.java:20-28); it owns one HIP stream;
 *   - host-buffer calls are synchronous: they return once outputs are visible to the host;
 *   - *_device calls take device pointers and are asynchronous on the context stream; errors
 *     detected by kernels are reported by jmodels_attn_context_synchronize;
 *   - outputs must not alias inputs (RS:535-539);
 *   - *_device calls may be captured into a HIP graph on the context stream. A context keeps
 *     grow-only scratch memory (split partials, arrival tickets, rotated queries) sized by the
 *     largest launch plan seen so far; a call whose plan needs more while the stream is being
 *     captured returns NOT_CAPTURABLE and enqueues nothing, so run each shape once outside the
 *     capture first. Scratch that is outgrown later stays allocated until the context is
 *     destroyed, so graphs captured earlier remain valid.
 *
 * Ownership change vs the reference: the library owns the KV cache, resident in HBM and
 * appended in place; Java holds an opaque handle instead of float[] buffers.
 */
#ifndef JMODELS_ATTN_H
#define JMODELS_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JMODELS_ATTN_ABI_VERSION 2u

#if defined(__GNUC__)
#define JMODELS_ATTN_API __attribute__((visibility("default")))
#else
#define JMODELS_ATTN_API
#endif

/* Status codes. 0-4 keep the meaning of RS:78-82. */
#define JMODELS_ATTN_OK 0
#define JMODELS_ATTN_NULL_POINTER 1
#define JMODELS_ATTN_INVALID_SHAPE 2     /* dims/counts inconsistent or unsupported */
#define JMODELS_ATTN_BUFFER_TOO_SMALL 3  /* an element count is below what the shape needs */
#define JMODELS_ATTN_PANIC 4             /* C++ exception caught at the boundary */
#define JMODELS_ATTN_DEVICE_ERROR 5      /* HIP runtime failure */
#define JMODELS_ATTN_OUT_OF_RANGE 6      /* layer/position/sequence out of range (the reference's
                                            IllegalArgumentException, BJ/cache/KvCache.java:237-244) */
#define JMODELS_ATTN_UNAVAILABLE 7       /* position not populated or overwritten (the reference's
                                            IllegalStateException, BJ/cache/KvCache.java:232-235,
                                            BJ/cache/LayeredKvCache.java:192-197) */
#define JMODELS_ATTN_NON_FINITE 8        /* an attention score was NaN or +inf; TensorOps.softmax
                                            rejects those (BJ/ops/TensorOps.java:1256-1269) */
#define JMODELS_ATTN_NOT_CAPTURABLE 9    /* the call needs more context scratch memory than was
                                            allocated so far, and the context stream is being
                                            captured into a graph: nothing was enqueued. Make the
                                            same call once outside the capture first (no
                                            counterpart in the reference, which has no graphs) */

/* Capability bits (RS:59-77 style). */
#define JMODELS_ATTN_CAP_DECODE_F32 (1ull << 0)      /* f32 KV split-K decode */
#define JMODELS_ATTN_CAP_DECODE_F16 (1ull << 1)      /* f16 KV split-K decode */
#define JMODELS_ATTN_CAP_PREFILL_MFMA (1ull << 2)    /* causal / sliding-window f16 MFMA prefill */
#define JMODELS_ATTN_CAP_RAGGED_DECODE (1ull << 3)   /* many sessions, ragged lengths, one launch */
#define JMODELS_ATTN_CAP_SLIDING_WINDOW (1ull << 4)  /* causal window max(0, p - w + 1) */
#define JMODELS_ATTN_CAP_RING_LAYERS (1ull << 5)     /* LayeredKvCache RING retention */
#define JMODELS_ATTN_CAP_DEVICE_POINTERS (1ull << 6) /* *_device entry points */
#define JMODELS_ATTN_CAP_QK_NORM (1ull << 7)         /* per-head RMS norm of q and k before RoPE */
#define JMODELS_ATTN_CAP_VALUE_NORM (1ull << 8)      /* unweighted per-head RMS norm of v (Gemma 4) */
#define JMODELS_ATTN_CAP_QUANT_MATMUL (1ull << 9)    /* Q4_0 / Q8_0 / Q5_0 / Q4_K / Q5_K / Q6_K
                                                        projections on device memory */

/* KV storage element types. F16 stores IEEE binary16 (round to nearest even), which widens to
 * exactly Float.float16ToFloat(Float.floatToFloat16(x)) — the reference's half-precision KV
 * (BJ/cache/KvCache.java:84-100). */
#define JMODELS_ATTN_KV_F32 0u
#define JMODELS_ATTN_KV_F16 1u

typedef struct jmodels_attn_context jmodels_attn_context;
typedef struct jmodels_attn_kv jmodels_attn_kv;
typedef struct jmodels_attn_rope jmodels_attn_rope;
typedef struct jmodels_attn_norm jmodels_attn_norm;

/* One attention layer's parameters for a call.
 *   layer           zero-based layer of the KV cache
 *   num_heads       query heads; must be a multiple of the cache's num_kv_heads; query head h
 *                   reads KV head h / (num_heads / num_kv_heads) (BJ/llama/LlamaForwardPass.java:1563)
 *   sliding_window  0 = global; else causal window, first position max(0, p - w + 1)
 *                   (LlamaConfig.attentionStartPosition, BJ/llama/LlamaConfig.java:184-195)
 *   neox            1 = split-half RoPE pairs (i, i + pairs), 0 = interleaved (2i, 2i+1)
 *                   (TensorOps.ropeNeox / rope, BJ/ops/TensorOps.java:1336-1390)
 *   scale           score multiplier; 0 selects (float)(1 / sqrt(key_length))
 *                   (BJ/llama/LlamaForwardPass.java:1559); Gemma 4 passes 1.0
 *   rope            NULL = this layer applies no RoPE (LlamaConfig.usesRope false)
 *   qk_norm         NULL = no QK-norm; else each q and k head is RMS-normalised with the
 *                   object's weights before RoPE (normalizeHead, BJ/llama/LlamaForwardPass.java:
 *                   1070-1083, 1672-1676), and each v head without a weight when the object
 *                   was made with JMODELS_ATTN_NORM_VALUE_RMS */
typedef struct jmodels_attn_layer {
  uint32_t layer;
  uint32_t num_heads;
  uint32_t sliding_window;
  uint32_t neox;
  float scale;
  uint32_t reserved;
  const jmodels_attn_rope* rope;
  const jmodels_attn_norm* qk_norm;
} jmodels_attn_layer;

/* ---------------------------------------------------------------- library and context */

/* jmodels_kernels_abi_version analogue (RS:469-472). */
JMODELS_ATTN_API uint32_t jmodels_attn_abi_version(void);
/* jmodels_kernels_capabilities analogue (RS:474-495). */
JMODELS_ATTN_API uint64_t jmodels_attn_capabilities(void);
/* Upper-case name of a status code ("OK", "INVALID_SHAPE", ...), like
 * NativeKernelLibrary.statusName (BN/NativeKernelLibrary.java:771-779). */
JMODELS_ATTN_API const char* jmodels_attn_status_name(int32_t status);
/* Detail message of the last failing call on this thread ("" if none). */
JMODELS_ATTN_API const char* jmodels_attn_last_error(void);

/* jmodels_kernels_context_create analogue (RS:496-520): NULL on failure (no such device, not a
 * gfx950, HIP error). */
JMODELS_ATTN_API jmodels_attn_context* jmodels_attn_context_create(int32_t device);
/* RS:521-537 analogue; NULL_POINTER for NULL. Destroys nothing else: KV caches and RoPE tables
 * must be destroyed first. */
JMODELS_ATTN_API int32_t jmodels_attn_context_destroy(jmodels_attn_context* ctx);
/* Waits for the context stream and reports errors recorded by kernels since the last call. */
JMODELS_ATTN_API int32_t jmodels_attn_context_synchronize(jmodels_attn_context* ctx);
/* The context's hipStream_t, for callers that order their own work (events, copies) with it. */
JMODELS_ATTN_API int32_t jmodels_attn_context_stream(jmodels_attn_context* ctx, void** stream_out);

/* ---------------------------------------------------------------- RoPE tables */

/* RotaryTable (BJ/ops/RotaryTable.java:48-75, 177-186): cos/sin for positions
 * [0, max_positions) computed on the host exactly as fillFactors does (frequency in double pow,
 * angle in float, cos/sin in double rounded to float) and kept in HBM. frequency_factors may be
 * NULL; otherwise factor_count == rotary_dim / 2 finite positive divisors. */
JMODELS_ATTN_API int32_t jmodels_attn_rope_create(jmodels_attn_context* ctx, uint32_t rotary_dim, float theta,
                                 float frequency_scale, const float* frequency_factors,
                                 uint32_t factor_count, uint32_t max_positions,
                                 jmodels_attn_rope** rope_out);
JMODELS_ATTN_API int32_t jmodels_attn_rope_destroy(jmodels_attn_rope* rope);

/* ---------------------------------------------------------------- QK-norm weights */

/* A layer's attn_q_norm / attn_k_norm weights (BJ/llama/LlamaWeights.java:99-101), kept in HBM.
 * Each head x (head_dim elements) becomes x * (1 / rms) * w with rms = (float)sqrt(sum(x^2) /
 * head_dim + eps) (TensorOps.rmsNorm, BJ/ops/TensorOps.java:50-58), applied before RoPE when the
 * weights are present. q_weight or k_weight may be NULL: that side is left as is, as
 * normalizeHead does for an empty weight array. head_dim must equal the cache's key_length. */
JMODELS_ATTN_API int32_t jmodels_attn_norm_create(jmodels_attn_context* ctx, uint32_t head_dim,
                                 const float* q_weight, const float* k_weight, float eps,
                                 jmodels_attn_norm** norm_out);
/* jmodels_attn_norm_create with flags. JMODELS_ATTN_NORM_VALUE_RMS also normalises each value
 * head without a weight before it is stored, as Gemma4ForwardPass does (BJ/gemma4/
 * Gemma4ForwardPass.java:990-996): Gemma4Math.normalizeWithoutWeight (BJ/gemma4/Gemma4Math.java:
 * 38-55), v * (float)(1 / sqrt(sum(v^2) / head_dim + eps)) with the mean and eps added in float
 * and the square root and reciprocal in double; eps must then be finite and > 0, and head_dim must
 * also equal the cache's value_length. Gemma 4 layers without a value projection pass the raw
 * keys as v (BJ/gemma4/Gemma4ForwardPass.java:966-968). Unknown flag bits: INVALID_SHAPE. */
#define JMODELS_ATTN_NORM_VALUE_RMS 1u
JMODELS_ATTN_API int32_t jmodels_attn_norm_create_ex(jmodels_attn_context* ctx, uint32_t head_dim,
                                    const float* q_weight, const float* k_weight, float eps,
                                    uint32_t flags, jmodels_attn_norm** norm_out);
JMODELS_ATTN_API int32_t jmodels_attn_norm_destroy(jmodels_attn_norm* norm);

/* ---------------------------------------------------------------- KV cache */

/* A device-resident KV cache for `sequences` independent sessions of one shape (each session is
 * one backend-java KvCache, BJ/llama/LlamaForwardPass.java:412-416). Allocated at max_seq_len up
 * front (no growth copies; BJ/cache/KvCache.java:284-322 grows lazily instead).
 * ring_capacity: NULL, or num_layers entries where 0 = LINEAR and c > 0 = RING of c slots
 * (BJ/cache/LayeredKvCache.java:41-64), any c > 0; c >= max_seq_len stores the layer linearly
 * (physicalLimit = min(ringCapacity, maxSeqLen), :128-129). A ring's device storage is rounded
 * up to a multiple of 32 slots; what it retains (contains, read, the window check) follows c. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_create(jmodels_attn_context* ctx, uint32_t sequences, uint32_t num_layers,
                               uint32_t max_seq_len, uint32_t num_kv_heads, uint32_t key_length,
                               uint32_t value_length, uint32_t dtype,
                               const uint32_t* ring_capacity, jmodels_attn_kv** kv_out);
/* One layer of a layered cache: LayeredKvCache.LayerSpec (BJ/cache/LayeredKvCache.java:41-64)
 * with keyDim = num_kv_heads * key_length and valueDim = num_kv_heads * value_length, as
 * Gemma4KvCache builds them per layer (BJ/gemma4/Gemma4KvCache.java:39-47; head counts and
 * head lengths per layer from Gemma4Config.numKvHeads / headDim, BJ/gemma4/Gemma4Config.java:
 * 172-192). ring_capacity 0 = LINEAR, else RING of that many slots (any value > 0). */
typedef struct jmodels_attn_layer_spec {
  uint32_t num_kv_heads;
  uint32_t key_length;
  uint32_t value_length;
  uint32_t ring_capacity;
} jmodels_attn_layer_spec;

/* LayeredKvCache constructor (BJ/cache/LayeredKvCache.java:124-156) for `sequences` sessions:
 * num_layers specs, each layer with its own kv heads, key/value lengths and retention. Attention
 * calls use the layer's own dimensions (jmodels_attn_layer.num_heads must be a multiple of that
 * layer's num_kv_heads). Decode supports key_length == value_length in {32, 64, 128, 256, 512}
 * (f16) or {16, ..., 512} (f32). Prefill of f16 caches runs the MFMA kernel at key lengths
 * 32-256 and the paired-stripe prefill kernel at 512; f32 caches run the d-sliced kernel
 * (32-512); other supported decode shapes run the decode kernel over chunks of the prefill's
 * rows. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_create_layered(jmodels_attn_context* ctx, uint32_t sequences,
                                       uint32_t num_layers, uint32_t max_seq_len,
                                       const jmodels_attn_layer_spec* specs, uint32_t dtype,
                                       jmodels_attn_kv** kv_out);
JMODELS_ATTN_API int32_t jmodels_attn_kv_destroy(jmodels_attn_kv* kv);
/* KvCache.clear (BJ/cache/KvCache.java:156-158) for one sequence, or all when sequence < 0. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_clear(jmodels_attn_kv* kv, int32_t sequence);
/* KvCache.discardFrom / LayeredKvCache.discardFrom (BJ/cache/KvCache.java:161-173,
 * BJ/cache/LayeredKvCache.java:212-223): position in [0, max_seq_len]. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_discard_from(jmodels_attn_kv* kv, uint32_t sequence, uint32_t position);
/* LayeredKvCache.contains (BJ/cache/LayeredKvCache.java:172-175): *out = 1 if available. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_contains(const jmodels_attn_kv* kv, uint32_t sequence, uint32_t layer,
                                 uint32_t position, int32_t* out);
/* KvCache.store without RoPE (BJ/cache/KvCache.java:51-73): host vectors of the layer's
 * key_dim/value_dim. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_store(jmodels_attn_context* ctx, jmodels_attn_kv* kv, uint32_t sequence,
                              uint32_t layer, uint32_t position, const float* key,
                              uint64_t key_elements, const float* value, uint64_t value_elements);
/* keySlice/valueSlice (BJ/cache/KvCache.java:105-115, 208-230): rows [from, to) in the
 * reference's [position][kv_head * head_dim] f32 layout; either output may be NULL. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_read(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                             uint32_t sequence, uint32_t layer, uint32_t from, uint32_t to,
                             float* keys, uint64_t key_elements, float* values,
                             uint64_t value_elements);
/* Device bytes held by the cache's K and V storage. */
JMODELS_ATTN_API int32_t jmodels_attn_kv_bytes(const jmodels_attn_kv* kv, uint64_t* bytes_out);

/* ---------------------------------------------------------------- attention */

/* RoPE + KV append for `count` rows (kernel 1). Row i belongs to sequence sequences[i] at
 * position positions[i]. q [count][num_heads*key_length] and k [count][num_kv_heads*key_length]
 * are rotated with the layer's RoPE (RotaryTable.apply, BJ/llama/LlamaForwardPass.java:1070-1083);
 * the rotated q is written to q_rotated (may be NULL); the rotated k and v
 * [count][num_kv_heads*value_length] are stored at (sequence, layer, position)
 * (KvCache.store, :1086). Rows must not repeat a (sequence, position). */
JMODELS_ATTN_API int32_t jmodels_attn_append(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* q_rotated,
                            uint64_t q_rotated_elements);

/* Grouped-query attention of `count` already-rotated query rows over their cached positions
 * [first, position] (groupedQueryAttention, BJ/llama/LlamaForwardPass.java:1543-1670):
 * split-K flash-decoding (kernel 2) plus the cross-split reduction (kernel 4).
 * out [count][num_heads*value_length] f32. */
JMODELS_ATTN_API int32_t jmodels_attn_attend(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, float* out, uint64_t out_elements);

/* One decode token for `count` sessions: append then attend (the per-layer attention block of
 * LlamaForwardPass.forwardSequenceInternal :1069-1128 for count == 1, and
 * attendIndependentSessions :793-839 for count > 1). */
JMODELS_ATTN_API int32_t jmodels_attn_decode(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                            const jmodels_attn_layer* layer, uint32_t count,
                            const uint32_t* sequences, const uint32_t* positions, const float* q,
                            uint64_t q_elements, const float* k, uint64_t k_elements,
                            const float* v, uint64_t v_elements, float* out,
                            uint64_t out_elements);

/* Causal prefill of n consecutive tokens of one sequence at start .. start+n-1
 * (prepareBatchedAttention + computeBatchedAttention, BJ/llama/LlamaForwardPass.java:1479-1541):
 * RoPE + append every row (one kernel-1 launch), then jmodels_attn_attend_causal: f16 caches at
 * head dims 32-256 run the MFMA kernel (kernel 3) with f16 queries; f32 caches at 32-512 run the
 * d-sliced prefill kernel (kernel 3b: the waves of a workgroup split the head dimension and add
 * their partial score tiles through LDS); f16 caches at 512 run the paired-stripe kernel (kernel
 * 3c: two stripes share each LDS-staged tile, each split over two waves; when the pairs fit the
 * compute units at once, the longer pairs run as two workgroups over halves of their tiles,
 * merged by the later one); other shapes run the decode kernel over chunks of the rows. */
JMODELS_ATTN_API int32_t jmodels_attn_prefill(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                             const jmodels_attn_layer* layer, uint32_t sequence, uint32_t start,
                             uint32_t n, const float* q, uint64_t q_elements, const float* k,
                             uint64_t k_elements, const float* v, uint64_t v_elements,
                             float* out, uint64_t out_elements);

/* Causal attention of rows start .. start+n-1 of one sequence whose K/V are already cached and
 * whose rotated queries are q [n][num_heads*key_length] (computeBatchedAttention,
 * BJ/llama/LlamaForwardPass.java:1515-1541): row b attends [first(start+b), start+b]. This is the
 * attention half of jmodels_attn_prefill (kernel 3 on f16 caches). */
JMODELS_ATTN_API int32_t jmodels_attn_attend_causal(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t sequence,
                                   uint32_t start, uint32_t n, const float* q,
                                   uint64_t q_elements, float* out, uint64_t out_elements);

/* Device-pointer variants of the five calls above: q/k/v/q_rotated/out are device pointers
 * (sequences/positions stay host arrays: they size the launch). Asynchronous on the context
 * stream; call jmodels_attn_context_synchronize before reading results or to collect errors. */
JMODELS_ATTN_API int32_t jmodels_attn_append_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, const float* k,
                                   uint64_t k_elements, const float* v, uint64_t v_elements,
                                   float* q_rotated, uint64_t q_rotated_elements);
JMODELS_ATTN_API int32_t jmodels_attn_attend_device(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, float* out,
                                   uint64_t out_elements);
JMODELS_ATTN_API int32_t jmodels_attn_decode_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                   const jmodels_attn_layer* layer, uint32_t count,
                                   const uint32_t* sequences, const uint32_t* positions,
                                   const float* q, uint64_t q_elements, const float* k,
                                   uint64_t k_elements, const float* v, uint64_t v_elements,
                                   float* out, uint64_t out_elements);
/* jmodels_attn_decode_device without any device allocation. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Instead of the context's grow-only
 * scratch it uses one fixed array per GPU, a file-scope device array of 41 MiB (64 KiB of arrival
 * tickets, 16 MiB of fused split partials, 16 MiB + 1 MiB of partials for the separate reduction,
 * 8 MiB of rotated queries) that each GPU the library runs on holds until the process ends. A
 * launch plan needing more than a region holds is refused with BUFFER_TOO_SMALL before anything
 * is enqueued. Every call on a GPU shares that GPU's array, whatever the context: calls that
 * overlap on one GPU (two contexts' streams, or two threads) race. Sequential calls are safe:
 * each launch leaves the exchange regions as it found them. */
JMODELS_ATTN_API int32_t jmodels_attn_decode_device_noalloc(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                           const jmodels_attn_layer* layer, uint32_t count,
                                           const uint32_t* sequences, const uint32_t* positions,
                                           const float* q, uint64_t q_elements, const float* k,
                                           uint64_t k_elements, const float* v,
                                           uint64_t v_elements, float* out,
                                           uint64_t out_elements);
JMODELS_ATTN_API int32_t jmodels_attn_attend_causal_device(jmodels_attn_context* ctx, const jmodels_attn_kv* kv,
                                          const jmodels_attn_layer* layer, uint32_t sequence,
                                          uint32_t start, uint32_t n, const float* q,
                                          uint64_t q_elements, float* out,
                                          uint64_t out_elements);
JMODELS_ATTN_API int32_t jmodels_attn_prefill_device(jmodels_attn_context* ctx, jmodels_attn_kv* kv,
                                    const jmodels_attn_layer* layer, uint32_t sequence,
                                    uint32_t start, uint32_t n, const float* q,
                                    uint64_t q_elements, const float* k, uint64_t k_elements,
                                    const float* v, uint64_t v_elements, float* out,
                                    uint64_t out_elements);

/* ---------------------------------------------------------------- quantized projections
 *
 * The projections on either side of attention: Q/K/V before the append
 * (BJ/llama/LlamaForwardPass.java:1043-1067, with addOptionalBias :1065-1067) and the output
 * projection plus residual after it (:1131-1138). GGUF weight formats use backend-native's codes
 * (RS:150-161), all six on the device: 0 = Q4_0 (18-byte blocks of 32), 1 = Q8_0 (34 bytes),
 * 5 = Q5_0 (22 bytes), 2 = Q4_K (144-byte blocks of 256), 4 = Q5_K (176 bytes), 3 = Q6_K (210).
 * Q4_0 / Q8_0 / Q5_0: activations quantized to Q8_0 per 32-element block, every output the
 * in-order chain of per-block fma(weightScale * activationScale, integer dot, sum), the
 * arithmetic backend-native's tests require of its Q4_0 kernel exactly (backend-native/src/test/
 * java/.../NativeKernelLibraryTest.java:67-84, 909-993). Q4_K / Q5_K / Q6_K: Q8_K activations and
 * the float order of backend-native's scalar row kernels (RS:3410-3577; its tests hold the
 * K-quant kernels to 2e-3 of the Java path). One call takes either 32-element block formats or
 * K-quants, not both (their activation formats differ).
 *
 * Batches of 16 activation rows and more run as a register-tiled matrix product on activations
 * quantized once into the context's scratch (the same bits as the matrix-vector path); such a
 * call made while the stream is captured returns NOT_CAPTURABLE when that scratch must grow first
 * (make the call once outside the capture). Smaller batches use no scratch memory.
 *
 * Device pointers, asynchronous on the context stream. weights:
 * [rows][cols / 32 or cols / 256] blocks, 2-byte aligned; input [batch][cols] f32, 16-byte
 * aligned, cols a multiple of the block size; output [batch][rows] per matrix, matrix after matrix (a grouped Q/K/V call
 * leaves q, k and v contiguous, the layout jmodels_attn_decode_device reads). addend_mode: 0 none,
 * 1 a bias [rows] added to every batch row (addOptionalBias), 2 a residual [batch][rows] added
 * (x[i] += attnProjected[i]; the residual may be the output itself, updated in place). output must
 * not alias input. */
#define JMODELS_ATTN_WEIGHTS_Q4_0 0u
#define JMODELS_ATTN_WEIGHTS_Q8_0 1u
#define JMODELS_ATTN_WEIGHTS_Q4_K 2u
#define JMODELS_ATTN_WEIGHTS_Q6_K 3u
#define JMODELS_ATTN_WEIGHTS_Q5_K 4u
#define JMODELS_ATTN_WEIGHTS_Q5_0 5u
#define JMODELS_ATTN_ADDEND_NONE 0u
#define JMODELS_ATTN_ADDEND_BIAS 1u
#define JMODELS_ATTN_ADDEND_RESIDUAL 2u

/* jmodels_quantized_f32_batched_matmul_with_context (RS:535-580) on device memory, plus the
 * addend. */
JMODELS_ATTN_API int32_t jmodels_attn_quantized_matmul_device(jmodels_attn_context* ctx, uint32_t format,
                                             const void* weights, uint64_t weight_bytes,
                                             const float* input, uint64_t input_elements,
                                             float* output, uint64_t output_elements,
                                             uint32_t batch_size, uint32_t rows, uint32_t cols,
                                             const float* addend, uint32_t addend_mode);
/* jmodels_quantized_f32_grouped_batched_matmul_with_context (RS:582-637) on device memory: up to
 * 16 matrices (1 allowed here) sharing one activation batch; addends (NULL with addend_mode 0)
 * holds one pointer per matrix. */
JMODELS_ATTN_API int32_t jmodels_attn_quantized_grouped_matmul_device(
    jmodels_attn_context* ctx, const uint32_t* formats, const void* const* weights,
    const uint64_t* weight_bytes, const uint32_t* rows, uint32_t matrix_count, const float* input,
    uint64_t input_elements, float* output, uint64_t output_elements, uint32_t batch_size,
    uint32_t cols, const float* const* addends, uint32_t addend_mode);

#ifdef __cplusplus
}
#endif
#endif
