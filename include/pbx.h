/*
 * pbx.h -- C ABI of the MI355X (gfx950) backend for PureBee's quantized
 * matmul / matvec instruction.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, and
 * returns an int status (PBX_OK == 0, negative PBX_E* on failure).  The
 * message for the last failure is returned by pbx_last_error(ctx)
 * (pbx_last_error(NULL) for failures that happen before a context exists).
 * Arguments are validated on the host before any HIP call, so every error
 * path can be exercised without a GPU.
 *
 * Weight orientation is GGUF's: a weight is N rows (output features) of K
 * columns (input features), row n holding K/32 consecutive blocks
 * (gguf.js:36-49; streaming-loader.js:257-259 reads N = dims[1], K = dims[0]).
 *
 * The reference interface each entry point replaces is cited beside it
 * (file:line in sammcj/purebee).  The reference is JavaScript: its "ABI" is
 * the JS module surface of wasm-q4.js, engine.js and purebee.js, which the
 * N-API addon (purebee_amd/napi) and the JS modules (purebee_amd/js) expose
 * on top of this header.
 */
#ifndef PBX_H
#define PBX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------- */
#define PBX_OK        0
#define PBX_EINVAL   -1   /* bad argument (shape, size, null pointer, type) */
#define PBX_ENODEV   -2   /* no HIP device / device index out of range      */
#define PBX_ENOMEM   -3   /* device or pinned host allocation failed         */
#define PBX_EHIP     -4   /* a HIP runtime call failed                       */
#define PBX_ENOTSUP  -5   /* shape or type not supported by any kernel       */
#define PBX_ELOAD    -6   /* code object missing or not loadable (hipModuleLoad) */
#define PBX_EIO      -7   /* a file could not be opened or mapped            */
#define PBX_ETIMEOUT -8   /* a bounded device-side wait gave up: data that one
                             workgroup publishes for another inside a launch
                             never arrived; the call's results are invalid   */

/* ---- weight types ----------------------------------------------------
 * GGML numbering, as gguf.js:30-33 (GGML_TYPE).  PBX_TYPE_Q8_REF is the
 * reference's own in-memory Q8 tensor (quantize.js:30-50, QuantizedTensor
 * 'q8_0'): int8 values of a [K,N] matrix laid out flat, one f32 scale per
 * 32 consecutive flat elements, consumed by matmul_q8 (quantize.js:224-266).
 */
#define PBX_TYPE_F32     0
#define PBX_TYPE_F16     1
#define PBX_TYPE_Q4_0    2
#define PBX_TYPE_Q4_1    3
#define PBX_TYPE_Q8_0    8
#define PBX_TYPE_Q6_K    14
#define PBX_TYPE_Q8_REF  100

typedef struct pbx_ctx pbx_ctx;
typedef struct pbx_weight pbx_weight;

/* ---- context ----------------------------------------------------------
 * Replaces wasmQ4.init() (wasm-q4.js:647-668) / engine.initWasm()
 * (engine.js:28-31): selects the device, creates the context's stream and
 * loads the gfx950 code object with hipModuleLoad.  A context is used from
 * one host thread at a time (the reference calls everything from the main
 * JS thread, thread-pool.js:3-7).
 */
int         pbx_init(int device, pbx_ctx **out);
void        pbx_shutdown(pbx_ctx *ctx);
const char *pbx_last_error(const pbx_ctx *ctx);
/* Device name (NUL-terminated, truncated to cap) and compute-unit count. */
int         pbx_device_info(pbx_ctx *ctx, char *name, size_t cap, int *cu_count);

/* ---- resident weights ------------------------------------------------
 * Replaces the per-call copy of the raw block bytes into WASM memory
 * (wasm-q4.js:735-738) and wasmSimd.allocWeights / engine.cacheWeight
 * (wasm-simd.js:406-414, engine.js:39-42): the bytes are copied to the GPU
 * once through pinned staging buffers and repacked there into the layout
 * the kernels read; the handle stays valid until pbx_weight_free.
 *
 * host/nbytes hold GGUF row-major blocks: N rows of K/32 blocks of
 * 18 B (Q4_0: fp16 d + 16 nibble bytes), 20 B (Q4_1: fp16 d, fp16 m +
 * 16 nibble bytes) or 34 B (Q8_0: fp16 d + 32 int8), or of K/256 blocks of
 * 210 B (Q6_K: ql[128], qh[64], int8 scales[16], fp16 d), gguf.js:36-49 and
 * 239-364; for PBX_TYPE_F32 / PBX_TYPE_F16, N*K little-endian floats /
 * halves.  K must be a multiple of 32 for every type (256 for Q6_K).
 */
int pbx_weight_upload(pbx_ctx *ctx, int type, int64_t N, int64_t K,
                      const void *host, size_t nbytes, pbx_weight **out);
/* The reference's QuantizedTensor 'q8_0' of shape [K,N] (quantize.js:30-50):
 * q = K*N int8 values, scales = ceil(K*N/32) f32 values. */
int pbx_weight_upload_q8ref(pbx_ctx *ctx, int64_t K, int64_t N,
                            const int8_t *q, const float *scales,
                            int64_t n_scales, pbx_weight **out);
/* Replaces wasmSimd.resetWeights (wasm-simd.js:511-513) / PureBee.FREE
 * (purebee.js:200-202) for a resident weight. */
int pbx_weight_free(pbx_ctx *ctx, pbx_weight *w);
int pbx_weight_info(const pbx_weight *w, int *type, int64_t *N, int64_t *K,
                    size_t *device_bytes);

/* ---- the instruction -------------------------------------------------
 * Y[M,N] = X[M,K] . W^T (+ bias[N]), fp32 in and out.
 *   M == 1   -> fused unpack/dequant/dot GEMV (one wavefront per row group)
 *   M >= 2   -> dequant -> LDS -> fp16 MFMA GEMM (quantized types)
 * Replaces, with the same arithmetic meaning:
 *   wasmQ4.q4_0_matvec(x, rawBuf, N, K)           wasm-q4.js:716-747
 *   quantizedMatvec(x, rawBuf, type, N, K)        llama-streaming.js:168-177
 *   AtomicsThreadPool.matvec(...)                 thread-pool.js:165-246
 *   wasmQ4.lmHead(hidden, emb, vocab, dim) (F32)  wasm-q4.js:798-839
 *   engine.tensorMulAdd(x, W, b)  (F32)           engine.js:180-244
 *   engine.tensorMulAddQ8(x, Wq, b) (Q8_REF)      engine.js:259-269,
 *                                                 quantize.js:224-266
 * pbx_linear takes host pointers and blocks until Y is written (the
 * reference's synchronous convention, wasm-q4.js:744-746).  pbx_linear_dev
 * takes device pointers and only enqueues on the context's stream.
 * bias may be NULL.
 */
int pbx_linear(pbx_ctx *ctx, const pbx_weight *W, const float *X, int64_t M,
               const float *bias, float *Y);
int pbx_linear_dev(pbx_ctx *ctx, const pbx_weight *W, const float *dX,
                   int64_t M, const float *dBias, float *dY);
/* pbx_linear_dev that allocates nothing: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The same
 * kernels and results as pbx_linear_dev; the M >= 4 GEMM's activation pair,
 * row scales and split-K partials live in one static device array of
 * PBX_NOALLOC_WORKSPACE_BYTES per GPU (held until the process ends) instead
 * of the context's grow-only buffers.  A shape that needs more workspace
 * fails with PBX_EINVAL.  Calls on one GPU share that array: calls that
 * overlap on one GPU (other contexts or streams) race. */
#define PBX_NOALLOC_WORKSPACE_BYTES (64u << 20)
int pbx_linear_dev_noalloc(pbx_ctx *ctx, const pbx_weight *W, const float *dX, int64_t M,
                           const float *dBias, float *dY);
/* Introspection for the two above, no reference counterpart (tests and
 * capacity planning): *grown_bytes = device workspace the allocating entry
 * points of this context have allocated so far (the noalloc one never adds
 * to it), *static_bytes = the static workspace of the noalloc one (0 when
 * it is unavailable); pbx_ctx_stream = the context's HIP stream (a
 * hipStream_t), on which every enqueueing entry point works, for callers
 * that capture that work into a graph or order their own work after it. */
int   pbx_workspace_info(const pbx_ctx *ctx, size_t *grown_bytes, size_t *static_bytes);
void *pbx_ctx_stream(const pbx_ctx *ctx);

/* Exact dequantisation of a resident weight to fp32, row-major [N,K]
 * (for PBX_TYPE_Q8_REF: [K,N], the reference's own orientation).
 * Replaces loadTensorData's Q4_0/Q8_0 branches (gguf.js:239-286) and
 * dequantize_q8 (quantize.js:170-181).  Bit-exact by construction. */
int pbx_dequant(pbx_ctx *ctx, const pbx_weight *W, float *Y);
int pbx_dequant_dev(pbx_ctx *ctx, const pbx_weight *W, float *dY);

/* ---- host-side quantisers (CPU) ---------------------------------------
 * Q8_0 with the numerics of quantize_q8 (quantize.js:79-109: absmax/127,
 * ECMAScript Math.round of x*127/absmax in double) applied per 32-block
 * along K of each row, the scale stored as fp16 (GGUF Q8_0 layout).
 * Q4_0 with d = absmax/8 stored as fp16 and nibble = clamp(round(x*8/absmax),
 * -8, 7) + 8, GGUF non-interleaved nibble order (gguf.js:259-286).
 * Q4_1 with d = (max-min)/15 and m = min stored as fp16 and nibble =
 * clamp(round((x-m)/d), 0, 15) against the stored values (GGUF Q4_1 layout,
 * gguf.js:288-314).  The reference reads Q4_1 but has no quantiser for it.
 * Q6_K (gguf.js:317-364 layout) with sub-block scales absmax/31 rounded
 * to int8 steps of d = max/127 (fp16) and codes clamp(round(x/(d*sc)),
 * -32, 31) + 32; the reference reads Q6_K but has no quantiser for it.
 * out must hold N*K/32*34 (Q8_0), N*K/32*18 (Q4_0), N*K/32*20 (Q4_1) or
 * N*K/256*210 (Q6_K, K % 256 == 0) bytes. */
int pbx_quantize_q8_0(const float *w, int64_t N, int64_t K, uint8_t *out);
int pbx_quantize_q4_0(const float *w, int64_t N, int64_t K, uint8_t *out);
int pbx_quantize_q4_1(const float *w, int64_t N, int64_t K, uint8_t *out);
int pbx_quantize_q6_k(const float *w, int64_t N, int64_t K, uint8_t *out);
/* quantize_q8 itself (quantize.js:79-109): flat, f32 scales (Q8_REF). */
int pbx_quantize_q8_ref(const float *w, int64_t n, int8_t *q, float *scales);

/* Seeded synthetic data: element i of the stream is a pure function of
 * (seed, i): SplitMix64 -> Box-Muller in double -> mean + std*z as float. */
int pbx_synth_normal(uint64_t seed, int64_t n, double mean, double std,
                     float *out);

/* ---- device memory, streams, timing (for callers on device pointers) -- */
int pbx_dev_alloc(pbx_ctx *ctx, size_t bytes, void **out);
int pbx_dev_free(pbx_ctx *ctx, void *p);
int pbx_memcpy_h2d(pbx_ctx *ctx, void *dst, const void *src, size_t bytes);
int pbx_memcpy_d2h(pbx_ctx *ctx, void *dst, const void *src, size_t bytes);
int pbx_memset_dev(pbx_ctx *ctx, void *dst, int value, size_t bytes);
/* Device-to-device copy by a plain kernel (bytes and both addresses 16-byte
 * aligned): a known-traffic kernel for calibrating hardware byte counters.
 * No reference counterpart. */
int pbx_dev_copy(pbx_ctx *ctx, void *dst, const void *src, size_t bytes);
int pbx_sync(pbx_ctx *ctx);
/* HIP events recorded on the context's stream: the kernels' own stream. */
int pbx_timer_start(pbx_ctx *ctx);
int pbx_timer_stop(pbx_ctx *ctx, double *elapsed_ms);
/* Enqueue `reps` passes over n_ops (W[i], dX[i] -> dY[i]) linears at row
 * count M and return the elapsed time between HIP events recorded on the
 * context's stream around the whole sequence. */
int pbx_bench_linear(pbx_ctx *ctx, int n_ops, const pbx_weight *const *W,
                     const float *const *dX, float *const *dY, int64_t M,
                     int reps, double *elapsed_ms);
/* The same pass captured once into a HIP graph and replayed `reps` times
 * (the launches stream without host launch gaps).  Timing helpers; no
 * reference counterpart. */
int pbx_bench_linear_graph(pbx_ctx *ctx, int n_ops, const pbx_weight *const *W,
                           const float *const *dX, float *const *dY, int64_t M,
                           int reps, double *elapsed_ms);

/* ---- resident model and on-GPU decode step ----------------------------
 * A Llama-family model held in device memory, replacing the reference's
 * runtimes for decode: LlamaRuntime.forward (llama.js:204-371) and
 * StreamingLlamaRuntime.forward/_runLayerQ4 (llama-streaming.js:505-606,
 * 738-815): RMSNorm (eps), q/k/v, RoPE on adjacent pairs with theta,
 * KV cache, grouped-query attention, output projection + residual, RMSNorm,
 * SwiGLU FFN + residual; final RMSNorm, LM head, greedy argmax (first
 * maximum, llama.js:432-442).  Activations and the KV cache are fp32.
 */
typedef struct pbx_model pbx_model;

typedef struct pbx_model_config {
  int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim;
  int32_t vocab_size, max_seq;
  int32_t weight_type;  /* every layer matrix: any PBX_TYPE_* but Q8_REF    */
  int32_t embed_type;   /* token_embd (row lookup and, when tied, LM head) */
  int32_t output_type;  /* untied LM head type, or -1: tied to token_embd  */
  float rms_eps;        /* 1e-5 in the reference (purebee.js:164)         */
  double rope_theta;    /* 10000 (llama.js:33) or the GGUF rope.freq_base */
} pbx_model_config;

/* Tensor ids for pbx_model_set_tensor, named as the GGUF tensors they take
 * (gguf.js:378-410).  Matrices are GGUF row-major blocks of their type,
 * [N rows = out features][K = in features]; norms are f32. */
#define PBX_T_TOKEN_EMBD   0   /* [vocab, dim]   embed_type            */
#define PBX_T_OUTPUT       1   /* [vocab, dim]   output_type (untied)  */
#define PBX_T_OUTPUT_NORM  2   /* [dim] f32                            */
#define PBX_T_ATTN_NORM    3   /* per layer: [dim] f32                 */
#define PBX_T_FFN_NORM     4   /* per layer: [dim] f32                 */
#define PBX_T_ATTN_Q       5   /* per layer: [dim, dim]                */
#define PBX_T_ATTN_K       6   /* per layer: [kv_dim, dim]             */
#define PBX_T_ATTN_V       7   /* per layer: [kv_dim, dim]             */
#define PBX_T_ATTN_OUTPUT  8   /* per layer: [dim, dim]                */
#define PBX_T_FFN_GATE     9   /* per layer: [hidden, dim]   (w1)      */
#define PBX_T_FFN_UP      10   /* per layer: [hidden, dim]   (w3)      */
#define PBX_T_FFN_DOWN    11   /* per layer: [dim, hidden]   (w2)      */

int pbx_model_create(pbx_ctx *ctx, const pbx_model_config *cfg, pbx_model **out);
int pbx_model_free(pbx_model *m);
/* Replaces the loaders' per-tensor reads (streaming-loader.js:245-299,
 * loadResidentWeights 324-335): one upload, resident afterwards. */
int pbx_model_set_tensor(pbx_model *m, int tensor, int layer, const void *data,
                         size_t nbytes);
/* forward(tokenIds, startPos) (llama.js:204, llama-streaming.js:738):
 * runs tokens[0..n) at positions start_pos.., writing the KV cache; returns
 * the last position's logits (if logits != NULL, [vocab]) and its argmax. */
int pbx_model_forward(pbx_model *m, const int32_t *tokens, int n_tokens,
                      int start_pos, float *logits, int32_t *next_token);
/* StreamingLlamaRuntime.forward(tokenIds, startPos, {maxLayers})
 * (llama-streaming.js:738-815): as pbx_model_forward, but only the first
 * max_layers layers run (0: all of them, `maxLayers || nLayers`; the limit
 * is min(max_layers, n_layers)), then the final RMSNorm and the LM head on
 * their output; the KV cache of the later layers is not written at these
 * positions.  *layers_used (if not NULL) receives the layers run, the
 * `layersUsed` of the reference's result. */
int pbx_model_forward_layers(pbx_model *m, const int32_t *tokens, int n_tokens,
                             int start_pos, int max_layers, float *logits,
                             int32_t *next_token, int *layers_used);
/* forward() over n tokens in ONE batched pass that keeps every position's
 * output (the reference computes them inside forward, llama.js:204-371, and
 * keeps only the last): logits [n][vocab] (or NULL) and next_tokens[n], the
 * argmax of each row (or NULL).  Quantized matrices run on the MFMA GEMM
 * with all n rows; this is the speculative verify of speculative.js:131-185
 * done as one forward instead of one forward per draft token. */
int pbx_model_forward_batch(pbx_model *m, const int32_t *tokens, int n_tokens,
                            int start_pos, float *logits, int32_t *next_tokens);
/* The greedy decode loop of generate() (llama.js:475-489): feeds `token` at
 * start_pos, then each step's argmax, n_steps times, entirely on the GPU;
 * out_tokens[i] is the token chosen by step i. */
int pbx_model_generate(pbx_model *m, int32_t token, int start_pos, int n_steps,
                       int32_t *out_tokens, float *last_logits);
/* The same loop stopping at the first token in eos_ids[0..n_eos), as
 * llama.js:475-489 stops at eosId (`if (nextToken === eosId) break`):
 * out_tokens receives the *n_out <= max_steps chosen tokens, the EOS last if
 * one was chosen, and the cache holds no row past the position that fed it.
 * Steps run in chunks of whole graph launches, the chunk's tokens checked
 * on the host after each. */
int pbx_model_generate_eos(pbx_model *m, int32_t token, int start_pos, int max_steps,
                           const int32_t *eos_ids, int n_eos, int32_t *out_tokens,
                           int *n_out);
/* resetCache / rollbackCache (llama-streaming.js:828-862): zero cache
 * positions >= pos of every layer. */
int pbx_model_reset_cache(pbx_model *m);
int pbx_model_rollback(pbx_model *m, int pos);
int pbx_model_info(const pbx_model *m, size_t *device_bytes, int *uses_graph);
/* Measurement: n_steps greedy decode steps launched kernel by kernel (no
 * graph), each kernel carrying a start and a stop HIP event that its own
 * dispatch stamps (hipExtModuleLaunchKernel).  op_us[i] is the mean
 * execution time of kernel i (the duration a kernel trace reports, without
 * the gaps between kernels), op_bytes[i] its mean algorithmic bytes (may be
 * NULL); *n_ops is the kernel count per step (arrays hold min(cap, *n_ops)
 * entries).
 * pbx_model_op_name gives "role:kernel" of kernel i (no reference
 * counterpart: the reference has no GPU kernels to profile). */
int pbx_model_profile(pbx_model *m, int32_t token, int start_pos, int n_steps,
                      double *op_us, double *op_bytes, int cap, int *n_ops);
int pbx_model_op_name(const pbx_model *m, int i, char *buf, size_t cap);
/* Test hook, no reference counterpart: makes the attention workgroups of
 * layer `layer`'s joined q|k|v + attention launch wait for cells tagged
 * `skew` epochs ahead (none ever are), giving up after `spin` polls (0: the
 * kernel's default), so that the bounded wait's error path can be tested
 * with every kernel still exiting normally; the call then fails with
 * PBX_ETIMEOUT.  layer < 0 restores the normal launch.  Returns
 * PBX_ENOTSUP when the model's step has no such launch. */
int pbx_model_test_handoff(pbx_model *m, int layer, int skew, int spin);
/* Measurement: the GEMV kernels of one role ("qkv", "o", "gate_up", "down",
 * "lm_head") launched back to back over every layer's weights, `reps`
 * passes between two HIP events on the model's stream; returns the mean
 * time and algorithmic bytes per launch.  Leaves the activations in an
 * unspecified state (the next forward re-embeds its token). */
int pbx_model_bench_role(pbx_model *m, const char *role, int reps,
                         double *us_per_launch, double *bytes_per_launch,
                         int *launches_per_rep);

/* ---- GGUF files ----------------------------------------------------------
 * The build's own GGUF v2/v3 reader, replacing GGUFParser and parseHeader
 * (gguf.js:76-194, streaming-loader.js:35-87): the file is mapped read-only,
 * header, metadata and tensor table are parsed with bounds checks, and
 * tensor data is served from the mapping (no copy).  Errors follow the
 * reference's: bad magic, a version outside 2..3, a tensor type the
 * reference cannot size (gguf.js:36-49, 206-213) fail the open.  pbx_gguf_*
 * calls take no context; pbx_last_error(NULL) names the failure.
 */
typedef struct pbx_gguf pbx_gguf;

typedef struct pbx_gguf_tensor {
  const char *name;      /* NUL-terminated, valid until pbx_gguf_close      */
  int32_t type;          /* GGML type id (gguf.js:30-33)                   */
  int32_t n_dims;        /* 1..4                                            */
  int64_t dims[4];       /* GGUF order: dims[0] = row length (K), dims[1] =
                            rows (N); unused dims are 1                     */
  uint64_t offset;       /* absolute file offset of the data                */
  uint64_t nbytes;       /* tensorByteSize (gguf.js:206-213)                */
  const void *data;      /* the bytes, inside the read-only mapping         */
} pbx_gguf_tensor;

int     pbx_gguf_open(const char *path, pbx_gguf **out);
void    pbx_gguf_close(pbx_gguf *g);
int     pbx_gguf_info(const pbx_gguf *g, uint32_t *version, int64_t *n_tensors,
                      int64_t *n_kv, uint64_t *data_start);
int     pbx_gguf_tensor_info(const pbx_gguf *g, int64_t i, pbx_gguf_tensor *out);
int64_t pbx_gguf_find_tensor(const pbx_gguf *g, const char *name);  /* -1: absent */
/* Metadata by key: integers (any integer type or bool), floats (f32/f64 or
 * an integer), strings (pointer into the mapping, not NUL-terminated),
 * arrays (element type and count). */
int pbx_gguf_get_int(const pbx_gguf *g, const char *key, int64_t *out);
int pbx_gguf_get_float(const pbx_gguf *g, const char *key, double *out);
int pbx_gguf_get_string(const pbx_gguf *g, const char *key, const char **str, uint64_t *len);
int pbx_gguf_get_array(const pbx_gguf *g, const char *key, uint32_t *elem_type,
                       uint64_t *count);
/* extractConfig (gguf.js:429-450) under general.architecture with the
 * reference's defaults (head_count_kv = head_count, rms eps 1e-5, rope
 * freq_base 10000); vocab_size = the tokenizer's token count
 * (streaming-loader.js:57) or token_embd's rows; weight/embed/output types
 * from blk.0.attn_q / token_embd / output (-1: tied).  max_seq <= 0 takes
 * min(context_length, 8192). */
int pbx_gguf_model_config(const pbx_gguf *g, int max_seq, pbx_model_config *cfg);
/* loadGGUFModel (gguf.js:778-839) / StreamingLlamaRuntime's loader
 * (streaming-loader.js:245-335) as one step: open, configure, create the
 * model and upload every tensor once, names mapped as gguf.js:378-410.
 * Token embedding and output rows past the vocabulary are not uploaded.
 * Tensors outside the Llama layout, layer matrices of mixed types and
 * shapes that disagree with the metadata are errors. */
int pbx_model_load_gguf(pbx_ctx *ctx, const char *path, int max_seq, pbx_model **out);

/* ---- speculative decoding ----------------------------------------------
 * SelfSpeculativeDecoder.generate (speculative.js:58-204) in its greedy
 * mode, with the draft taken from a separate (smaller) model instead of the
 * target's first layers.  Both caches are reset, the prompt is prefilled
 * into both, then each round drafts up to draft_count tokens with `draft`,
 * verifies them with `target`, accepts the longest agreeing prefix, emits
 * the target's own token at the first disagreement (or a bonus token when
 * every draft agrees) and rolls the target's cache back past the rejected
 * positions.  batched_verify = 1 verifies a round's drafts in one
 * pbx_model_forward_batch (M = drafts + 1); 0 verifies them one forward at
 * a time as the reference does.  Token ids outside a model's vocabulary are
 * taken modulo it (draft and target vocabularies may differ).
 * out_tokens receives the generated tokens (not the prompt): at most
 * max_tokens + 1 of them (the reference's bound), *n_out of them. */
typedef struct pbx_spec_stats {
  int32_t rounds, drafted, accepted;
  double prefill_ms, decode_ms;  /* host wall clock around the two phases */
} pbx_spec_stats;

int pbx_speculative_generate(pbx_model *target, pbx_model *draft, const int32_t *prompt,
                             int n_prompt, int max_tokens, int draft_count,
                             const int32_t *eos_ids, int n_eos, int batched_verify,
                             int32_t *out_tokens, int *n_out, pbx_spec_stats *stats);

/* SelfSpeculativeDecoder.generate (speculative.js:58-204) as the reference
 * runs it, greedy: the draft is the model's own first draft_layers layers
 * (forward([t], pos, {maxLayers: draftLayers}) and argmax, draft_count
 * times, speculative.js:96-111), on its own KV cache; the rest as
 * pbx_speculative_generate with target = draft = m.  Prompt tokens must lie
 * in the vocabulary. */
int pbx_self_speculative_generate(pbx_model *m, const int32_t *prompt, int n_prompt,
                                  int max_tokens, int draft_layers, int draft_count,
                                  const int32_t *eos_ids, int n_eos, int batched_verify,
                                  int32_t *out_tokens, int *n_out, pbx_spec_stats *stats);

#ifdef __cplusplus
}
#endif

#endif /* PBX_H */
