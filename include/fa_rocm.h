/* fa_rocm.h — C ABI of libfa_rocm.so, the MI355X (gfx950) implementation of
 * fiber/ai's EmbeddingGemma encoder path.
 *
 * Plain C: pointers, sizes and status codes; no C++ or torch types. Every
 * entry point returns 0 (FA_OK) on success or an FA_ERR_* code, with a
 * message available from fa_last_error(ctx). Argument errors the reference
 * reports by panicking with *tensor.Error{Op, Msg} (tensor/errors.go:5-31)
 * return FA_ERR_ARG here with the same kind of message, prefixed by the
 * reference's Op name; a cgo shim turns them back into that panic.
 *
 * Memory: "host" entry points (the drop-in replacements of the reference's
 * tensor/gemma functions) take host pointers, copy them to the device,
 * compute on the context's HIP stream and copy the result back before
 * returning, like the reference's functions return filled slices. The
 * "_dev" entry points take device pointers and only enqueue work on the
 * context's stream (fa_stream()); they are what a caller keeping data
 * resident in HBM uses.
 *
 * Threading: a context owns one HIP stream and per-call scratch; calls on
 * one context must be serialised by the caller (the reference's Embed is not
 * documented as goroutine-safe either, models/gemma/embed.go:15). Distinct
 * contexts may be used from distinct threads.
 *
 * HIP graphs: fa_similarities_topk_dev_noalloc is the entry point meant for
 * capture. The others are not capture-safe (they may grow device buffers on
 * a call, and fa_gemma_embed_ids_dev uploads its per-call plan from a pinned
 * host buffer that the next call rewrites and records events of the model):
 * they check hipStreamIsCapturing on the context's stream and return
 * FA_ERR_STATE while it is being captured.
 *
 * Tuning switches (environment, read once per process; unset = the measured
 * defaults; for A/B measurements only, results stay within the parity bars):
 *   FA_GEMM_XTILE=128x64v|64x128|64x64|128x128w8|128x256w8|small
 *                               force a split-bf16 product tile
 *   FA_GEMM_TILE=128x128|64x64|128x64v   force an fp32-MFMA product tile
 *   FA_GEMM_MFMA=f32            the model's and fa_matmul_fused's products on the fp32-MFMA
 *                               kernel (bf16 weights widened, float32 weights without the
 *                               three-plane rewrite)
 *   FA_ATTN_DENSE=0             fa_attention on the per-row kernel for every head dim
 *   FA_GEMM_KSPLIT=1            no K-split products in the encoder (also implied by
 *                               FA_GEMM_MFMA=f32)
 *   FA_MICROBATCH=0|<rows>      micro-batches off / from this many tokens (2048)
 *   FA_MICROBATCH_GROUPS=2..4   force the micro-batch count
 *   FA_ATTN_KEY_PARTS=1..8      force the key runs of the short-batch attention
 *   FA_ATTN_ROWS=64|128         force the tile attention's rows per work item
 *   FA_ATTN_PAIRS=0             64-row tile items on four single waves instead of
 *                               eight waves in head-dimension pairs
 *   FA_ATTN_XCD=1|0             force the XCD-local attention item order on / off
 *   FA_SMALL_KSPLIT=2           two (not four) K parts for a few-row batch's o/down
 *   FA_QKV_KSPLIT=1             no K split of a few-row batch's q|k|v product
 *   FA_SMALL_NARROW=0           no 16-feature tiles for the few-row gate|up product
 */
#ifndef FA_ROCM_H
#define FA_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FA_OK = 0,
  FA_ERR_ARG = 1,         /* bad shape/argument: the reference panics with *tensor.Error */
  FA_ERR_HIP = 2,         /* HIP runtime error (message carries hipGetErrorString) */
  FA_ERR_OOM = 3,         /* device allocation failed */
  FA_ERR_STATE = 4,       /* call out of order (e.g. embed before every weight is set) */
  FA_ERR_UNSUPPORTED = 5  /* a configuration this build does not implement */
};

enum { FA_DT_F32 = 0, FA_DT_BF16 = 1 };

/* Activation of a fused product: tensor.NoAct/ReLUAct/GELUAct
 * (tensor/matmul_fused.go:25-32). GELU is the tanh approximation
 * (internal/kernel/math.go:117-143). FA_ACT_TANH is (*Tensor).Tanh
 * (tensor/ops_unary.go:114, internal/kernel/generic.go:313-359) applied to
 * the product, which tensor.Fused does not offer: the gemma head's Dense
 * layers with a Tanh activation (models/gemma/model.go:296-301,
 * embed.go:415-418). */
enum { FA_ACT_NONE = 0, FA_ACT_RELU = 1, FA_ACT_GELU = 2, FA_ACT_TANH = 3 };

/* Layout of a product's right operand B (logical shape [k x n]):
 * FA_B_KN: row-major [k x n] with leading dimension ldb (the reference's
 *          w[in,out], tensor/matmul.go:42-72);
 * FA_B_NK: row-major [n x k] (a transposed view, i.e. a checkpoint's
 *          [out,in] weight or cluster.Similarities' docs, cluster.go:185-190). */
enum { FA_B_KN = 0, FA_B_NK = 1 };

typedef struct fa_ctx fa_ctx;
typedef struct fa_model fa_model;

/* ---- context -------------------------------------------------------- */

/* Create a context on HIP device `device` (one stream, default priority). */
int fa_create(int device, fa_ctx** out);
/* Destroy a context, after the models still open on it (fa_gemma_destroy).
 * NULL, or a handle already destroyed, is ignored. Contexts and models still
 * open when the process exits are destroyed by an exit handler the library
 * registers with atexit() at the first fa_create (after the HIP runtime has
 * initialised, so before the runtime's own teardown). */
void fa_destroy(fa_ctx* ctx);
/* Last error message of ctx, or of the calling thread when ctx is NULL
 * (for fa_create failures). Never NULL. */
const char* fa_last_error(const fa_ctx* ctx);
/* The context's HIP stream, as an opaque pointer (hipStream_t). */
void* fa_stream(fa_ctx* ctx);
/* Block until the context's stream is idle. */
int fa_sync(fa_ctx* ctx);
/* Version string of the library build. */
const char* fa_version(void);

/* Device memory helpers for callers without a HIP runtime of their own. */
int fa_device_alloc(fa_ctx* ctx, size_t bytes, void** out);
int fa_device_free(fa_ctx* ctx, void* ptr);
int fa_memcpy_h2d(fa_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */
int fa_memcpy_d2h(fa_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */

/* ---- tensor-level operators (drop-ins, host pointers) ------------------ */

/* Epilogue of a fused product, applied in the reference's order
 * Bias -> RowScale -> Act -> Mul -> Residual (internal/blas/gemm.go:276-347,
 * tensor.Fused, tensor/matmul_fused.go:11-23). Null pointers are skipped. */
typedef struct fa_epilogue {
  const float* bias;      /* [n] */
  const float* row_scale; /* [m] */
  int act;                /* FA_ACT_* */
  const float* mul;       /* [m x n], leading dimension ldm */
  int64_t ldm;
  const float* residual;  /* [m x n], leading dimension ldr */
  int64_t ldr;
} fa_epilogue;

/* C[m x n] = epilogue(A[m x k] . B) with A row-major (lda), B of dtype
 * b_dtype (FA_DT_F32 or FA_DT_BF16) in layout b_layout, C row-major (ldc).
 * Replaces tensor.MatMulFused (tensor/matmul_fused.go:40-96) and, with
 * e == NULL, the 2-D case of tensor.MatMul (tensor/matmul.go:19-72).
 * fp32 accumulation on the MFMA units; bf16 B is widened exactly. */
int fa_matmul_fused(fa_ctx* ctx, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, const void* b,
                    int64_t ldb, int b_dtype, int b_layout, const fa_epilogue* e, float* c, int64_t ldc);

/* Device-pointer variant of fa_matmul_fused: a, b, c and the epilogue's
 * arrays are device pointers; enqueues on fa_stream(ctx) and returns. */
int fa_matmul_fused_dev(fa_ctx* ctx, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, const void* b,
                        int64_t ldb, int b_dtype, int b_layout, const fa_epilogue* e, float* c, int64_t ldc);

/* A matrix operand of tensor.MatMul as the strided view the reference hands
 * its GEMM driver (blas.Mat{Data, Rows, Cols, RS, CS}, tensor/matmul.go:38-40)
 * plus the broadcast batch strides of matmulBatched (tensor/matmul.go:92-98):
 * element [i, j] of batch entry (z_0, ..., z_{nb-1}) is
 *   data[z_0*bstride[0] + ... + z_{nb-1}*bstride[nb-1] + i*rs + j*cs].
 * Strides are in elements and >= 0; a broadcast batch dimension has stride
 * 0, a transposed view has rs == 1 (tensor.T, Transpose(-2, -1)). */
#define FA_MAX_BATCH_DIMS 8
typedef struct fa_matrix {
  const float* data;
  int64_t rs, cs;
  int64_t bstride[FA_MAX_BATCH_DIMS];
} fa_matrix;

/* tensor.MatMul / MatMulFused on strided operands, the general case of
 * tensor/matmul.go:19-127: for every entry of the broadcast batch shape
 * batch[0..nbatch-1] (nbatch = 0: one 2-D product),
 *   out[z] = epilogue(A_z [m x k] . B_z [k x n]),
 * out contiguous [batch..., m, n] (the reference's fresh output tensor). A
 * and B are float32 views as described at fa_matrix; nothing is copied on
 * the host, the operands are read through their strides on the device
 * (transposed, offset, stride-0 broadcast views included). e (NULL for
 * none) is MatMulFused's epilogue and needs nbatch == 0. k == 0 gives
 * epilogue(0). Products are fp32-accurate (each fp32 value the exact sum of
 * three bf16 terms, fp32 accumulation on the bf16 MFMA). The caller does
 * 1-D promotion as the reference does (matmul.go:24-30): a 1-D left operand
 * is the row [1 x k], a 1-D right operand the column [k x 1]. Host pointers;
 * returns when out is filled. */
int fa_matmul_strided(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t m, int64_t n, int64_t k,
                      const fa_matrix* a, const fa_matrix* b, const fa_epilogue* e, float* out);
/* Device-pointer variant (a->data, b->data, out and the epilogue's arrays on
 * the device; batch and the fa_matrix structs on the host); enqueues on
 * fa_stream(ctx). */
int fa_matmul_strided_dev(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t m, int64_t n, int64_t k,
                          const fa_matrix* a, const fa_matrix* b, const fa_epilogue* e, float* out);

/* out[i] = sum_j x[i,j]^2 for row-major x [m x n].
 * Replaces (*Tensor).RowSumSquares (tensor/matmul_fused.go:125-143). */
int fa_row_sum_squares(fa_ctx* ctx, const float* x, int64_t m, int64_t n, float* out);

/* out = x / sqrt(mean(x^2) + eps) * g over the last dimension n of
 * row-major x [rows x n]; g has n elements (the caller passes 1+w for
 * Gemma). Replaces tensor.RMSNorm (tensor/attention.go:292-337). */
int fa_rmsnorm(fa_ctx* ctx, const float* x, const float* g, float eps, int64_t rows, int64_t n, float* out);

/* Rotary embedding, rotate-half convention, on contiguous x [rows x D]
 * whose row r sits at position positions[r % T] (x is [..., T, D]).
 * Angle tables in float64 rounded to float32 as the reference's.
 * Replaces tensor.RoPE (tensor/rope.go:20-61). */
int fa_rope(fa_ctx* ctx, const float* x, double base, const int32_t* positions, int64_t rows, int32_t T, int32_t D,
            float* out);

/* out = softmax(scale * q.k^T + mask) . v per (batch, head).
 * q: [B, H, T, D] with element strides (q_sb, q_sh) on the two lead
 * dimensions and rows of D contiguous at stride D; k, v: [B, H, S, D]
 * likewise (a head stride of 0 expresses grouped-query attention, the
 * reference's Expand). mask: additive, NULL or strides (m_sb, m_sh, m_sr,
 * m_sc) over [B, H, T, S] (0 where broadcast). out: [B, H, T, D]
 * contiguous. Masked weights are exactly 0 (exp of inputs below -87 flushes
 * to 0, internal/kernel/generic.go:278-307). Head dims 64, 128, 256 and
 * 512 with 16-byte aligned rows (batch and head strides multiples of 4) run
 * on the fp32 MFMA; other shapes on a per-row kernel (D <= 512).
 * Replaces tensor.AttentionScaled (tensor/attention.go:67-83,130-287). */
int fa_attention(fa_ctx* ctx, const float* q, const float* k, const float* v, int32_t B, int32_t H, int32_t T,
                 int32_t S, int32_t D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t v_sb,
                 int64_t v_sh, const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_sr, int64_t m_sc, float scale,
                 float* out);
/* Device-pointer variant of fa_attention (q, k, v, mask, out on the device;
 * enqueues on fa_stream(ctx)). */
int fa_attention_dev(fa_ctx* ctx, const float* q, const float* k, const float* v, int32_t B, int32_t H, int32_t T,
                     int32_t S, int32_t D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t v_sb,
                     int64_t v_sh, const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_sr, int64_t m_sc,
                     float scale, float* out);

/* Scores queries [nq x d] against docs [nd x d] (dot products, the rows
 * being unit length as cluster.Similarities requires, cluster.go:180-190) and
 * returns, per query, the topk largest scores in descending order with their
 * doc indices; equal scores are ordered by the lower index (the first-max
 * rule of (*Tensor).Argmax, tensor/reduce.go:269-297). 1 <= topk <= 32,
 * nq <= 65535. NaN scores rank below every number (the reference's Argmax
 * returns a NaN only when it is a row's first element; this build never
 * selects one); slots past a row's non-NaN scores get index -1 and value NaN.
 * From 128 queries with d % 32 == 0, topk <= 16 and 16-byte aligned rows the
 * scores are the exact dot products rounded to float32 and no score matrix is
 * formed (blocks of 256 queries); otherwise an fp32-MFMA product (fp32
 * accumulation, within a few units of the last place of the exact score) is
 * followed by a two-pass top-k. A query's scores, and its order among
 * candidates whose scores agree to that precision, can therefore differ
 * between a call with fewer than 128 queries (or topk > 16) and one with
 * more; fa_similarities_topk_dev_noalloc takes the exact path for any nq. */
int fa_similarities_topk(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs, int64_t nd, int32_t d,
                         int32_t topk, int32_t* idx, float* val);

/* Device-pointer variant of fa_similarities_topk (enqueue only). */
int fa_similarities_topk_dev(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs, int64_t nd, int32_t d,
                             int32_t topk, int32_t* idx, float* val);

/* fa_similarities_topk_dev without any allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops). Always the exact fused path (any
 * nq), with its scratch in a fixed 12 MiB array per device instead of the
 * context's buffers: d % 32 == 0 and d <= 2048, 1 <= topk <= 16, 16-byte
 * aligned rows, else FA_ERR_ARG. Device pointers; enqueues on
 * fa_stream(ctx). The array of a GPU belongs to the first context that calls
 * this entry point on it, until fa_destroy of that context: calls from other
 * contexts on that GPU return FA_ERR_STATE instead of racing on it. The
 * owner's calls are ordered by its stream; graphs captured from them share
 * the array too, so their replays must not overlap each other. */
int fa_similarities_topk_dev_noalloc(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs, int64_t nd,
                                     int32_t d, int32_t topk, int32_t* idx, float* val);

/* ---- cluster (cluster/cluster.go) ------------------------------------ */

/* out = x with every row scaled to unit length (x / sqrt(sum x^2)); rows of
 * length zero stay zero. x, out: [n x d] row-major; out may equal x.
 * Replaces cluster.Normalize (cluster/cluster.go:17-28). */
int fa_cluster_normalize(fa_ctx* ctx, const float* x, int64_t n, int32_t d, float* out);
/* Device-pointer variant (enqueue only). */
int fa_cluster_normalize_dev(fa_ctx* ctx, const float* x, int64_t n, int32_t d, float* out);

/* For every row of x [n x d], the index of the most similar of the k
 * centres [k x d] by dot product (the first index on equal scores, the
 * rule of (*Tensor).Argmax, tensor/reduce.go:269-297) and that
 * similarity. k >= 1. Replaces cluster.Nearest (cluster/cluster.go:134-146). */
int fa_cluster_nearest(fa_ctx* ctx, const float* x, int64_t n, const float* centres, int64_t k, int32_t d,
                       int32_t* index, float* similarity);
/* Device-pointer variant (enqueue only). */
int fa_cluster_nearest_dev(fa_ctx* ctx, const float* x, int64_t n, const float* centres, int64_t k, int32_t d,
                           int32_t* index, float* similarity);

/* k-means of the unit-length rows of x [n x d] into k groups by cosine
 * similarity, as cluster.KMeans (cluster/cluster.go:39-131): k-means++
 * seeding driven by Go's math/rand/v2 PCG seeded (seed, seed ^
 * 0x9e3779b97f4a7c15), then up to iters rounds of assignment and centre
 * update (an empty centre restarts on the worst-fitting row), stopping
 * when no row changed centre in a round after the first. Outputs the
 * fields of cluster.Result: centres [k x d] (unit length), assignment [n],
 * similarity [n] (each row's similarity to its centre at the last
 * assignment), sizes [k] and *iterations. 1 <= k <= n, else FA_ERR_ARG
 * ("cluster: k must be between 1 and the number of rows", the reference's
 * panic). n < 2^31. */
int fa_cluster_kmeans(fa_ctx* ctx, const float* x, int64_t n, int32_t d, int32_t k, int32_t iters, uint64_t seed,
                      float* centres, int32_t* assignment, float* similarity, int32_t* sizes, int32_t* iterations);
/* Device-pointer variant: x, centres, assignment, similarity and sizes in
 * device memory, *iterations on the host. Synchronises the context's stream
 * once per round (the early stop and the empty-centre restarts read the
 * round's change count and sizes). */
int fa_cluster_kmeans_dev(fa_ctx* ctx, const float* x, int64_t n, int32_t d, int32_t k, int32_t iters,
                          uint64_t seed, float* centres, int32_t* assignment, float* similarity, int32_t* sizes,
                          int32_t* iterations);

/* ---- the EmbeddingGemma model (models/gemma) ------------------------- */

#define FA_GEMMA_MAX_LAYERS 64

/* Hyper-parameters as read from config.json by gemma.LoadConfig
 * (models/gemma/config.go:19-58,153-227), Variant 0 (Gemma 3 text encoder),
 * plus the sentence-transformers head (model.go:236-310). */
typedef struct fa_gemma_config {
  int32_t hidden_size;            /* 768 */
  int32_t num_hidden_layers;      /* 24 */
  int32_t num_attention_heads;    /* 3 */
  int32_t num_key_value_heads;    /* 1 */
  int32_t head_dim;               /* 256 */
  int32_t intermediate_size;      /* 1152 */
  int32_t vocab_size;             /* 262144 */
  int32_t sliding_window;         /* 512 */
  int32_t use_bidirectional;      /* 1: window bound sliding_window/2+1 (config.go:331-339) */
  int32_t sliding_window_pattern; /* 6: layer l is full attention iff (l+1)%6 == 0 (config.go:213-225) */
  double rope_local_base_freq;    /* 1e4 */
  double rope_theta;              /* 1e6 */
  double query_pre_attn_scalar;   /* 256: score scale 1/sqrt(256) (model.go:100) */
  float rms_norm_eps;             /* 1e-6 */
  int32_t max_tokens;             /* 2048 (model.go:102-104) */
  int32_t n_dense;                /* head Dense layers (2: 768->3072->768), identity activation */
  int32_t dense_out[4];
  /* EmbeddingGemma 2 text tower (variant 2; models/gemma/config.go:247-297,
   * model.go:105-205, embed.go:247-377); all zero for the Gemma 3 encoder.
   * Variant 2 reads sliding_window as an inclusive radius (a sliding layer
   * attends while |i-j| <= sliding_window, config.go:331-335), scores are
   * not scaled (query_pre_attn_scalar unused, model.go:105-110), RMSNorm
   * weights multiply the normalised value as stored (no 1 + w,
   * model.go:128-140), v is RMS-normalised without a weight, and sliding
   * layers use rope_local_base_freq, full layers rope_theta. */
  int32_t variant;                     /* 0: Gemma 3 encoder; 2: EmbeddingGemma 2 */
  int32_t hidden_size_per_layer_input; /* P: width of each layer's per-layer input */
  int32_t embedding_dim;               /* output of embedding_projection (the pooled vector's projection) */
  int32_t layer_head_dim[FA_GEMMA_MAX_LAYERS];  /* per layer; 0 = head_dim */
  int32_t layer_kv_heads[FA_GEMMA_MAX_LAYERS];  /* per layer; 0 = num_key_value_heads */
  int32_t layer_sliding[FA_GEMMA_MAX_LAYERS];   /* variant 2: 1 sliding window, 0 full attention */
  /* Activation after each head Dense layer: FA_ACT_NONE (identity) or
   * FA_ACT_TANH ("torch.nn.modules.activation.Tanh", model.go:296-301). */
  int32_t dense_act[4];
} fa_gemma_config;

/* Create an empty model on ctx (no weights yet). Replaces the allocation
 * part of gemma.Load (models/gemma/model.go:76-232). */
int fa_gemma_create(fa_ctx* ctx, const fa_gemma_config* cfg, fa_model** out);
/* Release a model (gemma's Close, model.go:381). NULL, or a model already
 * released (with its context, or at exit), is ignored. */
void fa_gemma_destroy(fa_model* m);

/* Upload one checkpoint tensor by its Hugging Face name, as gemma.Load
 * reads them (model.go:142-191): "embed_tokens.weight", "norm.weight",
 * "layers.<i>.{input_layernorm,post_attention_layernorm,
 * pre_feedforward_layernorm,post_feedforward_layernorm}.weight",
 * "layers.<i>.self_attn.{q,k,v,o}_proj.weight", "layers.<i>.self_attn.
 * {q,k}_norm.weight", "layers.<i>.mlp.{gate,up,down}_proj.weight", and the
 * head's "dense.<i>.linear.weight" (model.go:277-304). Shapes are the
 * checkpoint's ([out, in] for matrices). FA_DT_BF16 matrices, and FA_DT_F32
 * ones whose values are all bf16-exact, are kept as bf16; any other FA_DT_F32
 * matrix (a float32 or float16 checkpoint, safetensors/convert.go:23-55) is
 * kept exactly as three bf16 planes hi + mid + lo and its products run the
 * six-term split kernel. Norm vectors are kept in float32 with Gemma's 1+w
 * applied (model.go:131-140). */
int fa_gemma_set_weight(fa_model* m, const char* name, int dtype, const int64_t* shape, int32_t ndim,
                        const void* data);

/* Check that every tensor was set and prepare the device-side tables
 * (RoPE cos/sin for both bases). */
int fa_gemma_finalize(fa_model* m);

/* Embeddings of B token-id sequences: ids [B x T] row-major, right-padded
 * (any pad value), lengths [B] with 1 <= lengths[b] <= T <= max_tokens;
 * out [B x dim], 1 <= dim <= final width (Matryoshka truncation before L2,
 * embed.go:421-427); dim <= 0 means the full width. Runs the encoder, masked
 * mean pooling, the Dense head and L2 normalisation. Host pointers; returns
 * when out is filled. Replaces (*Model).embedBatch (models/gemma/embed.go:
 * 118-157), the ids-level core of (*Model).Embed (embed.go:15-80). */
int fa_gemma_embed_ids(fa_model* m, const int32_t* ids, const int32_t* lengths, int32_t B, int32_t T, int32_t dim,
                       float* out);

/* Same computation on device-resident data: d_ids [B x T] on the device,
 * lengths on the HOST (they set the launch shapes), d_out [B x dim] on the
 * device. Enqueues on fa_stream(ctx) and returns without waiting. From
 * 2 048 tokens on, the layers of two to four token-balanced groups of
 * sequences (four for long sequences, two from 16 384 tokens, else three)
 * run on the model's own extra streams, forked from and joined back into
 * fa_stream(ctx), so the call stays ordered on that stream. */
int fa_gemma_embed_ids_dev(fa_model* m, const int32_t* d_ids, const int32_t* lengths, int32_t B, int32_t T,
                           int32_t dim, float* d_out);

/* The encoder's hidden states of a batch, as (*Model).encode returns them
 * before pooling (models/gemma/embed.go:160-240): with n_layers < 0, the
 * final hidden states h = RMSNorm(x; 1+w_final); with 0 <= n_layers <=
 * num_hidden_layers, the residual stream x after the first n_layers layers
 * (0: the scaled embedding gather, embed.go:175-176), for layer-by-layer
 * inspection. hidden receives the valid rows only, packed
 * in batch order: [sum(lengths) x hidden_size], sequence b's token t at row
 * lengths[0] + ... + lengths[b-1] + t. Arguments and errors as
 * fa_gemma_embed_ids. Host pointers; returns when hidden is filled. */
int fa_gemma_encode_ids(fa_model* m, const int32_t* ids, const int32_t* lengths, int32_t B, int32_t T,
                        int32_t n_layers, float* hidden);
/* Device-pointer variant (lengths on the host; enqueue only). */
int fa_gemma_encode_ids_dev(fa_model* m, const int32_t* d_ids, const int32_t* lengths, int32_t B, int32_t T,
                            int32_t n_layers, float* d_hidden);

/* Per-kernel timing with HIP events on the model's stream, for roofline
 * reporting: when enabled, each kernel launch of the forward pass is
 * bracketed by events and its duration accumulated under its kind. */
enum {
  FA_K_GEMM_QKV = 0,
  FA_K_GEMM_O = 1,
  FA_K_GEMM_GATEUP = 2,
  FA_K_GEMM_DOWN = 3,
  FA_K_GEMM_HEAD = 4,
  FA_K_ATTENTION = 5,
  FA_K_QKNORM_ROPE = 6,
  FA_K_RESIDUAL_NORM = 7,
  FA_K_GATHER = 8,
  FA_K_POOL_L2 = 9,
  FA_K_GEMM_PLE = 10,  /* EmbeddingGemma 2: per-layer input projection, gate and projection products */
  FA_K_PLE_NORM = 11,  /* EmbeddingGemma 2: per-layer input RMSNorm */
  FA_K_COUNT = 12
};
/* While enabled, every launch is bracketed by events and the forward runs
 * on one stream (no micro-batches), so the durations are those of
 * full-batch launches. */
int fa_gemma_set_profiling(fa_model* m, int enabled);
/* Accumulated launches, milliseconds, flops and bytes (algorithmic) for one
 * kind since the last reset; synchronises the stream. */
int fa_gemma_kernel_stats(fa_model* m, int kind, int64_t* launches, double* ms, double* flops, double* bytes);
int fa_gemma_reset_stats(fa_model* m);

#ifdef __cplusplus
}
#endif
#endif
