// Internal declarations shared by the translation units of libfa_rocm.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "fa_rocm.h"

namespace fa {

// ---- errors ----------------------------------------------------------------

struct Status {
  int code = FA_OK;
  std::string msg;
};

// Records msg as the last error of ctx (or of the thread when ctx is null)
// and returns code.
int set_error(fa_ctx* ctx, int code, const char* fmt, ...) __attribute__((format(printf, 3, 4)));

#define FA_HIP_CHECK(ctx, expr)                                                                        \
  do {                                                                                                 \
    hipError_t _e = (expr);                                                                            \
    if (_e != hipSuccess)                                                                              \
      return ::fa::set_error((ctx), FA_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                             __LINE__);                                                                \
  } while (0)

#define FA_CHECK_LAUNCH(ctx) FA_HIP_CHECK(ctx, hipGetLastError())

// ---- scratch arena ---------------------------------------------------------

// A device buffer that only grows. Used for the copies of host operands in
// the drop-in entry points and for the model's activations.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  int ensure(fa_ctx* ctx, size_t need);
  void release();
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// Scratch slots of fa_ctx (per-call device buffers of the entry points).
namespace slots {
enum : size_t {
  S_A = 0, S_B, S_C, S_BIAS, S_ROWSCALE, S_MUL, S_RES, S_X, S_G, S_OUT, S_COS, S_SIN, S_Q, S_K, S_V, S_MASK,
  S_CL_WORK, S_CL_X, S_CL_C, S_CL_OUT,  // cluster entry points
  S_TOPK,                               // top-k candidates
  S_BPLANES,                            // B operand as bf16 [n x k] planes (matmul drop-in)
  S_APACK,                              // A operand packed to [nb][m][kp] (strided matmul)
  S_COUNT
};
}  // namespace slots

}  // namespace fa

struct fa_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string last_error;
  // Per-slot scratch for the entry points. A fixed array: a reference to one
  // slot stays valid while others are taken.
  fa::DevBuf scratch[fa::slots::S_COUNT];
  int cu_count = 0;
  fa::DevBuf& slot(size_t i) { return scratch[i]; }
};

namespace fa {

// Handle registry (context.cpp): models are tracked with their context so
// that fa_destroy and the exit handler release them first. unregister_model
// returns whether m was live.
void register_model(fa_model* m, fa_ctx* ctx);
bool unregister_model(fa_model* m);
// Releases every resource of a model (model.cpp); m must not be registered.
void model_release(fa_model* m);

// FA_ERR_STATE when stream s is being captured into a HIP graph: the entry
// points that grow buffers or upload per-call plans cannot be captured.
int refuse_capture(fa_ctx* ctx, hipStream_t s, const char* op);

// Copies host data into scratch slot `slot` (grown as needed) and returns
// the device pointer via *out.
int stage_h2d(fa_ctx* ctx, size_t slot, const void* src, size_t bytes, void** out);

// float64 RoPE angle tables rounded to float32, [T, D/2] each (tensor/rope.go:36-50).
void rope_tables_host(double base, const int32_t* positions, int T, int D, std::vector<float>& cs,
                      std::vector<float>& sn);

// ---- kernels (launchers) -----------------------------------------------------

enum class Epi { None = 0, Generic = 1, GeGLU = 2 };

struct GemmArgs {
  int64_t m = 0, n = 0, k = 0;
  const float* a = nullptr;
  int64_t lda = 0;
  const void* b = nullptr;  // bf16 or f32
  int64_t ldb = 0;
  int b_dtype = FA_DT_BF16;
  int b_layout = FA_B_NK;
  float* c = nullptr;
  int64_t ldc = 0;
  // Generic epilogue
  const float* bias = nullptr;
  const float* row_scale = nullptr;
  int act = FA_ACT_NONE;
  const float* mul = nullptr;
  int64_t ldm = 0;
  const float* residual = nullptr;
  int64_t ldr = 0;
  Epi epi = Epi::None;
  // ksplit > 1: the K range is split in ksplit equal parts computed by
  // separate workgroups; part s writes its partial product (no epilogue) to
  // c + s * c_split, and the consumer adds the parts in order s = 0, 1, ...
  int ksplit = 1;
  int64_t c_split = 0;
  // b_terms = 3: B (bf16, [n x k]) is three planes hi, mid, lo of fp32
  // values, b_plane elements apart (fp32 weights that are not bf16-exact)
  int b_terms = 1;
  int64_t b_plane = 0;
  // the launch runs beside other streams' kernels (the encoder's
  // micro-batches): the tile choice can count on them to fill the CUs its
  // own tiles leave idle
  bool shared = false;
  // nbatch > 1 (b_terms = 3 only, at most kMaxGridZ): entry z computes
  // C + z*c_bs = A + z*a_bs times the planes at B + z*b_bs (bf16 elements)
  int64_t nbatch = 1;
  int64_t a_bs = 0, b_bs = 0, c_bs = 0;
};

constexpr int kMaxGridZ = 65535;

// Batch dimensions of a strided operand (tensor.MatMul's broadcast, the
// reference's walkRows over broadcast strides, tensor/matmul.go:92-98):
// entry z (row-major over dim[0..nd-1]) starts at sum_d idx_d * stride[d].
struct BatchMap {
  int nd = 0;
  int dim[FA_MAX_BATCH_DIMS] = {};
  int64_t stride[FA_MAX_BATCH_DIMS] = {};
};
// A view [nb][m][k] (element (z, i, p) at src[off(z) + i*rs + p*cs]) ->
// contiguous fp32 [nb][m][kp] with columns k..kp-1 zero (kp % 4 == 0).
// Entries z0 .. z0 + nb - 1 of the view.
int launch_pack_a(fa_ctx* ctx, const float* src, const BatchMap& bm, int z0, int64_t rs, int64_t cs, int64_t nb,
                  int64_t m, int64_t k, int64_t kp, float* dst, hipStream_t s);
// B view, logical [k x n] per entry (element (z, p, j) at src[off(z) + p*rs +
// j*cs]) -> three bf16 planes hi, mid, lo [n][kp] per entry, entry z at
// planes + 3*(z - z0)*n*kp for entries z0 .. z0 + nb - 1, columns k..kp-1
// zero (kp % 8 == 0).
int launch_split_b_view(fa_ctx* ctx, const float* src, const BatchMap& bm, int z0, int64_t rs, int64_t cs,
                        int64_t nb, int64_t n, int64_t k, int64_t kp, uint16_t* planes, hipStream_t s);

// B [k x n] (FA_B_KN) or [n x k] (FA_B_NK), leading dimension ldb -> bf16
// planes [n][k] at planes (k % 8 == 0): fp32 B as three planes hi, mid, lo
// (GemmArgs.b_terms = 3), bf16 B transposed as one plane.
int launch_split_b(fa_ctx* ctx, const void* b, int b_dtype, int64_t ldb, int layout, int64_t n, int64_t k,
                   uint16_t* planes, hipStream_t s);

// Launches C = epi(A . B) on stream. For Epi::GeGLU, B is the interleaved
// gate/up weight [2F x K] (32-row groups alternating gate, up) and C is
// [m x F] = gelu(gate) * up.
int launch_gemm(fa_ctx* ctx, const GemmArgs& g, hipStream_t stream);

// FA_GEMM_MFMA=f32 (comparisons): every product on the fp32-MFMA kernel, bf16
// weights widened and float32 weights taken as they are (no three-plane
// rewrite).
bool gemm_f32_mfma_forced();

// K-split factor the encoder uses for its N = hidden products (o, down):
// FA_GEMM_KSPLIT=1 or 2 (default 2); 1 under FA_GEMM_MFMA=f32.
int gemm_ksplit();

int launch_row_sum_squares(fa_ctx* ctx, const float* x, int64_t m, int64_t n, float* out, hipStream_t s);
int launch_rmsnorm(fa_ctx* ctx, const float* x, const float* g, float eps, int64_t rows, int64_t n, float* out,
                   hipStream_t s);
int launch_rope(fa_ctx* ctx, const float* x, const float* cos_t, const float* sin_t, int64_t rows, int32_t T,
                int32_t D, float* out, hipStream_t s);

struct AttnGenericArgs {
  const float *q, *k, *v, *mask;
  int32_t B, H, T, S, D;
  int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, m_sb, m_sh, m_sr, m_sc;
  float scale;
  float* out;
};
int launch_attention_generic(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s);
// The MFMA kernel for head_dim 64/128/256/512 with 16-byte aligned q/k/v rows
// (base pointers and batch/head strides): whether it applies (FA_ATTN_DENSE=0
// turns it off, for comparisons), and its launch.
bool attention_dense_ok(const AttnGenericArgs& a);
int launch_attention_dense(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s);

// Per-row top-k of scores [nq x nd] (1 <= topk <= 32, nq <= 65535) into
// idx/val [nq x topk]; scratch holds topk_scratch_bytes(nq, nd, topk) bytes
// of per-chunk candidates.
int topk_scratch_bytes(int64_t nq, int64_t nd, int32_t topk);

// Fused similarities + top-k (score.hip): no score matrix. Needs
// score_fused_ok(); scratch holds score_scratch_bytes(d, nwg) bytes with
// nwg = score_workgroups(nd, cus) workgroups per query block; the exact top
// k (1 <= topk <= 16) by float32-rounded dot product into idx/val [nq x topk].
int score_workgroups(int64_t nd, int cus);
// Records the device address of the no-alloc entry point's fixed scratch
// array for ctx's device (current); once per device.
int noalloc_scratch_init(fa_ctx* ctx);
// Gives up ctx's claim on its device's no-alloc array (context release).
void noalloc_release(const fa_ctx* ctx);
size_t score_scratch_bytes(int d, int nwg);
bool score_fused_ok(const float* q, int64_t ldq, const float* docs, int64_t ldd, int d, int topk);
int launch_score_topk(fa_ctx* ctx, const float* q, int64_t nq, int64_t ldq, const float* docs, int64_t nd,
                      int64_t ldd, int d, int topk, int32_t* idx, float* val, void* scratch, int nwg,
                      hipStream_t s);
int launch_topk(fa_ctx* ctx, const float* scores, int64_t nq, int64_t nd, int32_t topk, int32_t* idx, float* val,
                void* scratch, hipStream_t s);

// ---- model-path kernels -------------------------------------------------------

// For packed row r of sequence b at position t (cu_seqlens[b] <= r <
// cu_seqlens[b+1], t = r - cu_seqlens[b]): row_src[r] = b*T + t, pos[r] = t.
int launch_row_plan(fa_ctx* ctx, const int32_t* cu_seqlens, int32_t nseq, int32_t T, int64_t rows, int32_t* row_src,
                    int32_t* pos, hipStream_t s);

// Embedding gather of packed tokens: x[r] = E[ids_packed[r]] * scale and
// xn[r] = x[r] * rms_inv(x[r]) * g (the first layer's input norm).
// E: bf16 [vocab x d], or with plane > 0 three planes hi, mid, lo plane
// elements apart (a float32 table that is not bf16-exact), summed exactly.
int launch_embed_gather(fa_ctx* ctx, const int32_t* d_ids, const int32_t* d_row_src, const uint16_t* E, int64_t plane,
                        int64_t vocab, int64_t rows, int32_t d, float scale, const float* g_next, float eps, float* x,
                        float* xn, hipStream_t s);

// q/k RMSNorm with (1+g) and RoPE on the packed qkv buffer [rows x (H+2*Hkv)*D],
// in place; positions from d_pos (null: row i is position i, the rows being one sequence).
// With norm_v, the Hkv value heads are RMS-normalised too (unit gain, no
// rotation). D is 256 or 512. qkv2 (optional): the second K part of a
// K-split q|k|v product (same layout), added to qkv first, values included.
int launch_qknorm_rope(fa_ctx* ctx, float* qkv, int64_t rows, int32_t H, int32_t Hkv, int32_t D, const float* gq,
                       const float* gk, float eps, const int32_t* d_pos, const float* cos_t, const float* sin_t,
                       hipStream_t s, bool norm_v = false, const float* qkv2 = nullptr);

// pl [rows, nl*P] in place: each P-wide piece becomes RMSNorm(pl * scale; g).
int launch_ple_norm(fa_ctx* ctx, float* pl, int64_t rows, int32_t nl, int32_t P, float scale, const float* g,
                    float eps, hipStream_t s);

// x = (x + RMSNorm(o; g_post)) * scale; then xn = RMSNorm(x; g_next)
// (g_next may be null: then xn is not written).
// o2 (optional): the other n2 (1..3) partial products of a K-split GEMM,
// planes pstride floats apart, added to o in part order.
int launch_residual_norm(fa_ctx* ctx, const float* o, float* x, float* xn, int64_t rows, int32_t d,
                         const float* g_post, const float* g_next, float eps, hipStream_t s,
                         const float* o2 = nullptr, float scale = 1.f, int n2 = 1, int64_t pstride = 0);

// Fused varlen attention over packed tokens. qkv [rows x (H+2Hkv)*D]; out
// [rows x H*D]; window: keys with |i-j| >= window are masked (window <= 0:
// none).
struct AttnVarlenArgs {
  const float* qkv;
  float* out;
  int32_t H, Hkv, D;
  int32_t window;
  float scale;
  int64_t row0 = 0;  // packed row held by qkv's and out's first row (items' sequences start at or after it)
  // per work item (16-byte aligned, required): the first packed row of the
  // item's sequence, its length, its first key tile, 0; read beside the item
  // (no dependent load through a sequence table before q and K/V)
  const int32_t* item_ext = nullptr;
  // kparts > 1 (at most kMaxKeyParts): every item's keys are cut into kparts
  // runs, one workgroup each, summed by a second pass; part holds
  // attention_part_floats(kparts, rows, H, D) floats and rows is the row
  // count of qkv and out (every row a query)
  int32_t kparts = 1;
  int64_t rows = 0;
  float* part = nullptr;
};
constexpr int kMaxKeyParts = 8;
inline int64_t attention_part_floats(int kparts, int64_t rows, int H, int D) {
  return (int64_t)kparts * rows * H * (D + 2);
}
// d_items holds n_items triples (sequence, first query, head): one work item
// per query block of attention_varlen_qblock() queries and head; a.item_ext
// its n_items extents.
int launch_attention_varlen_items(fa_ctx* ctx, const AttnVarlenArgs& a, const int32_t* d_items, int32_t n_items,
                                  hipStream_t s);
// Queries per workgroup of the varlen kernel (the item granularity).
int attention_varlen_qblock();
// head_dim 256, split-bf16 attention over key/value tile images: writes,
// for tiles [t_lo, t_lo + tiles), the key image (keys normed, gained,
// rotated) and value image of each (tile, kv head) into img
// [tile][Hkv][2][3*32*256] bf16. Every sequence starts a tile; tile tt
// holds up to 32 consecutive tokens of one sequence, described by
// d_tile_ext[4 tt ..] (16-byte aligned): its first token's packed row, its
// token count (1..32), its first token's position in the sequence (for
// RoPE), 0. qkv starts at packed row row0.
int launch_kv_tiles(fa_ctx* ctx, const float* qkv, int64_t row0, int32_t H, int32_t Hkv, const float* gk, float eps,
                    const float* cos_t, const float* sin_t, const int32_t* d_tile_ext, int32_t t_lo, int32_t tiles,
                    uint16_t* img, hipStream_t s, bool norm_v = false);

struct AttnTilesArgs {
  const float* qkv;       // raw q read here (rows of the launch start at packed row row0)
  const uint16_t* img;    // launch_kv_tiles's images
  float* out;
  const int32_t* item_ext = nullptr;  // as AttnVarlenArgs::item_ext (required)
  int32_t H, Hkv;
  int32_t window;
  float scale;
  int64_t row0 = 0;
  // kparts > 1: part holds attention_part_floats(kparts, rows, H, 256)
  // floats indexed by absolute packed row (rows: the batch's row count);
  // the launch's own rows are [row0, row0 + nrows)
  int32_t kparts = 1;
  int64_t rows = 0, nrows = 0;
  float* part = nullptr;
  // q's RMSNorm gain (1 + g), eps and RoPE tables [positions][128]: q is
  // normed and rotated as the kernel loads it
  const float* gq = nullptr;
  float eps = 0.f;
  const float *cos_t = nullptr, *sin_t = nullptr;
  // 16-row blocks per work item, 4 or 8 (64 or 128 rows; 64-row items run
  // on eight waves in head-dimension pairs unless FA_ATTN_PAIRS=0)
  int32_t waves = 8;
};
// d_items holds n_items triples (sequence, first row, kv head): one item per
// attention_tiles_rows(a.waves) rows (token, query head of the kv head's
// group), row r = token * (H / Hkv) + head - kv head * (H / Hkv).
int launch_attention_tiles(fa_ctx* ctx, const AttnTilesArgs& a, const int32_t* d_items, int32_t n_items,
                           hipStream_t s);
int attention_tiles_rows(int waves);
int attention_tiles_keys();

// Zeroes bytes (a multiple of 16, 16-byte aligned) with a fill kernel.
int launch_zero(fa_ctx* ctx, void* p, size_t bytes, hipStream_t s);

// Masked mean pooling of the final normed hidden states over each
// sequence's valid rows: pooled[b] = sum rows * (1/L_b).
int launch_pool(fa_ctx* ctx, const float* h, const int32_t* cu_seqlens, int32_t nseq, int32_t d, float* pooled,
                hipStream_t s);

// out[b, :dim] = y[b, :dim] / sqrt(sum y^2 + 1e-12), y the sum of `parts`
// partial products at y + p * pstride (added in part order)
int launch_l2norm(fa_ctx* ctx, const float* y, int32_t nseq, int32_t width, int32_t dim, float* out, hipStream_t s,
                  int32_t parts = 1, int64_t pstride = 0);

// Final RMSNorm with (1+g) of x rows into h.
int launch_final_norm(fa_ctx* ctx, const float* x, int64_t rows, int32_t d, const float* g, float eps, float* h,
                      hipStream_t s);

}  // namespace fa
