// Bandwidth-bound row kernels: one wavefront per row (or per head of a row),
// 16-byte coalesced loads, wavefront reductions, rows held in registers
// between the reduction and the write.
//
//   row_sum_squares  (*Tensor).RowSumSquares   tensor/matmul_fused.go:125-143
//   rmsnorm          tensor.RMSNorm             tensor/attention.go:292-337
//   rope             tensor.RoPE                tensor/rope.go:20-87
//   embed_gather     E.Rows(ids)*sqrt(d) + the first pre-norm   models/gemma/embed.go:175-176,193-194
//   qknorm_rope      RMSNorm(q|k; 1+g) then RoPE, in place      embed.go:198-207
//   residual_norm    x += RMSNorm(o; 1+g_post); xn = RMSNorm(x; 1+g_next)   embed.go:216-225,231-237
//   pool             masked mean                embed.go:381-404
//   l2norm           y/sqrt(sum y^2 + 1e-12)    embed.go:472-475

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---- RowSumSquares -----------------------------------------------------------
__global__ __launch_bounds__(256) void row_sum_squares_kernel(const float* __restrict__ x, int64_t m, int64_t n,
                                                              float* __restrict__ out) {
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= m) return;
  const float* r = x + row * n;
  float s = 0.f;
  for (int64_t i = lane; i < n; i += kWave) s = fmaf(r[i], r[i], s);
  s = wave_sum(s);
  if (lane == 0) out[row] = s;
}

// ---- RMSNorm (generic n) -----------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ g,
                                                      float eps, int64_t rows, int64_t n, float* __restrict__ out) {
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* r = x + row * n;
  float s = 0.f;
  for (int64_t i = lane; i < n; i += kWave) s = fmaf(r[i], r[i], s);
  s = wave_sum(s);
  const float inv = rms_inv(s, (int)n, eps);
  float* o = out + row * n;
  for (int64_t i = lane; i < n; i += kWave) o[i] = r[i] * inv * g[i];
}

// EmbeddingGemma 2's per-layer inputs (embed.go:274-279): pl [rows, nl*P]
// in place, each P-wide piece v = pl * s normalised as RMSNorm(v; g). One
// wave per (row, layer).
__global__ __launch_bounds__(256) void ple_norm_kernel(float* __restrict__ pl, int64_t pieces, int P, float sc,
                                                       const float* __restrict__ g, float eps) {
  const int64_t piece = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (piece >= pieces) return;
  float* r = pl + piece * P;
  float s = 0.f;
  for (int i = lane; i < P; i += kWave) {
    const float v = r[i] * sc;
    s = fmaf(v, v, s);
  }
  s = wave_sum(s);
  const float inv = rms_inv(s, P, eps);
  for (int i = lane; i < P; i += kWave) r[i] = r[i] * sc * inv * g[i];
}

// ---- RoPE (generic) -------------------------------------------------------------
// One thread per rotated pair (row, i < D/2); tables are [T, D/2].
__global__ __launch_bounds__(256) void rope_kernel(const float* __restrict__ x, const float* __restrict__ cs,
                                                   const float* __restrict__ sn, int64_t rows, int T, int D,
                                                   float* __restrict__ out) {
  const int half = D / 2;
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= rows * half) return;
  int64_t row = gid / half;
  int i = (int)(gid - row * half);
  int t = (int)(row % T);
  float c = cs[(int64_t)t * half + i], s = sn[(int64_t)t * half + i];
  const float* so = x + row * D;
  float x1 = so[i], x2 = so[i + half];
  out[row * D + i] = x1 * c - x2 * s;
  out[row * D + i + half] = x1 * s + x2 * c;
}

// ---- model-path kernels (hidden size a multiple of 256, at most 1024) -----------
// NC = hidden/256 float4 chunks per lane.


// x[r] = E[ids[src[r]]] * scale; xn[r] = x[r] * rms_inv(x[r]) * g.
template <int NC>
__global__ __launch_bounds__(256) void embed_gather_kernel(const int32_t* __restrict__ ids,
                                                           const int32_t* __restrict__ row_src,
                                                           const uint16_t* __restrict__ E, int64_t plane,
                                                           int64_t vocab, int64_t rows, float scale,
                                                           const float* __restrict__ g, float eps,
                                                           float* __restrict__ x, float* __restrict__ xn) {
  constexpr int d = NC * 256;
  int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  // ids on the device are not validated by the host: clamp so a bad id
  // cannot read outside the table
  const int64_t id = min(max((int64_t)ids[row_src[row]], (int64_t)0), vocab - 1);
  const uint16_t* e = E + id * d;
  f32x4 v[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    uint2 h = *reinterpret_cast<const uint2*>(e + c * 256 + lane * 4);
    v[c].x = __uint_as_float(h.x << 16);
    v[c].y = __uint_as_float(h.x & 0xFFFF0000u);
    v[c].z = __uint_as_float(h.y << 16);
    v[c].w = __uint_as_float(h.y & 0xFFFF0000u);
    if (plane) {  // + mid + lo: the float32 value exactly
#pragma unroll
      for (int t = 1; t < 3; t++) {
        h = *reinterpret_cast<const uint2*>(e + t * plane + c * 256 + lane * 4);
        v[c].x += __uint_as_float(h.x << 16);
        v[c].y += __uint_as_float(h.x & 0xFFFF0000u);
        v[c].z += __uint_as_float(h.y << 16);
        v[c].w += __uint_as_float(h.y & 0xFFFF0000u);
      }
    }
    v[c].x *= scale;
    v[c].y *= scale;
    v[c].z *= scale;
    v[c].w *= scale;
  }
  const float inv = rms_inv(sumsq<NC>(v), d, eps);
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int col = c * 256 + lane * 4;
    *reinterpret_cast<f32x4*>(x + row * d + col) = v[c];
    f32x4 gg = *reinterpret_cast<const f32x4*>(g + col);
    f32x4 o;
    o.x = v[c].x * inv * gg.x; o.y = v[c].y * inv * gg.y; o.z = v[c].z * inv * gg.z; o.w = v[c].w * inv * gg.w;
    *reinterpret_cast<f32x4*>(xn + row * d + col) = o;
  }
}

// x = (x + RMSNorm(o; g_post)) * scale; xn = RMSNorm(x; g_next) when
// g_next != null. With o2 != null, o is the sum of a K-split GEMM's
// partial products o + o2[0] + ... + o2[n2 - 1] (planes pstride apart, in
// that order). scale is EmbeddingGemma 2's layer scalar after its
// per-layer-input block (embed.go:367-370), else 1.
template <int NC>
__global__ __launch_bounds__(256) void residual_norm_kernel(const float* __restrict__ o, const float* __restrict__ o2,
                                                            int n2, int64_t pstride,
                                                            float* __restrict__ x, float* __restrict__ xn,
                                                            int64_t rows, const float* __restrict__ g_post,
                                                            const float* __restrict__ g_next, float eps,
                                                            float scale) {
  int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // one wave per row
  if (row >= rows) return;
  residual_norm_row<NC>(o, o2, n2, pstride, x, xn, row, g_post, g_next, eps, scale, threadIdx.x & 63);
}

// Per (token, head): RMSNorm over D (256 or 512) with the head's gain vector
// (the encoder's stored 1+w, or EmbeddingGemma 2's weight as is), then
// rotate-half RoPE at the token's position; with norm_v, the value heads get
// the same RMSNorm with a unit gain and no rotation (EmbeddingGemma 2's
// v_norm, models/gemma/model.go:189). One wavefront holds a head's values,
// 4 per lane per 256: at D=256 the rotation partner of element i (< 128) is
// i+128, held by lane+32; at D=512 the partner of i (< 256) is i+256, held
// by the same lane. Block = one token: waves 0..H-1 are the query heads,
// H..H+Hkv-1 the keys, then the values. With qkv2 != null the q|k|v product
// was split in K and qkv2 holds its second part (same layout): every head,
// the values included, is the sum qkv + qkv2 (in that order), written back
// to qkv (the values unnormed unless norm_v).
template <int D>
__global__ __launch_bounds__(256) void qknorm_rope_kernel(float* __restrict__ qkv, const float* __restrict__ qkv2,
                                                          int64_t rows, int H, int Hkv,
                                                          const float* __restrict__ gq, const float* __restrict__ gk,
                                                          float eps, const int32_t* __restrict__ pos,
                                                          const float* __restrict__ cs, const float* __restrict__ sn,
                                                          int norm_v) {
  constexpr int NQ = D / 256, half = D / 2;
  const int64_t row = blockIdx.x;
  const int head = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows || head >= H + Hkv + (norm_v || qkv2 ? Hkv : 0)) return;
  const int width = (H + 2 * Hkv) * D;
  float* p = qkv + row * width + (int64_t)head * D;
  // every load is issued before the reduction: the head's values, its gains
  // and the token's RoPE table row (one dependent step through pos, none
  // without it)
  f32x4 v[NQ], gg[NQ];
  const float* g = head < H ? gq : gk;
  const bool rot = head < H + Hkv;
#pragma unroll
  for (int c = 0; c < NQ; c++) v[c] = *reinterpret_cast<const f32x4*>(p + c * 256 + lane * 4);
  if (qkv2) {
    const float* p2 = qkv2 + row * width + (int64_t)head * D;
#pragma unroll
    for (int c = 0; c < NQ; c++) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(p2 + c * 256 + lane * 4);
      v[c].x = v[c].x + w.x; v[c].y = v[c].y + w.y; v[c].z = v[c].z + w.z; v[c].w = v[c].w + w.w;
    }
    if (!rot && !norm_v) {  // a value head: the sum only
#pragma unroll
      for (int c = 0; c < NQ; c++) *reinterpret_cast<f32x4*>(p + c * 256 + lane * 4) = v[c];
      return;
    }
  }
  if (rot) {
#pragma unroll
    for (int c = 0; c < NQ; c++) gg[c] = *reinterpret_cast<const f32x4*>(g + c * 256 + lane * 4);
  }
  const int t = pos ? pos[row] : (int)row;  // null: the rows are one sequence's tokens 0, 1, ...
  const int i0 = D == 256 ? (lane & 31) * 4 : lane * 4;
  f32x4 cv = {0.f, 0.f, 0.f, 0.f}, svv = {0.f, 0.f, 0.f, 0.f};
  if (rot) {
    cv = *reinterpret_cast<const f32x4*>(cs + (int64_t)t * half + i0);
    svv = *reinterpret_cast<const f32x4*>(sn + (int64_t)t * half + i0);
  }
  const float inv = rms_inv(sumsq<NQ>(v), D, eps);
  if (!rot) {  // value head: unit gain, no rotation
#pragma unroll
    for (int c = 0; c < NQ; c++) {
      f32x4 r;
      r.x = v[c].x * inv; r.y = v[c].y * inv; r.z = v[c].z * inv; r.w = v[c].w * inv;
      *reinterpret_cast<f32x4*>(p + c * 256 + lane * 4) = r;
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < NQ; c++) {
    v[c].x = v[c].x * inv * gg[c].x; v[c].y = v[c].y * inv * gg[c].y;
    v[c].z = v[c].z * inv * gg[c].z; v[c].w = v[c].w * inv * gg[c].w;
  }
  const f32x4 c = cv, sv = svv;
  if constexpr (D == 256) {
    f32x4 w;
    w.x = lane_xor32(v[0].x); w.y = lane_xor32(v[0].y);
    w.z = lane_xor32(v[0].z); w.w = lane_xor32(v[0].w);
    f32x4 r;
    if (lane < 32) {  // y_i = x_i c - x_{i+h} s
      r.x = v[0].x * c.x - w.x * sv.x; r.y = v[0].y * c.y - w.y * sv.y;
      r.z = v[0].z * c.z - w.z * sv.z; r.w = v[0].w * c.w - w.w * sv.w;
    } else {  // y_{i+h} = x_i s + x_{i+h} c
      r.x = w.x * sv.x + v[0].x * c.x; r.y = w.y * sv.y + v[0].y * c.y;
      r.z = w.z * sv.z + v[0].z * c.z; r.w = w.w * sv.w + v[0].w * c.w;
    }
    *reinterpret_cast<f32x4*>(p + lane * 4) = r;
  } else {
    const f32x4 x0 = v[0], x1 = v[1];
    f32x4 r0, r1;
    r0.x = x0.x * c.x - x1.x * sv.x; r0.y = x0.y * c.y - x1.y * sv.y;
    r0.z = x0.z * c.z - x1.z * sv.z; r0.w = x0.w * c.w - x1.w * sv.w;
    r1.x = x0.x * sv.x + x1.x * c.x; r1.y = x0.y * sv.y + x1.y * c.y;
    r1.z = x0.z * sv.z + x1.z * c.z; r1.w = x0.w * sv.w + x1.w * c.w;
    *reinterpret_cast<f32x4*>(p + lane * 4) = r0;
    *reinterpret_cast<f32x4*>(p + 256 + lane * 4) = r1;
  }
}

// pooled[b, c] = (sum over the sequence's rows of h[., c]) * (1/L_b). One
// workgroup of 16 waves per (sequence, 256 columns): wave w adds rows w, w +
// 16, ... in order (lane: four columns, 16-byte loads, eight rows in
// flight), then the 16 wave sums are added in wave order, so the result does
// not depend on scheduling.
__global__ __launch_bounds__(1024) void pool_kernel(const float* __restrict__ h, const int32_t* __restrict__ cu,
                                                    int d, float* __restrict__ pooled) {
  __shared__ f32x4 part[16][64];
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.y * 256 + lane * 4;
  const int r0 = cu[b], r1 = cu[b + 1];
  f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
  int r = r0 + w;
  for (; r + 112 < r1; r += 128) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const f32x4*>(h + (int64_t)(r + 16 * u) * d + c);
#pragma unroll
    for (int u = 0; u < 8; u++) s += v[u];
  }
  for (; r < r1; r += 16) s += *reinterpret_cast<const f32x4*>(h + (int64_t)r * d + c);
  part[w][lane] = s;
  __syncthreads();
  if (w == 0) {
    f32x4 tot = part[0][lane];
#pragma unroll
    for (int i = 1; i < 16; i++) tot += part[i][lane];
    const int n = r1 - r0 > 0 ? r1 - r0 : 1;
    *reinterpret_cast<f32x4*>(pooled + (int64_t)b * d + c) = tot * (1.f / (float)n);
  }
}

// Key and value images of head_dim-256 layers for attention_tiles_kernel,
// one block per (tile of 32 tokens of one sequence, kv head): tile tt of
// sequence b (cut[b] <= tt < cut[b+1]) holds tokens 32 (tt - cut[b]) .. +31.
// Image pair [tt][kv head][key image | value image], 3 * 32 * 256 bf16 each:
//   key image [term][key][256]: the normed, gained and rotated key's exact
//   split terms, the 16-byte chunk c (dims 8c .. 8c+7) of key k at
//   position c ^ k (the 16 keys of one operand read hit distinct banks);
//   value image [term][dim][32 slots]: slot 8g + 4h + r holds key 16h + 4g +
//   r (the order in which the attention's probabilities meet the values),
//   the 16-byte chunk g of dim d at position g ^ ((d >> 1) & 3).
// Tokens past the sequence are zeros. With norm_v the values are first
// RMS-normed over their 256 dims with unit gain (models/gemma/gemma2.go;
// as qknorm_rope_kernel's value heads).
struct KvTilesParams {
  const float* qkv;
  int64_t row0;
  int H, Hkv;
  const float* gk;
  float eps;
  const float *cs, *sn;
  const int32_t* tile_ext;  // per tile (first packed row, keys, first key's position, 0)
  int t_lo, tiles;
  uint16_t* img;
  int norm_v;  // values RMS-normed with unit gain first (EmbeddingGemma 2, gemma2.go)
};

constexpr int kTileImg = 3 * 32 * 256;  // bf16 per key or value image
// floats per LDS row of the value transpose (128 dims): the column reads of
// one wave (16 consecutive dims x keys 4c + const, c = 0..3) land on banks
// 16c + dim mod 64, all distinct, since 4 * 132 = 16 (mod 64)
constexpr int kVtStride = 132;

// Keys 4 KPW part .. + 4 KPW - 1 of the key image of (tile, hk): wave w
// takes keys 4 KPW part + w, + 4, ... (KPW of them), 4 dims per lane; rows
// past the sequence are clamped to its last token (every load issued up
// front, none conditional) and written as zeros.
// The tile's first qkv row, its first key's position and its key count.
__device__ __forceinline__ void tile_extent(const KvTilesParams& a, int tile, int64_t& r_first, int& t0, int& n) {
  const int4 e = reinterpret_cast<const int4*>(a.tile_ext)[tile];
  r_first = e.x - a.row0;
  n = e.y;
  t0 = e.z;
}

template <int KPW>
__device__ __forceinline__ void key_tile(const KvTilesParams& a, int tile, int hk, int part, int wave, int lane) {
  constexpr int D = 256, half = D / 2;
  const int kb = 4 * KPW * part;
  int64_t r_first;  // qkv row of the tile's first token
  int t0, n;
  tile_extent(a, tile, r_first, t0, n);
  const int width = (a.H + 2 * a.Hkv) * D;
  uint16_t* kimg = a.img + ((int64_t)tile * a.Hkv + hk) * (2 * kTileImg);
  const f32x4 gg = *reinterpret_cast<const f32x4*>(a.gk + lane * 4);
  const int i0 = (lane & 31) * 4;
  f32x4 v[KPW], c[KPW], sv[KPW];
#pragma unroll
  for (int j = 0; j < KPW; j++) {
    const int64_t row = r_first + min(kb + wave + 4 * j, n - 1);
    v[j] = *reinterpret_cast<const f32x4*>(a.qkv + row * width + (int64_t)(a.H + hk) * D + lane * 4);
    const int t = t0 + min(kb + wave + 4 * j, n - 1);  // the key's position in its sequence
    c[j] = *reinterpret_cast<const f32x4*>(a.cs + (int64_t)t * half + i0);
    sv[j] = *reinterpret_cast<const f32x4*>(a.sn + (int64_t)t * half + i0);
  }
#pragma unroll
  for (int j = 0; j < KPW; j++) {
    const int k = kb + wave + 4 * j;
    f32x4 x[1] = {v[j]};
    const float inv = rms_inv(sumsq<1>(x), D, a.eps);
    x[0].x = x[0].x * inv * gg.x; x[0].y = x[0].y * inv * gg.y;
    x[0].z = x[0].z * inv * gg.z; x[0].w = x[0].w * inv * gg.w;
    f32x4 o;
    o.x = lane_xor32(x[0].x); o.y = lane_xor32(x[0].y);
    o.z = lane_xor32(x[0].z); o.w = lane_xor32(x[0].w);
    f32x4 r;
    if (lane < 32) {  // y_i = x_i c - x_{i+h} s
      r.x = x[0].x * c[j].x - o.x * sv[j].x; r.y = x[0].y * c[j].y - o.y * sv[j].y;
      r.z = x[0].z * c[j].z - o.z * sv[j].z; r.w = x[0].w * c[j].w - o.w * sv[j].w;
    } else {  // y_{i+h} = x_i s + x_{i+h} c
      r.x = o.x * sv[j].x + x[0].x * c[j].x; r.y = o.y * sv[j].y + x[0].y * c[j].y;
      r.z = o.z * sv[j].z + x[0].z * c[j].z; r.w = o.w * sv[j].w + x[0].w * c[j].w;
    }
    if (k >= n) r = f32x4{0.f, 0.f, 0.f, 0.f};
    uint32_t th[4], tm[4], tl[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const Split3 sp = split3(r[e]);
      th[e] = sp.h;
      tm[e] = sp.m;
      tl[e] = sp.l;
    }
    uint16_t* o16 = kimg + k * D + (((lane >> 1) ^ k) * 8) + (lane & 1) * 4;
    *reinterpret_cast<uint2*>(o16) = make_uint2(pack_hi16(th[0], th[1]), pack_hi16(th[2], th[3]));
    *reinterpret_cast<uint2*>(o16 + 32 * D) = make_uint2(pack_hi16(tm[0], tm[1]), pack_hi16(tm[2], tm[3]));
    *reinterpret_cast<uint2*>(o16 + 64 * D) = make_uint2(pack_hi16(tl[0], tl[1]), pack_hi16(tl[2], tl[3]));
  }
}

// Dims 128*half .. 128*half + 127 of the value image of (tile, hk): rows
// into LDS (clamped loads, zeros past the sequence), then transposed, 16
// bytes (8 slots of one dim and term) per store.
__device__ __forceinline__ void value_tile(const KvTilesParams& a, int tile, int hk, int half_, int wave, int lane,
                                           float (*Vt)[kVtStride]) {
  constexpr int D = 256;
  int64_t r_first;
  int t0, n;
  tile_extent(a, tile, r_first, t0, n);
  const int width = (a.H + 2 * a.Hkv) * D;
  uint16_t* vimg = a.img + ((int64_t)tile * a.Hkv + hk) * (2 * kTileImg) + kTileImg;
  float2 v[8];
  const float* vsrc = a.qkv + (int64_t)(a.H + a.Hkv + hk) * D + lane * 2;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int64_t row = r_first + min(wave + 4 * j, n - 1);
    v[j] = *reinterpret_cast<const float2*>(vsrc + row * width + 128 * half_);
  }
  if (a.norm_v) {
    // the key's sum of squares over all 256 dims: this half's two per lane
    // and the other half's, then the wave's sum (one key per j)
    float2 w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int64_t row = r_first + min(wave + 4 * j, n - 1);
      w[j] = *reinterpret_cast<const float2*>(vsrc + row * width + 128 * (1 - half_));
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float2 lo = half_ ? w[j] : v[j], hi = half_ ? v[j] : w[j];  // dims 2l, 2l+1 and 128 + 2l, 128 + 2l + 1
      const float ss = wave_sum(fmaf(hi.y, hi.y, fmaf(hi.x, hi.x, fmaf(lo.y, lo.y, lo.x * lo.x))));
      const float inv = rms_inv(ss, D, a.eps);
      v[j].x *= inv;
      v[j].y *= inv;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int k = wave + 4 * j;
    *reinterpret_cast<float2*>(&Vt[k][lane * 2]) = k < n ? v[j] : make_float2(0.f, 0.f);
  }
  __syncthreads();
  const int tid = wave * 64 + lane;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int u = tid + 256 * i;
    const int dl = u >> 2, c = u & 3;  // local dim, chunk of 8 slots: keys 4c .. 4c+3, 16 + 4c .. 16 + 4c+3
    const int d = 128 * half_ + dl;
    uint32_t th[8], tm[8], tl[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const Split3 sp = split3(Vt[(e >> 2) * 16 + 4 * c + (e & 3)][dl]);
      th[e] = sp.h;
      tm[e] = sp.m;
      tl[e] = sp.l;
    }
    uint16_t* o = vimg + d * 32 + ((c ^ ((d >> 1) & 3)) * 8);
    *reinterpret_cast<uint4*>(o) = make_uint4(pack_hi16(th[0], th[1]), pack_hi16(th[2], th[3]),
                                              pack_hi16(th[4], th[5]), pack_hi16(th[6], th[7]));
    *reinterpret_cast<uint4*>(o + 32 * D) = make_uint4(pack_hi16(tm[0], tm[1]), pack_hi16(tm[2], tm[3]),
                                                       pack_hi16(tm[4], tm[5]), pack_hi16(tm[6], tm[7]));
    *reinterpret_cast<uint4*>(o + 64 * D) = make_uint4(pack_hi16(tl[0], tl[1]), pack_hi16(tl[2], tl[3]),
                                                       pack_hi16(tl[4], tl[5]), pack_hi16(tl[6], tl[7]));
  }
}

// Dims 64 q .. 64 q + 63 of the value image of (tile, hk) (values not
// normed): lane l loads dims 2 (l mod 32), + 1 of keys w + 4 (2 j + l / 32)
// into LDS, then each thread transposes, splits and stores one 16-byte
// chunk (8 slots of one dim and term), as value_tile does for 128 dims.
__device__ __forceinline__ void value_quarter(const KvTilesParams& a, int tile, int hk, int q, int wave, int lane,
                                              float (*Vt)[kVtStride]) {
  constexpr int D = 256;
  int64_t r_first;
  int t0, n;
  tile_extent(a, tile, r_first, t0, n);
  const int width = (a.H + 2 * a.Hkv) * D;
  uint16_t* vimg = a.img + ((int64_t)tile * a.Hkv + hk) * (2 * kTileImg) + kTileImg;
  const float* vsrc = a.qkv + (int64_t)(a.H + a.Hkv + hk) * D + 64 * q + (lane & 31) * 2;
  float2 v[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int64_t row = r_first + min(wave + 4 * (2 * j + (lane >> 5)), n - 1);
    v[j] = *reinterpret_cast<const float2*>(vsrc + row * width);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int k = wave + 4 * (2 * j + (lane >> 5));
    *reinterpret_cast<float2*>(&Vt[k][(lane & 31) * 2]) = k < n ? v[j] : make_float2(0.f, 0.f);
  }
  __syncthreads();
  const int u = wave * 64 + lane;
  const int dl = u >> 2, c = u & 3;  // local dim, chunk of 8 slots: keys 4c .. 4c+3, 16 + 4c .. 16 + 4c+3
  const int d = 64 * q + dl;
  uint32_t th[8], tm[8], tl[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const Split3 sp = split3(Vt[(e >> 2) * 16 + 4 * c + (e & 3)][dl]);
    th[e] = sp.h;
    tm[e] = sp.m;
    tl[e] = sp.l;
  }
  uint16_t* o = vimg + d * 32 + ((c ^ ((d >> 1) & 3)) * 8);
  *reinterpret_cast<uint4*>(o) = make_uint4(pack_hi16(th[0], th[1]), pack_hi16(th[2], th[3]),
                                            pack_hi16(th[4], th[5]), pack_hi16(th[6], th[7]));
  *reinterpret_cast<uint4*>(o + 32 * D) = make_uint4(pack_hi16(tm[0], tm[1]), pack_hi16(tm[2], tm[3]),
                                                     pack_hi16(tm[4], tm[5]), pack_hi16(tm[6], tm[7]));
  *reinterpret_cast<uint4*>(o + 64 * D) = make_uint4(pack_hi16(tl[0], tl[1]), pack_hi16(tl[2], tl[3]),
                                                     pack_hi16(tl[4], tl[5]), pack_hi16(tl[6], tl[7]));
}

// QUARTERS (values not normed): blocks 8i + j of (tile t_lo + i / Hkv, kv
// head i % Hkv), j = 0..3 the key image's quarters of 8 keys, 4..7 the
// value image's quarters of 64 dims. Else (values RMS-normed, each block
// needing all of a key's dims) blocks 4i + j, j = 0, 1 the key image's
// halves of 16 keys, 2, 3 the value image's halves of 128 dims. Smaller
// blocks: more of a launch's loads in flight, a shorter serial chain per
// block.
template <bool QUARTERS>
__global__ __launch_bounds__(256) void kv_tiles_kernel(KvTilesParams a) {
  __shared__ __attribute__((aligned(16))) float Vt[32][kVtStride];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t b = blockIdx.x;
  constexpr int P = QUARTERS ? 8 : 4;  // blocks per (tile, kv head)
  const int tile = a.t_lo + (int)(b / (P * a.Hkv)), hk = (int)((b / P) % a.Hkv);
  const int part = (int)(b % P);
  if constexpr (QUARTERS) {
    if (part >= 4)
      value_quarter(a, tile, hk, part - 4, wave, lane, Vt);
    else
      key_tile<2>(a, tile, hk, part, wave, lane);
  } else {
    if (part >= 2)
      value_tile(a, tile, hk, part - 2, wave, lane, Vt);
    else
      key_tile<4>(a, tile, hk, part, wave, lane);
  }
}

__global__ __launch_bounds__(256) void zero_kernel(uint4* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// out[b, :dim] = y[b, :dim] / sqrt(sum(y[b, :dim]^2) + 1e-12), one wave per
// row; y = the sum of `parts` partial products y_p = y + p * pstride (K-split
// head product), added in part order.
__global__ __launch_bounds__(256) void l2norm_kernel(const float* __restrict__ y, int nseq, int width, int dim,
                                                     int parts, int64_t pstride, float* __restrict__ out) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= nseq) return;
  const float* r = y + (int64_t)b * width;
  auto value = [&](int i) {
    float v = r[i];
    for (int p = 1; p < parts; p++) v += r[p * pstride + i];
    return v;
  };
  constexpr int kHeld = 16;      // values per lane kept in registers (dim <= 1 024)
  constexpr int kHeldParts = 4;  // partial products loaded together (the head's K parts)
  float s = 0.f;
  if (dim <= kWave * kHeld && parts <= kHeldParts) {
    // every part's values loaded before the first sum (one round trip
    // instead of one per part and value), then added in part order
    float w[kHeldParts][kHeld];
#pragma unroll
    for (int p = 0; p < kHeldParts; p++)
#pragma unroll
      for (int t = 0; t < kHeld; t++) {
        const int i = lane + kWave * t;
        w[p][t] = (p < parts && i < dim) ? r[p * pstride + i] : 0.f;
      }
    float v[kHeld];
#pragma unroll
    for (int t = 0; t < kHeld; t++) {
      v[t] = w[0][t];
#pragma unroll
      for (int p = 1; p < kHeldParts; p++)
        if (p < parts) v[t] += w[p][t];
    }
#pragma unroll
    for (int t = 0; t < kHeld; t++) s = fmaf(v[t], v[t], s);
    s = wave_sum(s);
    const float nrm = sqrtf(s + 1e-12f);
#pragma unroll
    for (int t = 0; t < kHeld; t++) {
      const int i = lane + kWave * t;
      if (i < dim) out[(int64_t)b * dim + i] = v[t] / nrm;
    }
    return;
  }
  for (int i = lane; i < dim; i += kWave) {
    const float v = value(i);
    s = fmaf(v, v, s);
  }
  s = wave_sum(s);
  const float nrm = sqrtf(s + 1e-12f);
  for (int i = lane; i < dim; i += kWave) out[(int64_t)b * dim + i] = value(i) / nrm;
}

__global__ __launch_bounds__(256) void row_plan_kernel(const int32_t* __restrict__ cu, int nseq, int T, int64_t rows,
                                                       int32_t* __restrict__ row_src, int32_t* __restrict__ pos) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  int lo = 0, hi = nseq;  // cu[lo] <= r < cu[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu[mid] <= r) lo = mid; else hi = mid;
  }
  const int t = (int)(r - cu[lo]);
  row_src[r] = lo * T + t;
  pos[r] = t;
}

int blocks_for(int64_t rows, int per) { return (int)((rows + per - 1) / per); }

}  // namespace

int launch_row_plan(fa_ctx* ctx, const int32_t* cu_seqlens, int32_t nseq, int32_t T, int64_t rows, int32_t* row_src,
                    int32_t* pos, hipStream_t s) {
  if (rows == 0) return FA_OK;
  hipLaunchKernelGGL(row_plan_kernel, dim3(blocks_for(rows, 256)), dim3(256), 0, s, cu_seqlens, nseq, T, rows, row_src,
                     pos);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_row_sum_squares(fa_ctx* ctx, const float* x, int64_t m, int64_t n, float* out, hipStream_t s) {
  if (m == 0) return FA_OK;
  hipLaunchKernelGGL(row_sum_squares_kernel, dim3(blocks_for(m, 4)), dim3(256), 0, s, x, m, n, out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_rmsnorm(fa_ctx* ctx, const float* x, const float* g, float eps, int64_t rows, int64_t n, float* out,
                   hipStream_t s) {
  if (rows == 0 || n == 0) return FA_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, s, x, g, eps, rows, n, out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_ple_norm(fa_ctx* ctx, float* pl, int64_t rows, int32_t nl, int32_t P, float scale, const float* g,
                    float eps, hipStream_t s) {
  const int64_t pieces = rows * nl;
  if (pieces == 0 || P == 0) return FA_OK;
  hipLaunchKernelGGL(ple_norm_kernel, dim3(blocks_for(pieces, 4)), dim3(256), 0, s, pl, pieces, P, scale, g, eps);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_rope(fa_ctx* ctx, const float* x, const float* cos_t, const float* sin_t, int64_t rows, int32_t T,
                int32_t D, float* out, hipStream_t s) {
  int64_t work = rows * (D / 2);
  if (work == 0) return FA_OK;
  hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(work, 256)), dim3(256), 0, s, x, cos_t, sin_t, rows, T, D, out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_embed_gather(fa_ctx* ctx, const int32_t* d_ids, const int32_t* d_row_src, const uint16_t* E, int64_t plane,
                        int64_t vocab, int64_t rows, int32_t d, float scale, const float* g_next, float eps, float* x,
                        float* xn, hipStream_t s) {
  if (rows == 0) return FA_OK;
  dim3 grid(blocks_for(rows, 4)), block(256);
  switch (d) {
    case 256: hipLaunchKernelGGL(embed_gather_kernel<1>, grid, block, 0, s, d_ids, d_row_src, E, plane, vocab, rows, scale, g_next, eps, x, xn); break;
    case 512: hipLaunchKernelGGL(embed_gather_kernel<2>, grid, block, 0, s, d_ids, d_row_src, E, plane, vocab, rows, scale, g_next, eps, x, xn); break;
    case 768: hipLaunchKernelGGL(embed_gather_kernel<3>, grid, block, 0, s, d_ids, d_row_src, E, plane, vocab, rows, scale, g_next, eps, x, xn); break;
    case 1024: hipLaunchKernelGGL(embed_gather_kernel<4>, grid, block, 0, s, d_ids, d_row_src, E, plane, vocab, rows, scale, g_next, eps, x, xn); break;
    default: return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: hidden size %d not in {256,512,768,1024}", d);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_residual_norm(fa_ctx* ctx, const float* o, float* x, float* xn, int64_t rows, int32_t d,
                         const float* g_post, const float* g_next, float eps, hipStream_t s, const float* o2,
                         float scale, int n2, int64_t pstride) {
  if (rows == 0) return FA_OK;
  if (o2 && (n2 < 1 || n2 > 3)) return set_error(ctx, FA_ERR_ARG, "residual norm: %d extra K parts (1..3)", n2);
  // a short batch (C1: 128 rows) takes one row per workgroup, spread over
  // four times the CUs: every launch of this chain of small kernels is
  // latency, 1 % of C1's forward; from four rows per CU on, four per
  // workgroup
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  const int per = rows <= 4LL * cus ? 1 : 4;
  dim3 grid(blocks_for(rows, per)), block(64 * per);
  switch (d) {
    case 256: hipLaunchKernelGGL(residual_norm_kernel<1>, grid, block, 0, s, o, o2, n2, pstride, x, xn, rows, g_post, g_next, eps, scale); break;
    case 512: hipLaunchKernelGGL(residual_norm_kernel<2>, grid, block, 0, s, o, o2, n2, pstride, x, xn, rows, g_post, g_next, eps, scale); break;
    case 768: hipLaunchKernelGGL(residual_norm_kernel<3>, grid, block, 0, s, o, o2, n2, pstride, x, xn, rows, g_post, g_next, eps, scale); break;
    case 1024: hipLaunchKernelGGL(residual_norm_kernel<4>, grid, block, 0, s, o, o2, n2, pstride, x, xn, rows, g_post, g_next, eps, scale); break;
    default: return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: hidden size %d not in {256,512,768,1024}", d);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_qknorm_rope(fa_ctx* ctx, float* qkv, int64_t rows, int32_t H, int32_t Hkv, int32_t D, const float* gq,
                       const float* gk, float eps, const int32_t* d_pos, const float* cos_t, const float* sin_t,
                       hipStream_t s, bool norm_v, const float* qkv2) {
  if (D != 256 && D != 512) return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: head_dim %d not 256 or 512", D);
  if (rows == 0) return FA_OK;
  const int heads = H + Hkv + (norm_v || qkv2 ? Hkv : 0);
  dim3 grid((unsigned)rows, (unsigned)((heads + 3) / 4)), block(256);
  if (D == 256)
    hipLaunchKernelGGL(qknorm_rope_kernel<256>, grid, block, 0, s, qkv, qkv2, rows, H, Hkv, gq, gk, eps, d_pos,
                       cos_t, sin_t, norm_v ? 1 : 0);
  else
    hipLaunchKernelGGL(qknorm_rope_kernel<512>, grid, block, 0, s, qkv, qkv2, rows, H, Hkv, gq, gk, eps, d_pos,
                       cos_t, sin_t, norm_v ? 1 : 0);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_pool(fa_ctx* ctx, const float* h, const int32_t* cu_seqlens, int32_t nseq, int32_t d, float* pooled,
                hipStream_t s) {
  if (nseq == 0) return FA_OK;
  if (d % 256 != 0) return set_error(ctx, FA_ERR_UNSUPPORTED, "pool: width %d not a multiple of 256", d);
  dim3 grid(nseq, d / 256), block(1024);
  hipLaunchKernelGGL(pool_kernel, grid, block, 0, s, h, cu_seqlens, d, pooled);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_l2norm(fa_ctx* ctx, const float* y, int32_t nseq, int32_t width, int32_t dim, float* out, hipStream_t s,
                  int32_t parts, int64_t pstride) {
  if (nseq == 0) return FA_OK;
  if (parts < 1) return set_error(ctx, FA_ERR_ARG, "l2norm: %d parts", parts);
  hipLaunchKernelGGL(l2norm_kernel, dim3(blocks_for(nseq, 4)), dim3(256), 0, s, y, nseq, width, dim, parts, pstride,
                     out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_kv_tiles(fa_ctx* ctx, const float* qkv, int64_t row0, int32_t H, int32_t Hkv, const float* gk, float eps,
                    const float* cos_t, const float* sin_t, const int32_t* d_tile_ext, int32_t t_lo, int32_t tiles,
                    uint16_t* img, hipStream_t s, bool norm_v) {
  if (tiles == 0) return FA_OK;
  if (!d_tile_ext) return set_error(ctx, FA_ERR_ARG, "key/value tiles: no tile extents");
  KvTilesParams a;
  a.qkv = qkv; a.row0 = row0; a.H = H; a.Hkv = Hkv; a.gk = gk; a.eps = eps; a.cs = cos_t; a.sn = sin_t;
  a.tile_ext = d_tile_ext; a.t_lo = t_lo; a.tiles = tiles; a.img = img;
  a.norm_v = norm_v ? 1 : 0;
  if (norm_v)
    hipLaunchKernelGGL(kv_tiles_kernel<false>, dim3((unsigned)(4 * (int64_t)tiles * Hkv)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(kv_tiles_kernel<true>, dim3((unsigned)(8 * (int64_t)tiles * Hkv)), dim3(256), 0, s, a);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_zero(fa_ctx* ctx, void* p, size_t bytes, hipStream_t s) {
  if (bytes == 0) return FA_OK;
  if ((bytes & 15) || (reinterpret_cast<uintptr_t>(p) & 15))
    return set_error(ctx, FA_ERR_ARG, "zero: %zu bytes at %p not 16-byte aligned", bytes, p);
  const int64_t n = (int64_t)(bytes / 16);
  hipLaunchKernelGGL(zero_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, static_cast<uint4*>(p), n);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_final_norm(fa_ctx* ctx, const float* x, int64_t rows, int32_t d, const float* g, float eps, float* h,
                      hipStream_t s) {
  return launch_rmsnorm(ctx, x, g, eps, rows, d, h, s);
}

}  // namespace fa
