// Device-side math shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace fa {

// tanh as the reference computes it (internal/kernel/generic.go:313-359):
// identity below |x| < 4e-4, +-1 from |x| >= 9, otherwise an odd degree-13
// over even degree-6 rational after clamping to +-7.99881172180175781 (the
// published Eigen float approximation). The rational is evaluated for every
// input and the three cases are selects (they exclude each other), so the
// code has no branches: an epilogue holding many values per lane otherwise
// became one divergent branch region per value.
__device__ __forceinline__ float tanh_ref(float v) {
  const float c = fminf(fmaxf(v, -7.99881172180175781f), 7.99881172180175781f);
  const float v2 = c * c;
  float p = -2.76076847742355e-16f;
  p = fmaf(p, v2, 2.00018790482477e-13f);
  p = fmaf(p, v2, -8.60467152213735e-11f);
  p = fmaf(p, v2, 5.12229709037114e-08f);
  p = fmaf(p, v2, 1.48572235717979e-05f);
  p = fmaf(p, v2, 6.37261928875436e-04f);
  p = fmaf(p, v2, 4.89352455891786e-03f);
  p *= c;
  float q = 1.19825839466702e-06f;
  q = fmaf(q, v2, 1.18534705686654e-04f);
  q = fmaf(q, v2, 2.26843463243900e-03f);
  q = fmaf(q, v2, 4.89352518554385e-03f);
  // p / q from the hardware reciprocal: one Newton step on 1/q, then one
  // correction of the quotient (p - q r is exact in an fma). q lies in
  // [4.9e-3, 0.95] and |p| < q, so no scaling or special case applies, and
  // the result equals the correctly rounded quotient: checked on 2 million
  // points of the clamped range with the reciprocal off by up to one unit
  // in the last place either way. Six VALU instructions instead of the
  // general division's ten (v_div_scale, v_div_fmas, v_div_fixup).
  float rq = __builtin_amdgcn_rcpf(q);
  rq = fmaf(fmaf(-q, rq, 1.f), rq, rq);
  float r = p * rq;
  r = fmaf(fmaf(-q, r, p), rq, r);
  r = v >= 9.f ? 1.f : r;
  r = v <= -9.f ? -1.f : r;
  return (v > -0.0004f && v < 0.0004f) ? v : r;
}

// tanh-GELU, 0.5*x*(1 + tanh(sqrt(2/pi)*(x + 0.044715*x^3)))
// (internal/kernel/math.go:117-143).
__device__ __forceinline__ float gelu_tanh_ref(float x) {
  float u = x * x * x * 0.044715f + x;
  u *= 0.7978845608028654f;
  return (tanh_ref(u) + 1.f) * x * 0.5f;
}

// exp with the reference's flush: inputs below -87 give exactly 0
// (internal/kernel/generic.go:278-307), so masked softmax weights are exact
// zeros. Computed as 2^(x*log2 e) on the hardware exp2 (v_exp_f32) directly:
// every input that is not flushed maps to at least 2^-125.6, a normal
// float, where exp2f's guard for subnormal results (a range test, an offset
// and an ldexp around the same instruction) changes nothing.
__device__ __forceinline__ float exp_flush(float x) {
  return x < -87.f ? 0.f : __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// v of the lane 32 apart (lane ^ 32) by v_permlane32_swap, a VALU op: a
// swap of v with itself leaves the lane's own value in one result and the
// partner's in the other (the partner's is the second for lanes 0-31).
__device__ __forceinline__ float lane_xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 63) < 32 ? r[1] : r[0]);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wavefront (result in every lane): the xor
// butterfly over lane distances 32, 16, 8, 4, 2, 1, each step adding the
// partner's value to the lane's own, without an LDS round trip per step
// (ds_bpermute). 32 and 16: v_permlane32/16_swap (own and partner in the
// two results); 8, 4, 2, 1: DPP row rotations by 8, 4, 2, 1, which after
// the previous steps (the row's values repeat with period 2d) read exactly
// the xor-d partner. Same additions in the same order as a shuffle
// butterfly, so the same bits.
__device__ __forceinline__ float wave_sum(float v) {
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  v = v + dpp_f32<0x128>(v);  // row_ror:8
  v = v + dpp_f32<0x124>(v);  // row_ror:4
  v = v + dpp_f32<0x122>(v);  // row_ror:2
  v = v + dpp_f32<0x121>(v);  // row_ror:1
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// 1/sqrt(ss/n + eps) with the quotient in float32 and the square root and
// reciprocal in float64, rounded to float32 (models/gemma/embed.go:432-438,
// tensor/attention.go:328).
__device__ __forceinline__ float rms_inv(float ss, int n, float eps) {
  float t = ss / (float)n + eps;
  return (float)(1.0 / sqrt((double)t));
}

// Exact three-way bf16 split of an fp32 value: a = hi + mid + lo, hi is a
// with its low 16 bits cleared, mid the same of a - hi (exact in fp32),
// lo = a - hi - mid (at most 8 significant bits, so exact in bf16). The
// split-bf16 GEMM multiplies each term by a bf16 weight exactly and
// accumulates in fp32. Non-finite values do not survive the split
// (inf - inf).
struct Split3 {
  uint32_t h, m, l;  // fp32 bit patterns; the bf16 terms are the high halves
};

__device__ __forceinline__ Split3 split3(float a) {
  Split3 r;
  r.h = __float_as_uint(a) & 0xFFFF0000u;
  const float r1 = a - __uint_as_float(r.h);
  r.m = __float_as_uint(r1) & 0xFFFF0000u;
  r.l = __float_as_uint(r1 - __uint_as_float(r.m));
  return r;
}

// Two bf16 high halves packed as one dword, element `lo` first in memory.
__device__ __forceinline__ uint32_t pack_hi16(uint32_t lo, uint32_t hi) { return (lo >> 16) | (hi & 0xFFFF0000u); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Sum over the wave of the squares of a lane's NC float4 (a row of NC * 256
// values spread 4 per lane per 256), fixed order per lane then wave_sum.
template <int NC>
__device__ __forceinline__ float sumsq(const f32x4 (&v)[NC]) {
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    s = fmaf(v[c].x, v[c].x, s);
    s = fmaf(v[c].y, v[c].y, s);
    s = fmaf(v[c].z, v[c].z, s);
    s = fmaf(v[c].w, v[c].w, s);
  }
  return wave_sum(s);
}

// One row of the encoder's residual step, by one wave (lane: columns
// 256 c + 4 lane .. +3): x = (x + RMSNorm(o [+ parts]; g_post)) * scale,
// then xn = RMSNorm(x; g_next) when g_next != null (models/gemma/embed.go:
// 217-237). With o2 != null, a K-split product's other n2 partials sit at
// o2 + j * pstride (j < n2) and are added to o in part order.
template <int NC>
__device__ __forceinline__ void residual_norm_row(const float* __restrict__ o, const float* __restrict__ o2,
                                                  int n2, int64_t pstride,
                                                  float* __restrict__ x, float* __restrict__ xn, int64_t row,
                                                  const float* __restrict__ g_post, const float* __restrict__ g_next,
                                                  float eps, float scale, int lane) {
  constexpr int d = NC * 256;
  f32x4 ov[NC], xv[NC], gp[NC], gn[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int col = c * 256 + lane * 4;
    ov[c] = *reinterpret_cast<const f32x4*>(o + row * d + col);
    xv[c] = *reinterpret_cast<const f32x4*>(x + row * d + col);
  }
  // the gains load with the rows, not after the reductions
#pragma unroll
  for (int c = 0; c < NC; c++) gp[c] = *reinterpret_cast<const f32x4*>(g_post + c * 256 + lane * 4);
  if (g_next) {
#pragma unroll
    for (int c = 0; c < NC; c++) gn[c] = *reinterpret_cast<const f32x4*>(g_next + c * 256 + lane * 4);
  }
  // the other K parts, added in part order; up to kHeldParts of them all
  // loaded before the first sum (one round trip instead of one per part)
  constexpr int kHeldParts = 3;
  if (o2 && n2 <= kHeldParts) {
    f32x4 p2[kHeldParts][NC];
#pragma unroll
    for (int j = 0; j < kHeldParts; j++)
      if (j < n2) {
#pragma unroll
        for (int c = 0; c < NC; c++)
          p2[j][c] = *reinterpret_cast<const f32x4*>(o2 + j * pstride + row * d + c * 256 + lane * 4);
      }
#pragma unroll
    for (int j = 0; j < kHeldParts; j++)
      if (j < n2) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
          ov[c].x = ov[c].x + p2[j][c].x; ov[c].y = ov[c].y + p2[j][c].y;
          ov[c].z = ov[c].z + p2[j][c].z; ov[c].w = ov[c].w + p2[j][c].w;
        }
      }
  } else {
    for (int j = 0; o2 && j < n2; j++) {
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const f32x4 p2 = *reinterpret_cast<const f32x4*>(o2 + j * pstride + row * d + c * 256 + lane * 4);
        ov[c].x = ov[c].x + p2.x; ov[c].y = ov[c].y + p2.y; ov[c].z = ov[c].z + p2.z; ov[c].w = ov[c].w + p2.w;
      }
    }
  }
  const float inv = rms_inv(sumsq<NC>(ov), d, eps);
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int col = c * 256 + lane * 4;
    const f32x4 gg = gp[c];
    xv[c].x = xv[c].x + ov[c].x * inv * gg.x;
    xv[c].y = xv[c].y + ov[c].y * inv * gg.y;
    xv[c].z = xv[c].z + ov[c].z * inv * gg.z;
    xv[c].w = xv[c].w + ov[c].w * inv * gg.w;
    if (scale != 1.f) {
      xv[c].x = xv[c].x * scale; xv[c].y = xv[c].y * scale; xv[c].z = xv[c].z * scale; xv[c].w = xv[c].w * scale;
    }
    *reinterpret_cast<f32x4*>(x + row * d + col) = xv[c];
  }
  if (g_next == nullptr) return;
  const float inv2 = rms_inv(sumsq<NC>(xv), d, eps);
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int col = c * 256 + lane * 4;
    const f32x4 gg = gn[c];
    f32x4 r;
    r.x = xv[c].x * inv2 * gg.x; r.y = xv[c].y * inv2 * gg.y; r.z = xv[c].z * inv2 * gg.z; r.w = xv[c].w * inv2 * gg.w;
    *reinterpret_cast<f32x4*>(xn + row * d + col) = r;
  }
}

}  // namespace fa
