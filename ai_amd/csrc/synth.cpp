// Seeded synthetic inputs (weights, token ids, corpus) for the EmbeddingGemma
// path. Host-only. Declared in include/fa_synth.h.
#include "fa_synth.h"

#include <cmath>
#include <cstring>
#include <vector>
#include <algorithm>

namespace {

constexpr int64_t kChunk = int64_t(1) << 20;

inline uint64_t splitmix64(uint64_t& x) {
  uint64_t z = (x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t fnv1a(const char* s) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (; *s; ++s) {
    h ^= (uint8_t)*s;
    h *= 0x100000001B3ull;
  }
  return h;
}

struct Xoshiro {
  uint64_t s[4];
  Xoshiro(uint64_t seed, const char* name, uint64_t chunk) {
    uint64_t x = seed ^ (fnv1a(name) * 0x9E3779B97F4A7C15ull) ^ (chunk * 0xD1B54A32D192ED03ull);
    for (auto& v : s) v = splitmix64(x);
  }
  static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
  inline uint64_t next() {
    uint64_t r = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return r;
  }
  // uniform in [0, 1) with 53 bits
  inline double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
};

inline uint16_t bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

// Fill n normals of one stream chunk.
template <typename F>
void normals(uint64_t seed, const char* name, int64_t n, F&& put) {
  int64_t nchunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t c = 0; c < nchunks; c++) {
    Xoshiro g(seed, name, (uint64_t)c);
    int64_t i0 = c * kChunk, i1 = std::min(n, i0 + kChunk);
    for (int64_t i = i0; i < i1; i += 2) {
      double u1 = 1.0 - g.uniform();  // (0, 1]
      double u2 = g.uniform();
      double r = std::sqrt(-2.0 * std::log(u1));
      double a = 6.283185307179586 * u2;
      put(i, r * std::cos(a));
      if (i + 1 < i1) put(i + 1, r * std::sin(a));
    }
  }
}

}  // namespace

extern "C" {

void fa_synth_normal_bf16(uint64_t seed, const char* name, double std, int64_t n, uint16_t* out) {
  normals(seed, name, n, [&](int64_t i, double z) { out[i] = bf16_rne((float)(z * std)); });
}

void fa_synth_normal_f32(uint64_t seed, const char* name, double std, int64_t n, float* out) {
  normals(seed, name, n, [&](int64_t i, double z) { out[i] = (float)(z * std); });
}

void fa_bf16_to_f32(const uint16_t* in, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) {
    uint32_t u = (uint32_t)in[i] << 16;
    std::memcpy(&out[i], &u, 4);
  }
}

void fa_f32_to_bf16(const float* in, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) out[i] = bf16_rne(in[i]);
}

void fa_synth_uniform_i32(uint64_t seed, const char* name, int32_t lo, int32_t hi, int64_t n, int32_t* out) {
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo);
  if (span == 0) {
    for (int64_t i = 0; i < n; i++) out[i] = lo;
    return;
  }
  int64_t nchunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t c = 0; c < nchunks; c++) {
    Xoshiro g(seed, name, (uint64_t)c);
    int64_t i0 = c * kChunk, i1 = std::min(n, i0 + kChunk);
    for (int64_t i = i0; i < i1; i++) {
      // multiply-shift range reduction (Lemire), bias < 2^-32 for spans < 2^32
      unsigned __int128 p = (unsigned __int128)g.next() * span;
      out[i] = lo + (int32_t)(uint64_t)(p >> 64);
    }
  }
}

int fa_synth_zipf_i32(uint64_t seed, const char* name, double s, int32_t n_ranks, int32_t offset, int64_t n,
                      int32_t* out) {
  if (n_ranks <= 0) return -1;
  std::vector<double> cdf((size_t)n_ranks);
  double acc = 0;
  for (int32_t r = 1; r <= n_ranks; r++) {
    acc += std::pow((double)r, -s);
    cdf[(size_t)r - 1] = acc;
  }
  for (auto& v : cdf) v /= acc;
  cdf.back() = 1.0;
  int64_t nchunks = (n + kChunk - 1) / kChunk;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t c = 0; c < nchunks; c++) {
    Xoshiro g(seed, name, (uint64_t)c);
    int64_t i0 = c * kChunk, i1 = std::min(n, i0 + kChunk);
    for (int64_t i = i0; i < i1; i++) {
      double u = g.uniform();
      size_t k = (size_t)(std::upper_bound(cdf.begin(), cdf.end(), u) - cdf.begin());
      if (k >= (size_t)n_ranks) k = (size_t)n_ranks - 1;
      out[i] = (int32_t)(k + 1) + offset;
    }
  }
  return 0;
}

void fa_synth_unit_rows(uint64_t seed, const char* name, int64_t n, int32_t d, float* out) {
  std::vector<double> tmp((size_t)n * d);
  normals(seed, name, n * (int64_t)d, [&](int64_t i, double z) { tmp[(size_t)i] = z; });
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; r++) {
    double ss = 0;
    for (int32_t c = 0; c < d; c++) ss += tmp[(size_t)r * d + c] * tmp[(size_t)r * d + c];
    double inv = 1.0 / std::sqrt(ss);
    for (int32_t c = 0; c < d; c++) out[(size_t)r * d + c] = (float)(tmp[(size_t)r * d + c] * inv);
  }
}

}  // extern "C"
