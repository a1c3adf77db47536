// CPU oracle for the token loop. TEST INFRASTRUCTURE ONLY: the checker that
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg run against
// the HIP library. The shipped library never links or calls it.
//
// What it restates, function by function (reference = /root/reference of
// mohamadmsalman82/llama-cuda-runtime):
//   orc_embedding_lookup     src/kernels/elementwise.cu:25-41
//   orc_rmsnorm              src/kernels/rmsnorm.cu:21-63
//   orc_add_residual_rmsnorm src/kernels/rmsnorm.cu:68-119
//   orc_add_residual         src/kernels/elementwise.cu:43-62
//   orc_swiglu(_strided)     src/kernels/elementwise.cu:70-121
//   orc_merge_heads          src/kernels/elementwise.cu:124-143
//   orc_rope_q / _write_kv   src/kernels/rope.cu:33-87
//   orc_kv_offset            src/kv_cache.cuh:49-56
//   orc_gather_kv            src/kernels/attention.cu:302-316
//   orc_decode_attention     src/kernels/attention.cu:110-299
//   orc_choose_attention_splits src/kernels/attention.cu:419-431
//   orc_causal_softmax       src/kernels/attention.cu:42-100
//   orc_prefill_attention    src/model.cu:509-560
//   orc_gemv / orc_gemm      src/model.cu:38-45 (cublasGemmEx, fp32 compute)
//   orc_argmax               src/kernels/sampling.cu:37-67
//   orc_sample               src/kernels/sampling.cu:97-224
//   orc_rope_inv_freq        src/config.cpp:223-259
//   orc_model_*              src/model.cu:303-503, src/kv_cache.cu:24-127
//
// Where the reference leaves an order open (cuBLAS summation, thread
// scheduling, atomics) or uses an undocumented fast intrinsic (__expf,
// sincosf), this file fixes one: the same one the HIP kernels implement, so
// decode results compare bit for bit. How each function is pinned independently
// of the GPU code (reference known-answer tests, closed forms, exact-integer
// cases, fp64 brute force) is in tests/test_oracle.py.
//
// Build: oracle/Makefile (g++ -O3 -mavx2 -mfma -fopenmp -ffp-contract=off).
#include "lcr_oracle.h"

#include <immintrin.h>
#include <omp.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;

// ---------------------------------------------------------------------------
// Element conversions (src/dtype.cuh:41-54: round to nearest even)
// ---------------------------------------------------------------------------

inline float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint32_t f2u(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

inline float bf16_to_f(uint16_t b) { return u2f(static_cast<uint32_t>(b) << 16); }

inline uint16_t f_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline float half_to_f(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));  // inf / nan
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    // subnormal: value = man * 2^-24, exact in float
    const float v = static_cast<float>(man) * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

inline uint16_t f_to_half(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds to inf
  if (a < 0x38800000u) {
    // below the smallest normal half (2^-14): round a * 2^24 to an integer.
    const float v = u2f(a) * 16777216.0f;  // exact scaling by 2^24
    const float r = std::nearbyint(v);      // ties to even
    return static_cast<uint16_t>(sign | static_cast<uint16_t>(r));
  }
  // normal: rebias exponent, round the 13 dropped mantissa bits to nearest even
  uint32_t h = ((a >> 13) - (112u << 10));
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return static_cast<uint16_t>(sign | h);
}

inline float e2f(uint16_t b, int kind) { return kind == ORC_FP16 ? half_to_f(b) : bf16_to_f(b); }
inline uint16_t f2e(float f, int kind) { return kind == ORC_FP16 ? f_to_half(f) : f_to_bf16(f); }

// ---------------------------------------------------------------------------
// exp and sincos: the fixed operation sequences documented in the kernels'
// device_common.h (Cody-Waite + Taylor for exp in float; double-precision
// reduction by pi/2 + Maclaurin series for sin/cos).
// ---------------------------------------------------------------------------

float expf_fixed(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 88.72283f) return HUGE_VALF;
  const float k = std::rint(x * 1.44269504088896341f);
  float r = std::fma(k, -0.693145751953125f, x);
  r = std::fma(k, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-4f;
  p = std::fma(p, r, 1.38888888888888889e-3f);
  p = std::fma(p, r, 8.33333333333333333e-3f);
  p = std::fma(p, r, 4.16666666666666667e-2f);
  p = std::fma(p, r, 1.66666666666666667e-1f);
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  return std::ldexp(p, static_cast<int>(k));
}

void sincos_fixed(float angle, float* s_out, float* c_out) {
  const double x = static_cast<double>(angle);
  const double k = std::rint(x * 6.36619772367581382433e-01);
  double r = std::fma(-k, 1.57079632673412561417e+00, x);
  r = std::fma(-k, 6.07710050650619224932e-11, r);
  const double r2 = r * r;
  double sp = 2.81145725434552076320e-15;
  sp = std::fma(sp, r2, -7.64716373181981647590e-13);
  sp = std::fma(sp, r2, 1.60590438368216145994e-10);
  sp = std::fma(sp, r2, -2.50521083854417187751e-08);
  sp = std::fma(sp, r2, 2.75573192239858906526e-06);
  sp = std::fma(sp, r2, -1.98412698412698412698e-04);
  sp = std::fma(sp, r2, 8.33333333333333333333e-03);
  sp = std::fma(sp, r2, -1.66666666666666666667e-01);
  const double sin_r = std::fma(r * r2, sp, r);
  double cp = -1.56192069685862264622e-16;
  cp = std::fma(cp, r2, 4.77947733238738529744e-14);
  cp = std::fma(cp, r2, -1.14707455977297247139e-11);
  cp = std::fma(cp, r2, 2.08767569878680989792e-09);
  cp = std::fma(cp, r2, -2.75573192239858906526e-07);
  cp = std::fma(cp, r2, 2.48015873015873015873e-05);
  cp = std::fma(cp, r2, -1.38888888888888888889e-03);
  cp = std::fma(cp, r2, 4.16666666666666666667e-02);
  cp = std::fma(cp, r2, -0.5);
  const double cos_r = std::fma(r2, cp, 1.0);
  const int q = static_cast<int>(static_cast<long long>(k) & 3);
  double s, c;
  switch (q) {
    case 0: s = sin_r; c = cos_r; break;
    case 1: s = cos_r; c = -sin_r; break;
    case 2: s = -sin_r; c = -cos_r; break;
    default: s = -cos_r; c = sin_r; break;
  }
  *s_out = static_cast<float>(s);
  *c_out = static_cast<float>(c);
}

// softmax_combine with the product order fixed (src/kernels/reduce.cuh:45-52).
inline void softmax_combine(float* m, float* l, float om, float ol) {
  const float merged = std::fmax(*m, om);
  *l = std::fma(*l, expf_fixed(*m - merged), ol * expf_fixed(om - merged));
  *m = merged;
}

// Butterfly over `n` lanes (n a power of two), offsets from n/2 down to `lo`:
// v[i] += v[i ^ o] for every lane at once.
void butterfly(float* v, int n, int lo = 1) {
  std::vector<float> next(static_cast<size_t>(n));
  for (int o = n / 2; o >= lo; o >>= 1) {
    for (int i = 0; i < n; ++i) next[static_cast<size_t>(i)] = v[i] + v[i ^ o];
    std::copy(next.begin(), next.end(), v);
  }
}

// The RMSNorm sum of squares: 256 threads, chunks of 8 strided by 256, a
// 32-lane butterfly per group, then the 8 group sums through a 32-lane
// butterfly padded with zeros (src/kernels/rmsnorm.cu:32-46, reduce.cuh:23-37).
float norm_sum_squares(const float* v, int dim) {
  float part[256];
  const int chunks = dim / 8;
  for (int t = 0; t < 256; ++t) {
    float s = 0.0f;
    for (int c = t; c < chunks; c += 256) {
      for (int j = 0; j < 8; ++j) {
        const float x = v[8 * c + j];
        s = std::fma(x, x, s);
      }
    }
    for (int i = chunks * 8 + t; i < dim; i += 256) s = std::fma(v[i], v[i], s);
    part[t] = s;
  }
  float groups[32] = {0};
  for (int g = 0; g < 8; ++g) {
    butterfly(part + 32 * g, 32);
    groups[g] = part[32 * g];
  }
  butterfly(groups, 32);
  return groups[0];
}

inline float norm_scale(float total, int dim, float eps) {
  return 1.0f / std::sqrt(total / static_cast<float>(dim) + eps);
}

// ---------------------------------------------------------------------------
// GEMV order: blocks of 2048; lane l accumulates chunks l, l+64, l+128, l+192
// of the block (8 elements each, fma from +0, chunks past K skipped); 64-lane
// butterfly per block; block sums added left to right.
// ---------------------------------------------------------------------------

float dot_fixed(const uint16_t* w, const uint16_t* x, int K, int kind) {
  float total = 0.0f;
  const int blocks = (K + 2047) / 2048;
  float lanes[64];
  for (int b = 0; b < blocks; ++b) {
    for (int l = 0; l < 64; ++l) lanes[l] = 0.0f;
    for (int c = 0; c < 4; ++c) {
      const int base = b * 2048 + c * 512;
      if (base >= K) break;
      for (int l = 0; l < 64; ++l) {
        const int e = base + 8 * l;
        if (e >= K) break;
        float acc = lanes[l];
        for (int j = 0; j < 8; ++j) acc = std::fma(e2f(w[e + j], kind), e2f(x[e + j], kind), acc);
        lanes[l] = acc;
      }
    }
    butterfly(lanes, 64);
    total = (b == 0) ? lanes[0] : total + lanes[0];
  }
  return total;
}

// bf16 fast path of dot_fixed, vectorisable over lanes.
float dot_fixed_bf16(const uint16_t* w, const float* xf, int K) {
  float total = 0.0f;
  const int blocks = (K + 2047) / 2048;
  alignas(64) float lanes[64];
  for (int b = 0; b < blocks; ++b) {
    for (int l = 0; l < 64; ++l) lanes[l] = 0.0f;
    const bool full = b * 2048 + 2048 <= K;
    for (int c = 0; c < 4; ++c) {
      const int base = b * 2048 + c * 512;
      if (base >= K) break;
      if (full) {
        for (int j = 0; j < 8; ++j) {
#pragma omp simd
          for (int l = 0; l < 64; ++l) {
            const int e = base + 8 * l + j;
            lanes[l] = std::fma(bf16_to_f(w[e]), xf[e], lanes[l]);
          }
        }
      } else {
        for (int l = 0; l < 64; ++l) {
          const int e = base + 8 * l;
          if (e >= K) break;
          float acc = lanes[l];
          for (int j = 0; j < 8; ++j) acc = std::fma(bf16_to_f(w[e + j]), xf[e + j], acc);
          lanes[l] = acc;
        }
      }
    }
    butterfly(lanes, 64);
    total = (b == 0) ? lanes[0] : total + lanes[0];
  }
  return total;
}

void gemv_rows(int kind, void* y, int y_fp32, const uint16_t* W, const uint16_t* x, int N, int K) {
  std::vector<float> xf(static_cast<size_t>(K));
  for (int k = 0; k < K; ++k) xf[static_cast<size_t>(k)] = e2f(x[k], kind);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint16_t* row = W + static_cast<size_t>(n) * K;
    const float v = (kind == ORC_BF16) ? dot_fixed_bf16(row, xf.data(), K) : dot_fixed(row, x, K, kind);
    if (y_fp32) {
      static_cast<float*>(y)[n] = v;
    } else {
      static_cast<uint16_t*>(y)[n] = f2e(v, kind);
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention: the split-K schedule of the HIP kernel
// (attention_decode.h), lane by lane.
// ---------------------------------------------------------------------------

template <bool kPaged>
int64_t kv_offset(const orc_kv_view& v, int head, int position) {
  const int page = kPaged ? v.page_table[position / v.page_size] : 0;
  const int slot = kPaged ? position % v.page_size : position;
  return static_cast<int64_t>(page) * v.page_stride + static_cast<int64_t>(head) * v.head_stride +
         static_cast<int64_t>(slot) * v.head_dim;
}

inline int64_t kv_off(const orc_kv_view& v, bool paged, int head, int pos) {
  return paged ? kv_offset<true>(v, head, pos) : kv_offset<false>(v, head, pos);
}

constexpr int kAttnWaves = 8;  // waves per attention block (kernels/attention_decode.h)

struct SplitResult {
  std::vector<float> m, l, acc;  // [G], [G], [G][hd]
};

SplitResult attention_split(int kind, const std::vector<float>& qs, const orc_kv_view& view,
                            bool paged, int kv, int G, int begin, int end) {
  const int hd = view.head_dim;
  const int P = hd / 8;
  const int Q = 64 / P;
  const int length = std::max(0, end - begin);
  constexpr int W = kAttnWaves;
  std::vector<float> wm(W * G), wl(W * G), wacc(static_cast<size_t>(W) * G * hd);
  for (int w = 0; w < W; ++w) {
    std::vector<float> m(G, -FLT_MAX);
    std::vector<float> l_lane(static_cast<size_t>(64) * G, 0.0f);
    std::vector<float> acc(static_cast<size_t>(64) * G * 8, 0.0f);
    std::vector<float> s(static_cast<size_t>(64) * G), p(static_cast<size_t>(64) * G);
    std::vector<float> kf(static_cast<size_t>(64) * hd), vf(static_cast<size_t>(64) * hd);
    for (int tile = w; tile * 64 < length; tile += W) {
      const int tb = begin + tile * 64;
      const int count = std::min(64, end - tb);
      for (int pi = 0; pi < 64; ++pi) {
        for (int d = 0; d < hd; ++d) {
          if (pi < count) {
            const int64_t off = kv_off(view, paged, kv, tb + pi);
            kf[static_cast<size_t>(pi) * hd + d] = e2f(view.keys[off + d], kind);
            vf[static_cast<size_t>(pi) * hd + d] = e2f(view.values[off + d], kind);
          } else {
            kf[static_cast<size_t>(pi) * hd + d] = 0.0f;
            vf[static_cast<size_t>(pi) * hd + d] = 0.0f;
          }
        }
      }
      // Scores: P chunk partials per position, butterfly over the P lanes.
      for (int pi = 0; pi < 64; ++pi) {
        for (int g = 0; g < G; ++g) {
          float part[16];
          for (int j = 0; j < P; ++j) {
            float d = 0.0f;
            for (int e = 0; e < 8; ++e) {
              d = std::fma(qs[static_cast<size_t>(g) * hd + 8 * j + e],
                           kf[static_cast<size_t>(pi) * hd + 8 * j + e], d);
            }
            part[j] = d;
          }
          butterfly(part, P);
          s[static_cast<size_t>(pi) * G + g] = pi < count ? part[0] : -FLT_MAX;
        }
      }
      // Owner lane of position pi = j*Q + a is L = a*P + j.
      std::vector<float> r(G);
      for (int g = 0; g < G; ++g) {
        float tmax = -FLT_MAX;
        for (int pi = 0; pi < 64; ++pi) tmax = std::fmax(tmax, s[static_cast<size_t>(pi) * G + g]);
        const float mnew = std::fmax(m[g], tmax);
        r[g] = expf_fixed(m[g] - mnew);
        for (int pi = 0; pi < 64; ++pi) {
          const int L = (pi % Q) * P + pi / Q;
          const float pv = expf_fixed(s[static_cast<size_t>(pi) * G + g] - mnew);
          p[static_cast<size_t>(pi) * G + g] = pv;
          float& ll = l_lane[static_cast<size_t>(L) * G + g];
          ll = std::fma(ll, r[g], pv);
        }
        m[g] = mnew;
      }
      // Values: lane L = (j, a) holds positions i*Q + a, dims 8j..8j+7.
      for (int L = 0; L < 64; ++L) {
        const int j = L % P;
        const int a = L / P;
        for (int g = 0; g < G; ++g) {
          float* ac = &acc[(static_cast<size_t>(L) * G + g) * 8];
          for (int e = 0; e < 8; ++e) ac[e] = ac[e] * r[g];
          for (int i = 0; i < P; ++i) {
            const int pi = i * Q + a;
            const float pv = p[static_cast<size_t>(pi) * G + g];
            for (int e = 0; e < 8; ++e) {
              ac[e] = std::fma(pv, vf[static_cast<size_t>(pi) * hd + 8 * j + e], ac[e]);
            }
          }
        }
      }
    }
    // Wave totals.
    for (int g = 0; g < G; ++g) {
      float lv[64];
      for (int L = 0; L < 64; ++L) lv[L] = l_lane[static_cast<size_t>(L) * G + g];
      butterfly(lv, 64);
      wm[static_cast<size_t>(w) * G + g] = m[g];
      wl[static_cast<size_t>(w) * G + g] = lv[0];
      for (int e = 0; e < 8; ++e) {
        float av[64];
        for (int L = 0; L < 64; ++L) av[L] = acc[(static_cast<size_t>(L) * G + g) * 8 + e];
        butterfly(av, 64, P);
        for (int j = 0; j < P; ++j) {
          wacc[(static_cast<size_t>(w) * G + g) * hd + 8 * j + e] = av[j];
        }
      }
    }
  }
  SplitResult res;
  res.m.resize(G);
  res.l.resize(G);
  res.acc.resize(static_cast<size_t>(G) * hd);
  // Waves merge max first: M = max m_w, c_w = exp(m_w - M), then L and acc
  // accumulated in wave order (kernels/attention_decode.h step 7).
  for (int g = 0; g < G; ++g) {
    float tm = wm[g];
    for (int w = 1; w < W; ++w) tm = std::fmax(tm, wm[static_cast<size_t>(w) * G + g]);
    float c[W];
    for (int w = 0; w < W; ++w) c[w] = expf_fixed(wm[static_cast<size_t>(w) * G + g] - tm);
    float tl = 0.0f;
    for (int w = 0; w < W; ++w) tl = std::fma(wl[static_cast<size_t>(w) * G + g], c[w], tl);
    res.m[g] = tm;
    res.l[g] = tl;
    for (int d = 0; d < hd; ++d) {
      float merged = 0.0f;
      for (int w = 0; w < W; ++w) {
        merged = std::fma(c[w], wacc[(static_cast<size_t>(w) * G + g) * hd + d], merged);
      }
      res.acc[static_cast<size_t>(g) * hd + d] = merged;
    }
  }
  return res;
}

void decode_attention_impl(int kind, uint16_t* out, const uint16_t* q, const orc_kv_view& view,
                           int num_heads, int G, int seq_len, float scale, bool paged, int splits) {
  const int hd = view.head_dim;
  const int kv_heads = num_heads / G;
  splits = std::min(splits, seq_len);
  const int chunk = (seq_len + splits - 1) / splits;
#pragma omp parallel for schedule(dynamic)
  for (int kv = 0; kv < kv_heads; ++kv) {
    std::vector<float> qs(static_cast<size_t>(G) * hd);
    for (int g = 0; g < G; ++g) {
      for (int d = 0; d < hd; ++d) {
        qs[static_cast<size_t>(g) * hd + d] =
            e2f(q[static_cast<size_t>(kv * G + g) * hd + d], kind) * scale;
      }
    }
    std::vector<SplitResult> parts;
    for (int sp = 0; sp < splits; ++sp) {
      const int begin = sp * chunk;
      const int end = std::min(seq_len, begin + chunk);
      parts.push_back(attention_split(kind, qs, view, paged, kv, G, begin, end));
    }
    for (int g = 0; g < G; ++g) {
      const int head = kv * G + g;
      if (splits == 1) {
        const float inv = 1.0f / parts[0].l[g];
        for (int d = 0; d < hd; ++d) {
          out[static_cast<size_t>(head) * hd + d] = f2e(parts[0].acc[static_cast<size_t>(g) * hd + d] * inv, kind);
        }
        continue;
      }
      // Splits merge max first, like the waves (attention_decode.h step 8).
      float tm = parts[0].m[g];
      for (int sp = 1; sp < splits; ++sp) tm = std::fmax(tm, parts[sp].m[g]);
      std::vector<float> c(static_cast<size_t>(splits));
      for (int sp = 0; sp < splits; ++sp) c[static_cast<size_t>(sp)] = expf_fixed(parts[sp].m[g] - tm);
      float tl = 0.0f;
      for (int sp = 0; sp < splits; ++sp) tl = std::fma(parts[sp].l[g], c[static_cast<size_t>(sp)], tl);
      const float inv = 1.0f / tl;
      for (int d = 0; d < hd; ++d) {
        float sum = 0.0f;
        for (int sp = 0; sp < splits; ++sp) {
          sum = std::fma(c[static_cast<size_t>(sp)], parts[sp].acc[static_cast<size_t>(g) * hd + d], sum);
        }
        out[static_cast<size_t>(head) * hd + d] = f2e(sum * inv, kind);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Sampling
// ---------------------------------------------------------------------------

inline uint32_t order_key(float v) {
  const uint32_t b = f2u(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

}  // namespace

extern "C" {

const char* orc_last_error(void) { return g_error.c_str(); }

void orc_set_threads(int n) { omp_set_num_threads(n < 1 ? 1 : n); }
int orc_threads(void) { return omp_get_max_threads(); }

float orc_elem_to_float(uint16_t bits, int kind) { return e2f(bits, kind); }
uint16_t orc_float_to_elem(float value, int kind) { return f2e(value, kind); }
float orc_expf(float x) { return expf_fixed(x); }
void orc_sincosf(float angle, float* s, float* c) { sincos_fixed(angle, s, c); }

// src/config.cpp:223-259: theta^(-2i/d) in double rounded to float; llama3
// bands keep short wavelengths, divide long ones by the factor, and blend in
// between by (context/wavelength - low) / (high - low).
void orc_rope_inv_freq(int head_dim, float theta, int llama3, float factor, float low, float high,
                       int original_context, float* out) {
  const int pairs = head_dim / 2;
  for (int i = 0; i < pairs; ++i) {
    out[i] = static_cast<float>(1.0 / std::pow(static_cast<double>(theta),
                                               static_cast<double>(2 * i) / head_dim));
  }
  if (!llama3) return;
  const double ctx = original_context;
  const double long_wave = ctx / low;
  const double short_wave = ctx / high;
  for (int i = 0; i < pairs; ++i) {
    const double f = out[i];
    const double wl = 2.0 * M_PI / f;
    double v;
    if (wl < short_wave) {
      v = f;
    } else if (wl > long_wave) {
      v = f / factor;
    } else {
      const double t = (ctx / wl - low) / (high - low);
      v = (1.0 - t) * (f / factor) + t * f;
    }
    out[i] = static_cast<float>(v);
  }
}

int64_t orc_kv_offset(const orc_kv_view* view, int paged, int head, int position) {
  return kv_off(*view, paged != 0, head, position);
}

void orc_embedding_lookup(uint16_t* out, const uint16_t* table, const int32_t* ids, int tokens,
                          int dim) {
  for (int t = 0; t < tokens; ++t) {
    std::memcpy(out + static_cast<size_t>(t) * dim, table + static_cast<size_t>(ids[t]) * dim,
                static_cast<size_t>(dim) * 2);
  }
}

void orc_rmsnorm(int kind, uint16_t* out, const uint16_t* x, const uint16_t* w, int tokens,
                 int dim, float eps) {
  std::vector<float> v(static_cast<size_t>(dim));
  for (int t = 0; t < tokens; ++t) {
    const uint16_t* xr = x + static_cast<size_t>(t) * dim;
    for (int i = 0; i < dim; ++i) v[static_cast<size_t>(i)] = e2f(xr[i], kind);
    const float scale = norm_scale(norm_sum_squares(v.data(), dim), dim, eps);
    for (int i = 0; i < dim; ++i) {
      out[static_cast<size_t>(t) * dim + i] = f2e((v[static_cast<size_t>(i)] * scale) * e2f(w[i], kind), kind);
    }
  }
}

void orc_add_residual_rmsnorm(int kind, uint16_t* out, uint16_t* x, const uint16_t* delta,
                              const uint16_t* w, int tokens, int dim, float eps) {
  std::vector<float> v(static_cast<size_t>(dim));
  for (int t = 0; t < tokens; ++t) {
    uint16_t* xr = x + static_cast<size_t>(t) * dim;
    const uint16_t* dr = delta + static_cast<size_t>(t) * dim;
    for (int i = 0; i < dim; ++i) {
      v[static_cast<size_t>(i)] = e2f(xr[i], kind) + e2f(dr[i], kind);
      xr[i] = f2e(v[static_cast<size_t>(i)], kind);
    }
    const float scale = norm_scale(norm_sum_squares(v.data(), dim), dim, eps);
    for (int i = 0; i < dim; ++i) {
      out[static_cast<size_t>(t) * dim + i] = f2e((e2f(xr[i], kind) * scale) * e2f(w[i], kind), kind);
    }
  }
}

void orc_add_residual(int kind, uint16_t* x, const uint16_t* delta, int64_t count) {
  for (int64_t i = 0; i < count; ++i) x[i] = f2e(e2f(x[i], kind) + e2f(delta[i], kind), kind);
}

static inline float silu(float v) { return v / (1.0f + expf_fixed(-v)); }

void orc_swiglu(int kind, uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = f2e(silu(e2f(gate[i], kind)) * e2f(up[i], kind), kind);
}

void orc_swiglu_strided(int kind, uint16_t* out, const uint16_t* gate, const uint16_t* up,
                        int tokens, int width, int src_row_stride) {
  for (int t = 0; t < tokens; ++t) {
    const size_t src = static_cast<size_t>(t) * src_row_stride;
    for (int i = 0; i < width; ++i) {
      out[static_cast<size_t>(t) * width + i] =
          f2e(silu(e2f(gate[src + i], kind)) * e2f(up[src + i], kind), kind);
    }
  }
}

void orc_merge_heads(uint16_t* out, const uint16_t* heads, int tokens, int num_heads,
                     int head_dim) {
  for (int h = 0; h < num_heads; ++h) {
    for (int t = 0; t < tokens; ++t) {
      std::memcpy(out + (static_cast<size_t>(t) * num_heads + h) * head_dim,
                  heads + (static_cast<size_t>(h) * tokens + t) * head_dim,
                  static_cast<size_t>(head_dim) * 2);
    }
  }
}

static void rotate(float lo, float hi, float position, float freq, float* a, float* b) {
  float s, c;
  sincos_fixed(position * freq, &s, &c);
  *a = lo * c - hi * s;
  *b = hi * c + lo * s;
}

void orc_rope_q(int kind, uint16_t* q_heads, const uint16_t* q_proj, const float* inv_freq,
                int tokens, int start_position, int num_heads, int head_dim, int src_row_stride) {
  const int half = head_dim / 2;
  for (int t = 0; t < tokens; ++t) {
    const float pos = static_cast<float>(start_position + t);
    for (int h = 0; h < num_heads; ++h) {
      const size_t src = static_cast<size_t>(t) * src_row_stride + static_cast<size_t>(h) * head_dim;
      const size_t dst = (static_cast<size_t>(h) * tokens + t) * head_dim;
      for (int i = 0; i < half; ++i) {
        float a, b;
        rotate(e2f(q_proj[src + i], kind), e2f(q_proj[src + i + half], kind), pos, inv_freq[i], &a, &b);
        q_heads[dst + i] = f2e(a, kind);
        q_heads[dst + i + half] = f2e(b, kind);
      }
    }
  }
}

void orc_rope_write_kv(int kind, const orc_kv_view* view, const uint16_t* k_proj,
                       const uint16_t* v_proj, const float* inv_freq, int tokens,
                       int start_position, int paged, int src_row_stride) {
  const int hd = view->head_dim;
  const int half = hd / 2;
  for (int t = 0; t < tokens; ++t) {
    const int pos = start_position + t;
    for (int h = 0; h < view->num_kv_heads; ++h) {
      const size_t src = static_cast<size_t>(t) * src_row_stride + static_cast<size_t>(h) * hd;
      const int64_t dst = kv_off(*view, paged != 0, h, pos);
      for (int i = 0; i < half; ++i) {
        float a, b;
        rotate(e2f(k_proj[src + i], kind), e2f(k_proj[src + i + half], kind),
               static_cast<float>(pos), inv_freq[i], &a, &b);
        view->keys[dst + i] = f2e(a, kind);
        view->keys[dst + i + half] = f2e(b, kind);
      }
      for (int i = 0; i < hd; ++i) view->values[dst + i] = v_proj[src + i];
    }
  }
}

void orc_gather_kv(uint16_t* out_keys, uint16_t* out_values, const orc_kv_view* view,
                   int positions) {
  const int hd = view->head_dim;
  for (int h = 0; h < view->num_kv_heads; ++h) {
    for (int p = 0; p < positions; ++p) {
      const int64_t src = kv_offset<true>(*view, h, p);
      const size_t dst = (static_cast<size_t>(h) * positions + p) * hd;
      std::memcpy(out_keys + dst, view->keys + src, static_cast<size_t>(hd) * 2);
      std::memcpy(out_values + dst, view->values + src, static_cast<size_t>(hd) * 2);
    }
  }
}

int orc_choose_attention_splits(int num_kv_heads, int seq_len, int multiprocessors) {
  const int wanted = std::max(1, 2 * multiprocessors);
  const int kv = std::max(1, num_kv_heads);
  int splits = (wanted + kv - 1) / kv;
  splits = std::min(splits, std::max(1, seq_len / 256));
  return std::max(1, std::min(splits, 64));
}

// The model's split policy (llama-cuda-runtime_amd/csrc/model.cpp,
// decode_attention_splits): one split below 4096 positions; below 16384,
// ceil(CUs / num_heads) splits; from 16384, ceil(CUs / num_kv_heads); always
// at least 512 positions per split and at most 64 splits.
int orc_decode_step_splits(int num_heads, int num_kv_heads, int seq_len, int multiprocessors) {
  if (seq_len < 4096) return 1;
  const int per = seq_len < 16384 ? std::max(1, num_heads) : std::max(1, num_kv_heads);
  const int want = std::max(1, (multiprocessors + per - 1) / per);
  const int useful = std::max(1, seq_len / 512);
  return std::max(1, std::min(std::min(want, useful), 64));
}

void orc_decode_attention(int kind, uint16_t* out, const uint16_t* q, const orc_kv_view* view,
                          int num_heads, int heads_per_kv, int seq_len, float scale, int paged,
                          int splits) {
  decode_attention_impl(kind, out, q, *view, num_heads, heads_per_kv, seq_len, scale, paged != 0,
                        splits);
}

// 256 threads per row: online (max, sum) per thread, a softmax_combine
// butterfly inside each 32-thread group (each lane combining its own state
// first), the 8 group results combined in order (src/kernels/attention.cu:42-100).
void orc_causal_softmax(int kind, uint16_t* probs, const float* scores, int num_heads, int rows,
                        int keys, int start_position) {
  for (int h = 0; h < num_heads; ++h) {
    for (int r = 0; r < rows; ++r) {
      const size_t base = (static_cast<size_t>(h) * rows + r) * keys;
      const int limit = std::min(keys, start_position + r + 1);
      float m[256], l[256];
      for (int t = 0; t < 256; ++t) {
        float mm = -FLT_MAX, ll = 0.0f;
        for (int k = t; k < limit; k += 256) {
          const float s = scores[base + k];
          const float merged = std::fmax(mm, s);
          ll = std::fma(ll, expf_fixed(mm - merged), expf_fixed(s - merged));
          mm = merged;
        }
        m[t] = mm;
        l[t] = ll;
      }
      for (int o = 16; o > 0; o >>= 1) {
        float nm[256], nl[256];
        for (int t = 0; t < 256; ++t) {
          float a = m[t], b = l[t];
          softmax_combine(&a, &b, m[t ^ o], l[t ^ o]);
          nm[t] = a;
          nl[t] = b;
        }
        std::memcpy(m, nm, sizeof(m));
        std::memcpy(l, nl, sizeof(l));
      }
      float tm = m[0], tl = l[0];
      for (int w = 1; w < 8; ++w) softmax_combine(&tm, &tl, m[32 * w], l[32 * w]);
      const float inv = 1.0f / tl;
      for (int k = 0; k < keys; ++k) {
        const float p = k < limit ? expf_fixed(scores[base + k] - tm) * inv : 0.0f;
        probs[base + k] = f2e(p, kind);
      }
    }
  }
}

// The reference's prefill attention semantics (src/model.cu:509-560): fp32
// scores scaled once, causal limit, probabilities normalised and rounded to the
// element type, then the value product. Sums here are in double (the reference's
// cuBLAS order is unspecified), so this one is compared within a tolerance.
void orc_prefill_attention(int kind, uint16_t* out, const uint16_t* q_heads,
                           const orc_kv_view* view, int num_heads, int heads_per_kv, int tokens,
                           int start_position, float scale, int paged) {
  const int hd = view->head_dim;
  const int n = start_position + tokens;
  const int kv_heads = num_heads / heads_per_kv;
  // Keys and values of every kv head as floats, in position order.
  std::vector<float> kf(static_cast<size_t>(kv_heads) * n * hd), vf(kf.size());
#pragma omp parallel for collapse(2) schedule(static)
  for (int g = 0; g < kv_heads; ++g) {
    for (int k = 0; k < n; ++k) {
      const int64_t off = kv_off(*view, paged != 0, g, k);
      float* kr = kf.data() + (static_cast<size_t>(g) * n + k) * hd;
      float* vr = vf.data() + (static_cast<size_t>(g) * n + k) * hd;
      for (int i = 0; i < hd; ++i) {
        kr[i] = e2f(view->keys[off + i], kind);
        vr[i] = e2f(view->values[off + i], kind);
      }
    }
  }
#pragma omp parallel
  {
    std::vector<float> s(static_cast<size_t>(n));
    std::vector<double> qd(static_cast<size_t>(hd)), acc(static_cast<size_t>(hd));
#pragma omp for collapse(2) schedule(dynamic, 4)
    for (int h = 0; h < num_heads; ++h) {
      for (int r = 0; r < tokens; ++r) {
        const int g = h / heads_per_kv;
        const int limit = start_position + r + 1;
        const uint16_t* q = q_heads + (static_cast<size_t>(h) * tokens + r) * hd;
        for (int i = 0; i < hd; ++i) qd[static_cast<size_t>(i)] = e2f(q[i], kind);
        const float* K = kf.data() + static_cast<size_t>(g) * n * hd;
        const float* V = vf.data() + static_cast<size_t>(g) * n * hd;
        float m = -FLT_MAX;
        for (int k = 0; k < limit; ++k) {
          const float* kr = K + static_cast<size_t>(k) * hd;
          double d = 0.0;
          for (int i = 0; i < hd; ++i) d += qd[static_cast<size_t>(i)] * kr[i];
          s[static_cast<size_t>(k)] = static_cast<float>(d) * scale;
          m = std::fmax(m, s[static_cast<size_t>(k)]);
        }
        double l = 0.0;
        for (int k = 0; k < limit; ++k) l += std::exp(static_cast<double>(s[static_cast<size_t>(k)] - m));
        const float inv = static_cast<float>(1.0 / l);
        std::fill(acc.begin(), acc.end(), 0.0);
        for (int k = 0; k < limit; ++k) {
          const float p = e2f(f2e(static_cast<float>(std::exp(static_cast<double>(s[static_cast<size_t>(k)] - m))) * inv,
                                  kind), kind);
          const float* vr = V + static_cast<size_t>(k) * hd;
          for (int i = 0; i < hd; ++i) acc[static_cast<size_t>(i)] += static_cast<double>(p) * vr[i];
        }
        uint16_t* o = out + static_cast<size_t>(r) * num_heads * hd + static_cast<size_t>(h) * hd;
        for (int i = 0; i < hd; ++i) o[i] = f2e(static_cast<float>(acc[static_cast<size_t>(i)]), kind);
      }
    }
  }
}

void orc_gemv(int kind, void* y, int y_fp32, const uint16_t* W, const uint16_t* x, int N, int K) {
  gemv_rows(kind, y, y_fp32, W, x, N, K);
}

// Sixteen tokens of a bf16 GEMM at once: for every token the operation order
// of dot_fixed_bf16 (blocks of 2048, lanes of 8-element fma chains, the 64-lane
// butterfly, block sums left to right), vectorised over the tokens (two 8-wide
// vectors per lane), so each weight row is converted and read once per sixteen
// tokens. Bit-identical to sixteen gemv_rows calls. Of the butterfly only lane
// 0 is used, and after the step with offset o lane i holds v[i] + v[i + o] for
// i < o (and the same sum, commuted, for i >= o), so the reduction keeps the
// lower half at each step. xT is the token block transposed, [K][16].
constexpr int kTokenBlock = 16;

void gemm_rows_bf16_block(int tokens, void* Y, int y_fp32, const uint16_t* W, const float* xT, int N,
                          int K) {
#pragma omp parallel
  {
    std::vector<float> wf(static_cast<size_t>(K));
    alignas(32) float lanes[64][kTokenBlock];
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      const uint16_t* w = W + static_cast<size_t>(n) * K;
      for (int k = 0; k < K; ++k) wf[static_cast<size_t>(k)] = bf16_to_f(w[k]);
      alignas(32) float total[kTokenBlock] = {0};
      const int blocks = (K + 2047) / 2048;
      for (int b = 0; b < blocks; ++b) {
        std::memset(lanes, 0, sizeof(lanes));
        for (int c = 0; c < 4; ++c) {
          const int base = b * 2048 + c * 512;
          if (base >= K) break;
          const int nl = std::min(64, (K - base) / 8);  // lanes whose chunk starts below K
          int l0 = 0;
          // Four lanes at a time: eight independent fma chains (two token
          // halves per lane), each lane in its own element order.
          for (; l0 + 4 <= nl; l0 += 4) {
            __m256 a[4][2];
            for (int q = 0; q < 4; ++q) {
              a[q][0] = _mm256_load_ps(lanes[l0 + q]);
              a[q][1] = _mm256_load_ps(lanes[l0 + q] + 8);
            }
            const int e0 = base + 8 * l0;
            for (int j = 0; j < 8; ++j) {
              for (int q = 0; q < 4; ++q) {
                const int e = e0 + 8 * q + j;
                const __m256 wv = _mm256_broadcast_ss(&wf[static_cast<size_t>(e)]);
                const float* xr = xT + static_cast<size_t>(e) * kTokenBlock;
                a[q][0] = _mm256_fmadd_ps(wv, _mm256_load_ps(xr), a[q][0]);
                a[q][1] = _mm256_fmadd_ps(wv, _mm256_load_ps(xr + 8), a[q][1]);
              }
            }
            for (int q = 0; q < 4; ++q) {
              _mm256_store_ps(lanes[l0 + q], a[q][0]);
              _mm256_store_ps(lanes[l0 + q] + 8, a[q][1]);
            }
          }
          for (; l0 < nl; ++l0) {
            __m256 lo = _mm256_load_ps(lanes[l0]);
            __m256 hi = _mm256_load_ps(lanes[l0] + 8);
            for (int j = 0; j < 8; ++j) {
              const int e = base + 8 * l0 + j;
              const __m256 wv = _mm256_broadcast_ss(&wf[static_cast<size_t>(e)]);
              const float* xr = xT + static_cast<size_t>(e) * kTokenBlock;
              lo = _mm256_fmadd_ps(wv, _mm256_load_ps(xr), lo);
              hi = _mm256_fmadd_ps(wv, _mm256_load_ps(xr + 8), hi);
            }
            _mm256_store_ps(lanes[l0], lo);
            _mm256_store_ps(lanes[l0] + 8, hi);
          }
        }
        for (int o = 32; o >= 1; o >>= 1) {
          for (int i = 0; i < o; ++i) {
            _mm256_store_ps(lanes[i], _mm256_add_ps(_mm256_load_ps(lanes[i]), _mm256_load_ps(lanes[i + o])));
            _mm256_store_ps(lanes[i] + 8,
                            _mm256_add_ps(_mm256_load_ps(lanes[i] + 8), _mm256_load_ps(lanes[i + o] + 8)));
          }
        }
        for (int t = 0; t < kTokenBlock; ++t) total[t] = (b == 0) ? lanes[0][t] : total[t] + lanes[0][t];
      }
      for (int t = 0; t < tokens; ++t) {
        if (y_fp32) {
          static_cast<float*>(Y)[static_cast<size_t>(t) * N + n] = total[t];
        } else {
          static_cast<uint16_t*>(Y)[static_cast<size_t>(t) * N + n] = f_to_bf16(total[t]);
        }
      }
    }
  }
}

void orc_gemm(int kind, void* Y, int y_fp32, const uint16_t* X, const uint16_t* W, int T, int N,
              int K) {
  if (kind == ORC_BF16 && T > 1) {
    float* xT = static_cast<float*>(std::aligned_alloc(32, static_cast<size_t>(K) * kTokenBlock * sizeof(float)));
    for (int t0 = 0; t0 < T; t0 += kTokenBlock) {
      const int tb = std::min(kTokenBlock, T - t0);
      std::memset(xT, 0, static_cast<size_t>(K) * kTokenBlock * sizeof(float));
      for (int t = 0; t < tb; ++t) {
        const uint16_t* x = X + static_cast<size_t>(t0 + t) * K;
        for (int k = 0; k < K; ++k) xT[static_cast<size_t>(k) * kTokenBlock + t] = bf16_to_f(x[k]);
      }
      void* yblock = y_fp32 ? static_cast<void*>(static_cast<float*>(Y) + static_cast<size_t>(t0) * N)
                            : static_cast<void*>(static_cast<uint16_t*>(Y) + static_cast<size_t>(t0) * N);
      gemm_rows_bf16_block(tb, yblock, y_fp32, W, xT, N, K);
    }
    std::free(xT);
    return;
  }
  for (int t = 0; t < T; ++t) {
    void* yrow = y_fp32 ? static_cast<void*>(static_cast<float*>(Y) + static_cast<size_t>(t) * N)
                        : static_cast<void*>(static_cast<uint16_t*>(Y) + static_cast<size_t>(t) * N);
    gemv_rows(kind, yrow, y_fp32, W, X + static_cast<size_t>(t) * K, N, K);
  }
}

int32_t orc_argmax(const float* logits, int vocab) {
  unsigned long long best = 0;
  for (int i = 0; i < vocab; ++i) {
    const unsigned long long key = (static_cast<unsigned long long>(order_key(logits[i])) << 32) |
                                   static_cast<unsigned long long>(0xFFFFFFFFu - static_cast<uint32_t>(i));
    best = std::max(best, key);
  }
  return static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(best & 0xFFFFFFFFull));
}

int32_t orc_sample(const float* logits, int vocab, float temperature, int top_k, float top_p,
                   float uniform) {
  if (temperature <= 0.0f) return orc_argmax(logits, vocab);
  const float inv_t = 1.0f / temperature;
  float mx = -FLT_MAX;
  for (int i = 0; i < vocab; ++i) mx = std::fmax(mx, logits[i]);
  // Sum: 1024 threads, each over i = t, t + 1024, ...; 32-lane butterflies,
  // then the 32 group sums through one more (src/kernels/sampling.cu:134-143).
  std::vector<float> part(1024, 0.0f);
  int hist[256] = {0};
  for (int t = 0; t < 1024; ++t) {
    float s = 0.0f;
    for (int i = t; i < vocab; i += 1024) {
      const float scaled = (logits[i] - mx) * inv_t;
      s += expf_fixed(scaled);
      const int bin = std::min(255, static_cast<int>(-scaled * (256 / 20.0f)));
      if (bin >= 0) ++hist[bin];
    }
    part[static_cast<size_t>(t)] = s;
  }
  float groups[32];
  for (int g = 0; g < 32; ++g) {
    butterfly(part.data() + 32 * g, 32);
    groups[g] = part[static_cast<size_t>(32 * g)];
  }
  butterfly(groups, 32);
  const float total = groups[0];
  int running = 0, cutoff = 0;
  for (int b = 0; b < 256; ++b) {
    if (running + hist[b] > 1024) break;
    running += hist[b];
    cutoff = b + 1;
  }
  cutoff = std::max(cutoff, 1);
  // Candidates in index order, at most 1024, sorted by (value desc, index asc).
  std::vector<std::pair<float, int>> cand;
  for (int i = 0; i < vocab && static_cast<int>(cand.size()) < 1024; ++i) {
    const float scaled = (logits[i] - mx) * inv_t;
    const int bin = std::min(255, static_cast<int>(-scaled * (256 / 20.0f)));
    if (bin < cutoff) cand.emplace_back(scaled, i);
  }
  std::sort(cand.begin(), cand.end(), [](const std::pair<float, int>& a, const std::pair<float, int>& b) {
    return a.first > b.first || (a.first == b.first && a.second < b.second);
  });
  const int found = static_cast<int>(cand.size());
  const int limit = top_k > 0 ? std::min(found, top_k) : found;
  const float inv_total = 1.0f / total;
  int keep = 0;
  float kept = 0.0f;
  for (int i = 0; i < limit; ++i) {
    kept = std::fma(expf_fixed(cand[static_cast<size_t>(i)].first), inv_total, kept);
    ++keep;
    if (top_p < 1.0f && kept >= top_p) break;
  }
  if (keep == 0) keep = 1;
  const float target = uniform * kept;
  int picked = found > 0 ? cand[0].second : INT_MAX;
  float run = 0.0f;
  for (int i = 0; i < keep && i < found; ++i) {
    run = std::fma(expf_fixed(cand[static_cast<size_t>(i)].first), inv_total, run);
    picked = cand[static_cast<size_t>(i)].second;
    if (run >= target) break;
  }
  return picked;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Whole model (src/model.cu:303-503; KV cache src/kv_cache.cu:24-127)
// ---------------------------------------------------------------------------

struct orc_model {
  int kind = ORC_BF16;
  orc_config cfg{};
  orc_weights w{};
  std::vector<const uint16_t*> in_norm, qp, kp, vp, op, post, gp, up, dp;
  int max_seq = 0;
  bool paged = false;
  int page_size = 0;
  int prefill_chunk = 256;
  int multiprocessors = 256;
  int forced_splits = 0;
  int position = 0;
  int length = 0;
  std::vector<float> inv_freq;
  std::vector<uint16_t> keys, values;
  std::vector<int32_t> tables;
  int max_pages = 0;
  int pool_pages = 0;
  int pages_mapped = 0;
  std::vector<std::vector<float>> taps;

  orc_kv_view view(int layer) {
    orc_kv_view v{};
    v.num_kv_heads = cfg.num_kv_heads;
    v.head_dim = cfg.head_dim;
    v.page_size = page_size;
    if (!paged) {
      const size_t layer_el = static_cast<size_t>(cfg.num_kv_heads) * max_seq * cfg.head_dim;
      v.keys = keys.data() + layer * layer_el;
      v.values = values.data() + layer * layer_el;
      v.page_table = nullptr;
      v.page_stride = 0;
      v.head_stride = max_seq * cfg.head_dim;
    } else {
      v.keys = keys.data();
      v.values = values.data();
      v.page_table = tables.data() + static_cast<size_t>(layer) * max_pages;
      v.page_stride = cfg.num_kv_heads * page_size * cfg.head_dim;
      v.head_stride = page_size * cfg.head_dim;
    }
    return v;
  }

  void reserve(int len) {
    if (len <= length) return;
    if (paged) {
      const int have = (length + page_size - 1) / page_size;
      const int need = (len + page_size - 1) / page_size;
      for (int layer = 0; layer < cfg.num_layers; ++layer) {
        for (int p = have; p < need; ++p) tables[static_cast<size_t>(layer) * max_pages + p] = pages_mapped++;
      }
    }
    length = len;
  }

  void tap(const std::vector<uint16_t>& x, int tokens) {
    std::vector<float> f(static_cast<size_t>(tokens) * cfg.hidden_size);
    for (size_t i = 0; i < f.size(); ++i) f[i] = e2f(x[i], kind);
    taps.push_back(std::move(f));
  }

  // run_layers (src/model.cu:370-484) for `tokens` rows at start position.
  void run_layers(std::vector<uint16_t>& x, int tokens, int start, float* logits) {
    const int H = cfg.hidden_size, F = cfg.intermediate_size;
    const int qd = cfg.num_heads * cfg.head_dim, kvd = cfg.num_kv_heads * cfg.head_dim;
    const int G = cfg.num_heads / cfg.num_kv_heads;
    const float scale = 1.0f / std::sqrt(static_cast<float>(cfg.head_dim));
    std::vector<uint16_t> normed(static_cast<size_t>(tokens) * H), q(static_cast<size_t>(tokens) * qd),
        k(static_cast<size_t>(tokens) * kvd), v(static_cast<size_t>(tokens) * kvd),
        qh(static_cast<size_t>(tokens) * qd), attn(static_cast<size_t>(tokens) * qd),
        proj(static_cast<size_t>(tokens) * H), gate(static_cast<size_t>(tokens) * F),
        upv(static_cast<size_t>(tokens) * F), act(static_cast<size_t>(tokens) * F);
    taps.clear();
    tap(x, tokens);
    orc_rmsnorm(kind, normed.data(), x.data(), in_norm[0], tokens, H, cfg.rms_norm_eps);
    for (int layer = 0; layer < cfg.num_layers; ++layer) {
      orc_gemm(kind, q.data(), 0, normed.data(), qp[layer], tokens, qd, H);
      orc_gemm(kind, k.data(), 0, normed.data(), kp[layer], tokens, kvd, H);
      orc_gemm(kind, v.data(), 0, normed.data(), vp[layer], tokens, kvd, H);
      const orc_kv_view vw = view(layer);
      orc_rope_q(kind, qh.data(), q.data(), inv_freq.data(), tokens, start, cfg.num_heads, cfg.head_dim, qd);
      orc_rope_write_kv(kind, &vw, k.data(), v.data(), inv_freq.data(), tokens, start, paged, kvd);
      if (tokens == 1) {
        const int seq = start + 1;
        const int splits = forced_splits > 0 ? std::min(forced_splits, 64)
                                             : orc_decode_step_splits(cfg.num_heads, cfg.num_kv_heads, seq,
                                                                      multiprocessors);
        orc_decode_attention(kind, attn.data(), qh.data(), &vw, cfg.num_heads, G, seq, scale, paged, splits);
      } else {
        orc_prefill_attention(kind, attn.data(), qh.data(), &vw, cfg.num_heads, G, tokens, start, scale, paged);
      }
      orc_gemm(kind, proj.data(), 0, attn.data(), op[layer], tokens, H, qd);
      orc_add_residual_rmsnorm(kind, normed.data(), x.data(), proj.data(), post[layer], tokens, H, cfg.rms_norm_eps);
      orc_gemm(kind, gate.data(), 0, normed.data(), gp[layer], tokens, F, H);
      orc_gemm(kind, upv.data(), 0, normed.data(), up[layer], tokens, F, H);
      orc_swiglu(kind, act.data(), gate.data(), upv.data(), static_cast<int64_t>(tokens) * F);
      orc_gemm(kind, proj.data(), 0, act.data(), dp[layer], tokens, H, F);
      const uint16_t* next = layer + 1 < cfg.num_layers ? in_norm[layer + 1] : w.final_norm;
      orc_add_residual_rmsnorm(kind, normed.data(), x.data(), proj.data(), next, tokens, H, cfg.rms_norm_eps);
      tap(x, tokens);
    }
    {
      std::vector<float> f(static_cast<size_t>(tokens) * H);
      for (size_t i = 0; i < f.size(); ++i) f[i] = e2f(normed[i], kind);
      taps.push_back(std::move(f));
    }
    if (logits != nullptr) {
      orc_gemv(kind, logits, 1, w.lm_head, normed.data() + static_cast<size_t>(tokens - 1) * H, cfg.vocab_size, H);
    }
  }
};

extern "C" {

orc_model* orc_model_create(int kind, const orc_config* config, const orc_weights* weights,
                            int max_seq, int paged, int page_size, int prefill_chunk,
                            int multiprocessors, int attention_splits) {
  try {
    auto m = std::make_unique<orc_model>();
    m->kind = kind;
    m->cfg = *config;
    m->w = *weights;
    const int L = config->num_layers;
    m->in_norm.assign(weights->input_norm, weights->input_norm + L);
    m->qp.assign(weights->q_proj, weights->q_proj + L);
    m->kp.assign(weights->k_proj, weights->k_proj + L);
    m->vp.assign(weights->v_proj, weights->v_proj + L);
    m->op.assign(weights->o_proj, weights->o_proj + L);
    m->post.assign(weights->post_norm, weights->post_norm + L);
    m->gp.assign(weights->gate_proj, weights->gate_proj + L);
    m->up.assign(weights->up_proj, weights->up_proj + L);
    m->dp.assign(weights->down_proj, weights->down_proj + L);
    m->max_seq = max_seq;
    m->paged = paged != 0;
    m->prefill_chunk = std::min(prefill_chunk, max_seq);
    m->multiprocessors = multiprocessors;
    m->forced_splits = attention_splits;
    m->inv_freq.resize(static_cast<size_t>(config->head_dim / 2));
    orc_rope_inv_freq(config->head_dim, config->rope_theta, config->rope_llama3, config->rope_factor,
                      config->rope_low_freq_factor, config->rope_high_freq_factor,
                      config->rope_original_context, m->inv_freq.data());
    size_t elems;
    if (!m->paged) {
      m->page_size = max_seq;
      elems = static_cast<size_t>(L) * config->num_kv_heads * max_seq * config->head_dim;
    } else {
      m->page_size = page_size;
      m->max_pages = (max_seq + page_size - 1) / page_size;
      m->pool_pages = m->max_pages * L;
      elems = static_cast<size_t>(m->pool_pages) * config->num_kv_heads * page_size * config->head_dim;
      m->tables.assign(static_cast<size_t>(L) * m->max_pages, -1);
    }
    m->keys.assign(elems, 0);
    m->values.assign(elems, 0);
    return m.release();
  } catch (const std::exception& e) {
    g_error = e.what();
    return nullptr;
  }
}

void orc_model_destroy(orc_model* model) { delete model; }
void orc_model_reset(orc_model* model) {
  model->position = 0;
  model->taps.clear();
}
int orc_model_position(const orc_model* model) { return model->position; }

// Test hooks for the long-context case: the cache is filled from outside (the
// GPU's pre-filled cache, read back in logical order) and the position moved.
int orc_model_set_kv(orc_model* m, int layer, int positions, const uint16_t* keys,
                     const uint16_t* values) {
  if (layer < 0 || layer >= m->cfg.num_layers || positions < 0 || positions > m->max_seq) {
    g_error = "set_kv: layer or positions out of range";
    return -1;
  }
  m->reserve(positions);
  const orc_kv_view v = m->view(layer);
  const int hd = m->cfg.head_dim;
  for (int h = 0; h < m->cfg.num_kv_heads; ++h) {
    for (int pos = 0; pos < positions; ++pos) {
      const int64_t off = kv_off(v, m->paged, h, pos);
      const size_t src = (static_cast<size_t>(h) * positions + pos) * hd;
      std::memcpy(v.keys + off, keys + src, static_cast<size_t>(hd) * 2);
      std::memcpy(v.values + off, values + src, static_cast<size_t>(hd) * 2);
    }
  }
  return 0;
}

int orc_model_set_position(orc_model* m, int position) {
  if (position < 0 || position > m->max_seq) {
    g_error = "set_position: out of range";
    return -1;
  }
  m->reserve(position);
  m->position = position;
  return 0;
}

int orc_model_decode(orc_model* m, int token, float* logits) {
  if (m->position >= m->max_seq) {
    g_error = "sequence reached the cache limit";
    return -1;
  }
  if (token < 0 || token >= m->cfg.vocab_size) {
    g_error = "token id out of range";
    return -1;
  }
  m->reserve(m->position + 1);
  std::vector<uint16_t> x(static_cast<size_t>(m->cfg.hidden_size));
  orc_embedding_lookup(x.data(), m->w.embed, &token, 1, m->cfg.hidden_size);
  m->run_layers(x, 1, m->position, logits);
  m->position += 1;
  return 0;
}

int orc_model_prefill(orc_model* m, const int32_t* tokens, int count, int use_decode_path,
                      float* logits) {
  if (count <= 0) {
    g_error = "prefill needs at least one token";
    return -1;
  }
  if (m->position + count > m->max_seq) {
    g_error = "prompt exceeds the cache";
    return -1;
  }
  for (int i = 0; i < count; ++i) {
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size) {
      g_error = "token id out of range";
      return -1;
    }
  }
  if (use_decode_path) {
    std::vector<float> scratch(static_cast<size_t>(m->cfg.vocab_size));
    for (int i = 0; i < count; ++i) {
      const int rc = orc_model_decode(m, tokens[i], i + 1 == count ? logits : scratch.data());
      if (rc != 0) return rc;
    }
    return 0;
  }
  int consumed = 0;
  while (consumed < count) {
    const int chunk = std::min(m->prefill_chunk, count - consumed);
    m->reserve(m->position + chunk);
    std::vector<uint16_t> x(static_cast<size_t>(chunk) * m->cfg.hidden_size);
    orc_embedding_lookup(x.data(), m->w.embed, tokens + consumed, chunk, m->cfg.hidden_size);
    const bool last = consumed + chunk == count;
    m->run_layers(x, chunk, m->position, last ? logits : nullptr);
    m->position += chunk;
    consumed += chunk;
  }
  return 0;
}

size_t orc_model_tap(const orc_model* m, int index, float* out, size_t capacity) {
  if (index < 0 || static_cast<size_t>(index) >= m->taps.size()) return 0;
  const std::vector<float>& t = m->taps[static_cast<size_t>(index)];
  const size_t n = std::min(capacity, t.size());
  std::memcpy(out, t.data(), n * sizeof(float));
  return n;
}

const int32_t* orc_model_page_table(const orc_model* m, int layer) {
  if (!m->paged) return nullptr;
  return m->tables.data() + static_cast<size_t>(layer) * m->max_pages;
}

}  // extern "C"
