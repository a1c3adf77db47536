// Split-K GQA decode attention for one query token, as a device routine shared
// by the standalone launcher and the fused decode step.
//
// Work split. One 256-thread block per (kv head, split) and per set of query
// heads sharing that kv head: all of the group (the reference's shape) or a
// single head (more, lighter blocks when the context is short). Every value
// below is computed per query head with no operation mixing heads, so the
// result does not depend on how heads are grouped into blocks. Split s covers
// positions [s*chunk, min(seq_len, (s+1)*chunk)) with chunk = ceil(seq_len /
// splits), as in the reference (src/kernels/attention.cu:129-133). The range
// is cut into tiles of 64 positions; wave w of the block takes tiles w, w+4,
// w+8, ... .
//
// Tile layout. A position's key (or value) is head_dim/8 = P chunks of 16
// bytes. Lane L holds chunk j = L % P of positions i*(64/P) + L/P for
// i = 0..P-1, so each load instruction of the wave reads 64 consecutive chunks
// (1 KiB contiguous in the contiguous layout, whole 16-position page runs in
// the paged one).
//
// Arithmetic, in this exact order (the CPU oracle repeats it):
//  1. q is multiplied by `scale` in fp32 (the reference folds the scale into q,
//     attention.cu:138-145).
//  2. Partial dot of lane L for position i and head g: d = sum over the 8
//     elements of its chunk, d = fma(q, k, d) from d = 0.
//  3. The P partials of a position are added by a butterfly over the P lanes
//     holding it (offsets P/2, ..., 1), run as a reduce-scatter: afterwards lane
//     L owns the scores of position index i = L % P, i.e. position
//     (L % P)*(64/P) + L/P of the tile, for every head of the group. Positions
//     past the end of the range get score -FLT_MAX.
//  4. Per tile and head: M = max(m, max over the wave of the scores);
//     r = exp(m - M); p = exp(s - M) for the owned position;
//     l_lane = fma(l_lane, r, p); m = M.
//  5. The p of the tile go through LDS so lane L reads the P probabilities of
//     the positions it holds values for, and for each head g and element e:
//     acc = acc * r, then acc = fma(p_i, v_i[e], acc) for i = 0..P-1.
//  6. After its last tile a wave adds acc over the lanes holding the same chunk
//     (butterfly offsets 32, ..., P) and l over all 64 lanes (offsets 32..1).
//  7. Waves merge in order 0..3 exactly like the reference's warp merge
//     (attention.cu:221-240): (m, l) by softmax_combine,
//       M = max(m, m'), l = fma(l, exp(m - M), l' * exp(m' - M)),
//     then acc = sum over waves of fma(exp(m_w - M), acc_w, acc) from 0.
//  8. splits == 1: out = rne(acc * (1 / l)). Otherwise the block writes its
//     unnormalised (m, l, acc[head_dim]) to partials[head][split], and the
//     merge pass combines splits 0..splits-1 the same way as step 7, starting
//     from the identity (-FLT_MAX, 0), and writes rne(sum * (1 / L)).
#pragma once

#include "../kv_cache.h"
#include "device_common.h"

namespace lcr {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = 4;
constexpr int kAttnTile = 64;
constexpr int kPartialHeader = 2;

// Softmax combine of the reference (reduce.cuh:45-52) with the product order
// fixed: l = fma(l, exp(m - M), other_l * exp(other_m - M)).
__host__ __device__ __forceinline__ void softmax_combine(float* m, float* l, float other_m,
                                                         float other_l) {
  const float merged = fmaxf(*m, other_m);
  *l = __builtin_fmaf(*l, lcr_expf(*m - merged), other_l * lcr_expf(other_m - merged));
  *m = merged;
}

template <int kHeadDim, int kGroup>
struct AttnShared {
  float probs[kAttnWaves][64 * kGroup];
  float wave_m[kAttnWaves][kGroup];
  float wave_l[kAttnWaves][kGroup];
  float wave_acc[kAttnWaves][kGroup][kHeadDim];
  float merge_l[kGroup];
  float merge_m[kGroup];
  float merge_scale[kGroup][kAttnWaves];  // exp(m_w - M) per head and wave
};

// Step 3's reduce-scatter: at offset O the lane keeps the half of its N values
// whose position-index bit matches its own lane bit and adds the partner's
// copy of that half.
template <int O, int N>
__device__ __forceinline__ void reduce_scatter(float* vals, int lane) {
  const bool upper = (lane & O) != 0;
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const float lo = vals[k];
    const float hi = vals[k + N / 2];
    const float send = upper ? lo : hi;
    const float keep = upper ? hi : lo;
    vals[k] = keep + xor_lane<O>(send);
  }
  if constexpr (O > 1) reduce_scatter<O / 2, N / 2>(vals, lane);
}

// Step 6's sum over the lanes holding the same chunk: offsets 32, 16, ..., P.
template <int P>
__device__ __forceinline__ float sum_over_groups(float v) {
  v += xor_lane<32>(v);
  if constexpr (P <= 16) v += xor_lane<16>(v);
  if constexpr (P <= 8) v += xor_lane<8>(v);
  return v;
}

// One block: query heads qhead0 .. qhead0 + kGroup - 1, all reading kv head
// `kv_head`, over split `split`. `q` holds num_heads * kHeadDim elements (head h
// at h * kHeadDim). Writes either out (splits == 1) or partials.
template <bool kPaged, int kHeadDim, int kGroup>
__device__ __forceinline__ void decode_attention_block(
    AttnShared<kHeadDim, kGroup>& sh, elem_t* __restrict__ out, float* __restrict__ partials,
    const elem_t* __restrict__ q, const KvCacheView& view, int kv_head, int qhead0, int split,
    int splits, int seq_len, float scale) {
  constexpr int P = kHeadDim / 8;   // chunks per position
  constexpr int Q = 64 / P;         // positions per load instruction
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int j = lane % P;
  const int a = lane / P;

  const int chunk = (seq_len + splits - 1) / splits;
  const int begin = split * chunk;
  const int end = min(seq_len, begin + chunk);
  const int length = max(0, end - begin);

  float qv[kGroup][8];
#pragma unroll
  for (int g = 0; g < kGroup; ++g) {
    const vec16 raw = load16(q + static_cast<size_t>(qhead0 + g) * kHeadDim + 8 * j);
    unpack8(raw, qv[g]);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[g][e] *= scale;
  }

  float m[kGroup], l_lane[kGroup], acc[kGroup][8];
#pragma unroll
  for (int g = 0; g < kGroup; ++g) {
    m[g] = kSoftmaxIdentity;
    l_lane[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  }

  for (int tile = wave; tile * kAttnTile < length; tile += kAttnWaves) {
    const int tile_begin = begin + tile * kAttnTile;
    const int count = min(kAttnTile, end - tile_begin);

    vec16 kreg[P], vreg[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int pi = i * Q + a;
      if (pi < count) {
        const size_t off = view.offset<kPaged>(kv_head, tile_begin + pi) + 8 * j;
        kreg[i] = load16(view.keys + off);
        vreg[i] = load16(view.values + off);
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) kreg[i].w[w] = vreg[i].w[w] = 0u;
      }
    }

    // Step 2: partial dots, value index v = i * kGroup + g.
    float vals[P * kGroup];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      float kf[8];
      unpack8(kreg[i], kf);
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = __builtin_fmaf(qv[g][e], kf[e], d);
        vals[i * kGroup + g] = d;
      }
    }
    // Step 3: reduce-scatter butterfly over the P lanes of a position.
    reduce_scatter<P / 2, P * kGroup>(vals, lane);
    const int own = j * Q + a;  // owned position index within the tile
    float s[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) s[g] = own < count ? vals[g] : kSoftmaxIdentity;

    // Step 4.
    float r[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      const float mnew = fmaxf(m[g], wave_max(s[g]));
      r[g] = lcr_expf(m[g] - mnew);
      const float p = lcr_expf(s[g] - mnew);
      l_lane[g] = __builtin_fmaf(l_lane[g], r[g], p);
      m[g] = mnew;
      sh.probs[wave][lane * kGroup + g] = p;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Step 5.
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = acc[g][e] * r[g];
    }
    const float* pr = &sh.probs[wave][a * P * kGroup];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      float vf[8];
      unpack8(vreg[i], vf);
#pragma unroll
      for (int g = 0; g < kGroup; ++g) {
        const float p = pr[i * kGroup + g];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = __builtin_fmaf(p, vf[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // Step 6.
#pragma unroll
  for (int g = 0; g < kGroup; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = sum_over_groups<P>(acc[g][e]);
    l_lane[g] = wave_sum(l_lane[g]);
  }
  if (lane < P) {
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sh.wave_acc[wave][g][8 * lane + e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
      sh.wave_m[wave][g] = m[g];
      sh.wave_l[wave][g] = l_lane[g];
    }
  }
  __syncthreads();

  // Steps 7-8, by wave 0. The per-head factors (M, L, exp(m_w - M)) do not
  // depend on the element, so lane g computes them once for head g.
  if (wave == 0) {
    if (lane < kGroup) {
      const int g = lane;
      float tm = sh.wave_m[0][g];
      float tl = sh.wave_l[0][g];
#pragma unroll
      for (int w = 1; w < kAttnWaves; ++w) softmax_combine(&tm, &tl, sh.wave_m[w][g], sh.wave_l[w][g]);
      sh.merge_m[g] = tm;
      sh.merge_l[g] = tl;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) sh.merge_scale[g][w] = lcr_expf(sh.wave_m[w][g] - tm);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int idx = lane; idx < kGroup * kHeadDim; idx += 64) {
      const int g = idx / kHeadDim;
      const int d = idx % kHeadDim;
      const float tm = sh.merge_m[g];
      const float tl = sh.merge_l[g];
      float merged = 0.0f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        merged = __builtin_fmaf(sh.merge_scale[g][w], sh.wave_acc[w][g][d], merged);
      }
      const int head = qhead0 + g;
      if (splits == 1) {
        out[static_cast<size_t>(head) * kHeadDim + d] = float_to_elem(merged * (1.0f / tl));
      } else {
        float* slot = partials + (static_cast<size_t>(head) * splits + split) * (kPartialHeader + kHeadDim);
        if (d == 0) {
          slot[0] = tm;
          slot[1] = tl;
        }
        slot[kPartialHeader + d] = merged;
      }
    }
  }
}

constexpr int kMaxSplits = 64;

// Merge of the split partials of one query head. Every thread of the block
// calls it (it synchronises the block). Thread 0 folds the (m, l) of the
// splits in order; the factors exp(m_s - M) are then formed once per split and
// every thread sums its elements over the splits in order. `lds` holds
// 2 + kMaxSplits floats.
__device__ __forceinline__ void merge_split_partials(elem_t* __restrict__ out,
                                                     const float* __restrict__ partials, int head,
                                                     int splits, int head_dim, float* lds) {
  const int stride = kPartialHeader + head_dim;
  const float* base = partials + static_cast<size_t>(head) * splits * stride;
  if (threadIdx.x == 0) {
    float tm = kSoftmaxIdentity;
    float tl = 0.0f;
    for (int s = 0; s < splits; ++s) softmax_combine(&tm, &tl, base[s * stride], base[s * stride + 1]);
    lds[0] = tm;
    lds[1] = tl;
  }
  __syncthreads();
  const float tm = lds[0];
  const float inv = 1.0f / lds[1];
  for (int s = threadIdx.x; s < splits; s += blockDim.x) lds[2 + s] = lcr_expf(base[s * stride] - tm);
  __syncthreads();
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float sum = 0.0f;
    for (int s = 0; s < splits; ++s) {
      sum = __builtin_fmaf(lds[2 + s], base[s * stride + kPartialHeader + d], sum);
    }
    out[static_cast<size_t>(head) * head_dim + d] = float_to_elem(sum * inv);
  }
  __syncthreads();
}

}  // namespace lcr
