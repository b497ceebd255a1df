// GQA decode attention (one query token) over static K/V caches, split over
// 64-position tiles so that the two KV heads of Qwen2.5 still fill the chip.
//
// The math restates the CPU (ATen) rounding points of the eager attention chain
//   s  = round(q . k)              matmul, fp32 accumulation
//   s1 = round(s * scale)          mul by 1/sqrt(d)
//   s2 = round_add(s1 + mask)      add of the additive mask
//   p  = round(softmax_f32(s2))    softmax(dtype=f32) then to(model dtype)
//   o  = round(sum_s p * v)        matmul, fp32 accumulation
// so the two passes are:
//   k_attn_scores: s2 for every position of a tile, plus the tile's (max, sum exp)
//   k_attn_pv:     global (max, sum) per head from the tile stats, p for the tile,
//                  the tile's partial p.V; the last tile to finish (atomic ticket)
//                  adds the partials in tile order and writes the output.
// A position whose mask is -inf contributes exactly 0, so its K and V rows are
// never loaded: KV traffic follows the valid length, not the cache capacity.
// Each tile's K rows are read once and shared by the G query heads of its group.
#include "common.h"

#define AT_TILE 64
#define AT_D 128
#define AT_GMAX 8

__device__ __forceinline__ float ld_h(const void* p, long long i, int dt) {
  const uint16_t h = ((const uint16_t*)p)[i];
  return dt == HS_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ void unpack8(const uint4 v, int dt, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
    f[2 * i] = dt == HS_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
    f[2 * i + 1] = dt == HS_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
  }
}

__device__ __forceinline__ bool masked_out(const DecodeAttnArgs& a, long long p, float* mv) {
  if (a.mask_dtype < 0) { *mv = 0.f; return false; }
  *mv = ld_f(a.mask, p * a.mask_stride, a.mask_dtype);
  return *mv == -INFINITY;
}

extern "C" __global__ void __launch_bounds__(256) k_attn_scores(const DecodeAttnArgs a) {
  __shared__ float qs[AT_GMAX][AT_D];
  __shared__ float sc[AT_GMAX][AT_TILE];
  const int G = a.H / a.KVH;
  const int kvh = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < G * AT_D; i += 256) {
    const int h = i / AT_D, d = i % AT_D;
    qs[h][d] = ld_h(a.q, (long long)(kvh * G + h) * a.q_head_stride + d, a.dtype);
  }
  __syncthreads();
  const int g8 = lane >> 3, sub = lane & 7;
  const uint16_t* K = (const uint16_t*)a.k + (long long)kvh * a.kv_head_stride;
#pragma unroll
  for (int step = 0; step < 2; ++step) {
    const int tp = wave * 16 + step * 8 + g8;
    const long long p = (long long)tile * AT_TILE + tp;
    float mv = 0.f;
    const bool valid = p < a.S;
    const bool skip = !valid || masked_out(a, p, &mv);
    float dots[AT_GMAX];
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) dots[h] = 0.f;
    if (!skip) {
      const uint4* kr = (const uint4*)(K + p * AT_D + sub * 16);
      float kf[16];
      unpack8(kr[0], a.dtype, kf);
      unpack8(kr[1], a.dtype, kf + 8);
#pragma unroll
      for (int h = 0; h < AT_GMAX; ++h) {
        if (h < G) {
          float acc = 0.f;
#pragma unroll
          for (int j = 0; j < 16; ++j) acc = fmaf(qs[h][sub * 16 + j], kf[j], acc);
          dots[h] = acc;
        }
      }
    }
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      dots[h] += __shfl_xor(dots[h], 4, 64);
      dots[h] += __shfl_xor(dots[h], 2, 64);
      dots[h] += __shfl_xor(dots[h], 1, 64);
    }
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      if (h < G && sub == (h & 7)) {
        float s;
        if (skip) {
          s = -INFINITY;
        } else {
          s = round_to(dots[h], a.dtype);
          s = round_to(s * a.scale, a.dtype);
          if (a.mask_dtype >= 0) s = round_to(s + mv, a.add_dtype);
        }
        sc[h][tp] = s;
        if (valid) a.scores[(long long)(kvh * G + h) * a.S + p] = s;
      }
    }
  }
  __syncthreads();
  for (int h = wave; h < G; h += 4) {
    const float v = sc[h][lane];
    const float m = wave_max(v);
    const float e = (m == -INFINITY) ? 0.f : expf(v - m);
    const float l = wave_sum(e);
    if (lane == 0) {
      float* st = a.stats + ((long long)(kvh * G + h) * a.ntiles + tile) * 2;
      st[0] = m;
      st[1] = l;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) k_attn_pv(const DecodeAttnArgs a) {
  __shared__ float gm[AT_GMAX], gl[AT_GMAX];
  __shared__ float pr[AT_GMAX][AT_TILE];
  __shared__ float red[4][AT_GMAX][AT_D];
  __shared__ int is_last;
  const int G = a.H / a.KVH;
  const int kvh = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // global max and sum of exp for each head of the group
  for (int h = wave; h < G; h += 4) {
    const float* st = a.stats + (long long)(kvh * G + h) * a.ntiles * 2;
    float m = -INFINITY;
    for (int t = lane; t < a.ntiles; t += 64) m = fmaxf(m, st[2 * t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < a.ntiles; t += 64) {
      const float lt = st[2 * t + 1];
      if (lt > 0.f) l += lt * expf(st[2 * t] - m);
    }
    l = wave_sum(l);
    if (lane == 0) { gm[h] = m; gl[h] = l; }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * AT_TILE; i += 256) {
    const int h = i / AT_TILE, tp = i % AT_TILE;
    const long long p = (long long)tile * AT_TILE + tp;
    float pv = 0.f;
    if (p < a.S) {
      const float s = a.scores[(long long)(kvh * G + h) * a.S + p];
      if (s != -INFINITY) pv = round_to(expf(s - gm[h]) * (1.0f / gl[h]), a.dtype);
    }
    pr[h][tp] = pv;
  }
  __syncthreads();

  // partial o over this tile: lane owns dims 2*lane, 2*lane+1; wave owns 16 positions
  float acc[AT_GMAX][2];
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h) acc[h][0] = acc[h][1] = 0.f;
  const uint16_t* V = (const uint16_t*)a.v + (long long)kvh * a.kv_head_stride;
  for (int j = 0; j < 16; ++j) {
    const int tp = wave * 16 + j;
    const long long p = (long long)tile * AT_TILE + tp;
    if (p >= a.S) break;
    float mv;
    if (masked_out(a, p, &mv)) continue;
    const uint32_t w2 = *(const uint32_t*)(V + p * AT_D + 2 * lane);
    const uint16_t lo = (uint16_t)(w2 & 0xffffu), hi = (uint16_t)(w2 >> 16);
    const float v0 = a.dtype == HS_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
    const float v1 = a.dtype == HS_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      if (h < G) {
        acc[h][0] = fmaf(pr[h][tp], v0, acc[h][0]);
        acc[h][1] = fmaf(pr[h][tp], v1, acc[h][1]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h) {
    if (h < G) {
      red[wave][h][2 * lane] = acc[h][0];
      red[wave][h][2 * lane + 1] = acc[h][1];
    }
  }
  __syncthreads();
  float* part = a.part + ((long long)kvh * a.ntiles + tile) * G * AT_D;
  for (int i = threadIdx.x; i < G * AT_D; i += 256) {
    const int h = i / AT_D, d = i % AT_D;
    part[i] = ((red[0][h][d] + red[1][h][d]) + red[2][h][d]) + red[3][h][d];
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) is_last = (atomicAdd(&a.counters[kvh], 1) == a.ntiles - 1);
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* pk = a.part + (long long)kvh * a.ntiles * G * AT_D;
  for (int i = threadIdx.x; i < G * AT_D; i += 256) {
    float s = 0.f;
    for (int t = 0; t < a.ntiles; ++t) s += pk[(long long)t * G * AT_D + i];
    const int h = i / AT_D, d = i % AT_D;
    const long long o = (long long)(kvh * G + h) * AT_D + d;
    ((uint16_t*)a.out)[o] = a.dtype == HS_BF16 ? f32_to_bf16(s) : f32_to_f16(s);
  }
  if (threadIdx.x == 0) atomicExch(&a.counters[kvh], 0);
}
