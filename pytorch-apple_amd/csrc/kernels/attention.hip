// GQA decode attention (one query token) over static K/V caches, in two kernels
// with no cross-workgroup synchronisation inside either of them.
//
// The math restates the CPU (ATen) rounding points of the eager attention chain
//   s  = round(q . k)              matmul, fp32 accumulation
//   s1 = round(s * scale)          mul by 1/sqrt(d)
//   s2 = round_add(s1 + mask)      add of the additive mask
//   p  = round(softmax_f32(s2))    softmax(dtype=f32) then to(model dtype)
//   o  = round(sum_s p * v)        matmul, fp32 accumulation
// k_attn_scores: one workgroup per (64-position tile, KV head) computes s2 for the
//   G query heads of the group (each K row is read once and shared by the G heads)
//   and the tile's (max, sum exp) per head.
// k_attn_out:    one workgroup per (8-dim slice, KV head) folds the tile stats into
//   the global (max, sum) per head, forms p for every position exactly as above
//   and accumulates p * V over the whole sequence for its slice, so the output is
//   written in one pass with no partial-sum combine.
// Positions whose mask is -inf contribute exactly 0: their K rows are never loaded,
// and V rows of tiles that are entirely masked are skipped, so KV traffic follows
// the valid length rather than the cache capacity.
// Loads are issued in batches before their first use so that each wave keeps many
// HBM requests in flight (decode attention is latency-, not bandwidth-, limited).
#include "common.h"

#define AT_TILE 64
#define AT_D 128
#define AT_GMAX 8
#define AT_ROUND 8
#define AT_MAXTILES 1024

__device__ __forceinline__ void unpack8(const uint4 v, int dt, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
    f[2 * i] = dt == HS_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
    f[2 * i + 1] = dt == HS_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
  }
}

extern "C" __global__ void __launch_bounds__(256) k_attn_scores(const DecodeAttnArgs a) {
  __shared__ float qs[AT_GMAX][AT_D];
  __shared__ float sc[AT_GMAX][AT_TILE];
  __shared__ float mv[AT_TILE];
  __shared__ int live;
  const int G = a.H / a.KVH;
  const int kvh = blockIdx.y;
  const int tile = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long t0 = (long long)tile * AT_TILE;
  if (threadIdx.x == 0) live = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < G * AT_D; i += 256) {
    const int h = i / AT_D, d = i % AT_D;
    const uint16_t raw = ((const uint16_t*)a.q)[(long long)(kvh * G + h) * a.q_head_stride + d];
    qs[h][d] = a.dtype == HS_BF16 ? bf16_to_f32(raw) : f16_to_f32(raw);
  }
  if (threadIdx.x < AT_TILE) {
    const long long p = t0 + threadIdx.x;
    float m = -INFINITY;
    if (p < a.S) m = a.mask_dtype < 0 ? 0.f : ld_f(a.mask, p * a.mask_stride, a.mask_dtype);
    mv[threadIdx.x] = m;
    if (m != -INFINITY) live = 1;
  }
  __syncthreads();
  if (!live) {   // whole tile masked: contributes nothing (l = 0)
    if (threadIdx.x < G) {
      float* st = a.stats + ((long long)(kvh * G + threadIdx.x) * a.ntiles + tile) * 2;
      st[0] = -INFINITY;
      st[1] = 0.f;
    }
    return;
  }
  const int g8 = lane >> 3, sub = lane & 7;
  const uint16_t* K = (const uint16_t*)a.k + (long long)kvh * a.kv_head_stride;
  uint4 kr[2][2];
  bool use[2];
#pragma unroll
  for (int step = 0; step < 2; ++step) {
    const int tp = wave * 16 + step * 8 + g8;
    use[step] = mv[tp] != -INFINITY;
    const uint4* src = (const uint4*)(K + (t0 + tp) * AT_D + sub * 16);
    kr[step][0] = use[step] ? src[0] : make_uint4(0, 0, 0, 0);
    kr[step][1] = use[step] ? src[1] : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int step = 0; step < 2; ++step) {
    const int tp = wave * 16 + step * 8 + g8;
    float kf[16];
    unpack8(kr[step][0], a.dtype, kf);
    unpack8(kr[step][1], a.dtype, kf + 8);
    float dots[AT_GMAX];
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      float acc = 0.f;
      if (h < G) {
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = fmaf(qs[h][sub * 16 + j], kf[j], acc);
      }
      dots[h] = acc;
    }
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      dots[h] += __shfl_xor(dots[h], 4, 64);
      dots[h] += __shfl_xor(dots[h], 2, 64);
      dots[h] += __shfl_xor(dots[h], 1, 64);
    }
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      if (h < G && sub == h) {
        float s = -INFINITY;
        if (use[step]) {
          s = round_to(dots[h], a.dtype);
          s = round_to(s * a.scale, a.dtype);
          if (a.mask_dtype >= 0) s = round_to(s + mv[tp], a.add_dtype);
        }
        sc[h][tp] = s;
        if (t0 + tp < a.S) a.scores[(long long)(kvh * G + h) * a.S + t0 + tp] = s;
      }
    }
  }
  __syncthreads();
  for (int h = wave; h < G; h += 4) {
    const float v = sc[h][lane];
    const float m = wave_max(v);
    const float e = (m == -INFINITY || v == -INFINITY) ? 0.f : expf(v - m);
    const float l = wave_sum(e);
    if (lane == 0) {
      float* st = a.stats + ((long long)(kvh * G + h) * a.ntiles + tile) * 2;
      st[0] = m;
      st[1] = l;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) k_attn_out(const AttnOutArgs a) {
  __shared__ float gm[AT_GMAX], ginv[AT_GMAX];
  __shared__ unsigned char tile_live[AT_MAXTILES];
  __shared__ float red[256][AT_GMAX * 8 + 1];
  const int G = a.H / a.KVH;
  const int kvh = blockIdx.y;
  const int d0 = blockIdx.x * 8;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int t = threadIdx.x; t < a.ntiles; t += 256) tile_live[t] = 0;
  __syncthreads();
  for (int h = wave; h < G; h += 4) {
    const float* st = a.stats + (long long)(kvh * G + h) * a.ntiles * 2;
    float m = -INFINITY;
    for (int t = lane; t < a.ntiles; t += 64) m = fmaxf(m, st[2 * t]);
    m = wave_max(m);
    float l = 0.f;
    for (int t = lane; t < a.ntiles; t += 64) {
      const float lt = st[2 * t + 1];
      if (lt > 0.f) {
        l += lt * expf(st[2 * t] - m);
        tile_live[t] = 1;
      }
    }
    l = wave_sum(l);
    if (lane == 0) { gm[h] = m; ginv[h] = 1.0f / l; }
  }
  __syncthreads();
  float acc[AT_GMAX][8];
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;
  const uint16_t* V = (const uint16_t*)a.v + (long long)kvh * a.kv_head_stride + d0;
  const float* SC = a.scores + (long long)kvh * G * a.S;
  for (long long base = 0; base < a.S; base += 256 * AT_ROUND) {
    uint4 vr[AT_ROUND];
    float s[AT_ROUND][AT_GMAX];
#pragma unroll
    for (int r = 0; r < AT_ROUND; ++r) {
      const long long p = base + r * 256 + threadIdx.x;
      const bool ok = p < a.S && tile_live[p / AT_TILE];
      vr[r] = ok ? *(const uint4*)(V + p * AT_D) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int h = 0; h < AT_GMAX; ++h) s[r][h] = (ok && h < G) ? SC[(long long)h * a.S + p] : -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < AT_ROUND; ++r) {
      float vf[8];
      unpack8(vr[r], a.dtype, vf);
#pragma unroll
      for (int h = 0; h < AT_GMAX; ++h) {
        if (h < G && s[r][h] != -INFINITY) {
          const float p = round_to(expf(s[r][h] - gm[h]) * ginv[h], a.dtype);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(p, vf[j], acc[h][j]);
        }
      }
    }
  }
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) red[threadIdx.x][h * 8 + j] = acc[h][j];
  __syncthreads();
  // 4 threads per output value, each summing 64 rows; then a fixed-order 4-way combine
  const int o = threadIdx.x >> 2, q4 = threadIdx.x & 3;
  float part = 0.f;
  if (o < G * 8) {
    for (int i = q4 * 64; i < q4 * 64 + 64; ++i) part += red[i][o];
  }
  part += __shfl_xor(part, 1, 64);
  part += __shfl_xor(part, 2, 64);
  if (o < G * 8 && q4 == 0) {
    const int h = o >> 3, j = o & 7;
    const long long idx = (long long)(kvh * G + h) * AT_D + d0 + j;
    ((uint16_t*)a.out)[idx] = a.dtype == HS_BF16 ? f32_to_bf16(part) : f32_to_f16(part);
  }
}
