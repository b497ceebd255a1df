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
    // unconditional load; masked rows read the tile's first row instead (valid, discarded)
    const uint4* src = (const uint4*)(K + (t0 + (use[step] ? tp : 0)) * AT_D + sub * 16);
    kr[step][0] = src[0];
    kr[step][1] = src[1];
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

// ------------------------------------------------------------------ split-S flash decoding
//
// k_attn_flash: one workgroup per (split of `spl` positions, KV head). The q rows of
// the G heads and the split's mask are staged first; then every K and V row of the
// split is requested at once (8 lanes x 32 B per K row, 16 lanes x 16 B per V row),
// scores are formed with the model's rounding points (as in k_attn_scores), the
// split's (max m, sum l) per head computed, and sum_s exp(s - m) v_s accumulated.
// The partials are combined either by k_attn_combine or inside the next GEMV's
// prologue (gemv.hip): o = sum_t e^(m_t - M) o_t / sum_t e^(m_t - M) l_t. Compared
// with the CPU chain, only the bf16 rounding of the probabilities is not repeated.
#define FL_SPL 128

typedef __attribute__((ext_vector_type(2))) __bf16 fl_bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 fl_f16x2;

template <int DT>
__device__ __forceinline__ float fl_dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (DT == HS_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fl_bf16x2, a), __builtin_bit_cast(fl_bf16x2, b), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(fl_f16x2, a), __builtin_bit_cast(fl_f16x2, b), acc, false);
}

template <int DT>
__device__ __forceinline__ void flash_body(const FlashArgs& a) {
  __shared__ float mv[FL_SPL];
  __shared__ float sc[AT_GMAX][FL_SPL];
  __shared__ float red[4][AT_GMAX][AT_D];
  __shared__ int live;
  const int G = a.H / a.KVH;
  const int split = blockIdx.x, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long p0 = (long long)split * a.spl;
  const int npos = (int)min((long long)a.spl, a.S - p0);
  const int pw = a.spl >> 2;                       // positions per wave
  const int g8 = lane >> 3, sub = lane & 7;        // K: 8 lanes per row, 16 dims each
  const int g16 = lane >> 4, dv = (lane & 15) * 8; // V: 16 lanes per row, 8 dims each
  float* ml = a.part_ml + ((long long)(kvh * a.nsplit + split) * G) * 2;
  float* po = a.part_o + ((long long)(kvh * a.nsplit + split) * G) * AT_D;
  // q (this lane's 16 dims of each head, kept packed) and the split's mask, in one round trip
  uint4 qr[AT_GMAX][2];
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h) {
    const int hh = h < G ? h : 0;
    const uint4* src = (const uint4*)((const uint16_t*)a.q + (long long)(kvh * G + hh) * a.q_head_stride + sub * 16);
    qr[h][0] = src[0];
    qr[h][1] = src[1];
  }
  if (threadIdx.x == 0) live = 0;
  __syncthreads();
  if ((int)threadIdx.x < a.spl) {
    float m = -INFINITY;
    if ((int)threadIdx.x < npos)
      m = a.mask_dtype < 0 ? 0.f : ld_f(a.mask, (p0 + threadIdx.x) * a.mask_stride, a.mask_dtype);
    mv[threadIdx.x] = m;
    if (m != -INFINITY) live = 1;
  }
  __syncthreads();
  if (!live) {   // fully masked split: l = 0 and zero partials (combines read them unconditionally)
    if (threadIdx.x < G) {
      ml[threadIdx.x * 2] = -INFINITY;
      ml[threadIdx.x * 2 + 1] = 0.f;
    }
    for (int i = threadIdx.x; i < G * AT_D; i += 256) po[i] = 0.f;
    return;
  }
  const uint16_t* K = (const uint16_t*)a.k + (long long)kvh * a.kv_head_stride + p0 * AT_D;
  const uint16_t* V = (const uint16_t*)a.v + (long long)kvh * a.kv_head_stride + p0 * AT_D;
  // Every K and V load is issued unconditionally; a masked or out-of-split row reads row 0
  // of the split instead (valid memory) and is discarded, so all loads stay in flight.
  uint4 kr[FL_SPL / 32][2];
  uint4 vr[FL_SPL / 16];
#pragma unroll
  for (int st = 0; st < FL_SPL / 32; ++st) {
    const int tp = wave * pw + st * 8 + g8;
    const int row = (st * 8 < pw && mv[tp] != -INFINITY) ? tp : 0;
    const uint4* src = (const uint4*)(K + (long long)row * AT_D + sub * 16);
    kr[st][0] = src[0];
    kr[st][1] = src[1];
  }
#pragma unroll
  for (int st = 0; st < FL_SPL / 16; ++st) {
    const int tp = wave * pw + st * 4 + g16;
    const int row = (st * 4 < pw && mv[tp] != -INFINITY) ? tp : 0;
    vr[st] = *(const uint4*)(V + (long long)row * AT_D + dv);
  }
  // scores (packed dot products on the raw bf16/fp16 data) with the model's rounding points
#pragma unroll
  for (int st = 0; st < FL_SPL / 32; ++st) {
    if (st * 8 >= pw) break;
    const int tp = wave * pw + st * 8 + g8;
    const uint32_t kw[8] = {kr[st][0].x, kr[st][0].y, kr[st][0].z, kr[st][0].w,
                            kr[st][1].x, kr[st][1].y, kr[st][1].z, kr[st][1].w};
    float dots[AT_GMAX];
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      const uint32_t qw[8] = {qr[h][0].x, qr[h][0].y, qr[h][0].z, qr[h][0].w,
                              qr[h][1].x, qr[h][1].y, qr[h][1].z, qr[h][1].w};
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fl_dot2<DT>(qw[j], kw[j], acc);
      acc += __shfl_xor(acc, 4, 64);
      acc += __shfl_xor(acc, 2, 64);
      acc += __shfl_xor(acc, 1, 64);
      dots[h] = acc;
    }
    if (sub < G) {
      float d = dots[0];
#pragma unroll
      for (int h = 1; h < AT_GMAX; ++h) d = (sub == h) ? dots[h] : d;
      float s = -INFINITY;
      const float m = mv[tp];
      if (m != -INFINITY) {
        s = round_to(d, DT);
        s = round_to(s * a.scale, DT);
        if (a.mask_dtype >= 0) s = round_to(s + m, a.add_dtype);
      }
      sc[sub][tp] = s;
    }
  }
  __syncthreads();
  // split max / sum per head; sc becomes exp(s - m)
  for (int h = wave; h < G; h += 4) {
    float m = -INFINITY;
    for (int i = lane; i < a.spl; i += 64) m = fmaxf(m, sc[h][i]);
    m = wave_max(m);
    float l = 0.f;
    for (int i = lane; i < a.spl; i += 64) {
      const float s = sc[h][i];
      const float e = (s == -INFINITY) ? 0.f : expf(s - m);
      sc[h][i] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      ml[h * 2] = m;
      ml[h * 2 + 1] = l;
    }
  }
  __syncthreads();
  float acc[AT_GMAX][8];
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;
#pragma unroll
  for (int st = 0; st < FL_SPL / 16; ++st) {
    if (st * 4 >= pw) break;
    const int tp = wave * pw + st * 4 + g16;
    if (mv[tp] == -INFINITY) continue;   // p = 0 for every head; the loaded row is a stand-in
    float vf[8];
    unpack8(vr[st], DT, vf);
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h) {
      if (h < G) {
        const float p = sc[h][tp];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(p, vf[j], acc[h][j]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < AT_GMAX; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      acc[h][j] += __shfl_xor(acc[h][j], 16, 64);
      acc[h][j] += __shfl_xor(acc[h][j], 32, 64);
    }
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < AT_GMAX; ++h)
      if (h < G)
#pragma unroll
        for (int j = 0; j < 8; ++j) red[wave][h][dv + j] = acc[h][j];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * AT_D; i += 256) {
    const int h = i / AT_D, d = i % AT_D;
    po[i] = ((red[0][h][d] + red[1][h][d]) + red[2][h][d]) + red[3][h][d];
  }
}

extern "C" __global__ void __launch_bounds__(256) k_attn_flash(const FlashArgs a) { flash_body<HS_BF16>(a); }
extern "C" __global__ void __launch_bounds__(256) k_attn_flash_f16(const FlashArgs a) { flash_body<HS_F16>(a); }

// out[h, d] = round(sum_t e^(m_t - M) o_t[d] * (1 / sum_t e^(m_t - M) l_t)); one workgroup per head
extern "C" __global__ void __launch_bounds__(128) k_attn_combine(const CombineArgs a) {
  __shared__ float w[1024], lv[1024];
  __shared__ float inv_l;
  const int h = blockIdx.x;
  const int G = a.H / a.KVH, kvh = h / G, g = h % G;
  const float* ml = a.part_ml + ((long long)kvh * a.nsplit * G + g) * 2;
  for (int t = threadIdx.x; t < a.nsplit; t += 128) {   // all (m, l) loads in flight at once
    w[t] = ml[(long long)t * G * 2];
    lv[t] = ml[(long long)t * G * 2 + 1];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = -INFINITY;
    for (int t = 0; t < a.nsplit; ++t)
      if (lv[t] > 0.f) M = fmaxf(M, w[t]);
    float L = 0.f;
    for (int t = 0; t < a.nsplit; ++t) {
      const float e = lv[t] > 0.f ? expf(w[t] - M) : 0.f;
      w[t] = e;
      L += e * lv[t];
    }
    inv_l = 1.0f / L;
  }
  __syncthreads();
  const int d = threadIdx.x;
  float s = 0.f;
  for (int t = 0; t < a.nsplit; ++t)   // dead splits hold zero partials and weight 0
    s += w[t] * a.part_o[(((long long)kvh * a.nsplit + t) * G + g) * AT_D + d];
  const float o = s * inv_l;
  ((uint16_t*)a.out)[(long long)h * AT_D + d] = a.dtype == HS_BF16 ? f32_to_bf16(o) : f32_to_f16(o);
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
      const long long pc = ok ? p : 0;   // unconditional loads from a valid row, masked afterwards
      vr[r] = *(const uint4*)(V + pc * AT_D);
#pragma unroll
      for (int h = 0; h < AT_GMAX; ++h) {
        const float raw = SC[(long long)(h < G ? h : 0) * a.S + pc];
        s[r][h] = (ok && h < G) ? raw : -INFINITY;
      }
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
