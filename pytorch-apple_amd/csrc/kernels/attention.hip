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
// k_attn_flash: grid (nsplit, KVH, G), 256 threads (k_attn_flash_w16: 1024). Workgroup
// (t, kvh, g) handles query head kvh*G + g over the 16 * W positions of split t (W = 4 or
// 16 waves), 16 per wave. Spreading the
// heads of a GQA group over workgroups (rather than serving all G heads from one K/V
// read) gives G times more workgroups for the same split size; the G reads of a K/V
// tile happen together and are served by the caches, and the work per wave stays small,
// which is what decode attention is limited by (latency, not bytes).
// Per wave: each lane holds a quarter (32 dims) of one position's K row (4 lanes per
// position), the split's mask value for it and the matching quarter of q; scores are
// summed across the quad with DPP, rounded at the model's points (as in k_attn_scores),
// and the wave's (max, sum) come from DPP row rotations plus 4 lane reads. For P.V each
// lane owns 2 of the 128 dims over the wave's 16 positions, taking p from the owning
// lane with readlane. The 4 waves are merged in LDS into the split's partials
//   m_t = max s, l_t = sum exp(s - m_t), o_t = sum exp(s - m_t) v   (fp32).
// A wave whose 16 positions are all masked skips the arithmetic (its K/V loads are issued
// with the mask's, before the mask is known).
// The partials are combined by k_attn_combine (or in the prologue of the next GEMV,
// gemv.hip): o = sum_t e^(m_t - M) o_t / sum_t e^(m_t - M) l_t. Compared with the CPU
// chain, only the bf16 rounding of the probabilities is not repeated.
#define FL_PW 16      // positions per wave; a split is FL_PW * W positions (W waves)

typedef __attribute__((ext_vector_type(2))) __bf16 fl_bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 fl_f16x2;

template <int DT>
__device__ __forceinline__ float fl_dot2(uint32_t a, uint32_t b, float acc) {
  if constexpr (DT == HS_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(fl_bf16x2, a), __builtin_bit_cast(fl_bf16x2, b), acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(fl_f16x2, a), __builtin_bit_cast(fl_f16x2, b), acc, false);
}

// CHK (long caches): the workgroup first reads its split's mask values, and a split whose
// positions are all -inf (closed: it contributes exactly nothing) writes an empty partial without
// loading its K / V rows, so the rows read follow the open positions rather than the cache length.
// The open splits pay one more memory latency (mask, then K / V).
template <int DT, int W, bool CHK = false>
__device__ __forceinline__ void flash_body(const FlashArgs& a) {
  __shared__ float osh[W][AT_D];
  __shared__ float msh[W], lsh[W];
  const int G = a.H / a.KVH;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int split = blockIdx.x, kvh = blockIdx.y, g = blockIdx.z;
  if constexpr (CHK) {
    bool open = false;
    if (a.mask_dtype < 0) {
      open = true;
    } else if (threadIdx.x < FL_PW * W) {
      const long long p = (long long)split * (FL_PW * W) + threadIdx.x;
      open = p < a.S && ld_f(a.mask, p * a.mask_stride, a.mask_dtype) != -INFINITY;
    }
    if (!__syncthreads_or(open)) {
      const long long part = (long long)(kvh * a.nsplit + split) * G + g;
      if (threadIdx.x < AT_D) a.part_o[part * AT_D + threadIdx.x] = 0;
      if (threadIdx.x == 0) {
        a.part_ml[part * 2] = -INFINITY;
        a.part_ml[part * 2 + 1] = 0.f;
      }
      return;
    }
  }
  const long long p0 = (long long)split * (FL_PW * W) + wave * FL_PW;   // this wave's first position
  const int kq = lane >> 2, kc = lane & 3;                         // K: position p0 + kq, dims kc*32..+32
  const long long last = a.S - 1;
  const uint16_t* Kb = (const uint16_t*)a.k + (long long)kvh * a.kv_head_stride;
  const uint16_t* Vb = (const uint16_t*)a.v + (long long)kvh * a.kv_head_stride;
  // every load is issued up front with no branch: the mask value as raw bits, q, and the
  // wave's K and V rows (positions clamped to the cache; a masked position's rows are read
  // but weigh nothing), so one memory latency covers them all
  const void* mptr = a.mask_dtype < 0 ? a.q : a.mask;   // a.q: valid dummy address
  const FRaw mraw = ld_f_raw(mptr, min(p0 + kq, last) * a.mask_stride, a.mask_dtype);
  uint4 qr[4], kr[4];
  uint32_t vr[FL_PW];
  const uint4* qs = (const uint4*)((const uint16_t*)a.q + (long long)(kvh * G + g) * a.q_head_stride + kc * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) qr[j] = qs[j];
  const uint4* ks = (const uint4*)(Kb + min(p0 + kq, last) * AT_D + kc * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) kr[j] = ks[j];
#pragma unroll
  for (int t = 0; t < FL_PW; ++t) vr[t] = *(const uint32_t*)(Vb + min(p0 + t, last) * AT_D + 2 * lane);
  const float mdec = a.mask_dtype < 0 ? 0.f : ld_f_decode(mraw, a.mask_dtype);
  const float mval = (p0 + kq <= last) ? mdec : -INFINITY;
  const bool live = __ballot(mval != -INFINITY) != 0ull;   // wave-uniform
  float m_w = -INFINITY, l_w = 0.f, acc0 = 0.f, acc1 = 0.f;
  if (live) {
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      d = fl_dot2<DT>(qr[j].x, kr[j].x, d);
      d = fl_dot2<DT>(qr[j].y, kr[j].y, d);
      d = fl_dot2<DT>(qr[j].z, kr[j].z, d);
      d = fl_dot2<DT>(qr[j].w, kr[j].w, d);
    }
    d += HS_DPP(d, HS_QUAD_XOR1);
    d += HS_DPP(d, HS_QUAD_XOR2);
    float s = -INFINITY;
    if (mval != -INFINITY) {
      s = round_to(d, DT);
      s = round_to(s * a.scale, DT);
      if (a.mask_dtype >= 0) s = round_to(s + mval, a.add_dtype);
    }
    // the 4 lanes of a quad hold the same position: reduce over quads only
    float m = fmaxf(s, HS_DPP(s, HS_ROW_ROR4));
    m = fmaxf(m, HS_DPP(m, HS_ROW_ROR8));
    m = fmaxf(fmaxf(HS_RL(m, 0), HS_RL(m, 16)), fmaxf(HS_RL(m, 32), HS_RL(m, 48)));
    const float e = (s == -INFINITY) ? 0.f : __expf(s - m);
    float l = e + HS_DPP(e, HS_ROW_ROR4);
    l += HS_DPP(l, HS_ROW_ROR8);
    l_w = (HS_RL(l, 0) + HS_RL(l, 16)) + (HS_RL(l, 32) + HS_RL(l, 48));
    m_w = m;
#pragma unroll
    for (int t = 0; t < FL_PW; ++t) {
      float v0, v1;
      if constexpr (DT == HS_BF16) {
        v0 = bf16_to_f32((uint16_t)(vr[t] & 0xffffu));
        v1 = bf16_to_f32((uint16_t)(vr[t] >> 16));
      } else {
        v0 = f16_to_f32((uint16_t)(vr[t] & 0xffffu));
        v1 = f16_to_f32((uint16_t)(vr[t] >> 16));
      }
      const float p = HS_RL(e, 4 * t);
      acc0 = fmaf(p, v0, acc0);
      acc1 = fmaf(p, v1, acc1);
    }
  }
  osh[wave][2 * lane] = acc0;
  osh[wave][2 * lane + 1] = acc1;
  if (lane == 0) {
    msh[wave] = m_w;
    lsh[wave] = l_w;
  }
  __syncthreads();
  if (threadIdx.x < AT_D) {
    const int dd = threadIdx.x;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, msh[w]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = (lsh[w] > 0.f) ? __expf(msh[w] - M) : 0.f;
      o = fmaf(f, osh[w][dd], o);
      L = fmaf(f, lsh[w], L);
    }
    const long long part = (long long)(kvh * a.nsplit + split) * G + g;
    // the split's own normalised output in bf16 (half the bytes for the combine to read; its
    // weight e^(m - M) l is applied there): 2^-9 relative, below the output's own bf16 rounding
    a.part_o[part * AT_D + dd] = f32_to_bf16(L > 0.f ? o / L : 0.f);
    if (dd == 0) {
      a.part_ml[part * 2] = M;
      a.part_ml[part * 2 + 1] = L;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256) k_attn_flash(const FlashArgs a) { flash_body<HS_BF16, 4>(a); }
extern "C" __global__ void __launch_bounds__(256) k_attn_flash_f16(const FlashArgs a) { flash_body<HS_F16, 4>(a); }
// long caches: closed splits load no K / V rows
extern "C" __global__ void __launch_bounds__(256) k_attn_flash_chk(const FlashArgs a) { flash_body<HS_BF16, 4, true>(a); }
extern "C" __global__ void __launch_bounds__(256) k_attn_flash_chk_f16(const FlashArgs a) {
  flash_body<HS_F16, 4, true>(a);
}
// 8 or 16 waves, 128 or 256 positions per split: 2x or 4x fewer partials, for a combine folded
// into the next GEMV
extern "C" __global__ void __launch_bounds__(512) k_attn_flash_w8(const FlashArgs a) { flash_body<HS_BF16, 8>(a); }
extern "C" __global__ void __launch_bounds__(512) k_attn_flash_w8_f16(const FlashArgs a) { flash_body<HS_F16, 8>(a); }
extern "C" __global__ void __launch_bounds__(1024) k_attn_flash_w16(const FlashArgs a) { flash_body<HS_BF16, 16>(a); }
extern "C" __global__ void __launch_bounds__(1024) k_attn_flash_w16_f16(const FlashArgs a) { flash_body<HS_F16, 16>(a); }

// out[h, d] = round(sum_t e^(m_t - M) l_t o_t[d] / sum_t e^(m_t - M) l_t) over the splits' normalised
// outputs o_t (bf16); one workgroup of 128
// threads per head. Splits are folded in chunks of 64: lane t of every wave loads split t's
// (m, l), so each wave forms the chunk's weights itself (no LDS, no barrier) and thread d
// takes them with readlane while its 64 partial loads are already in flight.
#define CB_CHUNK 64
extern "C" __global__ void __launch_bounds__(128) k_attn_combine(const CombineArgs a) {
  const int h = blockIdx.x;
  const int G = a.H / a.KVH, kvh = h / G, g = h % G;
  const int d = threadIdx.x, lane = threadIdx.x & 63;
  const float* ml = a.part_ml + ((long long)kvh * a.nsplit * G + g) * 2;
  const uint16_t* po = a.part_o + ((long long)kvh * a.nsplit * G + g) * AT_D + d;
  float M = -INFINITY, L = 0.f, acc = 0.f;
  for (int c0 = 0; c0 < a.nsplit; c0 += CB_CHUNK) {
    const int n = min(CB_CHUNK, a.nsplit - c0);
    float ot[CB_CHUNK];
#pragma unroll
    for (int i = 0; i < CB_CHUNK; ++i) ot[i] = bf16_to_f32(po[(long long)(c0 + min(i, n - 1)) * G * AT_D]);
    float m = -INFINITY, l = 0.f;
    if (lane < n) {
      m = ml[(long long)(c0 + lane) * G * 2];
      l = ml[(long long)(c0 + lane) * G * 2 + 1];
    }
    if (!(l > 0.f)) m = -INFINITY;   // fully masked split
    const float Mn = fmaxf(M, wave_max(m));
    const float r = (M == -INFINITY) ? 0.f : __expf(M - Mn);
    const float f = (m == -INFINITY) ? 0.f : __expf(m - Mn);
    L = L * r + wave_sum(f * l);
    const float fl = f * l;   // the weight of split lane's normalised output
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int i = 0; i < CB_CHUNK; i += 4) {
      if (i < n) s0 = fmaf(HS_RL(fl, i), ot[i], s0);
      if (i + 1 < n) s1 = fmaf(HS_RL(fl, i + 1), ot[i + 1], s1);
      if (i + 2 < n) s2 = fmaf(HS_RL(fl, i + 2), ot[i + 2], s2);
      if (i + 3 < n) s3 = fmaf(HS_RL(fl, i + 3), ot[i + 3], s3);
    }
    acc = acc * r + ((s0 + s1) + (s2 + s3));
    M = Mn;
  }
  const float o = acc / L;
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

// ------------------------------------------------------------------ prefill attention (MFMA)
//
// k_attn_prefill: grid (ceil(T / 32), H), 256 threads. Workgroup (qb, h) computes the outputs of
// queries [32 qb, 32 qb + 32) of head h against all S keys of KV head h / (H / KVH), flash style;
// wave w takes the 32-position KV blocks w, w + 4, ... and the four waves are merged at the end.
// Per block, on v_mfma_f32_32x32x16 (D = 128, eight K steps):
//   S^T = K Q^T (positions as rows, queries as columns), so each lane holds 16 scores of ONE
//   query (lane l: query l % 32, positions 8i + 4(l / 32) + r): the online softmax and the
//   rescaling of that query's outputs stay in the lane, with one exchange with lane l ^ 32;
//   s = r(r(q.k) * scale) [+ mask, rounded to add_dtype] as the reference rounds them;
//   O^T += V^T P^T with P in bf16 / fp16 (reordered into the operand layout by two exchanges
//   with lane l ^ 32) and V^T staged through wave-private LDS (position pairs per dword).
// Each block's mask values are loaded with its K and V; a block whose 32 x 32 mask entries are
// all -inf (the causal upper triangle) is skipped. Scores of positions >= S are -inf; rows of
// queries >= T are computed from a clamped query and not stored. The output is written as
// [T, H, D], the layout the o_proj input needs after transpose(1, 2) + reshape.
#define PA_BQ 32
#define PA_BP 32
#define PA_VLD 40   // V^T row length in LDS (positions, padded): 16-byte fragment reads spread over the banks

typedef __attribute__((ext_vector_type(16))) float pa_f32x16;

template <int DT>
__device__ __forceinline__ pa_f32x16 pa_mfma(const uint4 a, const uint4 b, pa_f32x16 c) {
  if constexpr (DT == HS_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(__attribute__((ext_vector_type(8))) __bf16, a),
                                                   __builtin_bit_cast(__attribute__((ext_vector_type(8))) __bf16, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(__attribute__((ext_vector_type(8))) _Float16, a),
                                                  __builtin_bit_cast(__attribute__((ext_vector_type(8))) _Float16, b), c,
                                                  0, 0, 0);
}

template <int DT>
__device__ __forceinline__ uint32_t pa_pack2(float lo, float hi) {
  const uint16_t a = DT == HS_BF16 ? f32_to_bf16(lo) : f32_to_f16(lo);
  const uint16_t b = DT == HS_BF16 ? f32_to_bf16(hi) : f32_to_f16(hi);
  return (uint32_t)a | ((uint32_t)b << 16);
}

// MM: mask mode, 0 none, 1 16-bit mask of the model dtype (8-byte loads of 4 entries), 2 fp32 mask
template <int DT, int MM>
__device__ __forceinline__ void prefill_attn_body(const PrefillAttnArgs& a) {
  __shared__ __attribute__((aligned(16))) uint16_t vt[4][128][PA_VLD];
  __shared__ float ml[4][2][PA_BQ];
  __shared__ float ob[4][PA_BQ][128 + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, hi = lane >> 5;
  const int h = blockIdx.y, kvh = h / (a.H / a.KVH);
  const long long q0 = (long long)blockIdx.x * PA_BQ;
  const long long qrow = min(q0 + fr, a.T - 1);
  const uint16_t* Qp = (const uint16_t*)a.q + (long long)h * a.q_head_stride + qrow * 128;
  const uint16_t* Kb = (const uint16_t*)a.k + (long long)kvh * a.kv_head_stride;
  const uint16_t* Vb = (const uint16_t*)a.v + (long long)kvh * a.kv_head_stride;
  const void* mptr = MM == 0 ? a.q : a.mask;   // a.q: valid dummy address when there is no mask
  const long long mrow = qrow * a.mask_row_stride;
  auto rnd = [&](float f) { return round_to(f, DT); };

  uint4 qf[8];   // B operand of S^T: query fr, dims 16 ks + 8 hi .. + 8
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) qf[ks] = *(const uint4*)(Qp + ks * 16 + hi * 8);
  pa_f32x16 o[4];   // O^T: dims 32 t + 8i + 4 hi + r, query fr
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int nblk = (int)((a.S + PA_BP - 1) / PA_BP);
  // position blocks past the last open mask column of this workgroup's rows are closed for all
  // of them: not visited at all (no K/V loads), which is what a long static cache needs
  const int nb = a.blk_limit != nullptr ? min(nblk, a.blk_limit[blockIdx.x]) : nblk;
  const long long last = a.S - 1;
  // V staging: lane -> positions pr, pr + 1 (pr = 2 (lane % 16)), 16-byte chunks cg + 4j of the dims
  const int pr = 2 * (lane & 15), cg = lane >> 4;

  // MM 1: 16-bit mask with unit column stride (S % 4 == 0, 8-byte aligned rows; the host
  // checks): four positions per 8-byte load
  struct Blk {
    uint2 mq[4];   // mask bits, positions 8i + 4 hi + (0..3)
    uint4 kf[8];   // A operand of S^T: position fr, dims 16 ks + 8 hi .. + 8
    uint4 va[4], vb[4];
  };
  // issue every load of block `blk` (clamped to the last block: a spare load, never used)
  auto load = [&](int blk, Blk& b) {
    const long long p0 = (long long)min(blk, max(nb, 1) - 1) * PA_BP;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (MM == 1) {
        const long long p = min(p0 + 8 * i + 4 * hi, last & ~3ll);
        b.mq[i] = *(const uint2*)((const uint16_t*)mptr + mrow + p);
      } else if constexpr (MM == 2) {   // fp32: two entries per 8-byte load, the other pair below
        const long long p = min(p0 + 8 * i + 4 * hi, last);
        b.mq[i] = make_uint2(__float_as_uint(((const float*)mptr)[mrow + p * a.mask_col_stride]),
                             __float_as_uint(((const float*)mptr)[mrow + min(p + 1, last) * a.mask_col_stride]));
      } else {
        b.mq[i] = make_uint2(0, 0);
      }
    }
    const uint16_t* Kp = Kb + min(p0 + fr, last) * 128 + hi * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) b.kf[ks] = *(const uint4*)(Kp + ks * 16);
    const uint16_t* Va = Vb + min(p0 + pr, last) * 128;
    const uint16_t* Vc = Vb + min(p0 + pr + 1, last) * 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      b.va[j] = *(const uint4*)(Va + (cg + 4 * j) * 8);
      b.vb[j] = *(const uint4*)(Vc + (cg + 4 * j) * 8);
    }
  };
  auto compute = [&](int blk, const Blk& b) {
    const long long p0 = (long long)blk * PA_BP;
    float mv[16];
    bool any = false;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const long long p = p0 + 8 * (e >> 2) + 4 * hi + (e & 3);
      float m = 0.f;
      if constexpr (MM == 1) {
        const uint32_t w = (e & 2) ? b.mq[e >> 2].y : b.mq[e >> 2].x;
        const uint16_t bits = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
        m = DT == HS_BF16 ? bf16_to_f32(bits) : f16_to_f32(bits);
      } else if constexpr (MM == 2) {
        m = (e & 2) ? ((const float*)mptr)[mrow + min(p, last) * a.mask_col_stride]
                    : __uint_as_float((e & 1) ? b.mq[e >> 2].y : b.mq[e >> 2].x);
      }
      mv[e] = p > last ? -INFINITY : m;
      any = any || mv[e] != -INFINITY;
    }
    if (__ballot(any) == 0ull) return;   // wave-uniform: the whole 32 x 32 block is masked out

    // V^T of the block into this wave's LDS rows (dims), position pairs per dword
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = (cg + 4 * j) * 8;
      const uint32_t x[4] = {b.va[j].x, b.va[j].y, b.va[j].z, b.va[j].w};
      const uint32_t y[4] = {b.vb[j].x, b.vb[j].y, b.vb[j].z, b.vb[j].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *(uint32_t*)&vt[wave][d0 + 2 * i][pr] = (x[i] & 0xffffu) | (y[i] << 16);
        *(uint32_t*)&vt[wave][d0 + 2 * i + 1][pr] = (x[i] >> 16) | (y[i] & 0xffff0000u);
      }
    }
    // S^T = K Q^T
    pa_f32x16 s;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) s = pa_mfma<DT>(b.kf[ks], qf[ks], s);
    float sc[16], bm = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float v = rnd(rnd(s[e]) * a.scale);
      if constexpr (MM != 0) v = round_to(v + mv[e], a.add_dtype);
      if (mv[e] == -INFINITY) v = -INFINITY;
      sc[e] = v;
      bm = fmaxf(bm, v);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float m_new = fmaxf(m_run, bm);
    const float alpha = (m_run == -INFINITY) ? 0.f : __expf(m_run - m_new);
    float ps = 0.f;
    float pv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      pv[e] = (sc[e] == -INFINITY) ? 0.f : __expf(sc[e] - m_new);
      ps += pv[e];
    }
    ps += __shfl_xor(ps, 32, 64);
    l_run = l_run * alpha + ps;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[t][e] *= alpha;
    // P into the B-operand layout: lane half 0 needs positions 0-7 / 16-23, half 1 8-15 / 24-31;
    // group i holds positions 8i + 4 hi + (0..3)
    uint2 g[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) g[i] = make_uint2(pa_pack2<DT>(pv[4 * i], pv[4 * i + 1]), pa_pack2<DT>(pv[4 * i + 2], pv[4 * i + 3]));
    const uint2 send0 = hi ? g[0] : g[1], send1 = hi ? g[2] : g[3];
    const uint2 recv0 = make_uint2(__shfl_xor(send0.x, 32, 64), __shfl_xor(send0.y, 32, 64));
    const uint2 recv1 = make_uint2(__shfl_xor(send1.x, 32, 64), __shfl_xor(send1.y, 32, 64));
    const uint4 pf0 = hi ? make_uint4(recv0.x, recv0.y, g[1].x, g[1].y) : make_uint4(g[0].x, g[0].y, recv0.x, recv0.y);
    const uint4 pf1 = hi ? make_uint4(recv1.x, recv1.y, g[3].x, g[3].y) : make_uint4(g[2].x, g[2].y, recv1.x, recv1.y);
    // O^T += V^T P^T (the wave's own LDS writes above are complete before its reads: in-order LDS)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 v0 = *(const uint4*)&vt[wave][t * 32 + fr][hi * 8];
      const uint4 v1 = *(const uint4*)&vt[wave][t * 32 + fr][16 + hi * 8];
      o[t] = pa_mfma<DT>(v0, pf0, o[t]);
      o[t] = pa_mfma<DT>(v1, pf1, o[t]);
    }
  };
  // two blocks in flight: the loads of this wave's next block are issued before the current
  // block is computed (named register sets; loads past the last block re-read it)
  Blk ba, bb;
  load(wave, ba);
  for (int blk = wave; blk < nb; blk += 8) {
    load(blk + 4, bb);
    compute(blk, ba);
    if (blk + 4 >= nb) break;
    load(blk + 8, ba);
    compute(blk + 4, bb);
  }

  // merge the four waves: o_final = sum_w e^(m_w - M) o_w / sum_w e^(m_w - M) l_w
  if (hi == 0) {
    ml[wave][0][fr] = m_run;
    ml[wave][1][fr] = l_run;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) M = fmaxf(M, ml[w][0][fr]);
  const float f_own = (m_run == -INFINITY) ? 0.f : __expf(m_run - M);
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) ob[wave][fr][t * 32 + 8 * (e >> 2) + 4 * hi + (e & 3)] = o[t][e] * f_own;
  __syncthreads();
  // 256 threads x 16 outputs: query tid / 8, dims 16 (tid % 8) .. + 16
  const int qq = tid >> 3, d0 = (tid & 7) * 16;
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float mw = ml[w][0][qq];
    L += (mw == -INFINITY) ? 0.f : __expf(mw - fmaxf(fmaxf(ml[0][0][qq], ml[1][0][qq]), fmaxf(ml[2][0][qq], ml[3][0][qq]))) * ml[w][1][qq];
  }
  if (q0 + qq >= a.T) return;
  uint32_t pk[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      x0 += ob[w][qq][d0 + 2 * i];
      x1 += ob[w][qq][d0 + 2 * i + 1];
    }
    pk[i] = pa_pack2<DT>(x0 / L, x1 / L);
  }
  uint4* dst = (uint4*)((uint16_t*)a.out + (q0 + qq) * (long long)a.H * 128 + (long long)h * 128 + d0);
  dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
}

#define PA_KERNEL(NAME, DT, MM) \
  extern "C" __global__ void __launch_bounds__(256) NAME(const PrefillAttnArgs a) { prefill_attn_body<DT, MM>(a); }
PA_KERNEL(k_attn_prefill, HS_BF16, 1)              // 16-bit mask of the model dtype
PA_KERNEL(k_attn_prefill_nomask, HS_BF16, 0)
PA_KERNEL(k_attn_prefill_f32mask, HS_BF16, 2)
PA_KERNEL(k_attn_prefill_f16, HS_F16, 1)
PA_KERNEL(k_attn_prefill_f16_nomask, HS_F16, 0)
PA_KERNEL(k_attn_prefill_f16_f32mask, HS_F16, 2)

// k_mask_extent: grid (ceil(T / 32)), 1024 threads. nblk_out[qb] = 1 + c / 32 for the largest
// column c < S whose mask entry is not -inf in any of rows 32 qb .. 32 qb + 31 (rows past T are
// not read), 0 when there is none. Every block past it is closed for all of those rows, so
// k_attn_prefill leaves it out: its terms would be e^-inf = 0 exactly. NaN entries count as
// open. Wave w scans rows w and w + 16, lanes along the row, all loads of a 2048-column chunk
// (eight per lane) issued before the first is tested, so a scan of S <= 2048 is one memory
// latency. 16-bit masks are read four entries per 8-byte load (unit column stride, 8-byte aligned
// rows, S % 4 == 0: the host checks).
extern "C" __global__ void __launch_bounds__(1024) k_mask_extent(const MaskExtentArgs a) {
  __shared__ int best[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long q0 = (long long)blockIdx.x * 32;
  int mx = -1;
  for (int r = wave; r < 32; r += 16) {
    const long long t = q0 + r;
    if (t >= a.T) break;   // wave-uniform
    if (a.mask_dtype == HS_F32) {
      const float* row = (const float*)a.mask + t * a.row_stride;
      for (long long c0 = 0; c0 < a.S; c0 += 512) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const long long c = c0 + lane + 64 * j;
          v[j] = c < a.S ? row[c * a.col_stride] : -INFINITY;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (v[j] != -INFINITY) mx = max(mx, (int)(c0 + lane + 64 * j));
      }
    } else {
      const uint32_t ninf = a.mask_dtype == HS_BF16 ? 0xFF80u : 0xFC00u;
      const uint32_t ninf2 = ninf | (ninf << 16);
      const uint16_t* row = (const uint16_t*)a.mask + t * a.row_stride;
      for (long long c0 = 0; c0 < a.S; c0 += 2048) {
        uint2 w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const long long c = c0 + 4 * lane + 256 * j;
          w[j] = c < a.S ? *(const uint2*)(row + c) : make_uint2(ninf2, ninf2);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int c = (int)(c0 + 4 * lane + 256 * j);
          if ((w[j].y >> 16) != ninf) mx = max(mx, c + 3);
          else if ((w[j].y & 0xffffu) != ninf) mx = max(mx, c + 2);
          else if ((w[j].x >> 16) != ninf) mx = max(mx, c + 1);
          else if ((w[j].x & 0xffffu) != ninf) mx = max(mx, c);
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = max(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) best[wave] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = best[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) m = max(m, best[w]);
    a.nblk_out[blockIdx.x] = m < 0 ? 0 : m / PA_BP + 1;
  }
}
