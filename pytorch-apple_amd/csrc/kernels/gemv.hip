// Fused streaming GEMV kernels for decode (M <= 4 rows of activations).
//
// Weight rows are the HBM stream: every wave owns RPW rows and walks K with one
// 16-byte load per lane per 512 elements, accumulating in fp32 with v_dot2.
// Around that loop the kernels fold in the ops that the IR places next to each
// projection, at the CPU's rounding points:
//   prologue  NORM   y = round(w_n * round(x * rsqrt(mean(x^2) + eps)))  (RMSNorm), staged in LDS
//   epilogue  BIAS   out = round(acc + b)
//             RESID  out = round(r + round(acc + b))                     (linear then residual add)
//             SILU   out = round(round(silu(round(acc_g))) * round(acc_u)) (gate/up pair, SiLU*mul)
//             ARGMAX out = round(acc); each workgroup writes the largest (ordered value, ~index) key
//                    of its rows to its own slot per activation row (no atomics); k_argmax_finalize
//                    reduces the slots
// k_qkv_rope additionally applies rotary embedding to q/k row pairs (d, d+D/2) and
// writes k/v straight into the static caches at cache_position (index_copy in place).
#include "common.h"

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_v;

__device__ __forceinline__ float dot8_bf16(const uint4 a, const uint4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.x), __builtin_bit_cast(bf16x2_v, b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.y), __builtin_bit_cast(bf16x2_v, b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.z), __builtin_bit_cast(bf16x2_v, b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.w), __builtin_bit_cast(bf16x2_v, b.w), acc, false);
  return acc;
}

typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per step: non-temporal hint)
__device__ __forceinline__ uint4 ld_stream(const uint16_t* p) {
  const u32x4_v v = __builtin_nontemporal_load((const u32x4_v*)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf(const void* p, long long i) { return bf16_to_f32(((const uint16_t*)p)[i]); }
__device__ __forceinline__ float rbf(float f) { return bf16_to_f32(f32_to_bf16(f)); }

enum { EPI_BIAS = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_ARGMAX = 3 };
#define GEMV_MAXK 8960
#define GEMV_MB 4

// RMSNorm (norm = true) or a plain copy of `rows` <= ROWS activation rows of length K into LDS
// as bf16 bits (row m at xs + m*K); 256 threads, K % 8 == 0, K <= 4096, 16-byte aligned rows.
// Two halves: rows_fetch issues the 16-byte loads of x and the norm weight (one round), and
// rows_finish reduces the sums of squares (DPP plus one LDS exchange) and writes LDS. A kernel
// issues its weight loads between the two, so the norm runs while the weights stream in.
template <int ROWS>
struct RowsPre {
  uint4 xv[ROWS][2], wn[2];
};

template <int ROWS>
__device__ __forceinline__ void rows_fetch(RowsPre<ROWS>& p, const uint16_t* x, long long ldx, int rows,
                                           const uint16_t* w, int K, bool norm) {
  const int K8 = K >> 3;
  const uint16_t* wsrc = norm ? w : x;   // a valid address either way; unused without the norm
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int i = threadIdx.x + c * 256;
    const bool in = i < K8;
    p.wn[c] = in ? *(const uint4*)(wsrc + 8 * i) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int m = 0; m < ROWS; ++m)
      p.xv[m][c] = in ? *(const uint4*)(x + min(m, rows - 1) * ldx + 8 * i) : make_uint4(0, 0, 0, 0);
  }
}

template <int ROWS>
__device__ __forceinline__ void rows_finish(const RowsPre<ROWS>& p, int rows, int K, float eps, int n_dtype,
                                            bool norm, uint16_t* xs) {
  __shared__ float red[4][ROWS];
  const int K8 = K >> 3;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (!norm) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int i = threadIdx.x + c * 256;
#pragma unroll
      for (int m = 0; m < ROWS; ++m)
        if (m < rows && i < K8) *(uint4*)(xs + m * K + 8 * i) = p.xv[m][c];
    }
    __syncthreads();
    return;
  }
  float ss[ROWS];
#pragma unroll
  for (int m = 0; m < ROWS; ++m) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint32_t q[4] = {p.xv[m][c].x, p.xv[m][c].y, p.xv[m][c].z, p.xv[m][c].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = bf16_to_f32((uint16_t)(q[j] & 0xffffu)), hi = bf16_to_f32((uint16_t)(q[j] >> 16));
        acc = fmaf(lo, lo, acc);
        acc = fmaf(hi, hi, acc);
      }
    }
    ss[m] = wave_sum(acc);
  }
  if (lane == 0)
#pragma unroll
    for (int m = 0; m < ROWS; ++m) red[wave][m] = ss[m];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < ROWS; ++m) {
    if (m >= rows) break;
    const float tot = (red[0][m] + red[1][m]) + (red[2][m] + red[3][m]);
    const float r = 1.0f / sqrtf(tot / (float)K + eps);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int i = threadIdx.x + c * 256;
      if (i >= K8) continue;
      const uint32_t q[4] = {p.xv[m][c].x, p.xv[m][c].y, p.xv[m][c].z, p.xv[m][c].w};
      const uint32_t g[4] = {p.wn[c].x, p.wn[c].y, p.wn[c].z, p.wn[c].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float n0 = round_to(bf16_to_f32((uint16_t)(q[j] & 0xffffu)) * r, n_dtype);
        const float n1 = round_to(bf16_to_f32((uint16_t)(q[j] >> 16)) * r, n_dtype);
        const uint16_t y0 = f32_to_bf16(bf16_to_f32((uint16_t)(g[j] & 0xffffu)) * n0);
        const uint16_t y1 = f32_to_bf16(bf16_to_f32((uint16_t)(g[j] >> 16)) * n1);
        o[j] = (uint32_t)y0 | ((uint32_t)y1 << 16);
      }
      *(uint4*)(xs + m * K + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int n) {
  uint32_t b = __float_as_uint(v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)b << 32) | (unsigned long long)(0xFFFFFFFFu - (uint32_t)n);
}

// Workgroups stride over blocks of 4*RPW weight rows (grid.x may be smaller than the
// number of blocks), so a prologue is computed once per workgroup, not once per block.
// x = the decode attention output, combined from its split partials (see attention.hip):
// x[h*128 + d] = round(sum_t e^(m_t - M_h) o_t[d] / sum_t e^(m_t - M_h) l_t)
// Wave w combines heads w, w+4, w+8, w+12; lane d holds dims d and d+64 of each. attn_fetch
// loads every partial the wave needs (its heads' o_t, and lane t's (m_t, l_t)) in one round,
// issued before the weight loads; attn_finish combines them while the weights stream in.
// At most T splits (8 or 16) and 16 heads (checked on the host).
template <int T>
struct AttnPre {
  uint32_t o[4][T];   // dims 2 lane, 2 lane + 1 of head j, split t (bf16 pair)
  float m[4], l[4];
};

template <int T>
__device__ __forceinline__ void attn_fetch(const GemvArgs& a, AttnPre<T>& p) {
  const int H = a.attn_heads, NT = a.attn_splits, G = a.attn_heads / a.attn_kvh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (wave + 4 * j >= H) break;   // wave-uniform
    const int h = wave + 4 * j, kvh = h / G, g = h % G;
    const uint32_t* po = (const uint32_t*)(a.attn_o + ((long long)kvh * NT * G + g) * 128) + lane;
#pragma unroll
    for (int t = 0; t < T; ++t)   // splits past NT repeat the last one (weight 0 below)
      p.o[j][t] = po[(long long)min(t, NT - 1) * G * 64];
    const float* ml = a.attn_ml + (((long long)kvh * NT + min(lane, NT - 1)) * G + g) * 2;
    p.m[j] = ml[0];
    p.l[j] = ml[1];
  }
}

template <int T>
__device__ __forceinline__ void attn_finish(const GemvArgs& a, const AttnPre<T>& p, uint16_t* xs) {
  const int H = a.attn_heads, NT = a.attn_splits;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = wave + 4 * j;
    if (h >= H) break;   // wave-uniform
    const float mj = (lane < NT && p.l[j] > 0.f) ? p.m[j] : -INFINITY;   // dead splits weigh 0
    const float M = wave_max(mj);
    const float f = (mj == -INFINITY) ? 0.f : __expf(mj - M);
    const float fl = f * p.l[j];   // weight of split lane's normalised output
    const float L = wave_sum(fl);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const float ft = HS_RL(fl, t);
      s0 = fmaf(ft, bf16_to_f32((uint16_t)(p.o[j][t] & 0xffffu)), s0);
      s1 = fmaf(ft, bf16_to_f32((uint16_t)(p.o[j][t] >> 16)), s1);
    }
    *(uint32_t*)&xs[h * 128 + 2 * lane] = f32_to_bf16(s0 / L) | ((uint32_t)f32_to_bf16(s1 / L) << 16);
  }
  __syncthreads();
}

enum { PRO_NONE = 0, PRO_NORM = 1, PRO_ATTN = 2, PRO_ATTN16 = 3 };   // ATTN: <= 8 splits, ATTN16: <= 16

// KS > 1: the 4 waves of a workgroup share the same RPW rows and split K (chunk c goes to
// wave c % 4); the per-wave partial sums are added in LDS. Used for long rows (K = 8960),
// so that each wave's loads for a row fit in one round.
template <int PRO, int EPI, int RPW, int MB, int KS = 1>
__device__ __forceinline__ void gemv_body(const GemvArgs& a) {
  constexpr bool NORM = PRO != PRO_NONE;   // x comes from LDS
  __shared__ __attribute__((aligned(16))) uint16_t xs[NORM ? MB * 3072 : 8];
  __shared__ unsigned long long best_w[EPI == EPI_ARGMAX ? 4 * MB : 1];
  __shared__ float kred[KS > 1 ? 4 * MB * RPW * 2 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long m0 = (long long)blockIdx.y * MB;
  const int mrows = (int)min((long long)MB, a.M - m0);
  constexpr int NW = (EPI == EPI_SILU) ? 2 : 1;
  const uint16_t* W[NW];
  W[0] = (const uint16_t*)a.w;
  if constexpr (EPI == EPI_SILU) W[1] = (const uint16_t*)a.w2;
  constexpr int ROWS_WG = KS > 1 ? RPW : 4 * RPW;
  const int nblocks = (a.N + ROWS_WG - 1) / ROWS_WG;
  const int kstart = (KS > 1 ? wave * 512 : 0) + lane * 8;
  unsigned long long best[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) best[m] = 0ull;

  // Rounds of U chunks: every weight load of a round is issued before any is consumed,
  // so a wave keeps U*RPW*NW 16-byte loads in flight instead of waiting on each. Behind a
  // prologue the loads carry no branch: chunks past K re-read the row's last 16 bytes (one
  // address for the whole wave), so the number of loads after the prologue's is fixed and
  // the prologue waits for its own loads only. Without one, chunks past K are skipped.
  constexpr int U = 12 / (RPW * NW) > 0 ? 12 / (RPW * NW) : 1;   // 12 x 16 B loads per lane per round
  uint4 wv[U][RPW][NW];
  int n0 = KS > 1 ? blockIdx.x * RPW : (blockIdx.x * 4 + wave) * RPW;
  auto load_round = [&](int kb) {
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const int k = kb + c * 512 * KS;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const long long n = min(n0 + r, a.N - 1);
#pragma unroll
        for (int u = 0; u < NW; ++u) {
          if constexpr (PRO != PRO_NONE)   // unconditional (offset clamped; the dot loop skips k >= K)
            wv[c][r][u] = ld_stream(W[u] + n * a.K + min(k, a.K - 8));
          else
            wv[c][r][u] = k < a.K ? ld_stream(W[u] + n * a.K + k) : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };
  // prologue loads first, then the first weight round; the prologue's math then runs while
  // the weights are in flight (loads complete in issue order)
  constexpr int AT = PRO == PRO_ATTN16 ? 16 : 8;
  RowsPre<MB> rpre_x;
  AttnPre<AT> apre;
  if constexpr (PRO == PRO_NORM)
    rows_fetch<MB>(rpre_x, (const uint16_t*)a.x + m0 * a.ldx, a.ldx, mrows, (const uint16_t*)a.norm_w, a.K, true);
  if constexpr (PRO >= PRO_ATTN) attn_fetch<AT>(a, apre);
  load_round(kstart);
  if constexpr (PRO != PRO_NONE) __builtin_amdgcn_sched_barrier(0);   // loads issued before the prologue math
  if constexpr (PRO == PRO_NORM) rows_finish<MB>(rpre_x, mrows, a.K, a.eps, a.n_dtype, true, xs);
  if constexpr (PRO >= PRO_ATTN) attn_finish<AT>(a, apre, xs);
  // absent epilogue operands read a valid dummy address (the weights), so the loads carry no
  // branch and no wait; their flags are applied where the values are used
  const uint16_t* bias_p = (a.flags & 1) ? (const uint16_t*)a.bias : W[0];
  const uint16_t* bias2_p = (EPI == EPI_SILU && (a.flags & 4)) ? (const uint16_t*)a.bias2 : W[0];
  const uint16_t* resid_p = EPI == EPI_RESID ? (const uint16_t*)a.resid : W[0];
  for (int blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
  n0 = KS > 1 ? blk * RPW : (blk * 4 + wave) * RPW;
  if (blk != (int)blockIdx.x) load_round(kstart);
  if (n0 >= a.N) continue;
  // epilogue operands are fetched now so their latency hides behind the weight stream
  uint16_t bpre[RPW], b2pre[RPW], rpre[MB][RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int n = min(n0 + r, a.N - 1);
    bpre[r] = bias_p[n];
    b2pre[r] = bias2_p[n];
#pragma unroll
    for (int m = 0; m < MB; ++m)
      rpre[m][r] = resid_p[EPI == EPI_RESID ? (m0 + min(m, mrows - 1)) * a.ldr + n : n];
  }
  float acc[MB][RPW][NW];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int u = 0; u < NW; ++u) acc[m][r][u] = 0.f;
  for (int kb = kstart; kb < a.K; kb += 512 * U * KS) {
    if (kb != kstart) load_round(kb);
    // activations from global memory: the whole round's chunks are loaded before any is used
    // (offsets clamped, no branch), so they take one round trip, not one per chunk
    uint4 xr[NORM ? 1 : MB][NORM ? 1 : U];
    if constexpr (!NORM) {
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int c = 0; c < U; ++c)
          xr[m][c] = *(const uint4*)((const uint16_t*)a.x + (m0 + min(m, mrows - 1)) * a.ldx +
                                     min(kb + c * 512 * KS, a.K - 8));
    }
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const int k = kb + c * 512 * KS;
      if (k >= a.K) break;
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if (m < mrows) {
          uint4 xv;
          if constexpr (NORM) xv = *(const uint4*)(xs + m * a.K + k);
          else xv = xr[m][c];
#pragma unroll
          for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < NW; ++u) acc[m][r][u] = dot8_bf16(xv, wv[c][r][u], acc[m][r][u]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int u = 0; u < NW; ++u) acc[m][r][u] = wave_sum(acc[m][r][u]);
  if constexpr (KS > 1) {   // add the four waves' K-partials (fixed order)
    if (lane == 0)
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
          for (int u = 0; u < NW; ++u) kred[((wave * MB + m) * RPW + r) * NW + u] = acc[m][r][u];
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int u = 0; u < NW; ++u) {
          const int o = (m * RPW + r) * NW + u, st = MB * RPW * NW;
          acc[m][r][u] = ((kred[o] + kred[st + o]) + kred[2 * st + o]) + kred[3 * st + o];
        }
    __syncthreads();
  }

#pragma unroll
  for (int m = 0; m < MB; ++m) {
    if (m >= mrows) continue;
    const long long mm = m0 + m;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = n0 + r;
      if (n >= a.N) continue;
      float v = acc[m][r][0];
      if (a.flags & 1) v += bf16_to_f32(bpre[r]);
      v = rbf(v);
      if constexpr (EPI == EPI_RESID) v = bf16_to_f32(rpre[m][r]) + v;
      if constexpr (EPI == EPI_SILU) {
        float u = acc[m][r][1];
        if (a.flags & 4) u += bf16_to_f32(b2pre[r]);
        u = rbf(u);
        const float s = rbf(v / (1.f + expf(-v)));
        v = s * u;
      }
      if (lane == 0 && (KS == 1 || wave == 0)) ((uint16_t*)a.out)[mm * a.ldo + n] = f32_to_bf16(v);
      if constexpr (EPI == EPI_ARGMAX) {
        const unsigned long long key = argmax_key(rbf(v), n);
        best[m] = key > best[m] ? key : best[m];
      }
    }
  }
  }  // row blocks
  if constexpr (EPI == EPI_ARGMAX) {
    // one key per (activation row, workgroup); k_argmax_finalize reduces them
    if (lane == 0)
#pragma unroll
      for (int m = 0; m < MB; ++m) best_w[wave * MB + m] = best[m];
    __syncthreads();
    if (threadIdx.x < (unsigned)mrows) {
      unsigned long long k = 0ull;
      for (int w = 0; w < 4; ++w) k = best_w[w * MB + threadIdx.x] > k ? best_w[w * MB + threadIdx.x] : k;
      a.argmax_slot[(m0 + threadIdx.x) * gridDim.x + blockIdx.x] = k;
    }
  }
}

#define GEMV_KERNEL(NAME, NORM, EPI, RPW, MB) \
  extern "C" __global__ void __launch_bounds__(256) NAME(const GemvArgs a) { gemv_body<NORM, EPI, RPW, MB>(a); }
#define GEMV_KERNEL_KS(NAME, NORM, EPI, RPW, MB) \
  extern "C" __global__ void __launch_bounds__(256) NAME(const GemvArgs a) { gemv_body<NORM, EPI, RPW, MB, 4>(a); }

GEMV_KERNEL_KS(k_gemv_resid_ks_r2, false, EPI_RESID, 2, 1)
GEMV_KERNEL_KS(k_gemv_bias_ks_r2, false, EPI_BIAS, 2, 1)

GEMV_KERNEL(k_gemv_bias_r1, false, EPI_BIAS, 1, 1)
GEMV_KERNEL(k_gemv_bias_r4, false, EPI_BIAS, 4, 1)
GEMV_KERNEL(k_gemv_resid_r1, false, EPI_RESID, 1, 1)
GEMV_KERNEL(k_gemv_norm_bias_r1, true, EPI_BIAS, 1, 1)
GEMV_KERNEL(k_gemv_norm_silu_r1, true, EPI_SILU, 1, 1)
GEMV_KERNEL(k_gemv_silu_r1, false, EPI_SILU, 1, 1)
GEMV_KERNEL(k_gemv_norm_argmax_r4, true, EPI_ARGMAX, 4, 1)
GEMV_KERNEL(k_gemv_argmax_r4, false, EPI_ARGMAX, 4, 1)
GEMV_KERNEL(k_gemv_bias_m4, false, EPI_BIAS, 2, 4)
GEMV_KERNEL(k_gemv_resid_m4, false, EPI_RESID, 2, 4)
GEMV_KERNEL(k_gemv_norm_bias_m4, true, EPI_BIAS, 2, 4)
GEMV_KERNEL(k_gemv_norm_silu_m4, true, EPI_SILU, 1, 4)
GEMV_KERNEL(k_gemv_silu_m4, false, EPI_SILU, 1, 4)
GEMV_KERNEL(k_gemv_attn_bias_r2, PRO_ATTN, EPI_BIAS, 2, 1)
GEMV_KERNEL(k_gemv_attn_resid_r2, PRO_ATTN, EPI_RESID, 2, 1)
GEMV_KERNEL(k_gemv_attn16_bias_r2, PRO_ATTN16, EPI_BIAS, 2, 1)
GEMV_KERNEL(k_gemv_attn16_resid_r2, PRO_ATTN16, EPI_RESID, 2, 1)

// ---------------------------------------------------------------- skinny MFMA GEMM (M <= 16 MT)
//
// out = epi(x . W^T) for a handful of activation rows: the weights are the HBM stream, read
// once, and each weight element meets all M rows in one v_mfma_f32_16x16x32_bf16 (A: 16 weight
// rows x 32 k, B: 32 k x 16 activation rows). Operand layout (gfx950 16x16x32): lane l holds 8
// consecutive k, at offset 8 (l / 16) of the step, of A row l % 16 and of B column l % 16; D
// element (4 (l / 16) + i, l % 16) is the lane's register i. Activation rows past M read row
// M - 1 and are not stored.
// Each wave streams its K steps through a ring of R stages in LDS: a stage is one 16-byte
// global-to-LDS load per lane for A and per 16-row activation tile, landing at the lane's own
// 16 bytes, so the lane reads its fragment back as it was loaded. The loads are issued from
// inline assembly and waited for explicitly (the compiler neither counts nor serialises them),
// R - 1 stages ahead of the step being multiplied.
//   SILU (k_skinny_silu_*): one wave per workgroup and per tile of 8 gate rows over the same 8
//   up rows, the whole of K; the up half of each output pair is swapped across the wave halves
//   and the SiLU * up row leaves from registers.
//   BIAS / RESID: 8 waves split K into 8 ranges over one tile of 16 output rows (or 8, RW == 8,
//   rows 8..15 repeating 0..7: twice the workgroups for a short N at no extra HBM bytes); the
//   wave tiles are added in LDS in wave order.
// Epilogues at the GEMV kernels' rounding points.
typedef __attribute__((ext_vector_type(8))) __bf16 sk_bf16x8;
typedef __attribute__((ext_vector_type(4))) float sk_f32x4;
typedef __attribute__((address_space(3))) uint4 sk_lds16;   // LDS reads as ds_read, not flat loads

__device__ __forceinline__ void sk_dma16(const void* g, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void sk_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
__device__ __forceinline__ void sk_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Stages [s0, s0 + ns) of 64 k each, of one wave, into acc. A stage is NA KB of weight rows
// (NA = 2: 16 rows; 1: 8 rows that stand for rows 8..15 too) and 2 KB per 16-row activation
// tile, each KB one global-to-LDS load of 8 rows x 128 contiguous bytes: lane l carries
// 16-byte chunk (l & 7) ^ (l >> 3) of row l >> 3, so chunk c of row r sits in slot
// c ^ (r & 7) of the row's 8 and the fragment reads of 8 consecutive rows hit 8 bank groups.
// The weights (HBM) run RA stages ahead in their ring, the activations RB <= RA in theirs.
// Issue order, oldest first: A 0 .. RA - RB - 1, then (B p, A RA - RB + p) for p < RB, then at
// step s (B s + RB, A s + RA); so when B s has landed, at most NA + (RB - 1) (NA + 2 MT) later
// loads are outstanding, and A s (older) has landed too. With RB == RA each step issues
// (A, B) and waits until at most (RA - 1) (NA + 2 MT) are outstanding.
// wr[j] / xr[t][j]: this lane's row of load j (element 0 of the row).
template <int MT, int NA, int RA, int RB>
__device__ __forceinline__ void sk_stream(const uint16_t* const (&wr)[2], const uint16_t* const (&xr)[MT][2], int s0,
                                          int ns, int rot, sk_lds16* ring, sk_f32x4 (&acc)[MT]) {
  static_assert(RB >= 1 && RB <= RA, "ring depths");
  constexpr int WAITN = RB == RA ? (RA - 1) * (NA + 2 * MT) : NA + (RB - 1) * (NA + 2 * MT);
  const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15;
  const int cl = 8 * ((lane & 7) ^ (lane >> 3));   // this lane's source chunk (elements)
  const unsigned abase = __builtin_amdgcn_readfirstlane((unsigned)(size_t)ring);
  const unsigned bbase = abase + RA * NA * 1024u;   // B ring behind the A ring
  // the wave's stages are visited from rot on (mod ns): workgroups that run side by side then
  // read different column ranges of their rows, which spreads them over the memory channels
  auto col = [&](int s) {
    const int j = min(s, ns - 1) + rot;
    return ((s0 + (j >= ns ? j - ns : j)) << 6) + cl;
  };
  auto issue_a = [&](int s, int slot) {   // stage s (clamped to the last) into A slot
    const int k = col(s);
#pragma unroll
    for (int j = 0; j < NA; ++j) sk_dma16(wr[j] + k, abase + (unsigned)(slot * NA + j) * 1024u);
  };
  auto issue_b = [&](int s, int slot) {
    const int k = col(s);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < 2; ++j) sk_dma16(xr[t][j] + k, bbase + (unsigned)(slot * 2 * MT + 2 * t + j) * 1024u);
  };
  // fragment slots (16-byte units) of MFMA step u: A row ra, B row r16, chunk 4 u + q
  const int ra = NA == 1 ? (r16 & 7) : r16;
  int fa[2], fb[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    fa[u] = (ra >> 3) * 64 + (ra & 7) * 8 + ((4 * u + q) ^ (ra & 7));
    fb[u] = RA * NA * 64 + (r16 >> 3) * 64 + (r16 & 7) * 8 + ((4 * u + q) ^ (r16 & 7));
  }
#pragma unroll
  for (int p = 0; p < RA - RB; ++p) issue_a(p, p);
#pragma unroll
  for (int p = 0; p < RB; ++p) {
    if (RB == RA) issue_a(p, p);
    issue_b(p, p);
    if (RB != RA) issue_a(RA - RB + p, RA - RB + p);
  }
  // A slots cycle with period RA, B slots with period RB: unroll over their common multiple
  constexpr int U = RA % RB == 0 ? RA : RA * RB;
  for (int j0 = 0; j0 < ns; j0 += U) {
#pragma unroll
    for (int p = 0; p < U; ++p) {
      sk_vmcnt<WAITN>();   // stage j0 + p has landed
      const int sa = p % RA, sb = p % RB;
      // a stage past the wave's last (its slots re-read the last one) is multiplied as zeros
      const unsigned ok = j0 + p < ns ? 0xFFFFFFFFu : 0u;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint4 av = ring[sa * NA * 64 + fa[u]];
        av = make_uint4(av.x & ok, av.y & ok, av.z & ok, av.w & ok);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint4 bv = ring[sb * 2 * MT * 64 + fb[u] + 128 * t];
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sk_bf16x8, av),
                                                           __builtin_bit_cast(sk_bf16x8, bv), acc[t], 0, 0, 0);
        }
      }
      sk_lgkm0();   // these slots' reads are done before they are refilled
      if (RB == RA) issue_a(j0 + p + RA, sa);
      issue_b(j0 + p + RB, sb);
      if (RB != RA) issue_a(j0 + p + RA, sa);
    }
  }
  sk_vmcnt<0>();
}

template <int MT, int RA, int RB>
__device__ __forceinline__ void skinny_silu_body(const GemvArgs& a) {
  __shared__ uint4 ring[(RA * 2 + RB * 2 * MT) * 64];
  const int lane = threadIdx.x & 63, q = lane >> 4, r16 = lane & 15, lr = lane >> 3;
  const int K = a.K, n0 = blockIdx.x * 8;
  // loads: j = 0 the 8 gate rows, j = 1 the 8 up rows; lane l carries row l >> 3 of each
  const long long wrow = (long long)min(n0 + lr, a.N - 1) * K;
  const uint16_t* wr[2] = {(const uint16_t*)a.w + wrow, (const uint16_t*)a.w2 + wrow};
  const uint16_t* xr[MT][2];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 2; ++j) xr[t][j] = (const uint16_t*)a.x + min((long long)(t * 16 + 8 * j + lr), a.M - 1) * a.ldx;
  sk_f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = sk_f32x4{0.f, 0.f, 0.f, 0.f};
  sk_stream<MT, 2, RA, RB>(wr, xr, 0, K >> 6, (int)(blockIdx.x % (unsigned)(K >> 6)), (sk_lds16*)ring, acc);
  // lanes 0..31 hold gate rows 4 q + i, lanes 32..63 the up rows 8 + 4 (q - 2) + i of the same
  // columns: lane l takes lane l + 32's
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float g[4], u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[i] = acc[t][i];
      u[i] = __shfl_xor(acc[t][i], 32, 64);
    }
    const int m = t * 16 + r16;
    if (lane < 32 && m < a.M) {
      uint16_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = min(n0 + 4 * q + i, a.N - 1);
        float v = g[i], uu = u[i];
        if (a.flags & 1) v += bf(a.bias, n);
        if (a.flags & 4) uu += bf(a.bias2, n);
        v = rbf(v);
        uu = rbf(uu);
        h[i] = f32_to_bf16(rbf(v / (1.f + expf(-v))) * uu);
      }
      uint16_t* o = (uint16_t*)a.out + (long long)m * a.ldo + n0 + 4 * q;
      if (n0 + 4 * q + 3 < a.N && (((a.ldo | n0) & 3) == 0)) {
        *(uint2*)o = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + 4 * q + i < a.N) o[i] = h[i];
      }
    }
  }
}

// BIAS / RESID: 8 waves split K into 8 ranges of one output tile; their fp32 tiles are added in
// LDS in wave order.
template <int EPI, int MT, int RW, int RA, int RB>
__device__ __forceinline__ void skinny_body(const GemvArgs& a) {
  constexpr int NA = RW == 8 ? 1 : 2;
  constexpr int RING = (RA * NA + RB * 2 * MT) * 64;   // uint4 per wave
  __shared__ uint4 ring[8 * RING];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15, lr = lane >> 3;
  const int K = a.K, stages = K >> 6;
  const int per = (stages + 7) >> 3, s0 = wave * per, ns = max(min(per, stages - s0), 0);
  const uint16_t* wr[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) wr[j] = (const uint16_t*)a.w + (long long)min(blockIdx.x * RW + 8 * j + lr, a.N - 1) * K;
  const uint16_t* xr[MT][2];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int j = 0; j < 2; ++j) xr[t][j] = (const uint16_t*)a.x + min((long long)(t * 16 + 8 * j + lr), a.M - 1) * a.ldx;
  sk_f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = sk_f32x4{0.f, 0.f, 0.f, 0.f};
  if (ns > 0)   // wave-uniform
    sk_stream<MT, NA, RA, RB>(wr, xr, s0, ns, (int)(blockIdx.x % (unsigned)ns), (sk_lds16*)ring + wave * RING, acc);
  __syncthreads();   // every wave is done with its ring: its tiles go there
  float* red = (float*)ring;   // [8][MT][256]
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * MT + t) * 256 + (4 * q + i) * 16 + r16] = acc[t][i];
  __syncthreads();
  constexpr int NO = RW == 8 ? 8 : 16;
  for (int e = tid; e < MT * NO * 16; e += 512) {
    const int t = e / (NO * 16), i = (e / 16) % NO, mc = e % 16, m = t * 16 + mc;
    const int nn = blockIdx.x * RW + i;
    if (m >= a.M || nn >= a.N) continue;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) v += red[(w * MT + t) * 256 + i * 16 + mc];
    if (a.flags & 1) v += bf(a.bias, nn);
    v = rbf(v);
    if constexpr (EPI == EPI_RESID) v = bf(a.resid, (long long)m * a.ldr + nn) + v;
    ((uint16_t*)a.out)[(long long)m * a.ldo + nn] = f32_to_bf16(v);
  }
}

// SILU with the RMSNorm of x folded in (k_skinny_silu_norm_*, M <= 16 and K <= 1536 or 2048, or
// M <= 32 and K <= 1536 with two 16-row activation tiles, MT = 2, and 4 weight stages): SKN_W
// waves per workgroup, one tile of 8 gate + 8 up rows each. The workgroup normalises the 16
// activation rows once into LDS, laid out as the stages sk_stream's activation ring would hold
// (stage s: 2 KB at s * 2 KB, chunk c of row r in slot c ^ (r & 7)), while the first weight
// stages stream in; the waves then stream only their weights (RA stages ahead) and read their
// activation fragments from that copy. The norm is the GEMV prologue's (rows_finish): fp32 sum of
// squares, x * rsqrt(mean + eps) rounded to n_dtype, times the weight rounded to bf16.
// LDS: 32 KMAX bytes of rows and SKN_W RA 2 KB of weight stages (KMAX = 1536: 144 KB, one
// workgroup per CU with 96 KB of weights in flight). The activation rows are loaded before the
// first weight stages, so the norm does not wait behind them (a CU's loads complete in order).
// Measured at cfg1 T = 16 (the block, this kernel and the down GEMM): 8 waves of 6 stages 22.3 us;
// 7 x 6 or 7 x 5 22.6, 8 x 7 22.9, 10 x 5 23.3, 6 x 7 23.4, 5 x 8 23.7, 4 x 8 or 4 x 12 (280
// workgroups for 256 CUs) 30.0; the norm as a launch of its own before k_skinny_silu_mt1: 24.4-26.5.
constexpr int SKN_W = 8, SKN_RA = 6;
template <int KMAX, int RA, int SKN_W = SKN_W, int MT = 1>
__device__ __forceinline__ void skinny_silu_norm_body(const GemvArgs& a) {
  constexpr int SKN_MAX_K = KMAX, ROWS = 16 * MT;
  __shared__ uint4 xsr[ROWS * KMAX / 8];        // the normalised rows, stage layout (MT tiles per stage)
  __shared__ uint4 ring[SKN_W][RA * 2 * 64];    // each wave's weight stages
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15, lr = lane >> 3;
  const int K = a.K, ns = K >> 6, KC = K >> 9;   // stages of 64 k; 512-element chunks per row
  const int tile = blockIdx.x * SKN_W + wave, n0 = tile * 8;
  const bool live = n0 < a.N;                    // (wave-uniform) waves past N only normalise
  const long long wrow = (long long)min(n0 + lr, a.N - 1) * K;
  const uint16_t* wr[2] = {(const uint16_t*)a.w + wrow, (const uint16_t*)a.w2 + wrow};
  const int cl = 8 * ((lane & 7) ^ (lane >> 3));
  const int rot = (int)((unsigned)tile % (unsigned)ns);
  const unsigned abase = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(sk_lds16*)ring[wave]);
  auto issue_a = [&](int s, int slot) {   // visit s (clamped to the last) into slot
    const int j = min(s, ns - 1) + rot, k = ((j >= ns ? j - ns : j) << 6) + cl;
#pragma unroll
    for (int j2 = 0; j2 < 2; ++j2) sk_dma16(wr[j2] + k, abase + (unsigned)(slot * 2 + j2) * 1024u);
  };
  // the norm: wave w takes rows NR w .. NR w + NR - 1 of the ROWS (rows past M repeat row M - 1),
  // lane l chunk 64 j + l of each (8 elements)
  {
    constexpr int MAXC = SKN_MAX_K / 512, NR = (ROWS + SKN_W - 1) / SKN_W;
    uint4 xv[NR][MAXC], gv[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
      const int k8 = min(c, KC - 1) * 64 + lane;
      gv[c] = *(const uint4*)((const uint16_t*)a.norm_w + 8 * k8);
#pragma unroll
      for (int i = 0; i < NR; ++i)
        xv[i][c] = *(const uint4*)((const uint16_t*)a.x + min((long long)min(NR * wave + i, ROWS - 1), a.M - 1) * a.ldx + 8 * k8);
    }
    if (live) {
#pragma unroll
      for (int p = 0; p < RA; ++p) issue_a(p, p);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      if (NR * wave + i >= ROWS) break;   // (wave-uniform) past the rows
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        if (c >= KC) break;
        const uint32_t w4[4] = {xv[i][c].x, xv[i][c].y, xv[i][c].z, xv[i][c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float lo = bf16_to_f32((uint16_t)(w4[j] & 0xffffu)), hi = bf16_to_f32((uint16_t)(w4[j] >> 16));
          acc = fmaf(lo, lo, acc);
          acc = fmaf(hi, hi, acc);
        }
      }
      const float tot = wave_sum(acc);
      const float r = 1.0f / sqrtf(tot / (float)K + a.eps);
      const int row = NR * wave + i;
#pragma unroll
      for (int c = 0; c < MAXC; ++c) {
        if (c >= KC) break;
        const uint32_t w4[4] = {xv[i][c].x, xv[i][c].y, xv[i][c].z, xv[i][c].w};
        const uint32_t g4[4] = {gv[c].x, gv[c].y, gv[c].z, gv[c].w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float m0 = round_to(bf16_to_f32((uint16_t)(w4[j] & 0xffffu)) * r, a.n_dtype);
          const float m1 = round_to(bf16_to_f32((uint16_t)(w4[j] >> 16)) * r, a.n_dtype);
          const uint16_t y0 = f32_to_bf16(bf16_to_f32((uint16_t)(g4[j] & 0xffffu)) * m0);
          const uint16_t y1 = f32_to_bf16(bf16_to_f32((uint16_t)(g4[j] >> 16)) * m1);
          o[j] = (uint32_t)y0 | ((uint32_t)y1 << 16);
        }
        const int k8 = c * 64 + lane, s = k8 >> 3, ch = k8 & 7;   // stage, chunk of the stage
        const int tr = row & 15;                                  // row of its 16-row tile
        xsr[(s * MT + (row >> 4)) * 128 + (tr >> 3) * 64 + (tr & 7) * 8 + (ch ^ (tr & 7))] =
            make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  }
  __syncthreads();
  if (!live) return;
  sk_f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = sk_f32x4{0.f, 0.f, 0.f, 0.f};
  int fa[2], fb[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    fa[u] = (r16 >> 3) * 64 + (r16 & 7) * 8 + ((4 * u + q) ^ (r16 & 7));
    fb[u] = (r16 >> 3) * 64 + (r16 & 7) * 8 + ((4 * u + q) ^ (r16 & 7));
  }
  const sk_lds16* rw = (const sk_lds16*)ring[wave];
  const sk_lds16* xw = (const sk_lds16*)xsr;
  for (int j0 = 0; j0 < ns; j0 += RA) {
#pragma unroll
    for (int p = 0; p < RA; ++p) {
      sk_vmcnt<(RA - 1) * 2>();   // visit j0 + p has landed
      const int v = j0 + p, jr = min(v, ns - 1) + rot, st = jr >= ns ? jr - ns : jr;
      const unsigned ok = v < ns ? 0xFFFFFFFFu : 0u;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint4 av = rw[p * 128 + fa[u]];
        av = make_uint4(av.x & ok, av.y & ok, av.z & ok, av.w & ok);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint4 bv = xw[(st * MT + t) * 128 + fb[u]];
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sk_bf16x8, av),
                                                           __builtin_bit_cast(sk_bf16x8, bv), acc[t], 0, 0, 0);
        }
      }
      sk_lgkm0();   // this slot's reads are done before it is refilled
      issue_a(v + RA, p);
    }
  }
  sk_vmcnt<0>();
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float g[4], u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[i] = acc[t][i];
      u[i] = __shfl_xor(acc[t][i], 32, 64);
    }
    const int m = t * 16 + r16;
    if (lane < 32 && m < a.M) {
      uint16_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = min(n0 + 4 * q + i, a.N - 1);
        float v = g[i], uu = u[i];
        if (a.flags & 1) v += bf(a.bias, n);
        if (a.flags & 4) uu += bf(a.bias2, n);
        v = rbf(v);
        uu = rbf(uu);
        h[i] = f32_to_bf16(rbf(v / (1.f + expf(-v))) * uu);
      }
      uint16_t* o = (uint16_t*)a.out + (long long)m * a.ldo + n0 + 4 * q;
      if (n0 + 4 * q + 3 < a.N && (((a.ldo | n0) & 3) == 0)) {
        *(uint2*)o = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n0 + 4 * q + i < a.N) o[i] = h[i];
      }
    }
  }
}

extern "C" __global__ void __launch_bounds__(512) k_skinny_silu_norm_mt2_k1536(const GemvArgs a) {
  skinny_silu_norm_body<1536, 4, 8, 2>(a);
}
extern "C" __global__ void __launch_bounds__(64 * SKN_W) k_skinny_silu_norm_mt1_k1536(const GemvArgs a) {
  skinny_silu_norm_body<1536, SKN_RA>(a);
}
extern "C" __global__ void __launch_bounds__(64 * SKN_W) k_skinny_silu_norm_mt1_k2048(const GemvArgs a) {
  skinny_silu_norm_body<2048, SKN_RA>(a);
}

// SILU over up to 16 MT activation rows (k_wide_silu_mt*, MT = 4 or 8: 33 to 128 rows): a
// workgroup of 4 waves owns TA tiles of 8 gate + 8 up rows (the tiles of k_skinny_silu_*) and all
// MT activation tiles. A K stage of 64 is TA 2 KB of weight rows and MT 2 KB of activation rows
// (1 KB = 8 rows x 128 B, chunk c of row r in slot c ^ (r & 7)); it lands in one of R LDS slots,
// R - 1 stages ahead of the one being multiplied, its 2 TA + 2 MT loads dealt round-robin to the
// 4 waves (UPW each; a wave with fewer repeats the stage's last load, so every wave waits for the
// same count). Per stage a wave waits for its own loads of the stage, then one barrier makes the
// whole stage visible and frees the slot read one stage before, which the next issue refills.
// Wave w multiplies every weight tile of the stage by activation tiles w MT / 4 .. (w + 1) MT / 4
// - 1. Every weight element is read from HBM once; the activation rows (L2-resident) once per
// workgroup. Per CU that is 3 KB x K / 1536 per weight or activation row: at K = 1536, TA = 5,
// MT = 8, 80 weight rows and 128 activation rows, 624 KB.
// HALVES = 2: the rows split in two halves of 16 MT between two workgroups over the same weight
// tiles; workgroups b and b + 8 (dispatched to the same XCD, whose L2 then serves the second
// reader of each weight row) take the halves of tile group (b / 16) 8 + b % 8.
template <int MT, int TA, int R, int HALVES = 1>
__device__ __forceinline__ void wide_silu_body(const GemvArgs& a) {
  constexpr int TW = MT / 4, U = 2 * TA + 2 * MT, UPW = (U + 3) / 4, SLOT = U * 64;   // SLOT: uint4
  static_assert(MT % 4 == 0 && R >= 2, "shape");
  __shared__ uint4 ring[R * SLOT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15, lr = lane >> 3;
  const int bx = (int)blockIdx.x;
  const int grp = HALVES == 1 ? bx : ((bx >> 4) << 3) | (bx & 7), m0 = HALVES == 1 ? 0 : ((bx >> 3) & 1) * 16 * MT;
  const int K = a.K, ns = K >> 6, p0 = grp * TA * 8;   // stages; first output pair
  if (HALVES > 1 && (p0 >= a.N || m0 >= a.M)) return;   // (workgroup-uniform) past the tile groups or rows
  const int cl = 8 * ((lane & 7) ^ lr);                        // this lane's source chunk (elements)
  const uint16_t* src[UPW];
  unsigned dst[UPW];
  const unsigned base = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(sk_lds16*)ring);
#pragma unroll
  for (int j = 0; j < UPW; ++j) {
    const int u = min(wave + 4 * j, U - 1);
    if (u < 2 * TA) {   // weight tile u / 2, gate (u even) or up rows
      const long long row = min(p0 + 8 * (u >> 1) + lr, a.N - 1);
      src[j] = (const uint16_t*)((u & 1) ? a.w2 : a.w) + row * K + cl;
    } else {            // activation tile (u - 2 TA) / 2, rows 8 ((u - 2 TA) & 1) ..
      const int v = u - 2 * TA;
      src[j] = (const uint16_t*)a.x + min((long long)(m0 + 16 * (v >> 1) + 8 * (v & 1) + lr), a.M - 1) * a.ldx + cl;
    }
    dst[j] = __builtin_amdgcn_readfirstlane(base + (unsigned)u * 1024u);
  }
  auto issue = [&](int s) {   // stage s (clamped to the last) into slot s % R
    const int k = min(s, ns - 1) << 6;
    const unsigned so = (unsigned)(s % R) * (unsigned)SLOT * 16u;
#pragma unroll
    for (int j = 0; j < UPW; ++j) sk_dma16(src[j] + k, dst[j] + so);
  };
  int fa[2], fb[2];   // fragment slots (uint4) of MFMA step u within a 2-unit tile
#pragma unroll
  for (int u = 0; u < 2; ++u) fa[u] = fb[u] = (r16 >> 3) * 64 + (r16 & 7) * 8 + ((4 * u + q) ^ (r16 & 7));
  sk_f32x4 acc[TA][TW];
#pragma unroll
  for (int t = 0; t < TA; ++t)
#pragma unroll
    for (int i = 0; i < TW; ++i) acc[t][i] = sk_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < R - 1; ++p) issue(p);
  // The fragments of stage s are read from LDS while the MFMAs of stage s - 1 run on the
  // registers read the step before (one wave per SIMD: nothing else hides the LDS latency).
  const sk_lds16* rl = (const sk_lds16*)ring;
  uint4 av[2][2][TA], bv[2][2][TW];   // [register set][k half][tile]
  auto read = [&](int slot, int set) {
    const sk_lds16* st = rl + slot * SLOT;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int i = 0; i < TW; ++i) bv[set][u][i] = st[(2 * TA + 2 * (wave * TW + i)) * 64 + fb[u]];
#pragma unroll
      for (int t = 0; t < TA; ++t) av[set][u][t] = st[2 * t * 64 + fa[u]];
    }
  };
  auto mfma = [&](int set) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < TA; ++t)
#pragma unroll
        for (int i = 0; i < TW; ++i)
          acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sk_bf16x8, av[set][u][t]),
                                                              __builtin_bit_cast(sk_bf16x8, bv[set][u][i]), acc[t][i], 0, 0, 0);
  };
  static_assert(R % 2 == 0, "register sets alternate with the stage parity");
  for (int s0 = 0; s0 < ns; s0 += R) {
#pragma unroll
    for (int p = 0; p < R; ++p) {
      if (s0 + p >= ns) break;   // (uniform)
      sk_vmcnt<(R - 2) * UPW>();   // this wave's loads of stage s0 + p have landed
      sk_lgkm0();                  // and its reads of the stage before are in registers
      __syncthreads();             // every wave's: the stage is in LDS, slot (p - 1) % R is free
      issue(s0 + p + R - 1);
      read(p, p & 1);
      if (s0 + p > 0) mfma((p & 1) ^ 1);   // stage s0 + p - 1
    }
  }
  sk_lgkm0();
  if ((ns - 1) & 1)   // (uniform) register set of the last stage, a constant index either way
    mfma(1);
  else
    mfma(0);
  sk_vmcnt<0>();   // the clamped tail loads land before the workgroup's LDS is released
  // lanes 0..31 hold gate rows 4 q + i of the tile, lanes 32..63 the up rows of the same pairs
#pragma unroll
  for (int t = 0; t < TA; ++t) {
    const int n0 = p0 + 8 * t;
#pragma unroll
    for (int i2 = 0; i2 < TW; ++i2) {
      float g[4], u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[i] = acc[t][i2][i];
        u[i] = __shfl_xor(acc[t][i2][i], 32, 64);
      }
      const int m = m0 + (wave * TW + i2) * 16 + r16;
      if (lane < 32 && m < a.M && n0 < a.N) {
        uint16_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = min(n0 + 4 * q + i, a.N - 1);
          float v = g[i], uu = u[i];
          if (a.flags & 1) v += bf(a.bias, n);
          if (a.flags & 4) uu += bf(a.bias2, n);
          v = rbf(v);
          uu = rbf(uu);
          h[i] = f32_to_bf16(rbf(v / (1.f + expf(-v))) * uu);
        }
        uint16_t* o = (uint16_t*)a.out + (long long)m * a.ldo + n0 + 4 * q;
        if (n0 + 4 * q + 3 < a.N && (((a.ldo | n0) & 3) == 0)) {
          *(uint2*)o = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (n0 + 4 * q + i < a.N) o[i] = h[i];
        }
      }
    }
  }
}

// Measured on the cfg1 block (norm, this kernel, the down GEMM and its reduce) on MI355X, against
// the 64 x 64 SiLU GEMM tiles it replaces: T = 48 31.1 us against 31.9, T = 64 31.3 / 31.9, T = 100
// 37.6-38.1 / 38.7, T = 128 37.7-39.0 / 39.0-39.5 (4 stages; 6 stages 39.3-39.8). 3 or 4 weight
// tiles per workgroup (374 or 280 workgroups) 47.1 and 50.5, 7 (160) 44.9. What bounds it is each
// CU's intake of 624 KB at 30-37 GB/s: with the MFMAs taken out (loads and fragment reads only) the
// block took 37.4 us, and overlapping the fragment reads with the previous stage's MFMAs (below)
// did not change the time. Two 64-row workgroups per tile group (HALVES = 2, k_wide_silu_mt4x2,
// two per CU): the block at T = 100 36.9-37.2 us and at T = 128 37.8-38.1, against 37.6-38.1 and
// 38.3-38.5 with one 128-row workgroup.
#ifndef WIDE_TA
#define WIDE_TA 5
#endif
#ifndef WIDE_R8
#define WIDE_R8 4
#endif
#ifndef WIDE_R4
#define WIDE_R4 8
#endif
extern "C" __global__ void __launch_bounds__(256) k_wide_silu_mt8(const GemvArgs a) {
  wide_silu_body<8, WIDE_TA, WIDE_R8>(a);
}
extern "C" __global__ void __launch_bounds__(256) k_wide_silu_mt4(const GemvArgs a) {
  wide_silu_body<4, WIDE_TA, WIDE_R4>(a);
}
#ifndef WIDE_RH
#define WIDE_RH 4
#endif
extern "C" __global__ void __launch_bounds__(256) k_wide_silu_mt4x2(const GemvArgs a) {
  wide_silu_body<4, WIDE_TA, WIDE_RH, 2>(a);
}

#define SKINNY_SILU(NAME, MT, RA, RB) \
  extern "C" __global__ void __launch_bounds__(64) NAME(const GemvArgs a) { skinny_silu_body<MT, RA, RB>(a); }
#define SKINNY_KERNEL(NAME, EPI, MT, RW, RA, RB) \
  extern "C" __global__ void __launch_bounds__(512) NAME(const GemvArgs a) { skinny_body<EPI, MT, RW, RA, RB>(a); }
// ring depths (stages of weights, stages of activations) measured at M = 16 on MI355X: deeper
// rings were slower (gate/up 12.6 us with 6 stages, 12.9 with 7, 14.5 with 8; down 8.5 us with
// 4..6 and 10.2..13.8 with 12 weight stages ahead of 3 activation stages)
SKINNY_SILU(k_skinny_silu_mt1, 1, 6, 6)
SKINNY_SILU(k_skinny_silu_mt2, 2, 4, 4)
SKINNY_KERNEL(k_skinny_bias_mt1, EPI_BIAS, 1, 16, 4, 4)
SKINNY_KERNEL(k_skinny_bias_mt2, EPI_BIAS, 2, 16, 3, 3)
SKINNY_KERNEL(k_skinny_resid_mt1, EPI_RESID, 1, 16, 4, 4)
SKINNY_KERNEL(k_skinny_resid_mt2, EPI_RESID, 2, 16, 3, 3)
SKINNY_KERNEL(k_skinny_bias_mt1_r8, EPI_BIAS, 1, 8, 5, 5)
SKINNY_KERNEL(k_skinny_bias_mt2_r8, EPI_BIAS, 2, 8, 3, 3)
SKINNY_KERNEL(k_skinny_resid_mt1_r8, EPI_RESID, 1, 8, 5, 5)
SKINNY_KERNEL(k_skinny_resid_mt2_r8, EPI_RESID, 2, 8, 3, 3)

// One workgroup per activation row: the largest of the row's per-workgroup keys is the
// maximum logit with the smallest index among equal maxima (np.argmax's rule).
extern "C" __global__ void __launch_bounds__(256) k_argmax_finalize(const ArgmaxFinalizeArgs a) {
  argmax_finalize_body(a, blockIdx.x);
}

// ------------------------------------------------------------------------ q/k/v + RoPE + cache

// One wave per task; a task is a pair of weight rows:
//   q and k: rows (h*D + j, h*D + j + D/2) of one head, rotated together;
//   v:       rows (2t, 2t+1), plain.
// QC: 16-byte chunks of 512 elements per weight row and lane (K <= 512 * QC)
template <int QC>
__device__ __forceinline__ void qkv_body(const QKVArgs& a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[3072];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int D = a.D, half = a.D / 2;
  const int tq = a.H * half, tk = a.KVH * half, tv = a.KVH * D / 2;
  const int t0 = blockIdx.x * 4 + wave;
  const bool active = t0 < tq + tk + tv;
  const int t = active ? t0 : 0;
  int seg, r0, r1;
  const uint16_t* W;
  const void* B;
  if (t < tq) {
    seg = 0; W = (const uint16_t*)a.wq; B = a.bq;
    r0 = (t / half) * D + (t % half); r1 = r0 + half;
  } else if (t < tq + tk) {
    seg = 1; W = (const uint16_t*)a.wk; B = a.bk;
    const int u = t - tq;
    r0 = (u / half) * D + (u % half); r1 = r0 + half;
  } else {
    seg = 2; W = (const uint16_t*)a.wv; B = a.bv;
    const int u = t - tq - tk;
    r0 = 2 * u; r1 = 2 * u + 1;
  }
  // Loads in issue order: the activation row and norm weight (the prologue) and the rotary
  // operands, the weight rows (QC chunks of 512 per row), then the bias as
  // raw bits with no branch. Loads complete in order, so the norm and the rotary factors
  // wait only for their own loads and are computed while the weights stream in.
  const bool norm = (a.flags & 1) != 0;
  RowsPre<1> xp;
  rows_fetch<1>(xp, (const uint16_t*)a.x, 0, 1, (const uint16_t*)a.norm_w, a.K, norm);
  const IRaw pos_r = ld_i_raw(a.pos_ids, 0, a.pos_dtype);
  const IRaw cpos_r = ld_i_raw(a.cache_pos, 0, a.cpos_dtype);
  const float invf = a.inv_freq[(r0 % D) % half];
  uint4 w0[QC], w1[QC];
#pragma unroll
  for (int c = 0; c < QC; ++c) {   // no branch: chunks past K re-read the row's last 16 bytes
    const int k = min(lane * 8 + c * 512, a.K - 8);
    w0[c] = ld_stream(W + (long long)r0 * a.K + k);
    w1[c] = ld_stream(W + (long long)r1 * a.K + k);
  }
  const uint16_t* Bp = (a.flags & 2) ? (const uint16_t*)B : W;   // W: a valid dummy address
  const uint16_t b0r = Bp[r0], b1r = Bp[r1];
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the arithmetic below
  // rotary factors of angle inv_freq * position (fp32 product, as the reference forms it),
  // computed for every task with no branch or table load, so that neither the frequency load
  // nor a wait moves behind the weight loads; tasks without rotation ignore them
  const long long pos_v = ld_i_decode(pos_r, a.pos_dtype);
  float sf, cf;
  sincos_rot(invf * (float)pos_v, &sf, &cf);
  // an empty use keeps the factors here: otherwise they are sunk into the lane-0 epilogue and
  // computed after the dot products, on the kernel's critical path
  asm volatile("" ::"v"(sf), "v"(cf));
  rows_finish<1>(xp, 1, a.K, a.eps, a.n_dtype, norm, xs);
  if (!active) return;
  const long long cpos_v = ld_i_decode(cpos_r, a.cpos_dtype);
  const float b0 = (a.flags & 2) ? bf16_to_f32(b0r) : 0.f, b1 = (a.flags & 2) ? bf16_to_f32(b1r) : 0.f;
  const bool rope = (seg == 0 && (a.flags & 4)) || (seg == 1 && (a.flags & 8));
  const float rc = round_to(cf * a.rope_scaling, HS_BF16), rs = round_to(sf * a.rope_scaling, HS_BF16);
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int c = 0; c < QC; ++c) {
    const int k = lane * 8 + c * 512;
    if (k < a.K) {
      const uint4 xv = *(const uint4*)(xs + k);
      acc0 = dot8_bf16(xv, w0[c], acc0);
      acc1 = dot8_bf16(xv, w1[c], acc1);
    }
  }
  acc0 = wave_sum(acc0);
  acc1 = wave_sum(acc1);
  if (lane != 0) return;
  acc0 += b0;
  acc1 += b1;
  float v0 = rbf(acc0), v1 = rbf(acc1);
  if (rope) {
    const float c = rc, s = rs;
    const float e0 = rbf(rbf(v0 * c) + rbf(-v1 * s));   // x[j]*cos + (-x[j+D/2])*sin
    const float e1 = rbf(rbf(v1 * c) + rbf(v0 * s));    // x[j+D/2]*cos + x[j]*sin
    v0 = e0;
    v1 = e1;
  }
  if (seg == 0) {
    ((uint16_t*)a.q_out)[r0] = f32_to_bf16(v0);
    ((uint16_t*)a.q_out)[r1] = f32_to_bf16(v1);
    return;
  }
  const bool to_cache = (seg == 1) ? (a.flags & 16) : (a.flags & 32);
  void* dst = seg == 1 ? a.k_dst : a.v_dst;
  if (to_cache) {
    if (cpos_v < 0 || cpos_v >= a.cache_len) return;
    const long long o0 = (long long)(r0 / D) * a.kv_head_stride + cpos_v * D;
    const long long o1 = (long long)(r1 / D) * a.kv_head_stride + cpos_v * D;
    ((uint16_t*)dst)[o0 + r0 % D] = f32_to_bf16(v0);
    ((uint16_t*)dst)[o1 + r1 % D] = f32_to_bf16(v1);
  } else {
    ((uint16_t*)dst)[r0] = f32_to_bf16(v0);
    ((uint16_t*)dst)[r1] = f32_to_bf16(v1);
  }
}

extern "C" __global__ void __launch_bounds__(256) k_qkv_rope(const QKVArgs a) { qkv_body<6>(a); }       // K <= 3072
extern "C" __global__ void __launch_bounds__(256) k_qkv_rope_k1536(const QKVArgs a) { qkv_body<3>(a); } // K <= 1536

// ------------------------------------------------------------------ prefill RoPE + K/V cache rows
//
// One wave per (token t, slot): slots 0..H-1 are q heads, H..H+KVH-1 k heads, then v heads.
// Lane d takes the rotate-half pair (d, d + D/2) of the row:
//   out[d] = r(r(x[d] c) + r(-x[d + D/2] s)),  out[d + D/2] = r(r(x[d + D/2] c) + r(x[d] s))
// with c, s = r(cos / sin(inv_freq[d] * pos[t]) * scaling) and r() the model dtype's rounding:
// q*cos + rotate_half(q)*sin as the reference's graph evaluates it, op by op. q goes to
// [H, T, D]; k (rotated) and v to their caches at row cache_pos[t] (an in-place index_copy).
extern "C" __global__ void __launch_bounds__(256) k_rope_cache(const RopeCacheArgs a) {
  const int lane = threadIdx.x & 63;
  const int slots = a.H + 2 * a.KVH, half = a.D / 2;
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= (long long)a.T * slots) return;
  const int t = (int)(row / slots), slot = (int)(row % slots);
  const int seg = slot < a.H ? 0 : (slot < a.H + a.KVH ? 1 : 2);
  const int hd = seg == 0 ? slot : (seg == 1 ? slot - a.H : slot - a.H - a.KVH);
  if (lane >= half) return;
  const long long col = (long long)slot * a.D;   // q | k | v heads are consecutive D-wide column blocks
  const uint16_t* yr = (const uint16_t*)a.y + (long long)t * a.ldy + col;
  const bool f16 = a.dtype == HS_F16;
  auto ld = [&](int d) { return f16 ? f16_to_f32(yr[d]) : bf16_to_f32(yr[d]); };
  auto rd = [&](float f) { return round_to(f, a.dtype); };
  auto pk = [&](float f) { return f16 ? f32_to_f16(f) : f32_to_bf16(f); };
  float v0 = ld(lane), v1 = ld(lane + half);
  const bool rope = (seg == 0 && (a.flags & 4)) || (seg == 1 && (a.flags & 8));
  if (rope) {
    const long long pos = ld_i(a.pos_ids, t, a.pos_dtype);
    float sf, cf;
    sincos_rot(a.inv_freq[lane] * (float)pos, &sf, &cf);
    const float c = rd(cf * a.rope_scaling), s = rd(sf * a.rope_scaling);
    const float e0 = rd(rd(v0 * c) + rd(-v1 * s));
    const float e1 = rd(rd(v1 * c) + rd(v0 * s));
    v0 = e0;
    v1 = e1;
  }
  uint16_t* dst;
  if (seg == 0) {
    dst = (uint16_t*)a.q_out + ((long long)hd * a.T + t) * a.D;
  } else {
    const bool to_cache = seg == 1 ? (a.flags & 16) : (a.flags & 32);
    long long r = t;
    if (to_cache) {
      r = ld_i(a.cache_pos, t, a.cpos_dtype);
      if (r < 0 || r >= a.cache_len) return;
    }
    dst = (uint16_t*)(seg == 1 ? a.k_dst : a.v_dst) + (long long)hd * a.kv_head_stride + r * a.D;
  }
  dst[lane] = pk(v0);
  dst[lane + half] = pk(v1);
}

// ------------------------------------------------------------------ argmax over long rows
//
// k_argmax_part: grid (parts, rows), 256 threads; k_argmax_finalize: one workgroup per row.
// The bodies (argmax_part_body / argmax_finalize_body in common.h) are shared with the shim's
// hs_argmax_rows entry points.
extern "C" __global__ void __launch_bounds__(256) k_argmax_part(const ArgmaxPartArgs a) {
  argmax_part_body(a, blockIdx.x, blockIdx.y);
}
