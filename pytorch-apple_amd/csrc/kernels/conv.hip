// conv2d as an implicit GEMM on MFMA (gfx950 v_mfma_f32_32x32x16_{f16,bf16}), NCHW / OIHW.
//
//   C[m, co] = sum_k A[m, k] B[co, k]   m = (n, ho, wo), k = (ci, kh, kw), K = Cin*KH*KW
//   A[m, k]  = x[n, ci, ho*sh - ph + kh, wo*sw - pw + kw]   (0 outside the image)
//   B[co, k] = w[co, ci, kh, kw]                            (OIHW rows are K-contiguous)
// Workgroup tile 128 pixels x 128 output channels, K step 32, 256 threads as 2 x 2 waves
// of 64 x 64 (the same fragment layout as gemm.hip). A is gathered straight from the
// NCHW activations: thread t owns pixel t % 128 and 16 consecutive k of the step, so a
// wave's loads for one k walk 64 neighbouring pixels (contiguous for stride 1); the k ->
// (ci, kh, kw) decomposition is advanced incrementally, not divided per element. B rows
// are read with 16-byte loads when K % 8 == 0 (every conv but a 3-channel stem).
// Epilogue per (pixel, channel), the CPU path's rounding points:
//   v = round(acc (+ bias));  batch norm: v = round(v * a_c + b_c), a_c = w_c / sqrt(var_c + eps),
//   b_c = bias_c - mean_c * a_c;  residual: v = round(v + r);  ReLU: v = max(v, 0).
#include "common.h"

typedef __attribute__((ext_vector_type(8))) __bf16 cv_bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 cv_f16x8;
typedef __attribute__((ext_vector_type(16))) float cv_f32x16;

#define CV_BM 128
#define CV_BN 128
#define CV_BK 32
#define CV_LDS_K 40

template <int DT>
__device__ __forceinline__ cv_f32x16 cv_mfma(const uint4 a, const uint4 b, cv_f32x16 c) {
  if constexpr (DT == HS_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(cv_bf16x8, a), __builtin_bit_cast(cv_bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(cv_f16x8, a), __builtin_bit_cast(cv_f16x8, b),
                                                  c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ float cv_f(uint16_t h) {
  return DT == HS_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}
template <int DT>
__device__ __forceinline__ uint16_t cv_h(float f) {
  return DT == HS_BF16 ? f32_to_bf16(f) : f32_to_f16(f);
}
template <int DT>
__device__ __forceinline__ float cv_round(float f) {
  return cv_f<DT>(cv_h<DT>(f));
}

// KS: 1 = 1x1 kernel without padding (A is one strided plane read per k), 3 = 3x3, 0 = any
template <int DT, bool BVEC, int KS = 0>
__device__ __forceinline__ void conv_body(const ConvArgs& a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][CV_BM][CV_LDS_K];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][CV_BN][CV_LDS_K];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  // XCD-aware tile order (workgroup L runs on XCD L % 8): each XCD gets a contiguous range of
  // tiles, output-channel tiles fastest, so the channel tiles that share one gathered pixel
  // tile run back to back on the same XCD and find it in its L2
  const unsigned gx = gridDim.x, gy = gridDim.y;
  const unsigned total = gx * gy * gridDim.z;
  const unsigned lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const unsigned per = (total + 7) / 8, xcd = lin % 8, loc = lin / 8;
  const unsigned tall = total % 8 == 0 ? 8 : total % 8;
  const unsigned tile = xcd < tall ? xcd * per + loc : tall * per + (xcd - tall) * (per - 1) + loc;
  const unsigned tn = tile % gx, tm = (tile / gx) % gy, tkz = tile / (gx * gy);
  const long long m_base = (long long)tm * CV_BM;
  const int n_base = tn * CV_BN;
  const uint16_t* X = (const uint16_t*)a.x;
  const uint16_t* Wt = (const uint16_t*)a.w;
  const int HW = a.H * a.W;

  // this thread's A pixel and k range within a step. The 16 k of a thread are the same for
  // the whole wave (akg = wave / 2), so their (ci, kh, kw) decomposition is scalar work, and
  // each element costs one vector add, a validity test and the load.
  const int am = tid & (CV_BM - 1);
  const int akg = __builtin_amdgcn_readfirstlane(tid >> 7);
  const int M32 = (int)a.M;
  const int mg = min((int)m_base + am, M32 - 1);   // rows past M read a valid pixel; never stored
  const int HoWo = a.Ho * a.Wo;
  const int mn = mg / HoWo, mp = mg - mn * HoWo;
  const int hi0 = (mp / a.Wo) * a.sh - a.ph, wi0 = (mp % a.Wo) * a.sw - a.pw;
  const int pix = mn * a.Cin * HW + hi0 * a.W + wi0;   // element offset of (n, ci = 0, hi0, wi0); < 2^31
  // byte offsets from the (uniform) tensor base: 32-bit unsigned, so every load is
  // base + one vector add (the input is < 4 GiB; the host checks)
  const char* Xb = (const char*)a.x;
  const uint32_t HWb = (uint32_t)HW * 2u;
  // 3x3: bit kh * 3 + kw set when the tap (kh, kw) of this pixel is inside the image
  unsigned tapmask = 0;
  if constexpr (KS == 3) {
#pragma unroll
    for (int kh = 0; kh < 3; ++kh)
#pragma unroll
      for (int kw = 0; kw < 3; ++kw)
        if ((unsigned)(hi0 + kh) < (unsigned)a.H && (unsigned)(wi0 + kw) < (unsigned)a.W)
          tapmask |= 1u << (kh * 3 + kw);
  }

  uint32_t ra[8];    // 16 gathered A values, packed in pairs
  uint4 rb[2];       // B: 2 x 16 bytes (BVEC) ...
  uint32_t rbs[16];  // ... or 16 gathered values packed in pairs
  auto load_a = [&](int k0, uint32_t (&dst)[8]) {
    const int kb = __builtin_amdgcn_readfirstlane(k0 + akg * 16);
    if constexpr (KS == 1) {   // K % 32 == 0 and no padding (the host checks): every element is in range
      const uint32_t o0 = (uint32_t)pix * 2u + (uint32_t)kb * HWb;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint16_t v = *(const uint16_t*)(Xb + (o0 + (uint32_t)j * HWb));
        if (j & 1) dst[j >> 1] |= (uint32_t)v << 16;
        else dst[j >> 1] = v;
      }
    } else {
      const int KWr = KS == 3 ? 3 : a.KW, KHr = KS == 3 ? 3 : a.KH;
      int ci = kb / (KHr * KWr), r = kb - ci * (KHr * KWr), kh = r / KWr, kw = r - kh * KWr;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int k = kb + j;
        const int tap = kh * KWr + kw;
        const int so = ci * HW + kh * a.W + kw;   // scalar part of the offset
        bool ok;
        if constexpr (KS == 3) ok = k < a.K && ((tapmask >> tap) & 1u);
        else ok = k < a.K && (unsigned)(hi0 + kh) < (unsigned)a.H && (unsigned)(wi0 + kw) < (unsigned)a.W;
        // padded taps read element 0 (in bounds) and are replaced by 0
        const uint16_t ld = *(const uint16_t*)(Xb + (ok ? (uint32_t)(pix + so) * 2u : 0u));
        const uint16_t v = ok ? ld : (uint16_t)0;
        if (j & 1) dst[j >> 1] |= (uint32_t)v << 16;
        else dst[j >> 1] = v;
        if (++kw == KWr) {
          kw = 0;
          if (++kh == KHr) { kh = 0; ++ci; }
        }
      }
    }
  };
  // B staging: thread t -> channel row (t >> 2) and (t >> 2) + 64, 8 consecutive k at (t & 3) * 8
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = (tid >> 2) + 64 * i, col = (tid & 3) * 8;
      const int co = min(n_base + row, a.Cout - 1);
      const int k = k0 + col;
      if constexpr (BVEC) {
        rb[i] = k < a.K ? *(const uint4*)(Wt + (long long)co * a.K + k) : make_uint4(0, 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const uint16_t lo = (k + j < a.K) ? Wt[(long long)co * a.K + k + j] : 0;
          const uint16_t hi = (k + j + 1 < a.K) ? Wt[(long long)co * a.K + k + j + 1] : 0;
          rbs[i * 4 + j / 2] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
      }
    }
  };
  auto store = [&](int buf) {
    *(uint4*)&As[buf][am][akg * 16] = make_uint4(ra[0], ra[1], ra[2], ra[3]);
    *(uint4*)&As[buf][am][akg * 16 + 8] = make_uint4(ra[4], ra[5], ra[6], ra[7]);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = (tid >> 2) + 64 * i, col = (tid & 3) * 8;
      if constexpr (BVEC) *(uint4*)&Bs[buf][row][col] = rb[i];
      else *(uint4*)&Bs[buf][row][col] = make_uint4(rbs[i * 4], rbs[i * 4 + 1], rbs[i * 4 + 2], rbs[i * 4 + 3]);
    }
  };

  cv_f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // split K: workgroup z covers k in [z * kchunk, min(K, (z + 1) * kchunk))
  const int kz = (int)tkz;
  const int kbeg = kz * a.kchunk;
  const int nsteps = (min(a.K - kbeg, a.kchunk) + CV_BK - 1) / CV_BK;
  load_a(kbeg, ra);
  load_b(kbeg);
  store(0);
  __syncthreads();
  const int fr = lane & 31, fk = (lane >> 5) * 8;
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    if (s + 1 < nsteps) {
      load_a(kbeg + (s + 1) * CV_BK, ra);
      load_b(kbeg + (s + 1) * CV_BK);
    }
#pragma unroll
    for (int ks = 0; ks < CV_BK / 16; ++ks) {
      uint4 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = *(const uint4*)&As[buf][wr * 64 + i * 32 + fr][ks * 16 + fk];
#pragma unroll
      for (int j = 0; j < 2; ++j) bfr[j] = *(const uint4*)&Bs[buf][wc * 64 + j * 32 + fr][ks * 16 + fk];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = cv_mfma<DT>(bfr[j], af[i], acc[i][j]);   // D[channel][pixel]
    }
    if (s + 1 < nsteps) store(buf ^ 1);
    __syncthreads();
  }

  if (a.ksplit > 1) {   // raw fp32 partials [z][channel][pixel]; k_conv_reduce_* applies the epilogue
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = (int)m_base + wr * 64 + i * 32 + fr;
      if (m >= M32) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int co = n_base + wc * 64 + j * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
          if (co < a.Cout) a.part[((long long)kz * a.Cout + co) * a.M + m] = acc[i][j][e];
        }
    }
    return;
  }
  // epilogue. The MFMA operands are swapped (weights as the row operand), so each
  // accumulator register holds one channel for 32 consecutive pixels across the lanes:
  // stores (and residual loads) of a register are 64 contiguous bytes in NCHW.
  // Per-channel factors of the tile are computed once into LDS.
  __shared__ float s_al[CV_BN], s_be[CV_BN];
  if (tid < CV_BN) {
    const int cc = min(n_base + tid, a.Cout - 1);
    const float bias = (a.flags & 1) ? cv_f<DT>(((const uint16_t*)a.bias)[cc]) : 0.f;
    float al = 1.f, be = 0.f;
    if (a.flags & 2) {
      const float g = cv_f<DT>(((const uint16_t*)a.bn_w)[cc]), bb = cv_f<DT>(((const uint16_t*)a.bn_b)[cc]);
      const float mu = cv_f<DT>(((const uint16_t*)a.bn_mean)[cc]), var = cv_f<DT>(((const uint16_t*)a.bn_var)[cc]);
      al = g / sqrtf(var + a.eps);
      be = bb - mu * al;
    }
    s_al[tid] = al;
    s_be[tid] = be;
    ((float*)&Bs[0][0][0])[tid] = bias;   // Bs is free after the main loop
  }
  __syncthreads();
  const float* s_bias = (const float*)&Bs[0][0][0];
  if (a.flags & 16) {   // channels-last output [pixels, Cout] (Cout % 4 == 0): 4 channels per 8-byte store
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int m = (int)m_base + wr * 64 + i * 32 + fr;
      if (m >= M32) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int cl0 = wc * 64 + j * 32 + q * 8 + (lane >> 5) * 4;
          if (n_base + cl0 >= a.Cout) continue;
          const long long o = (long long)m * a.Cout + n_base + cl0;
          uint16_t h[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float v = cv_round<DT>(acc[i][j][q * 4 + r] + s_bias[cl0 + r]);
            if (a.flags & 2) v = cv_round<DT>(v * s_al[cl0 + r] + s_be[cl0 + r]);
            if (a.flags & 4) v = cv_round<DT>(v + cv_f<DT>(((const uint16_t*)a.resid)[o + r]));
            if (a.flags & 8) v = v != v ? v : fmaxf(v, 0.f);
            h[r] = cv_h<DT>(v);
          }
          *(uint2*)((uint16_t*)a.out + o) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = (int)m_base + wr * 64 + i * 32 + fr;
    if (m >= M32) continue;
    const int n = m / HoWo;
    const long long pixo = (long long)n * a.Cout * HoWo + (m - n * HoWo);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int cl = wc * 64 + j * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        const int co = n_base + cl;
        if (co >= a.Cout) continue;
        const long long o = pixo + (long long)co * HoWo;
        float v = cv_round<DT>(acc[i][j][e] + s_bias[cl]);
        if (a.flags & 2) v = cv_round<DT>(v * s_al[cl] + s_be[cl]);
        if (a.flags & 4) v = cv_round<DT>(v + cv_f<DT>(((const uint16_t*)a.resid)[o]));
        if (a.flags & 8) v = v != v ? v : fmaxf(v, 0.f);
        ((uint16_t*)a.out)[o] = cv_h<DT>(v);
      }
    }
  }
}

// Split-K reduction with the conv epilogue: one thread per 4 consecutive pixels of one channel
// (16-byte partial loads, M % 4 == 0: the host checks), partials summed in a fixed order.
template <int DT>
__device__ __forceinline__ void conv_reduce_body(const ConvArgs& a) {
  const long long total = (long long)a.Cout * a.M, quads = total / 4;
  const int HoWo = a.Ho * a.Wo;
  for (long long iq = (long long)blockIdx.x * 256 + threadIdx.x; iq < quads; iq += (long long)gridDim.x * 256) {
    const long long i = iq * 4;
    const int co = (int)(i / a.M);
    const long long m0 = i - (long long)co * a.M;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < a.ksplit; ++z) {
      const float4 p = *(const float4*)(a.part + (long long)z * total + i);
      acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
    }
    const float bias = (a.flags & 1) ? cv_f<DT>(((const uint16_t*)a.bias)[co]) : 0.f;
    float al = 1.f, be = 0.f;
    if (a.flags & 2) {
      const float g = cv_f<DT>(((const uint16_t*)a.bn_w)[co]), bb = cv_f<DT>(((const uint16_t*)a.bn_b)[co]);
      const float mu = cv_f<DT>(((const uint16_t*)a.bn_mean)[co]), var = cv_f<DT>(((const uint16_t*)a.bn_var)[co]);
      al = g / sqrtf(var + a.eps);
      be = bb - mu * al;
    }
    const float vs[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long long m = m0 + j;
      float v = cv_round<DT>(vs[j] + bias);
      if (a.flags & 2) v = cv_round<DT>(v * al + be);
      const long long n = m / HoWo, p = m - n * HoWo;
      const long long o = (a.flags & 16) ? m * a.Cout + co : (n * a.Cout + co) * HoWo + p;
      if (a.flags & 4) v = cv_round<DT>(v + cv_f<DT>(((const uint16_t*)a.resid)[o]));
      if (a.flags & 8) v = v != v ? v : fmaxf(v, 0.f);
      ((uint16_t*)a.out)[o] = cv_h<DT>(v);
    }
  }
}

#define CV_ATTRS __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
extern "C" __global__ void __launch_bounds__(256) k_conv_reduce_f16(const ConvArgs a) { conv_reduce_body<HS_F16>(a); }
extern "C" __global__ void __launch_bounds__(256) k_conv_reduce_bf16(const ConvArgs a) { conv_reduce_body<HS_BF16>(a); }
extern "C" __global__ void CV_ATTRS k_conv_f16(const ConvArgs a) { conv_body<HS_F16, true>(a); }
extern "C" __global__ void CV_ATTRS k_conv_f16_g(const ConvArgs a) { conv_body<HS_F16, false>(a); }
extern "C" __global__ void CV_ATTRS k_conv_f16_1x1(const ConvArgs a) { conv_body<HS_F16, true, 1>(a); }
extern "C" __global__ void CV_ATTRS k_conv_f16_3x3(const ConvArgs a) { conv_body<HS_F16, true, 3>(a); }
extern "C" __global__ void CV_ATTRS k_conv_bf16(const ConvArgs a) { conv_body<HS_BF16, true>(a); }
extern "C" __global__ void CV_ATTRS k_conv_bf16_g(const ConvArgs a) { conv_body<HS_BF16, false>(a); }
extern "C" __global__ void CV_ATTRS k_conv_bf16_1x1(const ConvArgs a) { conv_body<HS_BF16, true, 1>(a); }
extern "C" __global__ void CV_ATTRS k_conv_bf16_3x3(const ConvArgs a) { conv_body<HS_BF16, true, 3>(a); }

// ---------------------------------------------------------------- pooling / batch norm

// max over the window; positions outside the image are skipped (ATen's -inf padding)
extern "C" __global__ void __launch_bounds__(256) k_maxpool2d(const PoolArgs a) {
  const long long total = a.planes * a.Ho * a.Wo;
  const bool small = total < (1ll << 31) && a.planes * a.H * a.W < (1ll << 31);   // 32-bit index math
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    int wo, ho;
    long long pl;
    if (small) {
      const unsigned u = (unsigned)i, q = u / (unsigned)a.Wo;
      wo = (int)(u - q * (unsigned)a.Wo);
      const unsigned q2 = q / (unsigned)a.Ho;
      ho = (int)(q - q2 * (unsigned)a.Ho);
      pl = q2;
    } else {
      wo = (int)(i % a.Wo);
      ho = (int)((i / a.Wo) % a.Ho);
      pl = i / ((long long)a.Wo * a.Ho);
    }
    const long long x0 = pl * a.H * a.W;   // first element of the plane (any float dtype)
    float best = -INFINITY;
    bool nan = false;
    if (a.kh == 3 && a.kw == 3) {   // all nine loads in flight together (clamped addresses, masked values)
      float v[9];
      bool ok[9];
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        const int hi = ho * a.sh - a.ph + t / 3, wi = wo * a.sw - a.pw + t % 3;
        ok[t] = (unsigned)hi < (unsigned)a.H && (unsigned)wi < (unsigned)a.W;
        v[t] = ld_f(a.x, x0 + (ok[t] ? hi * a.W + wi : 0), a.dtype);
      }
#pragma unroll
      for (int t = 0; t < 9; ++t) {
        if (!ok[t]) continue;
        nan |= v[t] != v[t];
        best = fmaxf(best, v[t]);
      }
    } else {
      for (int kh = 0; kh < a.kh; ++kh) {
        const int hi = ho * a.sh - a.ph + kh;
        if (hi < 0 || hi >= a.H) continue;
        for (int kw = 0; kw < a.kw; ++kw) {
          const int wi = wo * a.sw - a.pw + kw;
          if (wi < 0 || wi >= a.W) continue;
          const float v = ld_f(a.x, x0 + hi * a.W + wi, a.dtype);
          nan |= v != v;
          best = fmaxf(best, v);
        }
      }
    }
    if (nan) best = NAN;
    st_f(a.out, i, a.dtype, best);   // a max of stored values: exact in the input dtype
  }
}

// out = round(x * a_c + b_c) (+ ReLU), a_c = w_c / sqrt(var_c + eps), b_c = bias_c - mean_c * a_c;
// x and out of dtype `dtype`, the four per-channel parameters of dtype `p_dtype` (any float dtype)
extern "C" __global__ void __launch_bounds__(256) k_batchnorm(const BatchNormArgs a) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < a.n; i += (long long)gridDim.x * 256) {
    const int c = (int)((i / a.hw) % a.C);
    const float al = ld_f(a.w, c, a.p_dtype) / sqrtf(ld_f(a.var, c, a.p_dtype) + a.eps);
    const float be = ld_f(a.b, c, a.p_dtype) - ld_f(a.mean, c, a.p_dtype) * al;
    float v = ld_f(a.x, i, a.dtype) * al + be;
    if (a.relu) v = v != v ? v : fmaxf(v, 0.f);
    st_f(a.out, i, a.dtype, v);
  }
}

// ---------------------------------------------------------------- channels-last pooling

// max pooling of an NHWC image [planes = N, H, W, C] into [N, Ho, Wo, C]: one thread per output
// pixel and 8 channels (16-byte loads and store); a 3 x 3 window issues its nine loads together
// (clamped addresses, masked values). NaN in a window gives NaN, as the NCHW kernel.
template <int DT>
__device__ __forceinline__ void maxpool_nhwc_body(const PoolArgs& a) {
  const int CG = a.C / 8;
  const long long total = a.planes * a.Ho * a.Wo * CG;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    const int cg = (int)(i % CG);
    long long t = i / CG;
    const int wo = (int)(t % a.Wo);
    t /= a.Wo;
    const int ho = (int)(t % a.Ho);
    const long long n = t / a.Ho;
    const uint16_t* x = (const uint16_t*)a.x + n * a.H * a.W * a.C + cg * 8;
    float best[8];
    bool nan[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) { best[c] = -INFINITY; nan[c] = false; }
    auto take = [&](const uint4 v) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint16_t hb = (uint16_t)(w[c >> 1] >> ((c & 1) * 16));
        const float f = cv_f<DT>(hb);
        nan[c] |= f != f;
        best[c] = fmaxf(best[c], f);
      }
    };
    if (a.kh == 3 && a.kw == 3) {
      uint4 v[9];
      bool ok[9];
#pragma unroll
      for (int tp = 0; tp < 9; ++tp) {
        const int hi = ho * a.sh - a.ph + tp / 3, wi = wo * a.sw - a.pw + tp % 3;
        ok[tp] = (unsigned)hi < (unsigned)a.H && (unsigned)wi < (unsigned)a.W;
        v[tp] = *(const uint4*)(x + (ok[tp] ? ((long long)hi * a.W + wi) * a.C : 0));
      }
#pragma unroll
      for (int tp = 0; tp < 9; ++tp)
        if (ok[tp]) take(v[tp]);
    } else {
      for (int kh = 0; kh < a.kh; ++kh)
        for (int kw = 0; kw < a.kw; ++kw) {
          const int hi = ho * a.sh - a.ph + kh, wi = wo * a.sw - a.pw + kw;
          if ((unsigned)hi < (unsigned)a.H && (unsigned)wi < (unsigned)a.W)
            take(*(const uint4*)(x + ((long long)hi * a.W + wi) * a.C));
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float f0 = nan[2 * c] ? NAN : best[2 * c], f1 = nan[2 * c + 1] ? NAN : best[2 * c + 1];
      o[c] = cv_h<DT>(f0) | ((uint32_t)cv_h<DT>(f1) << 16);
    }
    *(uint4*)((uint16_t*)a.out + ((n * a.Ho + ho) * a.Wo + wo) * a.C + cg * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}
extern "C" __global__ void __launch_bounds__(256) k_maxpool2d_nhwc_f16(const PoolArgs a) { maxpool_nhwc_body<HS_F16>(a); }
extern "C" __global__ void __launch_bounds__(256) k_maxpool2d_nhwc_bf16(const PoolArgs a) { maxpool_nhwc_body<HS_BF16>(a); }

// mean over the pixels of an NHWC image [n, hw, c] into [n, c] (a global average pool): one
// thread per image and 8 channels, 16-byte loads, fp32 sum divided by hw, rounded once
template <int DT>
__device__ __forceinline__ void mean_nhwc_body(const MeanNHWCArgs& a) {
  const int CG = a.c / 8;
  const long long total = a.n * CG;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
    const long long img = i / CG;
    const int cg = (int)(i - img * CG);
    const uint16_t* x = (const uint16_t*)a.x + img * a.hw * a.c + cg * 8;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < a.hw; ++p) {
      const uint4 v = *(const uint4*)(x + (long long)p * a.c);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) s[c] += cv_f<DT>((uint16_t)(w[c >> 1] >> ((c & 1) * 16)));
    }
    uint32_t o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = cv_h<DT>(s[2 * c] / (float)a.hw) | ((uint32_t)cv_h<DT>(s[2 * c + 1] / (float)a.hw) << 16);
    *(uint4*)((uint16_t*)a.out + img * a.c + cg * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}
extern "C" __global__ void __launch_bounds__(256) k_mean_nhwc_f16(const MeanNHWCArgs a) { mean_nhwc_body<HS_F16>(a); }
extern "C" __global__ void __launch_bounds__(256) k_mean_nhwc_bf16(const MeanNHWCArgs a) { mean_nhwc_body<HS_BF16>(a); }

// OIHW -> OHWI weight copies (the channels-last convs read k = (kh, kw, ci)), zero-padded to
// [Cout, khp, kwp, cp] where asked: one thread per 8 destination elements (one 16-byte store), each
// element decoded on its own; the tensor is found by a scan of the start offsets
extern "C" __global__ void __launch_bounds__(256) k_permute_ohwi(const PermuteOHWIArgs a) {
  const long long total8 = a.start[a.n] / 8;
  for (long long g = (long long)blockIdx.x * 256 + threadIdx.x; g < total8; g += (long long)gridDim.x * 256) {
    const long long e0 = g * 8;
    int i = 0;
    while (i + 1 < a.n && a.start[i + 1] <= e0) ++i;
    const long long e = e0 - a.start[i];
    const int cin = a.cin[i], kh = a.kh[i], kw = a.kw[i], cp = a.cp[i], kwp = a.kwp[i];
    const long long per = (long long)a.khp[i] * kwp * cp;
    const uint16_t* src = (const uint16_t*)a.src[i];
    uint32_t w[4];
    if (cp == cin && a.khp[i] == kh && kwp == kw && (cin & 7) == 0) {   // unpadded: 8 channels of one tap
      const int kk = kh * kw;
      const long long co = e / per;
      const int rem = (int)(e - co * per), t = rem / cin, ci = rem - t * cin;
      const uint16_t* s0 = src + (co * cin + ci) * kk + t;
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = s0[(2 * j) * kk] | ((uint32_t)s0[(2 * j + 1) * kk] << 16);
      *(uint4*)((uint16_t*)a.dst[i] + e) = make_uint4(w[0], w[1], w[2], w[3]);
      continue;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const long long ej = e + j;
      const long long co = ej / per;
      const int r = (int)(ej - co * per), y = r / (kwp * cp), xc = r - y * (kwp * cp), x = xc / cp, c = xc - x * cp;
      const uint16_t v = (y < kh && x < kw && c < cin) ? src[((co * cin + c) * kh + y) * kw + x] : (uint16_t)0;
      if (j & 1) w[j >> 1] |= (uint32_t)v << 16;
      else w[j >> 1] = v;
    }
    *(uint4*)((uint16_t*)a.dst[i] + e) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// NCHW image with C <= 4 channels -> zero-bordered channels-last [N, Hp, Wp, 4] (channels past C
// are 0): the input of the _convp GEMM, whose taps then never leave the buffer. One thread per
// output pixel (one 8-byte store).
extern "C" __global__ void __launch_bounds__(256) k_pad_nhwc4(const PadNHWCArgs a) {
  const long long total = a.n * a.Hp * a.Wp;
  const long long plane = (long long)a.H * a.W;
  for (long long p = (long long)blockIdx.x * 256 + threadIdx.x; p < total; p += (long long)gridDim.x * 256) {
    const int xo = (int)(p % a.Wp);
    const long long t = p / a.Wp;
    const int yo = (int)(t % a.Hp);
    const long long img = t / a.Hp;
    const int y = yo - a.top, x = xo - a.left;
    uint16_t v[4] = {0, 0, 0, 0};
    if ((unsigned)y < (unsigned)a.H && (unsigned)x < (unsigned)a.W) {
      const uint16_t* src = (const uint16_t*)a.x + img * a.C * plane + (long long)y * a.W + x;
      for (int c = 0; c < a.C; ++c) v[c] = src[c * plane];
    }
    *(uint2*)((uint16_t*)a.out + p * 4) = make_uint2(v[0] | ((uint32_t)v[1] << 16), v[2] | ((uint32_t)v[3] << 16));
  }
}
