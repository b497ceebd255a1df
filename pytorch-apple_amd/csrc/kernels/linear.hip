// Streaming linear (GEMV-shaped) kernels for small M: out = x . W^T (+ bias) (+ residual).
//
// W is [N, K] row-major bf16/fp16 and is the dominant HBM stream; each wave owns
// RPW weight rows and walks K with 16-byte loads per lane (one 1 KiB row slice per
// wave instruction), accumulating in fp32 with v_dot2 (two products per
// instruction). x rows are re-read from cache by every wave. A workgroup is four
// waves; grid.x covers N in 4*RPW-row blocks, grid.y covers M in MB-row blocks.
// Rounding: out = round(acc + bias); with a residual, out = round(resid + round(...)),
// the two roundings of ATen's linear followed by add.
#include "common.h"

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_v;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_v;

template <int DT>
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  if constexpr (DT == HS_BF16) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.x), __builtin_bit_cast(bf16x2_v, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.y), __builtin_bit_cast(bf16x2_v, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.z), __builtin_bit_cast(bf16x2_v, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a.w), __builtin_bit_cast(bf16x2_v, b.w), acc, false);
  } else {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a.x), __builtin_bit_cast(f16x2_v, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a.y), __builtin_bit_cast(f16x2_v, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a.z), __builtin_bit_cast(f16x2_v, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_v, a.w), __builtin_bit_cast(f16x2_v, b.w), acc, false);
  }
  return acc;
}

template <int DT>
__device__ __forceinline__ float ld_h(const void* p, long long i) {
  const uint16_t h = ((const uint16_t*)p)[i];
  return DT == HS_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

template <int DT>
__device__ __forceinline__ void st_h(void* p, long long i, float f) {
  ((uint16_t*)p)[i] = DT == HS_BF16 ? f32_to_bf16(f) : f32_to_f16(f);
}

template <int DT, int MB, int RPW>
__device__ __forceinline__ void linear_body(const LinearArgs& a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * RPW;
  const long long m0 = (long long)blockIdx.y * MB;
  if (n0 >= a.N) return;
  const uint16_t* W = (const uint16_t*)a.w;
  const uint16_t* X = (const uint16_t*)a.x;
  float acc[MB][RPW];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[m][r] = 0.f;

  for (int k = lane * 8; k < a.K; k += 512) {
    uint4 wv[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int n = min(n0 + r, a.N - 1);
      wv[r] = *(const uint4*)(W + (long long)n * a.K + k);
    }
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const long long mm = min(m0 + m, a.M - 1);
      const uint4 xv = *(const uint4*)(X + mm * a.ldx + k);
#pragma unroll
      for (int r = 0; r < RPW; ++r) acc[m][r] = dot8<DT>(xv, wv[r], acc[m][r]);
    }
  }
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[m][r] = wave_sum(acc[m][r]);

#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (lane != m * RPW + r) continue;
      const long long mm = m0 + m;
      const int n = n0 + r;
      if (mm >= a.M || n >= a.N) continue;
      float v = acc[m][r];
      if (a.has_bias) v += ld_h<DT>(a.bias, n);
      v = round_to(v, DT);
      if (a.has_resid) v = ld_h<DT>(a.resid, mm * a.ldr + n) + v;
      st_h<DT>(a.out, mm * a.ldo + n, v);
    }
}

extern "C" __global__ void __launch_bounds__(256) k_linear_bf16_m1(const LinearArgs a) { linear_body<HS_BF16, 1, 4>(a); }
extern "C" __global__ void __launch_bounds__(256) k_linear_bf16_m4(const LinearArgs a) { linear_body<HS_BF16, 4, 2>(a); }
extern "C" __global__ void __launch_bounds__(256) k_linear_f16_m1(const LinearArgs a) { linear_body<HS_F16, 1, 4>(a); }
extern "C" __global__ void __launch_bounds__(256) k_linear_f16_m4(const LinearArgs a) { linear_body<HS_F16, 4, 2>(a); }
