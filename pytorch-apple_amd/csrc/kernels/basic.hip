// Bandwidth-bound utility kernels for gfx950: strided copy/cast, fill, RMSNorm,
// embedding gather, rotary tables, in-place index_copy, masked softmax, last-dim
// mean and argmax, and a plain batched matmul for shapes no pattern claims.
// All arithmetic is fp32 with one rounding to the output dtype per IR op, the
// rounding points of ATen on the CPU.
#include "common.h"

// ---------------------------------------------------------------- copy / cast / fill

extern "C" __global__ void __launch_bounds__(256) k_copy(const CopyArgs a) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    long long rem = i, so = 0, dof = 0;
    for (int d = a.ndim - 1; d >= 0; --d) {
      const long long c = rem % a.shape[d];
      rem /= a.shape[d];
      so += c * a.sstride[d];
      dof += c * a.dstride[d];
    }
    if (a.sdtype == a.ddtype && (a.sdtype == HS_I64 || a.sdtype == HS_F64)) {
      ((long long*)a.dst)[dof] = ((const long long*)a.src)[so];
    } else if (a.sdtype == a.ddtype && (a.sdtype == HS_BF16 || a.sdtype == HS_F16)) {
      ((uint16_t*)a.dst)[dof] = ((const uint16_t*)a.src)[so];
    } else if (a.ddtype == HS_I64 || a.ddtype == HS_I32) {
      const long long v = (a.sdtype == HS_I64 || a.sdtype == HS_I32 || a.sdtype == HS_U8)
                              ? ld_i(a.src, so, a.sdtype) : (long long)ld_f(a.src, so, a.sdtype);
      if (a.ddtype == HS_I64) ((long long*)a.dst)[dof] = v; else ((int*)a.dst)[dof] = (int)v;
    } else {
      st_f(a.dst, dof, a.ddtype, ld_f(a.src, so, a.sdtype));
    }
  }
}

// Contiguous copy of a.n 16-byte chunks (src and dst 16-byte aligned, same dtype): the generic
// kernel above spends its time on per-element index arithmetic. Here workgroup b copies one
// contiguous range of ceil(n / grid) chunks, each thread with eight non-temporal 16-byte loads in
// flight (measured on 512 MiB: 5.7 TB/s of read + write, against 4.6 for a grid-stride loop with
// four cached loads and 4.7 for hipMemcpy device to device).
typedef unsigned int copy_u32x4 __attribute__((ext_vector_type(4)));
extern "C" __global__ void __launch_bounds__(256) k_copy16(const CopyArgs a) {
  const copy_u32x4* s = (const copy_u32x4*)a.src;
  copy_u32x4* d = (copy_u32x4*)a.dst;
  const long long n = a.n, C = (n + gridDim.x - 1) / gridDim.x;
  const long long b0 = (long long)blockIdx.x * C, e = min(b0 + C, n);
  for (long long i = b0 + threadIdx.x; i < e; i += 8 * 256) {
    copy_u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(s + min(i + u * 256, e - 1));   // past the range: re-read its last chunk
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (i + u * 256 < e) __builtin_nontemporal_store(v[u], d + i + u * 256);
  }
}

extern "C" __global__ void __launch_bounds__(256) k_fill(const FillArgs a) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    if (a.dtype == HS_I64) ((long long*)a.out)[i] = (long long)a.value;
    else if (a.dtype == HS_F64) ((double*)a.out)[i] = a.value;
    else st_f(a.out, i, a.dtype, (float)a.value);
  }
}

// ---------------------------------------------------------------- RMSNorm

// One 256-thread workgroup per row:
//   h = f32(x); r = rsqrt(mean(h*h) + eps); n = round_n(h*r); out = round_out(w * n)
extern "C" __global__ void __launch_bounds__(256) k_rmsnorm(const RMSNormArgs a) {
  __shared__ float red[4];
  const long long row = blockIdx.x;
  if (row >= a.rows) return;
  const void* x = (const char*)a.x + row * a.ldx * (a.x_dtype == HS_F32 ? 4 : 2);
  float ss = 0.f;
  for (int c = threadIdx.x; c < a.cols; c += 256) {
    const float h = ld_f(x, c, a.x_dtype);
    ss += h * h;
  }
  ss = block_sum256(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
  void* out = (char*)a.out + row * a.ldo * (a.out_dtype == HS_F32 ? 4 : 2);
  for (int c = threadIdx.x; c < a.cols; c += 256) {
    const float n = round_to(ld_f(x, c, a.x_dtype) * r, a.n_dtype);
    st_f(out, c, a.out_dtype, ld_f(a.w, c, a.w_dtype) * n);
  }
}

// Rows of 16-bit values, cols % 8 == 0 and cols <= 4096, w of the same dtype as x, 16-byte aligned
// rows: one wave per row, every 16-byte load of x and w issued before the first use (one memory
// latency), a wave reduction instead of a workgroup one, 16-byte stores. Same formula as k_rmsnorm.
extern "C" __global__ void __launch_bounds__(256) k_rmsnorm_w(const RMSNormArgs a) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.rows) return;   // wave-uniform
  const int nch = a.cols / 8;
  const uint16_t* x = (const uint16_t*)a.x + row * a.ldx;
  uint4 xv[8], wv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {   // chunks past the row re-read chunk 0 (no branch between the loads)
    const int c = lane + 64 * t < nch ? lane + 64 * t : 0;
    xv[t] = *(const uint4*)(x + c * 8);
    wv[t] = *(const uint4*)((const uint16_t*)a.w + c * 8);
  }
  const bool bf = a.x_dtype == HS_BF16;
  auto f = [&](uint32_t w32, int h) {
    const uint16_t b = (uint16_t)(w32 >> (16 * h));
    return bf ? bf16_to_f32(b) : f16_to_f32(b);
  };
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (lane + 64 * t >= nch) continue;
    const uint32_t q[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float h = f(q[c >> 1], c & 1);
      ss += h * h;
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
  uint16_t* out = (uint16_t*)a.out + row * a.ldo;
  const bool obf = a.out_dtype == HS_BF16;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int c = lane + 64 * t;
    if (c >= nch) continue;
    const uint32_t q[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w}, g[4] = {wv[t].x, wv[t].y, wv[t].z, wv[t].w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t v = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float n = round_to(f(q[k], h) * r, a.n_dtype);
        const float y = f(g[k], h) * n;
        v |= (uint32_t)(obf ? f32_to_bf16(y) : f32_to_f16(y)) << (16 * h);
      }
      o[k] = v;
    }
    *(uint4*)(out + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------- embedding gather (bit-exact)

extern "C" __global__ void __launch_bounds__(256) k_embedding(const EmbeddingArgs a) {
  const long long s = blockIdx.x;
  if (s >= a.n_ids) return;
  const long long id = ld_i(a.ids, s, a.ids_dtype);
  char* dst = (char*)a.out + s * a.row_bytes;
  const bool ok = id >= 0 && id < a.vocab;
  const char* src = (const char*)a.w + (ok ? id : 0) * a.row_bytes;
  if ((a.row_bytes & 15) == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0) {
    const long long nv = a.row_bytes >> 4;
    for (long long i = threadIdx.x; i < nv; i += blockDim.x) {
      uint4 v = ok ? ((const uint4*)src)[i] : make_uint4(0, 0, 0, 0);
      ((uint4*)dst)[i] = v;
    }
  } else {
    for (long long i = threadIdx.x; i < a.row_bytes; i += blockDim.x) dst[i] = ok ? src[i] : 0;
  }
}

// ---------------------------------------------------------------- rotary tables

// cos/sin[s, j] = cos/sin(inv_freq[j % half] * float(pos[s])) * scaling, rounded to out_dtype
extern "C" __global__ void __launch_bounds__(256) k_rope_table(const RopeTableArgs a) {
  const long long s = blockIdx.x;
  const int j = threadIdx.x;
  if (s >= a.S || j >= 2 * a.half) return;
  const float p = (float)ld_i(a.pos, s, a.pos_dtype);
  const float f = a.inv_freq[j % a.half] * p;
  st_f(a.cos_out, s * 2 * a.half + j, a.out_dtype, cosf(f) * a.scaling);
  st_f(a.sin_out, s * 2 * a.half + j, a.out_dtype, sinf(f) * a.scaling);
}

// ---------------------------------------------------------------- index_copy (in place, bit-exact)

// dst[o, index[j], i] = src[o, j, i]; indices outside [0, dim_size) are skipped.
extern "C" __global__ void __launch_bounds__(256) k_index_copy(const IndexCopyArgs a) {
  const long long total = a.outer * a.nidx * a.inner;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const long long i = t % a.inner;
    const long long j = (t / a.inner) % a.nidx;
    const long long o = t / (a.inner * a.nidx);
    const long long idx = ld_i(a.index, j, a.idx_dtype);
    if (idx < 0 || idx >= a.dim_size) continue;
    const long long so = o * a.src_so + j * a.src_sj + i * a.src_si;
    const long long dof = (o * a.dim_size + idx) * a.inner + i;
    if (a.elem_bytes == 2) ((uint16_t*)a.dst)[dof] = ((const uint16_t*)a.src)[so];
    else if (a.elem_bytes == 4) ((uint32_t*)a.dst)[dof] = ((const uint32_t*)a.src)[so];
    else ((uint64_t*)a.dst)[dof] = ((const uint64_t*)a.src)[so];
  }
}

// ---------------------------------------------------------------- softmax over the last dim

// a = round_add(x + mask) (when masked), then out = exp(a - max) / sum, fp32 inside.
extern "C" __global__ void __launch_bounds__(256) k_softmax(const SoftmaxArgs a) {
  __shared__ float red[4];
  const long long row = blockIdx.x;
  if (row >= a.rows) return;
  long long rem = row, xo = 0, mo = 0;
  for (int d = a.nlead - 1; d >= 0; --d) {
    const long long c = rem % a.lead_shape[d];
    rem /= a.lead_shape[d];
    xo += c * a.x_lead_stride[d];
    mo += c * a.mask_lead_stride[d];
  }
  auto val = [&](long long c) -> float {
    float v = ld_f(a.x, xo + c, a.x_dtype);
    if (a.has_mask) v = round_to(v + ld_f(a.mask, mo + c * a.mask_col_stride, a.mask_dtype), a.add_dtype);
    return v;
  };
  float m = -INFINITY;
  for (long long c = threadIdx.x; c < a.cols; c += 256) m = fmaxf(m, val(c));
  m = block_max256(m, red);
  float s = 0.f;
  for (long long c = threadIdx.x; c < a.cols; c += 256) s += expf(val(c) - m);
  s = block_sum256(s, red);
  const float inv = 1.0f / s;
  for (long long c = threadIdx.x; c < a.cols; c += 256)
    st_f(a.out, row * a.cols + c, a.out_dtype, expf(val(c) - m) * inv);
}

// ---------------------------------------------------------------- last-dim mean / argmax

// rows of at most 64 elements (e.g. a 7 x 7 global average pool): one wave per row
extern "C" __global__ void __launch_bounds__(256) k_mean_short(const ReduceLastArgs a) {
  const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.rows) return;   // wave-uniform
  const float v = lane < a.cols ? ld_f(a.x, row * a.cols + lane, a.x_dtype) : 0.f;
  const float s = wave_sum(v);
  if (lane == 0) st_f(a.out, row, a.out_dtype, s / (float)a.cols);
}

extern "C" __global__ void __launch_bounds__(256) k_mean_last(const ReduceLastArgs a) {
  __shared__ float red[4];
  const long long row = blockIdx.x;
  if (row >= a.rows) return;
  float s = 0.f;
  for (long long c = threadIdx.x; c < a.cols; c += 256) s += ld_f(a.x, row * a.cols + c, a.x_dtype);
  s = block_sum256(s, red);
  if (threadIdx.x == 0) st_f(a.out, row, a.out_dtype, s / (float)a.cols);
}

// first index of the maximum (np.argmax / torch.argmax tie rule); NaN counts as maximum
extern "C" __global__ void __launch_bounds__(256) k_argmax(const ReduceLastArgs a) {
  __shared__ float sv[256];
  __shared__ long long si[256];
  const long long row = blockIdx.x;
  if (row >= a.rows) return;
  float best = -INFINITY;
  long long bi = -1;
  for (long long c = threadIdx.x; c < a.cols; c += 256) {
    const float v = ld_f(a.x, row * a.cols + c, a.x_dtype);
    if (bi < 0 || v > best || (v != v && best == best)) { best = v; bi = c; }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) {
      const float v2 = sv[threadIdx.x + o];
      const long long i2 = si[threadIdx.x + o];
      const float v1 = sv[threadIdx.x];
      const long long i1 = si[threadIdx.x];
      bool take = false;
      if (i2 >= 0) {
        if (i1 < 0) take = true;
        else if (v1 != v1) take = (v2 != v2) && i2 < i1;
        else if (v2 != v2) take = true;
        else take = v2 > v1 || (v2 == v1 && i2 < i1);
      }
      if (take) { sv[threadIdx.x] = v2; si[threadIdx.x] = i2; }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (a.out_dtype == HS_I64) ((long long*)a.out)[row] = si[0];
    else ((int*)a.out)[row] = (int)si[0];
  }
}

// ---------------------------------------------------------------- generic batched matmul

// One output element per thread, fp32 accumulation, one rounding. For shapes that
// no fused kernel claims (e.g. unpatterned attention); not a performance path.
extern "C" __global__ void __launch_bounds__(256) k_bmm(const BmmArgs a) {
  long long nb = 1;
  for (int d = 0; d < a.nbatch; ++d) nb *= a.batch_shape[d];
  const long long total = nb * a.M * a.N;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const long long n = t % a.N;
    const long long m = (t / a.N) % a.M;
    long long b = t / (a.N * a.M), ao = 0, bo = 0;
    for (int d = a.nbatch - 1; d >= 0; --d) {
      const long long c = b % a.batch_shape[d];
      b /= a.batch_shape[d];
      ao += c * a.a_bstride[d];
      bo += c * a.b_bstride[d];
    }
    float acc = 0.f;
    for (long long k = 0; k < a.K; ++k)
      acc += ld_f(a.a, ao + m * a.a_sm + k * a.a_sk, a.a_dtype) * ld_f(a.b, bo + k * a.b_sk + n * a.b_sn, a.b_dtype);
    st_f(a.c, t, a.c_dtype, acc);
  }
}

// k_decode_advance: one thread. Moves a greedy decode loop's position inputs to the next step
// in place: p = cache_position + 1; cache_position = position_ids = p; mask[p] = 0 (the row
// was open on 0 .. p - 1 and -inf after). One launch instead of three host-issued copies.
// A step past the cache end (p >= S) changes nothing and sets *overflow, which the host checks.
extern "C" __global__ void __launch_bounds__(64) k_decode_advance(const AdvanceArgs a) {
  if (threadIdx.x != 0) return;
  const long long p = a.cpos[0] + 1;
  if (p < 0 || p >= a.S) {
    a.overflow[0] = 1;
    return;
  }
  a.cpos[0] = p;
  a.pos[0] = p;
  if (a.mask_bytes == 4) ((float*)a.mask)[p] = 0.f;
  else ((uint16_t*)a.mask)[p] = 0;
}
