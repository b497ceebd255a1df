// MFMA GEMM for prefill-shaped linears (M >= 64): out[m, n] = epi(sum_k x[m, k] w[n, k]).
//
// Both operands are K-contiguous ([M, K] activations, [N, K] weights as the model stores
// them), which is exactly the register layout of the gfx950 MFMA
// v_mfma_f32_32x32x16_{bf16,f16}: lane l holds 8 consecutive k of row (or column) l % 32
// at k offset 8 * (l / 32), and the 32x32 fp32 result sits in 16 registers per lane,
// element 4q + r at row 8q + 4(l / 32) + r, column l % 32.
// Workgroup tile BM x BN (BN columns per weight), K step 32, 256 threads as 2 x 2
// waves of (BM / 2) x (BN / 2) (or 4 x 1 waves: GEMM_KERNEL_W4). Tiles are double-buffered in LDS through registers: the
// global loads of step k+1 are in flight while step k is multiplied, then stored to the
// other buffer, one barrier per step. LDS rows are padded (40 elements) so the 16-byte
// fragment reads of 32 consecutive rows spread over the banks.
// Epilogues (fp32 accumulator, ATen's rounding points):
//   BIAS  out = round(acc + b)
//   RESID out = round(r + round(acc + b))
//   SILU  out = round(round(silu(round(acc_g + b_g))) * round(acc_u + b_u))   (NW = 2)
// Rows past M and columns past N are computed from clamped (valid) addresses and not stored.
// Grouped use (_grp): output columns [0, n1), [n1, n2), [n2, N) are computed from three
// weights (and biases), e.g. the q, k and v projections of one activation in one launch.
// Batched use (grid.z = batch * ksplit): batch b reads x + b*sx and w + (b / bdiv)*sw (the
// GQA head -> KV head map) and writes out + b*so. The _kn kernels take w as [K, N]
// (N-contiguous, e.g. V in P.V) and transpose it while staging into LDS.
#include "common.h"

typedef __attribute__((ext_vector_type(8))) __bf16 gm_bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 gm_f16x8;
typedef __attribute__((ext_vector_type(16))) float gm_f32x16;

enum { GE_BIAS = 0, GE_RESID = 1, GE_SILU = 2, GE_CONV = 3 };
#define GM_BK 32      // default K step

template <int DT>
__device__ __forceinline__ gm_f32x16 gm_mfma(const uint4 a, const uint4 b, gm_f32x16 c) {
  if constexpr (DT == HS_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gm_bf16x8, a), __builtin_bit_cast(gm_bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(gm_f16x8, a), __builtin_bit_cast(gm_f16x8, b),
                                                  c, 0, 0, 0);
}

template <int DT>
__device__ __forceinline__ float gm_ld(const void* p, long long i) {
  const uint16_t h = ((const uint16_t*)p)[i];
  return DT == HS_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

template <int DT>
__device__ __forceinline__ float gm_round(float f) {
  return DT == HS_BF16 ? bf16_to_f32(f32_to_bf16(f)) : f16_to_f32(f32_to_f16(f));
}

template <int DT>
__device__ __forceinline__ uint16_t gm_pack(float f) {
  return DT == HS_BF16 ? f32_to_bf16(f) : f32_to_f16(f);
}

// slot permutation of the direct-to-LDS rows (GM_SWZ_PAIR: rows 2j and 2j + 1 share one,
// for an LDS that serves 16 lanes of a 16-byte read per cycle)
#ifndef GM_SWZ_PAIR
#define GM_SWZ_PAIR 1
#endif
__device__ __forceinline__ int gm_swz(int r) { return GM_SWZ_PAIR ? (r >> 1) & 7 : r & 7; }

// 16 bytes per lane from global memory straight into LDS at m0 + 16 * lane (gfx950). Issued
// from inline assembly so that the compiler does not wait for every one of them before each
// LDS read (it cannot tell the stages apart); the waits are explicit (gm_vmcnt) instead, and
// the loop issues no other vector-memory loads.
__device__ __forceinline__ void gm_dma16(const void* g, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// s_waitcnt vmcnt(N), the other counters untouched
template <int N>
__device__ __forceinline__ void gm_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}
// wait until at most `after` stages of NI loads each are outstanding (after <= MAXA, uniform)
template <int NI, int MAXA>
__device__ __forceinline__ void gm_vmcnt_after(int after) {
  if constexpr (MAXA > 0) {
    if (after >= MAXA) {
      gm_vmcnt<MAXA * NI>();
      return;
    }
    gm_vmcnt_after<NI, MAXA - 1>(after);
  } else {
    gm_vmcnt<0>();
  }
}

// conv epilogue (conv.hip's rounding points): after v = round(acc + bias),
//   batch norm: v = round(v * al + be), al = w / sqrt(var + eps), be = bias - mean * al;
//   residual: v = round(v + r);  ReLU: v = max(v, 0) (NaN kept)
template <int DT>
__device__ __forceinline__ void gm_bn_factors(const GemmArgs& a, int n, float& al, float& be) {
  const float g = gm_ld<DT>(a.bn_w, n), bb = gm_ld<DT>(a.bn_b, n);
  const float mu = gm_ld<DT>(a.bn_mean, n), var = gm_ld<DT>(a.bn_var, n);
  al = g / sqrtf(var + a.eps);
  be = bb - mu * al;
}
template <int DT>
__device__ __forceinline__ float gm_conv_tail(const GemmArgs& a, float v, float al, float be, uint16_t r) {
  if (a.flags & 2) v = gm_round<DT>(v * al + be);
  if (a.flags & 4) v = gm_round<DT>(v + (DT == HS_BF16 ? bf16_to_f32(r) : f16_to_f32(r)));
  if (a.flags & 8) v = v != v ? v : fmaxf(v, 0.f);
  return v;
}

// STAGES 0: LDS double buffer filled through registers (the loads of step s + 1 are in flight
// while step s is multiplied). STAGES >= 2 (BK 64, not KN): the operands go from global memory
// straight into LDS (gfx950 global_load_lds_dwordx4), STAGES buffers deep, so the loads of
// steps s + 1 .. s + STAGES - 1 are in flight while step s is multiplied and no registers hold
// them. Those rows are unpadded 128-byte rows; 16-byte chunk c of row r sits in slot
// c ^ gm_swz(r), so the fragment reads of 8 consecutive rows hit 8 different bank groups.
// CV (direct-to-LDS only), A gathered from an NHWC image with row m = output pixel (see GemmArgs):
// 1: k = (kh, kw, ci), a whole 64-channel block per K step, padded taps read a.zero;
// 2: a zero-bordered 4-channel image, each 16-byte chunk two neighbouring taps of one kernel row.
template <int DT, int EPI, int NW, int BM, int BN, bool KN = false, int BK = GM_BK, bool GRP = false,
          int STAGES = 0, int CV = 0, int WR = 2, int LDSST = 0>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
  constexpr bool DMA = STAGES >= 2;
  // LDSST 1 (direct-to-LDS): the LDS of one stage, each K step loaded and waited for in turn (other
  // resident workgroups overlap the wait)
  constexpr int LST = LDSST > 0 ? LDSST : STAGES;
  static_assert(LDSST == 0 || (DMA && LDSST == 1), "LDS stages");
  static_assert(!DMA || (BK == 64 && !KN), "direct-to-LDS staging: BK 64, K-contiguous weights");
  static_assert(!CV || (DMA && NW == 1 && !GRP), "conv gather: direct-to-LDS, one weight");
  constexpr int LDK = BK + 8;             // padded LDS row (elements): fragment reads of 32 rows spread over the banks
  constexpr int CPR = BK / 8;             // 16-byte chunks per staged row
  constexpr int BNT = BN * NW;            // weight rows staged per step (BN columns per weight)
  // the 4 waves as WR rows x WC columns of (BM / WR) x (BN / WC) each (per weight)
  static_assert(WR == 1 || WR == 2 || WR == 4, "wave rows");
  constexpr int WC = 4 / WR, WM = BM / WR, WN = BN / WC;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile");
  constexpr int TI = WM / 32;             // 32-row MFMA tiles per wave
  constexpr int TJ = WN / 32;             // 32-column MFMA tiles per wave and weight
  constexpr int A_LD = BM * BK / 8 / 256;    // 16-byte A loads per thread per step
  constexpr int B_LD = BNT * BK / 8 / 256;   // 16-byte B loads per thread per step
  constexpr int SROW = 64;                   // DMA: elements per LDS row
  constexpr int SSTAGE = (BM + BNT) * SROW;  // DMA: elements per stage (A rows, then B rows)
  // one LDS buffer: the direct-to-LDS stages, or the register path's double-buffered A and B tiles
  // (so a direct-to-LDS kernel holds no unused arrays: 80 KB stages fit two workgroups per CU)
  __shared__ __attribute__((aligned(16))) uint16_t Ls[DMA ? LST * SSTAGE : 2 * (BM + BNT) * LDK];
  typedef uint16_t AsT[2][DMA ? 1 : BM][LDK];
  typedef uint16_t BsT[2][DMA ? 1 : BNT][LDK];
  AsT& As = *reinterpret_cast<AsT*>(&Ls[0]);
  BsT& Bs = *reinterpret_cast<BsT*>(&Ls[DMA ? 0 : 2 * BM * LDK]);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave / WC, wc = wave % WC;
  // XCD-aware tile order: workgroup L (dispatch order) runs on XCD L % 8, so L is remapped
  // to give each XCD a contiguous range of tiles, decoded M-tile fastest: the M tiles that
  // read the same weight tile run back to back on one XCD and share its L2, instead of
  // landing on different XCDs and fetching the weights once per XCD
  const unsigned gx = gridDim.x, gy = gridDim.y;
  const unsigned total = gx * gy * gridDim.z;
  const unsigned lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const unsigned per = (total + 7) / 8, xcd = lin % 8, loc = lin / 8;
  const unsigned tall = total % 8 == 0 ? 8 : total % 8;   // XCDs that get `per` tiles; the rest get per - 1
  const unsigned tile = xcd < tall ? xcd * per + loc : tall * per + (xcd - tall) * (per - 1) + loc;
  // conv with flags & 16 (an input larger than its weights): N tile fastest instead, so the N tiles
  // of one block of output pixels run back to back on one XCD and read its input rows once from
  // HBM, while the (smaller) weights stay in every XCD's L2
  const bool nfast = EPI == GE_CONV && (a.flags & 16);
  const unsigned tm = nfast ? (tile / gx) % gy : tile % gy, tn = nfast ? tile % gx : (tile / gy) % gx;
  const unsigned tz = tile / (gy * gx);
  const long long m_base = (long long)tm * BM;
  const int n_base = tn * BN;
  const int bz = tz / a.ksplit, kz = tz % a.ksplit;   // batch, K split
  const uint16_t* X = (const uint16_t*)a.x + bz * a.sx;
  const long long wofs = (long long)(bz / a.bdiv) * a.sw;
  // two named pointers (a runtime-indexed pointer array would live in scratch memory)
  const uint16_t* W0 = (const uint16_t*)a.w + wofs;
  const uint16_t* W1 = (const uint16_t*)(NW == 2 ? a.w2 : a.w) + wofs;
  // grouped: the tile's columns belong to one group (tile-aligned boundaries), whose weight
  // rows and bias start at the group's first column
  int g_lo = 0, g_hi = a.N;
  const void* g_bias = a.bias;
  if constexpr (GRP) {
    const int g = (n_base >= a.n1) + (n_base >= a.n2);
    g_lo = g == 0 ? 0 : (g == 1 ? a.n1 : a.n2);
    g_hi = g == 0 ? a.n1 : (g == 1 ? a.n2 : a.N);
    W0 = (const uint16_t*)(g == 0 ? a.w : (g == 1 ? a.w2 : a.w3)) + wofs;
    g_bias = g == 0 ? a.bias : (g == 1 ? a.bias2 : a.bias3);
  }
  uint16_t* OUT = (uint16_t*)a.out + bz * a.so;

  // global -> register staging of one K step, and register -> LDS. The staging lives in
  // named registers (A_LD, B_LD <= 2): a small per-thread array would be promoted to LDS by
  // the compiler, doubling the LDS traffic of the main loop.
  static_assert(DMA || (A_LD >= 1 && A_LD <= 4 && B_LD >= 1 && B_LD <= 4), "staging registers");
  uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
  auto a_ld = [&](int i, int k0) -> uint4 {
    const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
    const long long m = min(m_base + row, a.M - 1);
    return *(const uint4*)(X + m * a.ldx + k0 + col);
  };
  auto b_ld = [&](int i, int k0) -> uint4 {
    const int c = tid + 256 * i;
    if constexpr (KN) {   // w is [K, N]: 16-byte chunks along n, BNT / 8 chunks per k row (NW == 1)
      const int kr = c / (BNT / 8), nc = (c % (BNT / 8)) * 8;
      const int n = min(n_base + nc, a.N - 8);
      return *(const uint4*)(W0 + (long long)(k0 + kr) * a.ldw + n);
    } else {
      const int row = c / CPR, col = (c % CPR) * 8;
      if constexpr (GRP) {   // NW == 1: row of the tile's group
        const int n = min(n_base + row, g_hi - 1) - g_lo;
        return *(const uint4*)(W0 + (long long)n * a.ldw + k0 + col);
      }
      const int u = row / BN, n = min(n_base + row % BN, a.N - 1);
      return *(const uint4*)((u == 0 ? W0 : W1) + (long long)n * a.ldw + k0 + col);
    }
  };
  auto a_st = [&](int buf, int i, uint4 v) {
    const int c = tid + 256 * i, row = c / CPR, col = (c % CPR) * 8;
    *(uint4*)&As[buf][row][col] = v;
  };
  auto b_st = [&](int buf, int i, uint4 v) {
    const int c = tid + 256 * i;
    if constexpr (KN) {   // transpose into the [n][k] layout the fragments are read from
      const int kr = c / (BNT / 8), nc = (c % (BNT / 8)) * 8;
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        Bs[buf][nc + 2 * j][kr] = (uint16_t)(q[j] & 0xffffu);
        Bs[buf][nc + 2 * j + 1][kr] = (uint16_t)(q[j] >> 16);
      }
    } else {
      const int row = c / CPR, col = (c % CPR) * 8;
      *(uint4*)&Bs[buf][row][col] = v;
    }
  };
#define GM_LOAD_INTO(k0, A, B)            \
  do {                                    \
    A##0 = a_ld(0, (k0));                 \
    if (A_LD > 1) A##1 = a_ld(1, (k0));   \
    if (A_LD > 2) A##2 = a_ld(2, (k0));   \
    if (A_LD > 3) A##3 = a_ld(3, (k0));   \
    B##0 = b_ld(0, (k0));                 \
    if (B_LD > 1) B##1 = b_ld(1, (k0));   \
    if (B_LD > 2) B##2 = b_ld(2, (k0));   \
    if (B_LD > 3) B##3 = b_ld(3, (k0));   \
  } while (0)
#define GM_STORE_FROM(buf, A, B)          \
  do {                                    \
    a_st((buf), 0, A##0);                 \
    if (A_LD > 1) a_st((buf), 1, A##1);   \
    if (A_LD > 2) a_st((buf), 2, A##2);   \
    if (A_LD > 3) a_st((buf), 3, A##3);   \
    b_st((buf), 0, B##0);                 \
    if (B_LD > 1) b_st((buf), 1, B##1);   \
    if (B_LD > 2) b_st((buf), 2, B##2);   \
    if (B_LD > 3) b_st((buf), 3, B##3);   \
  } while (0)
#define GM_LOAD_STEP(k0) GM_LOAD_INTO(k0, ra, rb)
#define GM_STORE_STEP(buf) GM_STORE_FROM(buf, ra, rb)

  gm_f32x16 acc[NW][TI][TJ];
#pragma unroll
  for (int u = 0; u < NW; ++u)
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[u][i][j][e] = 0.f;

  // split K: workgroup z covers [z * kchunk, (z + 1) * kchunk)
  const int kbeg = kz * a.kchunk;
  const int nsteps = min(a.kchunk, a.K - kbeg) / BK;
  X += kbeg;
  if constexpr (KN) {
    W0 += (long long)kbeg * a.ldw;
  } else {
    W0 += kbeg;
    W1 += kbeg;
  }
  const int fr = lane & 31, fk = (lane >> 5) * 8;   // fragment row/column and k offset of this lane
  // residual operands of this lane's outputs, two rows per register: loaded before any store (as far
  // as the compiler knows a store may alias them, so loads interleaved with the stores would each
  // wait a memory latency), and on the direct-to-LDS path before the main loop, so that their
  // latency overlaps the operand loads instead of following the last MFMA
  constexpr bool HAS_R = EPI == GE_RESID || EPI == GE_CONV;
  const bool want_r = EPI == GE_RESID || (EPI == GE_CONV && (a.flags & 4));
  // row-chunk epilogue through LDS (see below): 8 columns per 16-byte residual load and store
  constexpr bool CAN_STAGE = NW == 1 && !GRP && BM * (BN + 8) + 4 * BN <= (DMA ? LST * SSTAGE : 2 * BM * LDK);
  const bool staged = CAN_STAGE && a.ksplit == 1 && (a.N & 7) == 0 && (a.ldo & 7) == 0 &&
                      (((size_t)a.out) & 15) == 0 && (!want_r || ((a.ldr & 7) == 0 && (((size_t)a.resid) & 15) == 0));
  uint32_t rr[HAS_R && !CAN_STAGE ? TJ : 1][HAS_R && !CAN_STAGE ? TI : 1][8];
  // row-chunk epilogue operands: the residual chunks (CH per thread) and the raw batch norm
  // parameters of column tid (tid < BN). On the direct-to-LDS path they are loaded before the
  // first stage is issued, so the first stage's wait covers their latency instead of the epilogue
  // waiting a memory latency of its own after the last MFMA
  constexpr int CH = BM * BN / 8 / 256;   // 16-byte chunks per thread (row-chunk epilogue)
  uint4 rv[CAN_STAGE && HAS_R ? CH : 1];
  float bnr[EPI == GE_CONV && CAN_STAGE ? 4 : 1];
  auto load_stage_operands = [&]() {
    if constexpr (CAN_STAGE && HAS_R) {
      if (want_r) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const int idx = tid + 256 * k, r = idx / (BN / 8), q = idx - r * (BN / 8);
          const long long m = min(m_base + r, a.M - 1);
          const int n0 = min(n_base + q * 8, a.N - 8);
          rv[k] = *(const uint4*)((const uint16_t*)a.resid + m * a.ldr + n0);
        }
      }
    }
    if constexpr (EPI == GE_CONV && CAN_STAGE) {
      if (tid < BN && (a.flags & 2)) {
        const int n = min(n_base + tid, a.N - 1);
        bnr[0] = gm_ld<DT>(a.bn_w, n);
        bnr[1] = gm_ld<DT>(a.bn_b, n);
        bnr[2] = gm_ld<DT>(a.bn_mean, n);
        bnr[3] = gm_ld<DT>(a.bn_var, n);
      }
    }
  };
  bool stage_ops_loaded = false;
  auto load_resid = [&](const int j0, const int j1) {   // column groups [j0, j1)
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      const int n = min(n_base + wc * WN + j * 32 + fr, a.N - 1);
#pragma unroll
      for (int i = 0; i < (HAS_R && !CAN_STAGE ? TI : 1); ++i)
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          uint32_t w = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int e = 2 * e2 + h;
            const long long m = min(m_base + wr * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3), a.M - 1);
            w |= (uint32_t)((const uint16_t*)a.resid)[m * a.ldr + n] << (16 * h);
          }
          rr[j][i][e2] = w;
        }
    }
  };
  if constexpr (!DMA) {
    auto compute = [&](const int buf) {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        uint4 af[TI], bfr[NW][TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i) af[i] = *(const uint4*)&As[buf][wr * WM + i * 32 + fr][ks * 16 + fk];
#pragma unroll
        for (int u = 0; u < NW; ++u)
#pragma unroll
          for (int j = 0; j < TJ; ++j)
            bfr[u][j] = *(const uint4*)&Bs[buf][u * BN + wc * WN + j * 32 + fr][ks * 16 + fk];
#pragma unroll
        for (int u = 0; u < NW; ++u)
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[u][i][j] = gm_mfma<DT>(af[i], bfr[u][j], acc[u][i][j]);
      }
    };
    GM_LOAD_STEP(0);
    GM_STORE_STEP(0);
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
      const int buf = s & 1;
      if (s + 1 < nsteps) GM_LOAD_STEP((s + 1) * BK);
      compute(buf);
      if (s + 1 < nsteps) GM_STORE_STEP(buf ^ 1);
      __syncthreads();
    }
  } else {
    // wave w fills rows [w * 8 * NA, (w + 1) * 8 * NA) of A and [w * 8 * NB, ...) of B; one
    // instruction writes 8 rows (1 KB): lane l -> row 8 * blk + l / 8, slot l % 8, which holds
    // chunk (l % 8) ^ gm_swz(row), so the lane fetches that chunk
    constexpr int NA = BM / 32, NB = BNT / 32;   // DMA instructions per wave and step
    const unsigned lds0 = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&Ls[0];
    const int lr = lane >> 3, ls = lane & 7;
    const char* asrc[NA];
    const char* bsrc[NB];
    int ghi[CV ? NA : 1], gwi[CV ? NA : 1];   // CV: top-left input tap of the row's pixel
    long long gpb[CV ? NA : 1];               // CV: element offset of (n, ghi, gwi) (+ the lane's chunk for CV 1)
    int lcs[CV ? NA : 1];                     // CV: the 16-byte chunk of the step this lane fetches
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const int row = (wave * NA + q) * 8 + lr;
      const long long m = min(m_base + row, a.M - 1);
      asrc[q] = (const char*)(X + m * a.ldx) + ((ls ^ gm_swz(row)) * 16);
      if constexpr (CV) {
        const int HoWo = a.cHo * a.cWo, mi = (int)m;
        const int n = mi / HoWo, p = mi - n * HoWo, ho = p / a.cWo, wo = p - ho * a.cWo;
        ghi[q] = ho * a.csh - a.cph;
        gwi[q] = wo * a.csw - a.cpw;
        lcs[q] = ls ^ gm_swz(row);
        gpb[q] = (((long long)n * a.cH + ghi[q]) * a.cW + gwi[q]) * a.cCin + (CV == 1 ? lcs[q] * 8 : 0);
      }
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int row = (wave * NB + q) * 8 + lr;
      const uint16_t* wrow;
      if constexpr (GRP) {
        wrow = W0 + (long long)(min(n_base + row, g_hi - 1) - g_lo) * a.ldw;
      } else {
        const int u = row / BN, n = min(n_base + row % BN, a.N - 1);
        wrow = (u == 0 ? W0 : W1) + (long long)n * a.ldw;
      }
      bsrc[q] = (const char*)wrow + ((ls ^ gm_swz(row)) * 16);
    }
    auto issue = [&](int st) {   // stage st of the K loop into LDS buffer st % LST
      const unsigned base = lds0 + (unsigned)((st % LST) * SSTAGE) * 2u;
      const long long kb = (long long)st * BK * 2;
      if constexpr (CV == 2) {   // chunk t of the K range: kernel row t / cpr, taps 2 (t % cpr), + 1
        const int cpr = a.cKW * a.cCin / 8;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          const int kt = kbeg / 8 + st * 8 + lcs[q], kh = kt / cpr, kwc = kt - kh * cpr;
          const uint16_t* src = (const uint16_t*)a.x + gpb[q] + (long long)kh * a.cW * a.cCin + kwc * 8;
          gm_dma16(src, __builtin_amdgcn_readfirstlane(base + (unsigned)((wave * NA + q) * 8 * SROW * 2)));
        }
      } else if constexpr (CV == 1) {   // one tap and one 64-channel block per step (uniform)
        const int k = kbeg + st * BK;
        const int tap = k / a.cCin, c0 = k - tap * a.cCin;
        const int kh = tap / a.cKW, kw = tap - kh * a.cKW;
        const long long toff = ((long long)kh * a.cW + kw) * a.cCin + c0;
#pragma unroll
        for (int q = 0; q < NA; ++q) {
          const int hi = ghi[q] + kh, wi = gwi[q] + kw;
          const bool ok = (unsigned)hi < (unsigned)a.cH && (unsigned)wi < (unsigned)a.cW;
          const char* src = ok ? (const char*)((const uint16_t*)a.x + gpb[q] + toff) : (const char*)a.zero;
          gm_dma16(src, __builtin_amdgcn_readfirstlane(base + (unsigned)((wave * NA + q) * 8 * SROW * 2)));
        }
      } else {
#pragma unroll
        for (int q = 0; q < NA; ++q)
          gm_dma16(asrc[q] + kb, __builtin_amdgcn_readfirstlane(base + (unsigned)((wave * NA + q) * 8 * SROW * 2)));
      }
#pragma unroll
      for (int q = 0; q < NB; ++q)
        gm_dma16(bsrc[q] + kb, __builtin_amdgcn_readfirstlane(base + (unsigned)((BM + (wave * NB + q) * 8) * SROW * 2)));
    };
    auto compute = [&](const int buf) {
      const uint16_t* LA = Ls + buf * SSTAGE;
      const uint16_t* LB = LA + BM * SROW;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int c = ks * 2 + (lane >> 5);   // this lane's 16-byte chunk of the 64-element row
        uint4 af[TI], bfr[NW][TJ];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
          const int r = wr * WM + i * 32 + fr;
          af[i] = *(const uint4*)&LA[r * SROW + ((c ^ gm_swz(r)) * 8)];
        }
#pragma unroll
        for (int u = 0; u < NW; ++u)
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            const int r = u * BN + wc * WN + j * 32 + fr;
            bfr[u][j] = *(const uint4*)&LB[r * SROW + ((c ^ gm_swz(r)) * 8)];
          }
#pragma unroll
        for (int u = 0; u < NW; ++u)
#pragma unroll
          for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) acc[u][i][j] = gm_mfma<DT>(af[i], bfr[u][j], acc[u][i][j]);
      }
    };
    constexpr int NI = NA + NB;   // vmcnt per stage
    // (kernels with the row-chunk epilogue load their residuals there instead)
    if constexpr (HAS_R && !CAN_STAGE)
      if (want_r && a.ksplit == 1) load_resid(0, TJ);   // issued first: the first stage's wait covers them
    if constexpr (CAN_STAGE)
      if (staged) {
        load_stage_operands();
        stage_ops_loaded = true;
      }
    if constexpr (LST == 1) {
      for (int s = 0; s < nsteps; ++s) {
        if (s > 0) __syncthreads();   // every wave is done with step s - 1's buffer
        issue(s);
        gm_vmcnt<0>();
        __syncthreads();   // every wave's part of step s is in LDS
        compute(0);
      }
    } else {
#pragma unroll
      for (int st = 0; st < STAGES - 1; ++st)
        if (st < nsteps) issue(st);
      for (int s = 0; s < nsteps; ++s) {
        // stage s has landed when at most the stages issued after it are outstanding
        gm_vmcnt_after<NI, STAGES - 2>(min(nsteps - 1 - s, STAGES - 2));
        __syncthreads();   // every wave's part of stage s is in LDS; every wave is done with step s - 1
        if (s + STAGES - 1 < nsteps) issue(s + STAGES - 1);   // into the buffer step s - 1 used
        compute(s % STAGES);
      }
    }
    gm_vmcnt<0>();
  }

  if (a.ksplit > 1) {   // raw fp32 partial sums; k_gemm_reduce_* applies the epilogue
#pragma unroll
    for (int u = 0; u < NW; ++u)
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int n = n_base + wc * WN + j * 32 + fr;
        if (n >= a.N) continue;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const long long m = m_base + wr * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
            if (m < a.M) a.part[(((long long)kz * NW + u) * a.M + m) * a.N + n] = acc[u][i][j][e];
          }
      }
    return;
  }
  // Row-chunk epilogue: the accumulators leave the MFMA layout (one column per lane, rows across
  // registers) through LDS, so that residual loads and output stores are 16 bytes of 8 columns of
  // one row each instead of 2-byte accesses spread over rows. round(acc + bias) is the first rounding
  // point, so holding it as a 16-bit value in LDS changes nothing; batch norm factors are computed
  // once per column. Residual chunks are loaded first, so their latency overlaps the LDS work.
  if constexpr (CAN_STAGE) {
    if (staged) {
      constexpr int TLD = BN + 8;               // padded row: the two half-waves' writes miss each other's banks
      uint16_t* T;
      if constexpr (DMA) T = Ls;
      else T = &As[0][0][0];
      float* F = (float*)(T + BM * TLD);
      if (!stage_ops_loaded) load_stage_operands();
      __syncthreads();   // every wave is done with the operand buffers
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int col = wc * WN + j * 32 + fr, n = n_base + col;
        const float b0 = ((a.flags & 1) && n < a.N) ? gm_ld<DT>(a.bias, n) : 0.f;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            T[(wr * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3)) * TLD + col] =
                gm_pack<DT>(acc[0][i][j][e] + b0);
      }
      if constexpr (EPI == GE_CONV) {
        if (tid < BN && (a.flags & 2)) {   // inference batch norm v * al + be (gm_bn_factors)
          const float al = bnr[0] / sqrtf(bnr[3] + a.eps);
          F[tid] = al;
          F[BN + tid] = bnr[1] - bnr[2] * al;
        }
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int idx = tid + 256 * k, r = idx / (BN / 8), q = idx - r * (BN / 8);
        const long long m = m_base + r;
        const int n0 = n_base + q * 8;
        if (m >= a.M || n0 >= a.N) continue;
        const uint4 tv = *(const uint4*)&T[r * TLD + q * 8];
        const uint32_t tw[4] = {tv.x, tv.y, tv.z, tv.w}, rw[4] = {rv[k].x, rv[k].y, rv[k].z, rv[k].w};
        uint32_t ow[4];
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          uint32_t o = 0;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = 2 * c2 + h;
            const uint16_t tb = (uint16_t)(tw[c2] >> (16 * h));
            float v = DT == HS_BF16 ? bf16_to_f32(tb) : f16_to_f32(tb);
            const uint16_t rb = want_r ? (uint16_t)(rw[c2] >> (16 * h)) : (uint16_t)0;
            if constexpr (EPI == GE_RESID) v = gm_round<DT>((DT == HS_BF16 ? bf16_to_f32(rb) : f16_to_f32(rb)) + v);
            if constexpr (EPI == GE_CONV) {
              const float al = (a.flags & 2) ? F[q * 8 + c] : 1.f, be = (a.flags & 2) ? F[BN + q * 8 + c] : 0.f;
              v = gm_conv_tail<DT>(a, v, al, be, rb);
            }
            o |= (uint32_t)gm_pack<DT>(v) << (16 * h);
          }
          ow[c2] = o;
        }
        *(uint4*)(OUT + m * a.ldo + n0) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
      return;
    }
  }
  // epilogue (register staging: one column group's residuals at a time, which keeps the epilogue
  // under the main loop's register count)
  if constexpr (HAS_R && !CAN_STAGE) {
    if (!want_r) {
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int e2 = 0; e2 < 8; ++e2) rr[j][i][e2] = 0;
    }
  }
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    if constexpr (HAS_R && !CAN_STAGE)
      if (want_r) load_resid(j, j + 1);
    const int n = n_base + wc * WN + j * 32 + fr;
    if (n >= a.N) continue;
    const float b0 = (a.flags & 1) ? gm_ld<DT>(g_bias, n - g_lo) : 0.f;
    const float b1 = (EPI == GE_SILU && (a.flags & 2)) ? gm_ld<DT>(a.bias2, n) : 0.f;
    float al = 1.f, be = 0.f;   // conv: inference batch norm v * al + be (the conv.hip factors)
    if (EPI == GE_CONV && (a.flags & 2)) gm_bn_factors<DT>(a, n, al, be);
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const long long m = m_base + wr * WM + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
        if (m >= a.M) continue;
        float v = gm_round<DT>(acc[0][i][j][e] + b0);
        // (kernels with the row-chunk epilogue come here only for odd shapes: plain loads, fewer registers)
        uint16_t r16 = 0;
        if constexpr (HAS_R && CAN_STAGE) {
          if (want_r) r16 = ((const uint16_t*)a.resid)[m * a.ldr + n];
        } else if constexpr (HAS_R) {
          r16 = (uint16_t)(rr[j][i][e >> 1] >> (16 * (e & 1)));
        }
        if constexpr (EPI == GE_RESID) v = gm_round<DT>((DT == HS_BF16 ? bf16_to_f32(r16) : f16_to_f32(r16)) + v);
        if constexpr (EPI == GE_CONV) v = gm_conv_tail<DT>(a, v, al, be, r16);
        if constexpr (EPI == GE_SILU) {
          const float up = gm_round<DT>(acc[NW - 1][i][j][e] + b1);
          const float sg = gm_round<DT>(v / (1.f + expf(-v)));
          v = gm_round<DT>(sg * up);
        }
        OUT[m * a.ldo + n] = gm_pack<DT>(v);
      }
    }
  }
}

#undef GM_LOAD_STEP
#undef GM_STORE_STEP
#undef GM_LOAD_INTO
#undef GM_STORE_FROM

// Split-K reduction and epilogue: one thread per output element (fixed summation order).
template <int DT, int EPI>
__device__ __forceinline__ void gemm_reduce_body(const GemmArgs& a) {
  const long long total = a.M * a.N;
  const long long plane = total;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long m = i / a.N;
    const int n = (int)(i % a.N);
    float g = 0.f, up = 0.f;
    for (int z = 0; z < a.ksplit; ++z) {
      g += a.part[((long long)z * a.nw) * plane + i];
      if constexpr (EPI == GE_SILU) up += a.part[((long long)z * a.nw + 1) * plane + i];
    }
    float v = gm_round<DT>(g + ((a.flags & 1) ? gm_ld<DT>(a.bias, n) : 0.f));
    if constexpr (EPI == GE_RESID) v = gm_round<DT>(gm_ld<DT>(a.resid, m * a.ldr + n) + v);
    if constexpr (EPI == GE_CONV) {
      float al = 1.f, be = 0.f;
      if (a.flags & 2) gm_bn_factors<DT>(a, n, al, be);
      v = gm_conv_tail<DT>(a, v, al, be, (a.flags & 4) ? ((const uint16_t*)a.resid)[m * a.ldr + n] : (uint16_t)0);
    }
    if constexpr (EPI == GE_SILU) {
      const float u = gm_round<DT>(up + ((a.flags & 2) ? gm_ld<DT>(a.bias2, n) : 0.f));
      const float sg = gm_round<DT>(v / (1.f + expf(-v)));
      v = gm_round<DT>(sg * u);
    }
    ((uint16_t*)a.out)[m * a.ldo + n] = gm_pack<DT>(v);
  }
}

// Split-K reduce with the residual epilogue, fused with the RMSNorm that reads its result (the
// next norm of a transformer layer): one workgroup per row, thread t owns the 16-byte column
// chunk t (N <= 2048). Its residual, norm weight and the partials of up to 8 splits are loaded
// in one round. Each element sums its partials in split order and is rounded as GE_RESID rounds
// it (as gemm_reduce_body); the row is stored and staged in LDS, and wave 0 takes the sum of
// squares over it in k_rmsnorm_w's lane and chunk order, so both outputs equal those of the
// reduce kernel followed by k_rmsnorm_w bit for bit, with one launch and one pass less.
template <int DT>
__device__ __forceinline__ void reduce_norm_body(const ReduceNormArgs& a) {
  __shared__ float xs[2048];
  __shared__ float rsh;
  const long long row = blockIdx.x;
  const int t = threadIdx.x;
  const int nch = a.N / 8;
  const bool own = t < nch;
  const int c = own ? t : 0;   // idle threads re-read chunk 0 and store nothing
  const long long plane = a.M * (long long)a.N;
  const float* p = a.part + row * a.N + 8 * c;
  const uint4 r = *(const uint4*)((const uint16_t*)a.resid + row * a.ldr + 8 * c);
  const uint4 g = *(const uint4*)((const uint16_t*)a.norm_w + 8 * c);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int z0 = 0; z0 < a.ksplit; z0 += 8) {
    float4 u[8], v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {   // past the last split: re-read it (not added)
      const long long z = min(z0 + j, a.ksplit - 1);
      u[j] = *(const float4*)(p + z * plane);
      v[j] = *(const float4*)(p + z * plane + 4);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (z0 + j >= a.ksplit) break;   // workgroup-uniform
      acc[0] += u[j].x; acc[1] += u[j].y; acc[2] += u[j].z; acc[3] += u[j].w;
      acc[4] += v[j].x; acc[5] += v[j].y; acc[6] += v[j].z; acc[7] += v[j].w;
    }
  }
  const uint32_t rq[4] = {r.x, r.y, r.z, r.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float b = (a.flags & 1) ? gm_ld<DT>(a.bias, 8 * c + e) : 0.f;
    const float v = gm_round<DT>(acc[e] + b);
    const uint16_t rb = (uint16_t)(rq[e >> 1] >> (16 * (e & 1)));
    acc[e] = gm_round<DT>((DT == HS_BF16 ? bf16_to_f32(rb) : f16_to_f32(rb)) + v);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = (uint32_t)gm_pack<DT>(acc[2 * k]) | ((uint32_t)gm_pack<DT>(acc[2 * k + 1]) << 16);
  if (own) {
    *(uint4*)((uint16_t*)a.out + row * a.ldo + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[8 * c + e] = acc[e];
  }
  __syncthreads();
  if (t < 64) {   // k_rmsnorm_w's order: lane l sums chunks l, l + 64, ... element by element
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cc = t + 64 * k;
      if (cc >= nch) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += xs[8 * cc + e] * xs[8 * cc + e];
    }
    ss = wave_sum(ss);
    if (t == 0) rsh = 1.0f / sqrtf(ss / (float)a.N + a.eps);
  }
  __syncthreads();
  if (!own) return;
  const float rs = rsh;
  const uint32_t gq[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t w2 = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float n = round_to(acc[2 * k + h] * rs, a.n_dtype);
      const uint16_t gb = (uint16_t)(gq[k] >> (16 * h));
      w2 |= (uint32_t)gm_pack<DT>((DT == HS_BF16 ? bf16_to_f32(gb) : f16_to_f32(gb)) * n) << (16 * h);
    }
    o[k] = w2;
  }
  *(uint4*)((uint16_t*)a.norm_out + row * a.ldn + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
}

extern "C" __global__ void __launch_bounds__(256) k_gemm_reduce_bf16_resid_norm(const ReduceNormArgs a) {
  reduce_norm_body<HS_BF16>(a);
}
extern "C" __global__ void __launch_bounds__(256) k_gemm_reduce_f16_resid_norm(const ReduceNormArgs a) {
  reduce_norm_body<HS_F16>(a);
}

// up to 2 waves per SIMD: the 64 accumulator registers plus staging and fragments need
// more than the default register budget, which would otherwise spill the staging to scratch
#define GM_ATTRS __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
// Each kernel comes in two K steps: 32, and 64 (suffix _k64: twice the MFMA work per barrier and
// per prefetch, which hides the operand latency better; 73.7 KB of LDS for 128 x 128 tiles, so two
// workgroups still share a CU). Measured at M = 512, K = 1536: lm_head 381 -> 312 us, gate/up
// 61 -> 51 us; K = 8960 down 39 -> 30 us. The host takes _k64 when K (and the split-K chunk) is a
// multiple of 64. Suffix _k64d: K step 64 with direct-to-LDS staging, ST buffers deep (the stage
// count fits two workgroups per CU where the tile allows). Measured at M = 512 (same launch,
// bit-identical results): gate/up 64 x 64 57 -> 52 us, down 128 x 128 with 4 K splits 31 -> 26 us,
// o_proj 64 x 64 with 2 K splits 15.8 -> 9.5 us, q | k | v 14.6 -> 11.4 us; the lm_head's 4,748
// tiles of 128 x 128 keep enough workgroups in flight without it (324 us against 367).
#define GEMM_KERNEL(NAME, DT, EPI, NW, BM, BN, ST)                                                      \
  extern "C" __global__ void GM_ATTRS NAME(const GemmArgs a) { gemm_body<DT, EPI, NW, BM, BN>(a); }     \
  extern "C" __global__ void GM_ATTRS NAME##_k64(const GemmArgs a) { gemm_body<DT, EPI, NW, BM, BN, false, 64>(a); } \
  extern "C" __global__ void GM_ATTRS NAME##_k64d(const GemmArgs a) {                                  \
    gemm_body<DT, EPI, NW, BM, BN, false, 64, false, ST>(a);                                           \
  }
#define GEMM_KERNEL_KN(NAME, DT, BM, BN)                                                                  \
  extern "C" __global__ void GM_ATTRS NAME(const GemmArgs a) { gemm_body<DT, GE_BIAS, 1, BM, BN, true>(a); } \
  extern "C" __global__ void GM_ATTRS NAME##_k64(const GemmArgs a) { gemm_body<DT, GE_BIAS, 1, BM, BN, true, 64>(a); }
#define GEMM_REDUCE(NAME, DT, EPI) \
  extern "C" __global__ void __launch_bounds__(256) NAME(const GemmArgs a) { gemm_reduce_body<DT, EPI>(a); }

// k_gemm_<dtype>_<epilogue>_m<BM>n<BN>: BN columns per weight; last argument: direct-to-LDS stages
GEMM_KERNEL(k_gemm_bf16_bias_m128n128, HS_BF16, GE_BIAS, 1, 128, 128, 4)
GEMM_KERNEL(k_gemm_bf16_bias_m64n128, HS_BF16, GE_BIAS, 1, 64, 128, 3)
GEMM_KERNEL(k_gemm_bf16_bias_m64n64, HS_BF16, GE_BIAS, 1, 64, 64, 4)
GEMM_KERNEL(k_gemm_bf16_resid_m128n128, HS_BF16, GE_RESID, 1, 128, 128, 4)
GEMM_KERNEL(k_gemm_bf16_resid_m64n128, HS_BF16, GE_RESID, 1, 64, 128, 3)
GEMM_KERNEL(k_gemm_bf16_resid_m64n64, HS_BF16, GE_RESID, 1, 64, 64, 4)
GEMM_KERNEL(k_gemm_bf16_silu_m128n64, HS_BF16, GE_SILU, 2, 128, 64, 3)
GEMM_KERNEL(k_gemm_bf16_silu_m64n64, HS_BF16, GE_SILU, 2, 64, 64, 3)
GEMM_KERNEL(k_gemm_f16_bias_m128n128, HS_F16, GE_BIAS, 1, 128, 128, 4)
GEMM_KERNEL(k_gemm_f16_bias_m64n128, HS_F16, GE_BIAS, 1, 64, 128, 3)
GEMM_KERNEL(k_gemm_f16_bias_m64n64, HS_F16, GE_BIAS, 1, 64, 64, 4)
GEMM_KERNEL(k_gemm_f16_resid_m128n128, HS_F16, GE_RESID, 1, 128, 128, 4)
GEMM_KERNEL(k_gemm_f16_resid_m64n128, HS_F16, GE_RESID, 1, 64, 128, 3)
GEMM_KERNEL(k_gemm_f16_resid_m64n64, HS_F16, GE_RESID, 1, 64, 64, 4)
// direct-to-LDS only, the 4 waves as 4 rows x 1 column (wave tile BM / 4 x BN per weight): for tile
// widths that are an odd multiple of 32 (BN = 96: 94 column tiles of a 8960-row weight pair, so
// M = 512 takes 376 workgroups, one round at two per CU; a 1536-row weight over K = 8960, 64
// tiles x 8 K splits, one round of 512)
#define GEMM_KERNEL_W4(NAME, DT, EPI, NW, BM, BN, ST)                                                   \
  extern "C" __global__ void GM_ATTRS NAME##_k64d(const GemmArgs a) {                                  \
    gemm_body<DT, EPI, NW, BM, BN, false, 64, false, ST, 0, 4>(a);                                     \
  }
GEMM_KERNEL_W4(k_gemm_bf16_silu_m128n96, HS_BF16, GE_SILU, 2, 128, 96, 2)
GEMM_KERNEL_W4(k_gemm_f16_silu_m128n96, HS_F16, GE_SILU, 2, 128, 96, 2)
GEMM_KERNEL_W4(k_gemm_bf16_resid_m128n96, HS_BF16, GE_RESID, 1, 128, 96, 2)
GEMM_KERNEL_W4(k_gemm_f16_resid_m128n96, HS_F16, GE_RESID, 1, 128, 96, 2)
GEMM_KERNEL_W4(k_gemm_bf16_bias_m128n96, HS_BF16, GE_BIAS, 1, 128, 96, 2)
GEMM_KERNEL_W4(k_gemm_f16_bias_m128n96, HS_F16, GE_BIAS, 1, 128, 96, 2)

// grouped (q | k | v projections of one activation into one [M, N] output; no split K)
#define GEMM_KERNEL_GRP(NAME, DT, BM, BN, ST)                                                                  \
  extern "C" __global__ void GM_ATTRS NAME(const GemmArgs a) { gemm_body<DT, GE_BIAS, 1, BM, BN, false, 32, true>(a); } \
  extern "C" __global__ void GM_ATTRS NAME##_k64(const GemmArgs a) { gemm_body<DT, GE_BIAS, 1, BM, BN, false, 64, true>(a); } \
  extern "C" __global__ void GM_ATTRS NAME##_k64d(const GemmArgs a) {                                              \
    gemm_body<DT, GE_BIAS, 1, BM, BN, false, 64, true, ST>(a);                                                     \
  }
// conv2d on channels-last activations (conv epilogue): _conv takes x as the [pixels, Cin] rows of
// an NHWC image (1 x 1, stride 1, no padding); _convg gathers the taps of any kernel / stride /
// padding (Cin % 64 == 0) with direct-to-LDS staging; _convp reads a zero-bordered 4-channel image
// (a network's first conv on a 3-channel input, after k_pad_nhwc4)
// direct-to-LDS convs: no cap on waves per SIMD (their registers fit 8), so the workgroups a CU's
// LDS holds all run (four 64 x 64 tiles at two stages were seen resident, three 128 x 64):
// short-K convs spend most of a tile waiting on its loads and its stores, which other resident
// workgroups overlap
// (ResNet-50 b32: 64 x 64 tiles on 56 x 56 1 x 1 convs 44 -> 34 us; the 7 x 7 stem 55 -> 45 us)
#ifndef GM_CONV_WPE
#define GM_CONV_WPE 8
#endif
#define GM_ATTRS_CONV __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, GM_CONV_WPE)))
#define GEMM_CONV(DTN, DT, BM, BN, ST)                                                                              \
  extern "C" __global__ void GM_ATTRS k_gemm_##DTN##_conv_m##BM##n##BN##_k64(const GemmArgs a) {                    \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64>(a);                                                                \
  }                                                                                                                 \
  extern "C" __global__ void GM_ATTRS_CONV k_gemm_##DTN##_conv_m##BM##n##BN##_k64d(const GemmArgs a) {              \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64, false, ST>(a);                                                     \
  }                                                                                                                 \
  extern "C" __global__ void GM_ATTRS_CONV k_gemm_##DTN##_convg_m##BM##n##BN##_k64d(const GemmArgs a) {             \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64, false, ST, 1>(a);                                                  \
  }                                                                                                                 \
  extern "C" __global__ void GM_ATTRS_CONV k_gemm_##DTN##_conv_m##BM##n##BN##_k64d2(const GemmArgs a) {             \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64, false, 2>(a);                                                      \
  }                                                                                                                 \
  extern "C" __global__ void GM_ATTRS_CONV k_gemm_##DTN##_convg_m##BM##n##BN##_k64d2(const GemmArgs a) {            \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64, false, 2, 1>(a);                                                   \
  }                                                                                                                 \
  extern "C" __global__ void GM_ATTRS_CONV k_gemm_##DTN##_convp_m##BM##n##BN##_k64d2(const GemmArgs a) {            \
    gemm_body<DT, GE_CONV, 1, BM, BN, false, 64, false, 2, 2>(a);                                                   \
  }
// short K (1 x 1 convs over few channels): the LDS of one stage, 16 KB at 64 x 64, so up to eight
// workgroups share a CU
extern "C" __global__ void GM_ATTRS_CONV k_gemm_f16_conv_m64n64_k64d1(const GemmArgs a) {
  gemm_body<HS_F16, GE_CONV, 1, 64, 64, false, 64, false, 2, 0, 2, 1>(a);
}
extern "C" __global__ void GM_ATTRS_CONV k_gemm_bf16_conv_m64n64_k64d1(const GemmArgs a) {
  gemm_body<HS_BF16, GE_CONV, 1, 64, 64, false, 64, false, 2, 0, 2, 1>(a);
}
GEMM_CONV(f16, HS_F16, 128, 128, 4)
GEMM_CONV(f16, HS_F16, 128, 64, 3)
GEMM_CONV(f16, HS_F16, 64, 128, 3)
GEMM_CONV(f16, HS_F16, 64, 64, 4)
GEMM_CONV(bf16, HS_BF16, 128, 128, 4)
GEMM_CONV(bf16, HS_BF16, 128, 64, 3)
GEMM_CONV(bf16, HS_BF16, 64, 128, 3)
GEMM_CONV(bf16, HS_BF16, 64, 64, 4)
GEMM_REDUCE(k_gemm_reduce_f16_conv, HS_F16, GE_CONV)
GEMM_REDUCE(k_gemm_reduce_bf16_conv, HS_BF16, GE_CONV)
GEMM_KERNEL_GRP(k_gemm_bf16_grp_m64n64, HS_BF16, 64, 64, 4)
GEMM_KERNEL_GRP(k_gemm_bf16_grp_m128n128, HS_BF16, 128, 128, 4)
GEMM_KERNEL_GRP(k_gemm_f16_grp_m64n64, HS_F16, 64, 64, 4)
GEMM_KERNEL_GRP(k_gemm_f16_grp_m128n128, HS_F16, 128, 128, 4)
GEMM_REDUCE(k_gemm_reduce_bf16_bias, HS_BF16, GE_BIAS)
GEMM_REDUCE(k_gemm_reduce_bf16_resid, HS_BF16, GE_RESID)
GEMM_REDUCE(k_gemm_reduce_bf16_silu, HS_BF16, GE_SILU)
GEMM_REDUCE(k_gemm_reduce_f16_bias, HS_F16, GE_BIAS)
GEMM_REDUCE(k_gemm_reduce_f16_resid, HS_F16, GE_RESID)
// batched matmuls (attention at prefill): B given as [K, N] (row-major, N % 8 == 0)
GEMM_KERNEL_KN(k_gemm_bf16_bias_m64n64_kn, HS_BF16, 64, 64)
GEMM_KERNEL_KN(k_gemm_bf16_bias_m128n128_kn, HS_BF16, 128, 128)
GEMM_KERNEL_KN(k_gemm_f16_bias_m64n64_kn, HS_F16, 64, 64)
GEMM_KERNEL_KN(k_gemm_f16_bias_m128n128_kn, HS_F16, 128, 128)
