// One decoder step of a Qwen2-style model in a single persistent launch (gfx950).
//
// The multi-kernel step is a chain of dependent launches per layer (RMSNorm + q/k/v + RoPE,
// attention, o_proj + residual, RMSNorm + gate/up + SiLU*mul, down + residual); every launch
// boundary costs a full drain and refill of the machine. Here one workgroup per CU runs every
// layer, and the dependencies between the parts of a layer are carried by the data itself:
//
//   * Exchange words: every activation a part hands to the next (q/k/v rows, attention
//     partials, the combined attention row, the residual stream, the SiLU*mul row) is written
//     as 32-bit words, the bf16 value in the low half and a 16-bit step tag in the high half,
//     with agent-scope atomic stores (one word per store: a reader never sees half a word).
//     A reader loads the words with agent-scope atomic loads and uses them once every word
//     carries the current step's tag; words not yet current are loaded again. There are no
//     counters, barriers or fences between workgroups.
//   * The step tag is the launch count (1..65535, never 0; the exchange area starts zeroed):
//     stale words from the previous step never match. Exchange slots are per layer, so a slot
//     is written once per step.
//   * Every wait is bounded: after 20 ms a workgroup records a timeout in the control word (and
//     in a host-visible word when the host passed one) and goes on, so the launch always ends; the
//     host checks the flag. The step is correct only with every workgroup resident at once (one
//     per CU): the host checks the device's CU count and the kernel's occupancy before using it.
//   * Weights (and the K/V rows of past positions) do not depend on the step's activations, so
//     each part issues its weight loads before it waits for its inputs: the wait overlaps the
//     weight stream instead of following it.
//
// Work split (NWG workgroups of 8 waves; all resident at once, one per CU):
//   A  q/k/v:      rows (H + 2 KVH) * D, at most 8 per workgroup, one per wave
//   B  attention:  workgroup (query head, slot) for slot < nsplit; slot j reads the 128-position
//                  chunks j, j + nsplit, ... that the mask leaves open (a chunk of -inf only is
//                  skipped: found once per step); the G heads of a KV head share its K/V rows in
//                  L2; partial (o / l, m, l)
//   C  combine:    one workgroup per query head merges the head's slot partials
//   D  o_proj:     hidden rows, at most 8 per workgroup, one per wave; + residual
//   E  gate/up:    inter rows spread over workgroups and waves; SiLU(gate) * up
//   F  down:       hidden rows, at most 8 per workgroup; the 8 waves split each row's K; + residual
//   G  lm_head:    final RMSNorm, vocab rows over all workgroups; logits and one argmax key per
//                  workgroup; workgroup 0 reduces the keys into the next token
// Rounding points are those of the multi-kernel path (and of ATen on the CPU): RMSNorm
// n = round(x * rsqrt(mean(x^2) + eps)), y = round(w * n); linear round(acc + b); RoPE
// round(round(x c) + round(-x' s)); attention scores round(round(round(q.k) * scale) + mask);
// residual round(r + round(acc)); SiLU*mul round(round(silu(round(g))) * round(u)). One
// difference: the head-major attention (dec_attend) keeps the probabilities exp(s - m) in fp32
// into P.V, where ATen's softmax rounds them to bf16 first; the KV-head-major form
// (dec_attend_kv) rounds them to bf16, as its MFMA operand.
#include "common.h"

#define DEC_THREADS 512
#define DEC_WAVES 8
#define DEC_D 128
#define DEC_SPL 128                   // positions per attention chunk: 8 waves x 16
#define DEC_MAXG 8                    // query heads per KV head, at most
#define DEC_TIMEOUT 2000000ull        // 20 ms of the 100 MHz real-time counter
#define DEC_OSTAGE 128                // o_proj or gate / up rows of one workgroup, at most
#ifndef DEC_ED
#define DEC_ED 3                      // gate/up rows in flight per wave (2: 0.780 ms, 3: 0.766 ms per step)
#endif
// down_proj rows per workgroup issued while E computes, of its 2 KC: they land before the h
// stores, so F streams fewer bytes after the SiLU * up row is out. DEC_RFE_N of them are issued
// once x1 is normalised, the rest once the LDS rows are summed (issuing a wave's loads stalls it
// while the memory pipe is full, so they are spread over E). 0.714 -> 0.690 ms per step with 2
// issued as soon as x1 is in (1: 0.695, 3: 0.700, 4: 0.705, 6: 0.721: the h stores queue behind
// the later ones); 0.681 with 1 + 1 (2 + 1: 0.683, 2 + 2: 0.692, 2 + 0: 0.690, 0 + 2: 0.686).
// With the current schedule, 4 A/B rounds on one box, kernel µs per launch: 1 + 2 666.1-667.0,
// 1 + 1 666.9-667.9, 2 + 1 667.5-668.7, 2 + 0 670.4-670.9, 1 + 3 679.0-679.8, 1 + 0 about 680.
#ifndef DEC_RFE
#define DEC_RFE 3
#endif
#ifndef DEC_RFE_N
#define DEC_RFE_N 1
#endif
#ifndef DEC_R4
#define DEC_R4 2                      // lm_head rows per wave in each of its two rounds in flight
#endif
#ifndef DEC_EARLY
#define DEC_EARLY 1   // o_proj workgroups issue E's first ring rows with their o_proj rows (0: 0.730 ms, 1: 0.717)
#endif
#define DEC_NE(KC) ((KC) == 3 ? 24 : ((KC) == 2 ? 32 : 48))   // gate/up rows in LDS per attention workgroup
#define DEC_SMEM (32 * (DEC_D + 4) * 2)   // per-part staging: the combine's partials of up to 32 slots

typedef __attribute__((ext_vector_type(2))) __bf16 dec_bf16x2;
typedef unsigned int dec_u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float ddot8(const uint4 a, const uint4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a.x), __builtin_bit_cast(dec_bf16x2, b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a.y), __builtin_bit_cast(dec_bf16x2, b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a.z), __builtin_bit_cast(dec_bf16x2, b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a.w), __builtin_bit_cast(dec_bf16x2, b.w), acc, false);
  return acc;
}

__device__ __forceinline__ float ddot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(dec_bf16x2, a), __builtin_bit_cast(dec_bf16x2, b), acc, false);
}

// Global-memory accesses through pointers the compiler cannot place in an address space (those
// read from the LDS copy of the layer table): the explicit global address space makes them global
// instructions; as flat instructions they would also count against the LDS wait counter, and every
// LDS access would then wait for every load in flight.
#define DEC_G(T, p) ((__attribute__((address_space(1))) T*)(p))

// 16-byte weight load (streamed once per step: non-temporal)
__device__ __forceinline__ uint4 ldw(const uint16_t* p) {
  const dec_u32x4 v = __builtin_nontemporal_load(DEC_G(const dec_u32x4, p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldg16(const void* p) {   // (uint4's copy constructor would make it generic)
  const dec_u32x4 v = *DEC_G(const dec_u32x4, p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ldg4(const void* p) { return *DEC_G(const uint32_t, p); }
__device__ __forceinline__ uint16_t ldg2(const void* p) { return *DEC_G(const uint16_t, p); }
__device__ __forceinline__ void stg2(void* p, uint16_t v) { *DEC_G(uint16_t, p) = v; }

// Per-part copies of the thread and workgroup ids that the compiler cannot prove equal across
// parts, so per-lane address arithmetic is recomputed inside each part instead of being hoisted
// out of the layer loop and kept live (spilled) across all of them.
#define DEC_PART_IDS()                                  \
  int tid = threadIdx.x, b = blockIdx.x;                \
  asm volatile("" : "+v"(tid));                         \
  asm volatile("" : "+s"(b));                           \
  const int lane = tid & 63, wave = tid >> 6;           \
  (void)lane; (void)wave; (void)b

// Progress stamps (optional): thread 0 of each workgroup records the real-time counter at
// fixed points of each part, slot k of layer l at trace[b * (L * 16 + 8) + l * 16 + k]; the
// final part uses slots L * 16 + k. A null trace pointer skips them.
#define DEC_STAMP(l, k)                                                                          \
  do {                                                                                           \
    if (a.trace != nullptr && threadIdx.x == 0)                                                  \
      a.trace[(long long)blockIdx.x * (a.L * 16 + 8) + (l) * 16 + (k)] = wall_clock64();         \
  } while (0)

#ifndef DEC_PROBE_ROUNDS
#define DEC_PROBE_ROUNDS 0
#endif
#define DEC_STAMPV(l, k, v)                                                                      \
  do {                                                                                           \
    if (DEC_PROBE_ROUNDS && a.trace != nullptr && threadIdx.x == 0)                              \
      a.trace[(long long)blockIdx.x * (a.L * 16 + 8) + (l) * 16 + (k)] = (v);                    \
  } while (0)
#define DEC_STAMPT(l, k) do { if (!DEC_PROBE_ROUNDS) DEC_STAMP(l, k); } while (0)

__device__ __forceinline__ float rb(float f) { return bf16_to_f32(f32_to_bf16(f)); }
__device__ __forceinline__ float bfh(uint16_t h) { return bf16_to_f32(h); }

// ---------------------------------------------------------------- exchange words

__device__ __forceinline__ void xput(uint32_t* p, uint16_t v, uint32_t tag) {
  __hip_atomic_store(p, (tag << 16) | (uint32_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long xget2(const uint32_t* p) {
  return __hip_atomic_load((unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A wait timed out: the control word (read by the host after a synchronisation) and, when the
// host passed one, a word in host memory that the host can read at any time.
__device__ __forceinline__ void dec_fail(uint32_t* err, int* herr) {
  __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (herr != nullptr) __hip_atomic_store(herr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Waits until the n words at src (n even, src 8-byte aligned) carry `tag` and copies their
// payloads (bf16 bits) to dst. Thread t owns word pairs t + NTH j, j < NPT: all of its loads are
// issued together, and only the pairs not yet current are loaded again, after a short sleep (every
// consumer re-reading every pair multiplies the traffic on the few memory channels that hold a
// small exchange slot: 256 workgroups gathering the 8,960-word SiLU * up row took 4-5 us that way).
// Returns after a __syncthreads(), so dst is complete for the whole workgroup.
template <int NPT, int NTH = DEC_THREADS>
__device__ __forceinline__ int xgather(const uint32_t* src, int n, uint32_t tag, uint16_t* dst, uint32_t* err,
                                       int* herr, int tid) {
  if (tid >= NTH) {   // waves outside the gathering set only meet the barrier
    __syncthreads();
    return 0;
  }
  int rounds = 0;
  const int np = n >> 1;
  const unsigned long long want = ((unsigned long long)tag << 48) | ((unsigned long long)tag << 16);
  const unsigned long long tmask = 0xFFFF0000FFFF0000ull;
  unsigned long long v[NPT];
  // every pair of the thread is loaded in each round with no branch (pairs past the end re-read
  // the last one and count as current), so a round costs one memory latency, not one per pair
#pragma unroll
  for (int j = 0; j < NPT; ++j) v[j] = xget2(src + 2 * min(tid + NTH * j, np - 1));
  const unsigned long long t0 = wall_clock64();
  while (true) {
    bool ok = true;
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      ok = ok && ((v[j] & tmask) == want || tid + NTH * j >= np);
    if (ok) break;
    if (wall_clock64() - t0 > DEC_TIMEOUT) {
      dec_fail(err, herr);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    ++rounds;
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if ((v[j] & tmask) != want) v[j] = xget2(src + 2 * min(tid + NTH * j, np - 1));
  }
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int i = tid + NTH * j;
    if (i < np) *(uint32_t*)(dst + 2 * i) = (uint32_t)(v[j] & 0xFFFFu) | (uint32_t)((v[j] >> 16) & 0xFFFF0000u);
  }
#if DEC_PROBE_ROUNDS
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) rounds = max(rounds, __shfl_xor(rounds, o, 64));
#endif
  __syncthreads();
  return rounds;
}

// 16 bytes per lane from global memory straight into LDS at m0 + 16 * lane (gfx950), from inline
// assembly: the compiler does not count these loads, so it inserts no wait for them (before a
// barrier or an LDS read); the waves that issue them wait explicitly (dec_vmcnt0) before the
// data is read, and issue no other vector-memory loads in between.
__device__ __forceinline__ void dec_dma16(const void* g, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dec_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
#define DEC_STR2(x) #x
#define DEC_STR(x) DEC_STR2(x)
#define DEC_VMCNT(q) asm volatile("s_waitcnt vmcnt(" DEC_STR(q) ")" ::: "memory")
#ifndef DEC_LDS_Q
#define DEC_LDS_Q 0
#endif

// Word offsets of one layer's exchange slots (all even, so word pairs are 8-byte aligned).
struct XLayout {
  long long qkv, part, att, x1, h, stride;
};

__device__ __forceinline__ XLayout xlayout(const PersistArgs& a) {
  XLayout o;
  const long long hid = a.hidden, G = a.H / a.KVH;
  o.qkv = hid;                                                        // [x_l: hidden] then q/k/v
  o.part = o.qkv + (long long)a.H * 3 * DEC_D;                       // per query head: q, its k, its v
  o.att = o.part + (long long)a.H * a.nsplit * (DEC_D + 4);          // per head: nsplit x (o[D], m, l)
  o.x1 = o.att + (long long)a.H * DEC_D;
  o.h = o.x1 + hid;
  o.stride = o.h + a.inter;
  o.stride += o.stride & 1;
  return o;
}

// ---------------------------------------------------------------- E's register ring

// Row of the k-th gate / up row a wave streams through registers: rows rs + wave + 8 k for
// k < n; rows past the wave's last re-read it, and a wave without rows reads the matrix's last
// row, so every load of the ring is unconditional.
__device__ __forceinline__ long long ering_row(int k, int rs, int nr, int wave, int inter) {
  const int n = (nr - wave + DEC_WAVES - 1) / DEC_WAVES;
  const long long rlast = min(rs + wave + (long long)DEC_WAVES * max(n - 1, 0), (long long)inter - 1);
  return min(rs + wave + (long long)DEC_WAVES * k, rlast);
}

template <int KC>
__device__ __forceinline__ void ering_load(uint4 (&g)[KC], uint4 (&u)[KC], const uint16_t* wg, const uint16_t* wu,
                                           long long r, int hid, int lane) {
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    g[c] = ldw(wg + r * hid + c * 512 + lane * 8);
    u[c] = ldw(wu + r * hid + c * 512 + lane * 8);
  }
}

// ---------------------------------------------------------------- workgroup RMSNorm

// xs = round(w * round_n(x * rsqrt(mean(x^2) + eps))) over the hidden values of x (LDS, bf16);
// thread t < hidden / 8 owns chunk t, whose norm weight wv it loaded before its inputs arrived.
__device__ __forceinline__ void block_norm(const uint16_t* x, uint4 wv, int hid, float eps, int n_dtype,
                                           uint16_t* xs, float* red, int tid) {
  const int t = tid, nch = hid >> 3;
  uint4 xv = make_uint4(0, 0, 0, 0);
  float ss = 0.f;
  if (t < nch) {
    xv = *(const uint4*)(x + 8 * t);
    const uint32_t q[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = bfh((uint16_t)(q[j] & 0xffffu)), hi = bfh((uint16_t)(q[j] >> 16));
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float tot = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  const float r = 1.0f / sqrtf(tot / (float)hid + eps);
  if (t < nch) {
    const uint32_t q[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t g[4] = {wv.x, wv.y, wv.z, wv.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float n0 = round_to(bfh((uint16_t)(q[j] & 0xffffu)) * r, n_dtype);
      const float n1 = round_to(bfh((uint16_t)(q[j] >> 16)) * r, n_dtype);
      o[j] = (uint32_t)f32_to_bf16(bfh((uint16_t)(g[j] & 0xffffu)) * n0) |
             ((uint32_t)f32_to_bf16(bfh((uint16_t)(g[j] >> 16)) * n1) << 16);
    }
    *(uint4*)(xs + 8 * t) = make_uint4(o[0], o[1], o[2], o[3]);
  }
  __syncthreads();
}

// the layer's input row into xres: the token's embedding row (layer 0) or the exchange words
template <int KC>
__device__ __forceinline__ int load_x(const PersistArgs& a, int l, const uint32_t* xw, long long tok, uint32_t tag,
                                      uint16_t* xres, uint32_t* err, int* herr, int tid) {
  if (l == 0) {
    const int nch = a.hidden >> 3;
    if (tid < nch) *(uint4*)(xres + 8 * tid) = *(const uint4*)(a.emb + tok * a.hidden + 8 * tid);
    __syncthreads();
    return 0;
  }
  return xgather<(KC + 1) / 2>(xw, a.hidden, tag, xres, err, herr, tid);
}

__device__ __forceinline__ unsigned long long key48(uint16_t hbits, unsigned idx) {
  // order-preserving bf16 bits (NaN above every number, -0 == +0) over the inverted index
  const float v = bfh(hbits);
  uint32_t o = hbits;
  o = (v == 0.f) ? 0x8000u : ((o & 0x8000u) ? (~o & 0xFFFFu) : (o | 0x8000u));
  o = (v != v) ? 0xFFFFu : o;
  return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

// A layer's tensors from the LDS copy of its table entry.
__device__ __forceinline__ DecodeLayerPtrs dec_layer(const void* const* t) {
  DecodeLayerPtrs P;
  __builtin_memcpy(&P, t, sizeof(P));
  return P;
}

// The chunks of attention slot `slot`, the same for every layer: bit i stands for chunk
// slot + nsplit i, set when the mask opens a position of it (every chunk without a mask).
// Chunks whose positions are all -inf contribute exactly nothing to the softmax, so their K / V
// rows are never loaded; the loop over the open chunks is bounded by the mask, not by S.
// Wave w checks half a chunk per round (chunk 4 q + w / 2, positions 64 (w & 1) + lane), all
// eight rounds' loads issued together. With a mask, each wave's bits go to obw[wave] and the
// caller ORs them after a barrier (the return value is 0); without one the bits are returned.
__device__ __forceinline__ uint32_t dec_scan_chunks(const PersistArgs& a, int slot, uint32_t* obw, int lane, int wave) {
  const int NT = a.nsplit;
  const long long last = a.S - 1;
  const int nch = (a.nchunk - slot + NT - 1) / NT;   // chunks of this slot (<= 32, checked on the host)
  if (a.mask_dtype < 0) return nch >= 32 ? 0xFFFFFFFFu : ((1u << nch) - 1u);
  FRaw mr[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const long long p = (long long)(slot + NT * (4 * q + (wave >> 1))) * DEC_SPL + 64 * (wave & 1) + lane;
    mr[q] = ld_f_raw(a.mask, min(p, last), a.mask_dtype);
  }
  uint32_t bits = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = 4 * q + (wave >> 1);
    const long long p = (long long)(slot + NT * i) * DEC_SPL + 64 * (wave & 1) + lane;
    const bool open = i < nch && p <= last && ld_f_decode(mr[q], a.mask_dtype) != -INFINITY;
    if (__ballot(open) != 0ull) bits |= 1u << i;
  }
  if (lane == 0) obw[wave] = bits;
  return 0u;
}

// ---- B: attention of one query head over the open chunks (ob) of its slot ---------------------------
// The first open chunk's K rows and mask values do not depend on this step's activations, so
// they are issued before B waits for its q / k / v (after A, whose input poll would otherwise
// wait behind them); its V rows, needed last, are issued once q / k / v are in, so the poll
// does not wait behind them either and their latency overlaps the scores. Further open chunks
// (caches longer than 128 nsplit positions) are loaded and folded in one after another: each
// wave keeps a running (max, sum, unnormalised output) over its 16 positions of every chunk.
// qkvw: the head's exchange block (q | k | v); partw: the slot's partial; kcache / vcache: the
// layer's caches (this step's row written by the slot's first head when the slot holds it).
// VEARLY: the first chunk's V rows are issued with its K rows, before the wait (for a workgroup
// with no other loads of its own in flight, whose wait would end after they land anyway).
template <bool VEARLY = false>
__device__ __forceinline__ void dec_attend(const PersistArgs& a, int l, uint16_t* kcache, uint16_t* vcache,
                                           const uint32_t* qkvw, uint32_t* partw, uint32_t ob, int kvh, int gq,
                                           int slot, long long cpos, uint32_t tag, uint32_t* err,
                                           unsigned char* smem, const float* rope_cs, float* red, float* red2,
                                           int tid, int lane, int wave) {
  const int NT = a.nsplit;
  const long long S = a.S, last = S - 1, kvs = a.kv_head_stride;
  const int kq = lane >> 2, kc = lane & 3;
  uint16_t* raw = (uint16_t*)smem;               // [3 * D]: q, k, v as produced
  const float* csh = rope_cs;                    // [64] cos, [64] sin (rounded, scaled)
  uint16_t* rot = (uint16_t*)(smem + 1536);      // [2 * D]: rotated q and k
  float* osh = (float*)(smem + 2048);            // [8][D] per-wave unnormalised outputs
  // then each wave's 16 attention weights of its current chunk at smem + 6144: [8][16] floats
  const uint16_t* Kb = kcache + (long long)kvh * kvs;
  const uint16_t* Vb = vcache + (long long)kvh * kvs;
  const bool cin = cpos >= 0 && cpos < S;
  float acc0 = 0.f, acc1 = 0.f, mw = -INFINITY, lw = 0.f;
  auto rope = [&]() {   // rotate_half RoPE: threads 0..63 q, 64..127 k
    if (tid < 128) {
      const int hs = tid >> 6, j = tid & 63;
      const float x0 = bfh(raw[hs * DEC_D + j]), x1 = bfh(raw[hs * DEC_D + j + 64]);
      const float c = csh[j], sn = csh[64 + j];
      rot[hs * DEC_D + j] = f32_to_bf16(rb(rb(x0 * c) + rb(-x1 * sn)));
      rot[hs * DEC_D + j + 64] = f32_to_bf16(rb(rb(x1 * c) + rb(x0 * sn)));
    }
    __syncthreads();
    // this step's K / V row goes into the caches (index_copy at cache_position), by the
    // first head's workgroup of the slot that holds the position, open or not
    if (cin && gq == 0 && (int)((cpos / DEC_SPL) % NT) == slot && tid < DEC_D) {
      stg2(kcache + (long long)kvh * kvs + cpos * DEC_D + tid, rot[DEC_D + tid]);
      stg2(vcache + (long long)kvh * kvs + cpos * DEC_D + tid, raw[2 * DEC_D + tid]);
    }
  };
  // one chunk folded into the wave's running softmax; p0: the wave's first position in it.
  // The wave holding cache_position uses the new K / V row (V chosen at its use, so no branch
  // joins the loaded V values, which would make the compiler wait for them there). For the
  // first chunk (mw = -inf) the rescaling factor is 0 and the result is that of a one-pass
  // softmax over the chunk.
  auto fold = [&](const uint4 (&kin)[4], const uint32_t (&vr)[16], FRaw mraw, long long p0) {
    uint4 kr[4] = {kin[0], kin[1], kin[2], kin[3]};
    const bool vnew = cin && cpos >= p0 && cpos < p0 + 16;
    const uint32_t vn = *(const uint32_t*)(raw + 2 * DEC_D + 2 * lane);
    if (vnew && p0 + kq == cpos) {
      const uint4* kn = (const uint4*)(rot + DEC_D + kc * 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) kr[j] = kn[j];
    }
    const float mdec = a.mask_dtype < 0 ? 0.f : ld_f_decode(mraw, a.mask_dtype);
    const float mval = (p0 + kq <= last) ? mdec : -INFINITY;
    const bool live = __ballot(mval != -INFINITY) != 0ull;
    if (live) {
      const uint4* qq = (const uint4*)(rot + kc * 32);
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 q4 = qq[j];
        d = ddot2(q4.x, kr[j].x, d);
        d = ddot2(q4.y, kr[j].y, d);
        d = ddot2(q4.z, kr[j].z, d);
        d = ddot2(q4.w, kr[j].w, d);
      }
      d += HS_DPP(d, HS_QUAD_XOR1);
      d += HS_DPP(d, HS_QUAD_XOR2);
      float sc = -INFINITY;
      if (mval != -INFINITY) {
        sc = rb(d);
        sc = rb(sc * a.scale);
        if (a.mask_dtype >= 0) sc = round_to(sc + mval, a.add_dtype);
      }
      float m = fmaxf(sc, HS_DPP(sc, HS_ROW_ROR4));
      m = fmaxf(m, HS_DPP(m, HS_ROW_ROR8));
      m = fmaxf(fmaxf(HS_RL(m, 0), HS_RL(m, 16)), fmaxf(HS_RL(m, 32), HS_RL(m, 48)));
      const float mn = fmaxf(mw, m);
      const float al = (mw == -INFINITY) ? 0.f : __expf(mw - mn);
      const float e = (sc == -INFINITY) ? 0.f : __expf(sc - mn);
      float ls = e + HS_DPP(e, HS_ROW_ROR4);
      ls += HS_DPP(ls, HS_ROW_ROR8);
      lw = lw * al + ((HS_RL(ls, 0) + HS_RL(ls, 16)) + (HS_RL(ls, 32) + HS_RL(ls, 48)));
      mw = mn;
      acc0 *= al;
      acc1 *= al;
      // the 16 positions' weights to every lane through the wave's own 64 bytes of LDS (one
      // wave's LDS accesses complete in order); 16 lane reads would each stall on the scalar unit
      float pv[16];
      {
        float* pb = (float*)(smem + 6144) + wave * 16;
        if ((lane & 3) == 0) pb[lane >> 2] = e;
#pragma unroll
        for (int j = 0; j < 4; ++j) *(float4*)&pv[4 * j] = ((const float4*)pb)[j];
      }
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float p = pv[t];
        const uint32_t vt = (vnew && p0 + t == cpos) ? vn : vr[t];
        acc0 = fmaf(p, bfh((uint16_t)(vt & 0xffffu)), acc0);
        acc1 = fmaf(p, bfh((uint16_t)(vt >> 16)), acc1);
      }
    }
  };
  if (ob != 0) {   // workgroup-uniform
    uint32_t rest = ob & (ob - 1);
    const long long q0 = (long long)(slot + NT * __builtin_ctz(ob)) * DEC_SPL + wave * 16;
    uint4 kr[4];
    FRaw mraw = {0, 0};
    if (a.mask_dtype >= 0) mraw = ld_f_raw(a.mask, min(q0 + kq, last), a.mask_dtype);
    const uint4* ks = (const uint4*)(Kb + min(q0 + kq, last) * DEC_D + kc * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) kr[j] = ldg16(ks + j);
    uint32_t vr[16];
    if constexpr (VEARLY) {
#pragma unroll
      for (int t = 0; t < 16; ++t) vr[t] = ldg4(Vb + min(q0 + t, last) * DEC_D + 2 * lane);
    }
    __syncthreads();
    xgather<1>(qkvw, 3 * DEC_D, tag, raw, err, a.host_err, tid);
    DEC_STAMP(l, 3);
    if constexpr (!VEARLY) {
#pragma unroll
      for (int t = 0; t < 16; ++t) vr[t] = ldg4(Vb + min(q0 + t, last) * DEC_D + 2 * lane);
    }
    rope();
    fold(kr, vr, mraw, q0);
    while (rest != 0) {   // workgroup-uniform
      const long long pc = (long long)(slot + NT * __builtin_ctz(rest)) * DEC_SPL + wave * 16;
      rest &= rest - 1;
      uint4 kr2[4];
      uint32_t vr2[16];
      FRaw m2 = {0, 0};
      if (a.mask_dtype >= 0) m2 = ld_f_raw(a.mask, min(pc + kq, last), a.mask_dtype);
      const uint4* ks2 = (const uint4*)(Kb + min(pc + kq, last) * DEC_D + kc * 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) kr2[j] = ldg16(ks2 + j);
#pragma unroll
      for (int t = 0; t < 16; ++t) vr2[t] = ldg4(Vb + min(pc + t, last) * DEC_D + 2 * lane);
      fold(kr2, vr2, m2, pc);
    }
  } else {   // every chunk of this slot is closed: an empty partial
    __syncthreads();
    xgather<1>(qkvw, 3 * DEC_D, tag, raw, err, a.host_err, tid);
    DEC_STAMP(l, 3);
    rope();
  }
  osh[wave * DEC_D + 2 * lane] = acc0;
  osh[wave * DEC_D + 2 * lane + 1] = acc1;
  if (lane == 0) {
    red[wave] = mw;
    red2[wave] = lw;
  }
  __syncthreads();
  if (tid < DEC_D + 4) {
    float M = -INFINITY;
#pragma unroll
    for (int w8 = 0; w8 < DEC_WAVES; ++w8) M = fmaxf(M, red[w8]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < DEC_WAVES; ++w8) {
      const float lv = red2[w8];
      const float f = lv > 0.f ? __expf(red[w8] - M) : 0.f;
      o = fmaf(f, osh[w8 * DEC_D + min(tid, DEC_D - 1)], o);
      L = fmaf(f, lv, L);
    }
    // the head's slot partial, one contiguous block: o / l (bf16), then m and l as four
    // 16-bit halves
    const uint32_t mb = __float_as_uint(M), lb = __float_as_uint(L);
    const int e = tid - DEC_D;
    const uint16_t v = tid < DEC_D ? f32_to_bf16(L > 0.f ? o / L : 0.f)
                                   : (uint16_t)(((e < 2 ? mb : lb) >> ((e & 1) ? 0 : 16)) & 0xFFFFu);
    xput(partw + tid, v, tag);
  }
}

// ---- B, KV-head-major (long caches): the G query heads of one KV head over the open chunks of its slot
// The head-major form gives every query head its own workgroups, so the G heads of a KV head each
// read its K / V rows (from L2 after the first); over a long cache that is G times the rows per
// workgroup (Qwen2.5-1.5B at 32,768 positions: 1 MB per workgroup and layer, ≈ 28 µs at the rate
// one CU reads). Here workgroup (KV head, slot) reads each of its rows once and scores them for all
// G heads at once on MFMA: per chunk each wave takes its 16 positions, S = K Q^T on
// v_mfma_f32_16x16x32_bf16 (16 positions x 16 heads, the heads past G zero), the online softmax of
// every head over the tile (a head's 16 scores sit in 4 registers of 4 lanes), and O += P V on
// v_mfma_f32_16x16x16_bf16 (P rounded to bf16, as the CPU path rounds the probabilities before
// P · V), V staged transposed through the wave's own LDS. Scores are rounded as in dec_attend
// (bf16 of the dot product, of its scaled value, of the masked sum). One partial per (query head,
// slot) as in dec_attend.
// qw: the KV head's G exchange blocks [q_h | k | v] (one contiguous range); partw: the layer's
// partials (query head h, slot s at (h NT + s) (D + 4)); osh: G x 8 waves x D floats of free LDS,
// then 8 x 4 KB for the waves' transposed V tiles.
typedef short dec_s16x4 __attribute__((ext_vector_type(4)));
typedef float dec_f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((ext_vector_type(8))) __bf16 dec_bf16x8;
__device__ __forceinline__ void dec_attend_kv(const PersistArgs& a, int l, uint16_t* kcache, uint16_t* vcache,
                                              const uint32_t* qw, uint32_t* partw, uint32_t ob, int kvh, int slot,
                                              long long cpos, uint32_t tag, uint32_t* err, unsigned char* smem,
                                              float* osh, const float* rope_cs, float* red, float* red2, int tid,
                                              int lane, int wave) {
  const int NT = a.nsplit, G = a.H / a.KVH;
  const long long S = a.S, last = S - 1, kvs = a.kv_head_stride;
  const int mq = lane >> 4, m16 = lane & 15;   // MFMA operand coordinates: k group, row / column
  uint16_t* raw = (uint16_t*)smem;                             // [G][3 D]: the G blocks as produced
  uint16_t* rot = (uint16_t*)(smem + G * 3 * DEC_D * 2);       // [G + 1][D]: each head's rotated q, then k
  uint32_t* vt = (uint32_t*)(osh + G * DEC_WAVES * DEC_D) + wave * (DEC_D * 8);   // [D][16 positions] bf16
  const float* csh = rope_cs;
  const uint16_t* Kb = kcache + (long long)kvh * kvs;
  const uint16_t* Vb = vcache + (long long)kvh * kvs;
  const bool cin = cpos >= 0 && cpos < S;
  // O[head 4 mq + r][dim 16 c + m16] in oacc[c][r]; the running max / sum of head m16
  dec_f32x4 oacc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) oacc[c] = dec_f32x4{0.f, 0.f, 0.f, 0.f};
  float mwk = -INFINITY, lwk = 0.f;
  uint4 qb[4];   // B of S = K Q^T: head m16's rotated q, dims 32 s + 8 mq .. (heads past G: zero)
  auto rope = [&]() {   // rotate_half RoPE of the G q rows and the k row
    for (int i = tid; i < (G + 1) * 64; i += DEC_THREADS) {
      const int hs = i >> 6, j = i & 63;
      const uint16_t* src = hs < G ? raw + hs * 3 * DEC_D : raw + DEC_D;
      const float x0 = bfh(src[j]), x1 = bfh(src[j + 64]);
      const float c = csh[j], sn = csh[64 + j];
      rot[hs * DEC_D + j] = f32_to_bf16(rb(rb(x0 * c) + rb(-x1 * sn)));
      rot[hs * DEC_D + j + 64] = f32_to_bf16(rb(rb(x1 * c) + rb(x0 * sn)));
    }
    __syncthreads();
    // this step's K / V row into the caches, by the workgroup of the slot that holds the position
    if (cin && (int)((cpos / DEC_SPL) % NT) == slot && tid < DEC_D) {
      stg2(kcache + (long long)kvh * kvs + cpos * DEC_D + tid, rot[G * DEC_D + tid]);
      stg2(vcache + (long long)kvh * kvs + cpos * DEC_D + tid, raw[2 * DEC_D + tid]);
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      qb[s4] = m16 < G ? *(const uint4*)(rot + m16 * DEC_D + 32 * s4 + 8 * mq) : make_uint4(0, 0, 0, 0);
  };
  // one chunk's 16 positions of this wave (p0 ..) folded into every head's running softmax.
  // kin: the A operand (position p0 + m16, dims 32 s + 8 mq ..); vr: dims 2 lane, 2 lane + 1 of
  // the 16 positions; mr: the mask values of positions p0 + 4 mq + r
  auto fold = [&](const uint4 (&kin)[4], const uint32_t (&vr)[16], const FRaw (&mr)[4], long long p0) {
    uint4 kr[4] = {kin[0], kin[1], kin[2], kin[3]};
    const bool vnew = cin && cpos >= p0 && cpos < p0 + 16;
    if (vnew && p0 + m16 == cpos) {   // this step's k row, not yet in the cache as read
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) kr[s4] = *(const uint4*)(rot + G * DEC_D + 32 * s4 + 8 * mq);
    }
    float mval[4];
    bool any = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float md = a.mask_dtype < 0 ? 0.f : ld_f_decode(mr[r], a.mask_dtype);
      mval[r] = (p0 + 4 * mq + r <= last) ? md : -INFINITY;
      any = any || mval[r] != -INFINITY;
    }
    if (__ballot(any) == 0ull) return;   // every position of the tile closed
    dec_f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4)
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dec_bf16x8, kr[s4]),
                                                     __builtin_bit_cast(dec_bf16x8, qb[s4]), sacc, 0, 0, 0);
    // sacc[r]: the score of position p0 + 4 mq + r for head m16
    float sc[4], m = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = -INFINITY;
      if (mval[r] != -INFINITY) {
        x = rb(sacc[r]);
        x = rb(x * a.scale);
        if (a.mask_dtype >= 0) x = round_to(x + mval[r], a.add_dtype);
      }
      sc[r] = x;
      m = fmaxf(m, x);
    }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const float mn = fmaxf(mwk, m);
    const float al = (mwk == -INFINITY) ? 0.f : __expf(mwk - mn);
    float e[4], ls = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e[r] = (sc[r] == -INFINITY) ? 0.f : __expf(sc[r] - mn);
      ls += e[r];
    }
    ls += __shfl_xor(ls, 16, 64);
    ls += __shfl_xor(ls, 32, 64);
    lwk = lwk * al + ls;
    mwk = mn;
    // P as the A operand of O = P V: lane l holds P[head m16][position 4 mq + r], the layout S has
    const dec_s16x4 pa = {(short)f32_to_bf16(e[0]), (short)f32_to_bf16(e[1]), (short)f32_to_bf16(e[2]),
                          (short)f32_to_bf16(e[3])};
    // O's rows are heads 4 mq + r: their rescale factors from the lanes that hold those heads
    float alr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) alr[r] = __shfl(al, 4 * mq + r, 64);
    // V transposed into the wave's LDS tile (the new v row in place of the cache's): dims 2 lane and
    // 2 lane + 1, two positions per word; one wave's LDS accesses complete in order
    const uint32_t vn = *(const uint32_t*)(raw + 2 * DEC_D + 2 * lane);
#pragma unroll
    for (int t = 0; t < 16; t += 2) {
      const uint32_t v0 = (vnew && p0 + t == cpos) ? vn : vr[t];
      const uint32_t v1 = (vnew && p0 + t + 1 == cpos) ? vn : vr[t + 1];
      vt[(2 * lane) * 8 + t / 2] = (v0 & 0xFFFFu) | (v1 << 16);
      vt[(2 * lane + 1) * 8 + t / 2] = (v0 >> 16) | (v1 & 0xFFFF0000u);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
#pragma unroll
      for (int r = 0; r < 4; ++r) oacc[c][r] *= alr[r];
      // B: V[positions 4 mq ..][dim 16 c + m16]
      const uint2 vb = *(const uint2*)(vt + (16 * c + m16) * 8 + 2 * mq);
      oacc[c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, __builtin_bit_cast(dec_s16x4, vb), oacc[c], 0, 0, 0);
    }
  };
  auto kload = [&](uint4 (&kr)[4], long long p0) {   // the A operand rows of a tile
    const uint16_t* kp = Kb + min(p0 + m16, last) * DEC_D + 8 * mq;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) kr[s4] = ldg16(kp + 32 * s4);
  };
  auto mload = [&](FRaw (&mr)[4], long long p0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) mr[r] = a.mask_dtype >= 0 ? ld_f_raw(a.mask, min(p0 + 4 * mq + r, last), a.mask_dtype)
                                                         : FRaw{0, 0};
  };
  if (ob != 0) {   // workgroup-uniform
    uint32_t rest = ob & (ob - 1);
    const long long q0 = (long long)(slot + NT * __builtin_ctz(ob)) * DEC_SPL + wave * 16;
    uint4 kr[4];
    FRaw mr[4];
    mload(mr, q0);
    kload(kr, q0);
    __syncthreads();
    xgather<3>(qw, G * 3 * DEC_D, tag, raw, err, a.host_err, tid);
    DEC_STAMP(l, 3);
    uint32_t vr[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) vr[t] = ldg4(Vb + min(q0 + t, last) * DEC_D + 2 * lane);
    rope();
    fold(kr, vr, mr, q0);
    while (rest != 0) {   // workgroup-uniform
      const long long pc = (long long)(slot + NT * __builtin_ctz(rest)) * DEC_SPL + wave * 16;
      rest &= rest - 1;
      uint4 kr2[4];
      uint32_t vr2[16];
      FRaw m2[4];
      mload(m2, pc);
      kload(kr2, pc);
#pragma unroll
      for (int t = 0; t < 16; ++t) vr2[t] = ldg4(Vb + min(pc + t, last) * DEC_D + 2 * lane);
      fold(kr2, vr2, m2, pc);
    }
  } else {   // every chunk of this slot is closed: empty partials
    __syncthreads();
    xgather<3>(qw, G * 3 * DEC_D, tag, raw, err, a.host_err, tid);
    DEC_STAMP(l, 3);
    rope();
  }
  // the wave's outputs of heads < G, and each head's (max, sum) from its lane m16 (of k group 0)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * mq + r;
    if (h < G) {
#pragma unroll
      for (int c = 0; c < 8; ++c) osh[(h * DEC_WAVES + wave) * DEC_D + 16 * c + m16] = oacc[c][r];
    }
  }
  if (mq == 0 && m16 < G) {
    red[wave * 8 + m16] = mwk;
    red2[wave * DEC_MAXG + m16] = lwk;
  }
  __syncthreads();
  for (int i = tid; i < G * (DEC_D + 4); i += DEC_THREADS) {
    const int g = i / (DEC_D + 4), e = i - g * (DEC_D + 4);
    float M = -INFINITY;
#pragma unroll
    for (int w8 = 0; w8 < DEC_WAVES; ++w8) M = fmaxf(M, red[w8 * 8 + g]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w8 = 0; w8 < DEC_WAVES; ++w8) {
      const float lv = red2[w8 * DEC_MAXG + g];
      const float f = lv > 0.f ? __expf(red[w8 * 8 + g] - M) : 0.f;
      o = fmaf(f, osh[(g * DEC_WAVES + w8) * DEC_D + min(e, DEC_D - 1)], o);
      L = fmaf(f, lv, L);
    }
    const uint32_t mb = __float_as_uint(M), lb = __float_as_uint(L);
    const int e2 = e - DEC_D;
    const uint16_t v = e < DEC_D ? f32_to_bf16(L > 0.f ? o / L : 0.f)
                                 : (uint16_t)(((e2 < 2 ? mb : lb) >> ((e2 & 1) ? 0 : 16)) & 0xFFFFu);
    const int hq = kvh * G + g;
    xput(partw + ((long long)hq * NT + slot) * (DEC_D + 4) + e, v, tag);
  }
  __syncthreads();   // osh is free LDS of the caller's, which it refills next
}

// ---- C with more slots than the staging area holds (KV-head-major: NT up to 128) -----------------------
// All NT partials in one gather by the whole workgroup, into pl (free LDS of the caller's: NT (D + 4)
// halves), then the combine as dec_combine (weights e^(m_t - M) l_t / L, the o rows summed in slot
// order). cw: NT floats of LDS.
__device__ __forceinline__ void dec_combine_big(const PersistArgs& a, int l, const uint32_t* partw, uint32_t* attw,
                                                uint32_t tag, uint32_t* err, uint16_t* pl, float* cw, int tid,
                                                int lane, int wave) {
  const int NT = a.nsplit;
  __syncthreads();
  xgather<(128 * (DEC_D + 4) / 2 + DEC_THREADS - 1) / DEC_THREADS>(partw, NT * (DEC_D + 4), tag, pl, err, a.host_err,
                                                                 tid);
  DEC_STAMP(l, 5);
  if (wave == 0) {
    float M = -INFINITY;
    for (int t = lane; t < NT; t += 64) {
      const uint16_t* e = pl + t * (DEC_D + 4) + DEC_D;
      const float m = __uint_as_float(((uint32_t)e[0] << 16) | e[1]), lv = __uint_as_float(((uint32_t)e[2] << 16) | e[3]);
      M = fmaxf(M, lv > 0.f ? m : -INFINITY);
    }
    M = wave_max(M);
    float L = 0.f;
    for (int t = lane; t < NT; t += 64) {
      const uint16_t* e = pl + t * (DEC_D + 4) + DEC_D;
      const float m = __uint_as_float(((uint32_t)e[0] << 16) | e[1]), lv = __uint_as_float(((uint32_t)e[2] << 16) | e[3]);
      const float f = lv > 0.f ? __expf(m - M) * lv : 0.f;
      cw[t] = f;
      L += f;
    }
    L = wave_sum(L);
    for (int t = lane; t < NT; t += 64) cw[t] = L > 0.f ? cw[t] / L : 0.f;
  }
  __syncthreads();
  if (wave < 4) {
    const int d = tid >> 1, q = tid & 1;
    float sacc = 0.f;
    for (int t = q; t < NT; t += 2) sacc = fmaf(cw[t], bfh(pl[t * (DEC_D + 4) + d]), sacc);
    sacc += HS_DPP(sacc, HS_QUAD_XOR1);
    if (q == 0) xput(attw + d, f32_to_bf16(sacc), tag);
  }
  DEC_STAMP(l, 6);
}

// ---- C: combine the slot partials of one query head (waves 0-3, 2 threads per dimension) ----------
// partw: the head's nsplit partials; attw: the head's D words of the attention row.
__device__ __forceinline__ void dec_combine(const PersistArgs& a, int l, const uint32_t* partw, uint32_t* attw,
                                            uint32_t tag, uint32_t* err, unsigned char* smem, float* red2,
                                            int tid, int lane, int wave) {
  const int NT = a.nsplit;
  uint16_t* pl = (uint16_t*)smem;   // [NT][D + 4]
  float* cw = red2;                 // [NT] weights e^(m_t - M) l_t / L (NT <= 32: red2 holds 64)
  __syncthreads();
  const int crd = xgather<(32 * (DEC_D + 4) + 2 * 256 - 1) / (2 * 256), 256>(partw, NT * (DEC_D + 4), tag, pl, err,
                                                                           a.host_err, tid);
  DEC_STAMPV(l, 7, crd);
  DEC_STAMP(l, 5);
  if (wave == 0) {
    float m = -INFINITY, lv = 0.f;
    if (lane < NT) {
      const uint16_t* e = pl + lane * (DEC_D + 4) + DEC_D;
      m = __uint_as_float(((uint32_t)e[0] << 16) | e[1]);
      lv = __uint_as_float(((uint32_t)e[2] << 16) | e[3]);
    }
    const float M = wave_max(lv > 0.f ? m : -INFINITY);
    const float f = lv > 0.f ? __expf(m - M) * lv : 0.f;
    const float L = wave_sum(f);
    if (lane < NT) cw[lane] = L > 0.f ? f / L : 0.f;
  }
  __syncthreads();
  if (wave < 4) {
    const int d = tid >> 1, q = tid & 1;
    float sacc = 0.f;
    for (int t = q; t < NT; t += 2) sacc = fmaf(cw[t], bfh(pl[t * (DEC_D + 4) + d]), sacc);
    sacc += HS_DPP(sacc, HS_QUAD_XOR1);
    if (q == 0) xput(attw + d, f32_to_bf16(sacc), tag);
  }
  DEC_STAMP(l, 6);
}

// ---- C spread over the head's attention workgroups: slot j combines dims j DS .. j DS + DS - 1 ----
// (DS = D / nsplit rounded up to even) of its head's nsplit partials, right after publishing its
// own, and publishes those dims of the attention row. Each slot gathers only the (m, l) words and
// its DS dims of every partial; the weights and sums are dec_combine's, in the same order, so the
// row is the same bit for bit. No workgroup waits behind another's weight loads for the partials.
__device__ __forceinline__ void dec_combine_slot(const PersistArgs& a, int l, const uint32_t* partw, uint32_t* attw,
                                                 int slot, uint32_t tag, uint32_t* err, unsigned char* smem,
                                                 float* red2, int tid, int lane, int wave) {
  const int NT = a.nsplit;
  const int DS = ((DEC_D + NT - 1) / NT + 1) & ~1, d0 = slot * DS, nd = min(DS, DEC_D - d0);
  if (nd <= 0) return;   // (workgroup-uniform) a trailing slot with no dims
  const int PW = DS / 2 + 2;        // 64-bit words per partial: DS / 2 of o, then (m, l)
  uint16_t* pl = (uint16_t*)smem;   // [NT][DS + 4]
  float* cw = red2;
  __syncthreads();
  {
    const unsigned long long want = ((unsigned long long)tag << 48) | ((unsigned long long)tag << 16);
    const unsigned long long tmask = 0xFFFF0000FFFF0000ull;
    const bool mine = tid < NT * PW;
    const int t = tid / PW, k = tid - t * PW;
    const int off = t * (DEC_D + 4) + (k < DS / 2 ? min(d0 + 2 * k, DEC_D - 2) : DEC_D + 2 * (k - DS / 2));
    unsigned long long v = mine ? xget2(partw + off) : want;
    const unsigned long long t0 = wall_clock64();
    while ((v & tmask) != want) {
      if (wall_clock64() - t0 > DEC_TIMEOUT) {
        dec_fail(err, a.host_err);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      v = xget2(partw + off);
    }
    if (mine) *(uint32_t*)(pl + t * (DS + 4) + 2 * k) = (uint32_t)(v & 0xFFFFu) | (uint32_t)((v >> 16) & 0xFFFF0000u);
  }
  __syncthreads();
  DEC_STAMP(l, 5);
  if (wave == 0) {
    float m = -INFINITY, lv = 0.f;
    if (lane < NT) {
      const uint16_t* e = pl + lane * (DS + 4) + DS;
      m = __uint_as_float(((uint32_t)e[0] << 16) | e[1]);
      lv = __uint_as_float(((uint32_t)e[2] << 16) | e[3]);
    }
    const float M = wave_max(lv > 0.f ? m : -INFINITY);
    const float f = lv > 0.f ? __expf(m - M) * lv : 0.f;
    const float L = wave_sum(f);
    if (lane < NT) cw[lane] = L > 0.f ? f / L : 0.f;
    __builtin_amdgcn_wave_barrier();
    for (int j = 0; j < nd; j += 32) {   // 32 dims per pass, two lanes each (every lane takes part)
      const int dj = j + (lane >> 1), d = min(dj, nd - 1), q = lane & 1;
      float sacc = 0.f;
      for (int t = q; t < NT; t += 2) sacc = fmaf(cw[t], bfh(pl[t * (DS + 4) + d]), sacc);
      sacc += HS_DPP(sacc, HS_QUAD_XOR1);
      if (q == 0 && dj < nd) xput(attw + d0 + d, f32_to_bf16(sacc), tag);
    }
  }
  DEC_STAMP(l, 6);
}

// ---------------------------------------------------------------- the step

// The step's LDS, declared once per kernel (both role instances of decode_body use it).
template <int KC, int NE>
struct DecShared {
  __attribute__((aligned(16))) unsigned char smem[DEC_SMEM];   // per-part staging (B, C; xs)
  __attribute__((aligned(16))) uint16_t xres[512 * KC];
  float red[DEC_WAVES * 8];
  float red2[DEC_WAVES * DEC_MAXG];
  float rope_cs[128];
  // an attention workgroup's first NE gate / up rows (row i: gate chunks, then up chunks, 1 KB
  // each); in the other workgroups, their o_proj rows (at most 2 NE), then (except the combine
  // workgroups) their first NEO gate / up rows. F stages the SiLU * up row here.
  __attribute__((aligned(16))) uint4 ebuf[NE * 2 * KC * 64];
  const void* ptab[2][14];   // the current and the next layer's tensors (DecodeLayerPtrs)
  unsigned long long kred[DEC_WAVES];
  float cwk[128];            // the combine's slot weights (KV-head-major: up to 128 slots)
  uint32_t obw[DEC_WAVES];   // the open-chunk scan: each wave's bits
  // a part's results (o_proj rows, gate / up rows) staged here, then published with one store
  // instruction per 64 words: many single-word stores spread over the waves are acknowledged far
  // more slowly while the memory system is busy with the weight stream
  uint16_t ostage[DEC_OSTAGE];
};

// KC: 512-element chunks of a hidden-long row per lane (hidden = 512 KC); IC: chunks per lane
// of a down_proj row whose K (inter) is split over the 8 waves (inter <= 4096 IC); RF: down_proj
// rows per workgroup, at most (2 KC: hidden rows over 256 workgroups); EM: gate/up rows per wave
// streamed through registers, at most; ED: those rows in flight per wave; NE: gate/up rows an
// attention workgroup loads into LDS once its attention part is done.
template <int KC, int IC, int EM, int ROLE, bool KVM, int RF = 2 * KC, int ED = DEC_ED, int NE = DEC_NE(KC), int RFE = DEC_RFE>
__device__ __forceinline__ void decode_body(const PersistArgs& a, DecShared<KC, NE>& sh) {
  auto& smem = sh.smem;
  auto& xres = sh.xres;
  auto& red = sh.red;
  auto& red2 = sh.red2;
  auto& rope_cs = sh.rope_cs;
  auto& ebuf = sh.ebuf;
  auto& ptab = sh.ptab;
  auto& kred = sh.kred;
  auto& ostage = sh.ostage;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x, NWG = a.nwg;
  const int hid = a.hidden, H = a.H, KVH = a.KVH, G = H / KVH, NT = a.nsplit;
  const XLayout X = xlayout(a);
  uint32_t* keys = a.ll + X.stride * a.L + hid;                 // nwg 64-bit key words
  uint32_t* ctl = keys + 2 * (long long)NWG;                    // [0] step tag, [1] timeout flag
  uint32_t* err = ctl + 1;
  uint32_t tag = (__hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u) & 0xFFFFu;
  tag = tag == 0 ? 1u : tag;
  // the three inputs loaded together with no dtype switch (int64 or int32, checked on the host): a
  // switch's branches would each wait for the load in flight, three cold round trips in a row
  const IRaw tokw = ld_i_raw(a.ids, 0, a.ids_dtype), posw = ld_i_raw(a.pos_ids, 0, a.pos_dtype);
  const IRaw cposw = ld_i_raw(a.cache_pos, 0, a.cpos_dtype);
  long long tok = ld_i_decode(tokw, a.ids_dtype);
  tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);   // ATen would raise; never read outside the table
  const long long posr = ld_i_decode(posw, a.pos_dtype);
  const long long cpos = ld_i_decode(cposw, a.cpos_dtype);
  const long long S = a.S, last = S - 1, kvs = a.kv_head_stride;
  uint16_t* xs = (uint16_t*)smem;
  DEC_STAMP(a.L, 7);
  // a decode loop advanced in the kernel has moved past the cache end: this step is reported
  if (a.adv_flag != nullptr && b == 0 && tid == 0 && (cpos < 0 || cpos >= S)) a.adv_flag[0] = 1;
  // rotary factors of this step's position (the same for every layer): cos and sin of
  // inv_freq[i] * position in fp32, times the scaling, rounded to bf16
  if (tid < 64) {
    float sf, cf;
    sincos_rot(a.inv_freq[tid] * (float)posr, &sf, &cf);
    rope_cs[tid] = round_to(cf * a.rope_scaling, HS_BF16);
    rope_cs[64 + tid] = round_to(sf * a.rope_scaling, HS_BF16);
  }

  // Roles. Workgroups b < NB (= H * nsplit) run attention: query head g = b / ntile of tile
  // b % ntile (KV head, slot). Slot j takes the cache's 128-position chunks j, j + nsplit,
  // j + 2 nsplit, ... The other ND run o_proj (RD rows each), and the
  // first H of them the combine of query head b - NB. An attention workgroup is done with its
  // latency-bound parts well before x1 exists, so it spends that time loading NE gate / up rows
  // into LDS, and takes NE more gate / up rows than the others; the rest are spread so that every
  // workgroup has about the same left to stream once x1 has arrived.
  // (KVM, the KV-head-major attention of long caches: workgroup b < NB = KVH nsplit takes KV head
  // b / nsplit, slot b % nsplit, for all G query heads)
  const int ntile = KVH * NT;
  const int NB = KVM ? ntile : ntile * G, ND = NWG - NB;
  constexpr bool att = ROLE == 0;   // (the kernel entry picks the role instance from b)
  const int tile = b % ntile, gq = KVM ? 0 : b / ntile;
  const int kvh = tile / NT, slot = tile % NT;
  constexpr bool comb = ROLE == 2;   // o_proj workgroups b in [NB, NB + H) also run the combine
  const int RD = (hid + ND - 1) / ND;                                   // <= 2 NE (checked on the host)
  // gate / up rows in LDS: NE on an attention workgroup; NEO behind the o_proj rows of an o_proj
  // workgroup that runs no combine (issued with its o_proj rows, they land while it waits for
  // the attention row); none on a combine workgroup, whose partials poll comes sooner
  const int NEO = max(2 * NE - RD, 0) / 2;
  const int NLC = att ? NE : (comb ? 0 : NEO);
  // gate / up rows streamed (the host's work split of the rows not held in LDS): RBA by an
  // attention workgroup, RBO by an o_proj workgroup (its stream starts only after o_proj), RBC by
  // a combine workgroup (fewer: it runs the combine before its o_proj rows, and with RBO rows it
  // published h and the next layer's rows last)
  const int RBA = a.rba, RBC = a.rbc, RBO = comb ? RBC : a.rbo;
  const int e0 = att ? b * (NE + RBA)                                   // first gate / up row
                     : NB * (NE + RBA) + min(b - NB, H) * RBC + max(b - NB - H, 0) * (a.rbo + NEO);
  const int ecnt = max(min(NLC + (att ? RBA : RBO), a.inter - e0), 0);  // its rows
  const int NL = min(NLC, ecnt);                                        // of which in LDS
  const unsigned EOFF = att ? 0u : (unsigned)(RD * KC * 1024);          // where they sit in ebuf
  // layer 0's tensors into LDS; each layer loads the next one's during its first part and stores
  // them in F, so no layer waits for its table at its start
  if (tid < 14) ptab[0][tid] = ((const void* const*)a.layers)[tid];
  // the open chunks this attention workgroup reads (the same for every layer)
  uint32_t ob = 0;
  if constexpr (att) ob = dec_scan_chunks(a, slot, sh.obw, lane, wave);
  __syncthreads();
  if constexpr (att) {
    if (a.mask_dtype >= 0) {
#pragma unroll
      for (int w8 = 0; w8 < DEC_WAVES; ++w8) ob |= sh.obw[w8];
    }
  }

  for (int l = 0; l < a.L; ++l) {
    const DecodeLayerPtrs P = dec_layer(ptab[l & 1]);
    const void* pnext = nullptr;
    if (tid < 14 && l + 1 < a.L) pnext = ((const void* const*)(a.layers + l + 1))[tid];
    uint32_t* XL = a.ll + X.stride * l;            // this layer's exchange slots
    uint32_t* XN = a.ll + X.stride * (l + 1);      // the next layer's input row (x_{l+1})

    // ---- A: RMSNorm, q / k / v rows (+ bias) -------------------------------------------------
    {
      DEC_PART_IDS();
      const int R = (H + 2 * KVH) * DEC_D, RB = (R + NWG - 1) / NWG;
      const int r = b * RB + wave;
      const bool has = wave < RB && r < R;
      const uint16_t* W;
      const uint16_t* B;
      int rr, seg;
      if (r < H * DEC_D) {
        W = P.wq; B = P.bq; rr = r; seg = 0;
      } else if (r < (H + KVH) * DEC_D) {
        rr = r - H * DEC_D; W = P.wk; B = P.bk; seg = 1;
      } else {
        rr = r - (H + KVH) * DEC_D; W = P.wv; B = P.bv; seg = 2;
      }
      // loads carry no branch: a wave without a row re-reads row 0 of q (unused)
      const long long rl = has ? rr : 0;
      const uint16_t* Wl = has ? W : P.wq;
      uint4 w[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) w[c] = ldw(Wl + rl * hid + c * 512 + lane * 8);
      const uint16_t bias = (has && (a.flags & 1)) ? ldg2(B + rr) : (uint16_t)0;
      const uint4 nw = tid < (hid >> 3) ? ldg16(P.norm1 + 8 * tid) : make_uint4(0, 0, 0, 0);
      __syncthreads();
      DEC_STAMPT(l, 0);
      const int ard = load_x<KC>(a, l, XL, tok, tag, xres, err, a.host_err, tid);
      DEC_STAMPV(l, 0, ard);
      DEC_STAMP(l, 1);
      block_norm(xres, nw, hid, a.eps, a.n_dtype, xs, red, tid);
      if (has) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = ddot8(*(const uint4*)(xs + c * 512 + lane * 8), w[c], acc);
        acc = wave_sum(acc);
        if (lane == 0) ostage[wave] = f32_to_bf16(acc + bfh(bias));
      }
      __syncthreads();
      // published by wave 0 in one store: exchange block of query head h is [q_h | k of its KV
      // head | v of its KV head], and a k or v row goes into the blocks of all G heads that read it
      if (wave == 0 && lane < RB * G) {
        const int j = lane / G, g = lane % G, rj = b * RB + j;
        if (rj < R) {
          const int sj = rj < H * DEC_D ? 0 : (rj < (H + KVH) * DEC_D ? 1 : 2);
          const int rrj = rj - (sj == 0 ? 0 : (sj == 1 ? H * DEC_D : (H + KVH) * DEC_D));
          const int hq = sj == 0 ? rrj / DEC_D : (rrj / DEC_D) * G + g;
          if (sj != 0 || g == 0) xput(XL + X.qkv + (long long)hq * 3 * DEC_D + sj * DEC_D + rrj % DEC_D, ostage[j], tag);
        }
      }
      DEC_STAMP(l, 2);
    }

    // E's ring of gate / up rows in registers (see E); an o_proj workgroup issues its first EP
    // rows with its o_proj rows when DEC_EARLY is set
    constexpr int EP = ED < EM ? ED : EM;
    uint4 wg[EP][KC], wu[EP][KC];
    const int rs = e0 + NL, nr = ecnt - NL;   // ring rows: rs .. rs + nr - 1 (nr <= 8 EM, checked on the host)
    auto load_row = [&](int d, int k) {
      ering_load<KC>(wg[d], wu[d], P.wg, P.wu, ering_row(k, rs, nr, threadIdx.x >> 6, a.inter), hid,
                     threadIdx.x & 63);
    };

    // ---- D's o_proj rows into LDS (o_proj workgroups): issued now, they land while B and C run ----
    if (!att) {
      DEC_PART_IDS();
      const long long d0 = (long long)(b - NB) * RD;
      const long long rmax = min(d0 + RD, (long long)hid) - 1;   // rows past the block re-read its last row
      const unsigned base = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&ebuf[0];
      for (int k = wave; k < RD * KC; k += DEC_WAVES) {
        const long long r = max(min(d0 + k / KC, rmax), 0ll);
        dec_dma16(P.wo + r * (H * DEC_D) + (k % KC) * 512 + lane * 8,
                  __builtin_amdgcn_readfirstlane(base + (unsigned)k * 1024u));
      }
      for (int k = wave; k < NL * 2 * KC; k += DEC_WAVES) {   // and the first NL gate / up rows
        const int i = k / (2 * KC), u = (k / KC) & 1, c = k % KC;
        dec_dma16((u ? P.wu : P.wg) + (long long)(e0 + i) * hid + c * 512 + lane * 8,
                  __builtin_amdgcn_readfirstlane(base + EOFF + (unsigned)k * 1024u));
      }
      if constexpr (DEC_EARLY && !comb) {
#pragma unroll
        for (int d = 0; d < EP; ++d) load_row(d, d);
      }
    }

    // ---- B: attention of one query head over the open chunks of its slot ----------------------------
    if constexpr (att) {
      DEC_PART_IDS();
      if constexpr (KVM) {   // (ebuf: its gate / up rows are loaded after this part)
        dec_attend_kv(a, l, P.kc, P.vc, XL + X.qkv + (long long)kvh * G * 3 * DEC_D, XL + X.part, ob, kvh, slot,
                      cpos, tag, err, smem, (float*)&ebuf[0], rope_cs, red, red2, tid, lane, wave);
      } else {
        const int hq = kvh * G + gq;
        dec_attend(a, l, P.kc, P.vc, XL + X.qkv + (long long)hq * 3 * DEC_D,
                   XL + X.part + ((long long)hq * NT + slot) * (DEC_D + 4), ob, kvh, gq, slot, cpos, tag, err, smem,
                   rope_cs, red, red2, tid, lane, wave);
      }
      DEC_STAMP(l, 4);
      if constexpr (!KVM) {
        if (a.flags & 2) {   // C by the head's attention workgroups (no combine workgroups)
          const int hq = kvh * G + gq;
          dec_combine_slot(a, l, XL + X.part + (long long)hq * NT * (DEC_D + 4), XL + X.att + (long long)hq * DEC_D,
                           slot, tag, err, smem, red2, tid, lane, wave);
        }
      }
      // this workgroup's first NL gate / up rows into LDS: its next wait (x1, in E) is some
      // microseconds away, and these land by then
      const unsigned base = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&ebuf[0];
      int nq = 0;
      for (int k = wave; k < NL * 2 * KC; k += DEC_WAVES) {
        const int i = k / (2 * KC), u = (k / KC) & 1, c = k % KC;
        dec_dma16((u ? P.wu : P.wg) + (long long)(e0 + i) * hid + c * 512 + lane * 8,
                  __builtin_amdgcn_readfirstlane(base + (unsigned)k * 1024u));
        if constexpr (DEC_LDS_Q > 0) {
          if (++nq >= DEC_LDS_Q) DEC_VMCNT(DEC_LDS_Q);
        }
      }
    }

    // ---- C: combine the slot partials of one query head ---------------------------------------------
    if (comb) {
      DEC_PART_IDS();
      const int h = b - NB;
      if constexpr (KVM)   // (its partials staged behind its o_proj rows: a combine workgroup holds no gate / up rows)
        dec_combine_big(a, l, XL + X.part + (long long)h * NT * (DEC_D + 4), XL + X.att + (long long)h * DEC_D, tag,
                        err, (uint16_t*)((unsigned char*)ebuf + EOFF), sh.cwk, tid, lane, wave);
      else
        dec_combine(a, l, XL + X.part + (long long)h * NT * (DEC_D + 4), XL + X.att + (long long)h * DEC_D, tag, err,
                    smem, red2, tid, lane, wave);
    }

    // ---- D: o_proj + residual (o_proj workgroups; the rows from LDS) ------------------------------------
    if (!att) {
      DEC_PART_IDS();
      dec_vmcnt0();   // this wave's o_proj rows have landed (long ago)
      __syncthreads();
      DEC_STAMPT(l, 7);
      const int drd = xgather<(KC + 1) / 2 * 2, 256>(XL + X.att, H * DEC_D, tag, xs, err, a.host_err, tid);
      if constexpr (!comb) DEC_STAMPV(l, 7, drd);
      DEC_STAMP(l, 8);
      const unsigned char* ob = (const unsigned char*)ebuf;
      const int d0 = (b - NB) * RD;
      uint4 xv[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) xv[c] = *(const uint4*)(xs + c * 512 + lane * 8);
      // rows wave + 8 k (RD <= 2 NE); the row sums of 8 of them at a time: lane 8 k ends with row k's
      constexpr int MD = (2 * NE + DEC_WAVES - 1) / DEC_WAVES;
#pragma unroll
      for (int q = 0; q < (MD + 7) / 8; ++q) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int i = wave + DEC_WAVES * (8 * q + k);
          v[k] = 0.f;
          if (8 * q + k < MD && i < RD && d0 + i < hid) {   // wave-uniform
            uint4 w[KC];
#pragma unroll
            for (int c = 0; c < KC; ++c) w[c] = *(const uint4*)(ob + (i * KC + c) * 1024 + lane * 16);
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < KC; ++c) acc = ddot8(xv[c], w[c], acc);
            v[k] = acc;
          }
        }
        const float sum = wave_sum8(v, lane);
        const int i = wave + DEC_WAVES * (8 * q + (lane >> 3));
        if ((lane & 7) == 0 && 8 * q + (lane >> 3) < MD && i < RD && d0 + i < hid)
          ostage[i] = f32_to_bf16(bfh(xres[d0 + i]) + rb(sum));
      }
      __syncthreads();
      if (tid < min(RD, hid - d0)) xput(XL + X.x1 + d0 + tid, ostage[tid], tag);
      DEC_STAMP(l, 9);
    }

    // ---- E: RMSNorm, gate / up, SiLU(gate) * up -----------------------------------------------------
    // Rows e0 .. e0 + NL - 1 are in LDS. The others, e0 + NL + w + 8 k for wave
    // w (at most EM), stream through a ring of registers with EP rows in flight: the first EP are
    // issued before x1 is awaited (they land during the hop), and each computed row's slot is
    // reloaded with the row EP further on. The code is unrolled over EM and every load is unconditional (a wave with fewer rows
    // re-reads its last one), so no loaded value flows through a branch join, which would make the
    // compiler wait for every load in flight. Results are published after the last row: a store
    // between the loads would sit in the same in-order completion count.
    // down_proj rows of F (rows b * RB + j): the first RFE are issued during E, after x1 is in,
    // when every load this workgroup issued before has landed, so they arrive during the gate / up
    // arithmetic (more of them would hold back the h stores behind them); the rest follow the
    // h stores
    uint4 fw[RF][IC];
    auto load_down = [&](int j) {
      const int RB = (hid + NWG - 1) / NWG, K8 = a.inter >> 3, wv = threadIdx.x >> 6, ln = threadIdx.x & 63;
      const long long rmaxf = min(b * RB + RB, hid) - 1;
      const long long r = min((long long)(b * RB + j), rmaxf);
#pragma unroll
      for (int k = 0; k < IC; ++k) {
        const int c = min(512 * k + 64 * wv + ln, K8 - 1);   // chunks past the row re-read its last one
        fw[j][k] = ldw(P.wd + r * a.inter + 8 * c);
      }
    };
    {
      DEC_PART_IDS();
      const int n = (nr - wave + DEC_WAVES - 1) / DEC_WAVES;   // this wave's (may be <= 0)
      if constexpr (att || comb || !DEC_EARLY) {
#pragma unroll
        for (int d = 0; d < EP; ++d) load_row(d, d);
      }
      const uint4 nw = tid < (hid >> 3) ? ldg16(P.norm2 + 8 * tid) : make_uint4(0, 0, 0, 0);
      if (att && wave >= 4) dec_vmcnt0();   // waves outside the x1 gather: their LDS loads have landed
      __syncthreads();
      DEC_STAMPT(l, 10);
      const int erd = xgather<(KC + 1) / 2 * 2, 256>(XL + X.x1, hid, tag, xres, err, a.host_err, tid);
      DEC_STAMPV(l, 10, erd);
      DEC_STAMP(l, 11);
      block_norm(xres, nw, hid, a.eps, a.n_dtype, xs, red, tid);
#pragma unroll
      for (int j = 0; j < (RFE < DEC_RFE_N ? RFE : DEC_RFE_N); ++j) load_down(j);
      uint4 xv[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c) xv[c] = *(const uint4*)(xs + c * 512 + lane * 8);
      // per-lane partial sums of this wave's rows: slot k < MLW is LDS row wave + 8 k, slot
      // MLW + k ring row k; summed over the wave 8 slots (16 values) at a time afterwards
      constexpr int MLW = (NE + DEC_WAVES - 1) / DEC_WAVES, NS = MLW + EM, NG = (NS + 7) / 8;
      float gs[8 * NG], us[8 * NG];
#pragma unroll
      for (int s = 0; s < 8 * NG; ++s) gs[s] = us[s] = 0.f;
      // the LDS rows first (a row's 2 KC reads issued together)
      if (NL > 0) {   // workgroup-uniform
        const unsigned char* eb = (const unsigned char*)ebuf + EOFF;
#pragma unroll
        for (int k = 0; k < MLW; ++k) {
          const int i = wave + DEC_WAVES * k, ii = min(i, NL - 1);
          uint4 eg[KC], eu[KC];
#pragma unroll
          for (int c = 0; c < KC; ++c) {
            eg[c] = *(const uint4*)(eb + ((ii * 2 + 0) * KC + c) * 1024 + lane * 16);
            eu[c] = *(const uint4*)(eb + ((ii * 2 + 1) * KC + c) * 1024 + lane * 16);
          }
          float g = 0.f, u = 0.f;
#pragma unroll
          for (int c = 0; c < KC; ++c) {
            g = ddot8(xv[c], eg[c], g);
            u = ddot8(xv[c], eu[c], u);
          }
          gs[k] = i < NL ? g : 0.f;
          us[k] = i < NL ? u : 0.f;
        }
      }
#pragma unroll
      for (int j = DEC_RFE_N; j < RFE; ++j) load_down(j);
#pragma unroll
      for (int k = 0; k < EM; ++k) {
        const int d = k % EP;
        float g = 0.f, u = 0.f;
        if (k < n) {   // wave-uniform
#pragma unroll
          for (int c = 0; c < KC; ++c) {
            g = ddot8(xv[c], wg[d][c], g);
            u = ddot8(xv[c], wu[d][c], u);
          }
        }
        if (k + EP < EM) load_row(d, k + EP);
        gs[MLW + k] = g;
        us[MLW + k] = u;
      }
      // lane 8 s + 4 j of group q ends with slot 8 q + s's gate (j = 0) or up (j = 1) total; lane
      // 8 s computes SiLU(gate) * up and stages it under the slot's row
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        float v[16];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          v[2 * s] = gs[8 * q + s];
          v[2 * s + 1] = us[8 * q + s];
        }
        const float t = wave_sum16(v, lane);
        // row_ror:12 moves lane j + 4's value (mod 16) to lane j: lane 8 s receives the up total
        const float gv = rb(t), uv = rb(HS_DPP(t, HS_ROW_ROR12));
        const uint16_t h = f32_to_bf16(rb(gv / (1.f + expf(-gv))) * uv);
        const int s = 8 * q + (lane >> 3);
        if ((lane & 7) == 0 && s < NS) {
          const int k = s < MLW ? s : s - MLW;
          const bool ok = s < MLW ? wave + DEC_WAVES * k < NL : k < n;
          if (ok) ostage[(s < MLW ? 0 : NL) + wave + DEC_WAVES * k] = h;
        }
      }
      __syncthreads();
      if (tid < ecnt) xput(XL + X.h + e0 + tid, ostage[tid], tag);
      DEC_STAMP(l, 12);
    }

    // ---- F: down_proj + residual (the 8 waves split each row's K) ---------------------------------------
    {
      DEC_PART_IDS();
      const int RB = (hid + NWG - 1) / NWG;
      const int K8 = a.inter >> 3;
      uint16_t* hs = (uint16_t*)ebuf;   // (this layer's gate / up and o_proj rows are consumed)
      __syncthreads();
      // the other weights are issued only now: a CU's memory requests complete in order, so loads
      // issued before the h stores would hold those stores back, and with them every workgroup's F
#pragma unroll
      for (int j = RFE; j < RF; ++j) load_down(j);
      DEC_STAMPT(l, 13);
      const int frd = xgather<(IC * 4096 / 2 + DEC_THREADS - 1) / DEC_THREADS>(XL + X.h, a.inter, tag, hs, err,
                                                                               a.host_err, tid);
      DEC_STAMPV(l, 13, frd);
      DEC_STAMP(l, 14);
      float part[RF];
#pragma unroll
      for (int j = 0; j < RF; ++j) part[j] = 0.f;
#pragma unroll
      for (int k = 0; k < IC; ++k) {
        const int c = 512 * k + 64 * wave + lane;
        if (c < K8) {
          const uint4 hv = *(const uint4*)(hs + 8 * c);
#pragma unroll
          for (int j = 0; j < RF; ++j) part[j] = ddot8(hv, fw[j][k], part[j]);
        }
      }
      {   // the RF (<= 8) row sums of this wave at once: lane 8 j ends with row j's
        static_assert(RF <= 8, "down_proj rows per workgroup");
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = j < RF ? part[j] : 0.f;
        const float sum = wave_sum8(v, lane);
        if ((lane & 7) == 0 && (lane >> 3) < RF) red[wave * 8 + (lane >> 3)] = sum;
      }
      if (tid < 14) ptab[(l + 1) & 1][tid] = pnext;   // the next layer's tensors (read after the barrier)
      __syncthreads();
      if (tid < RB && b * RB + tid < hid) {
        const int r = b * RB + tid;
        float acc = 0.f;
#pragma unroll
        for (int w8 = 0; w8 < DEC_WAVES; ++w8) acc += red[w8 * 8 + tid];
        xput(XN + r, f32_to_bf16(bfh(xres[r]) + rb(acc)), tag);
      }
      DEC_STAMP(l, 15);
    }
  }

  // ---- G: final RMSNorm, lm_head, logits and argmax keys -------------------------------------------
  // The vocabulary goes in rounds of 8 R4 rows, round k of workgroup b being rows (k NWG + b) 8 R4 ..:
  // at any time the workgroups stream one contiguous window of the matrix. (Each workgroup's own
  // contiguous 1/NWG of it took 67.2 us per step at Qwen2.5-1.5B's 467 MB, its slowest workgroup
  // 71.0; interleaved: 63.8 and 67.0.)
  {
    DEC_PART_IDS();
    uint32_t* XF = a.ll + X.stride * a.L;
    constexpr int R4 = DEC_R4;   // rows per wave per round; two rounds in flight
    const long long GSTEP = (long long)NWG * DEC_WAVES * R4;
    // the workgroups that take a share of the last, partial round are the last ones, not the
    // first: workgroup 0 gathers every workgroup's argmax key once its own share is done
    const long long V = a.vocab, rend = V;
    const int xtra = (int)(((V % GSTEP) + DEC_WAVES * R4 - 1) / (DEC_WAVES * R4));   // workgroups with one more round
    const long long r0 = (long long)((b + NWG - xtra) % NWG) * DEC_WAVES * R4;
    uint4 wc[R4][KC], wn[R4][KC];
    auto issue = [&](uint4 (&w)[R4][KC], long long base) {
#pragma unroll
      for (int i = 0; i < R4; ++i) {
        const long long r = base + wave + (long long)DEC_WAVES * i;
#pragma unroll
        for (int c = 0; c < KC; ++c) w[i][c] = ldw(a.lm_w + min(r, rend - 1) * hid + c * 512 + lane * 8);
      }
    };
    issue(wc, r0);
    const uint4 nw = tid < (hid >> 3) ? *(const uint4*)(a.norm_f + 8 * tid) : make_uint4(0, 0, 0, 0);
    __syncthreads();
    DEC_STAMP(a.L, 0);
    xgather<(KC + 1) / 2>(XF, hid, tag, xres, err, a.host_err, tid);
    DEC_STAMP(a.L, 1);
    block_norm(xres, nw, hid, a.eps_f, a.n_dtype, xs, red, tid);
    unsigned long long best = 0ull;
    for (long long base = r0; base < rend; base += GSTEP) {
      const bool more = base + GSTEP < rend;
      if (more) issue(wn, base + GSTEP);
#pragma unroll
      for (int i = 0; i < R4; ++i) {
        const long long r = base + wave + (long long)DEC_WAVES * i;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = ddot8(*(const uint4*)(xs + c * 512 + lane * 8), wc[i][c], acc);
        acc = wave_sum(acc);
        if (r < rend) {
          const uint16_t hb = f32_to_bf16(acc);
          if (lane == 0) a.logits[r] = hb;
          const unsigned long long k = key48(hb, (unsigned)r);
          best = k > best ? k : best;
        }
      }
      if (more) {
#pragma unroll
        for (int i = 0; i < R4; ++i)
#pragma unroll
          for (int c = 0; c < KC; ++c) wc[i][c] = wn[i][c];
      }
    }
    DEC_STAMP(a.L, 2);
    if (lane == 0) kred[wave] = best;
    __syncthreads();
    if (tid == 0) {
      unsigned long long k = kred[0];
#pragma unroll
      for (int w8 = 1; w8 < DEC_WAVES; ++w8) k = kred[w8] > k ? kred[w8] : k;
      __hip_atomic_store((unsigned long long*)(keys + 2 * (long long)b), ((unsigned long long)tag << 48) | k,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- workgroup 0: the next token from every workgroup's key, then the step tag ----------------------
  if (b == 0) {
    __syncthreads();   // thread 0 has read kred above
    unsigned long long k = 0ull;
    const unsigned long long t0 = wall_clock64();
    for (int i = tid; i < NWG; i += DEC_THREADS) {
      unsigned long long v = xget2(keys + 2 * (long long)i);
      while ((uint32_t)(v >> 48) != tag) {
        if (wall_clock64() - t0 > DEC_TIMEOUT) {
          dec_fail(err, a.host_err);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        v = xget2(keys + 2 * (long long)i);
      }
      const unsigned long long kk = v & 0xFFFFFFFFFFFFull;
      k = kk > k ? kk : k;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long other = __shfl_xor(k, o, 64);
      k = other > k ? other : k;
    }
    if (lane == 0) kred[wave] = k;
    __syncthreads();
    if (tid == 0) {
      unsigned long long m = kred[0];
#pragma unroll
      for (int w8 = 1; w8 < DEC_WAVES; ++w8) m = kred[w8] > m ? kred[w8] : m;
      const long long idx = (long long)(0xFFFFFFFFu - (uint32_t)(m & 0xFFFFFFFFull));
      if (a.out_dtype == HS_I64) *(long long*)a.next_token = idx;
      else *(int*)a.next_token = (int)idx;
      __hip_atomic_store(ctl, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // the next step's position inputs (every workgroup read its inputs before its argmax key,
      // and every key is in): one more position, its mask entry opened
      if (a.adv_flag != nullptr) {
        const long long p = a.adv_cpos[0] + 1;
        a.adv_cpos[0] = p;
        a.adv_pos[0] = p;
        if (p >= 0 && p < S) {
          if (a.adv_mask_bytes == 4) ((float*)a.adv_mask)[p] = 0.f;
          else ((uint16_t*)a.adv_mask)[p] = 0;
        }
      }
    }
    DEC_STAMP(a.L, 3);
  }
}

#define DECODE_KERNEL(KC, IC, EM) \
  extern "C" __global__ void __launch_bounds__(DEC_THREADS) k_decode_step_k##KC##_i##IC##_e##EM(const PersistArgs a) { \
    __shared__ DecShared<KC, DEC_NE(KC)> sh; \
    const int nb_ = a.H * a.nsplit; \
    if ((int)blockIdx.x < nb_) decode_body<KC, IC, EM, 0, false>(a, sh); \
    else if (!(a.flags & 2) && (int)blockIdx.x < nb_ + a.H) decode_body<KC, IC, EM, 2, false>(a, sh); \
    else decode_body<KC, IC, EM, 1, false>(a, sh); \
  }
// KV-head-major attention (long caches): nsplit slots per KV head, KVH nsplit attention workgroups
#define DECODE_KERNEL_KV(KC, IC, EM) \
  extern "C" __global__ void __launch_bounds__(DEC_THREADS) k_decode_step_k##KC##_i##IC##_e##EM##_kv(const PersistArgs a) { \
    __shared__ DecShared<KC, DEC_NE(KC)> sh; \
    const int nb_ = a.KVH * a.nsplit; \
    if ((int)blockIdx.x < nb_) decode_body<KC, IC, EM, 0, true>(a, sh); \
    else if ((int)blockIdx.x < nb_ + a.H) decode_body<KC, IC, EM, 2, true>(a, sh); \
    else decode_body<KC, IC, EM, 1, true>(a, sh); \
  }

DECODE_KERNEL(3, 3, 2)   // hidden 1536 (Qwen2.5-1.5B: inter 8960, 12 heads x 16 slots: 16 streamed rows)
DECODE_KERNEL(3, 3, 3)   // hidden 1536, up to 24 streamed gate/up rows per workgroup
DECODE_KERNEL(3, 3, 4)   // hidden 1536, up to 32
DECODE_KERNEL(3, 3, 6)   // hidden 1536, up to 48
DECODE_KERNEL(1, 1, 1)   // hidden 512, up to 8
DECODE_KERNEL(1, 1, 2)   // hidden 512, up to 16
DECODE_KERNEL(2, 2, 4)   // hidden 1024, up to 32
DECODE_KERNEL_KV(3, 3, 2)   // hidden 1536, KV-head-major attention
DECODE_KERNEL_KV(1, 1, 1)   // hidden 512, KV-head-major attention

// ================================================================ one attention block, one launch
//
// k_attn_step_k<KC>: a graph that is one decode-token attention block (optional input RMSNorm,
// q / k / v with optional biases, RoPE, the K / V rows written at cache_position, GQA attention
// over the mask's open chunks, o_proj with optional residual) as one launch. Its launch list is
// three dependent launches (q/k/v + RoPE + cache rows, split attention, combine + o_proj) around
// ~12 MB at Qwen2.5-1.5B's shape, whose launch boundaries take most of the time. These are the
// decode step's parts A-D for one layer, with the same exchange words, chunk walk and rounding
// points:
//   A  every workgroup: q / k / v rows b RB .. b RB + RB - 1 (RB <= 8), one per wave
//   B  workgroups b < NB = H nsplit: (query head, KV head, slot) as in the decode step, its
//      first chunk's K and V rows issued before it waits for q / k / v
//   C  workgroups NB .. NB + H - 1: one head's partials combined into its D attention words
//   D  workgroups NB + i, i < ceil(hidden / RD): o_proj rows i RD .. i RD + RD - 1 (loaded into
//      LDS once A is out); + residual; out
// Exchange words: [H][q | k | v], [H][nsplit][D + 4] partials, [H D] attention row, then the step
// tag and the timeout flag. Workgroup NB writes the new step tag once it holds the whole
// attention row: it depends on every workgroup's q / k / v rows, so every workgroup has read the
// old tag by then. (Every o_proj workgroup combining all the partials itself instead, one
// hand-off fewer, measured slower: 140 workgroups gathering 57 KB each.)
#define AST_ROWS 32   // o_proj rows per workgroup, at most (its LDS)

template <int KC>
struct AttnShared {
  __attribute__((aligned(16))) unsigned char smem[DEC_SMEM];   // B, C staging; the normalised x; the attention row
  __attribute__((aligned(16))) uint16_t xres[512 * KC];        // the input row
  __attribute__((aligned(16))) uint4 obuf[AST_ROWS * KC * 64];  // o_proj row i, chunk c: 1 KB at KC i + c
  float red[DEC_WAVES * 8];
  float red2[DEC_WAVES * DEC_MAXG];
  float rope_cs[128];
  const void* ptab[14];
  uint32_t obw[DEC_WAVES];
  uint16_t ostage[AST_ROWS];
};

template <int KC, int ROLE>
__device__ __forceinline__ void attn_step_body(const PersistArgs& a, AttnShared<KC>& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x, NWG = a.nwg;
  const int hid = a.hidden, H = a.H, KVH = a.KVH, G = H / KVH, NT = a.nsplit;
  const long long XP = (long long)H * 3 * DEC_D;                      // partials
  const long long XA = XP + (long long)H * NT * (DEC_D + 4);          // attention row
  uint32_t* ctl = a.ll + XA + (long long)H * DEC_D;                   // [0] step tag, [1] timeout flag
  uint32_t* err = ctl + 1;
  uint32_t tag = (__hip_atomic_load(ctl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u) & 0xFFFFu;
  tag = tag == 0 ? 1u : tag;
  const IRaw posw = ld_i_raw(a.pos_ids, 0, a.pos_dtype), cposw = ld_i_raw(a.cache_pos, 0, a.cpos_dtype);
  const long long posr = ld_i_decode(posw, a.pos_dtype);
  const long long cpos = ld_i_decode(cposw, a.cpos_dtype);
  uint16_t* xs = (uint16_t*)sh.smem;
  DEC_STAMP(0, 0);
  if (tid < 64) {   // rotary factors of this step's position, as in the decode step
    float sf, cf;
    sincos_rot(a.inv_freq[tid] * (float)posr, &sf, &cf);
    sh.rope_cs[tid] = round_to(cf * a.rope_scaling, HS_BF16);
    sh.rope_cs[64 + tid] = round_to(sf * a.rope_scaling, HS_BF16);
  }
  if (tid < 14) sh.ptab[tid] = ((const void* const*)a.layers)[tid];
  constexpr bool ATT = ROLE == 0, COMB = ROLE == 2;
  const int ntile = KVH * NT, NB = ntile * G;
  const int tile = b % ntile, gq = b / ntile, kvh = tile / NT, slot = tile % NT;
  const int RD = a.rows;                 // <= AST_ROWS (checked on the host)
  const long long d0 = (long long)(b - NB) * RD;
  uint32_t ob = 0;
  if constexpr (ATT) ob = dec_scan_chunks(a, slot, sh.obw, lane, wave);
  __syncthreads();
  if constexpr (ATT) {
    if (a.mask_dtype >= 0) {
#pragma unroll
      for (int w8 = 0; w8 < DEC_WAVES; ++w8) ob |= sh.obw[w8];
    }
  }
  const DecodeLayerPtrs P = dec_layer(sh.ptab);

  // ---- A: [RMSNorm], q / k / v rows (+ bias), published per query head ----------------------------
  {
    const int R = (H + 2 * KVH) * DEC_D, RB = (R + NWG - 1) / NWG;   // RB <= 8 (checked on the host)
    const int r = b * RB + wave;
    const bool has = wave < RB && r < R;
    const uint16_t* W;
    const uint16_t* B;
    int rr;
    if (r < H * DEC_D) {
      W = P.wq; B = P.bq; rr = r;
    } else if (r < (H + KVH) * DEC_D) {
      rr = r - H * DEC_D; W = P.wk; B = P.bk;
    } else {
      rr = r - (H + KVH) * DEC_D; W = P.wv; B = P.bv;
    }
    const long long rl = has ? rr : 0;   // a wave without a row re-reads row 0 of q (unused)
    const uint16_t* Wl = has ? W : P.wq;
    const bool norm = P.norm1 != nullptr;
    const int nch = hid >> 3;
    const uint4 xv = tid < nch ? ldg16(a.xin + 8 * tid) : make_uint4(0, 0, 0, 0);
    uint4 w[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) w[c] = ldw(Wl + rl * hid + c * 512 + lane * 8);
    const uint16_t bias = (has && (a.flags & 1)) ? ldg2(B + rr) : (uint16_t)0;
    const uint4 nw = (norm && tid < nch) ? ldg16(P.norm1 + 8 * tid) : make_uint4(0, 0, 0, 0);
    if (tid < nch) *(uint4*)(sh.xres + 8 * tid) = xv;
    __syncthreads();
    DEC_STAMP(0, 1);
    const uint16_t* xn = sh.xres;
    if (norm) {
      block_norm(sh.xres, nw, hid, a.eps, a.n_dtype, xs, sh.red, tid);
      xn = xs;
    }
    if (has) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < KC; ++c) acc = ddot8(*(const uint4*)(xn + c * 512 + lane * 8), w[c], acc);
      acc = wave_sum(acc);
      if (lane == 0) sh.ostage[wave] = f32_to_bf16(acc + bfh(bias));
    }
    __syncthreads();
    // one store by wave 0: a k or v row goes into the blocks of all G heads that read it
    if (wave == 0 && lane < RB * G) {
      const int j = lane / G, g = lane % G, rj = b * RB + j;
      if (rj < R) {
        const int sj = rj < H * DEC_D ? 0 : (rj < (H + KVH) * DEC_D ? 1 : 2);
        const int rrj = rj - (sj == 0 ? 0 : (sj == 1 ? H * DEC_D : (H + KVH) * DEC_D));
        const int hq = sj == 0 ? rrj / DEC_D : (rrj / DEC_D) * G + g;
        if (sj != 0 || g == 0) xput(a.ll + (long long)hq * 3 * DEC_D + sj * DEC_D + rrj % DEC_D, sh.ostage[j], tag);
      }
    }
    DEC_STAMP(0, 2);
  }

  if constexpr (ATT) {
    // ---- B ----
    const int hq = kvh * G + gq;
    dec_attend<true>(a, 0, P.kc, P.vc, a.ll + (long long)hq * 3 * DEC_D,
                     a.ll + XP + ((long long)hq * NT + slot) * (DEC_D + 4), ob, kvh, gq, slot, cpos, tag, err,
                     sh.smem, sh.rope_cs, sh.red, sh.red2, tid, lane, wave);
    DEC_STAMP(0, 4);
  } else {
    // ---- D's o_proj rows into LDS; the residual values ----
    const long long rmax = min(d0 + RD, (long long)hid) - 1;   // rows past the last re-read it
    const unsigned base = (unsigned)(size_t)(__attribute__((address_space(3))) void*)&sh.obuf[0];
    for (int k = wave; k < RD * KC; k += DEC_WAVES) {
      const long long r = max(min(d0 + k / KC, rmax), 0ll);
      dec_dma16(P.wo + r * hid + (k % KC) * 512 + lane * 8, __builtin_amdgcn_readfirstlane(base + (unsigned)k * 1024u));
    }
    const bool rin = a.resid != nullptr && tid < RD && d0 + tid < hid;
    const uint16_t rv = rin ? ldg2(a.resid + d0 + tid) : (uint16_t)0;
    // ---- C ----
    if constexpr (COMB) {
      const int h = b - NB;
      dec_combine(a, 0, a.ll + XP + (long long)h * NT * (DEC_D + 4), a.ll + XA + (long long)h * DEC_D, tag, err,
                  sh.smem, sh.red2, tid, lane, wave);
    }
    if (d0 >= hid) return;   // no o_proj rows (workgroup NB, which writes the tag, always has some)
    dec_vmcnt0();   // this wave's o_proj rows have landed (the gather's barrier publishes them to all)
    __syncthreads();
    DEC_STAMP(0, 7);
    xgather<(KC + 1) / 2 * 2, 256>(a.ll + XA, H * DEC_D, tag, xs, err, a.host_err, tid);
    DEC_STAMP(0, 8);
    if (b == NB && tid == 0) __hip_atomic_store(ctl, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // ---- D: o_proj [+ residual] -> out ----
    const unsigned char* ow = (const unsigned char*)sh.obuf;
    uint4 xa[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) xa[c] = *(const uint4*)(xs + c * 512 + lane * 8);
    constexpr int MD = (AST_ROWS + DEC_WAVES - 1) / DEC_WAVES;   // rows per wave, at most: wave + 8 k
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int i = wave + DEC_WAVES * k;
      v[k] = 0.f;
      if (k < MD && i < RD && d0 + i < hid) {   // wave-uniform
        uint4 wr[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) wr[c] = *(const uint4*)(ow + (i * KC + c) * 1024 + lane * 16);
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = ddot8(xa[c], wr[c], acc);
        v[k] = acc;
      }
    }
    const float sum = wave_sum8(v, lane);   // lane 8 k: row wave + 8 k
    const int i = wave + DEC_WAVES * (lane >> 3);
    if ((lane & 7) == 0 && (lane >> 3) < MD && i < RD && d0 + i < hid) sh.ostage[i] = f32_to_bf16(sum);
    __syncthreads();
    if (tid < RD && d0 + tid < hid) {
      uint16_t o = sh.ostage[tid];
      if (rin) o = f32_to_bf16(bfh(rv) + bfh(o));
      stg2(a.out + d0 + tid, o);
    }
    DEC_STAMP(0, 9);
  }
}

#define ATTN_STEP_KERNEL(KC) \
  extern "C" __global__ void __launch_bounds__(DEC_THREADS) k_attn_step_k##KC(const PersistArgs a) { \
    __shared__ AttnShared<KC> sh; \
    const int nb_ = a.H * a.nsplit; \
    if ((int)blockIdx.x < nb_) attn_step_body<KC, 0>(a, sh); \
    else if ((int)blockIdx.x < nb_ + a.H) attn_step_body<KC, 2>(a, sh); \
    else attn_step_body<KC, 1>(a, sh); \
  }

ATTN_STEP_KERNEL(1)   // hidden 512
ATTN_STEP_KERNEL(2)   // hidden 1024
ATTN_STEP_KERNEL(3)   // hidden 1536 (Qwen2.5-1.5B)
