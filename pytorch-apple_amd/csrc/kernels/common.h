// Shared definitions for the gfx950 kernels: dtype codes, bf16/fp16 helpers,
// wave64 reductions and the by-value argument structs of every kernel.
//
// Every kernel takes exactly one argument, a struct passed by value, so its
// kernarg segment is the struct's C layout. The host packs the same layout with
// ctypes; hs_argsize() in the shim reports sizeof() of each struct so the host
// can check the two agree. Fields are ordered 8-byte first, then 4-byte, so no
// implicit padding appears between them.
#pragma once

// hiprtc (generated kernels) provides the HIP device definitions and fixed-width
// integer types itself, so the headers are only included for hipcc builds
#if defined(__HIPCC__) && !defined(__HIPCC_RTC__)
#include <hip/hip_runtime.h>
#endif
#ifdef __HIPCC_RTC__
typedef signed char int8_t;
typedef unsigned char uint8_t;
typedef short int16_t;
typedef unsigned short uint16_t;
typedef int int32_t;
typedef unsigned int uint32_t;
typedef long long int64_t;
typedef unsigned long long uint64_t;
#else
#include <stdint.h>
#endif

#define HS_MAXD 6

enum HsDtype { HS_F32 = 0, HS_F16 = 1, HS_BF16 = 2, HS_I64 = 3, HS_I32 = 4, HS_U8 = 5, HS_F64 = 6 };

// ---------------------------------------------------------------- argument structs

struct CopyArgs {            // dst[idx(dshape, dstride)] = cast(src[idx(dshape, sstride)])
  void* dst;
  const void* src;
  long long n;
  long long shape[HS_MAXD];
  long long sstride[HS_MAXD];
  long long dstride[HS_MAXD];
  int ndim;
  int sdtype;
  int ddtype;
  int pad;
};

struct FillArgs {
  void* out;
  long long n;
  double value;
  int dtype;
  int pad;
};

struct AdvanceArgs {          // k_decode_advance: the next decode step's position inputs, on the device
  void* mask;                 // [S] additive mask row, element size mask_bytes (2 or 4): entry p set to 0
  long long* pos;             // position_ids [1, 1]
  long long* cpos;            // cache_position [1]
  int* overflow;              // set to 1 when a step would move past the cache end (nothing else written)
  long long S;
  int mask_bytes;
  int pad;
};

struct RMSNormArgs {          // out = w * round_n(x * rsqrt(mean(x^2) + eps)), one row per workgroup
  const void* x;
  const void* w;
  void* out;
  long long rows;
  long long ldx;
  long long ldo;
  int cols;
  float eps;
  int x_dtype;
  int w_dtype;
  int n_dtype;
  int out_dtype;
};

struct EmbeddingArgs {        // out[s, :] = w[ids[s], :]
  const void* w;
  const void* ids;
  void* out;
  long long n_ids;
  long long vocab;
  long long row_bytes;
  int ids_dtype;
  int pad;
};

struct RopeTableArgs {        // cos/sin[s, j] for j < 2*half from inv_freq[j % half] * pos[s]
  const float* inv_freq;
  const void* pos;
  void* cos_out;
  void* sin_out;
  long long S;
  int half;
  int pos_dtype;
  int out_dtype;
  float scaling;
};

struct IndexCopyArgs {        // dst[o, index[j], i] = src[o*s_o + j*s_j + i*s_i]
  void* dst;
  const void* src;
  const void* index;
  long long outer;
  long long dim_size;
  long long inner;
  long long nidx;
  long long src_so;
  long long src_sj;
  long long src_si;
  int idx_dtype;
  int elem_bytes;
};

struct SoftmaxArgs {          // out[row] = softmax(round_a(x[row] + mask[row'])) along the last dim
  const void* x;
  const void* mask;
  void* out;
  long long rows;
  long long cols;
  long long lead_shape[5];
  long long x_lead_stride[5];
  long long mask_lead_stride[5];
  long long mask_col_stride;
  int nlead;
  int x_dtype;
  int mask_dtype;
  int add_dtype;
  int out_dtype;
  int has_mask;
};

struct ReduceLastArgs {       // mean / argmax over the last dim of a [rows, cols] contiguous view
  const void* x;
  void* out;
  long long rows;
  long long cols;
  int x_dtype;
  int out_dtype;
};

struct ArgmaxPartArgs {       // per (row, column segment) argmax key of a [rows, cols] 16-bit view (gemv.hip)
  const void* x;              // rows of `cols` elements, 16-byte aligned, cols % 8 == 0
  unsigned long long* slot;   // [rows, parts] keys, reduced by k_argmax_finalize
  long long rows;
  long long cols;
  long long seg;              // columns per segment (multiple of 8); grid = (parts, rows)
  int x_dtype;                // bf16 or fp16
  int parts;
};

struct BmmArgs {              // c[b, m, n] = sum_k a[b, m, k] * b[b, k, n] (strided, broadcast batch)
  const void* a;
  const void* b;
  void* c;
  long long batch_shape[4];
  long long a_bstride[4];
  long long b_bstride[4];
  long long M;
  long long N;
  long long K;
  long long a_sm, a_sk, b_sk, b_sn;
  int nbatch;
  int a_dtype;
  int b_dtype;
  int c_dtype;
};

struct LinearArgs {           // out[m, n] = round(x[m, :] . w[n, :] + bias[n])   (bf16/fp16, K % 8 == 0)
  const void* x;
  const void* w;
  const void* bias;
  void* out;
  const void* resid;          // optional residual: out = round(resid + round(linear))
  long long M;
  long long ldx;
  long long ldo;
  long long ldr;
  int N;
  int K;
  int dtype;                  // HS_BF16 or HS_F16 for x, w, bias, out and resid alike
  int has_bias;
  int has_resid;
  int pad;
};

struct GemmArgs {             // MFMA GEMM (gemm.hip): out = epi(x . w^T), x [M, K], w [N, K], K % 32 == 0
  const void* x;              // [M, K] (row stride ldx), 16-byte aligned rows
  const void* w;              // [N, K] (row stride ldw); the _kn kernels take w as [K, N] (row stride ldw)
  const void* w2;             // second weight (SiLU * mul epilogue: w = gate, w2 = up) or null
  const void* bias;           // [N] or null
  const void* bias2;          // [N] or null (for w2)
  const void* resid;          // [M, N] (row stride ldr) or null
  void* out;                  // [M, N] (row stride ldo)
  float* part;                // split-K: fp32 partial sums [ksplit, NW, M, N], reduced by k_gemm_reduce_*
  const void* w3;             // grouped (_grp kernels): output columns [0, n1) use w / bias, [n1, n2) w2 / bias2,
  const void* bias3;          //   [n2, N) w3 / bias3 (row n - group start); n1, n2 multiples of the tile width
  long long M;
  long long ldx;
  long long ldw;
  long long ldo;
  long long ldr;
  long long sx;               // batched: element offsets of batch b: x + b*sx, w + (b / bdiv)*sw, out + b*so
  long long sw;
  long long so;
  int batch;                  // grid.z = batch * ksplit
  int bdiv;
  int N;
  int K;
  int flags;                  // 1: bias, 2: bias2
  int ksplit;                 // 1: epilogue in the GEMM; > 1: grid.z splits K into chunks of kchunk
  int kchunk;                 // K elements per split (multiple of 32)
  int nw;                     // weights (1, or 2 for SiLU * mul); read by the reduce kernel
  int n1;                     // grouped: first column of the second and third groups
  int n2;
  // conv epilogue (_conv kernels; flags 1 bias, 2 batch norm, 4 residual, 8 ReLU, as ConvArgs;
  // 16: tiles ordered N tile fastest)
  const void* bn_w;           // [N] batch norm weight, bias, running mean, running var
  const void* bn_b;
  const void* bn_mean;
  const void* bn_var;
  const void* zero;           // conv gather (_convg kernels): >= 16 zero bytes, read for padded taps
  float eps;
  // _convg: x is NHWC [*, cH, cW, cCin], row m = output pixel (n, ho, wo), padded taps read `zero`;
  // _convp: x is an already zero-bordered NHWC image [*, cH, cW, cCin = 4], k = (kh * cKW + kw) * 4 + c
  // with cKW even, so a 16-byte chunk is two neighbouring taps of one kernel row (always in bounds)
  int cH;                     // conv gather: x is NHWC [*, cH, cW, cCin], row m = output pixel (n, ho, wo),
  int cW;                     //   k = (kh * cKW + kw) * cCin + ci, cCin % 64 == 0; w is [N, KH * KW * Cin] (OHWI)
  int cCin;
  int cHo;
  int cWo;
  int cKW;
  int csh;
  int csw;
  int cph;
  int cpw;
};

struct ConvArgs {             // implicit-GEMM conv2d (conv.hip), NCHW activations, OIHW weights, groups 1
  const void* x;              // [N, Cin, H, W]
  const void* w;              // [Cout, Cin, KH, KW]
  const void* bias;           // [Cout] or null
  const void* bn_w;           // batch-norm (inference) of the conv output: weight, bias, running stats [Cout]
  const void* bn_b;
  const void* bn_mean;
  const void* bn_var;
  const void* resid;          // [N, Cout, Ho, Wo] added after the batch norm, or null
  void* out;                  // [N, Cout, Ho, Wo]
  float* part;                // split K: fp32 partial sums [ksplit, Cout, M], reduced by k_conv_reduce_*
  long long M;                // N * Ho * Wo
  int N, Cin, H, W, Cout, Ho, Wo, KH, KW, sh, sw, ph, pw;
  int K;                      // Cin * KH * KW
  float eps;
  int flags;                  // 1 bias, 2 batch norm, 4 residual add, 8 ReLU
  int ksplit;                 // 1: epilogue in the conv; > 1: grid.z splits K into chunks of kchunk
  int kchunk;                 // multiple of the K step (32)
};

struct PoolArgs {             // max pooling (conv.hip): NCHW, or NHWC for the _nhwc kernel
  const void* x;
  void* out;
  long long planes;           // N * C
  int H, W, Ho, Wo, kh, kw, sh, sw, ph, pw;
  int dtype;
  int C;                      // channels-last kernels (_nhwc): C (multiple of 8); unused otherwise
};

#define HS_OHWI_MAX 24
struct PermuteOHWIArgs {      // OIHW -> (zero-padded) OHWI copies of up to HS_OHWI_MAX 2-byte weights, one launch (conv.hip)
  const void* src[HS_OHWI_MAX];   // [Cout, cin, kh, kw]
  void* dst[HS_OHWI_MAX];         // [Cout, khp, kwp, cp]: zero where kh <= y, kw <= x or cin <= c
  long long start[HS_OHWI_MAX + 1];   // first element of tensor i in the joint index space; start[n] = total
  int cin[HS_OHWI_MAX];
  int kh[HS_OHWI_MAX];
  int kw[HS_OHWI_MAX];
  int cp[HS_OHWI_MAX];
  int khp[HS_OHWI_MAX];
  int kwp[HS_OHWI_MAX];           // Cout * khp * kwp * cp is a multiple of 8
  int n;
  int pad;
};

struct PadNHWCArgs {          // NCHW [N, C, H, W] -> zero-bordered NHWC [N, Hp, Wp, 4] (C <= 4) (conv.hip)
  const void* x;
  void* out;
  long long n;
  int C;
  int H;
  int W;
  int Hp;
  int Wp;
  int top;                    // rows / columns of zeros before the image
  int left;
  int pad;
};

struct MeanNHWCArgs {         // [n, hw, c] -> [n, c] mean over hw (conv.hip, global average pool of NHWC)
  const void* x;
  void* out;
  long long n;
  int hw;
  int c;                      // multiple of 8, 16-byte aligned rows
};

struct BatchNormArgs {        // inference batch norm over NCHW (channel = dim 1), optional ReLU
  const void* x;
  const void* w;
  const void* b;
  const void* mean;
  const void* var;
  void* out;
  long long n;                // N * C * HW
  long long hw;
  int C;
  float eps;
  int dtype;                  // x and out
  int relu;
  int p_dtype;                // w, b, mean, var
  int pad;
};

struct GemvArgs {             // fused decode GEMV (gemv.hip): prologue RMSNorm, epilogues bias/resid/silu/argmax
  const void* x;              // [M, K] bf16 activations (raw residual stream when NORM)
  const void* w;              // [N, K] bf16
  const void* bias;           // [N] or null
  void* out;                  // [M, N] bf16
  const void* resid;          // [M, N] residual (RESID)
  const void* w2;             // [N, K] second weight (SILU: up projection)
  const void* bias2;          // [N] or null
  const void* norm_w;         // [K] RMSNorm weight (NORM)
  unsigned long long* argmax_slot;  // [M, grid.x] packed (value, ~index) keys per workgroup (ARGMAX)
  const uint16_t* attn_o;     // ATTN prologue: split partials (bf16, normalised) of the decode attention feeding x
  const float* attn_ml;
  long long M;
  long long ldx;
  long long ldo;
  long long ldr;
  int N;
  int K;
  float eps;
  int n_dtype;                // rounding dtype of x * rsqrt(...) (the to(dtype) of the norm)
  int flags;                  // 1: bias, 4: bias2
  int attn_heads;             // ATTN prologue: H, KVH, nsplit (x = heads * 128 values)
  int attn_kvh;
  int attn_splits;
};

// ---- persistent decode step (decode.hip): one launch runs every layer of a decoder step
struct DecodeLayerPtrs {      // one decoder layer's tensors, gathered from the layer's launch records
  const uint16_t* norm1;      // [hidden] input RMSNorm weight
  const uint16_t* wq;         // [H*D, hidden]
  const uint16_t* bq;         // [H*D] or null
  const uint16_t* wk;         // [KVH*D, hidden]
  const uint16_t* bk;
  const uint16_t* wv;
  const uint16_t* bv;
  uint16_t* kc;               // K cache [KVH, S, D] (updated in place at cache_position)
  uint16_t* vc;               // V cache
  const uint16_t* wo;         // [hidden, H*D]
  const uint16_t* norm2;      // [hidden] post-attention RMSNorm weight
  const uint16_t* wg;         // [inter, hidden]
  const uint16_t* wu;         // [inter, hidden]
  const uint16_t* wd;         // [hidden, inter]
};

struct PersistArgs {
  const DecodeLayerPtrs* layers;   // [L] table in device memory
  const uint16_t* emb;        // [vocab, hidden] token embedding
  const void* ids;            // input_ids (one token)
  const void* pos_ids;        // position_ids (rotary position)
  const void* cache_pos;      // cache_position (cache row written)
  const void* mask;           // [S] additive mask row (bf16 / fp32)
  const float* inv_freq;      // [D/2]
  const uint16_t* norm_f;     // [hidden] final RMSNorm weight
  const uint16_t* lm_w;       // [vocab, hidden]
  uint16_t* logits;           // [vocab]
  void* next_token;           // [1] argmax of the logits
  uint32_t* ll;               // exchange words (low 16 bits payload, high 16 bits step tag) + keys + control
  unsigned long long* trace;  // null, or [nwg][L * 16 + 8] real-time stamps of each part's progress
  long long S;                // cache length
  long long kv_head_stride;   // elements between KV heads of a cache
  long long vocab;
  int L, hidden, inter, H, KVH, D;
  int nsplit;                 // attention workgroups (slots) per query head; slot j walks the cache's
                              // 128-position chunks j, j + nsplit, ... (those its mask leaves open)
  int nwg;                    // workgroups of the launch (all resident at once)
  int ids_dtype, pos_dtype, cpos_dtype, mask_dtype, add_dtype, n_dtype, out_dtype;
  int flags;                  // 1: q/k/v biases present; 2: the attention workgroups run the combine
  float eps, eps_f, scale, rope_scaling;
  // optional in-kernel decode advance (adv_flag null: none). After the step, the next step's
  // inputs: p = adv_cpos + 1; adv_cpos = adv_pos = p; adv_mask[p] = 0 when p < S. A step that
  // starts with cache_position outside [0, S) sets adv_flag[0] (it re-runs no position silently).
  void* adv_mask;             // [S] additive mask row, element size adv_mask_bytes (2 or 4)
  long long* adv_pos;         // position_ids [1, 1]
  long long* adv_cpos;        // cache_position [1]
  int* adv_flag;              // [0]: a step ran past the cache end
  int adv_mask_bytes, adv_pad;
  int nchunk;                 // 128-position chunks of the cache: ceil(S / 128), at most 32 per slot
  int rbo, rba, rbc;          // gate / up rows streamed through registers per o_proj / attention / combine
                              // workgroup
  int rows;                   // the attention step's o_proj rows per workgroup (unused by the decode step)
  int* host_err;              // null, or a host-visible word set to 1 when a wait times out
  // the one-block attention step (k_attn_step_k*): its input row, output row and residual row
  // (null: no residual); unused by the decode step
  const uint16_t* xin;
  uint16_t* out;
  const uint16_t* resid;
};

struct ArgmaxFinalizeArgs {   // out[m] = index of max over the `parts` keys of row m
  const unsigned long long* slot;   // [rows, parts] packed (ordered value, ~index) keys
  void* out;
  long long rows;
  int parts;
  int out_dtype;
};

struct QKVArgs {              // RMSNorm -> q/k/v projections -> RoPE -> K/V cache rows (gemv.hip)
  const void* x;
  const void* norm_w;
  const void* wq;
  const void* bq;
  const void* wk;
  const void* bk;
  const void* wv;
  const void* bv;
  const float* inv_freq;
  const void* pos_ids;
  const void* cache_pos;
  void* q_out;                // [H, D]
  void* k_dst;                // K cache [KVH, S, D] (flag 16) or [KVH, D]
  void* v_dst;                // V cache [KVH, S, D] (flag 32) or [KVH, D]
  long long kv_head_stride;
  long long cache_len;
  int K;
  int H;
  int KVH;
  int D;
  float eps;
  int n_dtype;
  int flags;                  // 1 norm, 2 bias, 4 rope q, 8 rope k, 16 k to cache, 32 v to cache
  int pos_dtype;
  int cpos_dtype;
  float rope_scaling;
};

struct RopeCacheArgs {        // prefill: RoPE of q and k from the q | k | v projection rows, K/V cache rows (gemv.hip)
  const void* y;              // [T, ldy]: columns q (H*D) | k (KVH*D) | v (KVH*D)
  const float* inv_freq;      // [D/2]
  const void* pos_ids;        // [T] int64 / int32
  const void* cache_pos;      // [T] int64 / int32
  void* q_out;                // [H, T, D]
  void* k_dst;                // K cache [KVH, S, D] (flag 16) or [KVH, T, D]
  void* v_dst;                // V cache [KVH, S, D] (flag 32) or [KVH, T, D]
  long long ldy;
  long long kv_head_stride;   // elements between KV heads of the destination
  long long cache_len;        // S (flag 16 / 32): rows at positions outside [0, S) are not written
  int T;
  int H;
  int KVH;
  int D;                      // even, <= 128
  int flags;                  // 4 rope q, 8 rope k, 16 k to cache, 32 v to cache
  int pos_dtype;
  int cpos_dtype;
  int dtype;                  // bf16 or fp16 storage
  float rope_scaling;
};

struct FusedArgs {            // generated elementwise chains: out[i] = chain(in0..in7 at strided offsets)
  void* out;
  const void* in[8];
  long long n;
};

struct DecodeAttnArgs {       // GQA decode attention over static caches, split over KV tiles
  const void* q;              // [H, D] (query heads contiguous, D contiguous)
  const void* k;              // [KVH, S, D]
  const void* v;              // [KVH, S, D]
  const void* mask;           // [S] with stride mask_stride (broadcast over heads)
  void* out;                  // [H, D]
  float* scores;              // scratch [H, S]
  float* stats;               // scratch [H, ntiles, 2]
  long long S;
  long long q_head_stride;
  long long kv_head_stride;
  long long mask_stride;
  int H;
  int KVH;
  int D;
  int ntiles;
  float scale;
  int mask_dtype;             // HS_BF16 / HS_F16 / HS_F32, or -1 for no mask
  int add_dtype;              // dtype of scores + mask in the model (rounding point)
  int dtype;                  // q/k/v/out dtype (HS_BF16 or HS_F16)
};

struct FlashArgs {            // split-S decode attention: per-split (max, sum, unnormalised p.V)
  const void* q;              // [H, D]
  const void* k;              // [KVH, S, D]
  const void* v;              // [KVH, S, D]
  const void* mask;           // [S] (stride mask_stride), broadcast over heads
  uint16_t* part_o;           // [KVH, nsplit, G, D] bf16 of the split's own softmax . V: sum_s e^(s - m) v_s / l
  float* part_ml;             // [KVH, nsplit, G, 2] (m, l) of the split; l = 0 when fully masked
  long long S;
  long long q_head_stride;
  long long kv_head_stride;
  long long mask_stride;
  int H;
  int KVH;
  int nsplit;
  int spl;                    // positions per split: 64 (FL_SPL)
  float scale;
  int mask_dtype;             // -1: no mask
  int add_dtype;
  int dtype;
};

struct PrefillAttnArgs {      // causal / masked attention of T queries over S keys (attention.hip, MFMA)
  const void* q;              // [H, T, D] (q_head_stride, row stride D)
  const void* k;              // [KVH, S, D] (kv_head_stride, row stride D)
  const void* v;              // [KVH, S, D]
  const void* mask;           // additive mask element (t, s) at t*mask_row_stride + s*mask_col_stride, or null
  void* out;                  // [T, H, D]: element (t, h, d) at t*H*D + h*D + d
  long long T;
  long long S;
  long long q_head_stride;
  long long kv_head_stride;
  long long mask_row_stride;
  long long mask_col_stride;
  int H;
  int KVH;
  float scale;
  int mask_dtype;             // -1: no mask
  int add_dtype;              // rounding dtype of (scores + mask)
  int dtype;                  // bf16 or fp16
  const int* blk_limit;       // per 32-query block: position blocks to visit (k_mask_extent), or null: all
};

struct ReduceNormArgs {       // split-K reduce + residual, then RMSNorm of the result (gemm.hip)
  const float* part;          // fp32 partial sums [ksplit, M, N]
  const void* bias;           // [N] or null (flags & 1)
  const void* resid;          // [M, N] (row stride ldr)
  void* out;                  // [M, N] (row stride ldo): round(resid + round(sum_z part + bias))
  const void* norm_w;         // [N], the dtype of out
  void* norm_out;             // [M, N] (row stride ldn): norm_w * round_n(out * rsqrt(mean(out^2) + eps))
  long long M;
  long long ldr;
  long long ldo;
  long long ldn;
  int N;                      // N % 8 == 0, N <= 2048, 16-byte aligned rows; grid = M workgroups
  int ksplit;
  float eps;
  int n_dtype;                // rounding dtype of the normalised value
  int flags;
};

struct MaskExtentArgs {       // k_mask_extent: last open mask column of each block of 32 query rows
  const void* mask;           // element (t, s) at t*row_stride + s*col_stride
  int* nblk_out;              // [ceil(T / 32)]: 1 + (last column != -inf) / 32, 0 when none
  long long T;
  long long S;
  long long row_stride;
  long long col_stride;       // 1 for 16-bit masks (8-byte aligned rows, S % 4 == 0); any for fp32
  int mask_dtype;             // HS_BF16 / HS_F16 / HS_F32
};

struct CombineArgs {          // out[h, d] = round(sum_t e^(m_t - M) l_t o_t[d] / sum_t e^(m_t - M) l_t), o_t normalised
  const uint16_t* part_o;     // bf16 [KVH, nsplit, G, D]
  const float* part_ml;
  void* out;                  // [H, D]
  int H;
  int KVH;
  int nsplit;
  int dtype;
};

struct AttnOutArgs {          // second attention pass: global softmax and p.V per 8-dim slice
  const float* scores;        // [H, S] s2 from k_attn_scores (-inf where masked)
  const float* stats;         // [H, ntiles, 2] tile (max, sum exp)
  const void* v;              // [KVH, S, D]
  const void* mask;           // unused by the kernel; kept for symmetry with DecodeAttnArgs
  void* out;                  // [H, D]
  long long S;
  long long kv_head_stride;
  long long mask_stride;
  int H;
  int KVH;
  int ntiles;
  int mask_dtype;
  int dtype;
  int C;                      // channels-last kernels (_nhwc): C (multiple of 8); unused otherwise
};

// host and device (the rotary sincos below is also built into a host test helper)
#ifdef __HIPCC__
#define HS_HD __host__ __device__
#else
#define HS_HD
#endif

// sin and cos of an fp32 angle (|x| < 2^30), branch-free and table-free so that no load or
// wait enters the caller's critical path: Cody-Waite reduction by pi/2 in double (k*pi/2 with
// a two-part pi/2), Taylor polynomials in double on |r| <= pi/4 (truncation error < 1e-17),
// quadrant by selects, then one rounding to fp32.
HS_HD inline void sincos_rot(float xf, float* s_out, float* c_out) {
  const double x = (double)xf;
  const double q = __builtin_rint(x * 0.63661977236758134308);   // 2/pi
  double r = __builtin_fma(-q, 1.57079632679489655800e+00, x);     // pi/2, high part
  r = __builtin_fma(-q, 6.12323399573676603587e-17, r);             // pi/2, low part
  const double r2 = r * r;
  // sin r = r (1 - r2/3! + r2^2/5! - ... - r2^7/15!),  cos r = 1 - r2/2! + ... + r2^8/16!
  double ps = -7.6471637318198164759e-13;                            // -1/15!
  ps = __builtin_fma(ps, r2, 1.6059043836821614599e-10);             //  1/13!
  ps = __builtin_fma(ps, r2, -2.5052108385441718775e-08);            // -1/11!
  ps = __builtin_fma(ps, r2, 2.7557319223985890653e-06);             //  1/9!
  ps = __builtin_fma(ps, r2, -1.9841269841269841270e-04);            // -1/7!
  ps = __builtin_fma(ps, r2, 8.3333333333333333333e-03);             //  1/5!
  ps = __builtin_fma(ps, r2, -1.6666666666666666667e-01);            // -1/3!
  const double sn = __builtin_fma(ps * r2, r, r);
  double pc = 4.7794773323873852974e-14;                             //  1/16!
  pc = __builtin_fma(pc, r2, -1.1470745597729724714e-11);            // -1/14!
  pc = __builtin_fma(pc, r2, 2.0876756987868098979e-09);             //  1/12!
  pc = __builtin_fma(pc, r2, -2.7557319223985890653e-07);            // -1/10!
  pc = __builtin_fma(pc, r2, 2.4801587301587301587e-05);             //  1/8!
  pc = __builtin_fma(pc, r2, -1.3888888888888888889e-03);            // -1/6!
  pc = __builtin_fma(pc, r2, 4.1666666666666666667e-02);             //  1/4!
  pc = __builtin_fma(pc, r2, -0.5);                                  // -1/2!
  const double cs = __builtin_fma(pc, r2, 1.0);
  const int k = (int)((long long)q & 3);   // x = k*pi/2 + r (mod 2 pi)
  const double sv = (k & 1) ? cs : sn, cv = (k & 1) ? sn : cs;
  *s_out = (float)((k & 2) ? -sv : sv);
  *c_out = (float)(((k + 1) & 2) ? -cv : cv);
}

#ifdef __HIPCC__
// ---------------------------------------------------------------- device helpers

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// round to nearest even, NaN -> quiet NaN with the top payload bits: one v_cvt_pk_bf16_f32 on
// gfx950 (checked against the integer formulation (u + 0x7fff + lsb) >> 16, NaN -> (u >> 16) |
// 0x40, on all 2^32 inputs: identical), no branch
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// value of element i of a typed buffer, as float
__device__ __forceinline__ float ld_f(const void* p, long long i, int dt) {
  switch (dt) {
    case HS_F32: return ((const float*)p)[i];
    case HS_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    case HS_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case HS_I64: return (float)((const long long*)p)[i];
    case HS_I32: return (float)((const int*)p)[i];
    case HS_U8: return (float)((const unsigned char*)p)[i];
    case HS_F64: return (float)((const double*)p)[i];
  }
  return 0.f;
}

__device__ __forceinline__ long long ld_i(const void* p, long long i, int dt) {
  switch (dt) {
    case HS_I64: return ((const long long*)p)[i];
    case HS_I32: return ((const int*)p)[i];
    case HS_U8: return ((const unsigned char*)p)[i];
    case HS_F32: return (long long)((const float*)p)[i];
  }
  return 0;
}

// Branch-free loads for values needed late in a kernel: the raw words are loaded with no
// dtype switch (so no wait follows the load) and decoded where the value is used.
// Integer element i of an int64 or int32 tensor: two 32-bit words (int64: its halves;
// int32: the element's word twice).
struct IRaw {
  uint32_t lo, hi;
};
__device__ __forceinline__ IRaw ld_i_raw(const void* p, long long i, int dt) {
  const bool wide = dt == HS_I64;
  const uint32_t* w = (const uint32_t*)((const char*)p + i * (wide ? 8 : 4));
  return IRaw{w[0], w[wide ? 1 : 0]};
}
__device__ __forceinline__ long long ld_i_decode(IRaw r, int dt) {
  return dt == HS_I64 ? (long long)(((unsigned long long)r.hi << 32) | r.lo) : (long long)(int)r.lo;
}
// Float element i of an fp32, fp16 or bf16 tensor: two 16-bit halves (fp32: low and high
// half; 16-bit types: the element twice).
struct FRaw {
  uint16_t lo, hi;
};
__device__ __forceinline__ FRaw ld_f_raw(const void* p, long long i, int dt) {
  const bool wide = dt == HS_F32;
  const uint16_t* h = (const uint16_t*)((const char*)p + i * (wide ? 4 : 2));
  return FRaw{h[0], h[wide ? 1 : 0]};
}
__device__ __forceinline__ float ld_f_decode(FRaw r, int dt) {
  if (dt == HS_F32) return __uint_as_float(((uint32_t)r.hi << 16) | r.lo);
  return dt == HS_BF16 ? bf16_to_f32(r.lo) : f16_to_f32(r.lo);
}

// round a float to the storage precision of dt (identity for fp32); both roundings are single
// conversions, so they are computed and selected rather than branched on
__device__ __forceinline__ float round_to(float f, int dt) {
  const float b = bf16_to_f32(f32_to_bf16(f));
  const float h = (float)(_Float16)f;
  return dt == HS_BF16 ? b : (dt == HS_F16 ? h : f);
}

__device__ __forceinline__ void st_f(void* p, long long i, int dt, float f) {
  switch (dt) {
    case HS_F32: ((float*)p)[i] = f; break;
    case HS_F16: ((uint16_t*)p)[i] = f32_to_f16(f); break;
    case HS_BF16: ((uint16_t*)p)[i] = f32_to_bf16(f); break;
    case HS_I64: ((long long*)p)[i] = (long long)f; break;
    case HS_I32: ((int*)p)[i] = (int)f; break;
    case HS_U8: ((unsigned char*)p)[i] = (unsigned char)(f != 0.f); break;
    case HS_F64: ((double*)p)[i] = (double)f; break;
  }
}

// Eight consecutive float-typed elements from element i (16-byte aligned for 16-bit dtypes, 32-byte
// for fp32): one or two 16-byte loads. ld1x8_f repeats element i eight times (an operand broadcast
// along the last dimension). st8_f writes eight values from element i with 16-byte stores.
__device__ __forceinline__ void ld8_f(const void* p, long long i, int dt, float* v) {
  if (dt == HS_F32) {
    const float4 a = ((const float4*)p)[i >> 2], b = ((const float4*)p)[(i >> 2) + 1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    return;
  }
  const uint4 q = ((const uint4*)p)[i >> 3];
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
    v[2 * j] = dt == HS_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
    v[2 * j + 1] = dt == HS_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
  }
}
__device__ __forceinline__ void ld1x8_f(const void* p, long long i, int dt, float* v) {
  const float x = ld_f(p, i, dt);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = x;
}
__device__ __forceinline__ void st8_f(void* p, long long i, int dt, const float* v) {
  if (dt == HS_F32) {
    ((float4*)p)[i >> 2] = make_float4(v[0], v[1], v[2], v[3]);
    ((float4*)p)[(i >> 2) + 1] = make_float4(v[4], v[5], v[6], v[7]);
    return;
  }
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t lo = dt == HS_BF16 ? f32_to_bf16(v[2 * j]) : f32_to_f16(v[2 * j]);
    const uint16_t hi = dt == HS_BF16 ? f32_to_bf16(v[2 * j + 1]) : f32_to_f16(v[2 * j + 1]);
    w[j] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  ((uint4*)p)[i >> 3] = make_uint4(w[0], w[1], w[2], w[3]);
}

// Cross-lane moves without LDS: DPP (quad permutes, rotations within a row of 16 lanes)
// and readlane. They need every lane of the wave active, which holds at every call site.
#define HS_DPP(v, ctrl) \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), 0xf, 0xf, false))
#define HS_RL(v, l) __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, (v)), (l)))
#define HS_QUAD_XOR1 0xB1
#define HS_QUAD_XOR2 0x4E
#define HS_ROW_ROR4 0x124
#define HS_ROW_ROR8 0x128
#define HS_ROW_ROR12 0x12C   // row_ror:n moves lane j's value to lane j + n (mod 16)

// sum / max over the 64 lanes of a wave; every lane gets the result
__device__ __forceinline__ float wave_sum(float v) {
  v += HS_DPP(v, HS_QUAD_XOR1);
  v += HS_DPP(v, HS_QUAD_XOR2);
  v += HS_DPP(v, HS_ROW_ROR4);
  v += HS_DPP(v, HS_ROW_ROR8);
  return (HS_RL(v, 0) + HS_RL(v, 16)) + (HS_RL(v, 32) + HS_RL(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, HS_DPP(v, HS_QUAD_XOR1));
  v = fmaxf(v, HS_DPP(v, HS_QUAD_XOR2));
  v = fmaxf(v, HS_DPP(v, HS_ROW_ROR4));
  v = fmaxf(v, HS_DPP(v, HS_ROW_ROR8));
  return fmaxf(fmaxf(HS_RL(v, 0), HS_RL(v, 16)), fmaxf(HS_RL(v, 32), HS_RL(v, 48)));
}

#define HS_ROW_MIRROR 0x140        // lane j of a row of 16 reads lane 15 - j
#define HS_ROW_HALF_MIRROR 0x141   // lane j of a half-row of 8 reads lane 7 - j

// Sums of several values over the 64 lanes at once, halving the values each step (each lane
// keeps one value of every exchanged pair and receives its partner's other one): 8 or 16
// values cost about as much as two or three single wave_sum calls. gfx950's permlane32 / 16
// swaps exchange the upper 32 lanes of one value with the lower 32 of another (odd rows of 16
// with even rows, for the 16-lane form), so one swap and one add halve two values.
__device__ __forceinline__ void hs_swap_add(float a, float b, bool rows16, float& out) {
  const unsigned ua = __builtin_bit_cast(unsigned, a), ub = __builtin_bit_cast(unsigned, b);
  if (rows16) {
    const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
    out = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
    out = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  }
}

// v[0..15] per lane -> in lane l, the total over the wave of value
// ((l >> 5) & 1) * 8 + ((l >> 4) & 1) * 4 + ((l >> 3) & 1) * 2 + ((l >> 2) & 1)
// (lane 8 s + 4 holds value 2 s + 1, lane 8 s value 2 s; the 4 lanes of a quad agree)
__device__ __forceinline__ float wave_sum16(const float (&v)[16], int lane) {
  float w[8], x[4], y[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) hs_swap_add(v[i], v[i + 8], false, w[i]);   // value bit 3 = lane bit 5
#pragma unroll
  for (int i = 0; i < 4; ++i) hs_swap_add(w[i], w[i + 4], true, x[i]);    // value bit 2 = lane bit 4
  const bool b3 = (lane & 8) != 0, b2 = (lane & 4) != 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)   // value bit 1 = lane bit 3 (lane j pairs with 15 - j)
    y[i] = (b3 ? x[i + 2] : x[i]) + HS_DPP(b3 ? x[i] : x[i + 2], HS_ROW_MIRROR);
  float z = (b2 ? y[1] : y[0]) + HS_DPP(b2 ? y[0] : y[1], HS_ROW_HALF_MIRROR);   // value bit 0 = lane bit 2
  z += HS_DPP(z, HS_QUAD_XOR2);
  z += HS_DPP(z, HS_QUAD_XOR1);
  return z;
}

// v[0..7] per lane -> in lane l, the total over the wave of value
// ((l >> 5) & 1) * 4 + ((l >> 4) & 1) * 2 + ((l >> 3) & 1) (every lane of an 8-lane group agrees)
__device__ __forceinline__ float wave_sum8(const float (&v)[8], int lane) {
  float w[4], x[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) hs_swap_add(v[i], v[i + 4], false, w[i]);
#pragma unroll
  for (int i = 0; i < 2; ++i) hs_swap_add(w[i], w[i + 2], true, x[i]);
  const bool b3 = (lane & 8) != 0;
  float z = (b3 ? x[1] : x[0]) + HS_DPP(b3 ? x[0] : x[1], HS_ROW_MIRROR);
  z += HS_DPP(z, HS_ROW_HALF_MIRROR);
  z += HS_DPP(z, HS_QUAD_XOR2);
  z += HS_DPP(z, HS_QUAD_XOR1);
  return z;
}

// ---------------------------------------------------------------- argmax over long rows
//
// argmax_part_body: workgroup (part, row) of 256 threads scans columns [part * seg, (part + 1) * seg)
// of row `row` with 16-byte loads (all of a thread's loads of a pass in flight together) and
// writes one key to slot[row * parts + part]; argmax_finalize_body: one workgroup per row takes
// the largest of its `parts` keys. The key orders like torch.argmax / np.argmax: larger value
// first, NaN above every number, -0.0 equal to +0.0, then the smaller index.
__device__ __forceinline__ unsigned long long argmax_key_nan(float v, unsigned idx) {
  uint32_t b = __float_as_uint(v);
  b = (v == 0.f) ? 0u : b;
  const uint32_t o = (v != v) ? 0xFFFFFFFFu : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
  return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ void argmax_part_body(const ArgmaxPartArgs& a, long long part, long long row) {
  __shared__ unsigned long long red[4];
  const long long c0 = part * a.seg, c1 = min(c0 + a.seg, a.cols);
  const uint16_t* xr = (const uint16_t*)a.x + row * a.cols;
  const bool f16 = a.x_dtype == HS_F16;
  unsigned long long best = 0ull;
  constexpr int U = 4;
  for (long long c = c0 + threadIdx.x * 8; c < c1; c += 256 * 8 * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long cc = c + (long long)u * 256 * 8;
      v[u] = cc < c1 ? *(const uint4*)(xr + cc) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long cc = c + (long long)u * 256 * 8;
      if (cc >= c1) break;
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint16_t hbits = (j & 1) ? (uint16_t)(w[j >> 1] >> 16) : (uint16_t)(w[j >> 1] & 0xffffu);
        const float f = f16 ? f16_to_f32(hbits) : bf16_to_f32(hbits);
        const unsigned long long k = argmax_key_nan(f, (unsigned)(cc + j));
        best = k > best ? k : best;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long other = __shfl_xor(best, o, 64);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = red[0];
    for (int w = 1; w < 4; ++w) k = red[w] > k ? red[w] : k;
    a.slot[row * a.parts + part] = k;
  }
}

__device__ __forceinline__ void argmax_finalize_body(const ArgmaxFinalizeArgs& a, long long m) {
  __shared__ unsigned long long red[256];
  if (m >= a.rows) return;
  unsigned long long k = 0ull;
  for (int i = threadIdx.x; i < a.parts; i += 256) {
    const unsigned long long v = a.slot[m * a.parts + i];
    k = v > k ? v : k;
  }
  red[threadIdx.x] = k;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o && red[threadIdx.x + o] > red[threadIdx.x]) red[threadIdx.x] = red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const long long idx = (long long)(0xFFFFFFFFu - (uint32_t)(red[0] & 0xFFFFFFFFull));
    if (a.out_dtype == HS_I64) ((long long*)a.out)[m] = idx;
    else ((int*)a.out)[m] = (int)idx;
  }
}

// sum over a 256-thread workgroup; every thread gets the result
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float block_max256(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
#endif
