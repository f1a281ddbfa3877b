// Shared device helpers of the MI355X (gfx950 / CDNA4) AWQ W4A16 kernels.
//
// Reference behaviour followed (paths relative to the jiayingsong2023/litevLLM checkout):
//   dequant value  (q - z) * s rounded once   vllm/model_executor/layers/quantization/tensor.py:857-858,
//                                             vllm/kernels/triton/awq_fused_gemm.py:1966, 1976
//   fp32 accumulation, one output rounding,   awq_fused_gemm.py:1969-1990
//   bias added in fp32 before that rounding
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "awq_w4a16.h"

namespace awq {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ constexpr uint32_t cdiv_u(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// Column offset held by nibble i of a packed word.
template <bool SEQ>
__host__ __device__ constexpr int nib_col(int i) {
  return SEQ ? i : (i < 4 ? 2 * i : 2 * (i - 4) + 1);  // AutoAWQ order {0,2,4,6,1,3,5,7}
}
// Nibble holding column offset c (inverse of nib_col).
template <bool SEQ>
__host__ __device__ constexpr int col_nib(int c) {
  return SEQ ? c : ((c & 1) ? 4 + (c >> 1) : (c >> 1));
}
static_assert(nib_col<false>(1) == 2 && nib_col<false>(4) == 1 && nib_col<false>(7) == 7, "AWQ order");
static_assert(col_nib<false>(nib_col<false>(3)) == 3 && col_nib<false>(nib_col<false>(6)) == 6, "inverse");

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

__device__ __forceinline__ uint16_t f2h_bits(float x) { return __builtin_bit_cast(uint16_t, (f16)x); }
__device__ __forceinline__ uint16_t f2bf_bits(float x) { return __builtin_bit_cast(uint16_t, (bf16)x); }
__device__ __forceinline__ float h_bits2f(uint16_t b) { return (float)__builtin_bit_cast(f16, b); }
__device__ __forceinline__ float bf_bits2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

template <typename T>
__device__ __forceinline__ uint16_t to_bits(float x) {
  if constexpr (std::is_same<T, f16>::value) return f2h_bits(x);
  else return f2bf_bits(x);
}
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)to_bits<T>(lo) | ((uint32_t)to_bits<T>(hi) << 16);
}
template <typename T>
__device__ __forceinline__ float from_bits(uint16_t b) {
  if constexpr (std::is_same<T, f16>::value) return h_bits2f(b);
  else return bf_bits2f(b);
}

// Magic-exponent int4 -> fp16 conversion.  For a 32-bit word m whose two 16-bit halves
// each hold four nibbles, nibble position P (0..3) of both halves becomes an f16x2:
//   P even: (bits & 0x000F000F) | 0x6400  ->  1024 + q  (nibble in mantissa bits 0-3)
//   P odd : (bits & 0x00F000F0) | 0x5400  ->    64 + q  (nibble in mantissa bits 4-7,
//                                                          exponent of 64 has ulp 1/16)
// P >= 2 first shifts the word right by 8.  Both forms are exact.
// The masks and magic exponents live in VGPRs (MagicK) so that each nibble pair costs a
// single v_and_or_b32: gfx9 VOP3 encodings cannot carry 32-bit literals, and with literal
// operands the compiler splits the operation into v_and_b32 + v_or_b32.
struct MagicK {
  uint32_t lo_mask, hi_mask, lo_magic, hi_magic;
};
__device__ __forceinline__ MagicK magic_consts() {
  MagicK k{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  asm volatile("" : "+v"(k.lo_mask), "+v"(k.hi_mask), "+v"(k.lo_magic), "+v"(k.hi_magic));
  return k;
}
// The same with the magic exponents in SGPRs (a VOP3 operation may read one SGPR), for
// kernels short of VGPRs.
__device__ __forceinline__ MagicK magic_consts_s() {
  MagicK k{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  asm volatile("" : "+v"(k.lo_mask), "+v"(k.hi_mask), "+s"(k.lo_magic), "+s"(k.hi_magic));
  return k;
}
template <int P>
__device__ __forceinline__ uint32_t magic_bits(uint32_t m, const MagicK& k) {
  const uint32_t v = (P >= 2) ? (m >> 8) : m;
  return (P & 1) ? ((v & k.hi_mask) | k.hi_magic) : ((v & k.lo_mask) | k.lo_magic);
}
// Zero operand matching magic_bits<P>: the same bias plus z, broadcast to both halves.
__device__ __forceinline__ uint32_t zero_magic(int p_odd, uint32_t z) {
  const uint32_t h = p_odd ? (0x5400u | (z << 4)) : (0x6400u | z);
  return h * 0x00010001u;
}

// Per-column dequant constants for one group.
//  FAST (f16 activations and f16 scales): zm = biased zero, sc = scale, both broadcast f16x2;
//  W = (magic - zm) * sc -- the subtraction is exact, the multiply rounds once.
//  otherwise: zm as above, scf = fp32 scale; W = T(float(magic - zm) * scf), exact product,
//  one rounding to T.
struct ColConst {
  uint32_t zm;
  uint32_t sc;   // f16x2 bits (FAST)
  float scf;     // fp32 scale (generic)
};

// Two dequantized values (two K-adjacent rows of one column) as 32 bits of T.
template <bool FAST, typename T>
__device__ __forceinline__ uint32_t deq2(uint32_t magic, const ColConst& cc) {
  const f16x2 d = as_h2(magic) - as_h2(cc.zm);  // exact small integers
  if constexpr (FAST) {
    return as_u(d * as_h2(cc.sc));
  } else {
    return pack2<T>((float)d.x * cc.scf, (float)d.y * cc.scf);
  }
}

template <typename T> struct MfmaOp;
template <> struct MfmaOp<f16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct MfmaOp<bf16> {
  static __device__ __forceinline__ f32x4 run(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ float load_bias(const void* bias, int dtype, int col) {
  if (dtype == AWQ_DTYPE_F16) return h_bits2f(((const uint16_t*)bias)[col]);
  if (dtype == AWQ_DTYPE_BF16) return bf_bits2f(((const uint16_t*)bias)[col]);
  if (dtype == AWQ_DTYPE_F32) return ((const float*)bias)[col];
  return 0.0f;
}

// act(g) of the reference's gated MLP kernels (awq_fused_gemm.py:1493-1502,
// gemma4_moe_int4.py:748-756): kind 1 is GELU in its tanh form written as
// g * sigmoid(2 * inner), 0.5 * (1 + tanh(y)) == sigmoid(2y); otherwise SiLU.
__device__ __forceinline__ float gated_act(float g, int kind) {
  if (kind == 1) {
    const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return g / (1.0f + expf(-2.0f * inner));
  }
  return g / (1.0f + expf(-g));
}
// The same activations from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: about
// one ulp each), for epilogues whose result is rounded to fp16 / bf16 right after: the fp32
// error (a few 1e-7 relative) is far below that rounding.  KIND is the compile-time kind.
template <int KIND>
__device__ __forceinline__ float gated_act_fast(float g) {
  constexpr float kLog2e = 1.4426950408889634f;
  float t = g;
  if constexpr (KIND == 1) t = 2.0f * 0.7978845608028654f * (g + 0.044715f * g * g * g);
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-t * kLog2e));
}

// Shared argument block of the GEMM kernels.
// The fp32 value as computed (rounded to fp32): the empty asm keeps the compiler from fusing
// the operation that produced it into a following fp16 conversion (a multiply and the
// conversion become one mixed-precision FMA that rounds once, not twice).
__device__ __forceinline__ float fp32_rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Sum of an fp64 value over the 64 lanes of a wave, returned in every lane: DPP steps within
// quads, half rows, rows, then the row broadcasts (both 32-bit halves moved together), and
// lane 63's total read out.  Lanes disabled by a step's row mask add zero.
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROWS, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROWS, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<0xB1, 0xF>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f64<0x4E, 0xF>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f64<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_f64<0x140, 0xF>(v);  // row_mirror
  v += dpp_f64<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f64<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum of an int over the 64 lanes of a wave, with no LDS traffic: shifts
// right by 1, 2, 4 and 8 lanes inside each row of 16 (lanes whose source lies before the row
// add zero), then the row broadcasts of lanes 15 and 31.
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
  return v;
}

// 1 / sqrt(var / K + eps) of the RMSNorm prologue: var / K + eps in fp32 as the reference
// computes it (rmsnorm_awq_fused.py:118), the reciprocal square root correctly rounded (fp64
// square root and division, rounded once to fp32).
__device__ __forceinline__ float rms_scale(float var, int K, float eps) {
  const float v = var / (float)K + eps;
  return (float)(1.0 / sqrt((double)v));
}

struct GemmArgs {
  const uint16_t* a;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint32_t* qz;
  const void* bias;
  uint16_t* c;
  float* partial;   // decode: [tiles, max_contrib, M, tile columns] fp32
  int* counters;    // decode: [tiles], zero on entry and on exit
  int64_t lda, ldc;
  int M, N, K, G;
  int bias_dtype;
  // decode only: 0 = plain GEMM; 1 + activation kind = gated epilogue.  Each 128-column tile
  // then holds 64 gate columns and the 64 up columns of the same outputs, and output column
  // 64 t + j (j < 64, below n_out) is act(gate) * up of tile t's columns j and 64 + j.
  int gate_act, n_out;
  // narrow decode kernel only: non-NULL = normalise the staged activation rows first
  // (RMSNorm prologue, fp16 rows; norm_w [K] fp16, or bf16 when norm_bf16)
  const uint16_t* norm_w;
  float eps;
  int norm_bf16;
  // decode kernels only: > 1 = a row-exact launch (awq_w4a16_gemm_rows_exact) of that many grid
  // rows, M = 1: grid row y computes row y of the call as a lone M = 1 call would (row_slice)
  int rows;
  // prefill stream kernel only: > 1 = split K into that many ranges of whole stage pairs, each
  // writing its fp32 sums to partial[split][M][N], summed in split order by a second launch
  int ksplit;
};

// Block coordinates of a stream-kernel decode launch: x = the block of the M = 1 plan (nblocks
// of them), y = the row of a row-exact launch (a 1-D grid of nblocks * rows blocks; other
// launches: (blockIdx.x, 0)).  The rows of one plan block are laid out to be dispatched
// together and, since the hardware deals blocks to the 8 XCDs round robin, on the same XCD:
// they read the same weight bytes, which that XCD's L2 serves to all but the first.  M = 4,
// N = 24576: 31.5 -> 24.3 us; N = 14336: 46.2 -> 39.3 us, against a 2-D grid (x, rows)
// dispatched row after row (A/B on one box).  The narrow kernel keeps that 2-D grid: its
// weights sit in the MALL, and the grouped order measured 5% slower there (M = 4, N = 4096).
struct BlockXY {
  int x, y;
};
__device__ __forceinline__ BlockXY decode_block(int rows, int nblocks) {
  const int b = (int)blockIdx.x;
  if (rows <= 1) return {b, 0};
  if ((nblocks & 7) == 0) {
    const int xcd = b & 7, i = b >> 3;
    return {(i / rows) * 8 + xcd, i % rows};
  }
  return {b % nblocks, b / nblocks};
}

// The M = 1 problem of row y of a row-exact launch: activation row y, output row y and, with
// split-K, the y-th set of `tiles` arrival counters and `parts` fp32 partial floats.  Row 0
// (every other launch) is the call itself.  Every other argument and the whole computation
// are those of the M = 1 call, so each row's bits equal a lone call's.
__device__ __forceinline__ GemmArgs row_slice(const GemmArgs& p, int tiles, int parts, int y) {
  GemmArgs q = p;
  q.a += (int64_t)y * p.lda;
  q.c += (int64_t)y * p.ldc;
  if (p.counters) {  // split-K workspace present
    q.counters += y * tiles;
    q.partial += (int64_t)y * parts;
  }
  return q;
}

// Work decomposition of the decode kernel: tiles x ksteps units; each tile's k-steps are cut
// into `splits` ranges of `per` k-steps (the last ones shorter or empty), one block each
// (block b: tile b / splits, range b % splits).
struct DecodeWork {
  int tiles, ksteps, splits, per;
};

// Raw per-group constants of one packed word: 8 scales (16 bytes) and the zero word.
struct WordSZ {
  u32x4 s4;
  uint32_t zw;
};

// Per-column dequant constants of the 8 nibbles of a word.
template <bool SEQ, bool FAST>
__device__ __forceinline__ void prep_consts(const WordSZ& sz, bool scale_bf16, ColConst (&cc)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = nib_col<SEQ>(i);
    const uint32_t sbits = (sz.s4[c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
    cc[i].zm = zero_magic(i & 1, (sz.zw >> (4 * i)) & 0xF);
    if constexpr (FAST) {
      cc[i].sc = sbits * 0x00010001u;
      cc[i].scf = 0.0f;
    } else {
      cc[i].sc = 0;
      cc[i].scf = scale_bf16 ? bf_bits2f((uint16_t)sbits) : h_bits2f((uint16_t)sbits);
    }
  }
}

// Constants of nibble I alone (as prep_consts computes them for all eight).
template <int I, bool SEQ, bool FAST>
__device__ __forceinline__ ColConst prep_const(const WordSZ& sz, bool scale_bf16) {
  constexpr int c = nib_col<SEQ>(I);
  const uint32_t sbits = (sz.s4[c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
  ColConst cc;
  cc.zm = zero_magic(I & 1, (sz.zw >> (4 * I)) & 0xF);
  if constexpr (FAST) {
    cc.sc = sbits * 0x00010001u;
    cc.scf = 0.0f;
  } else {
    cc.sc = 0;
    cc.scf = scale_bf16 ? bf_bits2f((uint16_t)sbits) : h_bits2f((uint16_t)sbits);
  }
  return cc;
}

// Decode constants of nibble i: the biased zero and the fp32 scale (the decode kernel feeds
// the MFMA the integers q - z and scales each group's sum).
template <bool SEQ, bool SBF>
__device__ __forceinline__ ColConst prep_const_int(const WordSZ& sz, int i) {
  const int c = nib_col<SEQ>(i);
  const uint32_t sbits = (sz.s4[c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
  ColConst cc;
  cc.zm = zero_magic(i & 1, (sz.zw >> (4 * i)) & 0xF);
  cc.sc = 0;
  cc.scf = SBF ? bf_bits2f((uint16_t)sbits) : h_bits2f((uint16_t)sbits);
  return cc;
}

// Row pairing with one byte permute: lo16(w0) | lo16(w1) << 16 and hi16(w0) | hi16(w1) << 16.
// (v_perm_b32 selects bytes 0-3 from its second operand and 4-7 from its first.)
__device__ __forceinline__ uint32_t pair_lo(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x05040100u);
}
__device__ __forceinline__ uint32_t pair_hi(uint32_t w0, uint32_t w1) {
  return __builtin_amdgcn_perm(w1, w0, 0x07060302u);
}

// Eight rows (k .. k+7) of one packed word, pre-paired into lo/hi words, -> MFMA operand
// (8 K-consecutive values of the column held by nibble I).
template <int I, bool FAST, typename T>
__device__ __forceinline__ u32x4 rows_operand(const uint32_t (&mlo)[4], const uint32_t (&mhi)[4],
                                              const ColConst& cc, const MagicK& k) {
  u32x4 r;
#pragma unroll
  for (int u = 0; u < 4; ++u) r[u] = deq2<FAST, T>(magic_bits<I & 3>(I < 4 ? mlo[u] : mhi[u], k), cc);
  return r;
}

// Eight rows (k .. k+7) of nibble I as the exact integers q - z in T: the subtraction of the
// biased zero is exact in fp16, and integers up to 15 in magnitude are exact in bf16.
template <int I, typename T>
__device__ __forceinline__ u32x4 int_operand(const uint32_t (&mlo)[4], const uint32_t (&mhi)[4], uint32_t zm,
                                             const MagicK& k) {
  u32x4 r;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const f16x2 d = as_h2(magic_bits<I & 3>(I < 4 ? mlo[u] : mhi[u], k)) - as_h2(zm);
    if constexpr (std::is_same<T, f16>::value) r[u] = as_u(d);
    else r[u] = pack2<bf16>((float)d.x, (float)d.y);
  }
  return r;
}

// Biased-integer MFMA operands of the decode kernels: eight rows (k .. k+7) of nibble I as
// exact values in T whose activation-weighted sums a kernel turns back into sum x (q - z)
// when it scales the group (biased_terms), using the group's activation sum, i.e. the same
// MFMA against ones:
//  * fp16 (exponent 6, 64 + mantissa / 16): nibbles P = 0, 1 of each 16-bit half are
//    masked into mantissa bits 4-7 (P = 0 after a 4-bit shift) and read 64 + q_P; nibbles
//    P = 2, 3 are moved there whole with their neighbour by one byte permute and read
//    64 + q_P + q_{P-1} / 16 -- one shift per word, one AND-OR or permute per pair of rows;
//  * bf16 (exponent 7, 128 + mantissa): nibble P shifted to bits 0-3 and masked, 128 + q_P.
// Small biases keep the fp32 sums' cancellation small (a bias of 1024, fp16 with the nibble
// at bits 0-3, costs up to 2 fp16 ulps on all-positive activations; 64 stays within the
// final rounding's half ulp).
struct BiasK {
  uint32_t mask, magic;
};
template <typename T>
__device__ __forceinline__ BiasK bias_consts() {
  BiasK k = std::is_same<T, f16>::value ? BiasK{0x00F000F0u, 0x54005400u} : BiasK{0x000F000Fu, 0x43004300u};
  asm volatile("" : "+v"(k.mask), "+v"(k.magic));  // VGPR operands (one constant-bus slot per VOP3)
  return k;
}
// 1.0 in both halves: the operand whose MFMA yields the activation sums
template <typename T>
__host__ __device__ constexpr uint32_t ones2() {
  return std::is_same<T, f16>::value ? 0x3C003C00u : 0x3F803F80u;
}
template <int I, typename T>
__device__ __forceinline__ u32x4 biased_operand(const uint32_t (&mlo)[4], const uint32_t (&mhi)[4], const BiasK& k) {
  constexpr int P = I & 3;
  u32x4 r;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t m = I < 4 ? mlo[u] : mhi[u];
    if constexpr (std::is_same<T, f16>::value) {
      const uint32_t w = (P == 0 || P == 2) ? (m << 4) : m;
      // P 2, 3: bytes 1 and 3 (the nibble and its lower neighbour) under the magic's high bytes
      r[u] = (P < 2) ? ((w & k.mask) | k.magic) : __builtin_amdgcn_perm(k.magic, w, 0x07030501u);
    } else {
      r[u] = ((m >> (4 * P)) & k.mask) | k.magic;
    }
  }
  return r;
}
// (bias + z) of nibble i of a zero word as fp32, built from its bits: 64 + z = 2^6 (1 + z/64),
// 128 + z = 2^7 (1 + z/128) (a bit-field extract and a shift-or, no conversion)
template <typename T>
__device__ __forceinline__ float biased_zero(uint32_t zw, int i) {
  const uint32_t z = (zw >> (4 * i)) & 0xFu;
  return std::is_same<T, f16>::value ? __builtin_bit_cast(float, 0x42800000u | (z << 17))
                                     : __builtin_bit_cast(float, 0x43000000u | (z << 16));
}
static_assert(__builtin_bit_cast(float, 0x42800000u | (15u << 17)) == 79.0f, "64 + 15");
static_assert(__builtin_bit_cast(float, 0x43000000u | (15u << 16)) == 143.0f, "128 + 15");
// Per-group coefficients that turn the biased sums of one 16-bit half (nibbles P = 0..3 at
// columns i0 + P) into the scaled sums s_P * sum x (q_P - z_P):
//   fp16: P 0, 1:  s acc_P - s (64 + z) ax
//         P 2:     s (acc_2 - acc_1 / 16) - s (60 + z) ax
//         P 3:     s (acc_3 - (acc_2 - acc_1 / 16) / 16) - s (60.25 + z) ax
//   bf16: every P: s acc_P - s (128 + z) ax
struct HalfCoef {
  float s[4], cz[4];
};
template <typename T>
__device__ __forceinline__ HalfCoef half_coef(const float (&s)[4], uint32_t zw, int i0) {
  HalfCoef h;
#pragma unroll
  for (int P = 0; P < 4; ++P) {
    float b = biased_zero<T>(zw, i0 + P);
    if constexpr (std::is_same<T, f16>::value) b -= (P == 2) ? 4.0f : (P == 3) ? 3.75f : 0.0f;
    h.s[P] = s[P];
    h.cz[P] = b * s[P];
  }
  return h;
}
// tot_P += the scaled sum of nibble P, all fused multiply-adds (the chain terms are taken off
// the raw sums first: t2 = acc_2 - acc_1 / 16, t3 = acc_3 - t2 / 16, which leaves biases
// 60 and 60.25 on them)
template <typename T>
__device__ __forceinline__ void biased_terms(float (&tot)[4], const float (&acc)[4], float ax, const HalfCoef& h) {
  float a[4] = {acc[0], acc[1], acc[2], acc[3]};
  if constexpr (std::is_same<T, f16>::value) {
    a[2] = __builtin_fmaf(-0.0625f, a[1], a[2]);
    a[3] = __builtin_fmaf(-0.0625f, a[2], a[3]);
  }
#pragma unroll
  for (int P = 0; P < 4; ++P) tot[P] = __builtin_fmaf(-h.cz[P], ax, __builtin_fmaf(a[P], h.s[P], tot[P]));
}
template <typename T>
__device__ __forceinline__ void biased_terms(f32x4 (&tot)[4], const f32x4 (&acc)[4], const f32x4& ax, const HalfCoef& h) {
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float t[4] = {tot[0][v], tot[1][v], tot[2][v], tot[3][v]};
    const float a[4] = {acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
    biased_terms<T>(t, a, ax[v], h);
#pragma unroll
    for (int P = 0; P < 4; ++P) tot[P][v] = t[P];
  }
}

// tot[i][mt] += the scaled sums of a group (AutoAWQ nibble order) from its biased sums acc,
// activation sums ax, raw scales s4 and zero word zw
template <typename T, bool SBF, int MT>
__device__ __forceinline__ void flush_biased(f32x4 (&tot)[8][MT], const f32x4 (&acc)[8][MT], const f32x4 (&ax)[MT],
                                             const u32x4& s4, uint32_t zw) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float sc[4];
#pragma unroll
    for (int P = 0; P < 4; ++P) {
      const int c = nib_col<false>(4 * h + P);
      const uint16_t sb = (uint16_t)(s4[c >> 1] >> (16 * (c & 1)));
      sc[P] = SBF ? bf_bits2f(sb) : h_bits2f(sb);
    }
    const HalfCoef hc = half_coef<T>(sc, zw, 4 * h);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 tv[4] = {tot[4 * h][mt], tot[4 * h + 1][mt], tot[4 * h + 2][mt], tot[4 * h + 3][mt]};
      const f32x4 av[4] = {acc[4 * h][mt], acc[4 * h + 1][mt], acc[4 * h + 2][mt], acc[4 * h + 3][mt]};
      biased_terms<T>(tv, av, ax[mt], hc);
#pragma unroll
      for (int P = 0; P < 4; ++P) tot[4 * h + P][mt] = tv[P];
    }
  }
}

// waits until no vector-memory operation of this wave is outstanding (gfx9 s_waitcnt
// encoding, expcnt and lgkmcnt unconstrained); as an intrinsic the compiler's own wait
// bookkeeping sees it
#define AWQ_WAIT_VMCNT0() __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8))
// the same, leaving at most N (< 64) vector-memory operations of this wave outstanding
#define AWQ_WAIT_VMCNT(N) \
  __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8) | ((N) & 0xF) | ((((N) >> 4) & 0x3) << 14))

// Raw, range-checked buffer descriptor as four SGPR words (for the LDS DMA below).
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t nbytes) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, nbytes, 0x00020000u};
}

// Buffer loads straight into LDS: lane l's 16 (lds_dma16) or 4 (lds_dma4) bytes land at
// lds + 16 l (+ 4 l).  Written as assembly so the compiler does not pair them with unrelated
// LDS reads (it cannot tell LDS buffers apart and would wait for every load in flight before
// each of them); a kernel waits for these loads itself before its barrier.  M0 carries the
// LDS address and nothing else in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const u32x4& rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const u32x4& rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}
// Buffer loads into registers issued as assembly, like the LDS DMA: the compiler does not
// track them, so a kernel waits for them itself (s_waitcnt vmcnt) and then passes every
// destination register through pin_after_wait(), which keeps uses after that wait and keeps
// the register live until then (a load still in flight must not land in a reused register).
__device__ __forceinline__ u32x4 asm_load16(const u32x4& rsrc, uint32_t voff, uint32_t soff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rsrc), "s"(soff) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t asm_load4(const u32x4& rsrc, uint32_t voff) {
  uint32_t v;
  asm volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc) : "memory");
  return v;
}
#pragma clang diagnostic pop
template <typename V>
__device__ __forceinline__ void pin_after_wait(V& v) {
  asm volatile("" : "+v"(v));
}

// Buffer resource over a whole tensor (raw addressing, bounds = nbytes).  Range checks
// cover the VGPR offset only (the SGPR offset is excluded), so anything that must read as
// zero past the end has to carry its position in the VGPR offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)nbytes, 0x00020000);
}

// Buffer cache-policy bit nt (non-temporal) for weight streams read exactly once: measured
// 4-6% faster on 50-115 MB decode streams, slower on ~8 MB ones (so the narrow kernel, which
// serves the small shapes, does not set it).
constexpr int kStreamNT = 0x2;
// Buffer cache-policy bits: sc1 = device scope.  Stores with it are visible to every XCD
// once complete; loads with it do not hit lines another XCD's L2 may hold stale.
constexpr int kDeviceCoherent = 0x10;

}  // namespace awq

// Host-side launchers (one per translation unit).
namespace awq_host {
int num_cus();
}
