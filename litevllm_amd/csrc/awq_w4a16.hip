// MI355X (gfx950 / CDNA4) AWQ W4A16 dequant-GEMM kernels behind a C ABI.
//
// Kernels (all hand-written for 64-wide wavefronts and the CDNA4 MFMA
// v_mfma_f32_16x16x32_{f16,bf16}):
//   * dequant_kernel_{kn,nk}  : int4 -> fp16/bf16/fp32 matrix, one packed word per thread.
//   * skinny_kn_kernel        : decode GEMV / skinny GEMM, M <= 32.  Each lane streams its
//                               weight words straight from HBM, row-pairs them with a byte
//                               permute, unpacks nibbles with the 0x6400/0x5400 magic-exponent
//                               trick, dequantizes exactly ((q - z) * s, one rounding) and feeds
//                               the MFMA with the activations as the 16-column operand.  K is split
//                               across the 4 waves of a block (LDS reduction) and across blocks
//                               (fp32 partials + last-arriving-block fixed-order reduction).
//   * gemm_kn_kernel          : prefill GEMM, M > 32.  Activation tiles are staged through LDS
//                               (XOR-swizzled 16-byte chunks, double buffered); each wave dequantizes
//                               its own weight columns in registers straight into MFMA operand layout.
//   * repack_*                : lossless reference-layout -> AutoAWQ-layout conversion.
//
// Reference behaviour followed (paths relative to the jiayingsong2023/litevLLM checkout):
//   dequant value  (q - z) * s rounded once   vllm/model_executor/layers/quantization/tensor.py:857-858,
//                                             vllm/kernels/triton/awq_fused_gemm.py:1966, 1976
//   fp32 accumulation, one output rounding,   awq_fused_gemm.py:1969-1990
//   bias added in fp32 before that rounding
//   contiguous split-K partition              awq_fused_gemm.py:1799-1801
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "awq_w4a16.h"

namespace {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
template <typename ST>
__device__ __forceinline__ float bits2f(uint16_t b) {
  if constexpr (std::is_same<ST, f16>::value) return h_bits2f(b);
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

// Two dequantized values (rows k, k+1 of one column, or two K-adjacent values) as 32 bits of T.
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

// ----------------------------------------------------------------------------------
// Standalone dequant.
// KN layouts: qweight [K, N/8]; thread = one word (k, j) -> out[k, 8j .. 8j+7].
template <bool SEQ, bool ZP, typename ST, int OUT>
__global__ void __launch_bounds__(256) dequant_kn_kernel(const uint32_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint32_t* __restrict__ qz,
                                                         void* __restrict__ out, int64_t K,
                                                         int64_t N, int G) {
  const int64_t NW = N >> 3;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= K * NW) return;
  const int64_t k = idx / NW, j = idx - k * NW;
  const int64_t g = k / G;
  const uint32_t w = qw[idx];
  const uint32_t zw = ZP ? qz[g * NW + j] : 0x88888888u;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = (w >> (4 * i)) & 0xF, z = (zw >> (4 * i)) & 0xF;
    const float s = bits2f<ST>(sc[g * N + 8 * j + nib_col<SEQ>(i)]);
    v[nib_col<SEQ>(i)] = (float)(q - z) * s;  // exact in fp32
  }
  const int64_t o = k * N + 8 * j;
  if constexpr (OUT == AWQ_DTYPE_F32) {
    f32x4* d = (f32x4*)((float*)out + o);
    d[0] = f32x4{v[0], v[1], v[2], v[3]};
    d[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    using T = typename std::conditional<OUT == AWQ_DTYPE_F16, f16, bf16>::type;
    u32x4 r;
    r[0] = pack2<T>(v[0], v[1]);
    r[1] = pack2<T>(v[2], v[3]);
    r[2] = pack2<T>(v[4], v[5]);
    r[3] = pack2<T>(v[6], v[7]);
    *(u32x4*)((uint16_t*)out + o) = r;
  }
}

// NK layout: qweight [N, K/8]; thread = one word (n, kw) -> out[n, 8kw .. 8kw+7].
template <bool ZP, typename ST, int OUT>
__global__ void __launch_bounds__(256) dequant_nk_kernel(const uint32_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint32_t* __restrict__ qz,
                                                         void* __restrict__ out, int64_t N,
                                                         int64_t K, int G) {
  const int64_t KW = K >> 3, NG = K / G, ZW = (NG + 7) >> 3;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= N * KW) return;
  const int64_t n = idx / KW, kw = idx - n * KW;
  const int64_t g = (kw * 8) / G;
  const uint32_t w = qw[idx];
  const int z = ZP ? (int)((qz[n * ZW + (g >> 3)] >> (4 * (g & 7))) & 0xF) : 8;
  const float s = bits2f<ST>(sc[n * NG + g]);
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)((int)((w >> (4 * i)) & 0xF) - z) * s;
  const int64_t o = n * K + 8 * kw;
  if constexpr (OUT == AWQ_DTYPE_F32) {
    f32x4* d = (f32x4*)((float*)out + o);
    d[0] = f32x4{v[0], v[1], v[2], v[3]};
    d[1] = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    using T = typename std::conditional<OUT == AWQ_DTYPE_F16, f16, bf16>::type;
    u32x4 r;
    r[0] = pack2<T>(v[0], v[1]);
    r[1] = pack2<T>(v[2], v[3]);
    r[2] = pack2<T>(v[4], v[5]);
    r[3] = pack2<T>(v[6], v[7]);
    *(u32x4*)((uint16_t*)out + o) = r;
  }
}

// ----------------------------------------------------------------------------------
// Shared argument block of the GEMM kernels.
struct GemmArgs {
  const uint16_t* a;
  const uint32_t* qw;
  const uint16_t* sc;
  const uint32_t* qz;
  const void* bias;
  uint16_t* c;
  float* partial;   // [nsplit, M, N] fp32 (skinny kernel with nsplit > 1)
  int* counters;    // [column tiles]   (zero on entry and on exit)
  int64_t lda, ldc;
  int M, N, K, G;
  int nsplit, steps_per_split;
  int bias_dtype;
};

// Raw per-group constants of one packed word: 8 scales (16 bytes) and the zero word.
struct WordSZ {
  u32x4 s4;
  uint32_t zw;
};

template <bool ZP>
__device__ __forceinline__ WordSZ load_sz(const GemmArgs& p, int g, int word) {
  WordSZ r;
  r.s4 = *(const u32x4*)(p.sc + (int64_t)g * p.N + 8 * word);
  r.zw = ZP ? p.qz[(int64_t)g * (p.N >> 3) + word] : 0x88888888u;
  return r;
}

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

// Buffer resource over a whole tensor (raw addressing, bounds = nbytes, loads past the end
// return zero).  Keeps per-row addresses out of VGPRs: the row offset rides in an SGPR.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)nbytes, 0x00020000);
}

// ----------------------------------------------------------------------------------
// Decode / skinny kernel, KN layouts (qweight [K, N/8]).
//  block = 4 waves, column tile = 16 lanes x WPL words x 8 = 128*WPL columns.
//  lane (q = lane/16, r = lane%16) owns words  tile*16*WPL + r*WPL + w  (w < WPL) and, per
//  32-row k-step, rows 8q .. 8q+7.  For each (w, nibble i) the lane builds one 16x32 MFMA
//  operand (16 weight columns x 32 k) and multiplies it with the activation operand
//  (32 k x 16 tokens), so a wave covers 128*WPL columns x 16*MT tokens.
//
//  Work is cut in whole quantization groups: split s of the grid covers groups
//  [s*I, (s+1)*I), and each of the 4 waves takes a contiguous quarter of those.  A wave's
//  loop handles 4 k-steps per iteration (4/SPG groups, SPG = k-steps per group) with a
//  4-deep register ring: while slot u is computed, the loads for the same slot of the next
//  iteration are already queued, and the group constants of the next iteration are loaded
//  once per group.  The body is straight-line, so the compiler's counter waits let the next
//  iteration's loads run under the current iteration's math.
//
//  Split-K: with nsplit > 1 every block publishes its fp32 partial tile with device-coherent
//  (sc0 sc1) stores, waits for them, and bumps the tile's arrival counter; the block that
//  arrives last reads all partials with device-coherent loads and sums them in split order.
//  No cache-wide writeback/invalidate fence is needed because every byte exchanged between
//  blocks bypasses the non-coherent part of the per-XCD L2.
constexpr int kCoherent = 0x11;  // buffer cache-policy bits sc0 | sc1: device-coherent access

#ifndef AWQ_SKINNY_WAVES_PER_EU
#define AWQ_SKINNY_WAVES_PER_EU 2
#endif
template <int WPL, int MT, int SPG, bool SEQ, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(AWQ_SKINNY_WAVES_PER_EU, AWQ_SKINNY_WAVES_PER_EU)))
skinny_kn_kernel(const GemmArgs p, int scale_bf16) {
  constexpr int NACC = WPL * 8 * MT;  // f32x4 accumulators per lane
  constexpr int CH = NACC < 16 ? NACC : 16;
  constexpr int PF = 4;               // k-steps per loop iteration (ring depth)
  constexpr int IG = PF / SPG;        // groups per iteration
  __shared__ f32x4 red[3 * CH * 64];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR) by construction
  const int q = lane >> 4, r = lane & 15;
  const int NW = p.N >> 3;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int word0 = tile * 16 * WPL + r * WPL;
  const bool wvalid = word0 < NW;
  const int wld = wvalid ? word0 : 0;  // clamped, always in bounds

  // group range of this wave
  const int ngroups = p.K / p.G;
  const int gs0 = split * p.steps_per_split;  // steps_per_split counts groups here
  const int gs1 = min(ngroups, gs0 + p.steps_per_split);
  const int per = (max(0, gs1 - gs0) + 3) >> 2;
  const int wg0 = min(gs1, gs0 + wave * per);
  const int wg1 = min(gs1, wg0 + per);

  f32x4 acc[WPL][8][MT];
#pragma unroll
  for (int w = 0; w < WPL; ++w)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[w][i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wg0 < wg1) {
    const int ks_begin = wg0 * SPG, ks_end = wg1 * SPG;  // k-steps [ks_begin, ks_end)
    const int ks_last = ks_end - 1;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, (uint32_t)((uint64_t)p.K * NW * 4u));
    const uint32_t row_bytes = (uint32_t)NW * 4u;
    const uint32_t lane_off = (uint32_t)(8 * q) * row_bytes + (uint32_t)wld * 4u;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u));
    // the whole row offset rides in the VGPR offset: buffer range checks cover the VGPR
    // offset only (the SGPR offset is excluded), so rows >= M read as zero
    uint32_t x_lane_off[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      x_lane_off[mt] = ((uint32_t)(mt * 16 + r) * (uint32_t)p.lda + 8u * (uint32_t)q) * 2u;
    const MagicK mk = magic_consts();

    uint32_t raw[PF][8][WPL];
    u32x4 xr[PF][MT];
    WordSZ szc[IG][WPL];  // raw constants of the groups of the iteration being computed
    ColConst cc[WPL][8];

    auto issue = [&](int ks, uint32_t (&dst)[8][WPL], u32x4 (&xd)[MT]) {
      const uint32_t kbase = (uint32_t)ks * 32u * row_bytes;  // wave-uniform
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int soff = (int)(kbase + (uint32_t)j * row_bytes);
        if constexpr (WPL == 4) {
          const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)lane_off, soff, 2));
          dst[j][0] = v[0]; dst[j][1] = v[1]; dst[j][2] = v[2]; dst[j][3] = v[3];
        } else if constexpr (WPL == 2) {
          const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrs, (int)lane_off, soff, 2));
          dst[j][0] = v[0]; dst[j][1] = v[1];
        } else {
          dst[j][0] = __builtin_amdgcn_raw_buffer_load_b32(wrs, (int)lane_off, soff, 2);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // rows >= M fall outside the buffer range and read as zero: no branch, so the
        // compiler's counter waits stay exact across the loop
        const uint32_t xoff = (uint32_t)(ks * 32) * 2u;
        xd[mt] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)x_lane_off[mt], (int)xoff, 0));
      }
    };
    // group constants through buffer loads too: as intrinsic calls they are not merged
    // with the prologue's loads into one load at the loop header (which would put them
    // right before their use and stall every group boundary)
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.sc, (uint32_t)((uint64_t)ngroups * p.N * 2u));
    const __amdgpu_buffer_rsrc_t zrs = make_rsrc(p.qz, ZP ? (uint32_t)((uint64_t)ngroups * NW * 4u) : 0u);
    auto issue_sz = [&](int g, WordSZ (&dst)[WPL]) {
      g = min(g, wg1 - 1);
      const int s_soff = (int)((uint32_t)g * (uint32_t)p.N * 2u);
      const int z_soff = (int)((uint32_t)g * (uint32_t)NW * 4u);
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        dst[w].s4 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)(16u * (uint32_t)(wld + w)), s_soff, 0));
        dst[w].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)(4u * (uint32_t)(wld + w)), z_soff, 0) : 0x88888888u;
      }
    };
    auto compute = [&](const uint32_t (&rw)[8][WPL], const u32x4 (&xv)[MT]) {
#pragma unroll
      for (int w = 0; w < WPL; ++w) {
        uint32_t mlo[4], mhi[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          mlo[u] = pair_lo(rw[2 * u][w], rw[2 * u + 1][w]);
          mhi[u] = pair_hi(rw[2 * u][w], rw[2 * u + 1][w]);
        }
#define AWQ_SKINNY_NIB(I)                                                        \
        {                                                                        \
          const u32x4 op = rows_operand<I, FAST, T>(mlo, mhi, cc[w][I], mk);     \
          _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                      \
              acc[w][I][mt] = MfmaOp<T>::run(op, xv[mt], acc[w][I][mt]);         \
        }
        AWQ_SKINNY_NIB(0) AWQ_SKINNY_NIB(1) AWQ_SKINNY_NIB(2) AWQ_SKINNY_NIB(3)
        AWQ_SKINNY_NIB(4) AWQ_SKINNY_NIB(5) AWQ_SKINNY_NIB(6) AWQ_SKINNY_NIB(7)
#undef AWQ_SKINNY_NIB
      }
    };
    auto prep = [&](const WordSZ (&szv)[WPL]) {
#pragma unroll
      for (int w = 0; w < WPL; ++w) prep_consts<SEQ, FAST>(szv[w], scale_bf16 != 0, cc[w]);
    };

    // prologue: first iteration's k-steps.  Slots past the wave's range re-load its last
    // k-step (cache hits, never used).  The slot that starts a group also carries that
    // group's raw constants, so they travel (and are waited for) with its weight words.
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (u % SPG == 0) issue_sz(min(ks_begin + u, ks_last) / SPG, szc[u / SPG]);
      issue(min(ks_begin + u, ks_last), raw[u], xr[u]);
    }

    int ks0 = ks_begin;
    for (; ks0 + PF <= ks_end; ks0 += PF) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        if (u % SPG == 0) prep(szc[u / SPG]);
        compute(raw[u], xr[u]);
        const int nks = min(ks0 + u + PF, ks_last);
        if (u % SPG == 0) issue_sz(nks / SPG, szc[u / SPG]);
        issue(nks, raw[u], xr[u]);
      }
    }
    // tail (only when the wave's range is not a multiple of PF k-steps)
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      if (ks0 + u < ks_end) {
        if (u % SPG == 0) prep(szc[u / SPG]);
        compute(raw[u], xr[u]);
      }
    }
  }

  // ---- cross-wave reduction (fixed order: wave 0 + wave 1 + wave 2 + wave 3) ----
#define AWQ_ACC_AT(IDX) acc[(IDX) / (8 * MT)][((IDX) / MT) % 8][(IDX) % MT]
#pragma unroll
  for (int c0 = 0; c0 < NACC; c0 += CH) {
    if (wave > 0) {
#pragma unroll
      for (int c = 0; c < CH; ++c) red[((wave - 1) * CH + c) * 64 + lane] = AWQ_ACC_AT(c0 + c);
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        f32x4 v = AWQ_ACC_AT(c0 + c);
        v += red[(0 * CH + c) * 64 + lane];
        v += red[(1 * CH + c) * 64 + lane];
        v += red[(2 * CH + c) * 64 + lane];
        AWQ_ACC_AT(c0 + c) = v;
      }
    }
    __syncthreads();
  }
#undef AWQ_ACC_AT

  // lane (q, r) of wave 0 holds, for accumulator [w][i][mt] element v, token mt*16 + r and
  // column 8 * (tile*16*WPL + (4q + v)*WPL + w) + nib_col(i).
  const int M = p.M, N = p.N;
  if (p.nsplit == 1) {
    if (wave == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        if (m >= M) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
#pragma unroll
          for (int w = 0; w < WPL; ++w) {
            const int word = tile * 16 * WPL + (4 * q + v) * WPL + w;
            if (word >= NW) continue;
            float o[8];
#pragma unroll
            for (int cidx = 0; cidx < 8; ++cidx) o[cidx] = acc[w][col_nib<SEQ>(cidx)][mt][v];
            if (p.bias) {
#pragma unroll
              for (int cidx = 0; cidx < 8; ++cidx) o[cidx] += load_bias(p.bias, p.bias_dtype, 8 * word + cidx);
            }
            u32x4 st;
            st[0] = pack2<T>(o[0], o[1]);
            st[1] = pack2<T>(o[2], o[3]);
            st[2] = pack2<T>(o[4], o[5]);
            st[3] = pack2<T>(o[6], o[7]);
            *(u32x4*)(p.c + (int64_t)m * p.ldc + 8 * word) = st;
          }
        }
      }
    }
    return;
  }

  // ---- split-K: publish the fp32 partial tile, the last block of the tile reduces ----
  const uint32_t part_bytes = (uint32_t)p.nsplit * (uint32_t)M * (uint32_t)N * 4u;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(p.partial, part_bytes);
  if (wave == 0) {
    const uint32_t split_off = (uint32_t)split * (uint32_t)M * (uint32_t)N * 4u;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      if (m >= M) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int w = 0; w < WPL; ++w) {
          const int word = tile * 16 * WPL + (4 * q + v) * WPL + w;
          if (word >= NW) continue;
          const uint32_t off = ((uint32_t)m * (uint32_t)N + 8u * (uint32_t)word) * 4u;
          const f32x4 lo = f32x4{acc[w][col_nib<SEQ>(0)][mt][v], acc[w][col_nib<SEQ>(1)][mt][v],
                                 acc[w][col_nib<SEQ>(2)][mt][v], acc[w][col_nib<SEQ>(3)][mt][v]};
          const f32x4 hi = f32x4{acc[w][col_nib<SEQ>(4)][mt][v], acc[w][col_nib<SEQ>(5)][mt][v],
                                 acc[w][col_nib<SEQ>(6)][mt][v], acc[w][col_nib<SEQ>(7)][mt][v]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), prs, (int)off, (int)split_off, kCoherent);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), prs, (int)(off + 16u), (int)split_off, kCoherent);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the partial stores have completed (device-coherent)
  __syncthreads();
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(&p.counters[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == p.nsplit - 1);
  }
  __syncthreads();
  if (!s_last) return;
  const int col0 = tile * 16 * WPL * 8;
  const int ncols = min(16 * WPL * 8, N - col0);
  const int nq = ncols >> 2;  // float4 chunks per row
  for (int idx = tid; idx < M * nq; idx += 256) {
    const int m = idx / nq, cq = idx - m * nq;
    const int col = col0 + 4 * cq;
    const uint32_t off = ((uint32_t)m * (uint32_t)N + (uint32_t)col) * 4u;
    const uint32_t sstride = (uint32_t)M * (uint32_t)N * 4u;
    f32x4 sum = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, 0, kCoherent));
    for (int sp = 1; sp < p.nsplit; ++sp)
      sum += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)off, (int)(sp * sstride), kCoherent));
    if (p.bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] += load_bias(p.bias, p.bias_dtype, col + e);
    }
    u32x2 st;
    st[0] = pack2<T>(sum[0], sum[1]);
    st[1] = pack2<T>(sum[2], sum[3]);
    *(u32x2*)(p.c + (int64_t)m * p.ldc + col) = st;
  }
  if (tid == 0) __hip_atomic_store(&p.counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------------------------
// Prefill GEMM kernel, KN layouts.  Block tile BM x 256, 4 waves in a 2 x 2 grid, wave tile
// (BM/2) x 128.  A (activations) goes through LDS in 64-wide k stages (double buffered,
// 16-byte chunks XOR-swizzled by row); each wave reads its own 16 weight words per row
// from global memory and dequantizes them into MFMA operands in registers.
template <int BM, bool SEQ, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(256) gemm_kn_kernel(const GemmArgs p, int scale_bf16,
                                                      int tiles_m, int tiles_n) {
  constexpr int BK = 64;
  constexpr int WM = BM / 2;
  constexpr int MTL = WM / 16;               // m-tiles per wave
  constexpr int ACH = BM * BK / 8 / 256;     // 16-byte A chunks per thread per stage
  __shared__ u32x4 lds_a[2][BM * BK / 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int wave_m = wave >> 1, wave_n = wave & 1;

  // XCD-aware tile order: blocks are dealt round-robin to the 8 XCDs; give each XCD a
  // contiguous range of tiles (row-tile major) so blocks sharing an A row-tile share an L2.
  const int ntiles = tiles_m * tiles_n;
  int bid = blockIdx.x;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int tm = bid / tiles_n, tn = bid - tm * tiles_n;
  const int m0 = tm * BM, n0 = tn * 256;

  const int NW = p.N >> 3;
  const int word = (n0 >> 3) + wave_n * 16 + r;
  const bool wvalid = word < NW;
  const int wld = wvalid ? word : 0;

  f32x4 acc[MTL][8];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[mt][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = p.K / BK;
  u32x4 areg[ACH];
  auto load_a = [&](int st) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      const int gr = min(m0 + row, p.M - 1);
      areg[i] = *(const u32x4*)(p.a + (int64_t)gr * p.lda + st * BK + ch * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i;
      const int row = c >> 3, ch = c & 7;
      lds_a[buf][row * 8 + (ch ^ (row & 7))] = areg[i];
    }
  };
  uint32_t braw[2][8];
  WordSZ bsz[2];
  auto load_b = [&](int st, uint32_t (&dst)[2][8], WordSZ (&szd)[2]) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        dst[sub][j] = __builtin_nontemporal_load(p.qw + (int64_t)(st * BK + sub * 32 + 8 * q + j) * NW + wld);
      szd[sub] = load_sz<ZP>(p, (st * BK + sub * 32) / p.G, wld);
    }
  };

  ColConst cc[8];
  int cur_g = -1;
  const MagicK mk = magic_consts();

  load_a(0);
  store_a(0);
  load_b(0, braw, bsz);
  __syncthreads();

  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    uint32_t bnext[2][8];
    WordSZ sznext[2];
    if (st + 1 < nst) {
      load_a(st + 1);
      load_b(st + 1, bnext, sznext);
    }
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int g = (st * BK + sub * 32) / p.G;
      if (g != cur_g) {
        cur_g = g;
        prep_consts<SEQ, FAST>(bsz[sub], scale_bf16 != 0, cc);
      }
      u32x4 af[MTL];
#pragma unroll
      for (int mt = 0; mt < MTL; ++mt) {
        const int row = wave_m * WM + mt * 16 + r;
        const int ch = sub * 4 + q;
        af[mt] = lds_a[buf][row * 8 + (ch ^ (row & 7))];
      }
      uint32_t mlo[4], mhi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        mlo[u] = pair_lo(braw[sub][2 * u], braw[sub][2 * u + 1]);
        mhi[u] = pair_hi(braw[sub][2 * u], braw[sub][2 * u + 1]);
      }
#define AWQ_GEMM_NIB(I)                                                          \
      {                                                                          \
        const u32x4 bop = rows_operand<I, FAST, T>(mlo, mhi, cc[I], mk);         \
        _Pragma("unroll") for (int mt = 0; mt < MTL; ++mt)                       \
            acc[mt][I] = MfmaOp<T>::run(af[mt], bop, acc[mt][I]);                \
      }
      AWQ_GEMM_NIB(0) AWQ_GEMM_NIB(1) AWQ_GEMM_NIB(2) AWQ_GEMM_NIB(3)
      AWQ_GEMM_NIB(4) AWQ_GEMM_NIB(5) AWQ_GEMM_NIB(6) AWQ_GEMM_NIB(7)
#undef AWQ_GEMM_NIB
    }
    if (st + 1 < nst) {
      store_a(buf ^ 1);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
        for (int j = 0; j < 8; ++j) braw[sub][j] = bnext[sub][j];
        bsz[sub] = sznext[sub];
      }
    }
    __syncthreads();
  }

  // lane (q, r) holds acc[mt][i][v] = C[row m0 + wave_m*WM + mt*16 + 4q + v][8*word + nib_col(i)]
  if (!wvalid) return;
  float bv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) bv[c] = p.bias ? load_bias(p.bias, p.bias_dtype, 8 * word + c) : 0.0f;
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = m0 + wave_m * WM + mt * 16 + 4 * q + v;
      if (row >= p.M) continue;
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[c] = acc[mt][col_nib<SEQ>(c)][v] + bv[c];
      u32x4 st;
      st[0] = pack2<T>(o[0], o[1]);
      st[1] = pack2<T>(o[2], o[3]);
      st[2] = pack2<T>(o[4], o[5]);
      st[3] = pack2<T>(o[6], o[7]);
      *(u32x4*)(p.c + (int64_t)row * p.ldc + 8 * word) = st;
    }
  }
}

// ----------------------------------------------------------------------------------
// Repack reference layout -> AutoAWQ layout.
// Weights: thread = 8x8 nibble block: input words (n0+e, kw) e<8 -> output words (8kw+t, n0/8) t<8.
__global__ void __launch_bounds__(256) repack_w_kernel(const uint32_t* __restrict__ in,
                                                       uint32_t* __restrict__ out, int64_t N,
                                                       int64_t K) {
  const int64_t KW = K >> 3, NWd = N >> 3;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= KW * NWd) return;
  const int64_t nb = idx / KW, kw = idx - nb * KW;  // consecutive threads: consecutive kw
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = in[(nb * 8 + e) * KW + kw];
#pragma unroll
  for (int t = 0; t < 8; ++t) {  // k = 8kw + t
    uint32_t o = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // output nibble i holds column 8nb + order[i]
      const int e = nib_col<false>(i);
      o |= ((w[e] >> (4 * t)) & 0xFu) << (4 * i);
    }
    out[(kw * 8 + t) * NWd + nb] = o;
  }
}
// Zeros: [N, ZW] sequential along groups -> [NG, N/8] interleaved; thread = output word.
__global__ void __launch_bounds__(256) repack_z_kernel(const uint32_t* __restrict__ in,
                                                       uint32_t* __restrict__ out, int64_t N,
                                                       int64_t NG) {
  const int64_t ZW = (NG + 7) >> 3, NWd = N >> 3;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= NG * NWd) return;
  const int64_t g = idx / NWd, j = idx - g * NWd;
  uint32_t o = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t n = 8 * j + nib_col<false>(i);
    o |= ((in[n * ZW + (g >> 3)] >> (4 * (g & 7))) & 0xFu) << (4 * i);
  }
  out[idx] = o;
}
// Scales: 2-byte transpose [N, NG] -> [NG, N].
__global__ void __launch_bounds__(256) repack_s_kernel(const uint16_t* __restrict__ in,
                                                       uint16_t* __restrict__ out, int64_t N,
                                                       int64_t NG) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= N * NG) return;
  const int64_t g = idx / N, n = idx - g * N;
  out[idx] = in[n * NG + g];
}

// ----------------------------------------------------------------------------------
// Host side.
int g_num_cus = 0;
std::once_flag g_cu_once;

int num_cus() {
  std::call_once(g_cu_once, [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_num_cus = n;
    else
      g_num_cus = 256;
  });
  return g_num_cus;
}

int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool dtype_16(int d) { return d == AWQ_DTYPE_F16 || d == AWQ_DTYPE_BF16; }

// ---- skinny planning ----
// Workspace layout: [0, AWQ_COUNTER_BYTES) arrival counters (zero between calls), then fp32
// partials.  The counter region sits at a fixed offset so calls of different shapes that
// share one workspace always find it zeroed.
constexpr size_t AWQ_COUNTER_BYTES = 65536;
constexpr int SKINNY_PF = 4;

struct SkinnyPlan {
  int wpl, mt;
  int tiles, nsplit, steps_per_split;
  size_t ws_bytes;
};

int pick_wpl(int64_t M, int64_t N) {
  const int64_t nw = N / 8;
  int wpl = 2;
  while (wpl > 1 && (nw % wpl) != 0) wpl >>= 1;
  return wpl;
}

SkinnyPlan plan_skinny(int64_t M, int64_t N, int64_t K, int64_t G, int split_k) {
  SkinnyPlan s{};
  s.wpl = pick_wpl(M, N);
  s.mt = (M > 16) ? 2 : 1;
  if (s.mt == 2) s.wpl = 1;
  const int64_t cols = 16 * s.wpl * 8;
  s.tiles = (int)cdiv(N, cols);
  const int64_t ng = K / G;       // partition unit: one quantization group
  const int64_t spg = G / 32;     // k-steps per group
  int64_t ns;
  if (split_k > 0) {
    ns = split_k;
  } else {
    // Fill the chip with one round of resident blocks (2 per CU) while giving every wave
    // at least 8 k-steps where the problem allows; prefer fewer partitions on ties.
    const int64_t slots = (int64_t)num_cus() * 2;
    const int64_t max_ns = std::max<int64_t>(1, (ng * spg) / 32);
    int64_t best = 1;
    double best_score = -1e30;
    for (int64_t c = 1; c <= max_ns; ++c) {
      const int64_t blocks = (int64_t)s.tiles * c;
      const double rounds = (double)cdiv(blocks, slots);
      const double fill = (double)blocks / (rounds * (double)slots);
      const double score = fill - 0.003 * (double)c - 0.25 * (rounds - 1.0);
      if (score > best_score + 1e-9) {
        best_score = score;
        best = c;
      }
    }
    ns = best;
  }
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, ng));
  s.steps_per_split = (int)cdiv(ng, ns);           // groups per partition
  s.nsplit = (int)cdiv(ng, s.steps_per_split);     // no empty partitions
  s.ws_bytes = 0;
  if (s.nsplit > 1) {
    const size_t part = (size_t)s.nsplit * (size_t)M * (size_t)N * sizeof(float);
    s.ws_bytes = AWQ_COUNTER_BYTES + part;
  }
  return s;
}

template <int WPL, int MT, bool SEQ, bool ZP, typename T, bool FAST>
void launch_skinny_t(const GemmArgs& a, const SkinnyPlan& s, int sbf, hipStream_t st) {
  dim3 grid(s.tiles, s.nsplit);
  const int spg = a.G / 32;
  if (spg == 4)
    hipLaunchKernelGGL((skinny_kn_kernel<WPL, MT, 4, SEQ, ZP, T, FAST>), grid, dim3(256), 0, st, a, sbf);
  else if (spg == 2)
    hipLaunchKernelGGL((skinny_kn_kernel<WPL, MT, 2, SEQ, ZP, T, FAST>), grid, dim3(256), 0, st, a, sbf);
  else
    hipLaunchKernelGGL((skinny_kn_kernel<WPL, MT, 1, SEQ, ZP, T, FAST>), grid, dim3(256), 0, st, a, sbf);
}

template <bool SEQ, bool ZP, typename T, bool FAST>
void launch_skinny_sel(const GemmArgs& a, const SkinnyPlan& s, int sbf, hipStream_t st) {
  if (s.mt == 2) {
    launch_skinny_t<1, 2, SEQ, ZP, T, FAST>(a, s, sbf, st);
  } else {
    if (s.wpl == 2) launch_skinny_t<2, 1, SEQ, ZP, T, FAST>(a, s, sbf, st);
    else launch_skinny_t<1, 1, SEQ, ZP, T, FAST>(a, s, sbf, st);
  }
}

template <int BM, bool SEQ, bool ZP, typename T, bool FAST>
void launch_gemm_t(const GemmArgs& a, int sbf, hipStream_t st) {
  const int tm = (int)cdiv(a.M, BM), tn = (int)cdiv(a.N, 256);
  hipLaunchKernelGGL((gemm_kn_kernel<BM, SEQ, ZP, T, FAST>), dim3(tm * tn), dim3(256), 0, st, a,
                     sbf, tm, tn);
}

int pick_bm(int64_t M, int64_t N) {
  const int64_t slots = num_cus();
  auto fill = [&](int64_t bm) {
    const int64_t blocks = cdiv(M, bm) * cdiv(N, 256);
    return (double)blocks / ((double)cdiv(blocks, slots) * (double)slots);
  };
  if (M >= 256 && fill(256) >= 0.99 * fill(128)) return 256;
  return 128;
}

template <bool SEQ, bool ZP, typename T, bool FAST>
void launch_gemm_sel(const GemmArgs& a, int sbf, hipStream_t st) {
  if (pick_bm(a.M, a.N) == 256) launch_gemm_t<256, SEQ, ZP, T, FAST>(a, sbf, st);
  else launch_gemm_t<128, SEQ, ZP, T, FAST>(a, sbf, st);
}

template <bool SEQ, bool ZP>
void dispatch_gemm(const GemmArgs& a, bool skinny, const SkinnyPlan& s, int act, int sdt,
                   hipStream_t st) {
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (act == AWQ_DTYPE_F16) {
    if (sdt == AWQ_DTYPE_F16) {
      if (skinny) launch_skinny_sel<SEQ, ZP, f16, true>(a, s, sbf, st);
      else launch_gemm_sel<SEQ, ZP, f16, true>(a, sbf, st);
    } else {
      if (skinny) launch_skinny_sel<SEQ, ZP, f16, false>(a, s, sbf, st);
      else launch_gemm_sel<SEQ, ZP, f16, false>(a, sbf, st);
    }
  } else {
    if (skinny) launch_skinny_sel<SEQ, ZP, bf16, false>(a, s, sbf, st);
    else launch_gemm_sel<SEQ, ZP, bf16, false>(a, sbf, st);
  }
}

template <typename F>
int with_out_dtype(int out_dtype, F&& f) {
  switch (out_dtype) {
    case AWQ_DTYPE_F16: f(std::integral_constant<int, AWQ_DTYPE_F16>{}); return AWQ_OK;
    case AWQ_DTYPE_BF16: f(std::integral_constant<int, AWQ_DTYPE_BF16>{}); return AWQ_OK;
    case AWQ_DTYPE_F32: f(std::integral_constant<int, AWQ_DTYPE_F32>{}); return AWQ_OK;
    default: return AWQ_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" {

int awq_w4a16_version(void) { return 100; }

const char* awq_w4a16_strerror(int code) {
  switch (code) {
    case AWQ_OK: return "ok";
    case AWQ_ERR_NULL: return "a required pointer is NULL";
    case AWQ_ERR_SHAPE: return "inconsistent sizes (need N % 8 == 0, K % group_size == 0, group_size % 32 == 0 for GEMM, % 8 for dequant)";
    case AWQ_ERR_UNSUPPORTED: return "unsupported dtype/layout/shape combination";
    case AWQ_ERR_WORKSPACE: return "workspace missing or too small";
    case AWQ_ERR_LAUNCH: return "HIP kernel launch failed";
    case AWQ_ERR_STRIDE: return "leading dimension smaller than the row length or misaligned";
    default: return "unknown error";
  }
}

int awq_w4a16_dequant(const int32_t* qweight, const void* scales, const int32_t* qzeros, void* out,
                      int64_t rows, int64_t cols, int32_t group_size, int32_t layout,
                      int32_t scale_dtype, int32_t out_dtype, void* stream) {
  if (!qweight || !scales || !out) return AWQ_ERR_NULL;
  if (rows < 0 || cols < 0 || group_size <= 0 || (group_size % 8) != 0) return AWQ_ERR_SHAPE;
  if (!dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const bool zp = qzeros != nullptr;
  const bool sbf = scale_dtype == AWQ_DTYPE_BF16;
  if (layout == AWQ_LAYOUT_AUTOAWQ || layout == AWQ_LAYOUT_KN_SEQ) {
    const int64_t K = rows, N = cols;
    if ((N % 8) != 0 || (K % group_size) != 0) return AWQ_ERR_SHAPE;
    const int64_t n = K * (N / 8);
    if (n == 0) return AWQ_OK;
    const dim3 grid((unsigned)cdiv(n, 256));
    const uint32_t* qw = (const uint32_t*)qweight;
    const uint32_t* qz = (const uint32_t*)qzeros;
    const uint16_t* sc = (const uint16_t*)scales;
    int rc = with_out_dtype(out_dtype, [&](auto od) {
      constexpr int OD = decltype(od)::value;
#define AWQ_DQ_KN(SEQ, ZP, ST) hipLaunchKernelGGL((dequant_kn_kernel<SEQ, ZP, ST, OD>), grid, dim3(256), 0, st, qw, sc, qz, out, K, N, (int)group_size)
      const bool seq = layout == AWQ_LAYOUT_KN_SEQ;
      if (seq) {
        if (zp) { if (sbf) AWQ_DQ_KN(true, true, bf16); else AWQ_DQ_KN(true, true, f16); }
        else { if (sbf) AWQ_DQ_KN(true, false, bf16); else AWQ_DQ_KN(true, false, f16); }
      } else {
        if (zp) { if (sbf) AWQ_DQ_KN(false, true, bf16); else AWQ_DQ_KN(false, true, f16); }
        else { if (sbf) AWQ_DQ_KN(false, false, bf16); else AWQ_DQ_KN(false, false, f16); }
      }
#undef AWQ_DQ_KN
    });
    if (rc != AWQ_OK) return rc;
    return launch_status();
  }
  if (layout == AWQ_LAYOUT_NK_SEQ) {
    const int64_t N = rows, K = cols;
    if ((K % 8) != 0 || (K % group_size) != 0) return AWQ_ERR_SHAPE;
    const int64_t n = N * (K / 8);
    if (n == 0) return AWQ_OK;
    const dim3 grid((unsigned)cdiv(n, 256));
    const uint32_t* qw = (const uint32_t*)qweight;
    const uint32_t* qz = (const uint32_t*)qzeros;
    const uint16_t* sc = (const uint16_t*)scales;
    int rc = with_out_dtype(out_dtype, [&](auto od) {
      constexpr int OD = decltype(od)::value;
#define AWQ_DQ_NK(ZP, ST) hipLaunchKernelGGL((dequant_nk_kernel<ZP, ST, OD>), grid, dim3(256), 0, st, qw, sc, qz, out, N, K, (int)group_size)
      if (zp) { if (sbf) AWQ_DQ_NK(true, bf16); else AWQ_DQ_NK(true, f16); }
      else { if (sbf) AWQ_DQ_NK(false, bf16); else AWQ_DQ_NK(false, f16); }
#undef AWQ_DQ_NK
    });
    if (rc != AWQ_OK) return rc;
    return launch_status();
  }
  return AWQ_ERR_UNSUPPORTED;
}

size_t awq_w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                      int32_t split_k, int32_t layout) {
  (void)group_size;
  (void)layout;
  if (M <= 0 || N <= 0 || K <= 0 || M > 32 || (K % 32) != 0) return 0;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
  if (group_size <= 0 || (group_size % 32) != 0 || (K % group_size) != 0) return 0;
  return plan_skinny(M, N, K, group_size, split_k).ws_bytes;
}

int awq_w4a16_gemm(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                   int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                   int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (!a || !qweight || !scales || !c) return AWQ_ERR_NULL;
  if (bias && bias_dtype == AWQ_DTYPE_NONE) return AWQ_ERR_UNSUPPORTED;
  if (!dtype_16(act_dtype) || !dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  if (bias && bias_dtype != AWQ_DTYPE_F16 && bias_dtype != AWQ_DTYPE_BF16 && bias_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if (M < 0 || N < 0 || K < 0 || group_size <= 0) return AWQ_ERR_SHAPE;
  if ((N % 8) != 0 || (group_size % 32) != 0 || (K % group_size) != 0) return AWQ_ERR_SHAPE;
  if (split_k < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || N == 0) return AWQ_OK;
  if (lda < K || ldc < N || (lda % 8) != 0 || (ldc % 8) != 0) return AWQ_ERR_STRIDE;
  if ((((uintptr_t)a) & 15) || (((uintptr_t)c) & 15) || (((uintptr_t)scales) & 15) ||
      (((uintptr_t)qweight) & 15))
    return AWQ_ERR_STRIDE;
  if (layout == AWQ_LAYOUT_NK_SEQ) return AWQ_ERR_UNSUPPORTED;
  if (K * (N / 8) * 4 > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;  // 32-bit buffer offsets
  if (layout != AWQ_LAYOUT_AUTOAWQ && layout != AWQ_LAYOUT_KN_SEQ) return AWQ_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;

  GemmArgs ga{};
  ga.a = (const uint16_t*)a;
  ga.qw = (const uint32_t*)qweight;
  ga.sc = (const uint16_t*)scales;
  ga.qz = (const uint32_t*)qzeros;
  ga.bias = bias;
  ga.c = (uint16_t*)c;
  ga.lda = lda;
  ga.ldc = ldc;
  ga.M = (int)M;
  ga.N = (int)N;
  ga.K = (int)K;
  ga.G = group_size;
  ga.bias_dtype = bias ? bias_dtype : AWQ_DTYPE_NONE;

  if (K == 0) return AWQ_ERR_SHAPE;
  // the decode kernel's group-aligned loop covers group sizes 32, 64 and 128
  const bool skinny = M <= 32 && (group_size == 32 || group_size == 64 || group_size == 128);
  SkinnyPlan sp{};
  if (skinny) {
    sp = plan_skinny(M, N, K, group_size, split_k);
    ga.nsplit = sp.nsplit;
    ga.steps_per_split = sp.steps_per_split;
    if (sp.ws_bytes) {
      if (!workspace || workspace_bytes < sp.ws_bytes) return AWQ_ERR_WORKSPACE;
      if ((size_t)sp.tiles * sizeof(int) > AWQ_COUNTER_BYTES) return AWQ_ERR_UNSUPPORTED;
      ga.counters = (int*)workspace;
      ga.partial = (float*)((char*)workspace + AWQ_COUNTER_BYTES);
    }
  } else {
    if ((K % 64) != 0) return AWQ_ERR_SHAPE;
    ga.nsplit = 1;
    ga.steps_per_split = (int)(K / 32);
  }
  const bool seq = layout == AWQ_LAYOUT_KN_SEQ;
  const bool zp = qzeros != nullptr;
  if (seq) {
    if (zp) dispatch_gemm<true, true>(ga, skinny, sp, act_dtype, scale_dtype, st);
    else dispatch_gemm<true, false>(ga, skinny, sp, act_dtype, scale_dtype, st);
  } else {
    if (zp) dispatch_gemm<false, true>(ga, skinny, sp, act_dtype, scale_dtype, st);
    else dispatch_gemm<false, false>(ga, skinny, sp, act_dtype, scale_dtype, st);
  }
  return launch_status();
}

int awq_w4a16_repack_nk_to_autoawq(const int32_t* qweight_nk, const int32_t* qzeros_nk,
                                   const void* scales_nk, int32_t* qweight_kn, int32_t* qzeros_kn,
                                   void* scales_kn, int64_t N, int64_t K, int32_t group_size,
                                   void* stream) {
  if (!qweight_nk || !qweight_kn || !scales_nk || !scales_kn) return AWQ_ERR_NULL;
  if (qzeros_nk && !qzeros_kn) return AWQ_ERR_NULL;
  if (N < 0 || K < 0 || group_size <= 0 || (N % 8) || (K % 8) || (K % group_size)) return AWQ_ERR_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const int64_t NG = K / group_size;
  const int64_t nw = (K / 8) * (N / 8);
  if (nw > 0)
    hipLaunchKernelGGL(repack_w_kernel, dim3((unsigned)cdiv(nw, 256)), dim3(256), 0, st,
                       (const uint32_t*)qweight_nk, (uint32_t*)qweight_kn, N, K);
  if (qzeros_nk && NG * (N / 8) > 0)
    hipLaunchKernelGGL(repack_z_kernel, dim3((unsigned)cdiv(NG * (N / 8), 256)), dim3(256), 0, st,
                       (const uint32_t*)qzeros_nk, (uint32_t*)qzeros_kn, N, NG);
  if (N * NG > 0)
    hipLaunchKernelGGL(repack_s_kernel, dim3((unsigned)cdiv(N * NG, 256)), dim3(256), 0, st,
                       (const uint16_t*)scales_nk, (uint16_t*)scales_kn, N, NG);
  return launch_status();
}

}  // extern "C"
