// Narrow decode kernel (M <= 32, N small against the chip): one block per 16 output columns
// over the whole K, so no split-K hand-off -- the role of the reference's decode kernels at
// BLOCK_M = 1 .. 32 (vllm/kernels/triton/awq_fused_gemm.py:1883-1990) for shapes whose 128-
// column tiles are too few to fill 256 CUs.
//
//  * Narrow stream layout (awq_w4a16_pack_decode_narrow): tile t = columns 16 t .. 16 t + 15,
//    K cut into quads of four 32-row k-steps (KQ = ceil(K / 128) per tile, k-steps past K
//    zero).  The (tile t, quad c) run of 1 KiB starts at byte (t * KQ + c) * 1024; lane
//    l = 16 q + r owns the 16 bytes at 16 l, its u32 number i being k-step s = 4 c + i: the
//    eight nibbles of column 16 t + r at rows 32 s + 8 q + j, rows 2u and 2u + 1 at nibble u of
//    the low and the high 16-bit half.  One u32 is then the lane's whole MFMA operand for one
//    k-step (pair u is magic_bits<u>), and one 16-byte load per lane brings four k-steps.
//  * Lane (q, r) multiplies the activations (16 tokens x 32 k) by column 16 t + r's 32 rows
//    with one v_mfma_f32_16x16x32 per k-step; the operand holds the exact integers q - z
//    (magic-exponent unpack, one packed subtraction per pair of rows), each group's sum is
//    scaled once by the column's fp32 scale -- unrounded weights, as in the wide decode
//    kernel and the reference's M = 1 formulation (awq_fused_gemm.py:1966-1971).
//  * Short launches are bounded by the instructions a wave runs before its first weight load
//    and after its last one lands, so each wave issues its weight loads (contiguous quads, a
//    ring of D quads) as its first memory operations; the block's DMA of scales, zero words
//    and activation rows into LDS follows, then one wait and one barrier.  The waves meet in
//    LDS at the end and sum in wave order (bitwise reproducible).
//  * Gated epilogue (GemmArgs::gate_act): the gate/up pair interleaved per 8 columns, so a
//    tile's columns c < 8 and 8 + c are the gate and up sums of output 8 t + c.
#include "awq_decode_kernel.h"

namespace awq {

// LDS of one block (bytes): the waves' sums [NWV][MROWS][16] fp32, then the tile's scales
// [groups][16] (2 B each), zero words [groups][2], and with XL the activation rows [xrows][K]
// (2 B).  Each region spans whole DMA instructions (a 64-lane DMA writes all 64 lanes' slots,
// those past the data as zeros), so no instruction reaches into the next region.
struct NarrowLds {
  uint32_t sc, zw, x, total;
};
__host__ __device__ inline NarrowLds narrow_lds(int nwv, int mrows, int ngroups, int K, bool zp, int xrows) {
  const uint32_t n_pieces = ((uint32_t)ngroups * 2u + 63u) / 64u;  // instructions for scales, and for zeros
  NarrowLds l;
  l.sc = (uint32_t)(nwv * mrows * 16 * 4);
  l.zw = l.sc + n_pieces * 1024u;
  l.x = l.zw + (zp ? n_pieces * 256u : 0u);
  l.total = l.x + ((uint32_t)xrows * (uint32_t)K / 8u + 63u) / 64u * 1024u;
  return l;
}

// RMSNorm prologue (rmsnorm_awq_fused.py:108-131) for one fp16 row staged by XL: the row
// arrives in registers instead of by DMA -- lane tid holds the 16-byte pieces pc = tid,
// tid + NT, .. (at most kNormCols of them) with the matching 16 bytes of the norm weights.
// The sum of squares (exact squares added in fp64: lanes by DPP, then the waves through
// `red`) is rounded once to fp32, rrms = rsqrt(var / K + eps) correctly rounded, and each
// element is written to the staged row in LDS as fp16((x * rrms) * norm_w).
constexpr int kNormCols = 6;

template <int NT>
struct NormRow {
  u32x4 x[kNormCols], g[kNormCols];

  __device__ __forceinline__ void load(const GemmArgs& p, int tid) {
    const int kp = p.K >> 3;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.a, (uint32_t)p.K * 2u);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(p.norm_w, (uint32_t)p.K * 2u);
#pragma unroll
    for (int u = 0; u < kNormCols; ++u) {
      if (u * NT < kp) {  // block-uniform
        const int pc = tid + u * NT;
        const int off = pc < kp ? (int)(16u * (uint32_t)pc) : (int)0x80000000;  // past the row: zeros
        x[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
        g[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 0));
      }
    }
  }

  // after the loads have landed: the row's sum, then (one barrier) the normalised pieces
  __device__ __forceinline__ void normalise(const GemmArgs& p, uint16_t* xs, float* red, int wave, int lane, int tid) {
    const int kp = p.K >> 3;
    double ss = 0.0;
#pragma unroll
    for (int u = 0; u < kNormCols; ++u) {
      if (u * NT < kp) {
        double s0 = 0.0, s1 = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const double lo = h_bits2f((uint16_t)(x[u][j] & 0xFFFF)), hi = h_bits2f((uint16_t)(x[u][j] >> 16));
          s0 += lo * lo;
          s1 += hi * hi;
        }
        ss += s0 + s1;
      }
    }
    double* rd = (double*)red;
    ss = wave_sum_f64(ss);
    if (lane == 0) rd[wave] = ss;
    __syncthreads();
    double var = 0.0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) var += rd[w];
    const float rr = rms_scale((float)var, p.K, p.eps);
    const bool nbf = p.norm_bf16 != 0;
#pragma unroll
    for (int u = 0; u < kNormCols; ++u) {
      const int pc = tid + u * NT;
      if (u * NT < kp && pc < kp) {
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint16_t glo = (uint16_t)(g[u][j] & 0xFFFF), ghi = (uint16_t)(g[u][j] >> 16);
          const float lo = fp32_rounded((h_bits2f((uint16_t)(x[u][j] & 0xFFFF)) * rr) * (nbf ? bf_bits2f(glo) : h_bits2f(glo)));
          const float hi = fp32_rounded((h_bits2f((uint16_t)(x[u][j] >> 16)) * rr) * (nbf ? bf_bits2f(ghi) : h_bits2f(ghi)));
          o[j] = (uint32_t)f2h_bits(lo) | ((uint32_t)f2h_bits(hi) << 16);
        }
        *(u32x4*)(xs + 8 * pc) = o;
      }
    }
    __syncthreads();
  }
};

// XL (one token tile): the M activation rows are staged in LDS once ([M][K]) and every lane
// reads its k-slice of row min(r, M - 1) from there (the MFMA's rows past M repeat a real row
// and are never read back); otherwise each quad's activations come with its weights, per lane.
// NORM (one fp16 row staged by XL, K / 8 <= kNormCols * NWV * 64): the row comes through
// registers and is staged normalised (RMSNorm prologue) before the first k-step.
template <int MT, int NWV, int SPG, bool ZP, typename T, bool SBF, bool ONE, bool XL, bool NORM = false>
__global__ void __launch_bounds__(NWV * 64) decode_narrow_kernel(const GemmArgs p_in, int tiles) {
  static_assert(!ONE || MT == 1, "");
  static_assert(!XL || MT == 1, "");
  static_assert(!NORM || (XL && ONE && std::is_same<T, f16>::value), "");
  static_assert(SPG == 1 || SPG == 2 || SPG == 4, "a quad holds whole groups or lies in one");
  // quads in flight per wave (measured at K = 4096: two, except four for one row in 8-wave blocks)
  constexpr int D = (XL && ONE && NWV == 8) ? 4 : 2;
  constexpr int MROWS = ONE ? 1 : 16 * MT;
  // grid row y of a row-exact launch: row y's M = 1 problem (the call itself otherwise); the
  // narrow kernel takes no workspace
  const GemmArgs p = row_slice(p_in, 0, 0, (int)blockIdx.y);
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t = blockIdx.x;
  const int KS = p.K >> 5, KQ = (KS + 3) >> 2;
  const int qa = KQ * wave / NWV, nq = KQ * (wave + 1) / NWV - qa;

  // ---- the wave's weight quads first: nothing but their addresses comes before them ----
  const uint32_t w_bytes = (uint32_t)tiles * (uint32_t)KQ * 1024u;
  const uint32_t w_lane_off = (uint32_t)lane * 16u;
  const uint32_t x_bytes = (uint32_t)((uint64_t)p.M * (uint64_t)p.lda * 2u);
  uint32_t x_lane_off[MT];
  if constexpr (!XL) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      x_lane_off[mt] = ((uint32_t)(mt * 16 + (lane & 15)) * (uint32_t)p.lda + 8u * (uint32_t)(lane >> 4)) * 2u;
  }
  u32x4 wr[D];
  u32x4 xr[XL ? 1 : D][XL ? 1 : 4][MT];
  int ic = qa, ileft = nq;
  auto issue = [&](int slot) {
    const int c = ic;  // wave-uniform
    const bool past = ileft <= 0;
    ++ic;
    --ileft;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(p.qw, past ? 0u : w_bytes);
    // non-temporal, like the stream kernel's weights (each weight byte is read once): 4.95 ->
    // 4.74 us at M = 1, N = 4096 and 7.28 -> 7.16 us at M = 4, N = 6144 (K = 4096).  The
    // constants' and activations' DMA below keeps the default policy: non-temporal there
    // measured 0.3 - 0.6 us slower.
    wr[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                             wrs, (int)w_lane_off, (int)(((uint32_t)t * (uint32_t)KQ + (uint32_t)c) * 1024u), kStreamNT));
    if constexpr (!XL) {
      // the k-step's byte offset rides in the SGPR offset, which the range check does not
      // cover: k-steps past K (the tile's last quad) get an empty range instead
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, (past || c * 4 + i >= KS) ? 0u : x_bytes);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xr[slot][i][mt] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)x_lane_off[mt], (c * 4 + i) * 64, 0));
      }
    }
  };
#pragma unroll
  for (int u = 0; u < D; ++u) issue(u);

  const int q = lane >> 4, r = lane & 15;
  const int NW = p.N >> 3;
  const int ngroups = p.K / p.G;
  const NarrowLds L = narrow_lds(NWV, MROWS, ngroups, p.K, ZP, XL ? p.M : 0);
  float* red = (float*)smem;
  const uint16_t* s_lds = (const uint16_t*)(smem + L.sc);
  const uint32_t* z_lds = (const uint32_t*)(smem + L.zw);
  const uint16_t* x_lds = (const uint16_t*)(smem + L.x);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)smem;

  // ---- then the tile's scales and zero words (and with XL the activation rows) by DMA into
  // LDS; wave w issues instructions w, w + NWV, ... of 64 lanes each ----
  {
    const u32x4 srs = rsrc_words(p.sc, (uint32_t)((uint64_t)ngroups * p.N * 2u));
    const u32x4 zrs = rsrc_words(p.qz, ZP ? (uint32_t)((uint64_t)ngroups * NW * 4u) : 0u);
    const u32x4 xrs = rsrc_words(p.a, x_bytes);
    const int n_s = (ngroups * 2 + 63) / 64;           // 16-byte pieces: group i / 2, half i % 2
    const int n_z = ZP ? (ngroups * 2 + 63) / 64 : 0;  // words: group i / 2, word 2t + i % 2
    const int kp = p.K / 8;                            // 16-byte pieces per activation row
    const int n_x = (XL && !NORM) ? (p.M * kp + 63) / 64 : 0;
    for (int j = wave; j < n_s + n_z + n_x; j += NWV) {
      if (j < n_s) {
        const int i = j * 64 + lane;
        const uint32_t voff = i < ngroups * 2 ? (((uint32_t)(i >> 1) * (uint32_t)p.N + 16u * (uint32_t)t + 8u * (uint32_t)(i & 1)) * 2u)
                                              : 0x80000000u;
        lds_dma16(srs, lds_base + L.sc + (uint32_t)j * 1024u, voff, 0u);
      } else if (j < n_s + n_z) {
        const int i = (j - n_s) * 64 + lane;
        const uint32_t voff = i < ngroups * 2 ? (((uint32_t)(i >> 1) * (uint32_t)NW + 2u * (uint32_t)t + (uint32_t)(i & 1)) * 4u)
                                              : 0x80000000u;
        lds_dma4(zrs, lds_base + L.zw + (uint32_t)(j - n_s) * 256u, voff, 0u);
      } else {
        const int i = (j - n_s - n_z) * 64 + lane;
        const int row = i / kp, pc = i - row * kp;
        lds_dma16(xrs, lds_base + L.x + (uint32_t)(j - n_s - n_z) * 1024u,
                  row < p.M ? ((uint32_t)row * (uint32_t)p.lda + 8u * (uint32_t)pc) * 2u : 0x80000000u, 0u);
      }
    }
  }
  NormRow<NWV * 64> npc;
  if constexpr (NORM) npc.load(p, tid);
  // every load of this wave has landed (the ring's first quads with it: they were issued
  // together); the barrier then covers every wave's DMA (with NORM the prologue's first)
  AWQ_WAIT_VMCNT0();
  if constexpr (NORM) npc.normalise(p, (uint16_t*)(smem + L.x), red, wave, lane, tid);
  else __syncthreads();

  f32x4 acc[MT], tot[MT];
  float tot1 = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = tot[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int zsh = 4 * col_nib<false>(r & 7);
  const int x_row_off = ONE ? 0 : min(r, p.M - 1) * p.K;  // XL: the lane's activation row in LDS
  const MagicK mk = magic_consts();

  uint32_t zm0 = 0, zm1 = 0;  // biased zero of the current group (even / odd nibble forms)
  float sf = 0.f;             // scale of the current group (0 before the first: flushes nothing)
  auto flush = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (ONE) tot1 += acc[mt][0] * sf;
      else tot[mt] += acc[mt] * sf;
      acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto prep = [&](int g) {
    const uint32_t z = ZP ? (z_lds[2 * g + (r >> 3)] >> zsh) & 0xFu : 8u;
    zm0 = zero_magic(0, z);
    zm1 = zero_magic(1, z);
    const uint16_t sb = s_lds[16 * g + r];
    sf = SBF ? bf_bits2f(sb) : h_bits2f(sb);
  };
  auto compute = [&](uint32_t w, int slot, int i, int ks) {
    u32x4 op;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t mb;
      switch (u) {
        case 0: mb = magic_bits<0>(w, mk); break;
        case 1: mb = magic_bits<1>(w, mk); break;
        case 2: mb = magic_bits<2>(w, mk); break;
        default: mb = magic_bits<3>(w, mk); break;
      }
      const f16x2 d = as_h2(mb) - as_h2((u & 1) ? zm1 : zm0);
      if constexpr (std::is_same<T, f16>::value) op[u] = as_u(d);
      else op[u] = pack2<bf16>((float)d.x, (float)d.y);
    }
    if constexpr (XL) {
      const u32x4 xv = *(const u32x4*)(x_lds + x_row_off + ks * 32 + 8 * q);
      acc[0] = MfmaOp<T>::run(xv, op, acc[0]);
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = MfmaOp<T>::run(xr[slot][i][mt], op, acc[mt]);
    }
  };

  // quads in order; a quad starts on a group boundary (SPG divides 4), so group changes fall
  // on fixed k-steps of it.  k-steps past K (the tile's last quad) are skipped.
  for (int done = 0; done < nq; done += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      if (done + u < nq) {  // wave-uniform
        const int c = qa + done + u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ks = 4 * c + i;
          if (ks < KS) {  // wave-uniform
            if (i % SPG == 0) {
              flush();
              prep(ks / SPG);
            }
            compute(wr[u][i], u, i, ks);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (done + D < nq) issue(u);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  flush();

  // ---- the waves' sums meet in LDS: lane (q, r), element v = token mt*16 + 4q + v, column r
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < (ONE ? 1 : 4); ++v) {
      const int m = mt * 16 + 4 * q + v;
      if (m < p.M) red[(wave * MROWS + m) * 16 + r] = ONE ? tot1 : tot[mt][v];
    }
  __syncthreads();
  if (p.gate_act) {
    // gated epilogue: columns c < 8 of the tile are gate sums, 8 + c the matching up sums
    for (int o = tid; o < p.M * 8; o += NWV * 64) {
      const int m = o >> 3, c = o & 7;
      float g = red[m * 16 + c], u = red[m * 16 + 8 + c];
#pragma unroll
      for (int w = 1; w < NWV; ++w) {
        g += red[(w * MROWS + m) * 16 + c];
        u += red[(w * MROWS + m) * 16 + 8 + c];
      }
      const int oc = t * 8 + c;
      if (oc < p.n_out) p.c[(int64_t)m * p.ldc + oc] = to_bits<T>(gated_act(g, p.gate_act - 1) * u);
    }
    return;
  }
  for (int o = tid; o < p.M * 16; o += NWV * 64) {
    const int m = o >> 4, c = o & 15;
    float sum = red[m * 16 + c];
#pragma unroll
    for (int w = 1; w < NWV; ++w) sum += red[(w * MROWS + m) * 16 + c];
    const int oc = t * 16 + c;
    if (oc < p.N) {
      if (p.bias) sum += load_bias(p.bias, p.bias_dtype, oc);
      p.c[(int64_t)m * p.ldc + oc] = to_bits<T>(sum);
    }
  }
}

// Narrow stream pack: thread = one lane's u32 of one (tile, quad) run, number i = k-step
// 4 c + i (zero past K and past N).
__global__ void __launch_bounds__(256) pack_narrow_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                          int64_t K, int64_t N, int64_t tiles) {
  const int64_t KS = K / 32, KQ = (KS + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= tiles * KQ * 256) return;
  const int i = (int)(idx & 3);
  const int l = (int)((idx >> 2) & 63);
  const int64_t tc = idx >> 8;
  const int64_t t = tc / KQ, s = (tc - t * KQ) * 4 + i;
  const int q = l >> 4, r = l & 15;
  const int64_t col = t * 16 + r;
  uint32_t v = 0;
  if (col < N && s < KS) {
    const int64_t NW = N / 8;
    const int sh = 4 * col_nib<false>((int)(col & 7));
    for (int j = 0; j < 8; ++j) {
      const uint32_t nib = (in[(s * 32 + 8 * q + j) * NW + (col >> 3)] >> sh) & 0xFu;
      v |= nib << ((j & 1) * 16 + (j >> 1) * 4);
    }
  }
  out[idx] = v;
}

}  // namespace awq

namespace awq_host {
using namespace awq;

static int narrow_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

int64_t decode_narrow_bytes(int64_t K, int64_t N) { return cdiv(N, 16) * cdiv(K / 32, 4) * 1024; }

int launch_pack_decode_narrow(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N, hipStream_t st) {
  const int64_t tiles = cdiv(N, 16);
  const int64_t n = tiles * cdiv(K / 32, 4) * 256;
  if (n > 0)
    hipLaunchKernelGGL(pack_narrow_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, (const uint32_t*)qweight_kn,
                       (uint32_t*)out, K, N, tiles);
  return narrow_status();
}

// 16 waves per block (one block per CU) when the tiles fit the CUs once and the activations
// come from LDS, else 8 (two per CU; with per-k-step activation loads 8 waves also measured
// faster at one tile per CU); one token tile stages its activation rows in LDS when they fit:
// in 64 KiB, or in the CU's 160 KiB when the tiles fit the CUs once (one block per CU anyway)
constexpr uint32_t kNarrowLdsMax = 65536, kNarrowLdsMaxOne = 163840;

template <int MT, bool ZP, typename T, bool SBF, bool ONE, bool XL, bool NORM = false>
static bool launch_narrow_t(const GemmArgs& a, hipStream_t st) {
  const int tiles = (int)cdiv(a.N, 16);
  const int spg = a.G / 32;
  const dim3 grid((unsigned)tiles, (unsigned)(a.rows > 1 ? a.rows : 1));
  const int nwv = (tiles <= num_cus() && XL) ? 16 : 8;
  const NarrowLds L = narrow_lds(nwv, ONE ? 1 : 16 * MT, a.K / a.G, a.K, ZP, XL ? a.M : 0);
  if (L.total > (tiles <= num_cus() ? kNarrowLdsMaxOne : kNarrowLdsMax)) return false;
  if (NORM && a.K / 8 > (int64_t)kNormCols * nwv * 64) return false;
#define AWQ_NARROW_L(NWV, SPG_) \
  hipLaunchKernelGGL((decode_narrow_kernel<MT, NWV, SPG_, ZP, T, SBF, ONE, XL, NORM>), grid, dim3((NWV) * 64), L.total, st, a, tiles)
  if (nwv == 16) {
    if (spg == 4) AWQ_NARROW_L(16, 4);
    else if (spg == 2) AWQ_NARROW_L(16, 2);
    else AWQ_NARROW_L(16, 1);
  } else {
    if (spg == 4) AWQ_NARROW_L(8, 4);
    else if (spg == 2) AWQ_NARROW_L(8, 2);
    else AWQ_NARROW_L(8, 1);
  }
#undef AWQ_NARROW_L
  return true;
}

template <bool ZP, typename T, bool SBF>
static bool launch_narrow_m(const GemmArgs& a, hipStream_t st) {
  if (a.M > 16) return launch_narrow_t<2, ZP, T, SBF, false, false>(a, st);
  if (a.M > 1)
    return launch_narrow_t<1, ZP, T, SBF, false, true>(a, st) || launch_narrow_t<1, ZP, T, SBF, false, false>(a, st);
  return launch_narrow_t<1, ZP, T, SBF, true, true>(a, st) || launch_narrow_t<1, ZP, T, SBF, true, false>(a, st);
}

// The RMSNorm prologue variant: one fp16 row, fp16 scales, the row staged in LDS (false when
// it does not fit; the caller then normalises in a launch of its own).  Only M = 1: for 2 .. 4
// rows the prologue measured no faster on MI355X than the separate row-norm launch (K = 4096,
// N = 6144: 11.0 us against 10.2 us of kernels plus the launch gap).
bool launch_decode_narrow_norm(const GemmArgs& a, bool zp, hipStream_t st) {
  if (a.M != 1 || !a.norm_w) return false;
  return zp ? launch_narrow_t<1, true, f16, false, true, true, true>(a, st)
            : launch_narrow_t<1, false, f16, false, true, true, true>(a, st);
}

bool launch_decode_narrow(const GemmArgs& a, bool zp, int act, int sdt, hipStream_t st) {
  const bool sbf = sdt == AWQ_DTYPE_BF16;
  if (act == AWQ_DTYPE_F16) {
    if (sbf) return zp ? launch_narrow_m<true, f16, true>(a, st) : launch_narrow_m<false, f16, true>(a, st);
    return zp ? launch_narrow_m<true, f16, false>(a, st) : launch_narrow_m<false, f16, false>(a, st);
  }
  if (sbf) return zp ? launch_narrow_m<true, bf16, true>(a, st) : launch_narrow_m<false, bf16, true>(a, st);
  return zp ? launch_narrow_m<true, bf16, false>(a, st) : launch_narrow_m<false, bf16, false>(a, st);
}

}  // namespace awq_host
