// Grouped MoE GEMMs for many routes per expert (prefill-sized batches) on gfx950: the work of
// moe_gemm_kernel (awq_moe_kernel.h) restructured like the prefill GEMM (awq_gemm.hip).
//
//  * A block computes 64 routes (rows of the expert's route list) x 256 columns of one
//    expert; blocks are numbered over the experts' row tiles (derived from the per-expert
//    route counts) times the column tiles, and blocks past the last row tile exit.
//  * k-stages of 64: the block gathers its 64 activation rows (x rows for gate_up, rows of
//    the intermediate for down) into LDS and dequantizes its weight tile once into LDS; the
//    weight comes from the MoE stream copy, where one 16-byte lane piece is one packed word
//    over 4 consecutive k-rows -- exactly one dequant thread's share.
//  * 8 waves in a 2 x 4 grid, wave tile 32 x 64, v_mfma_f32_16x16x32_{f16,bf16}.  For gate_up
//    each wave's 64 columns are 32 gate columns followed by the 32 up columns of the same
//    indices, so the activation epilogue act(gate) * up * route_weight pairs registers of the
//    same lane.  Rounding points match moe_gemm_kernel: fp32 sums, the intermediate rounded
//    once to the activation dtype, fp32 per-route rows from down.
#include "awq_moe_kernel.h"

namespace awq {

__device__ __forceinline__ int gswz_a(int row) { return row & 7; }
__device__ __forceinline__ int gswz_b(int n) { return (n ^ (n >> 4)) & 7; }

constexpr int kGBM = 64, kGBN = 256, kGBK = 64;

// MODE 0: gate_up (paired stream tiles, activation epilogue into the intermediate)
// MODE 1: down (plain stream tiles, fp32 per-route rows)
template <int MODE, int PD, bool ZP, typename T, bool FAST>
__global__ void __launch_bounds__(512, 2) moe_mfma_kernel(const MoeArgs p, int scale_bf16, int E, int tiles_n) {
  constexpr int NT = 512, BM = kGBM, BN = kGBN, BK = kGBK;
  constexpr int WM = 32, WN = 64, MTL = WM / 16, NTL = WN / 16;
  constexpr int CPR = BK / 8;  // 16-byte chunks per LDS row
  static_assert(BM * CPR == NT, "one activation chunk per thread per stage");
  static_assert((BN / 8) * (BK / 4) == NT, "one packed word x 4 k-rows per thread");
  __shared__ u32x4 lds_a[2][BM * CPR];
  __shared__ u32x4 lds_b[2][BN * CPR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int wave_m = wave >> 2, wave_n = wave & 3;

  // ---- which expert row tile: walk the experts' tile counts ----
  const int tn = blockIdx.x % tiles_n;
  int tmg = blockIdx.x / tiles_n;
  int e = 0, count = 0;
  for (; e < E; ++e) {
    count = p.counts[e];
    const int nt_e = (count + BM - 1) / BM;
    if (tmg < nt_e) break;
    tmg -= nt_e;
  }
  if (e >= E) return;  // past the last row tile (whole block)
  const int m0 = tmg * BM;
  const int* list = p.lists + (int64_t)e * p.R;

  const int KS = p.K >> 5;
  const int NW = p.N >> 3;
  const int ngroups = p.K / p.G;
  const uint32_t stream_bytes = (uint32_t)p.tiles * (uint32_t)KS * 2048u;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc((const char*)p.qw + (int64_t)e * stream_bytes, stream_bytes);
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(p.sc + (int64_t)e * ngroups * p.N, (uint32_t)ngroups * (uint32_t)p.N * 2u);
  const __amdgpu_buffer_rsrc_t zrs =
      make_rsrc(ZP ? (const void*)(p.qz + (int64_t)e * ngroups * NW) : (const void*)p.sc, ZP ? (uint32_t)ngroups * (uint32_t)NW * 4u : 0u);
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(p.a, (uint32_t)((uint64_t)p.rows_a * (uint64_t)p.lda * 2u));

  // ---- activation row gathered by this thread (one 16-byte chunk per stage) ----
  const int arow = tid >> 3, ach = tid & 7;
  int src = 0;
  {
    const int m = m0 + arow;
    if (m < count) {
      const int rt = list[m];
      src = MODE == 0 ? rt / p.topk : rt;
    }
  }
  // per-lane byte offsets are fixed; each stage adds a wave-uniform offset (SGPR)
  const uint32_t a_voff = ((uint32_t)src * (uint32_t)p.lda + 8u * (uint32_t)ach) * 2u;

  // ---- weight word of this thread: stream tile, lane, LDS row of each nibble column ----
  const int bw = tid & 31, kq = tid >> 5;  // word of the block, k-rows 4 kq .. 4 kq + 3
  int stile, slane, gword, nrow0;          // nrow0: LDS row of the word's column 0
  if constexpr (MODE == 0) {
    // block columns: gate words 16 tn .. 16 tn + 15 and their up words (2 stream tiles)
    stile = 2 * tn + (bw >> 4);
    slane = bw & 15;
    const int gw = 16 * tn + (bw >> 4) * 8 + (slane & 7);  // gate word index
    const int h = slane >> 3;                               // 0 gate, 1 up
    gword = gw < p.half ? (h ? p.half + gw : gw) : -1;
    const int gc = 64 * (bw >> 4) + 8 * (slane & 7);        // first gate column in the block
    nrow0 = 64 * (gc >> 5) + 32 * h + (gc & 31);
  } else {
    stile = 2 * tn + (bw >> 4);
    slane = bw & 15;
    const int w = 32 * tn + bw;
    gword = w < NW ? w : -1;
    nrow0 = 8 * bw;
  }
  const int stld = stile < p.tiles ? stile : p.tiles - 1;  // in-range reads for padding words
  const uint32_t wc = gword < 0 ? 0u : (uint32_t)gword;
  // k-step 2 s + kq / 8, rows 4 (kq % 8) .. + 3 of it: lane piece (kq & 1) of lane 16 q' + r
  const uint32_t b_voff = ((uint32_t)stld * (uint32_t)KS + (uint32_t)(kq >> 3)) * 2048u + (uint32_t)(kq & 1) * 1024u +
                          (uint32_t)(16 * ((kq & 7) >> 1) + slane) * 16u;
  // group of the thread's rows: (64 s + 4 kq) / G = 64 s / G + (G == 32 ? kq / 8 : 0)
  const int g_lane = p.G == 32 ? (kq >> 3) : 0;
  const uint32_t s_voff = 16u * wc + (uint32_t)g_lane * (uint32_t)p.N * 2u;
  const uint32_t z_voff = 4u * wc + (uint32_t)g_lane * (uint32_t)NW * 4u;

  f32x4 acc[MTL][NTL];
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nst = p.K / BK;  // a multiple of PD (the launcher picks PD so)
  const MagicK mk = magic_consts();
  // ring of PD stages of global data in registers: stage s + 1 + PD is requested right after
  // stage s + 1 went to LDS, so PD stages of MFMA work cover its latency
  u32x4 aring[PD], bring[PD];
  WordSZ szring[PD];
  u32x4 areg, braw;
  WordSZ bsz;
  auto load = [&](int s, int slot) {
    s = min(s, nst - 1);  // past the end: re-request the last stage (never written)
    aring[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)a_voff, s * BK * 2, 0));
    bring[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)b_voff, s * 4096, 0));
    const int gu = (s * BK) / p.G;  // wave-uniform part of the group
    szring[slot].s4 = __builtin_bit_cast(
        u32x4, __builtin_amdgcn_raw_buffer_load_b128(srs, (int)s_voff, (int)((uint32_t)gu * (uint32_t)p.N * 2u), 0));
    szring[slot].zw = ZP ? __builtin_amdgcn_raw_buffer_load_b32(zrs, (int)z_voff, (int)((uint32_t)gu * (uint32_t)NW * 4u), 0)
                         : 0x88888888u;
  };
  auto take = [&](int slot) {
    areg = aring[slot];
    braw = bring[slot];
    bsz = szring[slot];
  };
  auto write_a = [&](int buf) { lds_a[buf][arow * CPR + (ach ^ gswz_a(arow))] = areg; };
  auto write_b_nib = [&](int buf, int I, const uint32_t (&lo)[2], const uint32_t (&hi)[2]) {
    u32x2 v;
    const bool sb = scale_bf16 != 0;
#define AWQ_GM_CASE(II, SRC, P)                                            \
    case II: {                                                             \
      const ColConst c_ = prep_const<II, false, FAST>(bsz, sb);            \
      v[0] = deq2<FAST, T>(magic_bits<P>(SRC[0], mk), c_);                 \
      v[1] = deq2<FAST, T>(magic_bits<P>(SRC[1], mk), c_);                 \
      break;                                                               \
    }
    switch (I) {  // I is a constant after unrolling
      AWQ_GM_CASE(0, lo, 0) AWQ_GM_CASE(1, lo, 1) AWQ_GM_CASE(2, lo, 2) AWQ_GM_CASE(3, lo, 3)
      AWQ_GM_CASE(4, hi, 0) AWQ_GM_CASE(5, hi, 1) AWQ_GM_CASE(6, hi, 2)
      default: AWQ_GM_CASE(7, hi, 3)
    }
#undef AWQ_GM_CASE
    const int n = nrow0 + nib_col<false>(I);
    ((u32x2*)lds_b[buf])[(n * CPR + ((kq >> 1) ^ gswz_b(n))) * 2 + (kq & 1)] = v;
  };
  auto read_b = [&](int cb, int sub, u32x4 (&bf)[NTL]) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int n = wave_n * WN + nt * 16 + r;
      bf[nt] = lds_b[cb][n * CPR + ((sub * 4 + q) ^ gswz_b(n))];
    }
  };
  auto read_a = [&](int cb, int sub, int mt) {
    const int row = wave_m * WM + mt * 16 + r;
    return lds_a[cb][row * CPR + ((sub * 4 + q) ^ gswz_a(row))];
  };
  auto mfma = [&](int mt, const u32x4 (&bf)[NTL], const u32x4& af) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) acc[mt][nt] = MfmaOp<T>::run(af, bf[nt], acc[mt][nt]);
  };
  auto pairs = [&](uint32_t (&lo)[2], uint32_t (&hi)[2]) {
    lo[0] = pair_lo(braw[0], braw[1]);
    hi[0] = pair_hi(braw[0], braw[1]);
    lo[1] = pair_lo(braw[2], braw[3]);
    hi[1] = pair_hi(braw[2], braw[3]);
  };
  auto step = [&](int cb, int wb) {
    u32x4 bf[NTL];
    read_b(cb, 0, bf);
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) mfma(mt, bf, read_a(cb, 0, mt));
    __builtin_amdgcn_sched_barrier(0);
    read_b(cb, 1, bf);
    write_a(wb);
    uint32_t lo[2], hi[2];
    pairs(lo, hi);
#pragma unroll
    for (int mt = 0; mt < MTL; ++mt) {
      mfma(mt, bf, read_a(cb, 1, mt));
#pragma unroll
      for (int i = 0; i < 8 / MTL; ++i) write_b_nib(wb, mt * (8 / MTL) + i, lo, hi);
    }
  };

#pragma unroll
  for (int u = 0; u < PD; ++u) load(u, u);
  take(0);
  {
    write_a(0);
    uint32_t lo[2], hi[2];
    pairs(lo, hi);
#pragma unroll
    for (int I = 0; I < 8; ++I) write_b_nib(0, I, lo, hi);
  }
  load(PD, 0);
  __syncthreads();
  for (int s0 = 0; s0 < nst; s0 += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      const int s = s0 + u;
      take((u + 1) % PD);  // stage s + 1 (after the last stage: unread data)
      step(s & 1, (s & 1) ^ 1);
      load(s + 1 + PD, (u + 1) % PD);
      __syncthreads();
    }
  }

  // ---- epilogue: lane (q, r), acc[mt][nt][v] = row m0 + wave_m*WM + mt*16 + 4q + v,
  // LDS column wave_n*WN + nt*16 + r ----
#pragma unroll
  for (int mt = 0; mt < MTL; ++mt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = m0 + wave_m * WM + mt * 16 + 4 * q + v;
      if (m >= count) continue;
      const int rt = list[m];
      if constexpr (MODE == 0) {
        const float wgt = load_route_weight(p.rw, p.rw_dtype, rt);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int gc = 128 * tn + 32 * wave_n + nt * 16 + r;  // gate column
          if (gc >= 8 * p.half) continue;
          const float h = gated_act(acc[mt][nt][v], p.act_kind) * acc[mt][nt + 2][v] * wgt;
          ((uint16_t*)p.out)[(int64_t)rt * p.ldo + gc] = to_bits<T>(h);
        }
      } else {
#pragma unroll
        for (int nt = 0; nt < NTL; ++nt) {
          const int col = BN * tn + wave_n * WN + nt * 16 + r;
          if (col < p.N) ((float*)p.out)[(int64_t)rt * p.ldo + col] = acc[mt][nt][v];
        }
      }
    }
  }
}

}  // namespace awq

namespace awq_host {
using namespace awq;

template <int MODE, bool ZP, typename T, bool FAST>
static void launch_mfma_t(const MoeArgs& a, int E, int sbf, hipStream_t st) {
  const int tiles_n = MODE == 0 ? (int)cdiv(a.half, 16) : (int)cdiv(a.N / 8, 32);
  const int64_t tiles_m = cdiv(a.R, kGBM) + E;  // each expert adds at most one partial tile
  const dim3 grid((unsigned)(tiles_m * tiles_n));
  const int nst = a.K / kGBK;
  // a two-stage register ring keeps the kernel within 128 VGPRs, so two blocks (80 KB of LDS
  // each) share a CU and one block's stage barrier is covered by the other's MFMAs (a
  // four-stage ring at one block per CU measured 18% slower at T = 512)
  if (nst % 2 == 0)
    hipLaunchKernelGGL((moe_mfma_kernel<MODE, 2, ZP, T, FAST>), grid, dim3(512), 0, st, a, sbf, E, tiles_n);
  else
    hipLaunchKernelGGL((moe_mfma_kernel<MODE, 1, ZP, T, FAST>), grid, dim3(512), 0, st, a, sbf, E, tiles_n);
}

template <int MODE>
static void launch_mfma_mode(const MoeArgs& a, int E, bool zp, int act, int sbf, hipStream_t st) {
  if (act == AWQ_DTYPE_BF16) {
    zp ? launch_mfma_t<MODE, true, bf16, false>(a, E, sbf, st) : launch_mfma_t<MODE, false, bf16, false>(a, E, sbf, st);
  } else if (!sbf) {
    zp ? launch_mfma_t<MODE, true, f16, true>(a, E, sbf, st) : launch_mfma_t<MODE, false, f16, true>(a, E, sbf, st);
  } else {
    zp ? launch_mfma_t<MODE, true, f16, false>(a, E, sbf, st) : launch_mfma_t<MODE, false, f16, false>(a, E, sbf, st);
  }
}

void launch_moe_mfma(const MoeArgs& gu, const MoeArgs& dn, int E, bool zp, int act, int sbf, hipStream_t st) {
  launch_mfma_mode<0>(gu, E, zp, act, sbf, st);
  if (hipPeekAtLastError() != hipSuccess) return;
  launch_mfma_mode<1>(dn, E, zp, act, sbf, st);
}

}  // namespace awq_host
